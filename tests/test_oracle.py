"""Pins the CPU oracle before anything is checked against it (CPU only).

The reference commits no golden vectors for this path (its tests compare NPU and CPU routes on
seeded inputs), so each oracle function is pinned by checks that a plausible mistake would fail:
  * brute force per element from first principles (exact rational arithmetic where it matters);
  * the library routines the reference's CPU route itself calls (torch.round, torch._int_mm,
    F.conv2d in float64);
  * invariants and closed forms (max element -> +-127, ties to even, half-up vs half-away on
    negative ties, calibration boundaries at exact powers of two);
  * the independent C restatement (oracle/c) and the torch-CPU port (oracle/cpu_route.py);
  * the committed fixtures in tests/golden/ (regression; written by tests/golden/make_golden.py).
Each "discriminates" test also shows that a deliberately wrong variant, planted in the oracle's
arithmetic here on the CPU, fails the same check.
"""
import math
import os
from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import c_oracle, cpu_route
from oracle import xdna_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _bf16_values(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16).float().numpy()


def _f32_div(x, s):
    """The correctly rounded float32 quotient via float64 (exact double rounding for 24-bit operands)."""
    return np.float32(float(x) / float(s))


def _rint_half_even(v):
    f = math.floor(v)
    d = v - f
    if d > 0.5:
        return f + 1
    if d < 0.5:
        return f
    return f if f % 2 == 0 else f + 1


def brute_quant_row(row):
    amax = max(abs(float(v)) for v in row)
    s = np.float32(np.float32(max(amax, float(np.float32(1e-8)))) / np.float32(127))
    # the clamp-then-divide in float32 written out
    a = np.float32(amax) if np.float32(amax) > np.float32(1e-8) else np.float32(1e-8)
    s2 = _f32_div(a, np.float32(127))
    assert s == s2
    q = [max(-127, min(127, _rint_half_even(float(_f32_div(v, s2))))) for v in row]
    return np.array(q, np.int8), s2


# ------------------------------------------------------------------------------ quantize
@pytest.mark.parametrize("seed", range(4))
def test_quant_rows_brute_force(seed):
    x = _bf16_values((6, 37), seed)
    x[2] = 0.0                                   # zero row
    x[3, :] = 0.0
    x[3, 5] = -3.0                               # single non-zero: maps to -127
    q, s = O.quant_rows(x)
    for r in range(x.shape[0]):
        qb, sb = brute_quant_row(x[r])
        assert np.array_equal(q[r], qb) and s[r] == sb
    assert q[3, 5] == -127 and not q[2].any()


def test_quant_rows_invariants():
    x = _bf16_values((64, 300), 9, scale=3.0)
    q, s = O.quant_rows(x)
    assert np.abs(q).max() <= 127 and q.min() >= -127
    am = np.abs(x).argmax(axis=1)
    assert np.array_equal(np.abs(q[np.arange(64), am]), np.full(64, 127))
    # q * s reconstructs x within half a step
    err = np.abs(q.astype(np.float64) * s[:, None].astype(np.float64) - x.astype(np.float64))
    assert np.all(err <= s[:, None].astype(np.float64) * (0.5 + 1e-5))


def test_quant_rows_ties_to_even_and_discriminates():
    # s == 1 exactly (amax 127): x = k + 0.5 are exact ties
    x = np.array([[127.0, 2.5, -3.5, 0.5, -0.5, 1.5, 126.5, -126.5]], np.float32)
    q, s = O.quant_rows(x)
    assert s[0] == 1.0 and q[0].tolist() == [127, 2, -4, 0, 0, 2, 126, -126]
    # a half-away-from-zero variant fails the same check
    away = np.clip(np.sign(x) * np.floor(np.abs(x) / s[:, None] + 0.5), -127, 127).astype(np.int8)
    assert not np.array_equal(away, q)
    # a reciprocal-multiply variant gets this row wrong: x / s is a hair below 5.5, x * (1 / s) rounds up
    row = np.array([[1.0, 0.04330708459019661]], np.float32)
    qd, sd = O.quant_rows(row)
    recip = np.rint(row * (np.float32(1) / sd)[:, None])
    assert qd[0, 1] == brute_quant_row(row[0])[0][1] and recip[0, 1] != qd[0, 1]


def test_quant_rows_matches_torch_ops():
    """The reference's own expressions (runtime.py:145-148, :366-368) in torch, bf16 and fp32."""
    g = torch.Generator().manual_seed(5)
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        x = (torch.randn(33, 1000, generator=g) * 2).to(dt)
        x[4] = 0
        q_t, s_t = cpu_route.quant_rows(x)
        sx = x.abs().amax(dim=1, keepdim=True).float().clamp(min=1e-8) / 127
        q_g = torch.round(x.float() / sx).clamp(-127, 127).to(torch.int8)
        q, s = O.quant_rows(x.float().numpy())
        assert np.array_equal(q, q_t.numpy()) and np.array_equal(q, q_g.numpy())
        assert np.array_equal(s, s_t.numpy()) and np.array_equal(s, sx[:, 0].numpy())


def test_quant_rows_c_restatement():
    x = _bf16_values((300, 777), 12, scale=4.0)
    x[7] = 0
    q, s = O.quant_rows(x)
    qc, sc = c_oracle.quant_rows(x)
    assert np.array_equal(q, qc) and np.array_equal(s, sc)


# ------------------------------------------------------------------------------ GEMM
def test_gemm_brute_force_tiny():
    rng = np.random.default_rng(0)
    a = rng.integers(-127, 128, (5, 7), dtype=np.int8)
    w = rng.integers(-127, 128, (4, 7), dtype=np.int8)
    want = [[sum(int(a[i, k]) * int(w[j, k]) for k in range(7)) for j in range(4)] for i in range(5)]
    assert O.gemm_i32(a, w).tolist() == want
    # a transposed-operand mistake (a @ w instead of a @ w.T) is caught
    assert not np.array_equal(np.asarray(a[:4, :4], np.int64) @ np.asarray(w[:, :4], np.int64), O.gemm_i32(a[:4, :4], w[:, :4]))


@pytest.mark.parametrize("m,n,k", [(1, 8, 16), (37, 300, 200), (128, 512, 1024), (17, 33, 4096)])
def test_gemm_matches_int_mm_and_c(m, n, k):
    g = torch.Generator().manual_seed(m * n + k)
    a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    want = torch._int_mm(a, w.t().contiguous()).numpy()
    assert np.array_equal(O.gemm_i32(a.numpy(), w.numpy()), want)
    assert np.array_equal(c_oracle.gemm_i32(a.numpy(), w.numpy()), want)


# ------------------------------------------------------------------------------ dequant
def test_dequant_brute_force_association():
    rng = np.random.default_rng(3)
    acc = rng.integers(-2 ** 27, 2 ** 27, (40, 30), dtype=np.int64).astype(np.int32)
    sx = (rng.random(40) * 0.05 + 1e-3).astype(np.float32)
    sw = (rng.random(30) * 0.01 + 1e-4).astype(np.float32)
    b = (rng.standard_normal(30) * 0.01).astype(np.float32)
    y = O.dequant(acc, sx, sw, b)
    for i in range(40):
        for j in range(30):
            t = np.float32(float(acc[i, j]))                  # int32 -> float32, nearest even
            t = np.float32(float(t) * float(sx[i]))            # exact product, one rounding
            t = np.float32(float(t) * float(sw[j]))
            t = np.float32(float(t) + float(b[j]))
            assert y[i, j] == t
    # the other association acc * (sx * sw) differs somewhere on these values
    other = acc.astype(np.float32) * (sx[:, None] * sw[None, :]) + b
    assert not np.array_equal(other, y)
    assert np.array_equal(c_oracle.dequant(acc, sx, sw, b), y)


def test_to_bf16_matches_torch_and_brute_force():
    rng = np.random.default_rng(4)
    y = np.concatenate([rng.standard_normal(5000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 3.0e38, -1e-40], np.float32)])
    got = O.to_bf16(y)
    assert np.array_equal(got, torch.from_numpy(y).to(torch.bfloat16).float().numpy())
    # brute force: nearest of the two bf16 neighbours, ties to the even mantissa
    for v in y[:300]:
        u = np.float32(v).view(np.uint32)
        lo = np.uint32(u & 0xFFFF0000).view(np.float32)
        hi = np.uint32((u & 0xFFFF0000) + 0x10000).view(np.float32)
        dlo, dhi = abs(Fraction(float(v)) - Fraction(float(lo))), abs(Fraction(float(hi)) - Fraction(float(v)))
        pick = lo if dlo < dhi else hi if dhi < dlo else (lo if ((u >> 16) & 1) == 0 else hi)
        assert O.to_bf16(np.array([v], np.float32))[0] == pick


def test_to_f16_matches_torch_and_brute_force():
    """to_dtype(y, "f16") (every f16 GPU comparison's expected values) against torch's `.to(torch.float16)`
    and a brute force over all finite float16 values: the nearest one, ties to the even bit pattern, inf at
    and beyond 65520 (the largest finite value plus half its spacing), subnormals, signed zeros, NaN."""
    rng = np.random.default_rng(5)
    y = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 10,
                        (rng.standard_normal(2000) * 2.0 ** rng.integers(-30, 18, 2000)).astype(np.float32),
                        np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, -65520.0, 1e6, 2.0 ** -24, 2.0 ** -25,
                                  3 * 2.0 ** -26, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 6e-8, np.nan], np.float32)])
    got = O.to_dtype(y, "f16")
    want = torch.from_numpy(y).to(torch.float16).float().numpy()
    assert np.array_equal(got, want, equal_nan=True)
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f16 = bits.view(np.float16).astype(np.float64)
    fin = np.isfinite(f16)
    vals, vbits = f16[fin], bits[fin]
    for v in y[np.isfinite(y)][::7]:
        if abs(float(v)) >= 65520.0:
            pick = np.inf if v > 0 else -np.inf
        else:
            d = np.abs(vals - float(v))
            cand = np.flatnonzero(d == d.min())
            if len(cand) > 1:             # a tie: the even bit pattern (of the two neighbours)
                cand = [c for c in cand if vbits[c] % 2 == 0]
            pick = vals[cand[0]]
            if pick == 0.0:
                pick = np.copysign(0.0, float(v))
        assert O.to_dtype(np.array([v], np.float32), "f16")[0] == np.float32(pick), v
        assert np.signbit(O.to_dtype(np.array([v], np.float32), "f16")[0]) == np.signbit(np.float32(pick))


def test_linear_composite_matches_cpu_route():
    g = torch.Generator().manual_seed(8)
    x = torch.randn(50, 200, generator=g).to(torch.bfloat16)
    w = torch.randn(300, 200, generator=g) * 0.02
    b = torch.randn(300, generator=g) * 0.01
    w_kn, sw = cpu_route.weight_quant(w)
    want = cpu_route.linear(x, w_kn, sw, b)
    y, acc, xq, sx, swo = O.linear(x.float().numpy(), [w.numpy()], [b.numpy()], out_dtype="bf16")
    assert np.array_equal(y, want.float().numpy())
    # transposed form (x @ W with W [K, N]) quantizes per output column
    y2, *_ = O.linear(x.float().numpy(), [w.t().contiguous().numpy()], [b.numpy()], transposed=True, out_dtype="bf16")
    assert np.array_equal(y2, y)


# ------------------------------------------------------------------------------ conv
def test_conv_acc_brute_force_tiny():
    rng = np.random.default_rng(0)
    x = rng.integers(-60, 60, (2, 3, 4, 5), dtype=np.int8)
    w = rng.integers(-40, 40, (4, 3, 3, 3), dtype=np.int8)
    acc = O.conv3x3_acc(x, w)
    for n in range(2):
        for o in range(4):
            for yy in range(4):
                for xx in range(5):
                    s = 0
                    for c in range(3):
                        for ky in range(3):
                            for kx in range(3):
                                sy, sx = yy + ky - 1, xx + kx - 1
                                if 0 <= sy < 4 and 0 <= sx < 5:
                                    s += int(w[o, c, ky, kx]) * int(x[n, c, sy, sx])
                    assert acc[n, o, yy, xx] == s
    # a flipped kernel (correlation vs convolution) is caught
    flipped = O.conv3x3_acc(x, w[:, :, ::-1, ::-1])
    assert not np.array_equal(flipped, acc)


@pytest.mark.parametrize("n,ci,co,h,w", [(2, 3, 48, 13, 37), (1, 64, 32, 8, 16), (3, 16, 8, 5, 7)])
def test_conv_acc_matches_conv2d_and_c(n, ci, co, h, w):
    rng = np.random.default_rng(n + ci + co)
    x = rng.integers(-127, 128, (n, ci, h, w), dtype=np.int8)
    wt = rng.integers(-127, 128, (co, ci, 3, 3), dtype=np.int8)
    want = F.conv2d(torch.from_numpy(x).double(), torch.from_numpy(wt).double(), padding=1).numpy()
    acc = O.conv3x3_acc(x, wt)
    assert np.array_equal(acc, want.astype(np.int64))
    assert np.array_equal(c_oracle.conv3x3_acc(x, wt), acc.astype(np.int32))


def test_requant_closed_form_and_negative_ties():
    shift = 4
    vals = list(range(-200, 200)) + [-(2 * k + 1) * 8 for k in range(10)] + [2 ** 30, -2 ** 30]
    acc = np.array(vals, np.int64)
    for relu in (False, True):
        q = O.requant(acc, shift, relu)
        for v, got in zip(vals, q.tolist()):
            want = (v + 2 ** (shift - 1)) // 2 ** shift       # floor(v / 16 + 1/2): round half up
            want = min(255, max(0, want)) if relu else min(127, max(-128, want))
            assert got == want
        assert np.array_equal(c_oracle.requant(acc.astype(np.int32), shift, relu), q)
    # negative ties: -24 / 16 = -1.5 -> half up gives -1, half away would give -2
    assert O.requant(np.array([-24]), 4, False)[0] == -1
    away = int(np.sign(-24) * np.floor(abs(-24) / 16 + 0.5))
    assert away == -2 and away != O.requant(np.array([-24]), 4, False)[0]
    # matches the reference's integer expression in torch
    t = torch.tensor(vals, dtype=torch.int32)
    ref = ((t + (1 << (shift - 1))) >> shift).clamp_(-128, 127).to(torch.int8)
    assert np.array_equal(ref.numpy(), O.requant(acc, shift, False))


def test_calibrate_shift_boundaries():
    # relu: top * 1.25 == 255 * 2^k exactly for top = 204 * 2^k -> shift k; one more -> k + 1
    for k in range(1, 20):
        assert O.shift_from_top(float(204 * 2 ** k), True) == k
        assert O.shift_from_top(float(204 * 2 ** k + 1), True) == k + 1
    for top in (1000.0, 123456.0, 7.5e6):
        s = O.shift_from_top(top, False)
        assert 127 * 2 ** (s - 1) < top * 1.25 <= 127 * 2 ** s
    assert O.shift_from_top(3.0, False) == 1          # below the lower clamp
    assert O.shift_from_top(0.0, True) == 1 and O.shift_from_top(0.0, False) == 1
    assert O.shift_from_top(1e30, False) == 31
    acc = np.array([[-5000, 300], [20, -100]])
    assert O.calibrate_shift(acc, relu=False) == O.shift_from_top(5000.0, False)
    assert O.calibrate_shift(acc, relu=True) == O.shift_from_top(300.0, True)


def test_conv_composite_matches_cpu_route():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 16, 9, 11, generator=g)
    w = torch.randn(24, 16, 3, 3, generator=g) * 0.05
    b = torch.randn(24, generator=g) * 0.1
    for relu in (False, True):
        L = cpu_route.ConvLayerCPU(w, relu)
        xq, sx = cpu_route.conv_quant(x)
        L.calibrate(xq[0])
        q = L(xq)
        want = cpu_route.conv_dequant(q, L.scale, sx, b, torch.float32)
        y, qo, shift, xqo, sxo, wq, sw = O.conv3x3_int8(x.numpy(), w.numpy(), b.numpy(), relu)
        assert shift == L.shift
        assert np.array_equal(xqo, xq.numpy()) and np.array_equal(sxo, sx.flatten().numpy())
        assert np.array_equal(wq, L.wq.numpy()) and np.array_equal(sw, L.sw.numpy())
        assert np.array_equal(qo, q.numpy()) and np.array_equal(y, want.numpy())


# ------------------------------------------------------------------------------ fixtures
def test_golden_fixtures():
    path = os.path.join(GOLDEN, "golden.npz")
    d = np.load(path, allow_pickle=False)
    q, s = O.quant_rows(d["q_x"])
    assert np.array_equal(q, d["q_xq"]) and np.array_equal(s, d["q_sx"])
    acc = O.gemm_i32(d["g_a"], d["g_w"])
    assert np.array_equal(acc, d["g_acc"])
    y = O.to_bf16(O.dequant(d["g_acc"], d["d_sx"], d["d_sw"], d["d_bias"]))
    assert np.array_equal(y, d["d_y_bf16"])
    cacc = O.conv3x3_acc(d["c_x"], d["c_w"])
    assert np.array_equal(cacc, d["c_acc"])
    for relu in (0, 1):
        assert np.array_equal(O.requant(cacc, int(d["c_shift"][relu]), bool(relu)), d[f"c_q{relu}"])
        assert O.calibrate_shift(cacc[0], bool(relu)) == int(d["c_shift"][relu])


# ------------------------------------------------------------------------------ bf16 GEMM (precision "bf16")
def test_gemm_bf16_exact_rationals_tiny():
    """y against exact rational sums of the bf16-rounded operands (Python fractions)."""
    from fractions import Fraction

    rng = np.random.default_rng(7)
    x = (rng.standard_normal((3, 9)) * [[1e-3], [1.0], [50.0]]).astype(np.float32)
    w = rng.standard_normal((4, 9)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    y, bound = O.gemm_bf16(x, w, b)
    xb, wb = O.to_bf16(x), O.to_bf16(w)
    for m in range(3):
        for n in range(4):
            exact = sum(Fraction(float(xb[m, k])) * Fraction(float(wb[n, k])) for k in range(9)) + Fraction(float(b[n]))
            mag = sum(abs(Fraction(float(xb[m, k])) * Fraction(float(wb[n, k]))) for k in range(9))
            assert abs(Fraction(float(y[m, n])) - exact) <= mag * Fraction(9, 2 ** 53) + abs(exact) * Fraction(1, 2 ** 52)
            assert bound[m, n] > 0


def test_gemm_bf16_bound_contains_float32_and_rejects_wrong_operands():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((64, 1000)).astype(np.float32)
    w = (rng.standard_normal((300, 1000)) * 0.02).astype(np.float32)
    y, bound = O.gemm_bf16(x, w)
    y32 = O.to_bf16(x) @ O.to_bf16(w).T                  # a float32 summation of the same products
    assert (np.abs(y32.astype(np.float64) - y) <= bound).all()
    wrong = x.astype(np.float64) @ w.astype(np.float64).T  # operands not rounded to bf16
    assert (np.abs(wrong - y) > bound).mean() > 0.5        # the worst-case bound is loose; half still fail
    sq = rng.standard_normal((50, 50)).astype(np.float32)
    ws = rng.standard_normal((50, 50)).astype(np.float32)
    ys, bs = O.gemm_bf16(sq, ws)
    yt = O.to_bf16(sq).astype(np.float64) @ O.to_bf16(ws).astype(np.float64)   # x @ w instead of x @ w^T
    assert (np.abs(yt - ys) > bs).mean() > 0.5


def test_max_pool2_matches_torch():
    rng = np.random.default_rng(9)
    for shape in [(2, 3, 8, 6), (1, 5, 7, 9)]:
        y = rng.standard_normal(shape).astype(np.float32)
        want = torch.nn.functional.max_pool2d(torch.from_numpy(y), 2, 2).numpy()
        assert np.array_equal(O.max_pool2(y), want)


def test_qwen3_stack_matches_transformers():
    """oracle.qwen3_stack vs transformers' own Qwen3Model (float64, 2 layers of Qwen3-0.6B's widths,
    random weights, with a head and bias) under a prefix-block mask: the valid rows agree to float64
    rounding. Pins RMSNorm placement, q / k norms, RoPE (pairing, sign, angles), grouped-query heads
    and the SiLU MLP."""
    from models import Stack, prefix_mask
    from oracle import qwen3_stack as Q

    torch.manual_seed(5)
    net = Stack(layers=2, out=96, bias=True).double().eval()
    with torch.no_grad():                       # non-trivial norm weights
        for name, p in net.named_parameters():
            if "norm" in name:
                p.copy_(1 + 0.1 * torch.randn_like(p))
    lens, L = [19, 12], 19
    x = torch.randn(2, L, 1024, dtype=torch.float64)
    with torch.no_grad():
        y = net(x, prefix_mask(lens, L))
    layers, norm, inv_freq = Q.model_weights(net.llm)
    for b, n in enumerate(lens):
        want = Q.stack_forward(x[b, :n], layers, norm, net.head.weight, net.head.bias, inv_freq)
        err = float((y[b, :n] - want).norm() / want.norm())
        assert err < 1e-10, (b, err)
    # a plausible mistake fails: RoPE with the rotation's sign flipped
    bad = Q.rope
    try:
        Q.rope = lambda t, f: bad(t, -f)        # noqa: E731
        wrong = Q.stack_forward(x[0, :lens[0]], layers, norm, net.head.weight, net.head.bias, inv_freq)
    finally:
        Q.rope = bad
    assert float((y[0, :lens[0]] - wrong).norm() / wrong.norm()) > 1e-3
