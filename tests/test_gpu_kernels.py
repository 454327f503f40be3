"""GPU parity of every C-ABI entry point against the CPU oracle (bit-exact).

Each test calls the HIP library through its ctypes binding (torch_xdna.kernels) on seeded inputs and
compares with oracle/ (numpy restatement; the C restatement for the larger integer sums):
  * integers (quantized activations and weights, int32 sums, int8/uint8 conv outputs) bit for bit;
  * float32 scales and dequantized outputs bit for bit in float32, and bf16 / fp16 outputs bit
    for bit after the round-to-nearest-even cast (the 1e-6 relative / 1 ulp bound of the contract
    is not needed: the fused epilogue rounds exactly like the reference's CPU ops).
"""
import re

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import xdna_oracle as O

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _np(t):
    return t.detach().cpu().numpy()


def _f32(t):
    return t.detach().float().cpu().numpy()


def _rand(shape, dtype, seed, scale=1.0, outliers=0.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * scale
    if outliers:
        x = torch.where(torch.rand(*shape, generator=g) < outliers, x * 20, x)
    return x.to(dtype)


def _i8(shape, seed, lo=-127, hi=128):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi, shape, generator=g, dtype=torch.int8)


# ------------------------------------------------------------------------------ quantize
@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,k", [(1, 16), (5, 200), (7, 300), (64, 1024), (33, 4096), (3, 14336), (2, 40000),
                                    (9, 1), (2000, 8192), (1500, 14336), (4800, 14336), (700, 4112), (600, 20000)])
def test_quant_rows(gpu, dtype, rows, k):
    x = _rand((rows, k), DT[dtype], seed=rows * 1000 + k, outliers=1e-3)
    from torch_xdna import kernels

    xq, sx = kernels.quant_rows(x.to(gpu))
    q_ref, s_ref = O.quant_rows(_f32(x))
    k_pad = -(-k // 16) * 16
    assert xq.shape == (rows, k_pad)
    assert np.array_equal(_np(xq)[:, :k], q_ref)
    assert not _np(xq)[:, k:].any()
    assert np.array_equal(_np(sx).view(np.uint32), s_ref.view(np.uint32))


def test_quant_rows_ties_zero_rows_strided(gpu):
    from torch_xdna import kernels

    # amax 127 makes s == 1 exactly, so x = k + 0.5 are exact ties (round half to even);
    # amax 254 makes s == 2, so odd integers x are ties too; an all-zero row gives zeros.
    rows = [[127.0, 2.5, -3.5, 0.5, -0.5, 1.5, 126.5, -126.5] + [0.0] * 8,
            [254.0, 5.0, -5.0, 7.0, -7.0, 1.0, 3.0, -1.0] + [0.0] * 8,
            [0.0] * 16]
    base = torch.tensor(rows, dtype=torch.float32)
    big = torch.zeros(3, 48)
    big[:, :16] = base
    xq, sx = kernels.quant_rows(big.to(gpu)[:, :16])    # a view with row stride 48 != K
    q_ref, s_ref = O.quant_rows(base.numpy())
    assert np.array_equal(_np(xq)[:, :16], q_ref)
    assert np.array_equal(_np(sx), s_ref)
    assert _np(xq)[0, :8].tolist() == [127, 2, -4, 0, 0, 2, 126, -126]
    assert _np(xq)[1, :8].tolist() == [127, 2, -2, 4, -4, 0, 2, 0]


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("k", [1024, 200, 16384, 40000])
def test_quant_rows_near_half(gpu, dtype, k):
    """Quotients x / s placed within 6e-5 of half-integers, on both sides, exactly on them and at fractions
    of the float spacing there, under irregular scales: the kernels round fl(x / s) like torch (the fast
    product with 1 / s is trusted only farther than 2^-15 from a half-integer; nearer, the exact residual
    x - h * s decides). Covers the 16-element-group, per-vector and long-row paths."""
    from torch_xdna import kernels

    rng = np.random.default_rng(k + len(dtype))
    rows = 64
    amax = rng.uniform(0.5, 300.0, rows).astype(np.float32)
    s = (amax / np.float32(127)).astype(np.float32)
    half = rng.integers(-127, 127, (rows, k)).astype(np.float64) + 0.5
    d = rng.choice([0.0, 1e-7, -1e-7, 3e-6, -3e-6, 1.5e-5, -1.5e-5, 2.9e-5, -2.9e-5, 3.1e-5, -3.1e-5, 6e-5, -6e-5],
                   (rows, k))
    # every other column: offsets in units of the float spacing at the half-integer, around the half-spacing
    # boundary where fl(x / s) stops being the half-integer itself
    ulp = np.spacing(np.abs(half).astype(np.float32)).astype(np.float64)
    d_ulp = rng.choice([0.3, -0.3, 0.49, -0.49, 0.51, -0.51, 0.9, -0.9, 1.1, -1.1, 2.5, -2.5], (rows, k)) * ulp
    d[:, 1::2] = d_ulp[:, 1::2]
    x = ((half + d) * s[:, None].astype(np.float64)).astype(np.float32)
    x[:, 0] = amax                                   # fixes the row's amax, hence s
    xt = torch.from_numpy(x).to(DT[dtype])
    xq, sx = kernels.quant_rows(xt.to(gpu))
    q_ref, s_ref = O.quant_rows(_f32(xt))
    assert np.array_equal(_np(sx).view(np.uint32), s_ref.view(np.uint32))
    bad = _np(xq)[:, :k] != q_ref
    assert not bad.any(), f"{bad.sum()} of {bad.size} differ"


# ------------------------------------------------------------------------------ int32 GEMM
GEMM_SHAPES = [(1, 16, 64), (3, 50, 208), (16, 4096, 1024), (64, 1000, 512), (65, 300, 208), (200, 300, 208),
               (256, 512, 1024), (1000, 777, 96), (2048, 2048, 256), (4096, 4096, 128), (333, 4112, 48)]


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
def test_gemm_i32(gpu, m, n, k):
    from torch_xdna import kernels

    a = _i8((m, k), seed=m + 7 * n + 13 * k)
    w = _i8((n, k), seed=m + 7 * n + 13 * k + 1)
    c = kernels.mm_i8(a.to(gpu), w.to(gpu))
    want = c_oracle.gemm_i32(a.numpy(), w.numpy())
    got = _np(c)
    assert got.dtype == np.int32 and np.array_equal(got, want), f"{(got != want).sum()} of {got.size} differ"


def test_gemm_i32_extremes(gpu):
    """|sum| up to K * 127^2 with K = 16384 (no int32 overflow, no saturation)."""
    from torch_xdna import kernels

    k = 16384
    a = torch.full((20, k), 127, dtype=torch.int8)
    a[1::2] = -127
    w = torch.full((33, k), 127, dtype=torch.int8)
    c = _np(kernels.mm_i8(a.to(gpu), w.to(gpu)))
    assert c[0, 0] == 127 * 127 * k and c[1, 0] == -127 * 127 * k
    assert np.array_equal(c, c_oracle.gemm_i32(a.numpy(), w.numpy()))


# ------------------------------------------------------------------------------ fused dequant GEMM
@pytest.mark.parametrize("out", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("m,n,k,bias", [(1, 4096, 1024, True), (16, 1000, 512, False), (128, 3072, 1024, True),
                                        (300, 520, 1024, True), (700, 300, 208, False), (2048, 1024, 256, True)])
def test_gemm_dequant(gpu, out, m, n, k, bias):
    from torch_xdna import kernels

    x = _rand((m, k), torch.float32, seed=m + n + k, outliers=1e-3)
    wt = _rand((n, k), torch.float32, seed=m + n + k + 1, scale=0.02)
    b = _rand((n,), torch.float32, seed=m + n + k + 2, scale=0.01) if bias else None
    xq_r, sx_r = O.quant_rows(x.numpy())
    wq_r, sw_r = O.quant_rows(wt.numpy())
    k_pad = -(-k // 16) * 16
    xq, sx = kernels.quant_rows(x.to(gpu), k_pad)
    wq, sw = kernels.quant_rows(wt.to(gpu), k_pad)
    y = kernels.mm_i8_dequant(xq, sx, wq, sw, None if b is None else b.to(gpu), DT[out])
    acc = c_oracle.gemm_i32(xq_r, wq_r)
    want = O.to_dtype(O.dequant(acc, sx_r, sw_r, None if b is None else b.numpy()), out)
    got = _f32(y)
    bad = ~((got == want) | (np.isnan(got) & np.isnan(want)))
    assert not bad.any(), f"{bad.sum()} of {got.size} differ, e.g. {got[bad][:4]} vs {want[bad][:4]}"


@pytest.mark.parametrize("m,n,out", [(8192, 4096, "f32"), (8192, 8192, "bf16"), (8000, 4100, "f16")])
def test_gemm_dequant_large_output(gpu, m, n, out):
    """Fused-dequantize outputs of 128 MB (f32 8192 x 4096, bf16 8192 x 8192) and a ragged f16 one: every
    output against the oracle's float32 dequantize of the C oracle's sums, with bias."""
    from torch_xdna import kernels

    k = 256
    a, w = _i8((m, k), seed=m + 1), _i8((n, k), seed=n + 2)
    sx, sw, b = torch.rand(m) + 0.01, torch.rand(n) + 0.01, torch.randn(n)
    y = kernels.mm_i8_dequant(a.to(gpu), sx.to(gpu), w.to(gpu), sw.to(gpu), b.to(gpu), DT[out])
    want = O.to_dtype(O.dequant(c_oracle.gemm_i32(a.numpy(), w.numpy()), sx.numpy(), sw.numpy(), b.numpy()), out)
    got = _f32(y)
    bad = ~((got == want) | (np.isnan(got) & np.isnan(want)))
    assert not bad.any(), f"{bad.sum()} of {got.size} differ"


@pytest.mark.parametrize("out", ["f32", "bf16", "f16"])
def test_gemm_dequant_range(gpu, out):
    """Scales from 1e-45 to 3e38 put the fused epilogue's outputs in every float range (zero,
    subnormal in f32 / bf16 / f16, normal, overflow to inf) through the products and the hardware
    round-to-nearest-even conversions, against the oracle's float32 products and casts."""
    from torch_xdna import kernels

    m, n, k = 256, 512, 128
    a, w = _i8((m, k), 1), _i8((n, k), 2)
    rng = np.random.default_rng(3)
    sx = (10.0 ** rng.uniform(-30, 15, m)).astype(np.float32)
    sw = (10.0 ** rng.uniform(-20, 15, n)).astype(np.float32)
    sx[:4] = [0.0, 1e-45, np.finfo(np.float32).tiny, 3e38]
    y = kernels.mm_i8_dequant(a.to(gpu), torch.from_numpy(sx).to(gpu), w.to(gpu), torch.from_numpy(sw).to(gpu),
                              None, DT[out])
    with np.errstate(over="ignore", under="ignore"):
        want = O.to_dtype(O.dequant(c_oracle.gemm_i32(_np(a), _np(w)), sx, sw), out)
    got = _f32(y)
    assert np.isinf(want).any() and (want[np.isfinite(want) & (want != 0)] != 0).any()
    bad = ~((got == want) | (np.isnan(got) & np.isnan(want)))
    assert not bad.any(), f"{bad.sum()} of {got.size} differ, e.g. {got[bad][:4]} vs {want[bad][:4]}"


# ------------------------------------------------------------------------------ bf16 GEMM (precision "bf16")
def _bf16_bracket(got, want, bound, out):
    """got (the output dtype's values, as float32) must be the rounding of some v with
    |v - want| <= bound; rounding is monotonic, so it lies between the roundings of the two ends
    (widened by 2^-20 relative for the float64 -> float32 step)."""
    pad = bound * 1.0001 + np.abs(want) * 2.0 ** -20 + 1e-38
    lo = O.to_dtype((want - pad).astype(np.float32), out)
    hi = O.to_dtype((want + pad).astype(np.float32), out)
    bad = ~((got >= lo) & (got <= hi))
    assert not bad.any(), f"{bad.sum()} of {got.size} outside the bound, e.g. {got[bad][:3]} vs {want[bad][:3]}"


# ------------------------------------------------------------------------------ one row, quantize in the launch
def _row_oracle(x, wq, sw, b, kp, out):
    """The oracle's one-row W8A8 linear: quantize the row, pad it to kp, exact sums, dequantize, cast."""
    xq, sx = O.quant_rows(x.float().numpy())
    xq = np.pad(xq, ((0, 0), (0, kp - xq.shape[1])))
    acc = c_oracle.gemm_i32(xq, wq.numpy())
    return O.to_dtype(O.dequant(acc, sx, sw.numpy(), None if b is None else b.numpy()), out), sx


@pytest.mark.parametrize("xd", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("out", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("n,k,kp,bias", [(300, 1000, 1008, True), (4096, 4096, 4096, False), (14337, 4104, 4112, True),
                                         (7, 8, 16, False)])
def test_linear_row(gpu, xd, out, n, k, kp, bias):
    """xdna_linear_row (the row's quantize, the GEMM and the dequantize in one launch) against the oracle:
    every output and the row's scale bit for bit; x shorter than the weight rows (the padding counts as
    zeros, the weights there are not zero), K past whole 4 KB rounds, N ragged with 4 columns per wave
    (14337), 1 column per wave (300, 4096, 7)."""
    from torch_xdna import kernels

    if xd == "f32" and k % 4 or xd != "f32" and k % 8:
        pytest.skip("kx elements must fill 16-byte loads")
    x = _rand((1, k), DT[xd], seed=n + k, outliers=1e-2)
    wq = _i8((n, kp), seed=n + 1)
    sw = torch.rand(n) * 1e-3 + 1e-5
    b = _rand((n,), torch.float32, seed=n + 2) if bias else None
    sx = torch.full((1,), -1.0, device=gpu)
    y = kernels.linear_row(x.to(gpu), wq.to(gpu), sw.to(gpu), None if b is None else b.to(gpu), DT[out], sx=sx)
    want, sx_r = _row_oracle(x, wq, sw, b, kp, out)
    got = _f32(y)
    bad = ~((got == want) | (np.isnan(got) & np.isnan(want)))
    assert not bad.any(), f"{bad.sum()} of {got.size} differ, e.g. {got[bad][:4]} vs {want[bad][:4]}"
    assert _np(sx).view(np.uint32)[0] == sx_r.view(np.uint32)[0]


@pytest.mark.parametrize("n,k", [(4096, 4096), (14336, 4096), (4096, 14336)])
def test_linear_row_decode_shapes(gpu, n, k):
    """The C5 decode shapes at one row (bf16 in and out, bias) against the oracle and against the two
    launches it replaces (quant_rows, then the fused-dequantize GEMM), bit for bit."""
    from torch_xdna import kernels

    x = _rand((1, k), torch.bfloat16, seed=k, outliers=1e-3)
    wt = _rand((n, k), torch.float32, seed=n, scale=0.02).to(gpu)
    wq, sw = kernels.quant_rows(wt)
    b = _rand((n,), torch.float32, seed=n + k, scale=0.01).to(gpu)
    y = kernels.linear_row(x.to(gpu), wq, sw, b, torch.bfloat16)
    xq, sx = kernels.quant_rows(x.to(gpu), k)
    y2 = kernels.mm_i8_dequant(xq, sx, wq, sw, b, torch.bfloat16)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    want, _ = _row_oracle(x, wq.cpu(), sw.cpu(), b.cpu(), k, "bf16")
    assert np.array_equal(_f32(y), want)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_linear_row_special_rows(gpu, dtype):
    """Rows of zeros, with +inf / -inf / NaN, of subnormals, below the 1e-8 scale floor, with values on
    half-integers of the scale, and of the dtype's largest values: outputs (NaN where the scale is NaN) and
    scales against quant_rows + the fused-dequantize GEMM."""
    from torch_xdna import kernels

    k, n = 1024, 520
    dt = DT[dtype]
    base = _rand((1, k), torch.float32, seed=5)
    rows = {"zeros": torch.zeros(1, k), "tiny": base * 1e-12, "sub": base * 1e-40,
            "halves": torch.arange(k, dtype=torch.float32).view(1, k) % 255 - 127 + 0.5,
            "big": torch.full((1, k), float(torch.finfo(dt).max)) * torch.sign(base)}
    for name, v in (("pinf", float("inf")), ("ninf", float("-inf")), ("nan", float("nan"))):
        r = base.clone()
        r[0, 77] = v
        rows[name] = r
    wq = _i8((n, k), seed=9).to(gpu)
    sw = (torch.rand(n) * 1e-2 + 1e-4).to(gpu)
    for name, r in rows.items():
        xg = r.to(dt).to(gpu)
        sx1 = torch.empty(1, device=gpu)
        y = kernels.linear_row(xg, wq, sw, None, dt, sx=sx1)
        xq, sx2 = kernels.quant_rows(xg, k)
        y2 = kernels.mm_i8_dequant(xq, sx2, wq, sw, None, dt)
        a, b2 = _f32(y), _f32(y2)
        same = (a == b2) | (np.isnan(a) & np.isnan(b2))
        assert same.all(), f"{name}: {(~same).sum()} of {a.size} differ"
        s1, s2 = _np(sx1), _np(sx2)
        assert (s1.view(np.uint32) == s2.view(np.uint32)).all() or (np.isnan(s1) & np.isnan(s2)).all(), name


def test_linear_row_kmax_and_chunks(gpu):
    """The longest row (XDNA_LINEAR_ROW_KMAX, the most groups per thread) and a weight of more than 1 GB
    (33000 x 32768: two launches of row chunks, the scale written by the first), against the two
    launches it replaces."""
    from torch_xdna import kernels

    k = kernels.LINEAR_ROW_KMAX
    g = torch.Generator(device=gpu).manual_seed(3)
    x = torch.randn(1, k, generator=g, device=gpu).to(torch.bfloat16)
    for n in (600, 33000):
        wq = torch.randint(-127, 128, (n, k), generator=g, device=gpu, dtype=torch.int8)
        sw = torch.rand(n, generator=g, device=gpu) * 1e-3
        b = torch.randn(n, generator=g, device=gpu)
        sx1 = torch.empty(1, device=gpu)
        y = kernels.linear_row(x, wq, sw, b, torch.float32, sx=sx1)
        xq, sx2 = kernels.quant_rows(x, k)
        y2 = kernels.mm_i8_dequant(xq, sx2, wq, sw, b, torch.float32)
        assert torch.equal(y, y2), f"n={n}: {int((y != y2).sum())} differ"
        assert torch.equal(sx1, sx2)
        del wq


@pytest.mark.parametrize("out", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("m,n,k,bias", [(1, 4096, 1024, True), (16, 1000, 520, False), (64, 300, 200, True),
                                        (128, 3072, 1024, True), (300, 520, 1032, False), (700, 1000, 4096, True),
                                        (2048, 1024, 256, False)])
def test_gemm_bf16(gpu, out, m, n, k, bias):
    """xdna_gemm_bf16 against the oracle's bf16 GEMM within the float32-accumulation bound, through
    the small-M kernel (m <= 64) and the tile engine, K a multiple of 64 and not."""
    from torch_xdna import kernels

    x = _rand((m, k), torch.float32, seed=m + n + k)
    w = _rand((n, k), torch.float32, seed=m + n + k + 1, scale=0.05)
    b = _rand((n,), torch.float32, seed=m + n + k + 2, scale=0.1) if bias else None
    xb = kernels.bf16_rows(x.to(gpu), k)
    wb = kernels.bf16_rows(w.to(gpu), k)
    y = kernels.mm_bf16(xb, wb, None if b is None else b.to(gpu), DT[out])
    want, bound = O.gemm_bf16(x.numpy(), w.numpy(), None if b is None else b.numpy())
    _bf16_bracket(_f32(y), want, bound, out)


# ------------------------------------------------------------------------------ conv
def _conv_case(n, ci, co, h, w, seed):
    x = _rand((n, ci, h, w), torch.float32, seed=seed)
    wt = _rand((co, ci, 3, 3), torch.float32, seed=seed + 1, scale=0.05)
    return x, wt


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("n,ch,h,w,c_pad", [(8, 3, 224, 224, 16),    # an RGB batch (VGG-16's input)
                                            (2, 3, 13, 36, 16), (1, 3, 20, 24, 32), (2, 1, 5, 8, 16),
                                            (1, 5, 33, 40, 16),      # a partly filled last block
                                            (3, 17, 9, 16, 32), (2, 40, 8, 8, 48), (1, 64, 56, 56, 64),
                                            (2, 80, 8, 16, 96), (1, 256, 8, 64, 256), (2, 7, 5, 7, 16)])
def test_conv_quant(gpu, dtype, n, ch, h, w, c_pad):
    """Per-image quantize + NCHW -> NHWC of float / bf16 / fp16 images against the oracle, bit for bit:
    narrow images (c_pad <= 64, the pixel-major kernel), wide ones (the 256-channel tile), pixel counts
    that are not whole 16-byte loads (the scalar kernel), padding channels past ch zero, and an all-zero
    image beside ones with a single large value."""
    from torch_xdna import kernels

    x = _rand((n, ch, h, w), torch.float32, seed=n * 1000 + ch * 10 + h + w, scale=3.0)
    if n > 1:
        x[0] = 0.0
    x.view(n, -1)[-1, (ch * h * w) // 2] = -40.0
    x = x.to(DT[dtype])
    xq, sx = kernels.conv_quant(x.to(gpu), c_pad)
    xq_r, sx_r = O.conv_quant_images(x.float().numpy())
    got = _np(xq)
    assert got.shape == (n, h, w, c_pad)
    assert np.array_equal(got[..., :ch].transpose(0, 3, 1, 2), xq_r), f"{(got[..., :ch].transpose(0, 3, 1, 2) != xq_r).sum()} differ"
    assert not got[..., ch:].any()
    assert np.array_equal(_np(sx), sx_r)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("ch,c_pad", [(3, 16), (40, 48)])
def test_conv_quant_special(gpu, dtype, ch, c_pad):
    """Non-finite images: an image with +inf (its scale inf), one with -inf, one with a NaN (its scale NaN,
    as torch.amax propagates it) and a normal one. The reference's int8 cast of a NaN quotient is not defined
    (numpy and torch's CPU cast give what the platform gives), so the narrow-image kernel is held to the
    256-channel tile kernel on the same images bit for bit (scales NaN where NaN), and the normal image to
    the oracle."""
    from torch_xdna import kernels

    x = _rand((4, ch, 8, 12), torch.float32, seed=ch, scale=2.0)
    x[0, ch // 2, 3, 5] = float("inf")
    x[1, 0, 7, 11] = float("-inf")
    x[2, ch - 1, 0, 0] = float("nan")
    x = x.to(DT[dtype]).to(gpu)
    xq, sx = kernels.conv_quant(x, c_pad)              # the narrow-image kernel
    xq_t, sx_t = kernels.conv_quant(x, 256)            # the 256-channel tile kernel
    assert np.array_equal(_np(xq)[..., :ch], _np(xq_t)[..., :ch]) and not _np(xq)[..., ch:].any()
    s1, s2 = _np(sx), _np(sx_t)
    assert ((s1.view(np.uint32) == s2.view(np.uint32)) | (np.isnan(s1) & np.isnan(s2))).all()
    assert np.isinf(s1[:2]).all() and np.isnan(s1[2])
    xq_r, sx_r = O.conv_quant_images(x[3:].float().cpu().numpy())
    assert np.array_equal(_np(xq)[3:, ..., :ch].transpose(0, 3, 1, 2), xq_r) and np.array_equal(s1[3:], sx_r)


@pytest.mark.parametrize("n,ci,co,h,w", [(2, 3, 48, 13, 37), (1, 64, 128, 16, 64), (2, 16, 20, 5, 7),
                                         (1, 256, 256, 8, 64), (3, 40, 64, 9, 9),
                                         (1, 32, 256, 64, 256),      # larger tiles (every tile shape:
                                         (1, 16, 256, 256, 256),     # test_tiles_forced)
                                         # 16-channel inputs with co a multiple of 32 up to 128 (the
                                         # register-only kernel): RGB, gray, 5 and 16 channels, ragged
                                         # sizes, pixel counts off the 32-pixel blocks, several images
                                         (2, 3, 64, 13, 37), (1, 16, 32, 7, 5), (3, 1, 128, 9, 11),
                                         (2, 5, 96, 31, 17), (1, 3, 64, 224, 224), (4, 16, 128, 1, 3),
                                         # 32-, 48- and 64-channel inputs with co a multiple of 32 up to 128
                                         # (the resident-weight kernel): odd chunk counts, ragged sizes
                                         (2, 64, 64, 13, 37), (1, 40, 128, 9, 11), (3, 32, 96, 7, 5),
                                         (2, 20, 32, 15, 4), (1, 64, 128, 56, 56), (2, 48, 64, 1, 1)])
@pytest.mark.parametrize("relu", [False, True])
def test_conv3x3(gpu, n, ci, co, h, w, relu):
    from torch_xdna import kernels

    x, wt = _conv_case(n, ci, co, h, w, seed=n * 131 + ci * 7 + co + h + w)
    c_pad = -(-ci // 16) * 16
    xq, sx = kernels.conv_quant(x.to(gpu), c_pad)
    wq, sw = kernels.conv_weight_pack(wt.to(gpu), c_pad)
    xq_r, sx_r = O.conv_quant_images(x.numpy())
    wq_r, sw_r = O.conv_weight_quant(wt.numpy())
    # quantize + layout
    assert np.array_equal(_np(xq)[..., :ci], xq_r.transpose(0, 2, 3, 1)) and not _np(xq)[..., ci:].any()
    assert np.array_equal(_np(sx), sx_r)
    assert np.array_equal(_np(wq)[:, :, :ci], wq_r.reshape(co, ci, 9).transpose(0, 2, 1))
    assert not _np(wq)[:, :, ci:].any() and np.array_equal(_np(sw), sw_r)
    # calibration on image 0, then the requantized integers
    acc = c_oracle.conv3x3_acc(xq_r, wq_r)
    top = kernels.conv3x3_calibrate(xq[:1], wq, relu)
    want_top = int(np.clip(acc[0], 0, None).max()) if relu else int(np.abs(acc[0]).max())
    assert top == want_top
    shift = O.shift_from_top(float(top), relu)
    q = kernels.conv3x3(xq, wq, shift, relu)
    want_q = O.requant(acc, shift, relu)
    got_q = _np(q).transpose(0, 3, 1, 2)
    assert got_q.dtype == want_q.dtype and np.array_equal(got_q, want_q), f"{(got_q != want_q).sum()} differ"
    # dequant back to NCHW float
    scale = O.conv_scale(sw_r, shift)
    bias = _rand((co,), torch.float32, seed=5, scale=0.1)
    y = kernels.conv_dequant(q, relu, torch.from_numpy(scale).to(gpu), sx, bias.to(gpu), torch.float32)
    assert np.array_equal(_np(y), O.conv_dequant(want_q, scale, sx_r, bias.numpy()))
    # the conv with the dequantize fused into its epilogue: the same floats without the integers in memory
    y_fused = kernels.conv3x3_dequant(xq, wq, shift, relu, torch.from_numpy(scale).to(gpu), sx, bias.to(gpu),
                                      torch.float32)
    assert np.array_equal(_np(y_fused), O.conv_dequant(want_q, scale, sx_r, bias.numpy()))


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("n,ci,co,h,w", [(2, 3, 48, 13, 37), (3, 40, 64, 9, 9), (2, 16, 20, 5, 7), (5, 16, 36, 1, 3),
                                         (1, 64, 128, 16, 64), (1, 256, 256, 8, 64), (1, 32, 256, 64, 256),
                                         (2, 3, 64, 13, 37), (3, 16, 128, 9, 11),    # the 16-channel kernel's integers
                                         (2, 64, 64, 13, 37), (1, 40, 128, 9, 11)])  # the resident-weight kernel's
def test_conv3x3_dequant_fused(gpu, dtype, n, ci, co, h, w):
    """xdna_conv3x3_dequant against xdna_conv3x3_i8 + xdna_conv_dequant, bit for bit, in every output dtype,
    with and without ReLU and bias: images whose pixel counts are not multiples of 4 (runs of four pixels
    crossing images, one image of 3 pixels), channel counts off the tile widths, several images per launch."""
    from torch_xdna import kernels

    x, wt = _conv_case(n, ci, co, h, w, seed=n * 17 + ci + co + h * w)
    c_pad = -(-ci // 16) * 16
    xq, sx = kernels.conv_quant(x.to(gpu), c_pad)
    wq, sw = kernels.conv_weight_pack(wt.to(gpu), c_pad)
    for relu in (False, True):
        shift = O.shift_from_top(float(kernels.conv3x3_calibrate(xq[:1], wq, relu)), relu)
        scale = torch.from_numpy(O.conv_scale(sw.cpu().numpy(), shift)).to(gpu)
        q = kernels.conv3x3(xq, wq, shift, relu)
        for bias in (None, _rand((co,), torch.float32, seed=co, scale=0.1).to(gpu)):
            want = kernels.conv_dequant(q, relu, scale, sx, bias, DT[dtype])
            got = kernels.conv3x3_dequant(xq, wq, shift, relu, scale, sx, bias, DT[dtype])
            assert got.shape == want.shape and got.dtype == want.dtype
            assert torch.equal(got, want), f"{int((got != want).sum())} of {want.numel()} differ (relu {relu})"


@pytest.mark.parametrize("relu", [False, True])
@pytest.mark.parametrize("pool", [False, True])
@pytest.mark.parametrize("x_dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("n,co,h,w,c_pad", [(2, 64, 14, 10, 64), (1, 20, 9, 7, 32), (3, 48, 6, 6, 48),
                                             # whole 16-channel groups, a power-of-two group count (the wide
                                             # kernels): odd sizes, empty padding groups, partial tiles, one
                                             # image larger than 256 tiles (the max pass loops)
                                             (2, 16, 9, 9, 16), (1, 32, 15, 9, 64), (2, 128, 12, 10, 128),
                                             (1, 512, 6, 6, 512), (2, 256, 40, 38, 256), (1, 16, 520, 520, 16)])
def test_conv_requant_next(gpu, relu, pool, x_dtype, n, co, h, w, c_pad):
    """Conv chaining: the previous conv's NHWC q -> the next conv's NHWC int8 input and per-image scale,
    equal to dequantize -> cast -> [ReLU] -> [2x2 max-pool] -> per-image quantize through the oracle (bit
    for bit, padding channels zero)."""
    _check_requant_next(gpu, relu, pool, x_dtype, n, co, h, w, c_pad,
                        ((False, False), (True, False), (True, True)))


@pytest.mark.parametrize("relu", [False, True])
@pytest.mark.parametrize("n,co,h,w,c_pad,pool", [(4, 64, 224, 224, 64, False), (3, 16, 1024, 1024, 16, True)])
def test_conv_requant_next_wide_tiles(gpu, relu, n, co, h, w, c_pad, pool):
    """The same at sizes with at least two blocks of 1024 items per CU, where the wide kernels give each
    lane four items (the smaller cases above take one), with bias and the ReLU after it."""
    _check_requant_next(gpu, relu, pool, "f32", n, co, h, w, c_pad, ((True, True),))


@pytest.mark.parametrize("relu_y", [False, True])
@pytest.mark.parametrize("co,c_pad", [(64, 64), (20, 32)])
def test_conv_requant_next_nan_image(gpu, relu_y, co, c_pad):
    """An image whose input scale is NaN (a NaN somewhere in the layer's float input): its next scale is NaN,
    as the reference's dequantize, ReLU (torch.relu keeps NaN) and amax give; the other images are unaffected
    and equal the oracle. The integers of the NaN image are not compared: the reference's int8 cast of a NaN
    quotient is not defined."""
    from torch_xdna import kernels

    g = torch.Generator().manual_seed(co)
    q = torch.randint(-40, 40, (3, 9, 10, co), generator=g, dtype=torch.int8)
    scale = torch.rand(co, generator=g) * 1e-3 + 1e-5
    sx = torch.tensor([0.7, float("nan"), 0.3])
    bias = torch.randn(co, generator=g) * 0.1
    for pool in (False, True):
        xq, sxn = kernels.conv_requant_next(q.to(gpu), False, pool, scale.to(gpu), sx.to(gpu), bias.to(gpu),
                                            torch.float32, c_pad, relu_y=relu_y)
        got_s = _np(sxn)
        assert np.isnan(got_s[1]) and np.isfinite(got_s[[0, 2]]).all()
        for i in (0, 2):
            y = O.conv_dequant(_np(q[i:i + 1]).transpose(0, 3, 1, 2), scale.numpy(), sx[i:i + 1].numpy(), bias.numpy())
            if relu_y:
                y = np.maximum(y, 0)
            if pool:
                y = O.max_pool2(y)
            xq_r, sx_r = O.conv_quant_images(y)
            assert np.array_equal(_np(xq)[i:i + 1, ..., :co].transpose(0, 3, 1, 2), xq_r) and got_s[i] == sx_r[0]


def _check_requant_next(gpu, relu, pool, x_dtype, n, co, h, w, c_pad, variants):
    """variants: (with bias, relu_y) pairs; q in a narrow range with one spike per image (positive or
    negative) at a seeded place, so each image's scale comes from one item."""
    from torch_xdna import kernels

    g = torch.Generator().manual_seed(n * 100 + co + h)
    q = (torch.randint(0, 40, (n, h, w, co), generator=g, dtype=torch.uint8) if relu
         else torch.randint(-40, 40, (n, h, w, co), generator=g, dtype=torch.int8))
    for i in range(n):
        yi, xi, ci = (int(torch.randint(0, d, (1,), generator=g)) for d in (h, w, co))
        q[i, yi, xi, ci] = 250 if relu else (-127 if i % 2 else 126)
    scale = torch.rand(co, generator=g) * 1e-3 + 1e-5
    sx = torch.rand(n, generator=g) + 0.1
    bias = torch.randn(co, generator=g) * 0.1
    for with_bias, relu_y in variants:
        b = bias if with_bias else None
        xq, sxn = kernels.conv_requant_next(q.to(gpu), relu, pool, scale.to(gpu), sx.to(gpu),
                                            None if b is None else b.to(gpu), DT[x_dtype], c_pad, relu_y=relu_y)
        y = O.to_dtype(O.conv_dequant(_np(q).transpose(0, 3, 1, 2), scale.numpy(), sx.numpy(),
                                      None if b is None else b.numpy()), x_dtype)
        if relu_y:
            y = np.maximum(y, 0)
        if pool:
            y = O.max_pool2(y)
        xq_r, sx_r = O.conv_quant_images(y)
        got = _np(xq)
        assert got.shape == (n, y.shape[2], y.shape[3], c_pad)
        assert np.array_equal(got[..., :co].transpose(0, 3, 1, 2), xq_r) and not got[..., co:].any()
        assert np.array_equal(_np(sxn), sx_r)


def test_conv_layouts(gpu):
    from torch_xdna import kernels

    xq = _i8((2, 19, 5, 11), seed=3)
    nhwc = kernels.nchw_to_nhwc(xq.to(gpu), 32)
    assert np.array_equal(_np(nhwc)[..., :19], xq.numpy().transpose(0, 2, 3, 1)) and not _np(nhwc)[..., 19:].any()
    q = _i8((2, 5, 11, 21), seed=4)
    back = kernels.nhwc_to_nchw(q.to(gpu))
    assert np.array_equal(_np(back), q.numpy().transpose(0, 3, 1, 2))


# ------------------------------------------------------------------------------ HIP graph capture
def test_graph_replay(gpu):
    """The launchers captured into one HIP graph (activation quantize, fused GEMM, conv quantize, conv,
    conv dequantize; and an RGB chain: narrow-image quantize, 16-channel conv, wide-kernel requantize,
    conv): three replays, with new inputs copied in and eager work plus synchronization between them,
    each bit-identical to the eager result on the same inputs."""
    from torch_xdna import kernels

    x = _rand((300, 1024), torch.bfloat16, seed=51).to(gpu)
    wq, sw = kernels.quant_rows(_rand((520, 1024), torch.float32, seed=52, scale=0.02).to(gpu))
    xc = _rand((2, 64, 20, 24), torch.float32, seed=53).to(gpu)
    cwq, csw = kernels.conv_weight_pack(_rand((64, 64, 3, 3), torch.float32, seed=54, scale=0.05).to(gpu), 64)
    scale = csw * 2.0 ** 9
    xr = _rand((2, 3, 30, 34), torch.float32, seed=55).to(gpu)
    rwq, rsw = kernels.conv_weight_pack(_rand((64, 3, 3, 3), torch.float32, seed=56, scale=0.2).to(gpu), 16)
    rbias = _rand((64,), torch.float32, seed=57, scale=0.1).to(gpu)

    def path():
        xq, sx = kernels.quant_rows(x)
        y = kernels.mm_i8_dequant(xq, sx, wq, sw, None, torch.bfloat16)
        cq, csx = kernels.conv_quant(xc, 64)
        q = kernels.conv3x3(cq, cwq, 9, False)
        yc = kernels.conv_dequant(q, False, scale, csx, None, torch.float32)
        rq, rsx = kernels.conv_quant(xr, 16)
        q1 = kernels.conv3x3(rq, rwq, 7, False)
        nq, nsx = kernels.conv_requant_next(q1, False, True, rsw * 2.0 ** 7, rsx, rbias, torch.float32, 64,
                                            relu_y=True)
        return y, yc, kernels.conv3x3(nq, cwq, 9, True), nsx

    path()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = path()
    for rep in range(3):
        x.copy_(_rand((300, 1024), torch.bfloat16, seed=60 + rep).to(gpu))
        xc.copy_(_rand((2, 64, 20, 24), torch.float32, seed=70 + rep).to(gpu))
        xr.copy_(_rand((2, 3, 30, 34), torch.float32, seed=80 + rep).to(gpu))
        want = path()                       # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for got, ref in zip(outs, want):
            assert torch.equal(got, ref), f"replay {rep} differs from the eager result"


# ------------------------------------------------------------------------------ every tile shape
def test_direct_tile(gpu, tile_table):
    """The direct conv kernels as the tile "direct": the rule's choice for the shapes they take (c_pad 16 to
    64, co a multiple of 32 up to 128), a forced engine tile overrides it, a forced "direct" on a shape they
    do not take runs the rule's engine tile, GEMM kinds reject it; results equal the oracle's throughout."""
    from torch_xdna import kernels

    assert kernels.tile_get(gpu, "conv", 1000, 64, 9 * 16) == "direct"
    assert kernels.tile_get(gpu, "conv", 1000, 128, 9 * 64) == "direct"
    assert kernels.tile_get(gpu, "conv", 1000, 48, 9 * 64) != "direct"        # co not a multiple of 32
    assert kernels.tile_get(gpu, "conv", 1000, 64, 9 * 128) != "direct"       # c_pad 128
    assert kernels.tile_plan(gpu, "conv", 1000, 64, 9 * 16) == ("direct", 0, "auto")
    with pytest.raises(RuntimeError, match="only convs"):
        kernels.tile_set("i8", 1000, 64, 144, "direct")
    for n, ci, co, h, w_, tile in [(2, 64, 96, 16, 20, "t64x64"), (2, 3, 64, 13, 37, "t256x64"),
                                   (1, 48, 40, 13, 37, "direct"), (1, 128, 64, 8, 12, "direct")]:
        c_pad = -(-ci // 16) * 16
        kernels.tile_set("conv", n * h * w_, co, 9 * c_pad, tile)
        want_tile = tile if tile != "direct" else kernels.tile_plan(gpu, "conv", n * h * w_, co, 9 * c_pad)[0]
        assert want_tile != "direct" or (co % 32 == 0 and co <= 128 and c_pad <= 64)
        xq = _i8((n, ci, h, w_), seed=ci + h)
        wq = _i8((co, ci, 3, 3), seed=co + w_)
        packed = torch.zeros(co, 9, c_pad, dtype=torch.int8)
        packed[:, :, :ci] = wq.permute(0, 2, 3, 1).reshape(co, 9, ci)
        q = kernels.conv3x3(kernels.nchw_to_nhwc(xq.to(gpu), c_pad), packed.to(gpu), 9, False)
        acc = c_oracle.conv3x3_acc(xq.numpy(), wq.numpy())
        assert np.array_equal(_np(q).transpose(0, 3, 1, 2), O.requant(acc, 9, False)), (n, ci, co, h, w_, tile)



@pytest.fixture
def tile_table():
    """The library's tile table, emptied before and after the test."""
    from torch_xdna import kernels

    kernels.use_tuned(False)
    kernels.tile_clear()
    yield kernels
    kernels.tile_clear()
    kernels._tuned_applied = None


@pytest.mark.parametrize("tile", ["t256x256w8", "t256x256w4", "t256x128", "t128x256", "t128x128", "t64x64",
                                  "t192x256", "t256x192", "t64x32", "t32x64", "t32x32",
                                  "t64x64k2", "t64x64k4", "t32x64k4", "t32x32k4", "t128x128k2", "t128x256w8",
                                  "t256x128w8", "t256x256pp", "t256x64"])
def test_tiles_forced(gpu, tile, tile_table):
    """Each tile configuration of the engine, forced through the library's tile table: int32 and
    fused bf16 GEMMs with partial tiles and K both a multiple of 64 and not (for the K-group tiles:
    slice counts not a multiple of the groups, and a single slice per group), and the conv with both A
    loaders (C_pad % 64 == 0 and not; for K groups C_pad % (64 * groups) == 0 and not) and its
    calibration maximum, against the oracle."""
    from torch_xdna import kernels

    for m, n, k in [(700, 1000, 4160), (333, 520, 208), (700, 1000, 2080), (333, 520, 104)]:
        kernels.tile_set("i8", m, n, k, tile)
        kernels.tile_set("bf16", m, n, k, tile)
        assert kernels.tile_get(gpu, "i8", m, n, k) == tile
    convs = [(2, 64, 96, 16, 20), (1, 48, 40, 13, 37), (1, 256, 64, 8, 12), (1, 128, 48, 9, 10)]
    for n, ci, co, h, w_ in convs:
        kernels.tile_set("conv", n * h * w_, co, 9 * -(-ci // 16) * 16, tile)
        assert kernels.tile_get(gpu, "conv", n * h * w_, co, 9 * -(-ci // 16) * 16) == tile
    for m, n, k in [(700, 1000, 4160), (333, 520, 208)]:
        a, w = _i8((m, k), seed=m + k), _i8((n, k), seed=n + k)
        acc = c_oracle.gemm_i32(a.numpy(), w.numpy())
        assert np.array_equal(_np(kernels.mm_i8(a.to(gpu), w.to(gpu))), acc), (m, n, k)
        sx = torch.rand(m) + 0.01
        sw = torch.rand(n) + 0.01
        y = kernels.mm_i8_dequant(a.to(gpu), sx.to(gpu), w.to(gpu), sw.to(gpu), None, torch.bfloat16)
        assert np.array_equal(_f32(y), O.to_bf16(O.dequant(acc, sx.numpy(), sw.numpy()))), (m, n, k)
    for m, n, k in [(700, 1000, 2080), (333, 520, 104)]:          # the bf16 GEMM (K bytes = 2 k)
        x = _rand((m, k), torch.float32, seed=m + k)
        w = _rand((n, k), torch.float32, seed=n + k, scale=0.05)
        y = kernels.mm_bf16(kernels.bf16_rows(x.to(gpu), k), kernels.bf16_rows(w.to(gpu), k), None, torch.float32)
        want, bound = O.gemm_bf16(x.numpy(), w.numpy())
        _bf16_bracket(_f32(y), want, bound, "f32")
    for n, ci, co, h, w_ in convs:
        xq = _i8((n, ci, h, w_), seed=ci + h)
        wq = _i8((co, ci, 3, 3), seed=co + w_)
        c_pad = -(-ci // 16) * 16
        packed = torch.zeros(co, 9, c_pad, dtype=torch.int8)
        packed[:, :, :ci] = wq.permute(0, 2, 3, 1).reshape(co, 9, ci)
        x_nhwc = kernels.nchw_to_nhwc(xq.to(gpu), c_pad)
        acc = c_oracle.conv3x3_acc(xq.numpy(), wq.numpy())
        q = kernels.conv3x3(x_nhwc, packed.to(gpu), 9, False)
        assert np.array_equal(_np(q).transpose(0, 3, 1, 2), O.requant(acc, 9, False)), (n, ci, co, h, w_)
        scale = (torch.rand(co) + 0.5).to(gpu)
        sx = (torch.rand(n) + 0.5).to(gpu)
        want = kernels.conv_dequant(q, False, scale, sx, None, torch.float32)
        assert torch.equal(kernels.conv3x3_dequant(x_nhwc, packed.to(gpu), 9, False, scale, sx, None, torch.float32),
                           want), ("fused dequant", n, ci, co, h, w_)
        if n == 1:
            assert kernels.conv3x3_calibrate(x_nhwc, packed.to(gpu), False) == int(np.abs(acc).max())


def _ksplit(cus, bm, bn, kg, tiles, k):
    """Workgroups per tile along K that the library gives a launch: 1 above 64 x 64 or when the tiles fill
    more than half of the CUs, else up to CUs / tiles, at most 16, with at least 16 slices of 64 per K
    group (used here only to check that the test's shapes reach the split)."""
    if bm * bn > 64 * 64 or 2 * tiles > cus:
        return 1
    nk = -(-k // 64)
    ks = min(cus // tiles, nk // (16 * kg), 16)
    if ks < 2:
        return 1
    per = -(-nk // ks)
    return -(-nk // per)


KSPLIT_TILES = {"t32x32": (32, 32, 1), "t32x64": (32, 64, 1), "t64x32": (64, 32, 1), "t64x64": (64, 64, 1),
                "t64x64k2": (64, 64, 2), "t64x64k4": (64, 64, 4), "t32x64k4": (32, 64, 4), "t32x32k4": (32, 32, 4)}


@pytest.mark.parametrize("tile", sorted(KSPLIT_TILES))
def test_gemm_ksplit(gpu, tile, tile_table):
    """The K split across workgroups (xdna_gemm_i8_i32_ws / xdna_gemm_i8_dequant_ws): shapes whose tiles
    leave most of the CUs idle, K in whole and partial 64-byte slices and splits of unequal length, ragged
    M and N. The int32 sums against the oracle; the workspace calls equal the calls without a workspace for
    the int32 sums and the fused dequant to every dtype with and without bias; a workspace that holds only
    the counters (no split) gives the same; calls follow each other on one workspace, whose counters are
    zero again after them."""
    from torch_xdna import kernels

    L = kernels.lib()
    cus = kernels.num_cus(gpu)
    bm, bn, kg = KSPLIT_TILES[tile]
    st = kernels._stream(gpu)
    split_seen = False
    for m, n, k in [(16, 1000, 4160), (3, 200, 14336), (40, 130, 4112), (5, 260, 14352), (64, 64, 1040),
                    (100, 520, 3072)]:
        kernels.tile_set("i8", m, n, k, tile)
        assert kernels.tile_get(gpu, "i8", m, n, k) == tile
        assert L.xdna_gemm_ws_bytes(m, n, k) > 0
        ks = _ksplit(cus, bm, bn, kg, -(-m // bm) * -(-n // bn), k)
        split_seen |= ks > 1
        # the launch plan (the verify cache's key) names the split
        assert kernels.gemm_variant(gpu, m, n, k) == (tile if ks == 1 else f"{tile}/k{ks}"), (tile, m, n, k)
        a, w = _i8((m, k), seed=m + k), _i8((n, k), seed=n + 2 * k)
        ag, wg = a.to(gpu), w.to(gpu)
        acc = c_oracle.gemm_i32(a.numpy(), w.numpy())
        c = kernels.mm_i8(ag, wg)
        assert np.array_equal(_np(c), acc), (tile, m, n, k)
        c0 = torch.empty_like(c)
        assert L.xdna_gemm_i8_i32(kernels._ptr(ag), k, kernels._ptr(wg), k, kernels._ptr(c0), n, m, n, k, st) == 0
        assert torch.equal(c0, c), (tile, m, n, k)
        ws = torch.zeros(65536, dtype=torch.uint8, device=gpu)           # the counters only: no split
        c1 = torch.empty_like(c)
        assert L.xdna_gemm_i8_i32_ws(kernels._ptr(ag), k, kernels._ptr(wg), k, kernels._ptr(c1), n, m, n, k,
                                     kernels._ptr(ws), ws.numel(), st) == 0
        assert torch.equal(c1, c), (tile, m, n, k)
        sx, sw = (torch.rand(m) + 0.01).to(gpu), (torch.rand(n) + 0.01).to(gpu)
        b = torch.randn(n).to(gpu)
        for out in ("f32", "bf16", "f16"):
            for bias in (b, None):
                y = kernels.mm_i8_dequant(ag, sx, wg, sw, bias, DT[out])
                y0 = torch.empty_like(y)
                assert L.xdna_gemm_i8_dequant(kernels._ptr(ag), k, kernels._ptr(sx), kernels._ptr(wg), k,
                                              kernels._ptr(sw), kernels._ptr(bias), kernels._ptr(y0),
                                              kernels._DTYPE_CODE[DT[out]], n, m, n, k, st) == 0
                assert torch.equal(y, y0), (tile, m, n, k, out, bias is None)
        want = O.to_bf16(O.dequant(acc, sx.cpu().numpy(), sw.cpu().numpy(), b.cpu().numpy()))
        assert np.array_equal(_f32(kernels.mm_i8_dequant(ag, sx, wg, sw, b, torch.bfloat16)), want), (tile, m, n, k)
        if ks > 1:
            # back-to-back launches on one workspace: which workgroup of a tile arrives last (and so reads
            # the others' partials from other XCDs) varies between launches; every launch gives the sums
            outs = [kernels.mm_i8(ag, wg) for _ in range(24)]
            for o in outs:
                assert torch.equal(o, c), (tile, m, n, k, "repeated launch")
    assert split_seen, f"no shape of the test splits K with {tile}"
    torch.cuda.synchronize()
    for buf in kernels._ws_buf.values():
        assert int(buf[:65536].view(torch.int32).abs().sum()) == 0, "arrival counters not back to zero"


@pytest.mark.parametrize("tile", ["t256x256w8", "t128x256w8"])
def test_conv_halo(gpu, tile, tile_table):
    """The conv from a haloed input tile (the 8-wave 256 x 256 and 128 x 256 tiles when a tile is whole image
    rows, or a segment of one row, of one image): the input pixels of a tile and their one-pixel border are
    loaded once per 64-channel slice and read at each tap's offset. Image rows of 32 to 512 pixels (several
    rows per tile, one, half a row), 1, 2 and 4 channel slices, ragged and several column tiles, batches
    of one and two: the requantized integers against the oracle, the fused dequantize against the
    separate one and the calibration max."""
    from torch_xdna import kernels

    for n, ci, co, h, w_ in [(2, 64, 256, 8, 64), (1, 128, 200, 16, 32), (1, 256, 512, 4, 128),
                             (2, 64, 256, 3, 256), (1, 128, 256, 2, 512)]:
        c_pad = ci
        kernels.tile_set("conv", n * h * w_, co, 9 * c_pad, tile)
        assert kernels.tile_get(gpu, "conv", n * h * w_, co, 9 * c_pad) == tile
        xq = _i8((n, ci, h, w_), seed=ci + h + w_)
        wq = _i8((co, ci, 3, 3), seed=co + w_)
        packed = wq.permute(0, 2, 3, 1).reshape(co, 9, ci).contiguous()
        x_nhwc = kernels.nchw_to_nhwc(xq.to(gpu), c_pad)
        acc = c_oracle.conv3x3_acc(xq.numpy(), wq.numpy())
        for relu in (False, True):
            q = kernels.conv3x3(x_nhwc, packed.to(gpu), 12, relu)
            assert np.array_equal(_np(q).transpose(0, 3, 1, 2), O.requant(acc, 12, relu)), (tile, n, ci, co, h, w_, relu)
        scale = (torch.rand(co) + 0.5).to(gpu)
        sx = (torch.rand(n) + 0.5).to(gpu)
        want = kernels.conv_dequant(q, True, scale, sx, None, torch.float32)
        assert torch.equal(kernels.conv3x3_dequant(x_nhwc, packed.to(gpu), 12, True, scale, sx, None, torch.float32),
                           want), ("fused dequant", tile, n, ci, co, h, w_)
        top = kernels.conv3x3_calibrate(x_nhwc[:1], packed.to(gpu), False)
        assert top == int(np.abs(acc[:1]).max()), (tile, n, ci, co, h, w_)


@pytest.mark.parametrize("tile", ["t256x256w8", "t256x128w8", "t128x256", "t256x256pp"])
def test_tiles_tail_split(gpu, tile, tile_table):
    """A one-workgroup-per-CU tile whose last round of tiles would fill at most half of the CUs runs the
    whole rounds with that tile and the leftover rows as a second launch (for the conv, from a pixel
    offset into the same images), when the leftover rows fit one round of the tail's tile: the int8
    GEMM's int32 sums and fused dequant, the bf16 GEMM and the conv's requantized output, with full and
    partial last tiles, against the oracle; the tail's tile as the library picks it (a split after
    256 x 256 tiles, none after the others at these shapes) and as the tile table lists it for the
    tail's own shape (a K-group tile: its own loader for the conv)."""
    from torch_xdna import kernels

    cus = kernels.num_cus(gpu)
    bm, bn = (int(v) for v in re.match(r"t(\d+)x(\d+)", tile).groups())
    n, k = bn, 64
    for m, tail in [(bm * (cus + cus // 4), None), (bm * (cus + cus // 4) - 100, None),
                    (bm * (cus + cus // 4) - 100, "t128x128k2")]:
        m1 = bm * cus
        for kind, kk in (("i8", k), ("bf16", k)):
            kernels.tile_set(kind, m, n, kk, tile)
            kernels.tile_set(kind, m - m1, n, kk, tail or "auto")
        a, w = _i8((m, k), seed=m), _i8((n, k), seed=n + 1)
        acc = c_oracle.gemm_i32(a.numpy(), w.numpy())
        assert np.array_equal(_np(kernels.mm_i8(a.to(gpu), w.to(gpu))), acc), (tile, m, tail)
        sx, sw = torch.rand(m) + 0.01, torch.rand(n) + 0.01
        y = kernels.mm_i8_dequant(a.to(gpu), sx.to(gpu), w.to(gpu), sw.to(gpu), None, torch.float32)
        assert np.array_equal(_f32(y), O.dequant(acc, sx.numpy(), sw.numpy())), (tile, m, tail)
        x = _rand((m, k), torch.float32, seed=m)
        wf = _rand((n, k), torch.float32, seed=n, scale=0.05)
        yb = kernels.mm_bf16(kernels.bf16_rows(x.to(gpu), k), kernels.bf16_rows(wf.to(gpu), k), None, torch.float32)
        want, bound = O.gemm_bf16(x.numpy(), wf.numpy())
        _bf16_bracket(_f32(yb), want, bound, "f32")
    # conv: h * w pixels make about 1.25 rounds of row tiles; w = 317 is not a multiple of any tile
    # height, so the head ends and the tail starts mid-image and both have a partial last tile
    ci, co = 64, bn
    w_ = 317
    h = (bm * (cus + cus // 4) - 100) // w_
    h -= (h * w_) % bm == 0
    tiles = -(-(h * w_) // bm)
    assert tiles // cus == 1 and 0 < 2 * (tiles % cus) <= cus and (h * w_) % bm and (bm * cus) % w_
    kernels.tile_set("conv", h * w_, co, 9 * ci, tile)
    xq, wq = _i8((1, ci, h, w_), seed=h), _i8((co, ci, 3, 3), seed=co)
    packed = wq.permute(0, 2, 3, 1).reshape(co, 9, ci).contiguous()
    x_nhwc = kernels.nchw_to_nhwc(xq.to(gpu), ci)
    acc = c_oracle.conv3x3_acc(xq.numpy(), wq.numpy())
    want = O.requant(acc, 9, True)
    for tail in (None, "t128x128k2"):       # a K-group tail takes the general A loader (64 % (2 * 64) != 0)
        kernels.tile_set("conv", h * w_ - bm * cus, co, 9 * ci, tail or "auto")
        q = kernels.conv3x3(x_nhwc, packed.to(gpu), 9, True)
        assert np.array_equal(_np(q).transpose(0, 3, 1, 2), want), (tile, tail, h, w_)


@pytest.mark.parametrize("m,n,k", [(4100, 4100, 208), (2600, 7000, 1040), (8192, 2304, 4096), (300, 520, 4160),
                                   (2600, 7000, 256), (2600, 7000, 192), (2600, 7000, 112), (2600, 7000, 64)])
def test_pp_tile(gpu, m, n, k, tile_table):
    """The ping-pong tile (t256x256pp: two groups of four waves alternating memory and MFMA phases):
    more tiles than CUs with partial last row / column tiles, K not a multiple of 64, fewer tiles than
    CUs, and K of a few slices (fewer slices than LDS stages). int32 sums against torch._int_mm on the CPU (the reference's CPU kernel),
    the fused bf16 dequant against the CPU dequantize of those sums, and the bf16 GEMM bit for bit against
    the 8-wave tile, which sums the same products in the same order."""
    from torch_xdna import kernels

    for kind, kk in (("i8", k), ("bf16", k // 2)):
        kernels.tile_set(kind, m, n, kk, "t256x256pp")
    assert kernels.tile_plan(gpu, "i8", m, n, k)[0] == "t256x256pp"
    a, w = _i8((m, k), seed=m + k), _i8((n, k), seed=n + k)
    acc = kernels.mm_i8(a.to(gpu), w.to(gpu)).cpu()
    want = torch._int_mm(a, w.t().contiguous())
    assert torch.equal(acc, want), f"{int((acc != want).sum())} sums differ"
    sx, sw, b = torch.rand(m) + 0.01, torch.rand(n) * 0.01, torch.randn(n)
    y = kernels.mm_i8_dequant(a.to(gpu), sx.to(gpu), w.to(gpu), sw.to(gpu), b.to(gpu), torch.bfloat16).cpu()
    assert torch.equal(y, ((want.float() * sx[:, None]) * sw[None, :] + b[None, :]).to(torch.bfloat16))
    x = _rand((m, k // 2), torch.float32, seed=m).to(gpu)
    wf = _rand((n, k // 2), torch.float32, seed=n, scale=0.05).to(gpu)
    xb, wb = kernels.bf16_rows(x, k // 2), kernels.bf16_rows(wf, k // 2)
    yp = kernels.mm_bf16(xb, wb, None, torch.float32)
    kernels.tile_set("bf16", m, n, k // 2, "t256x256w8")
    yw = kernels.mm_bf16(xb, wb, None, torch.float32)
    assert torch.equal(yp, yw), "ping-pong and 8-wave bf16 sums differ"


@pytest.mark.parametrize("tile", ["small_w1", "small_w2", "small_w4", "small_w8", "small_w16", "t64x64", "t128x128"])
def test_tiles_forced_decode(gpu, tile, tile_table):
    """Decode-sized and mid-sized GEMMs with a forced tile: the small-M kernel at every width (also
    above 64 rows) and the tile engine below 64 rows; int32 sums, the fused bf16 dequant and the
    bf16 GEMM against the oracle. An entry for another shape leaves the rule in place."""
    from torch_xdna import kernels

    for m, n, k in [(1, 520, 4160), (16, 1000, 208), (100, 264, 1040)]:
        kernels.tile_set("i8", m, n, k, tile)
        kernels.tile_set("bf16", m, n, k // 2, tile)
        a, w = _i8((m, k), seed=m + k), _i8((n, k), seed=n + k)
        acc = c_oracle.gemm_i32(a.numpy(), w.numpy())
        assert np.array_equal(_np(kernels.mm_i8(a.to(gpu), w.to(gpu))), acc), (tile, m, n, k)
        sx, sw = torch.rand(m) + 0.01, torch.rand(n) + 0.01
        b = torch.randn(n)
        y = kernels.mm_i8_dequant(a.to(gpu), sx.to(gpu), w.to(gpu), sw.to(gpu), b.to(gpu), torch.bfloat16)
        assert np.array_equal(_f32(y), O.to_bf16(O.dequant(acc, sx.numpy(), sw.numpy(), b.numpy()))), (tile, m, n, k)
        x = _rand((m, k // 2), torch.float32, seed=m + k)
        wf = _rand((n, k // 2), torch.float32, seed=n + k, scale=0.05)
        yb = kernels.mm_bf16(kernels.bf16_rows(x.to(gpu), k // 2), kernels.bf16_rows(wf.to(gpu), k // 2), None,
                             torch.float32)
        want, bound = O.gemm_bf16(x.numpy(), wf.numpy())
        _bf16_bracket(_f32(yb), want, bound, "f32")
    assert kernels.tile_get(gpu, "i8", 1, 520, 4160) == tile
    assert kernels.tile_get(gpu, "i8", 1, 520, 4176) == "gemv_w4"      # not in the table: the rule
    assert kernels.tile_get(gpu, "i8", 16, 520, 4176).startswith("small_w")
    kernels.tile_set("i8", 1, 520, 4160, "auto")
    assert kernels.tile_get(gpu, "i8", 1, 520, 4160) == "gemv_w4"


@pytest.mark.parametrize("tile", ["gemv_w4", "gemv_w2", "gemv_w8"])
def test_gemv_one_row(gpu, tile, tile_table):
    """The one-row kernel (M = 1: 16 K segments on the MFMA's 16 columns, the trace summed): int32 sums,
    the fused dequant to every output dtype with and without bias, and the bf16 GEMM, against the
    oracle, for K from one 16-byte chunk to more than one 16 KB round and N not a multiple of the
    waves per workgroup. Forced on more rows, the tile falls back to the rule with the same results."""
    from torch_xdna import kernels

    for n, k in [(520, 16), (1001, 1040), (264, 4160), (300, 4096), (97, 4112), (130, 16400), (3, 14336)]:
        for m in (1, 3):
            kernels.tile_set("i8", m, n, k, tile)
            kernels.tile_set("bf16", m, n, k // 2 if k >= 32 else 8, tile)
            a, w = _i8((m, k), seed=m + k + n), _i8((n, k), seed=n + k)
            acc = c_oracle.gemm_i32(a.numpy(), w.numpy())
            assert np.array_equal(_np(kernels.mm_i8(a.to(gpu), w.to(gpu))), acc), (tile, m, n, k)
            sx, sw = torch.rand(m) + 0.01, torch.rand(n) + 0.01
            b = torch.randn(n)
            for out in ("f32", "bf16", "f16"):
                for bias in (b, None):
                    y = kernels.mm_i8_dequant(a.to(gpu), sx.to(gpu), w.to(gpu), sw.to(gpu),
                                              None if bias is None else bias.to(gpu), DT[out])
                    want = O.dequant(acc, sx.numpy(), sw.numpy(), None if bias is None else bias.numpy())
                    assert np.array_equal(_f32(y), O.to_dtype(want, out)), (tile, m, n, k, out, bias is None)
            kb = k // 2 if k >= 32 else 8
            x = _rand((m, kb), torch.float32, seed=m + k)
            wf = _rand((n, kb), torch.float32, seed=n + k, scale=0.05)
            bb = _rand((n,), torch.float32, seed=n, scale=0.1)
            yb = kernels.mm_bf16(kernels.bf16_rows(x.to(gpu), kb), kernels.bf16_rows(wf.to(gpu), kb), bb.to(gpu),
                                 torch.float32)
            want, bound = O.gemm_bf16(x.numpy(), wf.numpy(), bb.numpy())
            _bf16_bracket(_f32(yb), want, bound, "f32")
    assert kernels.tile_get(gpu, "i8", 1, 264, 4160) == tile


@pytest.mark.parametrize("tile", ["seg4_r2", "seg4_r4"])
def test_seg4_few_rows(gpu, tile, tile_table):
    """The few-row kernel (M <= 16: 4 weight rows x 4 K segments on the MFMA's rows, 4 activation rows x 4
    segments on its columns, quad sums): int32 sums, the fused dequant with and without bias and the bf16
    GEMM against the oracle, for every activation group count, K from one 16-byte chunk to 14336 bytes
    (partial steps and rounds), N not a multiple of the columns per workgroup; 17 rows fall back to the
    rule."""
    from torch_xdna import kernels

    for m, n, k in [(2, 520, 16), (3, 1001, 272), (4, 64, 1040), (5, 300, 4112), (8, 97, 2064), (11, 130, 14336),
                    (16, 1001, 4096), (16, 8, 256), (17, 200, 1040)]:
        kernels.tile_set("i8", m, n, k, tile)
        kb = max(8, k // 2)
        kernels.tile_set("bf16", m, n, kb, tile)
        a, w = _i8((m, k), seed=3 * m + k + n), _i8((n, k), seed=n + 2 * k)
        acc = c_oracle.gemm_i32(a.numpy(), w.numpy())
        assert np.array_equal(_np(kernels.mm_i8(a.to(gpu), w.to(gpu))), acc), (tile, m, n, k)
        sx, sw = torch.rand(m) + 0.01, torch.rand(n) + 0.01
        b = torch.randn(n)
        for out in ("f32", "bf16", "f16"):
            for bias in (b, None):
                y = kernels.mm_i8_dequant(a.to(gpu), sx.to(gpu), w.to(gpu), sw.to(gpu),
                                          None if bias is None else bias.to(gpu), DT[out])
                want = O.dequant(acc, sx.numpy(), sw.numpy(), None if bias is None else bias.numpy())
                assert np.array_equal(_f32(y), O.to_dtype(want, out)), (tile, m, n, k, out, bias is None)
        x = _rand((m, kb), torch.float32, seed=m + k)
        wf = _rand((n, kb), torch.float32, seed=n + k, scale=0.05)
        bb = _rand((n,), torch.float32, seed=n, scale=0.1)
        yb = kernels.mm_bf16(kernels.bf16_rows(x.to(gpu), kb), kernels.bf16_rows(wf.to(gpu), kb), bb.to(gpu),
                             torch.float32)
        want, bound = O.gemm_bf16(x.numpy(), wf.numpy(), bb.numpy())
        _bf16_bracket(_f32(yb), want, bound, "f32")
    assert kernels.tile_get(gpu, "i8", 16, 1001, 4096) == tile


def test_sweep_tool(gpu, tile_table, tmp_path):
    """python -m torch_xdna.sweep on small shapes of each kind: one exact, timed JSONL line per
    candidate tile; resuming skips finished lines; --summary writes a table the runtime can load."""
    import json

    from torch_xdna import sweep

    out = str(tmp_path / "sweep.jsonl")
    sweep.main(["--kind", "i8", "--rows", "16", "300", "--shapes", "520x256", "--out", out])
    sweep.main(["--kind", "bf16", "--rows", "300", "--shapes", "520x256", "--out", out])
    sweep.main(["--kind", "conv", "--convs", "2x48x40x13x37", "1x16x64x9x11", "--out", out])
    n_lines = sum(1 for _ in open(out))
    sweep.main(["--kind", "i8", "--rows", "16", "300", "--shapes", "520x256", "--out", out])   # resumed: no-op
    recs = [json.loads(line) for line in open(out)]
    want = len(sweep.candidates("i8", 16)) + len(sweep.candidates("i8", 300)) + \
        len(sweep.candidates("bf16", 300)) + len(sweep.candidates("conv", 2 * 13 * 37, 40, 9 * 48)) + \
        len(sweep.candidates("conv", 9 * 11, 64, 9 * 16))
    assert any(r["tiling"] == "direct" and r["plan"][0] == "direct" for r in
               (json.loads(line) for line in open(out)))       # the direct kernels swept where they run
    assert len(recs) == n_lines == want
    assert all(r["status"] == "ok" and r["exact"] and r["gpu_us"] > 0 for r in recs), recs
    assert {r["checked_against"] for r in recs} == {"cpu"}
    # each record names the launch plan its time belongs to: the forced tile heads it
    assert all(r["plan"][0] == r["tiling"] and len(r["rule_plan"]) == 3 for r in recs), recs
    out2 = str(tmp_path / "sweep_tiles.jsonl")           # --tiles: only the named tiles
    sweep.main(["--kind", "i8", "--rows", "300", "--shapes", "520x256", "--tiles", "t64x64", "t32x32k4", "--out", out2])
    assert sorted(json.loads(line)["tiling"] for line in open(out2)) == ["t32x32k4", "t64x64"]
    table_path = str(tmp_path / "tuned.json")
    sweep.main(["--summary", out, "--table", table_path])
    doc = json.load(open(table_path))
    for kind in ("i8", "bf16", "conv"):
        for key, v in doc.get(kind, {}).items():
            assert v["tiling"] in kernels_tiles() and v["gpu_us"] < v["rule_us"]


def kernels_tiles():
    from torch_xdna import kernels

    return kernels.TILES
