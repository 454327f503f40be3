"""xdna::qwen3_stack on the MI355X: its HIP kernels against float64 references, and the fused op
through torch.compile against the oracle (oracle/qwen3_stack.py, pinned to transformers'
Qwen3Model) and against the model run eagerly in float32 (the reference's own check, 10%).

Tolerances: the kernels round to bf16 (GEMM operands, q / k / v, attention probabilities), so
element checks allow 2 bf16 ulps and sequence checks a relative norm of 2e-2 (bf16 carries 8 bits:
a relative error of ~4e-3 per rounding, accumulated over the layers); the fused op against the fp32
model uses the reference test's 8% bound for its bfp16 NPU path.
"""
import pytest
import torch

from models import Stack, prefix_mask, rel_err
from oracle import qwen3_stack as Q

pytestmark = pytest.mark.gpu

BF16_ULP = 2.0 ** -7


def _close_bf16(got, want, ulps=2):
    """|got - want| <= ulps bf16 ulps of |want| (plus a floor for values near 0)."""
    got, want = got.double().cpu(), want.double().cpu()
    tol = ulps * BF16_ULP * want.abs() + 1e-6
    bad = (got - want).abs() > tol
    assert not bool(bad.any()), f"{int(bad.sum())} of {want.numel()} values differ, max {float((got - want).abs().max())}"


def test_rmsnorm_bf16(gpu):
    from torch_xdna import kernels

    g = torch.Generator().manual_seed(1)
    x = torch.randn(37, 1024, generator=g) * 3
    w = 1 + 0.1 * torch.randn(1024, generator=g)
    for wt in (w, w.to(torch.bfloat16)):
        y = kernels.rmsnorm_bf16(x.to(gpu), wt.to(gpu), 1e-6)
        _close_bf16(y, Q.rms_norm(x.double(), wt.double(), 1e-6))


def test_add_rmsnorm_bf16(gpu):
    """The residual add fused into the norm: x after the launch equals x + a in float32 (torch's CPU sum),
    and the normalized output equals the separate add then norm launches bit for bit (and the float64
    norm of x + a within the bf16 tolerance), for d of 1024 and 4096 and both weight dtypes."""
    from torch_xdna import kernels

    g = torch.Generator().manual_seed(11)
    for d in (1024, 4096):
        x = torch.randn(41, d, generator=g) * 3
        a = torch.randn(41, d, generator=g)
        w = 1 + 0.1 * torch.randn(d, generator=g)
        for wt in (w, w.to(torch.bfloat16)):
            xf = x.to(gpu)
            y = kernels.add_rmsnorm_bf16(xf, a.to(gpu), wt.to(gpu), 1e-6)
            assert torch.equal(xf.cpu(), x + a)
            xs = x.to(gpu)
            kernels.add_(xs, a.to(gpu))
            assert torch.equal(y, kernels.rmsnorm_bf16(xs, wt.to(gpu), 1e-6)), (d, wt.dtype)
            _close_bf16(y, Q.rms_norm((x + a).double(), wt.double(), 1e-6))


@pytest.mark.parametrize("tile", ["t64x64", "t32x64k4", "t128x128", "t256x256w8", "small_w2", "gemv_w4", "seg4_r2"])
def test_gemm_bf16_silu(gpu, tile):
    """The gate|up GEMM with SiLU(gate) * up in its epilogue, on the interleaved weight, against the float32
    GEMM of the concatenated weight then the separate SiLU kernel, with the same tile forced on both (their
    float sums then match), bit for bit; rows from 1 to 486, ragged rows and K, and the one-row and few-row
    tiles, which the fused form replaces by the small-M kernel (there only the float64 bound is checked)."""
    from torch_xdna import kernels

    kernels.use_tuned(False)
    kernels.tile_clear()
    try:
        g = torch.Generator().manual_seed(5)
        for m, inter, k in [(1, 3072, 1024), (5, 256, 1024), (16, 260, 40), (70, 3072, 1024), (486, 3072, 1024)]:
            x = (torch.randn(m, k, generator=g)).to(torch.bfloat16)
            gate = (torch.randn(inter, k, generator=g) * 0.05).to(torch.bfloat16)
            up = (torch.randn(inter, k, generator=g) * 0.05).to(torch.bfloat16)
            kernels.tile_set("bf16", m, 2 * inter, k, tile)
            xg = x.to(gpu)
            y = kernels.mm_bf16_silu(xg, kernels.gate_up_interleaved(gate, up).to(gpu))
            assert y.shape == (m, inter) and y.dtype == torch.bfloat16
            ref = kernels.silu_mul_bf16(kernels.mm_bf16(xg, torch.cat([gate, up]).to(gpu), None, torch.float32))
            if not tile.startswith(("gemv", "seg4")):
                assert torch.equal(y, ref), (tile, m, inter, k)
            gd, ud = x.double() @ gate.double().t(), x.double() @ up.double().t()
            want = torch.nn.functional.silu(gd) * ud
            err = (y.double().cpu() - want).abs().max() / want.abs().max()
            assert err < 2e-2, (tile, m, inter, k, float(err))
            kernels.tile_set("bf16", m, 2 * inter, k, "auto")
    finally:
        kernels.tile_clear()
        kernels._tuned_applied = None


def test_qk_norm_rope(gpu):
    """q / k heads RMSNorm'd and rotated at each token's own position; v lands transposed at its column."""
    from torch_xdna import kernels

    g = torch.Generator().manual_seed(2)
    T, nh, nkv = 45, 16, 8
    qkv = torch.randn(T, (nh + 2 * nkv) * 128, generator=g)
    qw, kw = 1 + 0.1 * torch.randn(128, generator=g), 1 + 0.1 * torch.randn(128, generator=g)
    inv_freq = 1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32) / 128))
    pos = torch.randint(0, 400, (T,), generator=g, dtype=torch.int32)
    vt_col = torch.randperm(T + 19, generator=g)[:T].to(torch.int32)
    vt = torch.zeros(nkv, 128, 64, dtype=torch.bfloat16, device=gpu)
    q, k = kernels.qk_norm_rope(qkv.to(gpu), nh, nkv, qw.to(gpu), kw.to(gpu), inv_freq.to(gpu), pos.to(gpu),
                                vt_col.to(gpu), 1e-6, vt)
    x = qkv.double()
    for heads, off, w, got in ((nh, 0, qw, q), (nkv, nh * 128, kw, k)):
        h = Q.rms_norm(x[:, off:off + heads * 128].view(T, heads, 128), w.double(), 1e-6)
        ang = pos.float()[:, None] * inv_freq[None, :]                         # float32 angles
        ang = torch.cat([ang, ang], -1)[:, None, :]
        rot = torch.cat([-h[..., 64:], h[..., :64]], -1)
        _close_bf16(got, h * ang.cos().double() + rot * ang.sin().double())
    v = qkv[:, (nh + nkv) * 128:].view(T, nkv, 128).to(torch.bfloat16)
    got_v = vt.cpu()[:, :, vt_col.long()].permute(2, 0, 1)
    assert torch.equal(got_v, v)


@pytest.mark.parametrize("lens", [[1], [31, 32, 33], [100, 65, 7], [257]])
def test_attention_bf16(gpu, lens):
    """Ragged sequences (partial and single query / key blocks): each sequence's heads against the
    float64 attention of the same bf16 q / k / v."""
    from torch_xdna import kernels

    g = torch.Generator().manual_seed(sum(lens))
    nh, nkv = 16, 8
    T = sum(lens)
    q = (torch.randn(T, nh, 128, generator=g) * 2).to(torch.bfloat16)
    k = (torch.randn(T, nkv, 128, generator=g) * 2).to(torch.bfloat16)
    v = torch.randn(T, nkv, 128, generator=g).to(torch.bfloat16)
    starts, vts, s, c = [], [], 0, 0
    for n in lens:
        starts.append(s)
        vts.append(c)
        s, c = s + n, c + -(-n // 32) * 32
    vt = torch.zeros(nkv, 128, -(-c // 8) * 8, dtype=torch.bfloat16)
    for n, s0, c0 in zip(lens, starts, vts):
        vt[:, :, c0:c0 + n] = v[s0:s0 + n].permute(1, 2, 0)
    i32 = dict(dtype=torch.int32, device=gpu)
    out = kernels.attention_bf16(q.to(gpu), k.to(gpu), vt.to(gpu), torch.tensor(starts, **i32),
                                 torch.tensor(lens, **i32), torch.tensor(vts, **i32), max(lens), 128 ** -0.5)
    out = out.cpu().double()
    for n, s0 in zip(lens, starts):
        want = Q.attention(q[s0:s0 + n].double(), k[s0:s0 + n].double(), v[s0:s0 + n].double())
        assert rel_err(out[s0:s0 + n], want) < 1e-2, n


def test_silu_mul_and_add(gpu):
    from torch_xdna import kernels

    g = torch.Generator().manual_seed(3)
    gu = torch.randn(29, 2 * 3072, generator=g) * 3
    y = kernels.silu_mul_bf16(gu.to(gpu))
    gd = gu.double()
    _close_bf16(y, torch.nn.functional.silu(gd[:, :3072]) * gd[:, 3072:])
    a, b = torch.randn(1000, generator=g), torch.randn(1000, generator=g)
    ag = a.to(gpu)
    kernels.add_(ag, b.to(gpu))
    assert torch.equal(ag.cpu(), a + b)


def _stats():
    from torch_xdna import runtime

    return runtime.stats.as_dict()


def _compiled(net):
    from torch_xdna import runtime

    torch._dynamo.reset()
    runtime.stats.reset()
    return torch.compile(net, backend="xdna", options={"fallback": "eager"})


NAME = "qwen3 stack 2 layers -> 1000"


def test_stack_fused(gpu):
    """Three sequences of a 2-layer stack + biased head in one fused call: close to the oracle and to
    the fp32 model, padding rows zero, the first call checked; a causal mask runs the plain graph."""
    torch.manual_seed(4)
    net = Stack(layers=2, out=1000, bias=True).eval().to(gpu)
    L, lens = 100, [100, 70, 37]
    x = torch.randn(3, L, 1024, device=gpu)
    mask = prefix_mask(lens, L, gpu)
    m = _compiled(net)
    with torch.no_grad():
        y, ref = m(x, mask), net(x, mask)
    s = _stats()
    assert s["stacks"] == {f"{NAME} on gpu": 1} and not s["fallbacks"], s
    assert len(s["checks"]) == 1 and s["checks"][0][1] < 0.05, s["checks"]
    layers, norm, inv_freq = Q.model_weights(net.llm)
    for b, n in enumerate(lens):
        want = Q.stack_forward(x[b, :n], layers, norm, net.head.weight, net.head.bias, inv_freq)
        assert rel_err(y[b, :n].cpu(), want) < 2e-2, (b, n)
        assert rel_err(y[b, :n], ref[b, :n]) < 0.08
    assert not y[1, 70:].any() and not y[2, 37:].any(), "padding rows are not zero"
    causal = torch.tril(torch.ones(L, L, dtype=torch.bool, device=gpu)).expand(3, 1, L, L).contiguous()
    with torch.no_grad():
        y2, ref2 = m(x, causal), net(x, causal)
    assert _stats()["stacks"] == {f"{NAME} on gpu": 1, f"{NAME} on cpu": 1}
    assert rel_err(y2, ref2) < 0.05


def test_stack_silent_wrong(gpu, monkeypatch):
    """A stack whose GPU output is wrong fails its first-call check and runs the plain graph from then
    on (the reference's case_stack_silent_wrong)."""
    from torch_xdna import kernels

    real = kernels.mm_bf16

    def corrupt(a, w, bias, out_dtype):
        y = real(a, w, bias, out_dtype)
        return y * 1.5 if w.shape[0] == 1000 else y       # the head

    monkeypatch.setattr(kernels, "mm_bf16", corrupt)
    torch.manual_seed(6)
    net = Stack(layers=2, out=1000).eval().to(gpu)
    x, mask = torch.randn(2, 64, 1024, device=gpu), prefix_mask([64, 50], 64, gpu)
    m = _compiled(net)
    with torch.no_grad():
        y, ref = m(x, mask), net(x, mask)
        m(x, mask)
    s = _stats()
    assert len(s["fallbacks"]) == 1 and "disagrees with the model" in s["fallbacks"][0][1], s["fallbacks"]
    assert s["stacks"] == {f"{NAME} on cpu": 2}, s["stacks"]
    assert max(rel_err(y[0], ref[0]), rel_err(y[1, :50], ref[1, :50])) < 0.05


def test_stack_graph_replays(gpu, monkeypatch):
    """The HIP graph of a call shape (captured on its second call) replays with new inputs: every
    replay equals the eager run of the same inputs bit for bit, with other GPU work and syncs between
    the replays."""
    from torch_xdna import Config, stack

    torch.manual_seed(7)
    net = Stack(layers=2, out=300).eval().to(gpu)
    weights = {}
    for i, Lr in enumerate(net.llm.layers):
        at, mlp = Lr.self_attn, Lr.mlp
        for key, t in dict(q=at.q_proj.weight, k=at.k_proj.weight, v=at.v_proj.weight, o=at.o_proj.weight,
                           gate=mlp.gate_proj.weight, up=mlp.up_proj.weight, down=mlp.down_proj.weight,
                           input_norm=Lr.input_layernorm.weight, post_norm=Lr.post_attention_layernorm.weight,
                           q_norm=at.q_norm.weight, k_norm=at.k_norm.weight).items():
            weights[(i, key)] = t
    weights.update(norm=net.llm.norm.weight, head=net.head.weight, inv_freq=net.llm.rotary_emb.inv_freq)
    sid = stack.register(stack.Plan([], None, None, 1, None, weights, None, 2, 300, stack.MAX_TOKENS))
    cfg = Config(policy="gpu")
    lens, L = [40, 23], 40
    mask = prefix_mask(lens, L, gpu)
    xs = [torch.randn(2, L, 1024, device=gpu) for _ in range(4)]
    with torch.no_grad():
        monkeypatch.setattr(stack, "USE_GRAPHS", False)
        want = [stack.run(cfg, sid, x, mask) for x in xs]
        stack._stacks[sid].shapes.clear()
        monkeypatch.setattr(stack, "USE_GRAPHS", True)
        for rep in range(3):
            for x, w in zip(xs, want):
                got = stack.run(cfg, sid, x, mask)
                torch.cuda.synchronize()
                assert torch.equal(got, w), f"replay {rep} differs from the eager run"
                _ = (torch.randn(256, 256, device=gpu) @ torch.randn(256, 256, device=gpu)).sum().item()
    assert stack._stacks[sid].shapes[(tuple(lens), L, torch.float32, xs[0].device)].graph is not None
