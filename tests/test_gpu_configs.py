"""BASELINE.json configs C1-C5 on the MI355X through the public ops, against the oracle.

Every config is compared in full. C1, C2, C3, the VGG16 layers of C4 and the decode / M=256 GEMMs
of C5 against the C oracle's int32 sums and the numpy oracle; the full-size 256-channel C4 convs and
the M = 2048 / 8192 C5 GEMMs against the reference's own CPU kernels on the same integers (torch's
exact float conv of the int8 values, torch._int_mm), which finish in seconds at these sizes, with
size-independent checks beside them: exact int64 row and column checksums of the int32 GEMM
(sum_n C = A (sum_n W), sum_m C = (sum_m A) W^T) and int64 conv sums at random positions.
"""
import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import xdna_oracle as O

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _cid(**kw):
    from torch_xdna import Config, ops

    return ops.config_id(Config(**kw))


def _stats():
    from torch_xdna import runtime

    return runtime.stats.as_dict()


def test_c1_single_linear(gpu):
    g = _gen(0)
    x = torch.randn(128, 1024, generator=g)
    w = torch.randn(3072, 1024, generator=g) * 0.02
    b = torch.randn(3072, generator=g) * 0.01
    y = torch.ops.xdna.linear(x.to(gpu), w.to(gpu), b.to(gpu), False, _cid(policy="gpu", verify="off"))
    assert _stats()["calls"] == {"gpu": 1}
    xq, sx = O.quant_rows(x.numpy())
    wq, sw = O.quant_rows(w.numpy())
    want = O.dequant(c_oracle.gemm_i32(xq, wq), sx, sw, b.numpy())
    assert np.array_equal(y.cpu().numpy(), want)


@pytest.mark.parametrize("N,K", [(4096, 4096), (14336, 4096), (4096, 14336)])
def test_c5_decode_one_row_op(gpu, N, K):
    """xdna::linear and xdna::linear_cat at one row (decode) on C5's weights: the route runs the one launch
    that quantizes the row itself (xdna_linear_row), verified against the CPU route on every call, and its
    outputs equal the oracle's bit for bit."""
    from torch_xdna import runtime

    g = _gen(N + K)
    x = torch.randn(1, K, generator=g).to(torch.bfloat16)
    w = torch.randn(N, K, generator=g) * 0.02
    b = torch.randn(N, generator=g) * 0.01
    runtime._verified.clear()
    cid = _cid(policy="gpu", verify="always")
    y = torch.ops.xdna.linear(x.to(gpu), w.to(gpu), b.to(gpu), False, cid)
    halves = [w[:N // 2], w[N // 2:]]
    y2 = torch.ops.xdna.linear_cat(x.to(gpu), [h.to(gpu) for h in halves], [b[:N // 2].to(gpu), b[N // 2:].to(gpu)],
                                   cid)
    assert _stats()["calls"] == {"gpu": 2}
    assert any(k[0] == "row" for k in runtime._verified), "the one-row launch did not run"
    xq, sx = O.quant_rows(x.float().numpy())
    wq, sw = O.quant_rows(w.numpy())
    want = O.to_bf16(O.dequant(c_oracle.gemm_i32(xq, wq), sx, sw, b.numpy()))
    assert y.dtype == torch.bfloat16 and np.array_equal(y.float().cpu().numpy(), want)
    wq2, sw2 = O.weight_quant_cat([h.numpy() for h in halves])
    want2 = O.to_bf16(O.dequant(c_oracle.gemm_i32(xq, wq2), sx, sw2, b.numpy()))
    assert np.array_equal(y2.float().cpu().numpy(), want2)


@pytest.mark.parametrize("M", [128, 512, 1024, 3000])
def test_c2_linear_cat(gpu, M):
    g = _gen(M)
    x = torch.randn(M, 1024, generator=g).to(torch.bfloat16)
    xd = torch.randn(M, 3072, generator=g).to(torch.bfloat16)
    qkv = [torch.randn(n, 1024, generator=g) * 0.02 for n in (2048, 1024, 1024)]
    gu = [torch.randn(3072, 1024, generator=g) * 0.02 for _ in range(2)]
    down = torch.randn(1024, 3072, generator=g) * 0.02
    cid = _cid(policy="gpu", verify="off")
    for inp, ws in ((x, qkv), (x, gu), (xd, [down])):
        if len(ws) > 1:
            y = torch.ops.xdna.linear_cat(inp.to(gpu), [w.to(gpu) for w in ws], [None] * len(ws), cid)
        else:
            y = torch.ops.xdna.linear(inp.to(gpu), ws[0].to(gpu), None, False, cid)
        xq, sx = O.quant_rows(inp.float().numpy())
        wq, sw = O.weight_quant_cat([w.numpy() for w in ws])
        want = O.to_bf16(O.dequant(c_oracle.gemm_i32(xq, wq), sx, sw))
        got = y.float().cpu().numpy()
        assert y.dtype == torch.bfloat16 and np.array_equal(got, want), f"{(got != want).sum()} differ"
    assert _stats()["calls"] == {"gpu": 3}


def test_c3_conv_chain(gpu):
    """4 x (conv3x3 256->256 + ReLU) on 1x256x64x64 through torch.compile, each layer's shift fixed on
    its first call, against the oracle's chain (quantize -> conv -> requant -> dequantize per layer)."""
    from models import VGGBlock, run

    torch.manual_seed(0)
    net = VGGBlock(256, 4).eval()
    for i, c in enumerate(net.convs):           # distinct weights per layer
        with torch.no_grad():
            c.weight.copy_(torch.randn(c.weight.shape, generator=_gen(11 + i)) * 0.02)
    x = torch.randn(1, 256, 64, 64, generator=_gen(12))
    y = run(net.to(gpu), x.to(gpu), policy="gpu", fallback="eager")
    s = _stats()
    assert s["calls"] == {"gpu": 4} and not s["fallbacks"], s
    h = x.numpy()
    for c in net.convs:
        xq, sx = O.conv_quant_images(h)
        wq, sw = O.conv_weight_quant(c.weight.detach().cpu().numpy())
        acc = c_oracle.conv3x3_acc(xq, wq)
        shift = O.calibrate_shift(acc[0], True)
        h = O.conv_dequant(O.requant(acc, shift, True), O.conv_scale(sw, shift), sx)
    assert np.array_equal(y.cpu().numpy(), h)


def _oracle_stack(net, x, dtype):
    """VGGStack through the oracle: per conv quantize -> int32 sums -> shift -> requant -> dequant
    (+ bias) -> cast, then the graph's ReLU / max-pool, as the unchained layers compute it."""
    h = x
    mods = list(net.features) + [torch.nn.ReLU()]
    i = 0
    while i < len(mods):
        m = mods[i]
        if isinstance(m, torch.nn.Conv2d):
            fused = m.bias is None and isinstance(mods[i + 1], torch.nn.ReLU)
            xq, sx = O.conv_quant_images(h)
            wq, sw = O.conv_weight_quant(m.weight.detach().cpu().numpy())
            acc = c_oracle.conv3x3_acc(xq, wq)
            shift = O.calibrate_shift(acc[0], fused)
            b = None if m.bias is None else m.bias.detach().cpu().numpy()
            h = O.to_dtype(O.conv_dequant(O.requant(acc, shift, fused), O.conv_scale(sw, shift), sx, b), dtype)
            i += 2 if fused else 1
            continue
        h = np.maximum(h, 0) if isinstance(m, torch.nn.ReLU) else O.max_pool2(h)
        i += 1
    return h


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_conv_chain_vgg_stack(gpu, dtype):
    """A VGG-style stack (biased convs with graph ReLUs, a fused ReLU, 2x2 max-pools, 40 / 48-channel
    layers) compiled into one xdna::conv3x3_chain: the int8 activation stays on the GPU between the
    convs, and the output equals the oracle's unchained composition bit for bit."""
    from models import VGGStack, run
    from torch_xdna import conv as xconv

    torch.manual_seed(5)
    net = VGGStack().eval()
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16}[dtype]
    x = torch.randn(3, 3, 36, 30, generator=_gen(21))
    xconv._layers.clear()
    y = run(net.to(gpu, tdt), x.to(gpu, tdt), policy="gpu", fallback="eager")
    s = _stats()
    assert s["calls"] == {"gpu": 5} and not s["fallbacks"], s
    net_f = net.float().cpu()
    want = _oracle_stack(net_f, O.to_dtype(x.numpy(), dtype), dtype)
    assert y.shape == want.shape
    assert np.array_equal(y.float().cpu().numpy(), want)


def _sampled_conv_check(xq_nchw, wq, q_nhwc, shift, relu, n_samples, seed):
    rng = np.random.default_rng(seed)
    nb, ci, h, w = xq_nchw.shape
    co = wq.shape[0]
    xp = np.zeros((nb, ci, h + 2, w + 2), np.int64)
    xp[:, :, 1:h + 1, 1:w + 1] = xq_nchw
    wl = wq.astype(np.int64)
    for _ in range(n_samples):
        b, y, x, o = rng.integers(nb), rng.integers(h), rng.integers(w), rng.integers(co)
        acc = int((xp[b, :, y:y + 3, x:x + 3] * wl[o]).sum())
        want = O.requant(np.array([acc]), shift, relu)[0]
        assert q_nhwc[b, y, x, o] == want, (b, y, x, o)


@pytest.mark.parametrize("shape", [(1, 256, 1536, 64), (8, 256, 256, 256)])
def test_c4_large_conv(gpu, shape):
    """C4's 256-channel convs at full size: the quantized images, the calibration max and every
    requantized output against the reference's CPU route (torch's exact float conv of the integers,
    oracle/cpu_route.py), plus sampled int64 sums as an independent check."""
    from oracle import cpu_route
    from torch_xdna import kernels

    nb, c, h, w = shape
    x = torch.randn(*shape, generator=_gen(21))
    wt = torch.randn(c, c, 3, 3, generator=_gen(22)) * 0.02
    xq, sx = kernels.conv_quant(x.to(gpu), c)
    wq, sw = kernels.conv_weight_pack(wt.to(gpu), c)
    top = kernels.conv3x3_calibrate(xq[:1], wq, True)
    shift = O.shift_from_top(float(top), True)
    q = kernels.conv3x3(xq, wq, shift, True)
    xq_nchw = xq.permute(0, 3, 1, 2).cpu()
    # quantize parity in full (numpy oracle)
    xq_r, sx_r = O.conv_quant_images(x.numpy())
    assert np.array_equal(xq_nchw.numpy(), xq_r) and np.array_equal(sx.cpu().numpy(), sx_r)
    # the reference's CPU route on the same integers: calibration max of image 0, then every output
    ref = cpu_route.ConvLayerCPU(wt, True)
    assert torch.equal(ref.wq, wq.view(c, 3, 3, c).permute(0, 3, 1, 2).cpu())
    acc0 = ref.acc(xq_nchw[:1])
    assert top == int(acc0.clamp(min=0).max())
    ref.calibrate(xq_nchw[0])
    assert ref.shift == shift
    want = ref(xq_nchw)
    got = q.permute(0, 3, 1, 2).cpu()
    assert torch.equal(got, want), f"{int((got != want).sum())} of {want.numel()} differ"
    wq_ref = ref.wq.numpy()
    _sampled_conv_check(xq_r, wq_ref, q.cpu().numpy(), shift, True, 500, seed=1)
    # the op's fused conv + dequantize (one launch, the tail split included; above 128 MB of output its
    # stores are non-temporal) against the reference's CPU dequantize of the CPU route's integers
    # (cpu_route.conv_dequant, conv.py:48-51) and against the two-launch form
    scale = torch.from_numpy(O.conv_scale(sw.cpu().numpy(), shift)).to(gpu)
    bias = (torch.randn(c, generator=_gen(23)) * 0.1).to(gpu)
    y1 = kernels.conv3x3_dequant(xq, wq, shift, True, scale, sx, bias, torch.float32)
    assert torch.equal(scale.cpu(), ref.scale)
    y_ref = cpu_route.conv_dequant(want, ref.scale, sx.cpu().view(-1, 1, 1, 1), bias.cpu(), torch.float32)
    y1c = y1.cpu()
    assert torch.equal(y1c, y_ref), f"{int((y1c != y_ref).sum())} of {y_ref.numel()} differ"
    del y1c, y_ref
    y2 = kernels.conv_dequant(q, True, scale, sx, bias, torch.float32)
    assert torch.equal(y1, y2), f"{int((y1 != y2).sum())} of {y2.numel()} differ"


@pytest.mark.parametrize("shape", [(1, 256, 1536, 64), (8, 256, 256, 256)])
def test_c4_op_full_size(gpu, shape):
    """The op xdna::conv3x3_fused as a GPU graph calls it, at C4's full sizes, twice on one layer: the first
    call quantizes, calibrates the shift on image 0, runs the fused conv + dequantize launch and compares
    it with the CPU composite (verify "first"); the second reuses the layer. Both outputs equal the
    reference composite on the CPU (oracle/cpu_route.py: quantize, exact conv, shift, dequantize), bit for
    bit, with no fallback."""
    from oracle import cpu_route
    from torch_xdna import Config, conv, ops, runtime

    conv._layers.clear()
    runtime.stats.reset()
    cid = ops.config_id(Config(policy="gpu", verify="first"))
    c = shape[1]
    wt = torch.randn(c, c, 3, 3, generator=_gen(31)) * 0.02
    ref = cpu_route.ConvLayerCPU(wt, True)
    wg = wt.to(gpu)
    for seed in (32, 33):
        x = torch.randn(*shape, generator=_gen(seed))
        y = torch.ops.xdna.conv3x3_fused(x.to(gpu), wg, None, True, cid).cpu()
        xq, sx = cpu_route.conv_quant(x)
        if ref.shift is None:
            ref.calibrate(xq[0])
        want = cpu_route.conv_dequant(ref(xq), ref.scale, sx, None, torch.float32)
        assert torch.equal(y, want), f"{int((y != want).sum())} of {want.numel()} differ"
        del x, y, xq, want
    layer = conv._layer(wg, shape[2], shape[3], True)
    assert layer.shift == ref.shift and layer.device == "gpu" and layer.checked == {"fused"}
    s = runtime.stats.as_dict()
    assert s["calls"] == {"gpu": 2} and not s["fallbacks"], s


# VGG16's thirteen 3x3 convs have these nine distinct (Ci, Co, H=W) shapes
VGG16_LAYERS = [(3, 64, 224), (64, 64, 224), (64, 128, 112), (128, 128, 112), (128, 256, 56), (256, 256, 56),
                (256, 512, 28), (512, 512, 28), (512, 512, 14)]


@pytest.mark.parametrize("ci,co,hw", VGG16_LAYERS)
def test_c4_vgg16_layer(gpu, ci, co, hw):
    """C4's VGG16 layers at batch 8 with ReLU: the quantized images and packed weights, the GPU
    calibration max on image 0 (it must give the oracle's shift), and every requantized output of the
    batch, against the C oracle's exact sums."""
    from torch_xdna import kernels

    g = _gen(ci * 1000 + hw)
    x = torch.randn(8, ci, hw, hw, generator=g)
    wt = torch.randn(co, ci, 3, 3, generator=g) * 0.02
    c_pad = kernels.round_up(ci, 16)
    xq, sx = kernels.conv_quant(x.to(gpu), c_pad)
    wq, sw = kernels.conv_weight_pack(wt.to(gpu), c_pad)
    xq_r, sx_r = O.conv_quant_images(x.numpy())
    wq_r, sw_r = O.conv_weight_quant(wt.numpy())
    assert np.array_equal(xq[..., :ci].permute(0, 3, 1, 2).cpu().numpy(), xq_r)
    assert not xq[..., ci:].any() and np.array_equal(sx.cpu().numpy(), sx_r)
    wq_g = wq.view(co, 3, 3, c_pad)
    assert np.array_equal(wq_g[..., :ci].permute(0, 3, 1, 2).cpu().numpy(), wq_r) and not wq_g[..., ci:].any()
    assert np.array_equal(sw.cpu().numpy(), sw_r)
    acc = c_oracle.conv3x3_acc(xq_r, wq_r)
    shift = O.calibrate_shift(acc[0], True)
    assert kernels.conv3x3_calibrate(xq[:1], wq, True) == int(np.maximum(acc[0], 0).max())
    q = kernels.conv3x3(xq, wq, shift, True)
    assert np.array_equal(q.permute(0, 3, 1, 2).cpu().numpy(), O.requant(acc, shift, True))


@pytest.mark.parametrize("M,N,K", [(8192, 14336, 4096), (8192, 4096, 14336), (8192, 4096, 4096),
                                   (2048, 14336, 4096), (2048, 4096, 14336), (2048, 4096, 4096)])
def test_c5_large_gemm(gpu, M, N, K):
    """C5's M = 2048 / 8192 GEMMs at full size: the quantized activation in full (numpy oracle), every
    int32 sum against torch._int_mm on the CPU (the reference's CPU kernel, runtime.py:162-163), every
    fused bf16 output against the reference's CPU dequantize of those sums, and exact int64 row /
    column checksums as an independent check of the sums."""
    from torch_xdna import kernels

    g = _gen(M + N + K)
    x = torch.randn(M, K, generator=g)
    x = torch.where(torch.rand(M, K, generator=g) < 1e-3, x * 20, x).to(torch.bfloat16)
    w = torch.randn(N, K, generator=g) * 0.02
    b = torch.randn(N, generator=g) * 0.01
    xq, sx = kernels.quant_rows(x.to(gpu))
    wq, sw = kernels.quant_rows(w.to(gpu))
    acc = kernels.mm_i8(xq, wq)
    y = kernels.mm_i8_dequant(xq, sx, wq, sw, b.to(gpu), torch.bfloat16)
    xq_r, sx_r = O.quant_rows(x.float().numpy())
    wq_r, sw_r = O.quant_rows(w.numpy())
    assert np.array_equal(xq.cpu().numpy(), xq_r) and np.array_equal(sx.cpu().numpy(), sx_r)
    assert np.array_equal(wq.cpu().numpy(), wq_r) and np.array_equal(sw.cpu().numpy(), sw_r)
    A, Wt = torch.from_numpy(xq_r), torch.from_numpy(wq_r)
    acc_r = torch._int_mm(A, Wt.t().contiguous())
    accg = acc.cpu()
    assert torch.equal(accg, acc_r), f"{int((accg != acc_r).sum())} int32 sums differ"
    row = accg.to(torch.int64).sum(1)
    col = accg.to(torch.int64).sum(0)
    assert torch.equal(row, A.long() @ Wt.long().sum(0)), "row checksums differ"
    assert torch.equal(col, Wt.long() @ A.long().sum(0)), "column checksums differ"
    # every bf16 output against the reference's CPU dequantize (torch ops, runtime.py:350-353) of the
    # exact sums; the numpy oracle's dequantize on a band of rows as an independent check
    sxt, swt = torch.from_numpy(sx_r), torch.from_numpy(sw_r)
    want = ((acc_r.float() * sxt[:, None]) * swt[None, :] + b[None, :]).to(torch.bfloat16)
    got = y.cpu()
    assert torch.equal(got, want), f"{int((got != want).sum())} bf16 outputs differ"
    r = slice(M // 2, M // 2 + 64)
    assert np.array_equal(got[r].float().numpy(), O.to_bf16(O.dequant(acc_r[r].numpy(), sx_r[r], sw_r, b.numpy())))


@pytest.mark.parametrize("M", [1, 16, 256])
@pytest.mark.parametrize("N,K", [(4096, 4096), (14336, 4096), (4096, 14336)])
def test_c5_decode_gemm(gpu, M, N, K):
    """C5's decode and M=256 GEMMs, every output against the C oracle."""
    from torch_xdna import kernels

    g = _gen(M * 7 + N + K)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = torch.randn(N, K, generator=g) * 0.02
    b = torch.randn(N, generator=g) * 0.01
    xq, sx = kernels.quant_rows(x.to(gpu))
    wq, sw = kernels.quant_rows(w.to(gpu))
    y = kernels.mm_i8_dequant(xq, sx, wq, sw, b.to(gpu), torch.bfloat16)
    acc = kernels.mm_i8(xq, wq)
    xq_r, sx_r = O.quant_rows(x.float().numpy())
    wq_r, sw_r = O.quant_rows(w.numpy())
    acc_r = c_oracle.gemm_i32(xq_r, wq_r)
    assert np.array_equal(acc.cpu().numpy(), acc_r)
    assert np.array_equal(y.float().cpu().numpy(), O.to_bf16(O.dequant(acc_r, sx_r, sw_r, b.numpy())))
