"""The reference's backend cases (tests/test_backend.py in the reference) on the MI355X.

Models live on the GPU (or on the host for the drop-in case) and are compiled with
torch.compile(backend="xdna"); the HIP kernels run the GEMMs and convs. Every case checks that the
GPU actually ran (stats calls on "gpu", no fallbacks) and that the output is bit-identical to the
reference's CPU route (policy "cpu") on the same inputs.
"""
import pytest
import torch

from models import CNN, Attn, Net, OddCNN, rel_err, run

pytestmark = pytest.mark.gpu


def _stats():
    from torch_xdna import runtime

    return runtime.stats.as_dict()


@pytest.mark.parametrize("rows", [37, 300, 700])
def test_numerics(gpu, rows):
    torch.manual_seed(rows)
    net = Net().eval().to(gpu)
    x = torch.randn(rows, 200, device=gpu)
    with torch.no_grad():
        ref = net(x)
    y = run(net, x, policy="gpu", fallback="eager")
    s = _stats()
    assert s["calls"] == {"gpu": 3} and not s["fallbacks"] and s["gpu_launches"] == 3, s
    y_cpu = run(net, x, policy="cpu", fallback="eager")
    assert _stats()["calls"] == {"cpu": 3}
    assert y.device == y_cpu.device and torch.equal(y, y_cpu), "GPU and CPU int8 routes differ"
    assert rel_err(y, ref) < 0.03


def test_numerics_inductor(gpu):
    """The rest of the graph compiled by Inductor; the xdna ops are extern calls in it."""
    torch.manual_seed(1)
    net = Net().eval().to(gpu)
    x = torch.randn(300, 200, device=gpu)
    y = run(net, x, policy="gpu")
    assert _stats()["calls"] == {"gpu": 3}
    y_cpu = run(net, x, policy="cpu")
    assert rel_err(y, y_cpu) < 1e-6


def test_split_and_eager(gpu):
    """A 3-D input of 699 rows: one launch per GEMM (no row buckets), bitwise == the CPU route."""
    torch.manual_seed(2)
    net = Net().eval().to(gpu)
    x = torch.randn(3, 233, 200, device=gpu)
    y_cpu = run(net, x, policy="cpu", fallback="eager")
    y = run(net, x, policy="gpu", fallback="eager", row_buckets=(128, 256))
    s = _stats()
    assert torch.equal(y, y_cpu) and s["gpu_launches"] == 3, s


def test_host_model_on_gpu(gpu):
    """A CPU-resident model (the reference's setting): GEMMs go to the GPU with the copies,
    outputs come back to the host bit-identical to the CPU route."""
    torch.manual_seed(3)
    net = Net().eval()
    x = torch.randn(300, 200)
    y = run(net, x, policy="gpu", fallback="eager")
    s = _stats()
    assert s["calls"] == {"gpu": 3} and not s["fallbacks"], s
    assert y.device.type == "cpu" and torch.equal(y, run(net, x, policy="cpu", fallback="eager"))


def test_auto_host_model(gpu):
    """policy "auto", the reference's default (config.py:17; its case_auto, tests/test_backend.py:82-94):
    a host-resident model's GEMMs are timed on the GPU and on the CPU once per (precision, row bucket,
    N, K), three decisions are recorded, the output equals the CPU route bit for bit, and a second
    compile reuses the decisions."""
    from torch_xdna import runtime

    torch.manual_seed(12)
    net = Net().eval()
    x = torch.randn(512, 200)
    y = run(net, x, policy="auto")
    s = _stats()
    d = s["decisions"]
    assert len(d) == 3 and all(v[0] in ("gpu", "cpu") and v[1] > 0 and v[2] > 0 for v in d.values()), d
    assert sum(s["calls"].values()) == 3 and not s["fallbacks"], s
    y_cpu = run(net, x, policy="cpu")
    assert y.device.type == "cpu" and torch.equal(y, y_cpu), "policy auto and the CPU route differ"
    y2 = run(net, x, policy="auto")
    assert torch.equal(y2, y_cpu) and len(runtime.decisions) == 3


def test_auto_host_conv(gpu):
    """policy "auto" on a host-resident conv net: each of the three rewritten convs is timed on the GPU
    and the CPU on its first call (conv.py:122-138) and keeps the faster; the output equals the CPU
    route's integers bit for bit."""
    from torch_xdna import conv as xconv

    torch.manual_seed(13)
    net = CNN().eval()
    x = torch.randn(2, 64, 32, 64)
    y = run(net, x, policy="auto", fallback="eager")
    s = _stats()
    assert len(s["decisions"]) == 3 and sum(s["calls"].values()) == 3 and not s["fallbacks"], s
    assert y.device.type == "cpu"
    for _, layer in xconv._layers.values():      # the same layers and shifts, on the CPU route
        layer.device = "cpu"
    y_cpu = run(net, x, policy="auto", fallback="eager")
    assert _stats()["calls"] == {"cpu": 3}
    assert torch.equal(y, y_cpu), "policy auto and the CPU route's integers differ"


def test_fusion(gpu):
    torch.manual_seed(4)
    net = Attn().eval().to(gpu)
    x = torch.randn(200, 256, device=gpu)
    with torch.no_grad():
        ref = net(x)
    y = run(net, x, policy="gpu", fallback="eager")
    assert _stats()["calls"] == {"gpu": 2}
    y_unfused = run(net, x, policy="gpu", fallback="eager", fuse=False)
    assert _stats()["calls"] == {"gpu": 4}
    assert torch.equal(y, run(net, x, policy="cpu", fallback="eager"))
    assert rel_err(y, ref) < 0.03 and rel_err(y_unfused, ref) < 0.03


def test_silent_wrong(gpu, monkeypatch):
    from torch_xdna import kernels

    real = kernels.mm_i8_dequant

    def corrupt(a, sx, w, sw, bias, dt):
        y = real(a, sx, w, sw, bias, dt)
        if w.shape[0] == 300:
            y[0, 0] += 1
        return y

    monkeypatch.setattr(kernels, "mm_i8_dequant", corrupt)
    torch.manual_seed(5)
    net = Net().eval().to(gpu)
    x = torch.randn(300, 200, device=gpu)
    y = run(net, x, policy="gpu", fallback="eager")
    s = _stats()
    assert torch.equal(y, run(net, x, policy="cpu", fallback="eager")), "wrong GPU value reached the output"
    assert len(s["fallbacks"]) == 1 and "disagrees with the CPU" in s["fallbacks"][0][1], s["fallbacks"]
    assert s["calls"] == {"gpu": 2, "cpu": 1}, s["calls"]


def test_launch_failure(gpu, monkeypatch):
    from torch_xdna import kernels

    def boom(*a, **k):
        raise RuntimeError("simulated HIP launch error")

    monkeypatch.setattr(kernels, "mm_i8_dequant", boom)
    torch.manual_seed(6)
    net = Net().eval().to(gpu)
    x = torch.randn(300, 200, device=gpu)
    y = run(net, x, policy="gpu", fallback="eager")
    s = _stats()
    assert torch.equal(y, run(net, x, policy="cpu", fallback="eager"))
    assert s["fallbacks"] and not s["gpu_available"] and s["calls"].get("cpu") == 3, s


def _conv_graph(gpu, net, x):
    import torch_xdna

    graphs = []

    def capture(gm, example_inputs):
        torch_xdna.offload_gemms(gm, example_inputs, torch_xdna.Config(policy="gpu"))
        graphs.append(gm)
        return gm.forward

    torch._dynamo.reset()
    with torch.no_grad():
        torch.compile(net.eval().to(gpu), backend=capture)(x.to(gpu))
    return [n for n in graphs[0].graph.nodes if n.op == "call_function"]


def test_conv_pass(gpu, monkeypatch):
    """The reference's case_conv_pass (which convs are rewritten, which ReLU is fused), with the
    conv-to-conv chaining switched off; then the chained graph of the same model."""
    from torch_xdna import backend
    from torch_xdna.conv import conv3x3_int8

    x = torch.randn(1, 64, 16, 64)
    with monkeypatch.context() as m:
        m.setattr(backend, "_chain_convs", lambda gm, cid: 0)
        nodes = _conv_graph(gpu, CNN(), x)
    convs = [n for n in nodes if n.target is conv3x3_int8]
    assert [n.args[3] for n in convs] == [False, True, False]
    assert sum(n.target in (torch.relu, torch.nn.functional.relu) for n in nodes) == 1
    assert sum(n.target is torch.conv2d for n in nodes) == 1

    nodes = _conv_graph(gpu, CNN(), x)
    chains = [n for n in nodes if n.target is torch.ops.xdna.conv3x3_chain.default]
    assert len(chains) == 1 and not any(n.target is conv3x3_int8 for n in nodes)
    _, ws, bs, relus, relu_after, pools, _ = chains[0].args
    assert (len(ws), relus, relu_after, pools) == (3, [False, True, False], [True, False, False], [False] * 3)
    assert not any(backend._is_relu(n) for n in nodes) and sum(n.target is torch.conv2d for n in nodes) == 1


@pytest.mark.parametrize("net_cls,shape,ncalls", [(CNN, (2, 64, 32, 64), 3), (OddCNN, (2, 3, 13, 37), 2)])
def test_conv(gpu, net_cls, shape, ncalls):
    from torch_xdna import conv as xconv

    torch.manual_seed(7)
    net = net_cls().eval().to(gpu)
    x = torch.randn(*shape, device=gpu)
    with torch.no_grad():
        ref = net(x)
    y = run(net, x, policy="gpu", fallback="eager")
    s = _stats()
    assert s["calls"] == {"gpu": ncalls} and not s["fallbacks"], s
    assert rel_err(y, ref) < 0.05
    for _, layer in xconv._layers.values():      # the same layers and shifts, on the CPU route
        layer.device = "cpu"
    y_cpu = run(net, x, policy="gpu", fallback="eager")
    assert _stats()["calls"] == {"cpu": ncalls}
    assert torch.equal(y, y_cpu), "GPU and CPU integers differ"


def test_conv_silent_wrong(gpu, monkeypatch):
    """A wrong value from the launch a GPU graph's conv runs (conv, requantize and dequantize in one
    kernel) is caught by verify="first" on that launch: the layer moves to the CPU."""
    from torch_xdna import kernels

    real = kernels.conv3x3_dequant

    def corrupt(xq, wq, shift, relu, scale, sx, bias, out_dtype):
        y = real(xq, wq, shift, relu, scale, sx, bias, out_dtype)
        if wq.shape[0] == 32:
            y[0, 0, 0, 0] += 1
        return y

    monkeypatch.setattr(kernels, "conv3x3_dequant", corrupt)
    torch.manual_seed(8)
    net = CNN().eval().to(gpu)
    x = torch.randn(1, 64, 32, 64, device=gpu)
    with torch.no_grad():
        ref = net(x)
    y = run(net, x, policy="gpu", fallback="eager")
    s = _stats()
    assert len(s["fallbacks"]) == 1 and "disagrees with the CPU" in s["fallbacks"][0][1], s["fallbacks"]
    assert s["calls"] == {"gpu": 2, "cpu": 1}, s["calls"]
    assert rel_err(y, ref) < 0.05


def test_ops_direct(gpu):
    """xdna::linear_i8 and xdna::conv3x3 called directly on GPU tensors (the reference's op contracts)."""
    from torch_xdna import Config, ops

    cid = ops.config_id(Config(policy="gpu", verify="off"))
    g = torch.Generator().manual_seed(9)
    w = torch.randn(300, 200, generator=g)
    xq = torch.randint(-127, 128, (37, 200), generator=g, dtype=torch.int8)
    acc, sw = torch.ops.xdna.linear_i8(xq.to(gpu), [w.to(gpu)], False, cid)
    assert acc.device.type == "cuda" and _stats()["calls"] == {"gpu": 1}
    wq = torch.round(w / (w.abs().amax(1).clamp(min=1e-8) / 127)[:, None]).clamp(-127, 127).to(torch.int8)
    assert torch.equal(acc.cpu(), torch._int_mm(xq, wq.t().contiguous()))
    wc = torch.randn(48, 3, 3, 3, generator=g)
    xc = torch.randint(-127, 128, (2, 3, 13, 37), generator=g, dtype=torch.int8)
    wg = wc.to(gpu)          # held: a layer is cached for as long as its weight lives
    for relu in (False, True):
        q, scale = torch.ops.xdna.conv3x3(xc.to(gpu), wg, relu, cid)
        from torch_xdna import conv as xconv

        layer = next(L for _, L in xconv._layers.values() if L.relu == relu)
        assert q.dtype == (torch.uint8 if relu else torch.int8) and q.shape == (2, 48, 13, 37)
        assert torch.equal(q.cpu(), layer.cpu(xc)) and torch.equal(scale.cpu(), layer.scale(torch.device("cpu")))


def test_precision_bf16(gpu):
    """precision="bf16" (runtime.py:299-313): the bf16 GEMM kernel runs on the GPU (verified on its
    first launch against the bf16 operands multiplied in float32, the reference's check) and agrees
    with the float32 CPU route to the reference's 5e-2 norm (here far closer)."""
    torch.manual_seed(11)
    net = Net().eval().to(gpu)
    x = torch.randn(300, 200, device=gpu)
    with torch.no_grad():
        ref = net(x)
    y = run(net, x, policy="gpu", fallback="eager", precision="bf16")
    s = _stats()
    assert s["calls"] == {"gpu": 3} and not s["fallbacks"] and s["gpu_launches"] == 3, s
    y_cpu = run(net, x, policy="cpu", fallback="eager", precision="bf16")
    assert _stats()["calls"] == {"cpu": 3}
    assert rel_err(y, y_cpu) < 1e-2 and rel_err(y, ref) < 1e-2
