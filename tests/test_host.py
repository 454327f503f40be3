"""Host logic on the CPU: options, the FX pass, routing, verify, fallback and stats.

The cases follow the reference's tests/test_backend.py (case_fusion, case_no_npu, case_numerics,
case_auto, case_silent_wrong, case_launch_failure, case_conv_pass, case_conv, case_conv_odd,
case_conv_silent_wrong). Cases that need a device run here against tests/fake_device.py (the
kernels' contracts computed by the oracle on the CPU); tests/test_gpu_backend.py runs them on the
MI355X with the real HIP kernels.
"""
import pytest
import torch

import fake_device
from models import CNN, Attn, Net, OddCNN, VGGStack, rel_err, run

torch.manual_seed(0)


# ------------------------------------------------------------------------------ options
def test_config_options():
    from torch_xdna import Config, set_config

    c = Config()
    assert c.policy == "auto" and c.min_rows == 16 and c.row_buckets == (128, 256, 512, 1024)
    assert Config(policy="npu").policy == "gpu" and Config(policy="npu") == Config(policy="gpu")
    assert c.merged({"row_buckets": [512, 128]}).row_buckets == (128, 512)
    with pytest.raises(AssertionError, match="unknown xdna options"):
        c.merged({"bogus": 1})
    with pytest.raises(AssertionError):
        Config(policy="tpu")
    with pytest.raises(AssertionError):
        Config(row_buckets=(100,))
    old = set_config(verbose=True)
    assert old.verbose
    set_config(verbose=False)


def test_backend_registered():
    import torch_xdna  # noqa: F401
    from torch._dynamo.backends.registry import _BACKENDS

    assert "xdna" in _BACKENDS


# ------------------------------------------------------------------------------ CPU-only cases
def test_fusion():
    """q/k/v -> one GEMM: 2 calls instead of 4 (reference case_fusion, runs without a device)."""
    from torch_xdna import runtime

    net = Attn().eval()
    x = torch.randn(200, 256)
    with torch.no_grad():
        ref = net(x)
    y = run(net, x, policy="cpu")
    fused = runtime.stats.as_dict()["calls"]
    y_unfused = run(net, x, policy="cpu", fuse=False)
    unfused = runtime.stats.as_dict()["calls"]
    assert fused == {"cpu": 2} and unfused == {"cpu": 4}, (fused, unfused)
    assert rel_err(y, ref) < 0.03 and rel_err(y_unfused, ref) < 0.03


def test_no_gpu(monkeypatch):
    """TORCH_XDNA_DISABLE_GPU=1: every GEMM on the CPU with the same int8 math, the fp kernel too,
    and convs left as float convs (reference case_no_npu)."""
    from torch_xdna import kernels, runtime

    monkeypatch.setenv("TORCH_XDNA_DISABLE_GPU", "1")
    kernels.reset()
    assert not kernels.available() and "TORCH_XDNA_DISABLE_GPU" in kernels.unavailable_reason()
    net = Net().eval()
    x = torch.randn(300, 200)
    with torch.no_grad():
        ref = net(x)
    y = run(net, x, policy="gpu", fallback="eager")
    assert runtime.stats.as_dict()["calls"] == {"cpu": 3}
    y_fp = run(net, x, policy="gpu", cpu_kernel="fp", fallback="eager")
    assert rel_err(y, ref) < 0.03 and rel_err(y_fp, ref) < 1e-5
    cnn = CNN().eval()
    xc = torch.randn(1, 64, 32, 64)
    with torch.no_grad():
        ref_c = cnn(xc)
    y_c = run(cnn, xc, policy="gpu", fallback="eager")
    assert runtime.stats.as_dict()["calls"] == {}
    assert rel_err(y_c, ref_c) < 1e-5


def test_linear_i8_op_cpu():
    """xdna::linear_i8 on the CPU route: exact int32, a fresh scale tensor, empty input."""
    from torch_xdna import Config, ops

    cid = ops.config_id(Config(policy="cpu"))
    w = torch.randn(300, 200)
    xq = torch.randint(-127, 128, (37, 200), dtype=torch.int8)
    acc, sw = torch.ops.xdna.linear_i8(xq, [w], False, cid)
    sw2 = torch.ops.xdna.linear_i8(xq, [w], False, cid)[1]
    assert sw.data_ptr() != sw2.data_ptr()
    wq = torch.round(w / sw[:, None]).clamp(-127, 127).to(torch.int8)
    assert torch.equal(acc, torch._int_mm(xq, wq.t().contiguous()))
    acc0, _ = torch.ops.xdna.linear_i8(xq[:0], [w], False, cid)
    assert acc0.shape == (0, 300) and acc0.dtype == torch.int32


def test_weight_cache_requantizes_after_inplace_update():
    from torch_xdna import runtime

    w = torch.randn(64, 32)
    a = runtime.qweight(w)
    assert runtime.qweight(w) is a
    sw_before = a.cpu()[1].clone()
    with torch.no_grad():
        w.mul_(2)
    b = runtime.qweight(w)
    assert b is not a and torch.equal(b.cpu()[1], sw_before * 2)


# ------------------------------------------------------------------------------ fake device
@pytest.fixture
def fake(monkeypatch):
    fake_device.install(monkeypatch)
    return monkeypatch


@pytest.mark.parametrize("rows", [37, 300, 700])
def test_numerics_fake(fake, rows):
    """policy gpu == policy cpu bit for bit, 3 GPU calls, close to fp32 (reference case_numerics)."""
    from torch_xdna import runtime

    net = Net().eval()
    x = torch.randn(rows, 200)
    with torch.no_grad():
        ref = net(x)
    y = run(net, x, policy="gpu", fallback="eager")
    s = runtime.stats.as_dict()
    assert s["calls"] == {"gpu": 3} and not s["fallbacks"], s
    y_cpu = run(net, x, policy="cpu", fallback="eager")
    assert torch.equal(y, y_cpu)
    assert rel_err(y, ref) < 0.03


def test_auto_fake(fake):
    """policy auto times both devices once per (precision, bucket, N, K): 3 decisions."""
    from torch_xdna import runtime

    net = Net().eval()
    x = torch.randn(512, 200)
    y = run(net, x, policy="auto", fallback="eager")
    assert torch.equal(y, run(net, x, policy="cpu", fallback="eager"))
    run(net, x, policy="auto", fallback="eager")
    d = runtime.stats.as_dict()["decisions"]
    assert len(d) == 3, d


def test_small_gemms_stay_on_cpu_for_host_tensors(fake):
    from torch_xdna import runtime

    net = Net().eval()
    run(net, torch.randn(8, 200), policy="gpu", fallback="eager")     # 8 rows < min_rows
    assert runtime.stats.as_dict()["calls"] == {"cpu": 3}


def test_silent_wrong_fake(fake):
    """A launch that returns one wrong value is caught on its first launch; that shape moves to the
    CPU and the output is still right (reference case_silent_wrong)."""
    from torch_xdna import kernels, runtime

    real = kernels.mm_i8      # host tensors: the graph runs quantize -> xdna::linear_i8 -> dequantize

    def corrupt(a, w, out=None):
        c = real(a, w)
        if w.shape[0] == 300:
            c[0, 0] += 1
        return c

    fake.setattr(kernels, "mm_i8", corrupt)
    net = Net().eval()
    x = torch.randn(300, 200)
    y = run(net, x, policy="gpu", fallback="eager")
    s = runtime.stats.as_dict()
    assert torch.equal(y, run(net, x, policy="cpu", fallback="eager"))
    assert len(s["fallbacks"]) == 1 and "disagrees with the CPU" in s["fallbacks"][0][1], s["fallbacks"]
    assert s["calls"] == {"gpu": 2, "cpu": 1}, s["calls"]


def test_precision_bf16_fake(fake):
    """precision="bf16" routes the linears to the bf16 GEMM launcher, verified on its first launch
    to the reference's 5e-2 norm against the bf16 operands in float32; a launch that disagrees moves
    that shape to the float32 CPU route (runtime.py:299-313)."""
    from torch_xdna import kernels, runtime

    net = Net().eval()
    x = torch.randn(300, 200)
    y = run(net, x, policy="gpu", fallback="eager", precision="bf16")
    s = runtime.stats.as_dict()
    assert s["calls"] == {"gpu": 3} and not s["fallbacks"], s
    y_cpu = run(net, x, policy="cpu", fallback="eager", precision="bf16")
    assert rel_err(y, y_cpu) < 1e-2
    real = kernels.mm_bf16
    fake.setattr(kernels, "mm_bf16", lambda a, w, b, dt: real(a, w, b, dt) * (2 if w.shape[0] == 300 else 1))
    y2 = run(net, x, policy="gpu", fallback="eager", precision="bf16", verify="always")   # shapes verified above
    s = runtime.stats.as_dict()
    assert len(s["fallbacks"]) == 1 and "disagrees with the CPU" in s["fallbacks"][0][1], s["fallbacks"]
    assert s["calls"] == {"gpu": 2, "cpu": 1} and rel_err(y2, y_cpu) < 1e-2, s


def test_verify_off_lets_wrong_values_through(fake):
    from torch_xdna import kernels

    real = kernels.mm_i8
    fake.setattr(kernels, "mm_i8", lambda *a: real(*a) + 1)
    net = Net().eval()
    x = torch.randn(300, 200)
    y = run(net, x, policy="gpu", fallback="eager", verify="off")
    assert not torch.equal(y, run(net, x, policy="cpu", fallback="eager"))


def test_launch_failure_fake(fake):
    """A launch that raises: the call still returns the right answer on the CPU, and after three
    failing shapes the device is retired (reference case_launch_failure)."""
    from torch_xdna import kernels, runtime

    def boom(*a, **k):
        raise RuntimeError("simulated HIP launch error")

    fake.setattr(kernels, "mm_i8", boom)
    net = Net().eval()
    x = torch.randn(300, 200)
    y = run(net, x, policy="gpu", fallback="eager")
    s = runtime.stats.as_dict()
    assert torch.equal(y, run(net, x, policy="cpu", fallback="eager"))
    assert s["fallbacks"] and not s["gpu_available"] and s["calls"].get("cpu") == 3, s
    assert "simulated HIP launch error" in s["gpu_unavailable_reason"]


def test_conv_pass_fake(fake):
    """Which convs the pass rewrites, and which ReLU it fuses (reference case_conv_pass)."""
    import torch_xdna
    from torch_xdna.conv import conv3x3_int8

    graphs = []

    def capture(gm, example_inputs):
        torch_xdna.offload_gemms(gm, example_inputs, torch_xdna.Config(policy="gpu"))
        graphs.append(gm)
        return gm.forward

    torch._dynamo.reset()
    with torch.no_grad():
        torch.compile(CNN().eval(), backend=capture)(torch.randn(1, 64, 16, 64))
    nodes = [n for n in graphs[0].graph.nodes if n.op == "call_function"]
    convs = [n for n in nodes if n.target is conv3x3_int8]
    assert [n.args[3] for n in convs] == [False, True, False], [n.args for n in convs]
    assert sum(n.target in (torch.relu, torch.nn.functional.relu) for n in nodes) == 1
    assert sum(n.target is torch.conv2d for n in nodes) == 1


@pytest.mark.parametrize("net_cls,shape,ncalls", [(CNN, (2, 64, 16, 32), 3), (OddCNN, (2, 3, 13, 37), 2)])
def test_conv_fake(fake, net_cls, shape, ncalls):
    """Convs on the (fake) device: the first launch of each layer verified, close to fp32, and the
    same integers as the CPU route (reference case_conv / case_conv_odd)."""
    from torch_xdna import conv as xconv
    from torch_xdna import runtime

    net = net_cls().eval()
    x = torch.randn(*shape)
    with torch.no_grad():
        ref = net(x)
    y = run(net, x, policy="gpu", fallback="eager")
    s = runtime.stats.as_dict()
    assert s["calls"] == {"gpu": ncalls} and not s["fallbacks"], s
    assert rel_err(y, ref) < 0.05
    for _, layer in xconv._layers.values():
        layer.device = "cpu"
    y_cpu = run(net, x, policy="gpu", fallback="eager")
    assert runtime.stats.as_dict()["calls"] == {"cpu": ncalls}
    assert torch.equal(y, y_cpu)


def test_conv_silent_wrong_fake(fake):
    from torch_xdna import kernels, runtime

    real = kernels.conv3x3

    def corrupt(xq, wq, shift, relu):
        q = real(xq, wq, shift, relu)
        if wq.shape[0] == 32:            # only c3 (128 -> 32)
            q[0, 0, 0, 0] += 1
        return q

    fake.setattr(kernels, "conv3x3", corrupt)
    net = CNN().eval()
    x = torch.randn(1, 64, 16, 32)
    with torch.no_grad():
        ref = net(x)
    y = run(net, x, policy="gpu", fallback="eager")
    s = runtime.stats.as_dict()
    assert len(s["fallbacks"]) == 1 and "disagrees with the CPU" in s["fallbacks"][0][1], s["fallbacks"]
    assert s["calls"] == {"gpu": 2, "cpu": 1}, s["calls"]
    assert rel_err(y, ref) < 0.05


def _compile_capture(net, x):
    """Compile net with the xdna passes and return (output, the rewritten graph)."""
    import torch_xdna
    from torch_xdna import runtime

    graphs = []

    def capture(gm, example_inputs):
        torch_xdna.offload_gemms(gm, example_inputs, torch_xdna.Config(policy="gpu"))
        graphs.append(gm)
        return gm.forward

    torch._dynamo.reset()
    runtime.stats.reset()
    with torch.no_grad():
        y = torch.compile(net, backend=capture)(x)
    return y, graphs[0]


@pytest.fixture
def chain_fake(fake):
    """The fake device, with its (CPU) tensors taken for GPU tensors by the conv-chaining pass and op,
    and a count of the chaining launches."""
    from torch_xdna import backend, kernels
    from torch_xdna import conv as xconv

    fake.setattr(backend, "_on_gpu", lambda x: True)
    fake.setattr(xconv, "_on_gpu", lambda t: True)
    calls = []

    def counted(*a, **k):
        calls.append(a[1:3] + (k.get("relu_y", False),))
        return fake_device.conv_requant_next(*a, **k)

    fake.setattr(kernels, "conv_requant_next", counted)
    xconv._layers.clear()
    return calls


def test_conv_chain_fake(chain_fake, fake):
    """conv -> ReLU -> conv -> ReLU -> pool -> conv(ReLU fused) -> pool -> conv -> ReLU -> conv becomes one
    xdna::conv3x3_chain, which gives the same output as the unchained layers (each calibrated from
    its own input in a fresh run)."""
    from torch_xdna import backend, runtime
    from torch_xdna import conv as xconv
    from torch_xdna.conv import conv3x3_int8

    torch.manual_seed(3)
    net = VGGStack().eval()
    x = torch.randn(2, 3, 20, 18)
    y, gm = _compile_capture(net, x)
    nodes = [n for n in gm.graph.nodes if n.op == "call_function"]
    chains = [n for n in nodes if n.target is torch.ops.xdna.conv3x3_chain.default]
    assert len(chains) == 1 and not any(n.target is conv3x3_int8 for n in nodes), nodes
    _, ws, bs, relus, relu_after, pools, _ = chains[0].args
    assert len(ws) == 5 and [b is not None for b in bs] == [True, True, False, True, True]
    assert relus == [False, False, True, False, False]
    assert relu_after == [True, True, False, True, False] and pools == [False, True, True, False, False]
    assert sum(backend._is_pool2(n) for n in nodes) == 0 and sum(backend._is_relu(n) for n in nodes) == 1
    s = runtime.stats.as_dict()
    assert s["calls"] == {"gpu": 5} and not s["fallbacks"], s
    assert chain_fake == [(False, False, True), (False, True, True), (True, True, False), (False, False, True)]
    assert y.shape == (2, 40, 5, 4)

    xconv._layers.clear()
    chain_fake.clear()
    fake.setattr(backend, "_chain_convs", lambda gm, cid: 0)
    y_parts, gm = _compile_capture(net, x)
    assert not chain_fake and sum(n.target is conv3x3_int8 for n in gm.graph.nodes) == 5
    assert torch.equal(y, y_parts)
    with torch.no_grad():
        assert rel_err(y, net(x)) < 0.05


def test_conv_chain_layer_failure_fake(chain_fake, fake):
    """A chain layer whose first launch disagrees with the CPU: it moves to the CPU and the chain runs
    as its parts, with the same result as the unchained layers."""
    from torch_xdna import kernels, runtime
    from torch_xdna import conv as xconv

    real = kernels.conv3x3

    def corrupt(xq, wq, shift, relu):
        q = real(xq, wq, shift, relu)
        if wq.shape[0] == 48:
            q[0, 0, 0, 0] += 1
        return q

    fake.setattr(kernels, "conv3x3", corrupt)
    torch.manual_seed(4)
    net = VGGStack().eval()
    x = torch.randn(1, 3, 16, 16)
    y, _ = _compile_capture(net, x)
    s = runtime.stats.as_dict()
    assert len(s["fallbacks"]) == 1 and "disagrees with the CPU" in s["fallbacks"][0][1], s["fallbacks"]
    assert s["calls"] == {"gpu": 4, "cpu": 1}, s["calls"]
    for _, layer in xconv._layers.values():
        layer.device = "cpu"
    fake.setattr(kernels, "conv3x3", real)
    y_cpu, _ = _compile_capture(net, x)
    assert torch.equal(y, y_cpu)


def test_conv_chain_fused_launch_verified_fake(chain_fake, fake):
    """The chain's last conv runs as one launch with its dequantize; under verify="first" that launch is
    what the first call compares with the CPU (not the conv alone), so a wrong value from it moves the layer
    to the CPU and the chain runs as its parts."""
    from torch_xdna import kernels, runtime
    from torch_xdna import conv as xconv

    real = kernels.conv3x3_dequant

    def corrupt(xq, wq, shift, relu, scale, sx, bias, out_dtype):
        y = real(xq, wq, shift, relu, scale, sx, bias, out_dtype)
        if wq.shape[0] == 40:           # the last conv (64 -> 40)
            y[0, 0, 0, 0] += 1
        return y

    fake.setattr(kernels, "conv3x3_dequant", corrupt)
    torch.manual_seed(5)
    net = VGGStack().eval()
    x = torch.randn(1, 3, 16, 16)
    y, _ = _compile_capture(net, x)
    s = runtime.stats.as_dict()
    assert len(s["fallbacks"]) == 1 and "one launch" in s["fallbacks"][0][1], s["fallbacks"]
    last = [L for _, L in xconv._layers.values() if L.co == 40]
    assert len(last) == 1 and last[0].device == "cpu"
    for _, layer in xconv._layers.values():
        layer.device = "cpu"
    fake.setattr(kernels, "conv3x3_dequant", real)
    y_cpu, _ = _compile_capture(net, x)
    assert torch.equal(y, y_cpu)


def test_report_text(fake):
    import torch_xdna

    run(Net().eval(), torch.randn(64, 200), policy="gpu", fallback="eager")
    text = torch_xdna.report()
    assert "GPU available: True" in text and "gpu :" in text.replace("gpu  :", "gpu :")
    assert '"gpu_launches"' in torch_xdna.report(as_json=True)
