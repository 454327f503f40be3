"""xdna::qwen3_stack's host logic on the CPU: which masks the fused op takes (the reference's
stack.lengths, torch_xdna/stack.py:328-352) and which graphs the backend fuses (stack.find / _plan,
stack.py:111-241). The GPU run is in test_gpu_stack.py."""
import pytest
import torch

from models import Stack, prefix_mask
from torch_xdna import stack


def test_lengths_prefix_masks():
    assert stack.lengths(prefix_mask([5, 3, 1], 5)) == [5, 3, 1]
    m = prefix_mask([4, 2], 4)
    m[1, :, 2:, :] = False                          # padding positions that see nothing
    assert stack.lengths(m) == [4, 2]
    f = torch.where(prefix_mask([3, 2], 3), 0.0, -1e9)
    assert stack.lengths(f) == [3, 2]                # float masks: 0 sees, large negative does not
    assert stack.lengths(prefix_mask([3], 3).expand(1, 16, 3, 3)) == [3]     # heads that agree


def test_lengths_rejects_other_masks():
    L = 6
    causal = torch.tril(torch.ones(L, L, dtype=torch.bool)).expand(2, 1, L, L)
    assert stack.lengths(causal) is None
    m = prefix_mask([4], L)
    m[0, 0, 1, 4] = True                            # a valid position that sees padding
    assert stack.lengths(m) is None
    m = prefix_mask([4], L)
    m[0, 0, 5, 4] = True                            # a padding position that sees another one
    assert stack.lengths(m) is None
    heads = prefix_mask([4], L).expand(1, 2, L, L).clone()
    heads[0, 1, 0, 3] = False                       # heads that differ
    assert stack.lengths(heads) is None
    assert stack.lengths(torch.where(prefix_mask([2], 3), 0.0, -1.0)) is None   # not a large negative
    assert stack.lengths(torch.ones(2, 3, 3)) is None                          # not 4-D


def _graph(net, x, mask):
    graphs = []

    def capture(gm, example_inputs):
        graphs.append((gm, example_inputs))
        return gm.forward

    torch._dynamo.reset()
    with torch.no_grad():
        torch.compile(net, backend=capture)(x, mask)
    return graphs[0]


@pytest.fixture
def as_gpu(monkeypatch):
    """Take the CPU example tensors for GPU ones in the stack matcher."""
    monkeypatch.setattr(stack, "_on_gpu", lambda t: True)


def test_find_and_fuse(as_gpu):
    """A 2-layer Qwen3 stack + biased head is found with every weight by role, and fusing replaces the
    stack and the head by one xdna::qwen3_stack node."""
    torch.manual_seed(0)
    net = Stack(layers=2, out=40, bias=True).eval()
    gm, ex = _graph(net, torch.randn(2, 8, 1024), prefix_mask([8, 5], 8))
    plan = stack.find(gm, ex)
    assert plan is not None and plan.layers == 2 and plan.out_features == 40
    assert plan.weights[(1, "q")] is net.llm.layers[1].self_attn.q_proj.weight
    assert plan.weights[(0, "k_norm")] is net.llm.layers[0].self_attn.k_norm.weight
    assert plan.weights["head"] is net.head.weight and plan.bias is net.head.bias
    assert len(plan.tensors()) == 2 * len(stack.LAYER_KEYS) + 3
    fused = stack.copy_module(gm)
    stack.fuse(fused, plan, 0, 0)
    ops = [n for n in fused.graph.nodes if n.op == "call_function"]
    assert [n.target for n in ops] == [torch.ops.xdna.qwen3_stack.default], ops
    assert len(gm.graph.nodes) > len(fused.graph.nodes)          # the original graph is untouched


def test_find_rejects(as_gpu, monkeypatch):
    """Not fused: other widths, a head that is not a linear, and (without the GPU) host tensors."""
    from transformers import Qwen3Config, Qwen3Model

    class Narrow(torch.nn.Module):
        def __init__(self):
            super().__init__()
            cfg = Qwen3Config(hidden_size=256, intermediate_size=512, num_hidden_layers=1, num_attention_heads=4,
                              num_key_value_heads=2, head_dim=64, vocab_size=16, rms_norm_eps=1e-6,
                              attn_implementation="sdpa")
            self.llm, self.head = Qwen3Model(cfg), torch.nn.Linear(256, 8)

        def forward(self, x, mask):
            return self.head(self.llm(inputs_embeds=x, attention_mask=mask)[0])

    gm, ex = _graph(Narrow().eval(), torch.randn(1, 4, 256), prefix_mask([4], 4))
    assert stack.find(gm, ex) is None

    class NoHead(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.s = Stack(layers=1, out=8)

        def forward(self, x, mask):
            return self.s.llm(inputs_embeds=x, attention_mask=mask)[0] * 2

    gm, ex = _graph(NoHead().eval(), torch.randn(1, 4, 1024), prefix_mask([4], 4))
    assert stack.find(gm, ex) is None
    monkeypatch.setattr(stack, "_on_gpu", lambda t: t.device.type == "cuda")
    gm, ex = _graph(Stack(layers=1, out=8).eval(), torch.randn(1, 4, 1024), prefix_mask([4], 4))
    assert stack.find(gm, ex) is None


def _mutated(gm, edit):
    """A copy of gm's graph with `edit(node)` applied to every node (edit returns True when it changed one)."""
    g = stack.copy_module(gm)
    changed = sum(bool(edit(n)) for n in list(g.graph.nodes))
    assert changed, "the mutation found nothing to change"
    g.recompile()
    return g


def _set_kw(target, key, value):
    def edit(n):
        if n.op == "call_function" and target in str(n.target):
            n.kwargs = {**n.kwargs, key: value}
            return True
    return edit


def _set_float(target, old, new):
    def edit(n):
        if n.op == "call_function" and target in str(n.target) and old in n.args:
            n.args = tuple(new if a == old else a for a in n.args)
            return True
    return edit


@pytest.mark.parametrize("what,edit", [
    ("causal attention", _set_kw("scaled_dot_product_attention", "is_causal", True)),
    ("attention dropout", _set_kw("scaled_dot_product_attention", "dropout_p", 0.1)),
    ("attention scale", _set_kw("scaled_dot_product_attention", "scale", 0.5)),
    ("no mask", _set_kw("scaled_dot_product_attention", "attn_mask", None)),
    ("RMSNorm eps", _set_float("add", 1e-06, 1e-05)),
    ("RoPE scaling", _set_float("mul", 1.0, 2.0)),
])
def test_find_rejects_mutations(as_gpu, what, edit):
    """One rule broken in an otherwise fusable graph (2 layers + head): the matcher turns it down. The
    unmutated graph is found, so each case isolates its rule."""
    torch.manual_seed(2)
    net = Stack(layers=2, out=24).eval()
    gm, ex = _graph(net, torch.randn(2, 6, 1024), prefix_mask([6, 3], 6))
    assert stack.find(gm, ex) is not None
    assert stack.find(_mutated(gm, edit), ex) is None, what


def test_find_rejects_model_variants(as_gpu):
    """Stacks the op is not built for: biased attention projections, another RMSNorm eps, and a stack whose
    output has a second user besides the head; a head without bias and one with both are found."""
    from transformers import Qwen3Config, Qwen3Model

    def qwen(**kw):
        cfg = dict(hidden_size=1024, intermediate_size=3072, num_hidden_layers=1, num_attention_heads=16,
                   num_key_value_heads=8, head_dim=128, vocab_size=16, rms_norm_eps=1e-6, attn_implementation="sdpa")
        cfg.update(kw)
        return Qwen3Model(Qwen3Config(**cfg))

    class Net(torch.nn.Module):
        def __init__(self, llm, twice=False, bias=False):
            super().__init__()
            self.llm, self.head, self.twice = llm, torch.nn.Linear(1024, 8, bias=bias), twice

        def forward(self, x, mask):
            h = self.llm(inputs_embeds=x, attention_mask=mask)[0]
            return self.head(h) + h[..., :8] if self.twice else self.head(h)

    torch.manual_seed(3)
    x, mask = torch.randn(1, 5, 1024), prefix_mask([5], 5)
    for net, found in ((Net(qwen()), True), (Net(qwen(), bias=True), True),
                       (Net(qwen(attention_bias=True)), False), (Net(qwen(rms_norm_eps=1e-5)), False),
                       (Net(qwen(), twice=True), False)):
        gm, ex = _graph(net.eval(), x, mask)
        assert (stack.find(gm, ex) is not None) == found, (net.llm.config.attention_bias, net.twice)


def test_backend_keeps_host_stacks_plain():
    """Without a GPU the backend compiles a stack model as a plain graph (its linears on the CPU's
    W8A8 route): no stack op runs, and the output stays within int8 error of the float model."""
    from models import rel_err
    from torch_xdna import runtime

    torch.manual_seed(1)
    net = Stack(layers=1, out=16).eval()
    x, mask = torch.randn(2, 6, 1024), prefix_mask([6, 4], 6)
    torch._dynamo.reset()
    runtime.stats.reset()
    with torch.no_grad():
        ref = net(x, mask)
        y = torch.compile(net, backend="xdna", options={"fallback": "eager"})(x, mask)
    assert not runtime.stats.as_dict()["stacks"]
    assert rel_err(y, ref) < 0.05


def test_gate_up_interleaved():
    """The fused SiLU GEMM's weight: gate and up rows in pairs, rows 4j, 4j + 1 gate rows 2j, 2j + 1 and rows
    4j + 2, 4j + 3 up rows 2j, 2j + 1; an odd row count is refused."""
    from torch_xdna import kernels

    gate = torch.arange(6 * 3).view(6, 3).float()
    up = -gate - 1
    w = kernels.gate_up_interleaved(gate, up)
    assert w.shape == (12, 3)
    order = [("g", 0), ("g", 1), ("u", 0), ("u", 1), ("g", 2), ("g", 3), ("u", 2), ("u", 3), ("g", 4), ("g", 5),
             ("u", 4), ("u", 5)]
    for r, (which, i) in enumerate(order):
        assert torch.equal(w[r], (gate if which == "g" else up)[i]), r
    with pytest.raises(ValueError):
        kernels.gate_up_interleaved(gate[:5], up[:5])
