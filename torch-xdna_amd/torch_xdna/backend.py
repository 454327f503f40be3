"""torch.compile(model, backend="xdna"): GEMMs and 3x3 convs against parameters run int8 on an MI355X.

The pass works on Dynamo's FX graph and takes the same nodes the reference's pass takes
(torch_xdna/backend.py:59-226 in the reference), so a model offloads the same work:

  GEMM sites    `F.linear(x, W, b)`; `x @ W`, `torch.mm`, `torch.matmul`, `x.matmul(W)` / `x.mm(W)`
                with exactly two positional operands; `torch.addmm(b, x, W)` (HF Conv1D) with
                alpha = beta = 1 and b absent or a 1-D parameter. W must be a 2-D float parameter
                (or buffer). Each becomes xdna::linear.
  shared input  with `fuse`, the xdna::linear nodes of one input (q/k/v, gate/up) become one
                xdna::linear_cat whose output is narrowed back into the members' values.
  int8 lowering with precision "int8" and cpu_kernel "int8", every linear / linear_cat becomes
                runtime.linear_int8: on a CPU graph quantize -> xdna::linear_i8 -> dequantize as
                graph ops, on a GPU graph the one fused HIP op.
  conv sites    (GPU route usable, policy != "cpu") conv2d 3x3 / stride 1 / padding 1 or "same" /
                dilation 1 / groups 1 of a 4-D float input and a parameter weight within the conv
                op's channel limit -> conv.conv3x3_int8; with `fuse`, a ReLU that is the only user
                of a bias-free conv is folded in (the requantize saturates to [0, 255]).
  conv chains   with `fuse`, on GPU graphs: conv3x3_int8 -> [ReLU] [2x2 max-pool] -> conv3x3_int8
                ... with single-use intermediates -> one xdna::conv3x3_chain (int8 NHWC between
                the convs).

Activation x activation products (attention) are left alone. Which device runs each op is decided
per call at run time (runtime.py, conv.py). The rest of the graph goes to Inductor or runs eagerly.
"""

import logging
import operator
from dataclasses import dataclass
from typing import Any, Optional

import torch
import torch.nn.functional as F

from . import config as _config
from . import kernels, ops

log = logging.getLogger("torch_xdna")

FLOATS = (torch.float32, torch.bfloat16, torch.float16)

_LINEAR_FNS = frozenset({torch._C._nn.linear, F.linear})
_MM_FNS = frozenset({operator.matmul, torch.matmul, torch.mm})
_MM_METHODS = frozenset({"matmul", "mm", "__matmul__"})
_CONV_FNS = frozenset({torch.conv2d, F.conv2d})
_RELU_FNS = frozenset({torch.relu, F.relu, torch.relu_})
_RELU_METHODS = frozenset({"relu", "relu_"})
_POOL_FNS = frozenset({F.max_pool2d, torch.max_pool2d})


def _calls(n, fns=frozenset(), methods=frozenset()):
    """Whether FX node n calls one of `fns` (call_function) or one of `methods` (call_method)."""
    return (n.op == "call_function" and n.target in fns) or (n.op == "call_method" and n.target in methods)


def _is_relu(n):
    return _calls(n, _RELU_FNS, _RELU_METHODS)


def _pair(v):
    return tuple(v) if isinstance(v, (tuple, list)) else (v, v)


def _bound(n, names, defaults):
    """The call's arguments by parameter name (positional ones first), defaults filled in."""
    got = dict(defaults)
    got.update(zip(names, n.args))
    got.update(n.kwargs)
    return got


@dataclass
class _Gemm:
    """One GEMM site: y = x @ W^T + b, or x @ W (+ b) when `transposed` (W given as [K, N])."""
    node: torch.fx.Node
    x: Any
    weight: Any
    bias: Any
    transposed: bool


class _Graph:
    """An FX graph under rewrite: which values are parameters (quantized once, so worth offloading),
    the example tensor of a value, and node replacement."""

    def __init__(self, gm, example_inputs):
        self.gm = gm
        self.graph = gm.graph
        placeholders = [n for n in gm.graph.nodes if n.op == "placeholder"]
        # Dynamo lifts module parameters and buffers to placeholders named *_parameters_* / *_buffers_*
        self.params = {n for n, ex in zip(placeholders, example_inputs)
                       if isinstance(ex, torch.nn.Parameter) or "_parameters_" in n.name or "_buffers_" in n.name}

    def is_param(self, v) -> bool:
        return isinstance(v, torch.fx.Node) and (v.op == "get_attr" or v in self.params)

    def tensor(self, v, meta_only=False) -> Optional[torch.Tensor]:
        """The example tensor of graph value v: a get_attr's attribute itself, else the node's
        recorded example value."""
        if not isinstance(v, torch.fx.Node):
            return None
        if v.op == "get_attr" and not meta_only:
            obj = self.gm
            for part in v.target.split("."):
                obj = getattr(obj, part)
            t = obj
        elif v.op in ("placeholder", "get_attr") or meta_only:
            t = v.meta.get("example_value")
        else:
            t = None
        return t if isinstance(t, torch.Tensor) else None

    def param(self, v, ndim, meta_only=False) -> Optional[torch.Tensor]:
        """v's example tensor when v is a parameter of `ndim` dimensions."""
        t = self.tensor(v, meta_only) if self.is_param(v) else None
        return t if t is not None and t.dim() == ndim else None

    def substitute(self, old, target, args):
        """A call of `target` on `args` takes over the value (and metadata) of node `old`, which is erased."""
        with self.graph.inserting_after(old):
            new = self.graph.call_function(target, args)
        new.meta.update(old.meta)
        old.replace_all_uses_with(new)
        self.graph.erase_node(old)
        return new


# ------------------------------------------------------------------------------ GEMMs
def _gemm_site(g: _Graph, n) -> Optional[_Gemm]:
    """n as a GEMM against a parameter, or None."""
    if _calls(n, _LINEAR_FNS):
        a = _bound(n, ("input", "weight", "bias"), {"bias": None})
        site = _Gemm(n, a.get("input"), a.get("weight"), a["bias"], False)
    elif _calls(n, _MM_FNS, _MM_METHODS) and len(n.args) == 2 and not n.kwargs:
        site = _Gemm(n, n.args[0], n.args[1], None, True)
    elif (n.op == "call_function" and n.target is torch.addmm and len(n.args) == 3
          and set(n.kwargs) <= {"alpha", "beta"} and all(v == 1 for v in n.kwargs.values())):
        b, x, w = n.args
        if b is not None and g.param(b, 1, meta_only=True) is None:
            return None
        site = _Gemm(n, x, w, b, True)
    else:
        return None
    wt = g.param(site.weight, 2)
    return site if wt is not None and wt.dtype in FLOATS else None


def _rewrite_gemms(g: _Graph, cid) -> int:
    sites = [s for s in (_gemm_site(g, n) for n in list(g.graph.nodes)) if s is not None]
    for s in sites:
        g.substitute(s.node, torch.ops.xdna.linear.default, (s.x, s.weight, s.bias, s.transposed, cid))
    return len(sites)


def _merge_shared_inputs(g: _Graph, cid):
    """xdna::linear nodes (F.linear form) reading one input -> one xdna::linear_cat + narrows: one launch
    and one quantize of the input instead of several."""
    by_input = {}
    for n in g.graph.nodes:
        if n.op == "call_function" and n.target is torch.ops.xdna.linear.default and not n.args[3]:
            by_input.setdefault(n.args[0], []).append(n)
    for x, members in by_input.items():
        widths = [g.tensor(m.args[1], meta_only=True) for m in members]
        if len(members) < 2 or any(t is None for t in widths):
            continue
        with g.graph.inserting_before(members[0]):
            cat = g.graph.call_function(torch.ops.xdna.linear_cat.default,
                                        (x, [m.args[1] for m in members], [m.args[2] for m in members], cid))
            offset = 0
            for m, t in zip(members, widths):
                part = g.graph.call_function(torch.narrow, (cat, -1, offset, int(t.shape[0])))
                part.meta.update(m.meta)
                m.replace_all_uses_with(part)
                offset += int(t.shape[0])
        for m in members:
            g.graph.erase_node(m)


def _lower_to_int8(g: _Graph, cid):
    """linear / linear_cat -> runtime.linear_int8 (quantize, integer GEMM, dequantize)."""
    from .runtime import linear_int8

    for n in list(g.graph.nodes):
        if n.op != "call_function":
            continue
        if n.target is torch.ops.xdna.linear.default:
            x, w, b, transposed, _ = n.args
            args = (x, [w], [b], transposed, cid)
        elif n.target is torch.ops.xdna.linear_cat.default:
            x, ws, bs, _ = n.args
            args = (x, list(ws), list(bs), False, cid)
        else:
            continue
        g.substitute(n, linear_int8, args)


# ------------------------------------------------------------------------------ convs
_CONV_ARGS = ("input", "weight", "bias", "stride", "padding", "dilation", "groups")
_CONV_DEFAULTS = {"bias": None, "stride": 1, "padding": 0, "dilation": 1, "groups": 1}


def _conv_eligible(g: _Graph, a) -> bool:
    from .conv import supported

    plain = (_pair(a["stride"]) == (1, 1) and _pair(a["dilation"]) == (1, 1) and a["groups"] == 1
             and (a["padding"] == "same" or _pair(a["padding"]) == (1, 1)))
    if not plain:
        return False
    wt = g.param(a["weight"], 4)
    xt = g.tensor(a["input"], meta_only=True)
    if wt is None or tuple(wt.shape[2:]) != (3, 3) or xt is None or xt.dim() != 4 or xt.dtype not in FLOATS:
        return False
    return supported(int(wt.shape[1]), int(wt.shape[0]), int(xt.shape[2]), int(xt.shape[3]))


def _rewrite_convs(g: _Graph, cid, cfg) -> int:
    """3x3 stride-1 convs of a parameter weight -> conv3x3_int8, with a lone ReLU of a bias-free conv
    folded into the requantize (unsigned saturation)."""
    from .conv import conv3x3_int8

    # int8 convs pay off only on the GPU: without it, or with policy "cpu", they stay float convs
    if cfg.policy == "cpu" or not kernels.available():
        return 0
    count = 0
    for n in list(g.graph.nodes):
        if not _calls(n, _CONV_FNS):
            continue
        a = _bound(n, _CONV_ARGS, _CONV_DEFAULTS)
        if not _conv_eligible(g, a):
            continue
        users = list(n.users)
        fold = cfg.fuse and a["bias"] is None and len(users) == 1 and _is_relu(users[0])
        last = users[0] if fold else n
        with g.graph.inserting_after(last):
            new = g.graph.call_function(conv3x3_int8, (a["input"], a["weight"], a["bias"], fold, cid))
        new.meta.update(last.meta)
        last.replace_all_uses_with(new)
        if fold:
            g.graph.erase_node(users[0])
        g.graph.erase_node(n)
        count += 1
    return count


def _is_pool2(n):
    """A 2x2 / stride-2 max-pool without padding, dilation, ceil mode or returned indices."""
    if not _calls(n, _POOL_FNS):
        return False
    a = _bound(n, ("input", "kernel_size", "stride", "padding", "dilation", "ceil_mode", "return_indices"),
               {"stride": None, "padding": 0, "dilation": 1, "ceil_mode": False, "return_indices": False})
    stride = a["stride"]
    if stride is None or (isinstance(stride, (list, tuple)) and len(stride) == 0):
        stride = a.get("kernel_size")
    try:
        return (_pair(a.get("kernel_size")) == (2, 2) and _pair(stride) == (2, 2) and _pair(a["padding"]) == (0, 0)
                and _pair(a["dilation"]) == (1, 1) and not a["ceil_mode"] and not a["return_indices"])
    except TypeError:
        return False


def _on_gpu(x):
    """Whether graph value x is a GPU tensor (its example value's device)."""
    xt = x.meta.get("example_value") if isinstance(x, torch.fx.Node) else None
    return isinstance(xt, torch.Tensor) and xt.device.type == "cuda"


def _chain_convs(gm, cid):
    """conv3x3_int8 -> [ReLU] [2x2 max-pool] -> conv3x3_int8 -> ... where every intermediate has that
    one use -> one xdna::conv3x3_chain, on GPU graphs: the activation stays NHWC int8 from conv to conv
    (the reference lists this as its next step, results/conv3x3_cascade.md:216-222). The ReLU is the
    graph ReLU after a biased conv, which the conv rewrite does not fold (backend.py:161-165)."""
    from .conv import conv3x3_int8

    def is_conv(n):
        return n.op == "call_function" and n.target is conv3x3_int8

    def following(n):
        """(next conv, ReLU between, pool between, the nodes between) when n's value reaches a conv's
        input through single-use ReLU / 2x2 max-pool nodes (at most one of each)."""
        relu = pool = False
        between = []
        cur = n
        while True:
            users = list(cur.users)
            if len(users) != 1 or not users[0].args or users[0].args[0] is not cur:
                return None
            u = users[0]
            if is_conv(u):
                return u, relu, pool, between
            if _is_relu(u) and not relu and len(u.args) <= 2 and set(u.kwargs) <= {"inplace"}:
                relu = True
            elif _is_pool2(u) and not pool:
                pool = True
            else:
                return None
            between.append(u)
            cur = u

    taken = set()
    count = 0
    for node in list(gm.graph.nodes):
        if not is_conv(node) or node in taken or not _on_gpu(node.args[0]):
            continue
        chain, relus_after, pools, between = [node], [], [], []
        cur = node
        while True:
            nxt = following(cur)
            if nxt is None:
                break
            conv_node, relu, pooled, mid = nxt
            if relu and cur.args[3]:        # a folded ReLU already: a second one changes nothing
                relu = False
            relus_after.append(relu)
            pools.append(pooled)
            between.extend(mid)
            chain.append(conv_node)
            cur = conv_node
        if len(chain) < 2:
            continue
        relus_after.append(False)
        pools.append(False)
        taken.update(chain)
        last = chain[-1]
        args = (chain[0].args[0], [c.args[1] for c in chain], [c.args[2] for c in chain],
                [c.args[3] for c in chain], relus_after, pools, cid)
        with gm.graph.inserting_after(last):
            new = gm.graph.call_function(torch.ops.xdna.conv3x3_chain.default, args)
        new.meta.update(last.meta)
        last.replace_all_uses_with(new)
        order = {n: i for i, n in enumerate(gm.graph.nodes)}
        for dead in sorted(chain + between, key=lambda n: -order[n]):
            gm.graph.erase_node(dead)
        count += 1
    return count


# ------------------------------------------------------------------------------ entry points
def offload_gemms(gm: torch.fx.GraphModule, example_inputs, cfg) -> int:
    """Rewrite the graph's offloadable GEMMs and 3x3 convs in place; return how many sites were taken."""
    g = _Graph(gm, example_inputs)
    cid = ops.config_id(cfg)
    taken = _rewrite_gemms(g, cid)
    if cfg.fuse:
        _merge_shared_inputs(g, cid)
    if cfg.precision == "int8" and cfg.cpu_kernel == "int8":
        _lower_to_int8(g, cid)
    taken += _rewrite_convs(g, cid, cfg)
    if cfg.fuse:
        _chain_convs(gm, cid)
    gm.graph.lint()
    gm.recompile()
    return taken


def _compile(gm, example_inputs, cfg):
    """The rewritten graph, run eagerly (fallback "eager") or compiled by Inductor."""
    taken = offload_gemms(gm, example_inputs, cfg)
    if cfg.verbose:
        log.warning("torch_xdna: %d GEMM / conv sites offloadable in a graph of %d nodes (policy=%s, fallback=%s)",
                    taken, len(gm.graph.nodes), cfg.policy, cfg.fallback)
    if cfg.fallback == "eager":
        return gm.forward
    from torch._inductor.compile_fx import compile_fx

    return compile_fx(gm, example_inputs)


def xdna_backend(gm: torch.fx.GraphModule, example_inputs, options=None, mode=None):
    """The torch.compile backend registered as "xdna"; `options` are torch_xdna.Config fields. A
    transformer stack the GPU runs as one op (stack.py) is split off first: the graph is then
    compiled twice, as the fused stack and as above, and a dispatcher picks per call."""
    cfg = _config.config.merged(options)
    stack_plan = None
    if cfg.stacks and cfg.policy != "cpu" and kernels.available():
        from . import stack

        stack_plan = stack.find(gm, example_inputs)
    if stack_plan is None:
        return _compile(gm, example_inputs, cfg)
    return stack.compile_fused(gm, example_inputs, cfg, ops.config_id(cfg), stack_plan, _compile)
