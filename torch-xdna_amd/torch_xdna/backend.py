"""torch.compile(model, backend="xdna"): GEMMs and 3x3 convs against parameters run int8 on an MI355X.

The pass rewrites Dynamo's FX graph the way the reference's backend does (torch_xdna/backend.py:59-256
in the reference), so the same nodes are offloaded:

  * `F.linear(x, W, b)`, `x @ W` / `torch.mm` / `torch.matmul` / `x.matmul(W)` and
    `torch.addmm(b, x, W)` (HF Conv1D) with W a static 2-D float parameter -> xdna::linear;
  * xdna::linear nodes reading the same input (q/k/v, gate/up) -> one xdna::linear_cat + narrows;
  * with precision "int8" and cpu_kernel "int8", linear / linear_cat -> runtime.linear_int8, which
    on a CPU graph is quantize -> xdna::linear_i8 -> dequantize as graph ops and on a GPU graph the
    single fused HIP op;
  * conv2d 3x3 / stride 1 / padding 1 or "same" / dilation 1 / groups 1 with a static weight ->
    conv.conv3x3_int8, fusing the ReLU of a bias-free conv whose only user it is (only when the GPU
    route is usable and policy != "cpu").

Activation x activation GEMMs (attention) are left alone. What runs where is decided per call at
run time (runtime.py, conv.py). The rest of the graph goes to Inductor or runs eagerly.
"""

import logging
import operator

import torch
import torch.nn.functional as F

from . import config as _config
from . import kernels, ops

log = logging.getLogger("torch_xdna")

LINEAR = {torch._C._nn.linear, F.linear}
CONV2D = {torch.conv2d, F.conv2d}
RELU = {torch.relu, F.relu, torch.relu_}
MATMUL = {operator.matmul, torch.matmul}
FLOATS = (torch.float32, torch.bfloat16, torch.float16)


def _static_placeholders(gm, example_inputs):
    """Placeholders that hold parameters or buffers (weights worth quantizing once)."""
    found = set()
    phs = [n for n in gm.graph.nodes if n.op == "placeholder"]
    for node, ex in zip(phs, example_inputs):
        if isinstance(ex, torch.nn.Parameter) or "_parameters_" in node.name or "_buffers_" in node.name:
            found.add(node)
    return found


def _example(node, attr):
    if node.op == "get_attr":
        return attr(node.target)
    if node.op == "placeholder":
        return node.meta.get("example_value")
    return None


def _gemm_args(node):
    """(x, w, b, transposed) when `node` is one of the GEMM forms the pass takes, else None."""
    if node.op == "call_function" and node.target in LINEAR:
        x = node.args[0] if node.args else node.kwargs.get("input")
        w = node.args[1] if len(node.args) > 1 else node.kwargs.get("weight")
        b = node.args[2] if len(node.args) > 2 else node.kwargs.get("bias")
        return x, w, b, False
    is_mm = ((node.op == "call_function" and node.target in MATMUL | {torch.mm})
             or (node.op == "call_method" and node.target in ("matmul", "mm", "__matmul__")))
    if is_mm and len(node.args) == 2 and not node.kwargs:
        return node.args[0], node.args[1], None, True           # x @ W with W [K, N]
    if (node.op == "call_function" and node.target is torch.addmm and len(node.args) == 3
            and set(node.kwargs) <= {"beta", "alpha"} and all(node.kwargs.get(k, 1) == 1 for k in ("beta", "alpha"))):
        b, x, w = node.args                                      # bias + x @ W (HF Conv1D)
        return x, w, b, True
    return None


def offload_gemms(gm: torch.fx.GraphModule, example_inputs, cfg) -> int:
    """Rewrite offloadable GEMMs and 3x3 convs in place; return how many."""
    static = _static_placeholders(gm, example_inputs)

    def attr(target):
        obj = gm
        for part in target.split("."):
            obj = getattr(obj, part)
        return obj

    def is_param(n):
        return isinstance(n, torch.fx.Node) and (n in static or n.op == "get_attr")

    def is_weight(n):
        if not is_param(n):
            return False
        t = _example(n, attr)
        return isinstance(t, torch.Tensor) and t.dim() == 2 and t.dtype in FLOATS

    def is_bias_vector(n):
        t = n.meta.get("example_value") if isinstance(n, torch.fx.Node) else None
        return is_param(n) and isinstance(t, torch.Tensor) and t.dim() == 1

    cid = ops.config_id(cfg)
    count = 0
    for node in list(gm.graph.nodes):
        m = _gemm_args(node)
        if m is None:
            continue
        x, w, b, transposed = m
        if node.target is torch.addmm and not (b is None or is_bias_vector(b)):
            continue
        if not is_weight(w):
            continue
        with gm.graph.inserting_after(node):
            new = gm.graph.call_function(torch.ops.xdna.linear.default, (x, w, b, transposed, cid))
        new.meta.update(node.meta)
        node.replace_all_uses_with(new)
        gm.graph.erase_node(node)
        count += 1
    if cfg.fuse:
        _fuse_shared_input(gm, cid)
    if cfg.precision == "int8" and cfg.cpu_kernel == "int8":
        _quantize_in_graph(gm, cid)
    count += _offload_convs(gm, static, cid, attr, cfg)
    if cfg.fuse:
        _chain_convs(gm, cid)
    gm.graph.lint()
    gm.recompile()
    return count


def _conv_args(node):
    """(x, weight, bias, stride, padding, dilation, groups) of a conv2d call."""
    names = ("input", "weight", "bias", "stride", "padding", "dilation", "groups")
    defaults = dict(bias=None, stride=1, padding=0, dilation=1, groups=1)
    args = dict(zip(names, node.args), **node.kwargs)
    return [args.get(k, defaults.get(k)) for k in names]


def _pair(v):
    return tuple(v) if isinstance(v, (tuple, list)) else (v, v)


def _is_relu(n):
    return ((n.op == "call_function" and n.target in RELU)
            or (n.op == "call_method" and n.target in ("relu", "relu_")))


def _offload_convs(gm, static, cid, attr, cfg):
    """3x3 / stride 1 / padding 1 / groups 1 convs of a parameter weight -> conv3x3_int8 (with a lone
    ReLU of a bias-free conv fused into the requantize as unsigned saturation)."""
    from .conv import conv3x3_int8, supported

    # int8 convs only pay off on the GPU: without it, or with policy "cpu", convs stay as they are
    if cfg.policy == "cpu" or not kernels.available():
        return 0
    count = 0
    for node in list(gm.graph.nodes):
        if node.op != "call_function" or node.target not in CONV2D:
            continue
        x, w, b, stride, padding, dilation, groups = _conv_args(node)
        if (_pair(stride) != (1, 1) or (padding != "same" and _pair(padding) != (1, 1))
                or _pair(dilation) != (1, 1) or groups != 1):
            continue
        if not (isinstance(w, torch.fx.Node) and (w in static or w.op == "get_attr")):
            continue
        wt = _example(w, attr)
        xt = x.meta.get("example_value") if isinstance(x, torch.fx.Node) else None
        if not (isinstance(wt, torch.Tensor) and wt.dim() == 4 and tuple(wt.shape[2:]) == (3, 3)
                and isinstance(xt, torch.Tensor) and xt.dim() == 4 and xt.dtype in FLOATS):
            continue
        if not supported(int(wt.shape[1]), int(wt.shape[0]), int(xt.shape[2]), int(xt.shape[3])):
            continue
        users = list(node.users)
        relu = users[0] if (cfg.fuse and b is None and len(users) == 1 and _is_relu(users[0])) else None
        last = relu or node
        with gm.graph.inserting_after(last):
            new = gm.graph.call_function(conv3x3_int8, (x, w, b, relu is not None, cid))
        new.meta.update(last.meta)
        last.replace_all_uses_with(new)
        if relu is not None:
            gm.graph.erase_node(relu)
        gm.graph.erase_node(node)
        count += 1
    return count


MAXPOOL2D = {F.max_pool2d, torch.max_pool2d}


def _is_pool2(n):
    """A 2x2 / stride-2 max-pool without padding, dilation, ceil mode or returned indices."""
    if n.op != "call_function" or n.target not in MAXPOOL2D:
        return False
    names = ("input", "kernel_size", "stride", "padding", "dilation", "ceil_mode", "return_indices")
    args = dict(zip(names, n.args), **n.kwargs)
    k = args.get("kernel_size")
    s = args.get("stride")
    if s is None or (isinstance(s, (list, tuple)) and len(s) == 0):
        s = k
    try:
        return (_pair(k) == (2, 2) and _pair(s) == (2, 2) and _pair(args.get("padding", 0)) == (0, 0)
                and _pair(args.get("dilation", 1)) == (1, 1) and not args.get("ceil_mode", False)
                and not args.get("return_indices", False))
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
    graph ReLU after a biased conv, which the conv rewrite does not fuse (backend.py:161-165)."""
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
            if relu and cur.args[3]:        # a fused ReLU already: a second one changes nothing
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


def _out_features(w):
    t = w.meta.get("example_value") if isinstance(w, torch.fx.Node) else None
    return int(t.shape[0]) if isinstance(t, torch.Tensor) else None


def _fuse_shared_input(gm, cid):
    """xdna::linear nodes reading the same input -> one xdna::linear_cat + narrows (one launch)."""
    groups = {}
    for node in gm.graph.nodes:
        if node.op == "call_function" and node.target is torch.ops.xdna.linear.default and not node.args[3]:
            groups.setdefault(node.args[0], []).append(node)
    for x, members in groups.items():
        if len(members) < 2:
            continue
        weights = [m.args[1] for m in members]
        sizes = [_out_features(w) for w in weights]
        if None in sizes:
            continue
        with gm.graph.inserting_before(members[0]):
            cat = gm.graph.call_function(torch.ops.xdna.linear_cat.default,
                                         (x, weights, [m.args[2] for m in members], cid))
            start = 0
            for m, n in zip(members, sizes):
                part = gm.graph.call_function(torch.narrow, (cat, -1, start, n))
                part.meta.update(m.meta)
                m.replace_all_uses_with(part)
                start += n
        for m in members:
            gm.graph.erase_node(m)


def _quantize_in_graph(gm, cid):
    """xdna::linear / linear_cat -> runtime.linear_int8 (quantize, integer GEMM, dequantize)."""
    from .runtime import linear_int8

    for node in list(gm.graph.nodes):
        if node.op != "call_function":
            continue
        if node.target is torch.ops.xdna.linear.default:
            x, w, b, transposed, _ = node.args
            weights, biases = [w], [b]
        elif node.target is torch.ops.xdna.linear_cat.default:
            x, weights, biases, _ = node.args
            transposed = False
        else:
            continue
        with gm.graph.inserting_after(node):
            new = gm.graph.call_function(linear_int8, (x, list(weights), list(biases), transposed, cid))
        new.meta.update(node.meta)
        node.replace_all_uses_with(new)
        gm.graph.erase_node(node)


def _compile(gm, example_inputs, cfg):
    n = offload_gemms(gm, example_inputs, cfg)
    if cfg.verbose:
        log.warning("torch_xdna: %d GEMMs / convs offloadable in a graph of %d nodes (policy=%s, fallback=%s)",
                    n, len(gm.graph.nodes), cfg.policy, cfg.fallback)
    if cfg.fallback == "eager":
        return gm.forward
    from torch._inductor.compile_fx import compile_fx

    return compile_fx(gm, example_inputs)


def xdna_backend(gm: torch.fx.GraphModule, example_inputs, options=None, mode=None):
    """The torch.compile backend; `options` are torch_xdna.Config fields."""
    cfg = _config.config.merged(options)
    if cfg.stacks and cfg.policy != "cpu" and kernels.available():
        from . import stack

        plan = stack.find(gm, example_inputs)
        if plan is not None:
            # the graph twice: the stack as one GPU op, and as usual; a dispatcher picks per call
            return stack.compile_fused(gm, example_inputs, cfg, ops.config_id(cfg), plan, _compile)
    return _compile(gm, example_inputs, cfg)
