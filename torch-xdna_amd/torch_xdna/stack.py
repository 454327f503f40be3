"""xdna::qwen3_stack: a Qwen3-0.6B-width transformer stack and its linear head as one op on the GPU.

Mirrors the reference's whole-stack op (torch_xdna/stack.py in the reference). The backend looks in
Dynamo's graph for a transformers `Qwen3Model` whose last hidden states feed only a linear layer,
with Qwen3-0.6B's widths (hidden 1024, 16 query / 8 key-value heads of 128, MLP 3072), any depth,
and bidirectional attention under a 4-D mask that is an input of the graph (stack.py:111-241). Such
a graph is compiled twice (stack.py:463-473):

  fused  the stack and its head replaced by xdna::qwen3_stack
  plain  the graph as the backend compiles any other

and a dispatcher picks one per call from the mask (stack.py:412-446): the fused graph when every
sequence's mask is a prefix block of 1 .. MAX_TOKENS positions followed only by padding positions
that see themselves or nothing (stack.py:328-352), the plain graph otherwise (a causal mask, for
one). The fused graph's rows for padding positions are zeros.

On the GPU the op packs the valid tokens of all sequences into one [T, 1024] float32 residual
stream and runs every layer with the HIP kernels: RMSNorm to bf16, the q/k/v, o, gate/up and down
projections on the tile engine's bf16 GEMM (float32 sums), q / k RMSNorm + RoPE, bidirectional
grouped-query attention (bf16 MFMA, online softmax in float32), SiLU * up, the residual adds; then
the final norm and the head (bias fused). The reference runs bfp16 operands on the NPU, one launch
per pair of sequences.

The first fused call of each attention shape (query blocks per sequence) is checked against the
original graph run eagerly (stack.py:448-460): the valid rows of the head's output must be within
10% (relative norm). A mismatch or a launch failure sends the stack to the plain graph for the rest
of the process.
"""

import copy
import logging
import operator
import re
import threading
import time
import weakref

import torch
import torch.nn.functional as F

from . import kernels
from .runtime import GPUResultMismatch, stats

log = logging.getLogger("torch_xdna")
_lock = threading.RLock()

LINEAR = {torch._C._nn.linear, F.linear}
SDPA = {torch._C._nn.scaled_dot_product_attention, F.scaled_dot_product_attention}
ADD = {operator.add, torch.add}
MUL = {operator.mul, torch.mul}
ROOTS = ("Qwen3Model",)
D, NH, NKV, DH, INTER, EPS = 1024, 16, 8, 128, 3072, 1e-6
LAYER_KEYS = ("q", "k", "v", "o", "gate", "up", "down", "input_norm", "post_norm", "q_norm", "k_norm")
SHAPES = dict(q=(NH * DH, D), k=(NKV * DH, D), v=(NKV * DH, D), o=(D, NH * DH), gate=(INTER, D), up=(INTER, D),
              down=(D, INTER), input_norm=(D,), post_norm=(D,), q_norm=(DH,), k_norm=(DH,))
VERIFY_TOL = 0.1
# Longest sequence the fused op takes. The reference's NPU program stops at 384 positions; the GPU
# attention streams the keys, so the cap only bounds the work of one call.
MAX_TOKENS = 4096
QBLOCK = 32                    # queries per attention wave

_PROJ = re.compile(r"layers\.(\d+)\.(?:self_attn\.(q|k|v|o)_proj|mlp\.(gate|up|down)_proj)")
_NORMS = {"input_layernorm": "input_norm", "post_attention_layernorm": "post_norm",
          "self_attn.q_norm": "q_norm", "self_attn.k_norm": "k_norm"}
_NORM = re.compile(r"layers\.(\d+)\.(" + "|".join(re.escape(k) for k in _NORMS) + ")")


# ------------------------------------------------------------------ finding a stack
class _NoStack(Exception):
    pass


class Plan:
    """A stack found in a graph. Nodes are kept by name, so the plan applies to copies."""

    def __init__(self, region, x, mask, mask_index, head, weights, bias, layers, out_features, max_tokens):
        self.region, self.x, self.mask, self.mask_index, self.head = region, x, mask, mask_index, head
        self.weights, self.bias = weights, bias       # role -> tensor; the head's bias or None
        self.layers, self.out_features, self.max_tokens = layers, out_features, max_tokens

    def tensors(self):
        """Every weight, in a fixed order: per layer LAYER_KEYS, then norm, head, inv_freq."""
        return [self.weights[(i, k)] for i in range(self.layers) for k in LAYER_KEYS] + \
            [self.weights["norm"], self.weights["head"], self.weights["inv_freq"]]


def _cls_name(c):
    return c.__name__ if isinstance(c, type) else str(c).rsplit(".", 1)[-1].strip("'>")


def _module_of(node):
    """(path, class name) of the innermost module a node ran in."""
    path, cls = list(node.meta["nn_module_stack"].values())[-1]
    return path, _cls_name(cls)


def _linear_operands(node):
    names = ("input", "weight", "bias")
    got = dict(zip(names, node.args), **{k: v for k, v in node.kwargs.items() if k in names})
    return got.get("input"), got.get("weight"), got.get("bias")


class _Params:
    """Role -> weight tensor of one stack: (layer, LAYER_KEYS name), "norm", "inv_freq", "head"."""

    def __init__(self, value):
        self.value, self.by_role = value, {}

    def is_param(self, node):
        return node.op == "placeholder" and (isinstance(self.value.get(node), torch.nn.Parameter)
                                             or "_parameters_" in node.name or "_buffers_" in node.name)

    def add(self, role, node):
        t = self.value.get(node)
        if not isinstance(t, torch.Tensor):
            raise _NoStack(f"{role}: no tensor")
        if self.by_role.setdefault(role, t) is not t:
            raise _NoStack(f"two tensors for {role}")

    def layer_count(self):
        idx = [r[0] for r in self.by_role if isinstance(r, tuple)]
        return max(idx) + 1 if idx else 0

    def check_shapes(self, layers):
        for i in range(layers):
            for key, shape in SHAPES.items():
                t = self.by_role.get((i, key))
                if t is None or tuple(t.shape) != shape:
                    raise _NoStack(f"layer {i} {key}: {None if t is None else tuple(t.shape)}, need {shape}")
        if tuple(getattr(self.by_role.get("norm"), "shape", ())) != (D,) or \
                tuple(getattr(self.by_role.get("inv_freq"), "shape", ())) != (DH // 2,):
            raise _NoStack("final norm / RoPE frequencies")


def _param_role(rel):
    """The role of a parameter used by a node of module path `rel` (relative to the Qwen3Model)."""
    m = _NORM.fullmatch(rel)
    if m:
        return int(m[1]), _NORMS[m[2]]
    return {"norm": "norm", "rotary_emb": "inv_freq"}.get(rel)


def _check_constants(node, cls, rel):
    """The op has RMSNorm's eps and RoPE without attention scaling built in."""
    consts = [a for a in node.args if isinstance(a, float)]
    if node.op != "call_function" or not consts:
        return
    if node.target in ADD and cls.endswith("RMSNorm") and any(abs(c - EPS) > 1e-12 for c in consts):
        raise _NoStack(f"RMSNorm eps {consts} (the op has {EPS})")
    if node.target in MUL and rel == "rotary_emb" and any(c != 1.0 for c in consts):
        raise _NoStack(f"RoPE attention scaling {consts}")


def _attention_mask(attn_nodes, layers, value):
    """The one 4-D mask input every attention uses, bidirectionally at head_dim ** -0.5."""
    masks = set()
    for n in attn_nodes:
        kw = dict(zip(("query", "key", "value", "attn_mask", "dropout_p", "is_causal", "scale"), n.args), **n.kwargs)
        scale = kw.get("scale")
        if kw.get("dropout_p", 0.0) != 0.0 or kw.get("is_causal", False) or \
                (scale is not None and abs(scale - DH ** -0.5) > 1e-6):
            raise _NoStack("attention: dropout, causal or another scale")
        masks.add(kw.get("attn_mask"))
    if len(attn_nodes) != layers or len(masks) != 1:
        raise _NoStack(f"{len(attn_nodes)} attentions for {layers} layers, {len(masks)} masks")
    mask = next(iter(masks))
    mv = value.get(mask)
    if not (isinstance(mask, torch.fx.Node) and mask.op == "placeholder" and isinstance(mv, torch.Tensor)
            and mv.dim() == 4 and (mv.dtype == torch.bool or mv.is_floating_point())):
        raise _NoStack("the attention mask is not a 4-D input of the graph")
    return mask


def _hidden_input(nodes, inside, mask, params, value):
    """The region's one tensor input besides the mask and the weights: GPU hidden states [B, L, 1024]."""
    ext = {a: None for n in nodes for a in n.all_input_nodes
           if a not in inside and a is not mask and not params.is_param(a)}
    tensors = [a for a in ext if not (a.op == "placeholder" and isinstance(value.get(a), (int, torch.SymInt)))]
    if len(tensors) != 1:
        raise _NoStack(f"inputs {[a.name for a in tensors]}")
    xv = tensors[0].meta.get("example_value")
    if not (isinstance(xv, torch.Tensor) and xv.dim() == 3 and xv.shape[-1] == D and xv.is_floating_point()):
        raise _NoStack("hidden states are not [B, L, 1024]")
    if not _on_gpu(xv):
        raise _NoStack("hidden states are not on the GPU")
    return tensors[0]


def _on_gpu(t):
    return t.device.type == "cuda"


def _head_of(nodes, inside, params):
    """The linear [N, 1024] of a parameter that alone consumes the region's one output."""
    outs = [n for n in nodes if any(u not in inside for u in n.users)]
    if len(outs) != 1 or len(outs[0].users) != 1:
        raise _NoStack("the stack's output has other users than one head")
    head = next(iter(outs[0].users))
    if not (head.op == "call_function" and head.target in LINEAR):
        raise _NoStack(f"the stack's output goes to {head.target}")
    hx, hw, hb = _linear_operands(head)
    W = params.value.get(hw) if params.is_param(hw) else None
    B = params.value.get(hb) if hb is not None and params.is_param(hb) else None
    if hx is not outs[0] or not isinstance(W, torch.Tensor) or W.dim() != 2 or W.shape[1] != D or \
            (hb is not None and not (isinstance(B, torch.Tensor) and tuple(B.shape) == (W.shape[0],))):
        raise _NoStack("the head is not a linear of a parameter [N, 1024]")
    return head, W, B


def find(gm, example_inputs):
    """The first stack + head in ``gm`` the GPU op takes, as a Plan, or None. Only graphs whose hidden
    states live on the GPU are fused (host tensors keep the plain graph)."""
    placeholders = [n for n in gm.graph.nodes if n.op == "placeholder"]
    value = dict(zip(placeholders, example_inputs))
    regions = {}
    for n in gm.graph.nodes:
        if n.op in ("call_function", "call_method", "call_module"):   # inputs carry their first user's module
            root = next((path for path, cls in (n.meta.get("nn_module_stack") or {}).values()
                         if _cls_name(cls) in ROOTS), None)
            if root is not None:
                regions.setdefault(root, []).append(n)
    for root, nodes in regions.items():
        try:
            return _match(root, nodes, value, placeholders)
        except _NoStack as e:
            log.info("torch_xdna: %s is not a stack the GPU op takes: %s", root, e)
    return None


def _match(root, nodes, value, placeholders):
    """A Plan for the Qwen3Model call `nodes` (module path `root`), or _NoStack with the reason."""
    inside = set(nodes)
    params = _Params(value)
    attn = []
    for n in nodes:
        path, cls = _module_of(n)
        rel = path[len(root) + 1:] if path != root else ""
        skip = None
        if n.op == "call_function" and n.target in LINEAR:
            _, w, b = _linear_operands(n)
            m = _PROJ.fullmatch(rel)
            if m is None or b is not None or not params.is_param(w):
                raise _NoStack(f"a linear in {rel or 'the root'}")
            params.add((int(m[1]), m[2] or m[3]), w)
            skip = w
        elif n.op == "call_function" and n.target in SDPA:
            attn.append(n)
        for a in n.all_input_nodes:
            if a is skip or not params.is_param(a):
                continue
            role = _param_role(rel)
            if role is None:
                raise _NoStack(f"parameter {a.name} used in {rel or 'the root'}")
            params.add(role, a)
        _check_constants(n, cls, rel)
    layers = params.layer_count()
    if layers < 1:
        raise _NoStack("no layers")
    params.check_shapes(layers)
    mask = _attention_mask(attn, layers, value)
    x = _hidden_input(nodes, inside, mask, params, value)
    head, W, B = _head_of(nodes, inside, params)
    params.by_role["head"] = W
    return Plan([n.name for n in nodes], x.name, mask.name, placeholders.index(mask), head.name, params.by_role, B,
                layers, int(W.shape[0]), MAX_TOKENS)


# ------------------------------------------------------------------ the fused graph
def copy_module(gm):
    """A GraphModule over the same attributes as ``gm`` with its own copy of the graph."""
    new = torch.fx.GraphModule(gm, copy.deepcopy(gm.graph))
    new.meta.update(gm.meta)
    return new


def fuse(gm, plan, stack_id, cfg_id):
    """Put xdna::qwen3_stack(x, mask) where the head was and drop the stack's nodes."""
    node = {n.name: n for n in gm.graph.nodes}
    head = node[plan.head]
    with gm.graph.inserting_before(head):
        op = gm.graph.call_function(torch.ops.xdna.qwen3_stack.default,
                                    (node[plan.x], node[plan.mask], stack_id, cfg_id))
    op.meta.update(head.meta)
    head.replace_all_uses_with(op)
    for name in [plan.head] + plan.region[::-1]:       # users before their inputs
        gm.graph.erase_node(node[name])
    gm.graph.lint()
    gm.recompile()


# ------------------------------------------------------------------ run time
class StackUnsupported(RuntimeError):
    pass


class _Stack:
    """One stack found by the backend: its weights (weakly), their GPU copies, the checks done."""

    def __init__(self, plan):
        self.refs = [weakref.ref(t) for t in plan.tensors()]
        self.bias = weakref.ref(plan.bias) if plan.bias is not None else None
        self.layers, self.N, self.max_tokens = plan.layers, plan.out_features, plan.max_tokens
        self.name = f"qwen3 stack {self.layers} layers -> {self.N}"
        self.verified = set()   # attention shapes whose first launch matched the model
        self.failed = None      # why the stack runs in the plain graph from now on
        self.capture = False    # keep a copy of the next output (for the check)
        self.captured = None
        self._packed = None     # (weakrefs, versions, device, packed weights)
        self.shapes = {}        # call shape -> _Shape (static buffers, HIP graph)
        self.lens_hint = None   # (mask, lengths) the dispatcher parsed for the call in flight

    def packed(self, dev):
        """The GEMM weights as bf16 [N, K] on dev (q|k|v and gate|up concatenated), the norms and
        RoPE frequencies as given; built again when a weight changed (its _version)."""
        ts = [r() for r in self.refs]
        if any(t is None for t in ts):
            raise RuntimeError("the stack's weights are gone")
        versions = tuple(t._version for t in ts)
        hit = self._packed
        if hit is not None and hit[1] == versions and hit[2] == dev and all(r() is t for r, t in zip(hit[0], ts)):
            return hit[3]
        n = len(LAYER_KEYS)

        def bf(*ws):
            return torch.cat([w.detach().to(dev) for w in ws]).to(torch.bfloat16).contiguous()

        def vec(w):
            w = w.detach().to(dev)
            return w.contiguous() if w.dtype in (torch.float32, torch.bfloat16, torch.float16) else w.float()

        layers = []
        for i in range(self.layers):
            L = dict(zip(LAYER_KEYS, ts[i * n:(i + 1) * n]))
            layers.append(dict(qkv=bf(L["q"], L["k"], L["v"]), o=bf(L["o"]), gu=bf(L["gate"], L["up"]),
                               down=bf(L["down"]), input_norm=vec(L["input_norm"]), post_norm=vec(L["post_norm"]),
                               q_norm=vec(L["q_norm"]), k_norm=vec(L["k_norm"])))
        norm, head, inv_freq = ts[self.layers * n:]
        bias = self.bias().detach().to(dev, torch.float32).contiguous() if self.bias is not None else None
        pk = dict(layers=layers, norm=vec(norm), head=bf(head), inv_freq=inv_freq.detach().to(dev, torch.float32),
                  bias=bias)
        self._packed = ([weakref.ref(t) for t in ts], versions, dev, pk)
        return pk

    def macs(self, lens):
        per_token = self.layers * (D * (NH + 2 * NKV) * DH + NH * DH * D + 3 * D * INTER) + D * self.N
        return per_token * sum(lens) + self.layers * sum(2 * NH * DH * n * n for n in lens)

    def fail(self, e):
        self.failed = f"{type(e).__name__}: {e}"[:300]
        stats.fallbacks.append((self.name, self.failed))
        log.warning("torch_xdna: GPU %s failed (%s); it runs as the plain graph from now on", self.name, self.failed)


_stacks = []    # stack id -> _Stack


def register(plan):
    with _lock:
        _stacks.append(_Stack(plan))
        return len(_stacks) - 1


def out_features(stack_id):
    return _stacks[stack_id].N


def lengths(mask):
    """Each sequence's length n when ``mask`` [B, H, L, L] (bool, or float with 0 for "sees" and a
    large negative value for "does not") is a prefix block: query positions < n see exactly the key
    positions < n, and every later position sees only itself or nothing (stack.py:328-352). None for
    any other mask (causal, heads that differ, ...)."""
    if not isinstance(mask, torch.Tensor) or mask.dim() != 4 or mask.shape[-1] != mask.shape[-2]:
        return None
    if mask.dtype == torch.bool:
        sees = mask
    elif mask.is_floating_point():
        sees = mask == 0
        if not bool((sees | (mask <= -1e4)).all()):
            return None
    else:
        return None
    if sees.shape[1] > 1 and not bool((sees == sees[:, :1]).all()):
        return None
    sees = sees[:, 0]                                   # [B, L, L]
    n = sees[:, 0].sum(-1)                              # what position 0 sees fixes the length
    i = torch.arange(sees.shape[-1], device=sees.device)
    valid_q = i[None, :, None] < n[:, None, None]       # [B, L, 1]
    block = valid_q & (i[None, None, :] < n[:, None, None])
    pad_ok = (sees == (i[:, None] == i[None, :])[None]) | ~sees.any(-1, keepdim=True)
    if not bool(torch.where(valid_q, sees == block, pad_ok).all()):
        return None
    return n.tolist()


def _groups(lens):
    """The attention shapes of a call (query blocks per sequence): each is checked on its first call."""
    return {-(-n // QBLOCK) for n in lens}


def _round_up(n, m):
    return -(-n // m) * m


class _Shape:
    """One call shape of a stack (sequence lengths, padded length, dtype, device): static input and
    output buffers, the attention metadata, and the call captured as a HIP graph. The first run is
    eager (it also warms the kernels up); the second captures; later calls copy the input in and
    replay the graph, so a call costs one launch of host work instead of ~11 per layer."""

    def __init__(self, st, pk, lens, L, dtype, dev):
        self.pk, self.lens, self.dev = pk, list(lens), dev
        B = len(lens)
        i32 = dict(dtype=torch.int32)
        cols = [_round_up(n, QBLOCK) for n in lens]
        starts = [sum(lens[:b]) for b in range(B)]
        vts = [sum(cols[:b]) for b in range(B)]
        self.rows = torch.cat([torch.arange(n) + b * L for b, n in enumerate(lens)]).to(dev)
        self.pos = torch.cat([torch.arange(n, **i32) for n in lens]).to(dev)
        self.vt_col = torch.cat([torch.arange(n, **i32) + c for n, c in zip(lens, vts)]).to(dev)
        meta = torch.tensor([starts, lens, vts], **i32).to(dev)
        self.seq_start, self.seq_len, self.seq_vt = (meta[r].contiguous() for r in range(3))
        # columns past a sequence's length stay zero: the attention reads them with zero weight
        self.vt = torch.zeros((NKV, DH, _round_up(sum(cols), 8)), dtype=torch.bfloat16, device=dev)
        self.x = torch.zeros((B, L, D), dtype=dtype, device=dev)
        self.out = torch.zeros((B * L, st.N), dtype=dtype, device=dev)   # padding rows stay zero
        self.runs, self.graph = 0, None

    def compute(self):
        """The whole op on self.x into the valid rows of self.out."""
        B, L = self.x.shape[:2]
        x2d = self.x.reshape(B * L, D).index_select(0, self.rows).float()
        y = _forward(self.pk, self, x2d)
        self.out.index_copy_(0, self.rows, y.to(self.out.dtype))

    def __call__(self, x):
        self.x.copy_(x)
        if not USE_GRAPHS or self.runs == 0:
            self.compute()
        elif self.graph is None:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.compute()
            self.graph = g
            g.replay()
        else:
            self.graph.replay()
        self.runs += 1
        return self.out.view(*self.x.shape[:2], -1).clone()


# Capture each call shape as a HIP graph (TORCH_XDNA_STACK_GRAPHS=0: every call eager).
USE_GRAPHS = __import__("os").environ.get("TORCH_XDNA_STACK_GRAPHS", "1") != "0"
MAX_SHAPES = 8                 # call shapes kept per stack (least recently used dropped)


def _forward(pk, shape, x2d):
    """The stack + head on the packed valid tokens x2d float32 [T, 1024] of the shape's sequences
    (one after another): float32 [T, N]."""
    T = x2d.shape[0]
    X = x2d.contiguous()
    max_len = max(shape.lens)
    for L in pk["layers"]:
        h = kernels.rmsnorm_bf16(X, L["input_norm"], EPS)
        qkv = kernels.mm_bf16(h, L["qkv"], None, torch.float32)
        q, k = kernels.qk_norm_rope(qkv, NH, NKV, L["q_norm"], L["k_norm"], pk["inv_freq"], shape.pos, shape.vt_col,
                                    EPS, shape.vt)
        att = kernels.attention_bf16(q, k, shape.vt, shape.seq_start, shape.seq_len, shape.seq_vt, max_len,
                                     DH ** -0.5)
        kernels.add_(X, kernels.mm_bf16(att.view(T, NH * DH), L["o"], None, torch.float32))
        h = kernels.rmsnorm_bf16(X, L["post_norm"], EPS)
        act = kernels.silu_mul_bf16(kernels.mm_bf16(h, L["gu"], None, torch.float32))
        kernels.add_(X, kernels.mm_bf16(act, L["down"], None, torch.float32))
    h = kernels.rmsnorm_bf16(X, pk["norm"], EPS)
    return kernels.mm_bf16(h, pk["head"], pk["bias"], torch.float32)


def run(cfg, stack_id, x, mask):
    """xdna::qwen3_stack: hidden states x [B, L, 1024] -> the head's output [B, L, N], on the GPU."""
    st = _stacks[stack_id]
    B, L = x.shape[:2]
    hint = st.lens_hint
    lens = hint[1] if hint is not None and hint[0] is mask else lengths(mask)
    if lens is not None and len(lens) == 1 and B > 1:
        lens = lens * B
    if lens is None or len(lens) != B or mask.shape[-1] != L or not all(1 <= n <= st.max_tokens for n in lens):
        raise StackUnsupported(f"{st.name}: the GPU op takes prefix-block masks of 1..{st.max_tokens} positions")
    if x.device.type != "cuda":
        raise StackUnsupported(f"{st.name}: the hidden states are not on the GPU")
    t0 = time.perf_counter()
    dev = x.device
    with _lock:
        pk = st.packed(dev)
        key = (tuple(lens), L, x.dtype, dev)
        shape = st.shapes.pop(key, None)
        if shape is None or shape.pk is not pk:           # new shape, or weights repacked
            shape = _Shape(st, pk, lens, L, x.dtype, dev)
        st.shapes[key] = shape                            # most recently used last
        while len(st.shapes) > MAX_SHAPES:
            st.shapes.pop(next(iter(st.shapes)))
        out = shape(x.detach())
        stats.launches += 1
        if st.capture:
            st.captured = out.float().clone()
    stats.calls["gpu"] += 1
    stats.seconds["gpu"] += time.perf_counter() - t0
    stats.macs["gpu"] += st.macs(lens)
    return out


class _Reached(Exception):
    pass


class _RunTo(torch.fx.Interpreter):
    """Runs a graph eagerly until one named node has its value."""

    def __init__(self, gm, target):
        super().__init__(gm, garbage_collect_values=True)
        self.extra_traceback = False
        self.target, self.value = target, None

    def run_node(self, n):
        out = super().run_node(n)
        if n.name == self.target:
            self.value = out
            raise _Reached()
        return out


def _value_at(gm, args, name):
    runner = _RunTo(gm, name)
    with torch.no_grad():
        try:
            runner.run(*args)
        except _Reached:
            pass
    if runner.value is None:
        raise RuntimeError(f"{name} not reached")
    return runner.value


class Dispatch:
    """What the backend returns for a graph with a stack: the fused graph when the GPU op takes the
    call, else the plain one; checks each attention shape's first fused call against the original
    graph (stack.py:412-460)."""

    def __init__(self, plan, stack_id, cfg, fused, plain, orig):
        self.plan, self.stack_id, self.cfg = plan, stack_id, cfg
        self.fused, self.plain, self.orig = fused, plain, orig

    def _fusable(self, st, args):
        """The call's sequence lengths when the fused graph takes it, else None."""
        if st.failed is not None or not kernels.available():
            return None
        lens = lengths(args[self.plan.mask_index])
        return lens if lens is not None and all(1 <= n <= st.max_tokens for n in lens) else None

    def __call__(self, *args):
        st = _stacks[self.stack_id]
        lens = self._fusable(st, args)
        if lens is not None:
            shapes = _groups(lens)
            verify = self.cfg.verify == "always" or (self.cfg.verify == "first" and not shapes <= st.verified)
            st.capture = verify
            st.lens_hint = (args[self.plan.mask_index], lens)
            try:
                out = self.fused(*args)
                if verify:
                    self._verify(st, args, lens, shapes)
                stats.stacks[(st.name, "gpu")] += 1
                return out
            except Exception as e:      # launch failure, or a mismatch
                st.fail(e)
            finally:
                st.capture, st.captured, st.lens_hint = False, None, None
        stats.stacks[(st.name, "cpu")] += 1
        return self.plain(*args)

    def _verify(self, st, args, lens, shapes):
        """The fused output's valid rows vs the original graph's head output, run eagerly."""
        if st.captured is None:
            raise RuntimeError("the fused graph did not run the stack op")
        want_all = _value_at(self.orig, args, self.plan.head)
        per_seq = lens * st.captured.shape[0] if len(lens) == 1 else lens
        got = torch.cat([st.captured[b, :n] for b, n in enumerate(per_seq)]).double()
        want = torch.cat([want_all[b, :n] for b, n in enumerate(per_seq)]).double()
        err = float((got - want).norm() / want.norm().clamp(min=1e-30))
        stats.checks.append((f"{st.name}, query blocks {sorted(shapes)}", round(err, 4)))
        if not bool(torch.isfinite(got).all()) or err > VERIFY_TOL:
            raise GPUResultMismatch(f"GPU {st.name} disagrees with the model: rel err {err:.3g}")
        st.verified |= shapes


def compile_fused(gm, example_inputs, cfg, cfg_id, plan, compile_graph):
    """The Dispatch over the fused and the plain compilation of ``gm`` (which this rewrites)."""
    orig = copy_module(gm)
    fused = copy_module(gm)
    sid = register(plan)
    fuse(fused, plan, sid, cfg_id)
    if cfg.verbose:
        log.warning("torch_xdna: %s (%d nodes) -> one GPU op", _stacks[sid].name, len(plan.region) + 1)
    return Dispatch(plan, sid, cfg, compile_graph(fused, example_inputs, cfg), compile_graph(gm, example_inputs, cfg),
                    orig)
