"""xdna::qwen3_stack: a Qwen3-0.6B-width transformer stack and its linear head as one op on the GPU.

The reference fuses one kind of subgraph into a single device op (torch_xdna/stack.py in the
reference): a transformers `Qwen3Model` of Qwen3-0.6B's widths (hidden 1024, 16 query and 8 key-value
heads of 128, MLP 3072), any depth, with bidirectional attention under a 4-D mask that is an input of
the graph, whose last hidden states feed only a linear layer (OmniVoice's backbone and audio heads).
The same subgraphs are taken here (the rules of stack.py:111-241): every linear of the stack is a
q/k/v/o or gate/up/down projection of a layer, without bias; every other parameter is a layer's
input / post-attention / q / k RMSNorm weight, the final norm's or the RoPE frequencies; RMSNorm eps
1e-6 and RoPE without attention scaling; one scaled_dot_product_attention per layer, all under the
same mask placeholder, no dropout, not causal, scale 1/sqrt(128); the hidden states the one other
tensor input; the head a linear of a parameter [N, 1024] (optional bias) that alone consumes the
stack's output.

The graph is then compiled twice, once with the stack and head replaced by xdna::qwen3_stack and
once as any other graph, and a dispatcher picks per call (stack.py:412-446): the fused graph when
every sequence's mask is a prefix block of 1 .. MAX_TOKENS positions followed by padding positions
that see themselves or nothing, the plain graph otherwise. The fused output's padding rows are zeros.
The first fused call of each attention shape is checked against the original graph run eagerly
(stack.py:448-460): its valid rows within 10% (relative norm) of the head's output, else, as after a
launch failure, the stack keeps to the plain graph for the rest of the process.

On the GPU the op packs the valid tokens of all sequences into one [T, 1024] float32 residual stream
and runs every layer with the HIP kernels: RMSNorm to bf16, the q|k|v, o, gate|up and down projections
on the tile engine's bf16 GEMM (float32 sums), q / k RMSNorm + RoPE, bidirectional grouped-query
attention (bf16 MFMA, online softmax in float32), SiLU * up and the residual adds; then the final norm
and the head (bias fused). Each call shape is captured as a HIP graph on its second call.
"""

import copy
import logging
import operator
import threading
import time
import weakref
from dataclasses import dataclass, field
from typing import Any, Optional

import torch
import torch.nn.functional as F

from . import kernels
from .runtime import GPUResultMismatch, stats

log = logging.getLogger("torch_xdna")
_lock = threading.RLock()

# Qwen3-0.6B's widths: hidden, query heads, key-value heads, head dim, MLP width; RMSNorm eps
D, NH, NKV, DH, INTER, EPS = 1024, 16, 8, 128, 3072, 1e-6
# a layer's weights in the order Plan.tensors() lists them, and their shapes
LAYER_SHAPES = {"q": (NH * DH, D), "k": (NKV * DH, D), "v": (NKV * DH, D), "o": (D, NH * DH),
                "gate": (INTER, D), "up": (INTER, D), "down": (D, INTER),
                "input_norm": (D,), "post_norm": (D,), "q_norm": (DH,), "k_norm": (DH,)}
LAYER_KEYS = tuple(LAYER_SHAPES)
VERIFY_TOL = 0.1               # relative norm error of the first fused call against the original graph
# Longest sequence the fused op takes. The reference's NPU program stops at 384 positions; the GPU
# attention streams the keys, so the cap only bounds the work of one call.
MAX_TOKENS = 4096
QBLOCK = 32                    # queries per attention wave

_ROOT_CLASS = "Qwen3Model"
_LINEAR = frozenset({torch._C._nn.linear, F.linear})
_SDPA = frozenset({torch._C._nn.scaled_dot_product_attention, F.scaled_dot_product_attention})
_ADD = frozenset({operator.add, torch.add})
_MUL = frozenset({operator.mul, torch.mul})


def _class_name(c):
    return c.__name__ if isinstance(c, type) else str(c).rsplit(".", 1)[-1].strip("'>")


def _on_gpu(t):
    return t.device.type == "cuda"


# ------------------------------------------------------------------ finding a stack
class _NoStack(Exception):
    """Why a Qwen3Model region is not a stack the op takes."""


@dataclass
class Plan:
    """A stack found in a graph; nodes are named, so the plan applies to copies of the graph.

    region: the names of the stack's nodes in graph order; x / mask / head: the names of the hidden
    states, the mask placeholder and the head; mask_index: the mask's position among the graph's
    inputs; weights: role -> tensor, a role being (layer, LAYER_KEYS entry), "norm", "inv_freq" or
    "head"; bias: the head's bias or None."""
    region: list
    x: Optional[str]
    mask: Optional[str]
    mask_index: int
    head: Optional[str]
    weights: dict
    bias: Any
    layers: int
    out_features: int
    max_tokens: int

    def tensors(self):
        """Every weight in a fixed order: each layer's LAYER_KEYS, then norm, head, inv_freq."""
        per_layer = [self.weights[(i, k)] for i in range(self.layers) for k in LAYER_KEYS]
        return per_layer + [self.weights[r] for r in ("norm", "head", "inv_freq")]


@dataclass(frozen=True)
class _Slot:
    """Where a stack parameter may appear: its role, how it enters the graph ("weight": the weight of a
    bias-free linear; "operand": an input of any other op) and the shape the op is built for."""
    role: str
    use: str
    shape: tuple


# Every parameter a fusable stack holds, keyed by the module path (below the Qwen3Model) of the node that
# uses it, with a layer's index written as "#". A parameter anywhere else, or used another way, means the
# region is not a stack the op takes (the rules of the reference's stack.py:111-241).
_SLOTS = {
    "layers.#.self_attn.q_proj": _Slot("q", "weight", LAYER_SHAPES["q"]),
    "layers.#.self_attn.k_proj": _Slot("k", "weight", LAYER_SHAPES["k"]),
    "layers.#.self_attn.v_proj": _Slot("v", "weight", LAYER_SHAPES["v"]),
    "layers.#.self_attn.o_proj": _Slot("o", "weight", LAYER_SHAPES["o"]),
    "layers.#.mlp.gate_proj": _Slot("gate", "weight", LAYER_SHAPES["gate"]),
    "layers.#.mlp.up_proj": _Slot("up", "weight", LAYER_SHAPES["up"]),
    "layers.#.mlp.down_proj": _Slot("down", "weight", LAYER_SHAPES["down"]),
    "layers.#.input_layernorm": _Slot("input_norm", "operand", LAYER_SHAPES["input_norm"]),
    "layers.#.post_attention_layernorm": _Slot("post_norm", "operand", LAYER_SHAPES["post_norm"]),
    "layers.#.self_attn.q_norm": _Slot("q_norm", "operand", LAYER_SHAPES["q_norm"]),
    "layers.#.self_attn.k_norm": _Slot("k_norm", "operand", LAYER_SHAPES["k_norm"]),
    "norm": _Slot("norm", "operand", (D,)),
    "rotary_emb": _Slot("inv_freq", "operand", (DH // 2,)),
}
_STACK_SLOTS = {k: v for k, v in _SLOTS.items() if not k.startswith("layers.#.")}


def _slot_key(rel):
    """(slot key, layer index) of a module path below the root: "layers.7.mlp.up_proj" -> ("layers.#.mlp.up_proj",
    7); a path outside the layers keeps its text and has no index."""
    head, sep, rest = rel.partition(".")
    idx, sep2, tail = rest.partition(".")
    if head == "layers" and sep and idx.isdigit():
        return "layers.#" + (sep2 + tail if sep2 else ""), int(idx)
    return rel, None


_SDPA_ARGS = ("query", "key", "value", "attn_mask", "dropout_p", "is_causal", "scale")


@dataclass
class _Census:
    """Facts about one Qwen3Model region, gathered in a single pass over its nodes: each linear with the
    slot of its module, each parameter used as an operand, the attentions' arguments, the float constants
    of RMSNorm adds and RoPE multiplies, the values that come from outside the region and the region's
    nodes whose value leaves it."""
    linears: list = field(default_factory=list)      # (slot key, layer, weight node, bias node, module path)
    operands: list = field(default_factory=list)     # (slot key, layer, parameter node, module path)
    attentions: list = field(default_factory=list)   # {argument name: value} of each attention call
    eps: list = field(default_factory=list)          # float constants added inside RMSNorm modules
    rope_scale: list = field(default_factory=list)   # float constants multiplied inside the RoPE module
    inputs: list = field(default_factory=list)       # outside tensors (not parameters, sizes or the mask)
    exits: list = field(default_factory=list)        # region nodes with a user outside the region


class _Candidate:
    """One Qwen3Model region (the nodes that ran inside module path `root`): its census, then the rules, each
    a generator of problems; the first problem rejects the region, none gives the Plan."""

    def __init__(self, root, nodes, example_of, placeholders):
        self.root, self.nodes, self.inside = root, nodes, set(nodes)
        self.example_of, self.placeholders = example_of, placeholders
        self.census = self._take_census()
        self.roles = {}
        self.layers = 0
        self.mask = None

    # ---- facts
    def _param(self, n):
        """Whether node n is a parameter or buffer of the model (a graph input Dynamo lifted from one)."""
        if not isinstance(n, torch.fx.Node) or n.op != "placeholder":
            return False
        return isinstance(self.example_of.get(n), torch.nn.Parameter) or any(
            tag in n.name for tag in ("_parameters_", "_buffers_"))

    def _module(self, n):
        path, cls = list(n.meta["nn_module_stack"].values())[-1]
        return path[len(self.root) + 1:] if path.startswith(self.root + ".") else "", _class_name(cls)

    def _take_census(self):
        c = _Census()
        seen = set()
        for n in self.nodes:
            rel, cls = self._module(n)
            key, layer = _slot_key(rel)
            fn = n.target if n.op == "call_function" else None
            skip = None
            if fn in _LINEAR:
                _, w, bias = _linear_operands(n)
                c.linears.append((key, layer, w, bias, rel))
                skip = w
            elif fn in _SDPA:
                call = dict(zip(_SDPA_ARGS, n.args))
                call.update(n.kwargs)
                c.attentions.append(call)
            if fn is not None:
                consts = [v for v in n.args if isinstance(v, float)]
                if fn in _ADD and cls.endswith("RMSNorm"):
                    c.eps += consts
                if fn in _MUL and rel == "rotary_emb":
                    c.rope_scale += consts
            for a in n.all_input_nodes:
                if a is skip:
                    continue
                if self._param(a):
                    c.operands.append((key, layer, a, rel))
                elif a not in self.inside and a not in seen:
                    seen.add(a)
                    c.inputs.append(a)
            if any(u not in self.inside for u in n.users):
                c.exits.append(n)
        return c

    def _claim(self, role, node):
        """Binds a role to the tensor behind node; a second, different tensor for one role is a problem."""
        t = self.example_of.get(node)
        if not isinstance(t, torch.Tensor):
            return f"no tensor behind {role}"
        if self.roles.setdefault(role, t) is not t:
            return f"{role} is bound to two different tensors"
        return None

    # ---- rules
    def _parameters(self):
        """Every linear is a bias-free projection of a parameter at a weight slot; every other parameter sits
        at an operand slot; each role is one tensor."""
        for key, layer, w, bias, rel in self.census.linears:
            slot = _SLOTS.get(key)
            if slot is None or slot.use != "weight" or bias is not None or not self._param(w):
                yield f"linear at '{rel or '<root>'}' is not a bias-free projection of a stack parameter"
                return
            yield from filter(None, [self._claim((layer, slot.role), w)])
        for key, layer, a, rel in self.census.operands:
            slot = _SLOTS.get(key)
            if slot is None or slot.use != "operand":
                yield f"parameter {a.name} is used at '{rel or '<root>'}', which holds no stack parameter"
                return
            yield from filter(None, [self._claim(slot.role if layer is None else (layer, slot.role), a)])

    def _shapes(self):
        """Layers 0 .. L-1, each with every per-layer role at the op's shape, and the stack-level roles."""
        self.layers = 1 + max((r[0] for r in self.roles if isinstance(r, tuple)), default=-1)
        if self.layers == 0:
            yield "the region holds no layer"
            return
        for (i, key) in ((i, k) for i in range(self.layers) for k in LAYER_KEYS):
            got = self.roles.get((i, key))
            if got is None or tuple(got.shape) != LAYER_SHAPES[key]:
                yield f"layer {i}: {key} is {'missing' if got is None else tuple(got.shape)}, the op takes " \
                      f"{LAYER_SHAPES[key]}"
                return
        for slot in _STACK_SLOTS.values():
            got = self.roles.get(slot.role)
            if got is None or tuple(got.shape) != slot.shape:
                yield f"{slot.role} is {'missing' if got is None else tuple(got.shape)}, the op takes {slot.shape}"
                return

    def _constants(self):
        """The op's RMSNorm eps and its RoPE (no attention scaling) are built in."""
        if any(abs(v - EPS) > 1e-12 for v in self.census.eps):
            yield f"RMSNorm eps {self.census.eps}, the op's is {EPS}"
        elif any(v != 1.0 for v in self.census.rope_scale):
            yield f"RoPE scaled by {self.census.rope_scale}"

    def _attention(self):
        """One bidirectional, dropout-free attention per layer at scale 1/sqrt(head dim), all under one mask
        that is a 4-D bool or float input of the graph."""
        calls = self.census.attentions
        odd = [c for c in calls if c.get("dropout_p", 0.0) != 0.0 or c.get("is_causal", False)
               or (c.get("scale") is not None and abs(c["scale"] - DH ** -0.5) > 1e-6)]
        if odd:
            yield "an attention with dropout, a causal mask or another scale"
            return
        masks = {id(c.get("attn_mask")): c.get("attn_mask") for c in calls}
        if len(calls) != self.layers or len(masks) != 1:
            yield f"{len(calls)} attention calls under {len(masks)} masks for {self.layers} layers"
            return
        (m,) = masks.values()
        ex = self.example_of.get(m) if isinstance(m, torch.fx.Node) and m.op == "placeholder" else None
        if not (isinstance(ex, torch.Tensor) and ex.dim() == 4 and (ex.dtype == torch.bool or ex.is_floating_point())):
            yield "the attention mask is not a 4-D bool / float input of the graph"
            return
        self.mask = m

    def _hidden_states(self):
        """Besides parameters, the mask and sizes, one tensor enters: GPU hidden states [B, L, 1024]."""
        ins = [a for a in self.census.inputs if a is not self.mask and not (
            a.op == "placeholder" and isinstance(self.example_of.get(a), (int, torch.SymInt)))]
        if len(ins) != 1:
            yield f"{len(ins)} tensors enter the region ({[a.name for a in ins]}), not just the hidden states"
            return
        t = ins[0].meta.get("example_value")
        if not (isinstance(t, torch.Tensor) and t.dim() == 3 and t.shape[-1] == D and t.is_floating_point()):
            yield "the hidden states are not a float [B, L, 1024] tensor"
        elif not _on_gpu(t):
            yield "the hidden states are host tensors"
        else:
            self.x = ins[0]

    def _head(self):
        """One value leaves the region, into a linear of a parameter [N, 1024] (bias optional) and nothing else."""
        ex = self.census.exits
        users = list(ex[0].users) if len(ex) == 1 else []
        if len(users) != 1:
            yield "the stack's result has another user than one head"
            return
        head = users[0]
        if not (head.op == "call_function" and head.target in _LINEAR):
            yield f"the stack's result feeds {head.target}, not a linear head"
            return
        hx, hw, hb = _linear_operands(head)
        w = self.example_of.get(hw) if self._param(hw) else None
        b = self.example_of.get(hb) if hb is not None and self._param(hb) else None
        good_w = hx is ex[0] and isinstance(w, torch.Tensor) and w.dim() == 2 and w.shape[1] == D
        good_b = hb is None or (isinstance(b, torch.Tensor) and tuple(b.shape) == (w.shape[0],))
        if not (good_w and good_b):
            yield "the head is not a linear of a [N, 1024] parameter (with an [N] bias or none)"
            return
        self.head_node, self.head_w, self.head_b = head, w, b

    RULES = (_parameters, _shapes, _constants, _attention, _hidden_states, _head)

    def plan(self):
        for rule in self.RULES:
            for problem in rule(self):
                raise _NoStack(problem)
        weights = dict(self.roles, head=self.head_w)
        return Plan([n.name for n in self.nodes], self.x.name, self.mask.name, self.placeholders.index(self.mask),
                    self.head_node.name, weights, self.head_b, self.layers, int(self.head_w.shape[0]), MAX_TOKENS)


def _linear_operands(node):
    names = ("input", "weight", "bias")
    got = dict(zip(names, node.args))
    got.update({k: v for k, v in node.kwargs.items() if k in names})
    return got.get("input"), got.get("weight"), got.get("bias")


def find(gm, example_inputs):
    """The first stack + head in ``gm`` the GPU op takes, as a Plan, or None. Only graphs whose hidden
    states live on the GPU are fused (host tensors keep the plain graph)."""
    placeholders = [n for n in gm.graph.nodes if n.op == "placeholder"]
    example_of = dict(zip(placeholders, example_inputs))
    regions = {}
    for n in gm.graph.nodes:
        if n.op not in ("call_function", "call_method", "call_module"):
            continue                    # inputs carry the module of their first user
        stack_ = n.meta.get("nn_module_stack") or {}
        root = next((path for path, cls in stack_.values() if _class_name(cls) == _ROOT_CLASS), None)
        if root is not None:
            regions.setdefault(root, []).append(n)
    for root, nodes in regions.items():
        try:
            return _Candidate(root, nodes, example_of, placeholders).plan()
        except _NoStack as e:
            log.info("torch_xdna: %s is not a stack the GPU op takes: %s", root, e)
    return None


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


def _truncated(gm, name):
    """A copy of ``gm`` that returns the value of node `name` (and computes nothing after it)."""
    probe = copy_module(gm)
    target = next(n for n in probe.graph.nodes if n.name == name)
    out = next(n for n in probe.graph.nodes if n.op == "output")
    probe.graph.erase_node(out)
    probe.graph.output(target)
    probe.graph.eliminate_dead_code()
    probe.recompile()
    return probe


# ------------------------------------------------------------------ run time
class StackUnsupported(RuntimeError):
    pass


@dataclass(eq=False)
class _Stack:
    """A registered stack: its weights (weakly), their packed GPU copies, the check state, the call
    shapes (static buffers, HIP graph)."""
    refs: list
    bias: Any
    layers: int
    N: int
    max_tokens: int
    name: str = ""
    verified: set = field(default_factory=set)   # attention shapes whose first fused call matched
    failed: Optional[str] = None                 # why the stack keeps to the plain graph
    capture: bool = False                        # keep a copy of the next output (for the check)
    captured: Any = None
    shapes: dict = field(default_factory=dict)   # call shape -> _Shape, least recently used first
    lens_hint: Any = None                        # (mask, lengths) parsed by the dispatcher for this call
    _packed: Any = None                          # (weakrefs, versions, device, packed weights)

    @classmethod
    def of(cls, plan):
        st = cls([weakref.ref(t) for t in plan.tensors()],
                 weakref.ref(plan.bias) if plan.bias is not None else None,
                 plan.layers, plan.out_features, plan.max_tokens)
        st.name = f"qwen3 stack {st.layers} layers -> {st.N}"
        return st

    def packed(self, dev):
        """The GEMM weights as bf16 [N, K] on dev (q|k|v concatenated, gate and up interleaved in row pairs
        for the GEMM with the SiLU fused), the norms and RoPE frequencies as given; built again when a
        weight changed (its _version)."""
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
            Lw = dict(zip(LAYER_KEYS, ts[i * n:(i + 1) * n]))
            gu = kernels.gate_up_interleaved(Lw["gate"].detach().to(dev), Lw["up"].detach().to(dev))
            layers.append(dict(qkv=bf(Lw["q"], Lw["k"], Lw["v"]), o=bf(Lw["o"]), gu=bf(gu),
                               down=bf(Lw["down"]), input_norm=vec(Lw["input_norm"]), post_norm=vec(Lw["post_norm"]),
                               q_norm=vec(Lw["q_norm"]), k_norm=vec(Lw["k_norm"])))
        norm, head, inv_freq = ts[self.layers * n:]
        bias = self.bias().detach().to(dev, torch.float32).contiguous() if self.bias is not None else None
        pk = dict(layers=layers, norm=vec(norm), head=bf(head), inv_freq=inv_freq.detach().to(dev, torch.float32),
                  bias=bias)
        self._packed = ([weakref.ref(t) for t in ts], versions, dev, pk)
        return pk

    def macs(self, lens):
        """Multiply-accumulates of a call: per token, each layer's four projections (q|k|v, o, gate|up,
        down) and the head; per sequence and layer, the attention's two [n x n x 128] products per head."""
        proj = D * (NH + 2 * NKV) * DH + NH * DH * D + 2 * D * INTER + INTER * D
        tokens = sum(lens)
        attn = sum(n * n for n in lens) * 2 * NH * DH
        return tokens * (self.layers * proj + D * self.N) + self.layers * attn

    def give_up(self, e):
        self.failed = f"{type(e).__name__}: {e}"[:300]
        stats.fallbacks.append((self.name, self.failed))
        log.warning("torch_xdna: GPU %s failed (%s); it runs as the plain graph from now on", self.name, self.failed)


_stacks = []    # stack id -> _Stack


def register(plan):
    """A stack id for the plan (its index in the process-wide registry)."""
    with _lock:
        _stacks.append(_Stack.of(plan))
        return len(_stacks) - 1


def out_features(stack_id):
    return _stacks[stack_id].N


def lengths(mask):
    """Each sequence's length n when ``mask`` [B, H, L, L] (bool, or float with 0 for "sees" and a
    large negative value for "does not", the same for every head) is a prefix block: query positions
    below n see exactly the key positions below n, and every later position sees only itself or
    nothing (stack.py:328-352). None for any other mask (causal, heads that differ, ...)."""
    if not isinstance(mask, torch.Tensor) or mask.dim() != 4 or mask.shape[-1] != mask.shape[-2]:
        return None
    if mask.dtype == torch.bool:
        sees = mask
    elif mask.is_floating_point():
        sees = mask == 0
        if not bool((sees | (mask <= -1e4)).all()):
            return None              # neither "sees" nor "does not"
    else:
        return None
    if not bool((sees == sees[:, :1]).all()):
        return None                  # heads differ
    sees = sees[:, 0]
    L = sees.shape[-1]
    n = sees[:, 0].sum(-1)           # how many keys position 0 sees: the length if anything
    pos = torch.arange(L, device=sees.device)
    valid = pos[None, :] < n[:, None]                               # [B, L]
    block = valid[:, :, None] & valid[:, None, :]                   # the prefix block
    own = torch.eye(L, dtype=torch.bool, device=sees.device)[None]  # a padding row seeing itself
    rows_ok = torch.where(valid[:, :, None], sees == block, (sees == own) | ~sees.any(-1, keepdim=True))
    return n.tolist() if bool(rows_ok.all()) else None


def _attention_shapes(lens):
    """The attention shapes of a call (query blocks per sequence); each is checked on its first call."""
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

    def norm(w, pending):
        # a residual add is always followed by a norm: the two run as one launch
        return kernels.rmsnorm_bf16(X, w, EPS) if pending is None else kernels.add_rmsnorm_bf16(X, pending, w, EPS)

    down = None                           # the MLP output still to be added to X
    for L in pk["layers"]:
        h = norm(L["input_norm"], down)
        qkv = kernels.mm_bf16(h, L["qkv"], None, torch.float32)
        q, k = kernels.qk_norm_rope(qkv, NH, NKV, L["q_norm"], L["k_norm"], pk["inv_freq"], shape.pos, shape.vt_col,
                                    EPS, shape.vt)
        att = kernels.attention_bf16(q, k, shape.vt, shape.seq_start, shape.seq_len, shape.seq_vt, max_len,
                                     DH ** -0.5)
        h = norm(L["post_norm"], kernels.mm_bf16(att.view(T, NH * DH), L["o"], None, torch.float32))
        act = kernels.mm_bf16_silu(h, L["gu"])
        down = kernels.mm_bf16(act, L["down"], None, torch.float32)
    h = norm(pk["norm"], down)
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
    stats.record("gpu", t0, st.macs(lens))
    return out


class Dispatch:
    """What the backend returns for a graph with a stack: calls the fused graph when the GPU op takes
    the call (prefix-block mask, lengths within the cap, the stack not given up), else the plain one;
    the first fused call of each attention shape is checked against the original graph's head output,
    computed eagerly (stack.py:412-460)."""

    def __init__(self, plan, stack_id, cfg, fused, plain, orig):
        self.plan, self.stack_id, self.cfg = plan, stack_id, cfg
        self.fused, self.plain = fused, plain
        self.reference = _truncated(orig, plan.head)     # the original graph, up to the head's value

    def _lengths(self, st, args):
        if st.failed is not None or not kernels.available():
            return None
        lens = lengths(args[self.plan.mask_index])
        if lens is None or not all(1 <= n <= st.max_tokens for n in lens):
            return None
        return lens

    def __call__(self, *args):
        st = _stacks[self.stack_id]
        lens = self._lengths(st, args)
        if lens is None:
            stats.stacks[(st.name, "cpu")] += 1
            return self.plain(*args)
        shapes = _attention_shapes(lens)
        check = self.cfg.verify == "always" or (self.cfg.verify == "first" and not shapes <= st.verified)
        st.capture, st.lens_hint = check, (args[self.plan.mask_index], lens)
        try:
            out = self.fused(*args)
            if check:
                self._check(st, args, lens, shapes)
        except Exception as e:          # a launch failure, or a mismatch
            st.give_up(e)
            stats.stacks[(st.name, "cpu")] += 1
            return self.plain(*args)
        finally:
            st.capture, st.captured, st.lens_hint = False, None, None
        stats.stacks[(st.name, "gpu")] += 1
        return out

    def _check(self, st, args, lens, shapes):
        """The fused output's valid rows against the original graph's head output, relative norm."""
        if st.captured is None:
            raise RuntimeError("the fused graph did not run the stack op")
        with torch.no_grad():
            want_all = self.reference(*args)
        per_seq = lens * st.captured.shape[0] if len(lens) == 1 else lens
        got = torch.cat([st.captured[b, :n] for b, n in enumerate(per_seq)]).double()
        want = torch.cat([want_all[b, :n] for b, n in enumerate(per_seq)]).double()
        err = float((got - want).norm() / want.norm().clamp(min=1e-30))
        stats.checks.append((f"{st.name}, query blocks {sorted(shapes)}", round(err, 4)))
        if not bool(torch.isfinite(got).all()) or err > VERIFY_TOL:
            raise GPUResultMismatch(f"GPU {st.name} disagrees with the model: rel err {err:.3g}")
        st.verified |= shapes


def compile_fused(gm, example_inputs, cfg, cfg_id, plan, compile_graph):
    """The Dispatch over the fused and the plain compilation of ``gm`` (which the plain compilation
    rewrites in place)."""
    orig = copy_module(gm)
    fused = copy_module(gm)
    sid = register(plan)
    fuse(fused, plan, sid, cfg_id)
    if cfg.verbose:
        log.warning("torch_xdna: %s (%d nodes) -> one GPU op", _stacks[sid].name, len(plan.region) + 1)
    return Dispatch(plan, sid, cfg, compile_graph(fused, example_inputs, cfg), compile_graph(gm, example_inputs, cfg),
                    orig)
