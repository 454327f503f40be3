"""CPU restatement of xdna::qwen3_stack's math -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this module; the product
never imports it.

The stack is transformers' Qwen3Model (the reference's whole-stack op, torch_xdna/stack.py, fuses it
with the linear head that reads its last hidden states). The model code is a third-party dependency
of the reference (transformers, not vendored in the reference; 5.15.0 here): this module restates
its published algorithm (models/qwen3/modeling_qwen3.py: Qwen3RMSNorm, Qwen3RotaryEmbedding with
the default rope type, apply_rotary_pos_emb / rotate_half, Qwen3Attention with q_norm / k_norm and
grouped-query SDPA, Qwen3MLP with SiLU) in float64 for one sequence of n valid tokens whose
attention sees exactly those n tokens (the prefix-block masks the op takes, stack.py:328-352).

Pinned by tests/test_oracle.py against transformers' own Qwen3Model in float64 on the same weights
(a wrong rotate_half sign, RoPE pairing, GQA head mapping or norm placement fails it).
"""
import torch

F64 = torch.float64


def rms_norm(x, w, eps):
    """w * (x * rsqrt(mean(x^2) + eps)) over the last dim (Qwen3RMSNorm): the normalization runs in
    float32 whatever x's dtype, and its result is cast back before the weight multiplies it."""
    xf = x.to(torch.float32)
    return w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)


def rope(x, inv_freq):
    """x [n, heads, dh] at positions 0 .. n-1: x cos + rotate_half(x) sin with the angle of dim j being
    pos * inv_freq[j % (dh / 2)]; rotate_half(x) = cat(-x[dh/2:], x[:dh/2]). The angles and their cos /
    sin are float32 whatever the model's dtype (Qwen3RotaryEmbedding computes them in float32 and
    casts the result), the rotation itself in float64."""
    n, dh = x.shape[0], x.shape[-1]
    ang = torch.arange(n, dtype=torch.float32)[:, None] * inv_freq.to(torch.float32)[None, :]   # [n, dh/2]
    ang = torch.cat([ang, ang], -1)[:, None, :]                                                  # [n, 1, dh]
    rot = torch.cat([-x[..., dh // 2:], x[..., :dh // 2]], -1)
    return x * ang.cos().to(F64) + rot * ang.sin().to(F64)


def attention(q, k, v):
    """Bidirectional grouped-query attention: q [n, nh, dh], k / v [n, nkv, dh]; q head h reads kv
    head h // (nh / nkv); scale dh ** -0.5. Returns [n, nh, dh]."""
    nh, nkv, dh = q.shape[1], k.shape[1], q.shape[2]
    rep = nh // nkv
    k = k.repeat_interleave(rep, dim=1)
    v = v.repeat_interleave(rep, dim=1)
    s = torch.einsum("qhd,khd->hqk", q, k) * dh ** -0.5
    return torch.einsum("hqk,khd->qhd", s.softmax(-1), v)


def layer(x, w, eps, inv_freq, nh, nkv, dh):
    """One Qwen3DecoderLayer on x [n, d] float64; w holds the layer's weights by role."""
    n = x.shape[0]
    h = rms_norm(x, w["input_norm"], eps)
    q = (h @ w["q"].T).view(n, nh, dh)
    k = (h @ w["k"].T).view(n, nkv, dh)
    v = (h @ w["v"].T).view(n, nkv, dh)
    q = rope(rms_norm(q, w["q_norm"], eps), inv_freq)
    k = rope(rms_norm(k, w["k_norm"], eps), inv_freq)
    x = x + attention(q, k, v).reshape(n, nh * dh) @ w["o"].T
    h = rms_norm(x, w["post_norm"], eps)
    g, u = h @ w["gate"].T, h @ w["up"].T
    return x + (torch.nn.functional.silu(g) * u) @ w["down"].T


def stack_forward(x, layers, norm, head, bias, inv_freq, eps=1e-6, nh=16, nkv=8, dh=128):
    """The stack + head on one sequence's valid tokens x [n, d]: float64 [n, N]."""
    c = lambda t: t.detach().to("cpu", F64)      # noqa: E731
    x = c(x)
    for w in layers:
        x = layer(x, {k: c(v) for k, v in w.items()}, eps, c(inv_freq), nh, nkv, dh)
    y = rms_norm(x, c(norm), eps) @ c(head).T
    return y + c(bias) if bias is not None else y


def model_weights(llm):
    """The per-layer weights of a transformers Qwen3Model by role, its final norm and inv_freq."""
    layers = []
    for L in llm.layers:
        a, m = L.self_attn, L.mlp
        layers.append(dict(q=a.q_proj.weight, k=a.k_proj.weight, v=a.v_proj.weight, o=a.o_proj.weight,
                           gate=m.gate_proj.weight, up=m.up_proj.weight, down=m.down_proj.weight,
                           input_norm=L.input_layernorm.weight, post_norm=L.post_attention_layernorm.weight,
                           q_norm=a.q_norm.weight, k_norm=a.k_norm.weight))
    return layers, llm.norm.weight, llm.rotary_emb.inv_freq
