"""xdna::linear / linear_cat / linear_i8 / conv3x3, the custom ops the backend puts in place of
offloadable GEMMs and convs; xdna::conv3x3_fused and xdna::conv3x3_chain, the GPU forms of the conv
composite and of a chain of them; and xdna::qwen3_stack, the fused transformer-stack op (its GPU
implementation is stack.py).

The schemas, fake (meta) functions and the `cfg_id` indirection are those of the reference
(torch_xdna/ops.py:14-89 in the reference), so graphs built for it run unchanged. To the rest of
torch.compile each op is opaque with a shape function; Inductor compiles everything around it and
calls it as an extern kernel.
"""

from typing import Optional

import torch

from . import conv, runtime, stack

_configs = []  # cfg_id -> Config; the op's arguments must be plain values


def config_id(cfg) -> int:
    for i, c in enumerate(_configs):
        if c == cfg:
            return i
    _configs.append(cfg)
    return len(_configs) - 1


@torch.library.custom_op("xdna::linear", mutates_args=())
def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
           transposed: bool, cfg_id: int) -> torch.Tensor:
    return runtime.linear(_configs[cfg_id], x, weight, bias, transposed)


@linear.register_fake
def _(x, weight, bias, transposed, cfg_id):
    N = weight.shape[1] if transposed else weight.shape[0]
    return x.new_empty(*x.shape[:-1], N)


@torch.library.custom_op("xdna::linear_cat", mutates_args=())
def linear_cat(x: torch.Tensor, weights: list[torch.Tensor], biases: list[Optional[torch.Tensor]],
               cfg_id: int) -> torch.Tensor:
    """Linears that read the same input, as one GEMM: the outputs concatenated on the last dim."""
    return runtime.linear_cat(_configs[cfg_id], x, weights, biases)


@linear_cat.register_fake
def _(x, weights, biases, cfg_id):
    return x.new_empty(*x.shape[:-1], sum(w.shape[0] for w in weights))


@torch.library.custom_op("xdna::linear_i8", mutates_args=())
def linear_i8(xq: torch.Tensor, weights: list[torch.Tensor], transposed: bool,
              cfg_id: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The integer part of W8A8 linears that read the same input: int8 xq [R, K] ->
    (acc [R, N] int32, sw [N] float32), with x @ W^T ~= acc * sx[:, None] * sw for the row scales sx
    that gave xq. Several weights are one GEMM, their outputs concatenated."""
    return runtime.linear_i8(_configs[cfg_id], xq, weights, transposed)


@linear_i8.register_fake
def _(xq, weights, transposed, cfg_id):
    N = sum(w.shape[1] if transposed else w.shape[0] for w in weights)
    return xq.new_empty((xq.shape[0], N), dtype=torch.int32), xq.new_empty((N,), dtype=torch.float32)


@torch.library.custom_op("xdna::conv3x3", mutates_args=())
def conv3x3(xq: torch.Tensor, weight: torch.Tensor, relu: bool, cfg_id: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The integer part of a 3x3 / stride-1 / padding-1 conv of a [Co, Ci, 3, 3] parameter weight:
    int8 xq [N, Ci, H, W] -> (q [N, Co, H, W] int8, uint8 with relu; scale [Co] float32), with
    relu?(conv2d(x, weight)) ~= q * scale[co] * sx for the activation scale sx that gave xq."""
    return conv.conv3x3(_configs[cfg_id], xq, weight, relu)


@conv3x3.register_fake
def _(xq, weight, relu, cfg_id):
    q = xq.new_empty((xq.shape[0], weight.shape[0], xq.shape[2], xq.shape[3]),
                     dtype=torch.uint8 if relu else torch.int8)
    return q, weight.new_empty((weight.shape[0],), dtype=torch.float32)


@torch.library.custom_op("xdna::conv3x3_fused", mutates_args=())
def conv3x3_fused(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], relu: bool,
                  cfg_id: int) -> torch.Tensor:
    """relu?(conv2d(x, weight, bias, padding=1)) through int8 as one op: the same numbers as the
    quantize -> xdna::conv3x3 -> dequantize composite, with all three steps in HIP kernels."""
    return conv.conv3x3_fused(_configs[cfg_id], x, weight, bias, relu)


@conv3x3_fused.register_fake
def _(x, weight, bias, relu, cfg_id):
    return x.new_empty((x.shape[0], weight.shape[0], x.shape[2], x.shape[3]))


@torch.library.custom_op("xdna::conv3x3_chain", mutates_args=())
def conv3x3_chain(x: torch.Tensor, weights: list[torch.Tensor], biases: list[Optional[torch.Tensor]],
                  relus: list[bool], relu_after: list[bool], pools: list[bool], cfg_id: int) -> torch.Tensor:
    """Consecutive conv3x3_int8 layers as one op: layer i's output, through a ReLU when relu_after[i]
    and a 2x2 max-pool when pools[i], feeds layer i + 1. On the GPU the activation stays NHWC int8
    between the convs, with the same integers as the unfused layers (results/conv3x3_cascade.md:216-222
    in the reference). relus[i] is conv3x3_int8's fused ReLU; relu_after[i] is a graph ReLU after a
    biased conv."""
    return conv.conv3x3_chain(_configs[cfg_id], cfg_id, x, list(weights), list(biases), list(relus),
                              list(relu_after), list(pools))


@conv3x3_chain.register_fake
def _(x, weights, biases, relus, relu_after, pools, cfg_id):
    h, w = x.shape[2], x.shape[3]
    for p in pools[:-1]:
        if p:
            h, w = h // 2, w // 2
    return x.new_empty((x.shape[0], weights[-1].shape[0], h, w))


@torch.library.custom_op("xdna::qwen3_stack", mutates_args=())
def qwen3_stack(x: torch.Tensor, mask: torch.Tensor, stack_id: int, cfg_id: int) -> torch.Tensor:
    """A Qwen3 stack found by the backend, and its head, on hidden states x [B, L, 1024] under a
    prefix-block mask: the head's output [B, L, N], zero on padding rows (ops.py:79-89 in the
    reference)."""
    return stack.run(_configs[cfg_id], stack_id, x, mask)


@qwen3_stack.register_fake
def _(x, mask, stack_id, cfg_id):
    return x.new_empty((x.shape[0], x.shape[1], stack.out_features(stack_id)))
