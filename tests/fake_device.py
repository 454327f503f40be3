"""A CPU stand-in for the GPU launchers of torch_xdna.kernels -- TEST INFRASTRUCTURE.

Routing, verify, fallback, stats and the FX pass are host logic; this fake lets the CPU suite run
them without a GPU. Each fake launcher computes its kernel's contract with the oracle on CPU tensors
(same shapes, layouts and dtypes as the real launcher), and `kernels.gpu_device` returns the CPU, so
the runtime's "gpu" route runs end to end here. The GPU suite runs the same logic on the real device.
"""
import numpy as np
import torch

from oracle import xdna_oracle as O

_NP_OF = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


def _to_torch(y, dtype):
    return torch.from_numpy(np.ascontiguousarray(y, dtype=np.float32)).to(dtype)


def quant_rows(x2d, k_pad=None, out=None):
    R, K = x2d.shape
    k_pad = -(-K // 16) * 16 if k_pad is None else k_pad
    q, s = O.quant_rows(x2d.float().numpy()) if R else (np.zeros((0, K), np.int8), np.zeros(0, np.float32))
    xq = torch.zeros((R, k_pad), dtype=torch.int8)
    xq[:, :K] = torch.from_numpy(q)
    sx = torch.from_numpy(s)
    if out is not None:
        out[0].copy_(xq)
        out[1].copy_(sx)
        return out
    return xq, sx


def pad_k(xq, k_pad):
    out = torch.zeros((xq.shape[0], k_pad), dtype=torch.int8)
    out[:, :xq.shape[1]] = xq
    return out


def mm_i8(a, w, out=None):
    return torch.from_numpy(O.gemm_i32(a.numpy(), w.numpy()))


def mm_i8_dequant(a, sx, w, sw, bias, out_dtype):
    acc = O.gemm_i32(a.numpy(), w.numpy())
    y = O.dequant(acc, sx.numpy(), sw.numpy(), None if bias is None else bias.float().numpy())
    return _to_torch(O.to_dtype(y, _NP_OF[out_dtype]), out_dtype)


def linear_row(x2d, w, sw, bias, out_dtype, sx=None):
    xq, s = quant_rows(x2d, w.shape[1])
    if sx is not None:
        sx[:1].copy_(s)
    return mm_i8_dequant(xq, s, w, sw, bias, out_dtype)


def bf16_rows(x2d, k_pad):
    out = torch.zeros((x2d.shape[0], k_pad), dtype=torch.bfloat16)
    out[:, :x2d.shape[1]] = x2d
    return out


def mm_bf16(a, w, bias, out_dtype):
    y, _ = O.gemm_bf16(a.float().numpy(), w.float().numpy(), None if bias is None else bias.float().numpy())
    return _to_torch(O.to_dtype(y.astype(np.float32), _NP_OF[out_dtype]), out_dtype)


def conv_weight_pack(weight, ci_pad):
    wq, sw = O.conv_weight_quant(weight.float().numpy())
    co, ci = wq.shape[:2]
    packed = np.zeros((co, 9, ci_pad), np.int8)
    packed[:, :, :ci] = wq.reshape(co, ci, 9).transpose(0, 2, 1)
    return torch.from_numpy(packed), torch.from_numpy(sw)


def _unpack(wq, ci):
    co = wq.shape[0]
    return wq.numpy()[:, :, :ci].transpose(0, 2, 1).reshape(co, ci, 3, 3)


def conv_quant(x, c_pad):
    q, s = O.conv_quant_images(x.float().numpy())
    n, c, h, w = q.shape
    out = np.zeros((n, h, w, c_pad), np.int8)
    out[..., :c] = q.transpose(0, 2, 3, 1)
    return torch.from_numpy(out), torch.from_numpy(s)


def _nchw(xq):
    return xq.numpy().transpose(0, 3, 1, 2)


def conv3x3(xq, wq, shift, relu):
    ci = xq.shape[3]
    acc = O.conv3x3_acc(_nchw(xq), _unpack(wq, ci))
    return torch.from_numpy(np.ascontiguousarray(O.requant(acc, shift, relu).transpose(0, 2, 3, 1)))


def conv3x3_calibrate(xq, wq, relu):
    acc = O.conv3x3_acc(_nchw(xq), _unpack(wq, xq.shape[3]))
    return int(np.clip(acc, 0, None).max()) if relu else int(np.abs(acc).max())


def conv_dequant(q, relu, scale, sx, bias, out_dtype):
    y = O.conv_dequant(q.numpy().transpose(0, 3, 1, 2), scale.numpy(), sx.numpy(),
                       None if bias is None else bias.float().numpy())
    return _to_torch(O.to_dtype(y, _NP_OF[out_dtype]), out_dtype)


def conv3x3_dequant(xq, wq, shift, relu, scale, sx, bias, out_dtype):
    return conv_dequant(conv3x3(xq, wq, shift, relu), relu, scale, sx, bias, out_dtype)


def conv_requant_next(q, relu, pool, scale, sx, bias, x_dtype, c_pad_next, relu_y=False):
    y = O.to_dtype(O.conv_dequant(q.numpy().transpose(0, 3, 1, 2), scale.numpy(), sx.numpy(),
                                  None if bias is None else bias.float().numpy()), _NP_OF[x_dtype])
    if relu_y:
        y = np.maximum(y, 0)
    if pool:
        y = O.max_pool2(y)
    return conv_quant(torch.from_numpy(np.ascontiguousarray(y, dtype=np.float32)), c_pad_next)


def nchw_to_nhwc(xq, c_pad):
    n, c, h, w = xq.shape
    out = torch.zeros((n, h, w, c_pad), dtype=torch.int8)
    out[..., :c] = xq.permute(0, 2, 3, 1)
    return out


def nhwc_to_nchw(q):
    return q.permute(0, 3, 1, 2).contiguous()


LAUNCHERS = ("quant_rows", "pad_k", "mm_i8", "mm_i8_dequant", "linear_row", "bf16_rows", "mm_bf16", "conv_weight_pack", "conv_quant", "conv3x3",
             "conv3x3_calibrate", "conv_dequant", "conv3x3_dequant", "conv_requant_next", "nchw_to_nhwc", "nhwc_to_nchw")


def install(monkeypatch):
    """Route torch_xdna's GPU launchers to this fake for the duration of a test."""
    import sys

    from torch_xdna import kernels

    me = sys.modules[__name__]
    monkeypatch.setitem(kernels._state, "ok", True)       # mark_broken() can still retire it
    monkeypatch.setitem(kernels._state, "error", None)
    monkeypatch.setattr(kernels, "gpu_device", lambda t: torch.device("cpu"))
    monkeypatch.setattr(kernels, "gemm_variant", lambda dev, M, N, K, kind=0: "fake")
    monkeypatch.setattr(kernels, "use_tuned", lambda on: None)
    for name in LAUNCHERS:
        monkeypatch.setattr(kernels, name, getattr(me, name))
