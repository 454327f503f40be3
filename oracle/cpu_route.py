"""The reference's CPU route restated with the same torch CPU kernels -- TEST INFRASTRUCTURE.

This is the `cpu_baseline` of bench.py (kind "port"): the reference computes its CPU route with
torch library kernels (`torch._int_mm`, `F.conv2d` of int8-valued floats), so the port calls the
same kernels in the same order. It is also a third independent check of the numpy and C
restatements in the tests. The product never imports it.

Functions and the reference lines they follow (paths relative to the reference root):
  quant_rows        torch_xdna/runtime.py:145-148
  weight_quant      torch_xdna/runtime.py:59-66
  linear            torch_xdna/runtime.py:326-355 (int8 route, `_gemm` :285-296, `_cpu_acc` :162-163)
  conv_quant        torch_xdna/conv.py:45-46
  ConvLayerCPU      torch_xdna/conv.py:57-76, :86-92
  conv_dequant      torch_xdna/conv.py:48-51
"""

import math

import torch
import torch.nn.functional as F


def quant_rows(x2d):
    x = x2d.float()
    s = x.abs().amax(dim=1).clamp(min=1e-8) / 127
    return torch.round(x / s[:, None]).clamp(-127, 127).to(torch.int8), s


def weight_quant(w, transposed=False):
    """(w_kn int8 [K, N] for torch._int_mm, sw float32 [N])."""
    wf = w.detach().float()
    if transposed:
        wf = wf.t()
    q, sw = quant_rows(wf)
    return q.t().contiguous(), sw


def int_mm(xq, w_kn):
    return torch._int_mm(xq, w_kn)


def linear(x, w_kn, sw, bias=None):
    """y = dequant(int_mm(quant(x))) + bias, in x.dtype."""
    x2d = x.reshape(-1, x.shape[-1])
    xq, sx = quant_rows(x2d)
    acc = int_mm(xq, w_kn)
    y = acc.float() * sx[:, None] * sw[None, :]
    if bias is not None:
        y += bias.float()
    return y.to(x.dtype).reshape(*x.shape[:-1], -1)


def conv_quant(x):
    sx = x.abs().amax(dim=(1, 2, 3), keepdim=True).float().clamp(min=1e-8) / 127
    return torch.round(x.float() / sx).clamp(-127, 127).to(torch.int8), sx


class ConvLayerCPU:
    """Weights, shift and the integer conv of one layer on the CPU."""

    def __init__(self, weight, relu):
        wf = weight.detach().float()
        self.sw = wf.abs().amax(dim=(1, 2, 3)).clamp(min=1e-8) / 127
        self.wq = torch.round(wf / self.sw[:, None, None, None]).clamp(-127, 127).to(torch.int8)
        self.cpu_dtype = (torch.float32 if 127 * float(self.wq.abs().sum(dim=(1, 2, 3)).max()) < 2 ** 24
                          else torch.float64)
        self.relu = relu
        self.shift = self.scale = None

    def acc(self, xq):
        return F.conv2d(xq.to(self.cpu_dtype), self.wq.to(self.cpu_dtype), padding=1)

    def calibrate(self, xq0):
        acc = self.acc(xq0[None])
        top = float(acc.clamp(min=0).max()) if self.relu else float(acc.abs().max())
        self.shift = min(31, max(1, math.ceil(math.log2(max(top * 1.25, 1.0) / (255 if self.relu else 127)))))
        self.scale = self.sw * 2.0 ** self.shift

    def __call__(self, xq):
        q = (self.acc(xq).to(torch.int32) + (1 << (self.shift - 1))) >> self.shift
        return q.clamp_(0, 255).to(torch.uint8) if self.relu else q.clamp_(-128, 127).to(torch.int8)


def conv_dequant(q, scale, sx, bias, dtype):
    y = q.float() * (scale.view(1, -1, 1, 1) * sx)
    if bias is not None:
        y = y + bias.float().view(1, -1, 1, 1)
    return y.to(dtype)
