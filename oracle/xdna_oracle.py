"""CPU oracle for the int8 hot path (W8A8 GEMM and int8 3x3 conv) -- TEST INFRASTRUCTURE.

This module is the checker, never the product. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it. The product (`torch_xdna`) never imports anything
under `oracle/`, and its GPU path fails loudly when the HIP library is missing.

It restates, in numpy, what the reference computes on its CPU route, function by function. Every
function cites the reference lines it follows (paths relative to the reference repository root).
Inputs are numpy arrays; floating-point inputs are float32 arrays whose values are those of the
tensor the reference would see (bf16 and fp16 values convert to float32 exactly, so amax, division
and rounding are unchanged by the widening).

How each function is pinned (tests/test_oracle.py):

* quant_rows / weight quant / conv quant: brute force per element with the correctly rounded
  float32 quotient computed in float64 (exact for 24-bit operands: 53 >= 2*24+2), ties-to-even
  rounding written out by hand; invariants (the row's largest |x| maps to +-127, zero rows give
  zeros, |q| <= 127); torch's own ops (`torch.round(x / s)`), which are what the reference calls.
* gemm_i32: Python triple loop on tiny inputs, `torch._int_mm` (the reference's CPU kernel), and
  the independent C restatement in oracle/c.
* dequant: per-element float64 brute force of the fixed association ((acc*sx)*sw)+b, each step
  rounded to float32 once; a swapped association (acc*(sx*sw)) fails it on the fixtures.
* conv3x3_acc: direct 7-loop Python on tiny shapes, float64 `F.conv2d` (exact for these
  integers), and the C restatement.
* requant: closed form floor(acc / 2^s + 1/2) with Python integers, including negative ties,
  which separate round-half-up from round-half-away.
* calibrate: closed-form boundaries (top * 1.25 / 127 at exact powers of two).
* gemm_bf16: exact rational arithmetic (Python fractions) on tiny inputs; the bound is checked to
  contain numpy's float32 matmul of the same operands and to be violated by a wrong operand
  (a transposed or unrounded weight).
"""

import math

import numpy as np

F32 = np.float32
_EPS = F32(1e-8)      # torch casts clamp(min=1e-8) to the tensor's dtype (float32)
_Q = F32(127)


def quant_rows(x):
    """Per-row symmetric int8 quantization.

    Follows torch_xdna/runtime.py:145-148 (`_quant_rows`), :366-368 (`linear_int8`) and
    :64-65 (`QWeight`): s = amax(|x|, row).clamp(min=1e-8) / 127 in float32,
    q = round_half_even(x / s).clamp(-127, 127) as int8, with IEEE float32 division.

    x: float32 [R, K] (K >= 1). Returns (q int8 [R, K], s float32 [R]).
    """
    x = np.ascontiguousarray(x, dtype=F32)
    assert x.ndim == 2 and x.shape[1] >= 1
    amax = np.abs(x).max(axis=1)
    s = np.maximum(amax, _EPS) / _Q            # float32 / float32: correctly rounded
    q = np.rint(x / s[:, None])                # rint: round half to even
    return np.clip(q, -127, 127).astype(np.int8), s.astype(F32)


def weight_quant(w, transposed=False):
    """`QWeight.__init__` (torch_xdna/runtime.py:59-66): per-output-channel int8 of a weight.

    w: float32 [N, K] (or [K, N] when transposed, the `x @ W` form). Returns
    (wq int8 [N, K] -- K contiguous, the layout the GPU kernels read -- and sw float32 [N]).
    The reference keeps the transpose `w_kn` [K, N] for torch._int_mm (runtime.py:66); it holds
    the same integers.
    """
    w = np.asarray(w, dtype=F32)
    if transposed:
        w = w.T
    return quant_rows(w)


def weight_quant_cat(ws):
    """`qweight` of several weights (runtime.py:107): concatenated on N, then quantized per row."""
    return quant_rows(np.concatenate([np.asarray(w, dtype=F32) for w in ws], axis=0))


def gemm_i32(xq, wq):
    """Exact int32 sums acc[m, n] = sum_k xq[m, k] * wq[n, k].

    The reference's kernel is `torch._int_mm(xq, w_kn)` (runtime.py:162-163) with
    w_kn = wq.T; |acc| <= K * 127^2 fits int32 for every K the hot path sees.
    """
    acc = np.asarray(xq, dtype=np.int64) @ np.asarray(wq, dtype=np.int64).T
    assert np.abs(acc).max(initial=0) < 2 ** 31
    return acc.astype(np.int32)


def dequant(acc, sx, sw, bias=None):
    """y = (acc.float() * sx) * sw (+ bias.float()) in float32, left to right.

    torch_xdna/runtime.py:350-353 and :429-432 (`acc.float() * sx[:, None] * qw.sw[None, :]`,
    then `y += bias.float()`), and :370-373 for the in-graph form. Returns float32 [M, N];
    cast with to_dtype() for bf16/fp16 outputs (`.to(x.dtype)`).
    """
    y = np.asarray(acc).astype(F32) * np.asarray(sx, dtype=F32)[:, None]
    y = y * np.asarray(sw, dtype=F32)[None, :]
    if bias is not None:
        y = y + np.asarray(bias, dtype=F32)[None, :]
    return y


def to_bf16(y):
    """float32 -> bfloat16 with round-to-nearest-even (torch's `.to(torch.bfloat16)`).

    Returns the bf16 values as float32 (exactly representable), NaN kept as NaN.
    """
    u = np.ascontiguousarray(y, dtype=F32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(F32).copy()
    nan = np.isnan(y)
    out[nan] = np.nan
    return out


def gemm_bf16(x, w, bias=None):
    """precision "bf16": y = bf16(x) @ bf16(w)^T (+ bias), the math of the reference's bf16 route
    (runtime.py:218-236: operands rounded to bf16 in the staging copies, float32 accumulation;
    :299-313 and :340-344 for the bias).

    Float32 accumulation is not associative, so instead of one float32 result this returns
    (y, bound): y is the sum of the bf16 products in float64 (each product is exact; the float64
    summation error, at most K 2^-53 sum |x w|, is 2^-29 of the float32 bound below), and
    bound[m, n] = gamma_K * sum_k |x_mk w_nk| (+ 2^-24 |y| for the bias addition), with
    gamma_K = K u / (1 - K u), u = 2^-24: the worst-case error of any float32 summation order
    (Higham, Accuracy and Stability of Numerical Algorithms, 2nd ed., sec. 3.1). A float32 result
    must satisfy |y32 - y| <= bound; a bf16 / fp16 output may also differ by its final rounding.
    """
    xb = to_bf16(np.asarray(x, dtype=F32)).astype(np.float64)
    wb = to_bf16(np.asarray(w, dtype=F32)).astype(np.float64)
    K = xb.shape[1]
    y = xb @ wb.T
    mag = np.abs(xb) @ np.abs(wb).T
    u = 2.0 ** -24
    gamma = K * u / (1 - K * u)
    bound = gamma * mag
    if bias is not None:
        y = y + np.asarray(bias, dtype=F32).astype(np.float64)[None, :]
        bound = bound + u * (np.abs(y) + bound)
    return y, bound


def to_dtype(y, dtype):
    """`.to(x.dtype)` for the output dtypes of the hot path: 'f32', 'bf16', 'f16'."""
    if dtype == "f32":
        return np.asarray(y, dtype=F32)
    if dtype == "bf16":
        return to_bf16(y)
    if dtype == "f16":
        with np.errstate(over="ignore"):      # beyond the float16 range the cast gives inf, as torch's does
            return np.asarray(y, dtype=F32).astype(np.float16).astype(F32)
    raise ValueError(dtype)


def linear(x, weights, biases, transposed=False, out_dtype="f32"):
    """W8A8 `xdna::linear` / `xdna::linear_cat` on the CPU route (runtime.py:326-355, :402-434).

    x: float32 [R, K]; weights: list of [N_i, K] ([K, N_i] if transposed); biases: list of
    [N_i] or None. Returns (y as out_dtype values in float32, acc, xq, sx, sw).
    """
    xq, sx = quant_rows(x)
    if transposed:
        wq, sw = weight_quant_cat([np.asarray(w, dtype=F32).T for w in weights])
    else:
        wq, sw = weight_quant_cat(weights)
    acc = gemm_i32(xq, wq)
    bias = None
    if any(b is not None for b in biases):
        bias = np.concatenate([np.asarray(b, dtype=F32) if b is not None
                               else np.zeros(np.asarray(w).shape[1 if transposed else 0], F32)
                               for w, b in zip(weights, biases)])
    return to_dtype(dequant(acc, sx, sw, bias), out_dtype), acc, xq, sx, sw


# ---------------------------------------------------------------------------------------- conv
def conv_quant_images(x):
    """Per-image int8 quantization of an NCHW activation (torch_xdna/conv.py:45-46).

    sx = amax(|x|, dims (1, 2, 3)).float().clamp(min=1e-8) / 127; xq = round(x / sx).clamp(+-127).
    Returns (xq int8 [N, C, H, W], sx float32 [N]).
    """
    x = np.asarray(x, dtype=F32)
    n = x.shape[0]
    q, s = quant_rows(x.reshape(n, -1))
    return q.reshape(x.shape), s


def conv_weight_quant(w):
    """`ConvLayer.__init__` (torch_xdna/conv.py:58-60): int8 per output channel over (Ci, 3, 3).

    Returns (wq int8 [Co, Ci, 3, 3], sw float32 [Co]).
    """
    w = np.asarray(w, dtype=F32)
    q, s = quant_rows(w.reshape(w.shape[0], -1))
    return q.reshape(w.shape), s


def conv3x3_acc(xq, wq):
    """Exact int sums of a 3x3, stride-1, padding-1 conv: int64 [N, Co, H, W].

    The reference computes them as an exact float conv of the integers (conv.py:86-87) and, in its
    research harnesses, with the padded nine-tap sum restated here
    (npu_kernels/conv3x3_array.py:176-182, conv3x3_strips.py:180-186).
    """
    xq = np.asarray(xq, dtype=np.int64)
    wq = np.asarray(wq, dtype=np.int64)
    n, ci, h, w = xq.shape
    co = wq.shape[0]
    xp = np.zeros((n, ci, h + 2, w + 2), np.int64)
    xp[:, :, 1:h + 1, 1:w + 1] = xq
    acc = np.zeros((n, co, h, w), np.int64)
    for ky in range(3):
        for kx in range(3):
            acc += np.einsum("oc,nchw->nohw", wq[:, :, ky, kx], xp[:, :, ky:ky + h, kx:kx + w])
    return acc


def requant(acc, shift, relu):
    """Shift, round half up, saturate (torch_xdna/conv.py:89-92).

    q = (acc + (1 << (shift - 1))) >> shift with an arithmetic shift (floor), then clamp to
    [0, 255] as uint8 with a fused ReLU, else to [-128, 127] as int8.
    """
    acc = np.asarray(acc, dtype=np.int64)
    q = (acc + (1 << (shift - 1))) >> shift
    if relu:
        return np.clip(q, 0, 255).astype(np.uint8)
    return np.clip(q, -128, 127).astype(np.int8)


def calibrate_shift(acc0, relu):
    """`ConvLayer.calibrate` (torch_xdna/conv.py:71-75) from the integer sums of image 0.

    top = max(acc, 0) with ReLU else max |acc|; shift = min(31, max(1, ceil(log2(max(top * 1.25,
    1) / (255 if relu else 127))))) in Python float arithmetic.
    """
    acc0 = np.asarray(acc0, dtype=np.int64)
    top = float(np.clip(acc0, 0, None).max()) if relu else float(np.abs(acc0).max())
    return shift_from_top(top, relu)


def shift_from_top(top, relu):
    """The shift formula of torch_xdna/conv.py:75 for a given top (a float)."""
    return min(31, max(1, math.ceil(math.log2(max(top * 1.25, 1.0) / (255 if relu else 127)))))


def conv_scale(sw, shift):
    """`self.scale = self.sw * 2.0 ** self.shift` (torch_xdna/conv.py:76), float32 [Co]."""
    return (np.asarray(sw, dtype=F32) * F32(2.0 ** shift)).astype(F32)


def conv_dequant(q, scale, sx, bias=None):
    """y = q.float() * (scale.view(1, -1, 1, 1) * sx) (+ bias) in float32 (torch_xdna/conv.py:48-50).

    The per-(image, channel) factor scale[co] * sx[n] is formed first, then multiplied into q.
    """
    q = np.asarray(q)
    f = np.asarray(scale, dtype=F32)[None, :] * np.asarray(sx, dtype=F32)[:, None]   # [N, Co]
    y = q.astype(F32) * f[:, :, None, None]
    if bias is not None:
        y = y + np.asarray(bias, dtype=F32)[None, :, None, None]
    return y


def max_pool2(y):
    """2x2 / stride-2 max-pool of NCHW y, floor mode (torch.nn.functional.max_pool2d(y, 2, 2)), the
    pool between the convs of a VGG-style chain (examples/conv_xdna.py, vgg16)."""
    y = np.asarray(y)
    n, c, h, w = y.shape
    ho, wo = h // 2, w // 2
    v = y[:, :, :2 * ho, :2 * wo].reshape(n, c, ho, 2, wo, 2)
    return v.max(axis=(3, 5))


def conv3x3_layer(xq, wq, shift, relu):
    """`ConvLayer.cpu` (torch_xdna/conv.py:89-92): the int8/uint8 output of one layer."""
    return requant(conv3x3_acc(xq, wq), shift, relu)


def conv3x3_int8(x, w, bias, relu, shift=None):
    """The whole `conv3x3_int8` composite (torch_xdna/conv.py:43-51) with first-call calibration
    (conv.py:171-172: the shift comes from image 0 of the first call).

    Returns (y float32 [N, Co, H, W], q, shift, xq, sx, wq, sw).
    """
    xq, sx = conv_quant_images(x)
    wq, sw = conv_weight_quant(w)
    acc = conv3x3_acc(xq, wq)
    if shift is None:
        shift = calibrate_shift(acc[0], relu)
    q = requant(acc, shift, relu)
    y = conv_dequant(q, conv_scale(sw, shift), sx, bias)
    return y, q, shift, xq, sx, wq, sw
