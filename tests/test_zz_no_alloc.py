"""xdna_conv_quant_nhwc_noalloc (the no-allocation form of xdna_conv_quant_nhwc) through the C ABI.

The entry point keeps the per-image block maxima in a file-scope device array of the library instead of
a caller workspace. Two calls in a row, the second with a smaller input, must each equal the workspace
entry point's results bit for bit (int8 NHWC activation and the float32 per-image scales); a batch above
XDNA_NOALLOC_MAX_IMAGES is rejected before anything is launched.
"""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

F32, BF16 = 0, 1
MAX_IMAGES = 1024       # XDNA_NOALLOC_MAX_IMAGES
WS_PER_IMAGE = 256      # XDNA_AMAX_WS_PER_IMAGE


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _both(L, dev, x, dtype_code, c_pad):
    """(q, sx) from the workspace entry point and from the no-allocation one, on torch's stream."""
    nb, ch, h, w = x.shape
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    q_ref = torch.full((nb, h, w, c_pad), 77, dtype=torch.int8, device=dev)
    sx_ref = torch.full((nb,), -1.0, device=dev)
    ws = torch.full((nb, WS_PER_IMAGE), float("nan"), device=dev)
    rc = L.xdna_conv_quant_nhwc(_ptr(x), dtype_code, nb, ch, h, w, _ptr(q_ref), c_pad, _ptr(sx_ref), _ptr(ws), st)
    assert rc == 0, L.xdna_last_error()
    q = torch.full((nb, h, w, c_pad), -77, dtype=torch.int8, device=dev)
    sx = torch.full((nb,), -2.0, device=dev)
    rc = L.xdna_conv_quant_nhwc_noalloc(_ptr(x), dtype_code, nb, ch, h, w, _ptr(q), c_pad, _ptr(sx), st)
    assert rc == 0, L.xdna_last_error()
    torch.cuda.synchronize(dev)
    return q_ref, sx_ref, q, sx


def test_noalloc_matches_workspace_entry(gpu):
    from torch_xdna import kernels

    L = kernels.lib()
    g = torch.Generator().manual_seed(31)
    # first call: 6 images (larger), float32 with channel padding; second: 2 smaller bf16 images, so the
    # scratch still holds the first call's maxima in slots the second call does not use
    x1 = (torch.randn(6, 40, 17, 24, generator=g) * 3).to(gpu)
    x2 = torch.randn(2, 16, 9, 8, generator=g).to(torch.bfloat16).to(gpu)
    for x, code, c_pad in ((x1, F32, 48), (x2, BF16, 16)):
        q_ref, sx_ref, q, sx = _both(L, gpu, x, code, c_pad)
        assert torch.equal(q, q_ref), "int8 activations differ from the workspace entry point"
        assert torch.equal(sx, sx_ref), "per-image scales differ from the workspace entry point"
        assert bool((sx > 0).all())
    # the same large call again after the small one: the kept scratch contents do not leak into it
    q_ref, sx_ref, q, sx = _both(L, gpu, x1, F32, 48)
    assert torch.equal(q, q_ref) and torch.equal(sx, sx_ref)


def test_noalloc_rejects_batches_above_the_limit(gpu):
    from torch_xdna import kernels

    L = kernels.lib()
    p = ctypes.c_void_p(16)
    assert L.xdna_conv_quant_nhwc_noalloc(p, F32, MAX_IMAGES + 1, 3, 4, 4, p, 16, p, None) == -1
    assert b"XDNA_NOALLOC_MAX_IMAGES" in L.xdna_last_error()
    assert L.xdna_conv_quant_nhwc_noalloc(None, F32, 0, 3, 4, 4, None, 16, None, None) == 0
