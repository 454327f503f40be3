"""The GPU side: the HIP library `_lib/libxdna_hip.so` (gfx950) through its C ABI.

Mirrors the role of the reference's NPU interface (torch_xdna/kernels.py in the reference):
`available()` / `unavailable_reason()` / `mark_broken()` decide whether the device may be used,
and one module-level launcher per kernel family (`mm_i8` and friends) does a launch, so tests can
monkeypatch a launcher exactly as the reference's tests patch `kernels.mm_i8`
(tests/test_backend.py:139-146, :165-168).

Every launcher takes torch tensors on one GPU, allocates its outputs with torch's caching
allocator on that device, enqueues on torch's current stream and returns without synchronizing.
A non-zero status from the library raises RuntimeError with the library's message. There is no
CPU fallback in this module: if the library is missing, the launchers raise.
"""

import contextlib
import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libxdna_hip.so")
ABI_VERSION = 1

F32, BF16, F16 = 0, 1, 2
_DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

_lock = threading.RLock()
_state = {"ok": None, "error": None}
_lib = None
_cus = {}


def round_up(x, m):
    return -(-x // m) * m


# ------------------------------------------------------------------------------ availability
def available() -> bool:
    """True if xdna ops can run on the GPU in this process (library loads, a GPU is visible)."""
    with _lock:
        if _state["ok"] is None:
            try:
                for var in ("TORCH_XDNA_DISABLE_GPU", "TORCH_XDNA_DISABLE_NPU"):
                    if os.environ.get(var) == "1":
                        raise RuntimeError(f"disabled by {var}=1")
                lib()
                if not torch.cuda.is_available():
                    raise RuntimeError("no GPU visible to torch (torch.cuda.is_available() is False)")
                _state["ok"] = True
            except Exception as e:  # any missing piece means: no GPU route
                _state["ok"], _state["error"] = False, f"{type(e).__name__}: {e}"
        return _state["ok"]


def unavailable_reason():
    return _state["error"]


def mark_broken(err: BaseException):
    """Launches kept failing: stop routing to the GPU for the rest of the process."""
    with _lock:
        _state["ok"], _state["error"] = False, f"{type(err).__name__}: {err}"


def reset():
    """Forget the availability decision (tests and env changes)."""
    with _lock:
        _state["ok"], _state["error"] = None, None


def lib():
    """The loaded library; raises if it is not built or its ABI version differs."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(f"HIP library not built: {LIB_PATH} (run `make -C torch-xdna_amd` "
                                   "or __graft_entry__.build())")
            L = ctypes.CDLL(LIB_PATH)
            L.xdna_abi_version.restype = ctypes.c_int
            got = L.xdna_abi_version()
            if got != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH} has ABI version {got}, expected {ABI_VERSION}")
            _declare(L)
            _lib = L
        return _lib


def _declare(L):
    p, i64, i = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    sig = {
        "xdna_last_error": ([], ctypes.c_char_p),
        "xdna_device_info": ([p, p, p], i),
        "xdna_quant_rows": ([p, i, i64, i64, i64, p, i64, i64, p, p], i),
        "xdna_gemm_i8_i32": ([p, i64, p, i64, p, i64, i64, i64, i64, p], i),
        "xdna_gemm_i8_dequant": ([p, i64, p, p, i64, p, p, p, i, i64, i64, i64, i64, p], i),
        "xdna_gemm_ws_bytes": ([i64, i64, i64], i64),
        "xdna_gemm_ksplit": ([i64, i64, i64, p, p], i),
        "xdna_gemm_i8_i32_ws": ([p, i64, p, i64, p, i64, i64, i64, i64, p, i64, p], i),
        "xdna_gemm_i8_dequant_ws": ([p, i64, p, p, i64, p, p, p, i, i64, i64, i64, i64, p, i64, p], i),
        "xdna_linear_row": ([p, i, i64, p, i64, p, p, p, i, i64, i64, p, p], i),
        "xdna_gemm_bf16": ([p, i64, p, i64, p, p, i, i64, i64, i64, i64, p], i),
        "xdna_gemm_bf16_silu": ([p, i64, p, i64, p, i64, i64, i64, i64, p], i),
        "xdna_pad_rows_i8": ([p, i64, i64, i64, p, i64, i64, p], i),
        "xdna_conv_quant_nhwc": ([p, i, i64, i64, i64, i64, p, i64, p, p, p], i),
        "xdna_conv_quant_nhwc_noalloc": ([p, i, i64, i64, i64, i64, p, i64, p, p], i),
        "xdna_conv_weight_pack": ([p, i, i64, i64, p, i64, p, p], i),
        "xdna_conv3x3_i8": ([p, i64, i64, i64, i64, p, i64, i, i, p, p, p], i),
        "xdna_conv_dequant": ([p, i, i64, i64, i64, i64, p, p, p, p, i, p], i),
        "xdna_conv3x3_dequant": ([p, i64, i64, i64, i64, p, i64, i, i, p, p, p, p, i, p], i),
        "xdna_conv_requant_next": ([p, i, i, i, i64, i64, i64, i64, p, p, p, i, p, i64, p, p, p], i),
        "xdna_nchw_to_nhwc_i8": ([p, i64, i64, i64, i64, p, i64, p], i),
        "xdna_nhwc_to_nchw_i8": ([p, i64, i64, i64, i64, p, p], i),
        "xdna_tile_set": ([i, i64, i64, i64, i], i),
        "xdna_tile_get": ([i, i64, i64, i64], i),
        "xdna_tile_plan": ([i, i64, i64, i64, p, p, p], i),
        "xdna_tile_clear": ([], i),
        "xdna_rmsnorm_bf16": ([p, i64, i64, p, i, ctypes.c_float, p, p], i),
        "xdna_add_rmsnorm_bf16": ([p, p, i64, i64, p, i, ctypes.c_float, p, p], i),
        "xdna_qk_norm_rope": ([p, i64, i, i, p, p, i, p, p, p, ctypes.c_float, p, p, p, i64, p], i),
        "xdna_attention_bf16": ([p, p, p, i64, p, p, p, i64, i64, i, i, ctypes.c_float, p, p], i),
        "xdna_silu_mul_bf16": ([p, i64, i64, p, p], i),
        "xdna_add_f32": ([p, p, i64, p], i),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes, f.restype = args, res


EXPORTS = ("xdna_abi_version", "xdna_last_error", "xdna_device_info", "xdna_quant_rows", "xdna_gemm_i8_i32",
           "xdna_gemm_i8_dequant", "xdna_gemm_ws_bytes", "xdna_gemm_ksplit", "xdna_gemm_i8_i32_ws", "xdna_gemm_i8_dequant_ws",
           "xdna_linear_row",
           "xdna_gemm_bf16", "xdna_gemm_bf16_silu", "xdna_pad_rows_i8", "xdna_conv_quant_nhwc",
           "xdna_conv_quant_nhwc_noalloc", "xdna_conv_weight_pack",
           "xdna_conv3x3_i8", "xdna_conv_dequant", "xdna_conv3x3_dequant", "xdna_conv_requant_next", "xdna_nchw_to_nhwc_i8",
           "xdna_nhwc_to_nchw_i8",
           "xdna_tile_set", "xdna_tile_get", "xdna_tile_plan", "xdna_tile_clear", "xdna_rmsnorm_bf16",
           "xdna_add_rmsnorm_bf16", "xdna_qk_norm_rope",
           "xdna_attention_bf16", "xdna_silu_mul_bf16", "xdna_add_f32")


def _check(status, what):
    if status != 0:
        msg = lib().xdna_last_error().decode(errors="replace")
        raise RuntimeError(f"xdna {what} failed (status {status}): {msg}")


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(dev):
    """torch's current stream on dev, as the raw HIP stream handle the library launches on."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    return ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(idx))


_NOCTX = contextlib.nullcontext()


def _on(dev):
    """Device context for a launch on dev: none when dev is already the current device (the common
    case, and switching costs microseconds per launch)."""
    idx = dev.index
    if idx is None or idx == torch.cuda.current_device():
        return _NOCTX
    return torch.cuda.device(idx)


def _need_gpu(*ts):
    dev = ts[0].device
    for t in ts:
        if t is not None and (t.device.type != "cuda" or t.device != dev):
            raise ValueError(f"xdna launchers take tensors on one GPU, got {t.device} and {dev}")
    return dev


def gpu_device(t):
    """The GPU a tensor's GPU route runs on: its own device, or the current GPU for host tensors."""
    return t.device if t.device.type == "cuda" else torch.device("cuda", torch.cuda.current_device())


def num_cus(dev) -> int:
    """Compute units of the device (the library's launch shaping uses the same figure)."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _cus:
        n, a, b = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        with torch.cuda.device(idx):
            _check(lib().xdna_device_info(ctypes.byref(n), ctypes.byref(a), ctypes.byref(b)), "device_info")
        _cus[idx] = n.value
    return _cus[idx]


# ------------------------------------------------------------------------------ tiles
KIND_I8, KIND_BF16, KIND_CONV = 0, 1, 2          # XDNA_KIND_*
KINDS = {"i8": KIND_I8, "bf16": KIND_BF16, "conv": KIND_CONV}
# XDNA_TILE_* by id: the tile engine's workgroup tiles, the small-M kernel by waves, the one-row kernel,
# the few-row kernel, tile-engine tiles with 2 or 4 K groups per workgroup, and the direct conv kernels
TILES = ("auto", "t256x256w8", "t256x256w4", "t256x128", "t128x256", "t128x128", "t64x64",
         "small_w1", "small_w2", "small_w4", "small_w8", "small_w16", "t192x256", "t256x192", "t64x32", "t32x64",
         "t32x32", "gemv_w4", "gemv_w2", "gemv_w8", "seg4_r2", "seg4_r4", "t64x64k2", "t64x64k4", "t32x64k4",
         "t32x32k4", "t128x128k2", "t128x256w8", "t256x128w8", "t256x256pp", "t256x64", "direct")
TILE_ID = {name: i for i, name in enumerate(TILES)}


def direct_ok(N, K) -> bool:
    """Whether the direct conv kernels (tile "direct") take a conv of N = co, K = 9 c_pad: c_pad 16, 32, 48
    or 64 and co a multiple of 32 up to 128, as the library's rule decides (xdna_mm.hip direct_ok)."""
    return K % 9 == 0 and K // 9 in (16, 32, 48, 64) and N % 32 == 0 and N <= 128


def tile_set(kind, M, N, K, tile):
    """Make every later launch of exactly (kind, M, N, K) use `tile` (a TILES name; "auto" removes the
    entry). For convs M = n*h*w, N = Co, K = 9*Ci_pad. Results do not depend on the tile."""
    _check(lib().xdna_tile_set(KINDS.get(kind, kind), M, N, K, TILE_ID[tile]), "tile_set")
    _ws_need.clear()


def tile_get(dev, kind, M, N, K) -> str:
    """The tile the next launch of (kind, M, N, K) on dev uses: the table's entry, else the library's
    built-in rule."""
    with _on(dev):
        t = lib().xdna_tile_get(KINDS.get(kind, kind), M, N, K)
    if t < 0:
        _check(t, "tile_get")
    return TILES[t]


def tile_clear():
    _check(lib().xdna_tile_clear(), "tile_clear")
    _ws_need.clear()


def tile_plan(dev, kind, M, N, K):
    """(head tile, m1, tail tile) of the next launch of (kind, M, N, K) on dev: rows [0, m1) with the
    head tile and rows [m1, M) with the tail tile, or (head, 0, "auto") for one launch."""
    head, m1, tail = ctypes.c_int(), ctypes.c_int64(), ctypes.c_int()
    with _on(dev):
        _check(lib().xdna_tile_plan(KINDS.get(kind, kind), M, N, K, ctypes.byref(head), ctypes.byref(m1),
                                    ctypes.byref(tail)), "tile_plan")
    return TILES[head.value], m1.value, TILES[tail.value]


def gemm_variant(dev, M, N, K, kind=KIND_I8) -> str:
    """The kernels a GEMM of M x N x K runs (the library's plan): the head tile, after a tail split
    "+<tail tile>@<first tail row>", and for an int8 launch that splits K across workgroups "/k<splits>"
    after its tile. One NPU-program key of the reference (runtime.py:207) corresponds to one
    (variant, N, K) here."""
    head, m1, tail = tile_plan(dev, kind, M, N, K)
    hk = tk = 1
    if kind == KIND_I8 and K % 16 == 0 and K >= 16:
        a, b = ctypes.c_int(), ctypes.c_int()
        with _on(dev):
            _check(lib().xdna_gemm_ksplit(M, N, K, ctypes.byref(a), ctypes.byref(b)), "gemm_ksplit")
        hk, tk = a.value, b.value
    head = head if hk == 1 else f"{head}/k{hk}"
    tail = tail if tk == 1 else f"{tail}/k{tk}"
    return head if m1 == 0 else f"{head}+{tail}@{m1}"


TUNED_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tuned", "mi355x.json")
_tuned = None
_tuned_applied = None


def tuned_table():
    """{(kind, M, N, K): tile} from a sweep (python -m torch_xdna.sweep); TORCH_XDNA_TUNED overrides the
    shipped table (the reference's kernels.tuned_table, torch_xdna/kernels.py:126-141)."""
    global _tuned
    with _lock:
        if _tuned is None:
            import json
            import re

            path = os.environ.get("TORCH_XDNA_TUNED") or TUNED_PATH
            table = {}
            if os.path.exists(path):
                with open(path) as f:
                    doc = json.load(f)
                for kind in KINDS:
                    for key, v in doc.get(kind, {}).items():
                        m = re.fullmatch(r"(\d+)x(\d+)x(\d+)", key)
                        if m and v.get("tiling") in TILE_ID and v["tiling"] != "auto":
                            table[(kind,) + tuple(int(x) for x in m.groups())] = v["tiling"]
            _tuned = table
        return _tuned


def tiling_for(kind, M, N, K):
    """The swept best tile for this launch when the table has one, else None (the library's rule)."""
    return tuned_table().get((kind, M, N, K))


def use_tuned(on: bool):
    """Register the tuned table in the library (Config.tuned_tilings) or take it out; a no-op when
    already in that state."""
    global _tuned_applied
    on = bool(on)
    if _tuned_applied is on:
        return
    with _lock:
        if _tuned_applied is on:
            return
        for (kind, M, N, K), tile in tuned_table().items():
            tile_set(kind, M, N, K, tile if on else "auto")
        _tuned_applied = on


# ------------------------------------------------------------------------------ launchers
def quant_rows(x2d, k_pad=None, out=None):
    """(xq int8 [R, k_pad], sx float32 [R]) of a [R, K] float tensor (bf16/fp16/fp32), K zero-padded
    to k_pad (default: the next multiple of 16). Same integers and scales as
    `torch.round(x.float() / s).clamp(-127, 127)` with s = amax.clamp(1e-8) / 127.
    `out=(xq, sx)` writes into given tensors (rows of xq may be a slice of a larger buffer)."""
    dev = _need_gpu(x2d)
    if x2d.dtype not in _DTYPE_CODE:
        raise TypeError(f"quant_rows takes float32/bfloat16/float16, got {x2d.dtype}")
    R, K = x2d.shape
    if x2d.stride(1) != 1:
        x2d = x2d.contiguous()
    k_pad = round_up(K, 16) if k_pad is None else k_pad
    if out is None:
        xq = torch.empty((R, k_pad), dtype=torch.int8, device=dev)
        sx = torch.empty((R,), dtype=torch.float32, device=dev)
    else:
        xq, sx = out
        _need_gpu(x2d, xq, sx)
        if xq.shape != (R, k_pad) or xq.stride(1) != 1 or sx.shape != (R,) or not sx.is_contiguous():
            raise ValueError("quant_rows: bad out tensors")
    if R:
        with _on(dev):
            _check(lib().xdna_quant_rows(_ptr(x2d), _DTYPE_CODE[x2d.dtype], R, K, x2d.stride(0), _ptr(xq),
                                         xq.stride(0), k_pad, _ptr(sx), _stream(dev)), "quant_rows")
    return xq, sx


def pad_k(xq, k_pad):
    """An int8 [R, K] tensor as [R, k_pad] with 16-byte aligned rows (copy only when needed)."""
    dev = _need_gpu(xq)
    R, K = xq.shape
    if K == k_pad and xq.stride(1) == 1 and xq.stride(0) % 16 == 0 and xq.data_ptr() % 16 == 0:
        return xq
    if xq.stride(1) != 1:
        xq = xq.contiguous()
    out = torch.empty((R, k_pad), dtype=torch.int8, device=dev)
    if R:
        with _on(dev):
            _check(lib().xdna_pad_rows_i8(_ptr(xq), R, K, xq.stride(0), _ptr(out), k_pad, k_pad, _stream(dev)),
                   "pad_rows_i8")
    return out


# The int8 GEMMs' K-split workspace (xdna_gemm_*_ws): the bytes a shape's plan can use, per device (they
# follow the tile table, so tile_set / tile_clear forget them), and one buffer per device and stream whose
# counter bytes are zero from its allocation on (each call leaves them zero). Under graph capture the
# GEMMs run without a workspace (no split; the same results), so no captured graph holds one.
_ws_need = {}
_ws_buf = {}


def _gemm_ws(dev, M, N, K):
    """(pointer, bytes) of the workspace for an int8 GEMM of M x N x K on dev's current stream, or
    (None, 0) when its plan splits nothing."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (idx, M, N, K)
    need = _ws_need.get(key)
    if need is None:
        with _on(dev):
            need = lib().xdna_gemm_ws_bytes(M, N, K)
        if need < 0:
            _check(need, "gemm_ws_bytes")
        _ws_need[key] = need
    if need == 0 or torch.cuda.is_current_stream_capturing():
        return None, 0
    skey = (idx, torch._C._cuda_getCurrentRawStream(idx))
    buf = _ws_buf.get(skey)
    if buf is None or buf.numel() < need:
        buf = torch.zeros(need, dtype=torch.uint8, device=torch.device("cuda", idx))
        _ws_buf[skey] = buf
    return _ptr(buf), buf.numel()


def mm_i8(a, w, out=None):
    """c [M, N] int32 = a [M, Kp] @ w [N, Kp]^T, int8 operands with 16-byte aligned rows, Kp % 16 == 0
    (the role of the reference's kernels.mm_i8, without its padding rules)."""
    dev = _need_gpu(a, w)
    M, K = a.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"mm_i8: K mismatch {a.shape} vs {w.shape}")
    c = torch.empty((M, N), dtype=torch.int32, device=dev) if out is None else out
    if M and N:
        with _on(dev):
            ws, wsb = _gemm_ws(dev, M, N, K)
            _check(lib().xdna_gemm_i8_i32_ws(_ptr(a), a.stride(0), _ptr(w), w.stride(0), _ptr(c), c.stride(0), M, N,
                                             K, ws, wsb, _stream(dev)), "gemm_i8_i32")
    return c


def mm_i8_dequant(a, sx, w, sw, bias, out_dtype):
    """y [M, N] = ((float(a @ w^T) * sx[:, None]) * sw[None, :] + bias) as out_dtype, in one kernel."""
    dev = _need_gpu(a, sx, w, sw, bias)
    M, K = a.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"mm_i8_dequant: K mismatch {a.shape} vs {w.shape}")
    y = torch.empty((M, N), dtype=out_dtype, device=dev)
    if M and N:
        with _on(dev):
            ws, wsb = _gemm_ws(dev, M, N, K)
            _check(lib().xdna_gemm_i8_dequant_ws(_ptr(a), a.stride(0), _ptr(sx), _ptr(w), w.stride(0), _ptr(sw),
                                                 _ptr(bias), _ptr(y), _DTYPE_CODE[out_dtype], y.stride(0), M, N, K,
                                                 ws, wsb, _stream(dev)), "gemm_i8_dequant")
    return y


# XDNA_LINEAR_ROW_KMAX: the longest weight row (bytes) xdna_linear_row takes (its int8 row sits in LDS)
LINEAR_ROW_KMAX = 32768


def linear_row_ok(x2d, k_pad):
    """Whether xdna_linear_row takes this activation for weights of k_pad columns: one row of
    float32 / bfloat16 / float16, contiguous and 16-byte aligned, its bytes a multiple of 16, and
    k_pad <= LINEAR_ROW_KMAX."""
    R, K = x2d.shape
    return (R == 1 and x2d.dtype in _DTYPE_CODE and (x2d.stride(1) == 1 or K == 1) and x2d.data_ptr() % 16 == 0
            and (K * x2d.element_size()) % 16 == 0 and K <= k_pad <= LINEAR_ROW_KMAX and k_pad % 16 == 0)


def linear_row(x2d, w, sw, bias, out_dtype, sx=None):
    """y [1, N] = the W8A8 linear of the one row x2d [1, K] (linear_row_ok) against w [N, Kp] int8, in
    one launch: the row's quantize (quant_rows' integers and scale) + the GEMM + the dequantize
    ((acc * s) * sw (+ bias)) as out_dtype, bit for bit quant_rows followed by mm_i8_dequant. sx: an
    optional float32 [1] tensor that receives the row's scale."""
    dev = _need_gpu(x2d, w, sw, bias, sx)
    K = x2d.shape[1]
    N, Kp = w.shape
    if not linear_row_ok(x2d, Kp) or w.stride(1) != 1 or w.stride(0) % 16 != 0:
        raise ValueError(f"linear_row: unsupported operands {x2d.dtype} {tuple(x2d.shape)}, w {tuple(w.shape)}")
    if sx is not None and (sx.dtype != torch.float32 or sx.numel() < 1):
        raise ValueError("linear_row: sx must be a float32 tensor of at least one element")
    y = torch.empty((1, N), dtype=out_dtype, device=dev)
    if N:
        with _on(dev):
            _check(lib().xdna_linear_row(_ptr(x2d), _DTYPE_CODE[x2d.dtype], K, _ptr(w), w.stride(0), _ptr(sw),
                                         _ptr(bias), _ptr(y), _DTYPE_CODE[out_dtype], N, Kp, _ptr(sx),
                                         _stream(dev)), "linear_row")
    return y


def bf16_rows(x2d, k_pad):
    """x2d as bf16 [R, k_pad] rows the bf16 GEMM reads (round to nearest even; zero columns past K,
    16-byte aligned rows): the tensor itself when it already qualifies, else one copy."""
    _need_gpu(x2d)
    R, K = x2d.shape
    if (x2d.dtype == torch.bfloat16 and K == k_pad and x2d.stride(1) == 1 and x2d.stride(0) % 8 == 0
            and x2d.data_ptr() % 16 == 0):
        return x2d
    out = torch.zeros((R, k_pad), dtype=torch.bfloat16, device=x2d.device) if K != k_pad else \
        torch.empty((R, k_pad), dtype=torch.bfloat16, device=x2d.device)
    out[:, :K].copy_(x2d)
    return out


def mm_bf16(a, w, bias, out_dtype):
    """y [M, N] = (a @ w^T (+ bias)) as out_dtype, bf16 operands a [M, Kp] and w [N, Kp] (Kp % 8 == 0,
    16-byte aligned rows), float32 accumulation and bias, in one kernel (precision "bf16")."""
    dev = _need_gpu(a, w, bias)
    M, K = a.shape
    N = w.shape[0]
    if w.shape[1] != K or a.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise ValueError(f"mm_bf16: bf16 [M, K] x [N, K] operands, got {a.dtype} {tuple(a.shape)}, "
                         f"{w.dtype} {tuple(w.shape)}")
    y = torch.empty((M, N), dtype=out_dtype, device=dev)
    if M and N:
        with _on(dev):
            _check(lib().xdna_gemm_bf16(_ptr(a), a.stride(0), _ptr(w), w.stride(0), _ptr(bias), _ptr(y),
                                        _DTYPE_CODE[out_dtype], y.stride(0), M, N, K, _stream(dev)), "gemm_bf16")
    return y


def gate_up_interleaved(gate, up):
    """The [2 I, K] weight xdna_gemm_bf16_silu takes: gate and up rows interleaved in pairs (rows 4j, 4j + 1
    gate rows 2j, 2j + 1; rows 4j + 2, 4j + 3 up rows 2j, 2j + 1). I must be even."""
    I, K = gate.shape
    if up.shape != (I, K) or I % 2:
        raise ValueError(f"gate_up_interleaved: two [I, K] weights with I even, got {tuple(gate.shape)} {tuple(up.shape)}")
    return torch.stack([gate.reshape(I // 2, 2, K), up.reshape(I // 2, 2, K)], dim=1).reshape(2 * I, K)


def mm_bf16_silu(a, w_gu):
    """bf16 [M, I] = silu(a @ gate^T) * (a @ up^T) in one kernel, with w_gu the bf16 [2 I, Kp] weight of
    gate_up_interleaved: the values of mm_bf16 (float32 out, gate|up concatenated) then silu_mul_bf16."""
    dev = _need_gpu(a, w_gu)
    M, K = a.shape
    N2 = w_gu.shape[0]
    if w_gu.shape[1] != K or a.dtype != torch.bfloat16 or w_gu.dtype != torch.bfloat16 or N2 % 4:
        raise ValueError(f"mm_bf16_silu: bf16 [M, K] x [2I, K] operands (2I a multiple of 4), got {a.dtype} "
                         f"{tuple(a.shape)}, {w_gu.dtype} {tuple(w_gu.shape)}")
    y = torch.empty((M, N2 // 2), dtype=torch.bfloat16, device=dev)
    if M and N2:
        with _on(dev):
            _check(lib().xdna_gemm_bf16_silu(_ptr(a), a.stride(0), _ptr(w_gu), w_gu.stride(0), _ptr(y), y.stride(0),
                                             M, N2, K, _stream(dev)), "gemm_bf16_silu")
    return y


AMAX_WS_PER_IMAGE = 256        # XDNA_AMAX_WS_PER_IMAGE: scratch floats per image of the per-image max


def conv_quant(x, c_pad):
    """Per-image int8 of an NCHW float x -> (xq NHWC [N, H, W, c_pad] int8, sx float32 [N])."""
    dev = _need_gpu(x)
    x = x.contiguous()
    n, c, h, w = x.shape
    xq = torch.empty((n, h, w, c_pad), dtype=torch.int8, device=dev)
    sx = torch.empty((n,), dtype=torch.float32, device=dev)
    ws = torch.empty((n, AMAX_WS_PER_IMAGE), dtype=torch.float32, device=dev)
    if n:
        with _on(dev):
            _check(lib().xdna_conv_quant_nhwc(_ptr(x), _DTYPE_CODE[x.dtype], n, c, h, w, _ptr(xq), c_pad, _ptr(sx),
                                              _ptr(ws), _stream(dev)), "conv_quant_nhwc")
    return xq, sx


def conv_weight_pack(weight, ci_pad):
    """Quantize-once of a [Co, Ci, 3, 3] weight on its GPU -> (wq [Co, 9, ci_pad] int8, sw [Co])."""
    dev = _need_gpu(weight)
    wt = weight.detach().contiguous()
    if wt.dtype not in _DTYPE_CODE:
        wt = wt.float()
    co, ci = wt.shape[:2]
    wq = torch.empty((co, 9, ci_pad), dtype=torch.int8, device=dev)
    sw = torch.empty((co,), dtype=torch.float32, device=dev)
    with _on(dev):
        _check(lib().xdna_conv_weight_pack(_ptr(wt), _DTYPE_CODE[wt.dtype], co, ci, _ptr(wq), ci_pad, _ptr(sw),
                                           _stream(dev)), "conv_weight_pack")
    return wq, sw


def conv3x3(xq, wq, shift, relu):
    """int8 NHWC [N, H, W, c_pad] (*) wq [Co, 9, c_pad] -> NHWC [N, H, W, Co] int8 (uint8 if relu),
    requantized by `shift` with round half up and saturation."""
    dev = _need_gpu(xq, wq)
    n, h, w, c_pad = xq.shape
    co = wq.shape[0]
    y = torch.empty((n, h, w, co), dtype=torch.uint8 if relu else torch.int8, device=dev)
    if n:
        with _on(dev):
            _check(lib().xdna_conv3x3_i8(_ptr(xq), n, h, w, c_pad, _ptr(wq), co, int(shift), int(bool(relu)),
                                         _ptr(y), None, _stream(dev)), "conv3x3_i8")
    return y


def conv3x3_calibrate(xq, wq, relu):
    """max(acc, 0) (relu) or max |acc| over the int32 sums of NHWC xq; synchronizes (first call only)."""
    dev = _need_gpu(xq, wq)
    n, h, w, c_pad = xq.shape
    co = wq.shape[0]
    top = torch.empty((1,), dtype=torch.int32, device=dev)
    with _on(dev):
        _check(lib().xdna_conv3x3_i8(_ptr(xq), n, h, w, c_pad, _ptr(wq), co, 1, int(bool(relu)), None, _ptr(top),
                                     _stream(dev)), "conv3x3_i8 (calibrate)")
    return int(top.item())


def conv_dequant(q, relu, scale, sx, bias, out_dtype):
    """NHWC q [N, H, W, Co] -> NCHW y = q * (scale[co] * sx[n]) (+ bias[co]) as out_dtype."""
    dev = _need_gpu(q, scale, sx, bias)
    n, h, w, co = q.shape
    y = torch.empty((n, co, h, w), dtype=out_dtype, device=dev)
    if n:
        with _on(dev):
            _check(lib().xdna_conv_dequant(_ptr(q), int(bool(relu)), n, h, w, co, _ptr(scale), _ptr(sx), _ptr(bias),
                                           _ptr(y), _DTYPE_CODE[out_dtype], _stream(dev)), "conv_dequant")
    return y


def conv3x3_dequant(xq, wq, shift, relu, scale, sx, bias, out_dtype):
    """conv3x3 followed by conv_dequant in one launch, bit for bit: NHWC int8 xq [N, H, W, c_pad] (*) wq
    [Co, 9, c_pad], requantized by `shift`, dequantized with scale [Co] and sx [N] (+ bias [Co]) ->
    NCHW y [N, Co, H, W] as out_dtype."""
    dev = _need_gpu(xq, wq, scale, sx, bias)
    n, h, w, c_pad = xq.shape
    co = wq.shape[0]
    y = torch.empty((n, co, h, w), dtype=out_dtype, device=dev)
    if n:
        with _on(dev):
            _check(lib().xdna_conv3x3_dequant(_ptr(xq), n, h, w, c_pad, _ptr(wq), co, int(shift), int(bool(relu)),
                                              _ptr(scale), _ptr(sx), _ptr(bias), _ptr(y), _DTYPE_CODE[out_dtype],
                                              _stream(dev)), "conv3x3_dequant")
    return y


def conv_requant_next(q, relu, pool, scale, sx, bias, x_dtype, c_pad_next, relu_y=False):
    """Conv chaining: NHWC q [N, H, W, Co] of one conv -> (NHWC int8 [N, H', W', c_pad_next], sx [N])
    for the next, equal to dequantize (cast to x_dtype) -> [ReLU if relu_y] -> [2x2 max-pool] ->
    per-image quantize."""
    dev = _need_gpu(q, scale, sx, bias)
    n, h, w, co = q.shape
    ho, wo = (h // 2, w // 2) if pool else (h, w)
    xq = torch.empty((n, ho, wo, c_pad_next), dtype=torch.int8, device=dev)
    sxn = torch.empty((n,), dtype=torch.float32, device=dev)
    ws = torch.empty((n, AMAX_WS_PER_IMAGE), dtype=torch.float32, device=dev)
    if n:
        with _on(dev):
            _check(lib().xdna_conv_requant_next(_ptr(q), int(bool(relu)), int(bool(relu_y)), int(bool(pool)), n, h, w,
                                                co, _ptr(scale), _ptr(sx), _ptr(bias), _DTYPE_CODE[x_dtype], _ptr(xq),
                                                c_pad_next, _ptr(sxn), _ptr(ws), _stream(dev)), "conv_requant_next")
    return xq, sxn


def nchw_to_nhwc(xq, c_pad):
    """int8 NCHW [N, C, H, W] -> NHWC [N, H, W, c_pad] (zero channels past C)."""
    dev = _need_gpu(xq)
    xq = xq.contiguous()
    n, c, h, w = xq.shape
    out = torch.empty((n, h, w, c_pad), dtype=torch.int8, device=dev)
    if n:
        with _on(dev):
            _check(lib().xdna_nchw_to_nhwc_i8(_ptr(xq), n, c, h, w, _ptr(out), c_pad, _stream(dev)), "nchw_to_nhwc")
    return out


def nhwc_to_nchw(q):
    """NHWC [N, H, W, C] (int8 or uint8) -> NCHW [N, C, H, W] of the same dtype."""
    dev = _need_gpu(q)
    q = q.contiguous()
    n, h, w, c = q.shape
    out = torch.empty((n, c, h, w), dtype=q.dtype, device=dev)
    if n:
        with _on(dev):
            _check(lib().xdna_nhwc_to_nchw_i8(_ptr(q), n, c, h, w, _ptr(out), _stream(dev)), "nhwc_to_nchw")
    return out


# ------------------------------------------------------------------------------ qwen3 stack pieces
def _wcode(t):
    return _DTYPE_CODE[t.dtype]


def rmsnorm_bf16(x, w, eps):
    """bf16(w * (x * rsqrt(mean(x^2) + eps))) of float32 rows x [R, D] (D a multiple of 256)."""
    dev = _need_gpu(x, w)
    R, D = x.shape
    y = torch.empty((R, D), dtype=torch.bfloat16, device=dev)
    if R:
        with _on(dev):
            _check(lib().xdna_rmsnorm_bf16(_ptr(x), R, D, _ptr(w), _wcode(w), float(eps), _ptr(y), _stream(dev)),
                   "rmsnorm_bf16")
    return y


def add_rmsnorm_bf16(x, a, w, eps):
    """x += a, then rmsnorm_bf16(x, w, eps), in one launch (x, a float32 [R, D], contiguous; D a multiple
    of 256): the same values as add_ followed by rmsnorm_bf16."""
    dev = _need_gpu(x, a, w)
    R, D = x.shape
    if a.shape != x.shape or not (x.is_contiguous() and a.is_contiguous()):
        raise ValueError("add_rmsnorm_bf16: x and a must be contiguous tensors of one shape")
    y = torch.empty((R, D), dtype=torch.bfloat16, device=dev)
    if R:
        with _on(dev):
            _check(lib().xdna_add_rmsnorm_bf16(_ptr(x), _ptr(a), R, D, _ptr(w), _wcode(w), float(eps), _ptr(y),
                                               _stream(dev)), "add_rmsnorm_bf16")
    return y


def qk_norm_rope(qkv, nh, nkv, q_w, k_w, inv_freq, pos, vt_col, eps, vt):
    """Per token of qkv float32 [T, (nh + 2 nkv) * 128]: q / k heads RMSNorm'd and rotated (RoPE at
    pos), v heads written transposed into vt [nkv, 128, ld_vt] at columns vt_col. Returns bf16
    (q [T, nh, 128], k [T, nkv, 128])."""
    dev = _need_gpu(qkv, q_w, k_w, inv_freq, pos, vt_col, vt)
    T = qkv.shape[0]
    q = torch.empty((T, nh, 128), dtype=torch.bfloat16, device=dev)
    k = torch.empty((T, nkv, 128), dtype=torch.bfloat16, device=dev)
    if T:
        with _on(dev):
            _check(lib().xdna_qk_norm_rope(_ptr(qkv), T, nh, nkv, _ptr(q_w), _ptr(k_w), _wcode(q_w), _ptr(inv_freq),
                                           _ptr(pos), _ptr(vt_col), float(eps), _ptr(q), _ptr(k), _ptr(vt),
                                           vt.shape[-1], _stream(dev)), "qk_norm_rope")
    return q, k


def attention_bf16(q, k, vt, seq_start, seq_len, seq_vt, max_len, scale):
    """Bidirectional grouped-query attention per sequence: bf16 [T, nh, 128]."""
    dev = _need_gpu(q, k, vt, seq_start, seq_len, seq_vt)
    T, nh = q.shape[:2]
    nkv = k.shape[1]
    out = torch.empty((T, nh, 128), dtype=torch.bfloat16, device=dev)
    if T:
        with _on(dev):
            _check(lib().xdna_attention_bf16(_ptr(q), _ptr(k), _ptr(vt), vt.shape[-1], _ptr(seq_start), _ptr(seq_len),
                                             _ptr(seq_vt), seq_len.shape[0], int(max_len), nh, nkv, float(scale),
                                             _ptr(out), _stream(dev)), "attention_bf16")
    return out


def silu_mul_bf16(gu):
    """bf16(silu(gate) * up) of gu float32 [T, 2 * inter] (gate columns first)."""
    dev = _need_gpu(gu)
    T, two = gu.shape
    y = torch.empty((T, two // 2), dtype=torch.bfloat16, device=dev)
    if T:
        with _on(dev):
            _check(lib().xdna_silu_mul_bf16(_ptr(gu), T, two // 2, _ptr(y), _stream(dev)), "silu_mul_bf16")
    return y


def add_(x, y):
    """x += y (float32, same shape, contiguous)."""
    dev = _need_gpu(x, y)
    if x.numel():
        with _on(dev):
            _check(lib().xdna_add_f32(_ptr(x), _ptr(y), x.numel(), _stream(dev)), "add_f32")
    return x
