"""Runtime of the xdna::linear ops: weight cache, routing GPU <-> CPU, verify, fallback, stats.

Mirrors the reference's runtime (torch_xdna/runtime.py in the reference) with the NPU replaced by
one MI355X GPU. Every offloaded GEMM is W8A8: weights per output channel, activations per row,
int8 x int8 -> int32, dequantized in fp32. The GPU route runs the HIP kernels of `kernels`
(quantize -> MFMA GEMM with the dequantize fused into its epilogue); the CPU route is the
reference's own (torch CPU quantize, torch._int_mm, dequantize). Both compute the same integers and
round the dequantize identically, so a result does not depend on where it ran.

Routing (`_choose`, the reference's runtime.py:250-268):
  * tensors already on the GPU take the GPU route unless policy="cpu" or that shape's GPU launch
    failed before; if the HIP library is missing they raise instead of silently using the CPU;
  * host tensors follow the reference's rules (policy, min_rows, min_macs, autotune per
    (precision, row bucket, N, K)), with the GPU route paying the host <-> device copies.
Verify (`_check`, runtime.py:174-188): the first GPU launch of every (kernel variant, N, K) is
compared bit for bit with the CPU route; a mismatch raises GPUResultMismatch, which moves that shape
to the CPU (`_gpu_failed`, runtime.py:275-282); three failing shapes retire the GPU.
"""

import bisect
import logging
import threading
import time
import weakref
from collections import Counter, defaultdict

import torch

from . import kernels

log = logging.getLogger("torch_xdna")
_lock = threading.RLock()


# ------------------------------------------------------------------------------ stats
class Stats:
    """Where the offloaded work went, for report(): per device ("gpu" / "cpu") the op calls, the wall
    seconds inside the ops and the multiply-accumulates; GPU kernel launches; the shapes that fell back
    to the CPU and why; whole-stack dispatches and their first-call checks. reset() clears it (the
    autotune decisions below are kept)."""

    def __init__(self):
        self.reset()

    def reset(self):
        self.calls, self.seconds, self.macs = Counter(), defaultdict(float), Counter()
        self.launches = 0
        self.fallbacks = []             # (shape or layer, error text)
        self.stacks = Counter()         # (stack name, "gpu" fused / "cpu" plain graph) -> graph calls
        self.checks = []                # (stack, relative error) of first fused calls

    def record(self, device, since, macs):
        """One op call on `device` that started at perf_counter() value `since`."""
        self.calls[device] += 1
        self.seconds[device] += time.perf_counter() - since
        self.macs[device] += macs

    def as_dict(self):
        ok, why = kernels.available(), kernels.unavailable_reason()
        d = {"calls": dict(self.calls),
             "seconds": {dev: round(t, 4) for dev, t in self.seconds.items()},
             "gmacs": {dev: round(m / 1e9, 3) for dev, m in self.macs.items()},
             "gpu_launches": self.launches, "fallbacks": list(self.fallbacks),
             "stacks": {f"{name} on {dev}": n for (name, dev), n in self.stacks.items()},
             "checks": list(self.checks),
             "decisions": {"x".join(str(p) for p in key): v for key, v in decisions.items()},
             "gpu_available": ok, "gpu_unavailable_reason": why}
        # the reference's names for the same figures
        d.update(npu_launches=d["gpu_launches"], npu_available=ok, npu_unavailable_reason=why)
        return d


# Autotune results outlive stats.reset(): key -> (device, gpu_ms, cpu_ms)
decisions = {}
stats = Stats()


# ------------------------------------------------------------------------------ weights
class QWeight:
    """One weight (or several concatenated on the output dim), quantized once per device.

    `gpu(dev)`: int8 [N, Kp] (K zero-padded to a multiple of 16, K contiguous) and sw [N] on the GPU,
    quantized there by the HIP kernel. `cpu()`: the reference's int8 [K, N] (`w_kn`, for
    torch._int_mm) and sw on the CPU (runtime.py:59-66). Both hold the same integers and scales.
    """

    def __init__(self, ws, transposed: bool):
        self.srcs = [w.detach() for w in ws]
        self.transposed = transposed
        self.sizes = [int(w.shape[1] if transposed else w.shape[0]) for w in ws]
        self.N = sum(self.sizes)
        self.K = int(ws[0].shape[0] if transposed else ws[0].shape[1])
        self.Kp = kernels.round_up(self.K, 16)
        self._gpu = {}
        self._gpu_bf16 = {}
        self._cpu = None

    def _rows(self, w, dev):
        """The weight as [N_i, K] K-contiguous rows of a float dtype the kernel reads, on dev."""
        w = w.to(dev)
        if w.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            w = w.float()
        if self.transposed:      # given as [K, N] (x @ W): one-time transposed copy
            w = w.t()
        return w.contiguous()

    def gpu(self, dev):
        hit = self._gpu.get(dev)
        if hit is None:
            wq = torch.empty((self.N, self.Kp), dtype=torch.int8, device=dev)
            sw = torch.empty((self.N,), dtype=torch.float32, device=dev)
            r0 = 0
            for w, n in zip(self.srcs, self.sizes):
                kernels.quant_rows(self._rows(w, dev), self.Kp, out=(wq[r0:r0 + n], sw[r0:r0 + n]))
                r0 += n
            hit = self._gpu[dev] = (wq, sw)
        return hit

    def gpu_bf16(self, dev):
        """bf16 [N, Kp] copy of the float weight on dev for precision "bf16" (QWeight.npu_bf16,
        runtime.py:80-86): round to nearest even, zero columns past K; made on first use."""
        hit = self._gpu_bf16.get(dev)
        if hit is None:
            wb = torch.zeros((self.N, self.Kp), dtype=torch.bfloat16, device=dev)
            r0 = 0
            for w, n in zip(self.srcs, self.sizes):
                wb[r0:r0 + n, :self.K].copy_(self._rows(w, dev))
                r0 += n
            hit = self._gpu_bf16[dev] = wb
        return hit

    def cpu(self):
        if self._cpu is None:
            wf = torch.cat([w.cpu().float() for w in self.srcs], dim=1 if self.transposed else 0)
            if self.transposed:
                wf = wf.t()
            sw = wf.abs().amax(dim=1).clamp(min=1e-8) / 127
            q = torch.round(wf / sw[:, None]).clamp(-127, 127).to(torch.int8)
            self._cpu = (q.t().contiguous(), sw)
        return self._cpu

    def sw(self, dev):
        """The weight scales [N] on dev (a fresh tensor is the caller's job)."""
        if dev.type == "cuda":
            return self.gpu(dev)[1]
        return self.cpu()[1]

    def w_fp(self):
        """The float weight [N, K] (precision bf16 / cpu_kernel fp routes)."""
        ws = [w.t() if self.transposed else w for w in self.srcs]
        return ws[0] if len(ws) == 1 else torch.cat(ws)


class _WeightCache:
    """QWeights by their source weights' identity: (data_ptr, shape, _version) of every weight and the
    transposed flag (runtime.py:99-110), so an in-place update (a new _version) quantizes again. An
    entry also checks that its weights are the very tensors it was made from (a freed tensor's memory
    can be reused by another) and is dropped when one of them is garbage-collected."""

    def __init__(self):
        self.entries = {}

    def clear(self):
        self.entries.clear()

    def __len__(self):
        return len(self.entries)

    def get(self, ws, transposed):
        key = (tuple((w.data_ptr(), tuple(w.shape), w._version) for w in ws), transposed)
        hit = self.entries.get(key)
        if hit is not None and all(alive() is w for alive, w in zip(hit[0], ws)):
            return hit[1]
        qw = QWeight(ws, transposed)

        def drop(_, key=key, qw=qw):    # only this entry: the key may have been reused since
            if self.entries.get(key, (None, None))[1] is qw:
                del self.entries[key]

        alive = []
        for w in ws:
            try:
                alive.append(weakref.ref(w, drop))
            except TypeError:           # not weak-referenceable: kept alive by the entry
                alive.append(lambda w=w: w)
        self.entries[key] = (alive, qw)
        return qw


_weights = _WeightCache()


def qweight(ws, transposed: bool = False) -> QWeight:
    """The cached QWeight of one weight, or of several concatenated on N (the fused linears)."""
    ws = list(ws) if isinstance(ws, (list, tuple)) else [ws]
    with _lock:
        return _weights.get(ws, transposed)


# ------------------------------------------------------------------------------ the CPU route
def _quant_rows(x2d):
    """runtime.py:145-148."""
    x = x2d.float()
    s = x.abs().amax(dim=1).clamp(min=1e-8) / 127
    return torch.round(x / s[:, None]).clamp(-127, 127).to(torch.int8), s


def _bucket(rows, buckets):
    """The smallest row bucket that holds `rows` (the largest when none does): the row group of the
    reference's autotune and verify keys."""
    i = bisect.bisect_left(buckets, rows)
    return buckets[min(i, len(buckets) - 1)]


def _cpu_acc(xq, qw):
    """runtime.py:162-163: exact int32 sums on the CPU."""
    return torch._int_mm(xq.cpu(), qw.cpu()[0])


def _dequant(acc, sx, sw, bias, dtype):
    """runtime.py:350-353: ((acc * sx) * sw) + bias in fp32, then the output dtype."""
    y = acc.float() * sx[:, None] * sw[None, :]
    if bias is not None:
        y += bias.float()
    return y.to(dtype)


def _cpu_linear(x2d, qw, bias, dtype):
    xq, sx = _quant_rows(x2d.cpu())
    acc = torch._int_mm(xq, qw.cpu()[0])
    return _dequant(acc, sx, qw.cpu()[1], None if bias is None else bias.cpu(), dtype)


# ------------------------------------------------------------------------------ the GPU route
_verified = {}    # program key -> True once a launch of it matched the CPU


class GPUResultMismatch(RuntimeError):
    """A GPU program returned something the CPU route disagrees with."""


NPUResultMismatch = GPUResultMismatch   # the reference's name


def _program(cfg, kind, dev, R, qw, dtype=None):
    """The verify key of a GPU GEMM call: what the reference's key names for an NPU program
    (runtime.py:207: dtype, row bucket, Np, Kp, tiling), here the kernel kind, the library's launch
    plan for these rows (head tile, and a tail split's first row and tile), the row bucket, N, K and
    the output dtype."""
    tk = kernels.KIND_BF16 if kind == "bf16" else kernels.KIND_I8
    plan = kernels.gemm_variant(dev, R, qw.N, qw.Kp, tk)
    return (kind, plan, _bucket(R, cfg.row_buckets), qw.N, qw.K, None if dtype is None else str(dtype))


def _check(cfg, key, got, want, exact=True):
    """Compare one launch with the CPU route unless this program was already verified (Config.verify
    "first"; "always" checks every launch, "off" none): bit for bit, or (exact=False, the bf16 GEMM)
    to the reference's 5e-2 relative norm with finite values (runtime.py:174-188)."""
    if cfg.verify == "off" or (cfg.verify == "first" and _verified.get(key)):
        return
    want = want()
    got = got.cpu()
    if not exact:
        err = ((got.float() - want.float()).norm() / want.float().norm().clamp(min=1e-30)).item()
        if not (bool(torch.isfinite(got).all()) and err < 5e-2):
            raise GPUResultMismatch(f"GPU program {key} disagrees with the CPU: rel err {err:.3g}, "
                                    f"non-finite {int((~torch.isfinite(got)).sum())}")
        _verified[key] = True
        return
    if not torch.equal(got, want):
        bad = (got != want)
        if got.is_floating_point():
            bad = bad & ~(torch.isnan(got) & torch.isnan(want))
        if bad.any():
            raise GPUResultMismatch(f"GPU program {key} disagrees with the CPU: "
                                    f"{int(bad.sum())} of {got.numel()} values differ")
    _verified[key] = True


def _gpu_linear(cfg, x2d, qw, bias, dtype):
    """y [R, N] = W8A8(x2d) on the GPU: quantize kernel, then the GEMM with the fused dequantize; a single
    row (decode) whose layout allows it as one launch that quantizes the row itself (xdna_linear_row)."""
    dev = kernels.gpu_device(x2d)
    xg = x2d.to(dev)
    wq, sw = qw.gpu(dev)
    b = None if bias is None else bias.to(dev, torch.float32).contiguous()
    if kernels.linear_row_ok(xg, qw.Kp):
        y = kernels.linear_row(xg, wq, sw, b, dtype)
        key = ("row", "rowq", _bucket(1, cfg.row_buckets), qw.N, qw.K, str(dtype))
    else:
        xq, sx = kernels.quant_rows(xg, qw.Kp)
        y = kernels.mm_i8_dequant(xq, sx, wq, sw, b, dtype)
        key = _program(cfg, "dq", dev, x2d.shape[0], qw, dtype)
    stats.launches += 1
    _check(cfg, key, y, lambda: _cpu_linear(x2d, qw, bias, dtype))
    return y


def _gpu_bf16(cfg, x2d, qw, bias, dtype):
    """y [R, N] of precision "bf16" on the GPU: bf16 operands, float32 accumulation and bias, cast to
    dtype, one kernel (runtime.py:212-237, :299-313)."""
    dev = kernels.gpu_device(x2d)
    xb = kernels.bf16_rows(x2d.to(dev), qw.Kp)
    wb = qw.gpu_bf16(dev)
    b = None if bias is None else bias.to(dev, torch.float32).contiguous()
    y = kernels.mm_bf16(xb, wb, b, dtype)
    stats.launches += 1

    def want():     # the reference's check: the bf16 operands multiplied in float32 (runtime.py:233-234)
        yb = xb[:, :qw.K].cpu().float() @ wb[:, :qw.K].cpu().float().t()
        if bias is not None:
            yb += bias.cpu().float()
        return yb.to(dtype)
    _check(cfg, _program(cfg, "bf16", dev, x2d.shape[0], qw, dtype), y, want, exact=False)
    return y


def _cpu_bf16(x2d, w_fp, bias, dtype):
    """The reference's CPU route of precision "bf16": the float32 GEMM (runtime.py:306-313)."""
    y = x2d.cpu().float() @ w_fp.cpu().float().t()
    if bias is not None:
        y += bias.cpu().float()
    return y.to(dtype)


def _gpu_acc(cfg, xq, qw):
    """int32 [R, N] on the GPU from int8 [R, K] (xdna::linear_i8)."""
    dev = kernels.gpu_device(xq)
    wq, _ = qw.gpu(dev)
    a = kernels.pad_k(xq.to(dev), qw.Kp)
    acc = kernels.mm_i8(a, wq)
    stats.launches += 1
    _check(cfg, _program(cfg, "i8", dev, xq.shape[0], qw), acc, lambda: _cpu_acc(xq, qw))
    return acc


# ------------------------------------------------------------------------------ routing
def _time(fn, reps=3):
    """One warm call, then the best of `reps` (runtime.py:240-247), synchronizing the GPU."""
    def run():
        out = fn()
        if torch.cuda.is_available():
            torch.cuda.synchronize()
        return out
    run()
    best = float("inf")
    for _ in range(reps):
        t = time.perf_counter()
        run()
        best = min(best, time.perf_counter() - t)
    return best * 1e3


_failed = set()          # shapes whose GPU launch raised or mismatched: CPU from then on
MAX_GPU_FAILURES = 3     # distinct failing shapes before the GPU is retired for the process
MAX_NPU_FAILURES = MAX_GPU_FAILURES


def _key(cfg, R, qw):
    return (cfg.precision, _bucket(R, cfg.row_buckets), qw.N, qw.K)


def _require_lib():
    """A GPU tensor needs the HIP library: never route it to the CPU because the library is missing."""
    if not kernels.available():
        reason = kernels.unavailable_reason() or ""
        if "not built" in reason or "ABI version" in reason:
            raise RuntimeError(f"torch_xdna: GPU tensor but the HIP library is unusable: {reason}")


def _choose(cfg, R, qw, on_gpu, gpu_fn, cpu_fn):
    """'gpu' or 'cpu' for a call of R rows; gpu_fn / cpu_fn run it on either (for autotune)."""
    if cfg.policy == "cpu":
        return "cpu"
    if kernels.available():
        kernels.use_tuned(cfg.tuned_tilings)
    if on_gpu:
        _require_lib()
        if not kernels.available() or _key(cfg, R, qw) in _failed:
            return "cpu"
        return "gpu"
    if R < cfg.min_rows or R * qw.N * qw.K < cfg.min_macs:
        return "cpu"
    if not kernels.available():
        return "cpu"
    key = _key(cfg, R, qw)
    if key in _failed:
        return "cpu"
    if cfg.policy == "gpu":
        return "gpu"
    hit = decisions.get(key)
    if hit is None:
        gpu_ms, cpu_ms = _time(gpu_fn), _time(cpu_fn)
        hit = ("gpu" if gpu_ms < cpu_ms else "cpu", round(gpu_ms, 3), round(cpu_ms, 3))
        decisions[key] = hit
        if cfg.verbose:
            log.warning("torch_xdna autotune %s: gpu %.3f ms, cpu %.3f ms -> %s", key, gpu_ms, cpu_ms, hit[0])
    return hit[0]


def _gpu_failed(cfg, R, qw, e):
    shape = _key(cfg, R, qw)
    _failed.add(shape)
    stats.fallbacks.append((shape, f"{type(e).__name__}: {e}"[:300]))
    log.warning("torch_xdna: GPU GEMM %s failed (%s); it runs on the CPU from now on", shape, e)
    if len(_failed) >= MAX_GPU_FAILURES:
        kernels.mark_broken(e)
        log.warning("torch_xdna: %d GPU failures, GPU retired for this process", len(_failed))


def _float_only(cfg):
    """cpu_kernel "fp" with no GPU route: the op is the float linear itself."""
    return cfg.cpu_kernel == "fp" and (cfg.policy == "cpu" or not kernels.available())


# ------------------------------------------------------------------------------ the ops
def _linear_impl(cfg, x, qw, bias, w_fp_fn):
    """Shared body of linear / linear_cat (runtime.py:326-355, :402-434)."""
    shape = x.shape[:-1]
    x2d = x.reshape(-1, x.shape[-1])
    R = x2d.shape[0]
    on_gpu = x.device.type == "cuda"
    t0 = time.perf_counter()
    if cfg.precision == "bf16":
        # runtime.py:299-313 / :340-345: the bf16 GEMM on the GPU, the float32 GEMM on the CPU
        with _lock:
            device = _choose(cfg, R, qw, on_gpu, lambda: _gpu_bf16(cfg, x2d, qw, bias, x.dtype),
                             lambda: _cpu_bf16(x2d, w_fp_fn(), bias, x.dtype))
            y = None
            if device == "gpu":
                try:
                    y = _gpu_bf16(cfg, x2d, qw, bias, x.dtype)
                except Exception as e:
                    _gpu_failed(cfg, R, qw, e)
                    device = "cpu"
            if y is None:
                y = _cpu_bf16(x2d, w_fp_fn(), bias, x.dtype)
        stats.record(device, t0, R * qw.N * qw.K)
        return y.to(x.device).reshape(*shape, qw.N)
    with _lock:
        device = _choose(cfg, R, qw, on_gpu, lambda: _gpu_linear(cfg, x2d, qw, bias, x.dtype),
                         lambda: _cpu_linear(x2d, qw, bias, x.dtype))
        y = None
        if device == "gpu":
            try:
                y = _gpu_linear(cfg, x2d, qw, bias, x.dtype)
            except Exception as e:  # launch failure or mismatch: this shape moves to the CPU
                _gpu_failed(cfg, R, qw, e)
                device = "cpu"
        if y is None:
            if cfg.cpu_kernel == "fp":
                y = torch.nn.functional.linear(x2d.cpu(), w_fp_fn().cpu().to(x.dtype),
                                               None if bias is None else bias.cpu())
            else:
                y = _cpu_linear(x2d, qw, bias, x.dtype)
    stats.record(device, t0, R * qw.N * qw.K)
    return y.to(x.device).reshape(*shape, qw.N)


def linear(cfg, x, weight, bias, transposed):
    """y = x @ W^T + b (or x @ W when transposed) with W8A8 math on the chosen device."""
    N = weight.shape[1] if transposed else weight.shape[0]
    if x.numel() == 0 or x.reshape(-1, x.shape[-1]).shape[0] == 0:
        return x.new_zeros(*x.shape[:-1], N)
    w_fp = weight.t() if transposed else weight
    if _float_only(cfg):
        return torch.nn.functional.linear(x, w_fp.to(x.dtype), bias)
    qw = qweight(weight, transposed)
    return _linear_impl(cfg, x, qw, bias, lambda: w_fp)


def linear_cat(cfg, x, weights, biases):
    """torch.cat([F.linear(x, w, b) for w, b in zip(weights, biases)], -1) as one W8A8 GEMM."""
    N = sum(w.shape[0] for w in weights)
    if x.reshape(-1, x.shape[-1]).shape[0] == 0:
        return x.new_zeros(*x.shape[:-1], N)
    if any(b is not None for b in biases):
        bias = torch.cat([b if b is not None else w.new_zeros(w.shape[0]) for w, b in zip(weights, biases)])
    else:
        bias = None
    if _float_only(cfg):
        return torch.nn.functional.linear(x, torch.cat(list(weights)).to(x.dtype), bias)
    qw = qweight(list(weights))
    return _linear_impl(cfg, x, qw, bias, lambda: torch.cat(list(weights)))


def linear_int8(x, weights, biases, transposed: bool, cfg_id: int):
    """torch.cat([F.linear(x, w, b) ...], -1) through W8A8: what the backend puts in the graph
    (runtime.py:358-374).

    On the CPU only the integer GEMM is a custom op (xdna::linear_i8) and the quantize / dequantize
    are ordinary torch ops that Inductor fuses with their neighbours, as in the reference. On the GPU
    the whole linear stays one opaque op (xdna::linear / xdna::linear_cat), whose HIP kernels fuse
    the dequantize into the GEMM; Inductor then generates nothing for the hot path.
    """
    if x.device.type == "cuda":
        if len(weights) == 1:
            return torch.ops.xdna.linear(x, weights[0], biases[0], transposed, cfg_id)
        return torch.ops.xdna.linear_cat(x, list(weights), list(biases), cfg_id)
    x2 = x.reshape(-1, x.shape[-1])
    sx = x2.abs().amax(dim=1, keepdim=True).float().clamp(min=1e-8) / 127
    xq = torch.round(x2.float() / sx).clamp(-127, 127).to(torch.int8)
    acc, sw = torch.ops.xdna.linear_i8(xq, weights, transposed, cfg_id)
    y = acc.float() * sx * sw
    if any(b is not None for b in biases):
        sizes = [w.shape[1] if transposed else w.shape[0] for w in weights]
        y = y + torch.cat([b.float() if b is not None else y.new_zeros(n) for b, n in zip(biases, sizes)])
    return y.to(x.dtype).reshape(*x.shape[:-1], y.shape[-1])


def linear_i8(cfg, xq, weights, transposed):
    """(int32 acc [R, N], weight scales [N]) of xdna::linear_i8 (runtime.py:377-399): the integer GEMM of
    an already quantized activation, on the device _choose picks; a GPU failure moves the shape to the
    CPU. The scales are a fresh tensor: Inductor may reuse an extern op's output buffer once it is dead."""
    t0 = time.perf_counter()
    qw = qweight(list(weights), transposed)
    dev = xq.device
    R = xq.shape[0]
    if R == 0:
        return xq.new_zeros((0, qw.N), dtype=torch.int32), qw.sw(dev).to(dev).clone()
    with _lock:
        device = _choose(cfg, R, qw, dev.type == "cuda", lambda: _gpu_acc(cfg, xq, qw), lambda: _cpu_acc(xq, qw))
        acc = None
        if device == "gpu":
            try:
                acc = _gpu_acc(cfg, xq, qw)
            except Exception as e:      # launch failure or mismatch
                _gpu_failed(cfg, R, qw, e)
                device = "cpu"
        if acc is None:
            acc = _cpu_acc(xq, qw)
    stats.record(device, t0, R * qw.N * qw.K)
    sw = qw.gpu(kernels.gpu_device(xq))[1] if device == "gpu" else qw.cpu()[1]
    return acc.to(dev), sw.to(dev).clone()
