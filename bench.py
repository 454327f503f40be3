"""Benchmark of the int8 hot path on one MI355X: W8A8 GEMM and int8 conv3x3 TOPS vs the rooflines.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload headline|c1|c2|c3|c4|c5|...]

One step is one pass of the hot path over one batch of synthetic, seeded input (BASELINE.json
configs; seed 0), with inputs and device-resident int8 weights already in HBM:

  headline (default)  the largest single-GPU config, C5's M=8192 W8A8 linear: bf16 x [8192, 4096]
                with 0.1% outliers x20 -> per-row quantize -> int8 MFMA GEMM against the int8
                weight [14336, 4096] with the dequantize + bias fused into its epilogue -> bf16 y.
                The same JSON line carries sub-records, each with its own roofline and CPU
                baseline: C4's 256-channel conv at 1x256x1536x64 and 8x256x256x256 run as the op
                (xdna::conv3x3_fused: per-image quantize -> conv with the calibrated shift ->
                dequantize, ReLU fused), with the conv kernel's back-to-back time beside it; C2; the
                decode GEMMs (HBM-bound); the activation quantize alone at bf16 8192 x 14336 and
                8192 x 4096 (HBM-bound); the C3 chain end to end; and VGG-16's features at batch 8.
  c2            Qwen3-0.6B projections as xdna::linear_cat runs them on the GPU: for M in
                {128, 512, 1024, 3000}, bf16 x -> quantize -> fused GEMM -> bf16, for qkv
                (N 4096, K 1024), gate/up (N 6144, K 1024) and down (N 1024, K 3072).
  c1            one W8A8 linear, fp32 x [128, 1024], W [3072, 1024], bias.
  c3            4 x (conv3x3 + ReLU), 256 ch, 1x256x64x64, chained on the GPU.
  c4            C4's two 256-channel convs as the op (the headline's sub-records alone).
  c5            the headline's main record alone.
  decode        the C5 decode GEMMs (M 1 and 16), HBM-bound: roofline in GB/s of algorithmic bytes.
  quant         the activation quantize kernel alone, bf16 [8192, 14336] and [8192, 4096].
  bf16          precision "bf16" on the C2 shapes: the bf16 MFMA GEMM (bf16 in / out, float32 sums).
  vgg16         VGG-16 features at batch 8 through torch.compile(backend="xdna"), convs chained.
  stack         xdna::qwen3_stack on OmniVoice's step shapes.
  copy          calibration of the HBM byte counters (a 1 GiB read + 1 GiB write elementwise kernel).

Weight / activation sets are rotated so a step's working set exceeds the 256 MB MALL. Timing:
W untimed steps, then K steps bracketed by torch.cuda.synchronize(); the dominant kernel is also
timed per launch with HIP events on the stream it runs on (torch's current stream). The timed
steps are enqueued behind a GPU spin kernel that outlasts the host's enqueue time, so they run back
to back and the events measure GPU time only; the ungated wall-clock time per step (host launch
cost included) is reported beside it. Rank 0 prints one JSON line.

CPU baseline: the reference's CPU route (oracle/cpu_route.py: torch CPU quantize, torch._int_mm or
an exact float conv of the integers, dequantize) on the GPU box's host cores, timed by the
reference's protocol (tools/cpu_baseline.py:14-26: 5 warm-up runs, then 60 timed runs, min / p25 /
median) with as many torch threads as the process has CPUs (and at the reference's 16 beside it when
that differs), with the thread count, os.cpu_count() and the CPU model; each record says what its
sample is.
"""

import argparse
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "torch-xdna_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

from torch_xdna import kernels  # noqa: E402

PEAK_INT8_TOPS = 5000.0     # MI355X dense int8 MFMA, TOP/s (5.0 POP/s)
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA, TFLOP/s
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E, GB/s
MALL_BYTES = 256 << 20
METRIC = "W8A8 GEMM & int8 conv3x3 TOPS on 1 MI355X; % of int8 MFMA peak / HBM BW"
WORKLOADS = ["headline", "c1", "c2", "c3", "c4", "c5", "decode", "quant", "bf16", "vgg16", "stack", "copy", "libref"]


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="headline", choices=WORKLOADS)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--operands", default="randn", choices=["randn", "zeros"],
                    help="zeros: all-zero activations and weights on the GEMM workloads (a diagnostic of the power "
                         "limit: the same work with the least switching; never the reported configuration)")
    ap.add_argument("--tile", default=None,
                    help="force this tile (a kernels.TILES name) on every GEMM shape of the c1/c2/c5/decode "
                         "workloads instead of the built-in rule and the tuned table (results do not depend on it)")
    return ap.parse_args()


def gen(seed):
    return torch.Generator().manual_seed(seed)


# ------------------------------------------------------------------------------ GEMM workloads
def gemm_sets(shapes, dev, nsets_min=1, x_dtype=torch.bfloat16, bias=False, seed=0, zeros=False):
    """Per set: for each (M, N, K): x [M, K] (0.1% outliers x20), quantized weight [N, K] + sw
    (+ bias) on the GPU. zeros: x and the weight all zero (int8 operands all zero: the same work with
    the least switching in the MFMA units, to separate the power limit from the schedule's own)."""
    g = gen(seed)
    per_set = sum(M * K * x_dtype.itemsize + N * K + M * N * 2 + M * K for M, N, K in shapes)
    nsets = max(nsets_min, -(-(MALL_BYTES + (64 << 20)) // per_set))
    sets = []
    for _ in range(nsets):
        items = []
        for M, N, K in shapes:
            x = torch.randn(M, K, generator=g)
            x = torch.where(torch.rand(M, K, generator=g) < 1e-3, x * 20, x).to(x_dtype).to(dev)
            w = (torch.randn(N, K, generator=g) * 0.02).to(dev)
            if zeros:
                x.zero_()
                w.zero_()
            b = (torch.randn(N, generator=g) * 0.01).to(dev) if bias else None
            wq, sw = kernels.quant_rows(w)
            items.append((x, wq, sw, b, M, N, K))
        sets.append(items)
    torch.cuda.synchronize()
    return sets


def row_fused(x, wq):
    """Whether the route runs this shape as one launch that quantizes its single row itself
    (xdna_linear_row: decode, M = 1), as runtime._gpu_linear decides."""
    return kernels.linear_row_ok(x, wq.shape[1])


def run_gemm_step_split(items, ev=None):
    """One step ordered as all activation quantizes, then all fused GEMMs (the same work as
    quantize -> GEMM per shape; a single row, which the route quantizes inside its GEMM launch, has
    no quantize launch and runs with the GEMMs); ev = three events recorded at the start, between the
    two groups and at the end, so ev[1] -> ev[2] brackets exactly the step's GEMM launches, back to back."""
    if ev:
        ev[0].record()
    qs = [None if row_fused(x, wq) else kernels.quant_rows(x) for x, wq, sw, b, M, N, K in items]
    if ev:
        ev[1].record()
    for (x, wq, sw, b, M, N, K), q in zip(items, qs):
        if q is None:
            kernels.linear_row(x, wq, sw, b, x.dtype)
        else:
            kernels.mm_i8_dequant(q[0], q[1], wq, sw, b, x.dtype)
    if ev:
        ev[2].record()


def gemm_bytes(M, N, K, xbytes, ybytes, bias, fused=False):
    """Algorithmic HBM bytes of the fused-epilogue GEMM launch: A int8 + W int8 + sx + sw (+ bias) + y;
    fused (a single row quantized inside the launch): the float row instead of A int8 and sx."""
    a = M * K * xbytes if fused else M * K + 4 * M
    return a + N * K + 4 * N + (4 * N if bias else 0) + M * N * ybytes


def quant_bytes(M, K, xbytes):
    return M * K * xbytes + M * K + 4 * M


# ------------------------------------------------------------------------------ CPU baseline
def cpu_host():
    """The host CPU the baseline ran on: /proc/cpuinfo's model string (with family / model / stepping), the
    logical CPUs the OS reports (os.cpu_count()) and those this process may run on (its affinity mask)."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k in ("model name", "cpu family", "model", "stepping", "cpu MHz", "cache size") and k not in info:
                    info[k] = v
                if not line.strip() and "model name" in info:
                    break
    except OSError:
        pass
    if "model name" not in info:
        import platform

        info["model name"] = platform.processor() or "unknown"
    ncpu = os.cpu_count() or 1
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = ncpu
    return {"cpu_model": info.pop("model name"), "cpuinfo": info, "os_cpu_count": ncpu, "affinity_cpus": aff}


# The reference's CPU baseline ran 16 threads (tools/cpu_baseline.py:11); ours runs as many threads as the
# process has CPUs (os.cpu_count(), bounded by the affinity mask: more threads than CPUs only oversubscribe),
# with the 16-thread figure beside it when the two differ.
REF_THREADS = 16


def cpu_threads():
    h = cpu_host()
    return max(1, min(h["os_cpu_count"], h["affinity_cpus"]))


def _time_protocol(step, warmup, reps, budget_s):
    for _ in range(warmup):
        step()
    ts = []
    t_end = time.perf_counter() + budget_s
    while len(ts) < reps and (time.perf_counter() < t_end or len(ts) < 10):
        t = time.perf_counter()
        step()
        ts.append(time.perf_counter() - t)
    ts.sort()
    return ts


def cpu_protocol(step, ops, sample, budget_s=20.0, warmup=5, reps=60, unit="TOPS"):
    """Times `step` by the reference's protocol (tools/cpu_baseline.py:14-26): `warmup` untimed runs,
    then `reps` timed runs (fewer when they would exceed budget_s, at least 10), min / p25 / median, with
    torch's CPU threads set to the process's CPUs (cpu_threads()). value = ops / min time, in TOPS (or
    TFLOP/s for a float route), or GB/s when unit is "GB/s" (ops then counts bytes). When that thread count
    is not the reference's 16, the same protocol at 16 threads follows (budget_s / 2), as at_16_threads."""
    scale = 1e9 if unit == "GB/s" else 1e12
    saved = torch.get_num_threads()
    nthr = cpu_threads()
    rank = lambda ts, p: ts[int(p * len(ts))]   # noqa: E731  (ts[15] / ts[30] of 60, as the reference)
    try:
        torch.set_num_threads(nthr)
        ts = _time_protocol(step, warmup, reps, budget_s)
        rec = {"value": round(ops / ts[0] / scale, 3), "unit": unit, "cores": nthr, "kind": "port",
               "sample": sample, **cpu_host(), "threads_set": f"torch.set_num_threads({nthr})",
               "warmup": warmup, "reps": len(ts), "min_ms": round(ts[0] * 1e3, 3),
               "p25_ms": round(rank(ts, 0.25) * 1e3, 3), "median_ms": round(rank(ts, 0.5) * 1e3, 3)}
        if nthr != REF_THREADS:
            torch.set_num_threads(REF_THREADS)
            t16 = _time_protocol(step, min(warmup, 2), reps, budget_s / 2)
            rec["at_16_threads"] = {"value": round(ops / t16[0] / scale, 3), "min_ms": round(t16[0] * 1e3, 3),
                                    "median_ms": round(rank(t16, 0.5) * 1e3, 3), "reps": len(t16)}
    finally:
        torch.set_num_threads(saved)
    return rec


def cpu_baseline_gemm(shapes, x_dtype, bias, label, budget_s=20.0):
    """The reference's CPU route (oracle/cpu_route.py: quantize, torch._int_mm, dequantize + bias) on
    the same shapes, one step per timed run."""
    from oracle import cpu_route

    g = gen(1)
    data = []
    for M, N, K in shapes:
        x = torch.randn(M, K, generator=g)
        x = torch.where(torch.rand(M, K, generator=g) < 1e-3, x * 20, x).to(x_dtype)
        w = torch.randn(N, K, generator=g) * 0.02
        b = torch.randn(N, generator=g) * 0.01 if bias else None
        w_kn, sw = cpu_route.weight_quant(w)
        data.append((x, w_kn, sw, b))

    def step():
        for x, w_kn, sw, b in data:
            cpu_route.linear(x, w_kn, sw, b)

    ops = sum(2 * M * N * K for M, N, K in shapes)
    return cpu_protocol(step, ops, f"{label}: the full step (torch CPU quantize + torch._int_mm + dequantize"
                        + (" + bias" if bias else "") + ")", budget_s)


def cpu_baseline_conv(n, c, h, w, layers, sample, relu=True, budget_s=20.0):
    """The reference's CPU conv route (quantize per image, exact float conv of the integers, shift /
    round / saturate, dequantize) over `layers` layers of c -> c channels on [n, c, h, w]; the shift
    of each layer is fixed on the first run (a warm-up run), as the reference fixes it on the first
    call."""
    from oracle import cpu_route

    g = gen(1)
    x = torch.randn(n, c, h, w, generator=g)
    convs = [cpu_route.ConvLayerCPU(torch.randn(c, c, 3, 3, generator=g) * 0.02, relu) for _ in range(layers)]

    def step():
        y = x
        for L in convs:
            xq, sx = cpu_route.conv_quant(y)
            if L.shift is None:
                L.calibrate(xq[0])
            y = cpu_route.conv_dequant(L(xq), L.scale, sx, None, torch.float32)

    ops = 2 * n * h * w * c * c * 9 * layers
    return cpu_protocol(step, ops, sample, budget_s)


# ------------------------------------------------------------------------------ main
def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {a.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    kernels.lib()   # fails loudly if the HIP library is not built
    kernels.use_tuned(True)     # the shipped tile table, as Config.tuned_tilings (default) applies it
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    res = {"metric": METRIC, "unit": "TOPS", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
           "data": "synthetic (seed 0, randn)" if a.operands == "randn" else
                   "synthetic, all-zero GEMM operands (power-limit diagnostic, not the benchmark)"}
    bench = {"headline": bench_headline, "c1": bench_c1, "c2": bench_c2, "c3": bench_c3, "c4": bench_c4,
             "c5": bench_c5, "decode": bench_decode, "quant": bench_quant, "bf16": bench_bf16, "vgg16": bench_vgg16,
             "stack": bench_stack, "copy": bench_copy, "libref": bench_libref}[a.workload]
    res.update(bench(a, dev))
    print(json.dumps(res), flush=True)


def timed_steps(a, step, timer):
    """W warm-up steps, an ungated wall-clock pass of the K steps (host launch cost included), then
    the gated timed region (gated_timed_steps). Returns (GPU seconds per step, host seconds per step)."""
    for i in range(a.warmup):
        step(i, None)
    host = eager_seconds(a, step)
    return gated_timed_steps(a, step, timer, host * 1e3), host


_SLEEP_CYCLES_PER_MS = None


def gate(ms):
    """Holds torch's current stream for about `ms` milliseconds with a GPU spin kernel, so that the
    host can enqueue a whole timed region before the GPU reaches it: the region's kernels then run
    back to back and HIP events between them bracket GPU work only."""
    global _SLEEP_CYCLES_PER_MS
    if _SLEEP_CYCLES_PER_MS is None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1000)
        e0.record()
        torch.cuda._sleep(2_000_000)
        e1.record()
        torch.cuda.synchronize()
        _SLEEP_CYCLES_PER_MS = 2_000_000 / max(e0.elapsed_time(e1), 1e-3)
    torch.cuda._sleep(int(ms * _SLEEP_CYCLES_PER_MS))


# GPU time of untimed work run behind the gate, right before a timed region. Under a sustained int8
# load the card sits at its 1400 W board limit, and after the idle gate its power controller takes about
# 15 ms to settle: the first few launches run fast, the next ones up to 25% slow, then the clock recovers
# (per-dispatch durations of the M=8192 GEMM: 442 -> 569 -> ~450 us). The pre-heat keeps that transient,
# which a continuously busy job does not see, out of the timed region.
PREHEAT_MS = 50.0


def preheat_count(ms_per_unit, cap=500):
    """Units of work (steps or launches) that fill about PREHEAT_MS of GPU time."""
    return int(min(cap, math.ceil(PREHEAT_MS / max(ms_per_unit, 1e-3))))


def gated_timed_steps(a, step, timer, host_ms_per_step):
    """The timed region: a gate covering the host's enqueue time (1.5 x the measured ungated time + 2
    ms), untimed pre-heat steps (about PREHEAT_MS of work), then K eager steps between two events;
    step(i, t) records per-launch events of the dominant kernel with t. Returns GPU seconds per step."""
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    heat = preheat_count(host_ms_per_step)
    gate(1.5 * host_ms_per_step * (a.steps + heat) + 2.0)
    for i in range(heat):
        step(i, None)
    e0.record()
    for i in range(a.steps):
        step(i, timer)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / a.steps


def back_to_back_us(calls, launches):
    """Microseconds per launch of `launches` calls (cycling through `calls`) queued behind a gate and
    untimed pre-heat launches (about PREHEAT_MS of work), run back to back between two events (no
    events between the launches)."""
    for fn in calls:
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for fn in calls:
        fn()
    torch.cuda.synchronize()
    heat = preheat_count((time.perf_counter() - t0) * 1e3 / len(calls))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    gate(2.0 + 0.05 * (launches + heat))
    for i in range(heat):
        calls[i % len(calls)]()
    e0.record()
    for i in range(launches):
        calls[i % len(calls)]()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / launches


def per_shape_us(sets, launches=10):
    """Microseconds per launch of each shape's fused GEMM (for a single row the one launch that also
    quantizes it): `launches` back-to-back launches of that
    shape behind a gate and a pre-heat, between two events. The launches cycle through enough copies of the weight
    (the sets' own, then clones) that they span more than the 256 MB Infinity Cache, so a weight is
    never read from the cache a previous launch filled."""
    out = []
    for j in range(len(sets[0])):
        ops = []
        wbytes = sets[0][j][1].numel()
        ncopies = max(len(sets), min(64, -(-(MALL_BYTES + (64 << 20)) // wbytes)))
        launches = max(launches, ncopies)
        weights = [sets[i][j][1] if i < len(sets) else sets[0][j][1].clone() for i in range(ncopies)]
        for i in range(launches):
            x, wq, sw, b, M, N, K = sets[i % len(sets)][j]
            ops.append((x if row_fused(x, wq) else kernels.quant_rows(x), weights[i % ncopies], sw, b, x.dtype))
        calls = [lambda o=o: kernels.linear_row(o[0], o[1], o[2], o[3], o[4]) if torch.is_tensor(o[0]) else
                 kernels.mm_i8_dequant(o[0][0], o[0][1], o[1], o[2], o[3], o[4]) for o in ops]
        out.append(back_to_back_us(calls, launches))
    return out


def eager_seconds(a, step):
    """Wall-clock seconds per step of K steps launched eagerly without a gate (host launch cost
    included)."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(a.steps):
        step(i, None)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / a.steps


def traffic(workload):
    """Measured HBM bytes per launch of the dominant kernel (FETCH_SIZE + WRITE_SIZE per dispatch,
    scaled by the same counters on a copy of known size), from profiles/hbm_traffic.json, which
    records the rocprofv3 commands that measured them; None when not measured."""
    try:
        with open(os.path.join(ROOT, "profiles", "hbm_traffic.json")) as f:
            t = json.load(f)[workload]
        return t["bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def shape_variant(dev, M, N, K, fused):
    """The kernel variant a shape launches: "rowq" for a single row quantized inside the launch, else the
    library's tile choice (tuned table applied)."""
    return "rowq" if fused else kernels.gemm_variant(dev, M, N, kernels.round_up(K, 16))


def gemm_kernels(dev, shapes, fused=None):
    """The GEMM kernels the shapes launch (per shape the variant of shape_variant)."""
    fused = fused or [False] * len(shapes)
    tiles = sorted({shape_variant(dev, M, N, K, f) for (M, N, K), f in zip(shapes, fused)})
    kernel_of = {"small": "mm_small_kernel", "gemv": "mm_gemv_kernel", "seg4": "mm_seg4_kernel",
                 "rowq": "mm_rowq_kernel"}
    names = sorted({kernel_of.get(t.split("_")[0], "mm_tile_kernel") for t in tiles})
    return f"{' + '.join(names)} (EPI_DQ): {', '.join(tiles)}"


def roofline_us(ops, nbytes):
    """Lower bound on a launch's duration from the two MI355X ceilings, in microseconds."""
    return max(ops / (PEAK_INT8_TOPS * 1e12), nbytes / (PEAK_HBM_GBS * 1e9)) * 1e6


def gemm_result(a, dev, shapes, x_dtype, bias, workload, label, bound="mfma"):
    if a.tile:
        for M, N, K in shapes:
            kernels.tile_set("i8", M, N, kernels.round_up(K, 16), a.tile)
        workload += f" (tile forced: {a.tile})"
    if a.operands == "zeros":
        workload += " (operands all zero: power-limit diagnostic)"
    # at least three distinct sets, together beyond the Infinity Cache (the measurement protocol)
    sets = gemm_sets(shapes, dev, 3, x_dtype=x_dtype, bias=bias, zeros=a.operands == "zeros")
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(a.steps)]
    step = lambda i, t: run_gemm_step_split(sets[i % len(sets)], ev[i] if t else None)   # noqa: E731
    for i in range(a.warmup):
        step(i, None)
    host = eager_seconds(a, step)
    sec = gated_timed_steps(a, step, True, host * 1e3)
    q_ms = [e[0].elapsed_time(e[1]) for e in ev]      # per step: the quantizes, back to back
    g_ms = [e[1].elapsed_time(e[2]) for e in ev]      # per step: the GEMMs, back to back
    reps = a.steps
    per_shape = per_shape_us(sets)
    ops_step = sum(2 * M * N * K for M, N, K in shapes)
    yb = 2 if x_dtype != torch.float32 else 4
    xb = x_dtype.itemsize
    nshape = len(shapes)
    g_sec = sum(g_ms) / 1e3                            # GEMM launches of the timed steps
    fused = [row_fused(x, wq) for x, wq, sw, b, M, N, K in sets[0]]
    launch_bytes = [gemm_bytes(M, N, K, xb, yb, bias, f) for (M, N, K), f in zip(shapes, fused)]
    g_bytes = sum(launch_bytes) * reps
    nq = nshape - sum(fused)
    q_bytes = sum(quant_bytes(M, K, xb) for (M, N, K), f in zip(shapes, fused) if not f) * reps
    q_sec = sum(q_ms) / 1e3
    achieved = ops_step * reps / g_sec / 1e12
    bound_us = sum(roofline_us(2 * M * N * K, nb) for (M, N, K), nb in zip(shapes, launch_bytes))
    out = {"value": round(ops_step / sec / 1e12, 2), "ms_per_step": round(sec * 1e3, 4),
           "host_ms_per_step": round(host * 1e3, 4),
           "timing": "GPU time of K eager steps enqueued behind a gate and about 50 ms of untimed pre-heat "
                     "steps (kernels back to back), each "
                     "step's quantizes then its GEMMs with events between; host_ms_per_step: the same "
                     "steps launched without a gate, wall clock",
           "config": {"workload": workload, "shapes_mnk": shapes, "x_dtype": str(x_dtype).replace("torch.", ""),
                      "bias": bias, "rotating_sets": len(sets),
                      "quantize": "a launch of its own" + ("" if not any(fused) else
                                                           "; single rows (M = 1): inside their GEMM launch "
                                                           "(xdna_linear_row)")},
           "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s",
                        "frac": round(achieved / PEAK_INT8_TOPS, 4),
                        "traffic": None if a.tile or a.operands != "randn" else traffic(label.lower()),
                        "kernel": gemm_kernels(dev, shapes, fused),
                        "launches": nshape * reps, "avg_launch_us": round(g_sec / (nshape * reps) * 1e6, 2),
                        "alg_bytes_per_launch": round(g_bytes / (nshape * reps)),
                        "hbm_GBs_equiv": round(g_bytes / g_sec / 1e9, 1),
                        "frac_of_attainable": round(bound_us * reps / (g_sec * 1e6), 4)},
           "quantize": None if nq == 0 else {"achieved_GBs": round(q_bytes / q_sec / 1e9, 1), "peak": PEAK_HBM_GBS,
                                             "avg_launch_us": round(q_sec / (nq * reps) * 1e6, 2),
                                             "launches": nq * reps},
           "per_shape": []}
    if bound == "hbm":
        gbs = g_bytes / g_sec / 1e9
        out["roofline"].update({"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                "frac": round(gbs / PEAK_HBM_GBS, 4), "TOPS": round(achieved, 2)})
    for j, (M, N, K) in enumerate(shapes):
        t = per_shape[j] / 1e6
        b = gemm_bytes(M, N, K, xb, yb, bias, fused[j])
        tile = shape_variant(dev, M, N, K, fused[j])
        out["per_shape"].append({"mnk": [M, N, K], "tile": tile,
                                 "us": round(t * 1e6, 2), "TOPS": round(2 * M * N * K / t / 1e12, 1),
                                 "GBs": round(b / t / 1e9, 1),
                                 "roofline_us": round(roofline_us(2 * M * N * K, b), 2)})
    if not a.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_gemm(shapes, x_dtype, bias, label)
    return out


def bench_c2(a, dev):
    shapes = []
    for M in (128, 512, 1024, 3000):
        shapes += [(M, 4096, 1024), (M, 6144, 1024), (M, 1024, 3072)]
    return gemm_result(a, dev, shapes, torch.bfloat16, False,
                       "C2 Qwen3-0.6B linear_cat qkv/gate-up/down, M in {128,512,1024,3000}, bf16", "C2")


def bench_c1(a, dev):
    return gemm_result(a, dev, [(128, 3072, 1024)], torch.float32, True, "C1 single W8A8 linear fp32 128x3072x1024",
                       "C1")


def bench_c5(a, dev):
    """The headline's main record: C5's M=8192 W8A8 linear (quantize + fused GEMM, bf16 + bias)."""
    return gemm_result(a, dev, [(8192, 14336, 4096)], torch.bfloat16, True,
                       "C5 W8A8 linear M=8192 N=14336 K=4096: bf16 x (0.1% outliers x20) -> per-row quantize -> "
                       "int8 MFMA GEMM + fused dequantize + bias -> bf16", "C5")


def bench_headline(a, dev):
    """C5 M=8192 (the largest single-GPU config) as the line; as sub-records, each with its own roofline
    and CPU baseline: C4's two 256-channel convs (as the op), C2, the decode GEMMs (M 1 and 16, HBM-bound),
    the activation quantize alone at 8192 x 14336 and 8192 x 4096 (HBM-bound), the C3 chain, and VGG-16's
    features at batch 8 through torch.compile(backend="xdna")."""
    out = bench_c5(a, dev)
    out["sub"] = (bench_c4(a, dev)["sub"] + [dict(bench_c2(a, dev), workload_key="C2"),
                                              dict(bench_decode(a, dev), workload_key="decode")]
                  + bench_quant(a, dev)["sub"] + [dict(bench_c3(a, dev), workload_key="C3"),
                                                  dict(bench_vgg16(a, dev), workload_key="VGG-16 b8")])
    return out


def bench_bf16(a, dev):
    """precision "bf16" on the C2 shapes: bf16 x and weights, the bf16 MFMA GEMM with float32
    accumulation, bf16 out (no quantize); one step = the 12 GEMMs between two events."""
    shapes = []
    for M in (128, 512, 1024, 3000):
        shapes += [(M, 4096, 1024), (M, 6144, 1024), (M, 1024, 3072)]
    g = gen(0)
    per_set = sum(2 * (M * K + N * K + M * N) for M, N, K in shapes)
    nsets = max(1, -(-(MALL_BYTES + (64 << 20)) // per_set))
    sets = [[(torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev),
              (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)) for M, N, K in shapes]
            for _ in range(nsets)]
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(a.steps)]

    def step(i, t):
        if t:
            ev[i][0].record()
        for x, w in sets[i % nsets]:
            kernels.mm_bf16(x, w, None, torch.bfloat16)
        if t:
            ev[i][1].record()

    for i in range(a.warmup):
        step(i, None)
    host = eager_seconds(a, step)
    sec = gated_timed_steps(a, step, True, host * 1e3)
    g_sec = sum(e[0].elapsed_time(e[1]) for e in ev) / 1e3
    flops = sum(2 * M * N * K for M, N, K in shapes)
    ach = flops * a.steps / g_sec / 1e12
    out = {"metric": "bf16 GEMM TFLOP/s (precision bf16) on 1 MI355X", "unit": "TFLOP/s", "dtype": "bf16",
           "value": round(flops / sec / 1e12, 2), "ms_per_step": round(sec * 1e3, 4),
           "host_ms_per_step": round(host * 1e3, 4),
           "config": {"workload": "precision bf16 on the C2 shapes: 12 bf16 GEMMs per step, bf16 out",
                      "shapes_mnk": shapes, "rotating_sets": nsets},
           "roofline": {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(ach / PEAK_BF16_TFLOPS, 4), "traffic": traffic("bf16"),
                        "kernel": "mm_tile_kernel (EPI_BF_BF16)",
                        "avg_launch_us": round(g_sec / (len(shapes) * a.steps) * 1e6, 2)}}
    if not a.no_cpu_baseline:
        xs = [(torch.randn(M, K, generator=g), torch.randn(N, K, generator=g) * 0.02) for M, N, K in shapes]

        def cpu_step():
            for x, w in xs:          # the reference's CPU route of precision bf16 (runtime.py:306-313)
                (x.float() @ w.float().t()).to(torch.bfloat16)
        out["cpu_baseline"] = dict(cpu_protocol(cpu_step, flops, "the full step: torch CPU float32 matmul, the "
                                                "reference's CPU route of precision bf16"), unit="TFLOP/s")
    return out


def bench_decode(a, dev):
    shapes = [(M, N, K) for M in (1, 16) for N, K in ((4096, 4096), (14336, 4096), (4096, 14336))]
    out = gemm_result(a, dev, shapes, torch.bfloat16, True,
                      "C5 decode W8A8 GEMMs M in {1,16}, (N,K) in {(4096,4096),(14336,4096),(4096,14336)}, "
                      "bf16 + bias", "decode", bound="hbm")
    out["unit"] = "TOPS"
    return out


def quant_kernel_name(K, dtype):
    """The activation-quantize kernel xdna_quant_rows launches for rows of K elements of `dtype` (16-byte
    aligned rows, K % 16 == 0): a wavefront per row up to 2048 elements, else a 256-thread block per row."""
    return "quant_rows_wave_kernel" if K <= 2048 else "quant_rows_block_kernel"


def quant_record(a, dev, M, K, x_dtype=torch.bfloat16):
    """The activation quantize alone (xdna_quant_rows: per-row amax, scale, int8 rows) on x [M, K]: K
    launches back to back behind the gate and a pre-heat, between two events, on rotating inputs that
    together exceed the Infinity Cache. value and roofline: algorithmic bytes (M K in + M K int8 out + 4 M
    scales) per second of launch time."""
    g = gen(0)
    xb = x_dtype.itemsize
    nsets = max(3, -(-(MALL_BYTES + (64 << 20)) // (M * K * (xb + 1))))
    xs = [torch.randn(M, K, generator=g).to(x_dtype).to(dev) for _ in range(nsets)]
    outs = [(torch.empty((M, K), dtype=torch.int8, device=dev), torch.empty((M,), dtype=torch.float32, device=dev))
            for _ in range(nsets)]
    us = back_to_back_us([lambda x=x, o=o: kernels.quant_rows(x, out=o) for x, o in zip(xs, outs)],
                         max(3 * nsets, a.steps))
    b = quant_bytes(M, K, xb)
    gbs = b / (us * 1e3)
    rec = {"workload_key": f"quantize {M}x{K}", "metric": "activation quantize GB/s on 1 MI355X", "unit": "GB/s",
           "value": round(gbs, 1), "ms_per_step": round(us / 1e3, 5), "dtype": f"{str(x_dtype)[6:]}->int8",
           "config": {"workload": f"per-row activation quantize of {str(x_dtype)[6:]} [{M}, {K}] -> int8 rows + "
                                  "float32 row scales (xdna_quant_rows)", "rotating_inputs": nsets},
           "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                        "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic(f"quant_{M}x{K}"),
                        "kernel": quant_kernel_name(K, x_dtype), "avg_launch_us": round(us, 2),
                        "alg_bytes_per_launch": b,
                        "timing": "launches back to back behind the gate and a pre-heat, events around them"}}
    if not a.no_cpu_baseline:
        rows = max(1, min(M, (64 << 20) // (K * 4)))       # a sample of about 64 MB of float32 work per run
        xc = torch.randn(rows, K, generator=gen(1)).to(x_dtype)
        from oracle import cpu_route

        rec["cpu_baseline"] = cpu_protocol(lambda: cpu_route.quant_rows(xc), quant_bytes(rows, K, xb),
                                           f"{rows} of the {M} rows (bytes scaled as the GPU's): torch CPU quantize "
                                           "(amax, divide, round, clamp, int8), the reference's expression",
                                           unit="GB/s")
    return rec


def bench_quant(a, dev):
    """The activation quantize alone on the bf16 shapes it serves: 8192 x 14336 (the down projection's input
    at C5's M) and 8192 x 4096 (the headline's own). The first is the line, both are sub-records."""
    recs = [quant_record(a, dev, 8192, 14336), quant_record(a, dev, 8192, 4096)]
    out = {k: v for k, v in recs[0].items() if k != "workload_key"}
    out["sub"] = recs
    return out


def bench_copy(a, dev):
    """Calibration for the HBM counters: an elementwise kernel that reads and writes 1 GiB each
    (bitwise_not of int32), whose FETCH_SIZE / WRITE_SIZE should read 1 GiB each."""
    n = 1 << 28
    src = torch.randint(-2 ** 31, 2 ** 31 - 1, (n,), dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    sec, host = timed_steps(a, lambda i, tm: torch.bitwise_not(src, out=dst), None)
    b = 2 * n * 4
    gbs = b / sec / 1e9
    return {"metric": "copy GB/s on 1 MI355X (counter calibration)", "unit": "GB/s",
            "value": round(b / sec / 1e9, 1), "ms_per_step": round(sec * 1e3, 4), "host_ms_per_step": round(host * 1e3, 4),
            "dtype": "int32",
            "config": {"workload": "bitwise_not int32 [2^28]: reads 1 GiB, writes 1 GiB"},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": b, "kernel": "torch elementwise"}}


def bench_libref(a, dev):
    """Reference point, not this library: the vendor library's GEMMs on C5's shape 8192x14336x4096 with the
    same gate and pre-heat. hipBLASLt's int8 GEMM (torch._int_mm: int8 operands, int32 out, no quantize,
    dequantize or bias) and its fp8 GEMM (torch._scaled_mm, e4m3 operands, unit scales, bf16 out), each on
    rotating weights that span more than the Infinity Cache."""
    M, N, K = 8192, 14336, 4096
    g = gen(0)
    a8 = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(dev)
    nw = max(2, -(-(MALL_BYTES + (64 << 20)) // (N * K)))
    ws = [torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev) for _ in range(nw)]
    ops = 2 * M * N * K
    i8_us = back_to_back_us([lambda w=w: torch._int_mm(a8, w.t()) for w in ws], max(20, a.steps))
    out = {"metric": "vendor GEMM TOPS on 1 MI355X (reference point)", "unit": "TOPS", "dtype": "int8",
           "value": round(ops / i8_us / 1e6, 1), "ms_per_step": round(i8_us / 1e3, 4),
           "config": {"workload": "hipBLASLt via torch._int_mm, 8192x14336x4096 int8 -> int32 (no dequant)",
                      "rotating_weights": nw},
           "roofline": {"bound": "mfma", "achieved": round(ops / i8_us / 1e6, 1), "peak": PEAK_INT8_TOPS,
                        "unit": "TFLOP/s", "frac": round(ops / i8_us / 1e6 / PEAK_INT8_TOPS, 4), "traffic": None,
                        "kernel": "hipBLASLt int8", "avg_launch_us": round(i8_us, 2)}}
    try:
        f8 = torch.float8_e4m3fn
        af = (torch.randn(M, K, generator=g) * 0.5).to(f8).to(dev)
        wf = [(torch.randn(N, K, generator=g) * 0.5).to(f8).to(dev) for _ in range(nw)]
        one = torch.ones((), device=dev)
        f8_us = back_to_back_us([lambda w=w: torch._scaled_mm(af, w.t(), scale_a=one, scale_b=one,
                                                              out_dtype=torch.bfloat16) for w in wf], max(20, a.steps))
        out["fp8"] = {"kernel": "hipBLASLt fp8 e4m3 via torch._scaled_mm, bf16 out", "avg_launch_us": round(f8_us, 2),
                      "TFLOPs": round(ops / f8_us / 1e6, 1)}
    except (RuntimeError, TypeError) as e:           # fp8 GEMM unavailable in this torch build
        out["fp8"] = {"error": f"{type(e).__name__}: {e}"[:200]}
    return out


def conv_layer_data(dev, n, c, h, w, seed=0):
    g = gen(seed)
    x = torch.randn(n, c, h, w, generator=g).to(dev)
    wt = (torch.randn(c, c, 3, 3, generator=g) * 0.02).to(dev)
    c_pad = -(-c // 16) * 16
    wq, sw = kernels.conv_weight_pack(wt, c_pad)
    return x, wq, sw, c_pad


def conv_op_record(a, dev, shape, sample_shape):
    """One 256-channel conv as the op runs it on a GPU graph (xdna::conv3x3_fused with ReLU fused):
    per-image quantize of the NCHW float32 input into NHWC int8, the implicit-GEMM conv with the
    calibrated shift and the requantize fused, dequantize back to NCHW float32. The layer's first call
    (weight quantize-once, shift calibration on image 0) runs in the warm-up. value: op-level TOPS
    (GPU time of K op calls behind the gate and a pre-heat); roofline: the conv kernel alone, its launches back to
    back on the same inputs (the op's own conv call, measured with events on its stream)."""
    from torch_xdna import Config, conv, ops

    n, c, h, w = shape
    cid = ops.config_id(Config(policy="gpu", verify="off"))
    xs = []
    nsets = max(3, -(-(MALL_BYTES + (64 << 20)) // (n * c * h * w * 9)))   # float in + int8 + float out
    g = gen(0)
    for _ in range(nsets):
        xs.append(torch.randn(n, c, h, w, generator=g).to(dev))
    wt = (torch.randn(c, c, 3, 3, generator=g) * 0.02).to(dev)
    op = torch.ops.xdna.conv3x3_fused
    sec, host = timed_steps(a, lambda i, tm: op(xs[i % nsets], wt, None, True, cid), None)
    layer = conv._layer(wt, h, w, True)
    if layer.device != "gpu" or layer.shift is None:
        raise SystemExit(f"conv {shape} did not run on the GPU: {layer.device}")
    # the op's conv launch alone (conv, requantize and dequantize to NCHW float32 in one kernel), back to
    # back on the op's own quantized inputs
    wq, _ = layer.gpu_weights(dev)
    qs = [kernels.conv_quant(x, layer.ci_pad) for x in xs[:3]]
    scale = layer.scale(dev)
    conv_us = back_to_back_us([lambda xq=xq, sx=sx: kernels.conv3x3_dequant(xq, wq, layer.shift, True, scale, sx, None,
                                                                            torch.float32) for xq, sx in qs],
                              max(3, a.steps))
    # and the conv with its requantize alone (NHWC int8 out), the engine's own figure
    only_us = back_to_back_us([lambda xq=xq: kernels.conv3x3(xq, wq, layer.shift, True) for xq, _ in qs],
                              max(3, a.steps))
    ops_ = 2 * n * h * w * c * c * 9
    ach = ops_ / (conv_us / 1e6) / 1e12
    conv_bytes = n * c * h * w * (1 + 4) + 9 * c * c + 4 * c + 4 * n   # int8 in, float32 out, scales
    label = f"C4 conv3x3 {c}->{c} on {n}x{c}x{h}x{w}"
    rec = {"workload_key": f"C4 {n}x{c}x{h}x{w}", "value": round(ops_ / sec / 1e12, 2), "unit": "TOPS",
           "ms_per_step": round(sec * 1e3, 4), "host_ms_per_step": round(host * 1e3, 4),
           "config": {"workload": f"{label} + ReLU as the op xdna::conv3x3_fused: float32 NCHW in -> per-image "
                                  "quantize -> int8 implicit-GEMM conv (calibrated shift, round half up, uint8 "
                                  "saturate) -> dequantize -> float32 NCHW out (the last three in one launch)",
                      "shift": layer.shift,
                      "plan": list(kernels.tile_plan(dev, "conv", n * h * w, c, 9 * layer.ci_pad)),
                      "rotating_inputs": nsets},
           "roofline": {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s",
                        "frac": round(ach / PEAK_INT8_TOPS, 4), "traffic": traffic(f"c4_{n}x{c}x{h}x{w}"),
                        "kernel": "mm_tile_kernel (conv, EPI_REQUANT with the dequantize fused, NCHW float32 out)",
                        "avg_launch_us": round(conv_us, 2),
                        "conv_only": {"kernel": "mm_tile_kernel (conv, EPI_REQUANT, NHWC uint8 out)",
                                      "avg_launch_us": round(only_us, 2),
                                      "frac": round(ops_ / (only_us / 1e6) / 1e12 / PEAK_INT8_TOPS, 4)},
                        "alg_bytes_per_launch": conv_bytes,
                        "timing": "conv kernel launches back to back behind the gate and a pre-heat, events around them"}}
    if not a.no_cpu_baseline:
        sn, sc, sh, sw_ = sample_shape
        rec["cpu_baseline"] = cpu_baseline_conv(
            sn, sc, sh, sw_, 1, f"one layer at {sn}x{sc}x{sh}x{sw_}"
            + (" (the full shape)" if sample_shape == shape else f" (a {sn * sh * sw_}/{n * h * w} pixel sample "
               f"of {n}x{c}x{h}x{w})") + ": torch CPU per-image quantize + exact float conv2d of the integers + "
            "shift + dequantize, shift fixed in the first warm-up run")
    return rec


def bench_c4(a, dev):
    """C4's two 256-channel convs as the op (sub-records of the headline line); the first is the line."""
    recs = [conv_op_record(a, dev, (1, 256, 1536, 64), (1, 256, 1536, 64)),
            conv_op_record(a, dev, (8, 256, 256, 256), (1, 256, 256, 256))]
    out = {k: v for k, v in recs[0].items() if k != "workload_key"}
    out["sub"] = recs
    return out


def bench_c3(a, dev):
    n, c, h, w, L = 1, 256, 64, 64, 4
    g = gen(0)
    x = torch.randn(n, c, h, w, generator=g).to(dev)
    c_pad = c
    layers = []
    for _ in range(L):
        wt = (torch.randn(c, c, 3, 3, generator=g) * 0.02).to(dev)
        layers.append(kernels.conv_weight_pack(wt, c_pad) + (None,))
    # calibrate the shifts on the first pass (first call of each layer)
    shifts = []
    y = x
    for wq, sw, _ in layers:
        xq, sx = kernels.conv_quant(y, c_pad)
        top = kernels.conv3x3_calibrate(xq[:1], wq, True)
        import math
        shift = min(31, max(1, math.ceil(math.log2(max(top * 1.25, 1.0) / 255))))
        shifts.append(shift)
        scale = sw * 2.0 ** shift
        y = kernels.conv_dequant(kernels.conv3x3(xq, wq, shift, True), True, scale, sx, None, torch.float32)
    scales = [sw * 2.0 ** s for (wq, sw, _), s in zip(layers, shifts)]

    def step_parts(i, ct=None):
        """Each layer as conv3x3_int8 alone, the launches of the GPU op xdna::conv3x3_fused: quantize, then
        the conv with its requantize and dequantize to float32 in one launch."""
        y = x
        for (wq, sw, _), s, sc in zip(layers, shifts, scales):
            xq, sx = kernels.conv_quant(y, c_pad)
            y = kernels.conv3x3_dequant(xq, wq, s, True, sc, sx, None, torch.float32)
        return y

    def step(i, ct=None):
        """The chained layers, the launches of xdna::conv3x3_chain on the GPU: the activation stays NHWC
        int8 between convs, and the last conv dequantizes in its own launch."""
        xq, sx = kernels.conv_quant(x, c_pad)
        for j, ((wq, sw, _), s, sc) in enumerate(zip(layers, shifts, scales)):
            if j == L - 1:
                return kernels.conv3x3_dequant(xq, wq, s, True, sc, sx, None, torch.float32)
            q = ct(kernels.conv3x3, xq, wq, s, True) if ct else kernels.conv3x3(xq, wq, s, True)
            xq, sx = kernels.conv_requant_next(q, True, False, sc, sx, None, torch.float32, c_pad)

    if not torch.equal(step(0), step_parts(0)):
        raise SystemExit("chained and per-layer C3 outputs differ")
    sec_parts, _ = timed_steps(a, step_parts, None)
    sec, host = timed_steps(a, step, None)
    # the dominant kernel alone: the step's four conv launches on their chained inputs, back to back, as the
    # step runs them (the last with its dequantize)
    convs, xq, sx = [], *kernels.conv_quant(x, c_pad)
    for j, ((wq, sw, _), s, sc) in enumerate(zip(layers, shifts, scales)):
        if j == L - 1:
            convs.append(lambda xq=xq, wq=wq, s=s, sc=sc, sx=sx: kernels.conv3x3_dequant(xq, wq, s, True, sc, sx,
                                                                                          None, torch.float32))
        else:
            convs.append(lambda xq=xq, wq=wq, s=s: kernels.conv3x3(xq, wq, s, True))
            xq, sx = kernels.conv_requant_next(kernels.conv3x3(xq, wq, s, True), True, False, sc, sx, None,
                                               torch.float32, c_pad)
    conv_us = back_to_back_us(convs, L * a.steps)
    ops = 2 * n * h * w * c * c * 9
    ach = ops / (conv_us / 1e6) / 1e12
    out = {"value": round(ops * L / sec / 1e12, 2), "ms_per_step": round(sec * 1e3, 4),
           "host_ms_per_step": round(host * 1e3, 4), "unchained_ms_per_step": round(sec_parts * 1e3, 4),
           "config": {"workload": "C3 4x (conv3x3 256->256 + ReLU) on 1x256x64x64, chained: quantize once, "
                                  "int8 NHWC requantize between convs, dequantize once"},
           "roofline": {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s",
                        "frac": round(ach / PEAK_INT8_TOPS, 4), "traffic": traffic("c3"), "kernel": "mm_tile_kernel (conv)",
                        "avg_launch_us": round(conv_us, 2)}}
    if not a.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_conv(n, c, h, w, L, "the full C3 step (4 layers, each quantized from and "
                                                "dequantized to float32 on the CPU)")
    return out


VGG16_CFG = [64, 64, "M", 128, 128, "M", 256, 256, 256, "M", 512, 512, 512, "M", 512, 512, 512, "M"]


def vgg16_features():
    """torchvision's VGG-16 `features` layout: biased 3x3 convs, in-place ReLUs, 2x2 max-pools."""
    layers, c = [], 3
    for v in VGG16_CFG:
        if v == "M":
            layers.append(torch.nn.MaxPool2d(2, 2))
        else:
            layers += [torch.nn.Conv2d(c, v, 3, padding=1), torch.nn.ReLU(inplace=True)]
            c = v
    return torch.nn.Sequential(*layers)


def bench_vgg16(a, dev):
    """VGG-16 features at batch 8 (C4's VGG shapes, torchvision's layout with bias, ReLU and pools)
    through torch.compile(backend="xdna"): the 13 convs become one xdna::conv3x3_chain. The same
    model with the chaining pass off (each conv quantized from and dequantized to float32) is timed
    beside it; both must give the same output."""
    import torch_xdna
    from torch_xdna import backend, runtime

    n, hw = 8, 224
    torch.manual_seed(0)
    net = vgg16_features().eval().to(dev)
    x = torch.randn(n, 3, hw, hw, generator=gen(0)).to(dev)
    ops, c, size = 0, 3, hw
    for v in VGG16_CFG:
        if v == "M":
            size //= 2
        else:
            ops += 2 * n * size * size * c * v * 9
            c = v

    def timed_model(chain):
        """Compile (from a fresh Dynamo cache, the chaining pass on or off), check that every conv ran on
        the GPU, then time it. Returns (output, GPU s / step, host s / step)."""
        torch._dynamo.reset()
        runtime.stats.reset()
        saved = backend._chain_convs
        if not chain:
            backend._chain_convs = lambda gm, cid: 0
        try:
            m = torch.compile(net, backend="xdna", options={"policy": "gpu", "fallback": "eager"})
            with torch.no_grad():
                y = m(x)
        finally:
            backend._chain_convs = saved
        st = runtime.stats.as_dict()
        if st["fallbacks"] or set(st["calls"]) != {"gpu"}:
            raise SystemExit(f"VGG-16 convs did not all run on the GPU: {st}")

        def step(i, ct=None):
            with torch.no_grad():
                return m(x)

        return (y,) + timed_steps(a, step, None)

    y_parts, sec_parts, host_parts = timed_model(False)
    y_chain, sec, host = timed_model(True)
    if not torch.equal(y_chain, y_parts):
        raise SystemExit("chained and per-layer VGG-16 outputs differ")
    ach = ops / sec / 1e12
    out = {"value": round(ach, 2), "ms_per_step": round(sec * 1e3, 4), "host_ms_per_step": round(host * 1e3, 4),
           "unchained_ms_per_step": round(sec_parts * 1e3, 4),
           "unchained_host_ms_per_step": round(host_parts * 1e3, 4),
           "config": {"workload": "VGG-16 features (13 conv3x3 + bias + ReLU, 5 max-pools) at 8x3x224x224 fp32, "
                                  "torch.compile(backend='xdna'), convs chained as int8 NHWC on the GPU"},
           "roofline": {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s",
                        "frac": round(ach / PEAK_INT8_TOPS, 4), "traffic": None,
                        "kernel": "whole step (13 convs, their quantize / requantize passes, the final pool)"}}
    if not a.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_vgg16(net, n, hw, ops)
    return out


def cpu_baseline_vgg16(net, n, hw, ops):
    """The reference's CPU route for the whole VGG-16 features at batch n (what its backend runs on the CPU,
    conv.py:43-51 per conv): per conv, per-image quantize, exact float conv of the integers, shift / round /
    saturate, dequantize + bias; the graph's ReLUs and 2x2 max-pools in float32 between. Each conv's shift is
    fixed on the first run (a warm-up run), as the reference fixes it on the first call."""
    from oracle import cpu_route

    x = torch.randn(n, 3, hw, hw, generator=gen(1))
    net = net.to("cpu")
    mods = list(net.features if hasattr(net, "features") else net)
    layers = []
    for m in mods:
        if isinstance(m, torch.nn.Conv2d):
            layers.append(("conv", cpu_route.ConvLayerCPU(m.weight.detach(), False), m.bias.detach()))
        elif isinstance(m, torch.nn.MaxPool2d):
            layers.append(("pool", None, None))
        else:
            layers.append(("relu", None, None))

    def step():
        y = x
        for kind, L, b in layers:
            if kind == "conv":
                xq, sx = cpu_route.conv_quant(y)
                if L.shift is None:
                    L.calibrate(xq[0])
                y = cpu_route.conv_dequant(L(xq), L.scale, sx, b, torch.float32)
            elif kind == "pool":
                y = torch.nn.functional.max_pool2d(y, 2, 2)
            else:
                y = torch.relu(y)
        return y

    return cpu_protocol(step, ops, f"the full step: VGG-16 features at {n}x3x{hw}x{hw} through the reference's CPU "
                        "route (per conv: torch CPU quantize + exact float conv2d of the integers + shift + dequantize "
                        "+ bias; ReLU and max-pool in float32)", budget_s=25.0, warmup=2)


# OmniVoice's backbone step (the reference's results/omnivoice_npu.md:3-12): 28 Qwen3-0.6B layers,
# the final norm and 8 x 1025 audio heads, cond + uncond sequences; the NPU step (the dispatch alone)
STACK_SHAPES = {"short": ((58, 43), 12.5), "mid": ((113, 92), 21.7), "long": ((264, 222), 55.3)}


def bench_stack(a, dev):
    """xdna::qwen3_stack on OmniVoice's step shapes: the op alone (GPU time of K steps behind a gate),
    each shape's output checked against the transformers model run eagerly in float32."""
    from transformers import Qwen3Config, Qwen3Model

    from torch_xdna import Config, stack

    torch.manual_seed(0)
    cfg = Qwen3Config(hidden_size=1024, intermediate_size=3072, num_hidden_layers=28, num_attention_heads=16,
                      num_key_value_heads=8, head_dim=128, vocab_size=16, rms_norm_eps=1e-6,
                      rope_parameters={"rope_type": "default", "rope_theta": 1e6}, attn_implementation="sdpa")
    llm = Qwen3Model(cfg).eval().to(dev)
    head = torch.nn.Linear(1024, 8 * 1025, bias=False).to(dev)
    weights = {}
    for i, Lr in enumerate(llm.layers):
        at, mlp = Lr.self_attn, Lr.mlp
        for key, t in dict(q=at.q_proj.weight, k=at.k_proj.weight, v=at.v_proj.weight, o=at.o_proj.weight,
                           gate=mlp.gate_proj.weight, up=mlp.up_proj.weight, down=mlp.down_proj.weight,
                           input_norm=Lr.input_layernorm.weight, post_norm=Lr.post_attention_layernorm.weight,
                           q_norm=at.q_norm.weight, k_norm=at.k_norm.weight).items():
            weights[(i, key)] = t
    weights.update(norm=llm.norm.weight, head=head.weight, inv_freq=llm.rotary_emb.inv_freq)
    plan = stack.Plan([], None, None, 1, None, weights, None, 28, 8 * 1025, stack.MAX_TOKENS)
    sid = stack.register(plan)
    conf = Config(policy="gpu")
    per_shape, steps = {}, {}
    for name, (lens, npu_ms) in STACK_SHAPES.items():
        L = max(lens)
        g = gen(1)
        x = torch.randn(len(lens), L, 1024, generator=g).to(dev)
        mask = torch.zeros(len(lens), 1, L, L, dtype=torch.bool)
        for b, n in enumerate(lens):
            mask[b, :, :n, :n] = True
            i = torch.arange(n, L)
            mask[b, :, i, i] = True
        mask = mask.to(dev)
        with torch.no_grad():
            y = stack.run(conf, sid, x, mask)
            ref = head(llm(inputs_embeds=x, attention_mask=mask)[0])
        err = max(float((y[b, :n] - ref[b, :n]).float().norm() / ref[b, :n].float().norm()) for b, n in enumerate(lens))
        if not err < 0.08:
            raise SystemExit(f"stack {name}: rel err {err:.3g} vs the float32 model")
        st = stack._stacks[sid]

        def op(i, t, st=st, x=x, mask=mask, lens=lens):
            st.lens_hint = (mask, list(lens))   # what the dispatcher hands over after parsing the mask
            return stack.run(conf, sid, x, mask)

        with torch.no_grad():
            sec, host = timed_steps(a, op, None)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(a.steps):
                st.lens_hint = None
                stack.run(conf, sid, x, mask)
            torch.cuda.synchronize()
            call = (time.perf_counter() - t0) / a.steps
        st.lens_hint = None
        macs = st.macs(list(lens))
        per_shape[name] = {"tokens": list(lens), "gpu_ms": round(sec * 1e3, 3), "host_ms": round(host * 1e3, 3),
                           "call_ms_with_mask_parse": round(call * 1e3, 3), "TOPS": round(2 * macs / sec / 1e12, 1),
                           "reference_npu_step_ms": npu_ms, "rel_err_vs_fp32": round(err, 4),
                           "hip_graph": stack.USE_GRAPHS}
        steps[name] = (sec, host, macs)
    sec, host, macs = steps["long"]
    ach = 2 * macs / sec / 1e12
    out = {"metric": "Qwen3 stack step (OmniVoice backbone) TOPS on 1 MI355X", "unit": "TOPS", "value": round(ach, 2),
           "ms_per_step": round(sec * 1e3, 4), "host_ms_per_step": round(host * 1e3, 4), "dtype": "bf16",
           "vs_baseline": round(STACK_SHAPES["long"][1] / (sec * 1e3), 2),
           "baseline": "the reference's NPU step for the long text, 55.3 ms (results/omnivoice_npu.md:12); "
                       "vs_baseline = that / ms_per_step",
           "config": {"workload": "xdna::qwen3_stack, 28 Qwen3-0.6B layers + norm + 8x1025 heads, 2 sequences of "
                                  "264 / 222 tokens (OmniVoice long text)"},
           "roofline": {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(ach / PEAK_BF16_TFLOPS, 4), "traffic": None,
                        "kernel": "whole op (bf16 GEMMs, attention, norms)"},
           "per_shape": per_shape}
    if not a.no_cpu_baseline:
        llm_c, head_c = llm.to("cpu"), head.to("cpu")
        lens = STACK_SHAPES["short"][0]
        L = max(lens)
        x = torch.randn(len(lens), L, 1024, generator=gen(2))
        mask = torch.zeros(len(lens), 1, L, L, dtype=torch.bool)
        for b, n in enumerate(lens):
            mask[b, :, :n, :n] = True
            i = torch.arange(n, L)
            mask[b, :, i, i] = True
        def cpu_step():
            with torch.no_grad():
                head_c(llm_c(inputs_embeds=x, attention_mask=mask)[0])
        out["cpu_baseline"] = cpu_protocol(cpu_step, 2 * stack._stacks[sid].macs(list(lens)),
                                           "the short-text step (58 / 43 tokens) of the same model eagerly in float32 "
                                           "on the CPU (transformers)", budget_s=20.0, warmup=1)
    return out


if __name__ == "__main__":
    main()
