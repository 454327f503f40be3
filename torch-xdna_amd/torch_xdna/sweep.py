"""Sweep the GPU tiles of the W8A8 GEMM, the bf16 GEMM and the int8 conv per shape, and build the
tuned table the runtime applies (Config.tuned_tilings).

The MI355X counterpart of the reference's tools/sweep.py (same CLI shape, one JSONL line per shape x
tiling, resumable, `--summary`). For every shape, every tile the library builds is forced through
the library's tile table, checked for exact results (int8: int32 sums equal to the CPU's
torch._int_mm, or for shapes too large for the CPU in seconds, to the rule's tile on the GPU; conv:
requantized integers equal to the CPU's exact float conv of the integers, or the rule's tile; bf16:
the reference's 5e-2 relative-norm check against a float32 matmul of the bf16 operands) and timed
as back-to-back launches between two events behind a GPU spin gate (GPU time only); launches of
weight-streaming shapes (up to 256 rows) cycle through copies of the weight that span more than the
256 MB Infinity Cache, so every launch reads its weight from HBM.

usage: python -m torch_xdna.sweep [--kind i8|bf16|conv] [--rows 128 512 1024 3000]
                                  [--shapes 4096x1024 ...] [--convs 1x256x256x64x64 ...]
                                  [--tiles t256x256w8 ...] [--out sweep.jsonl]
       python -m torch_xdna.sweep --summary sweep.jsonl [--table torch_xdna/tuned/mi355x.json]

Shapes: GEMMs as NxK (with --rows M), convs as NxCixCoxHxW. The table keeps, per shape, the fastest
exact tile when it beats the library's rule by more than 2%.
"""

import argparse
import itertools
import json
import os
import sys
import time

import torch

from . import kernels

# BASELINE shapes: C1, C2 (Qwen3-0.6B linear_cat qkv / gate-up / down), C5 (K=4096 with N 4096 / 14336,
# K=14336 with N 4096)
GEMM_SHAPES = [(3072, 1024), (4096, 1024), (6144, 1024), (1024, 3072), (4096, 4096), (14336, 4096), (4096, 14336)]
GEMM_ROWS = [1, 16, 128, 256, 512, 1024, 2048, 3000, 8192]
# C3, C4 and the VGG-16 layers at batch 8
CONV_SHAPES = [(1, 256, 256, 64, 64), (1, 256, 256, 1536, 64), (8, 3, 64, 224, 224), (8, 64, 64, 224, 224),
               (8, 64, 128, 112, 112), (8, 128, 128, 112, 112), (8, 128, 256, 56, 56), (8, 256, 256, 56, 56),
               (8, 256, 512, 28, 28), (8, 512, 512, 28, 28), (8, 512, 512, 14, 14)]
CPU_CHECK_MACS = 1 << 31          # exactness against the CPU up to this many MACs, else against the rule
ENGINE_TILES = [t for t in kernels.TILES if t.startswith("t")]
SMALL_TILES = [t for t in kernels.TILES if t.startswith("small")]
GEMV_TILES = [t for t in kernels.TILES if t.startswith("gemv")]
SEG4_TILES = [t for t in kernels.TILES if t.startswith("seg4")]
DIRECT_TILES = ["direct"]


def candidates(kind, M, N=None, K=None):
    """Tiles to try: every tile-engine shape (and, for convs of N = co, K = 9 c_pad, the direct kernels
    where they take the shape: kernels.direct_ok); the small-M kernel's widths for up to 256 rows; the
    one-row kernel's widths for one row; the few-row kernel's widths for up to 16 rows."""
    if kind == "conv":
        return ENGINE_TILES + (DIRECT_TILES if N is None or kernels.direct_ok(N, K) else [])
    if M > 256:
        return list(ENGINE_TILES)
    return ENGINE_TILES + SMALL_TILES + (GEMV_TILES if M == 1 else []) + (SEG4_TILES if M <= 16 else [])


_cycles_per_ms = None


def _gate(ms):
    """Hold the stream ~ms with a spin kernel, so the launches queued behind it run back to back."""
    global _cycles_per_ms
    if _cycles_per_ms is None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1000)
        e0.record()
        torch.cuda._sleep(1_000_000)
        e1.record()
        torch.cuda.synchronize()
        _cycles_per_ms = 1_000_000 / max(e0.elapsed_time(e1), 1e-3)
    torch.cuda._sleep(int(ms * _cycles_per_ms))


def gpu_us(fn, reps=48):
    """Microseconds per launch of fn: reps launches behind a gate, between two events."""
    fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    fn()
    torch.cuda.synchronize()
    host_ms = (time.perf_counter() - t0) * 1e3
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _gate(min(200.0, 2.0 + 1.5 * host_ms * reps))
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def _gen(seed):
    return torch.Generator().manual_seed(seed)


MALL_BYTES = 256 << 20             # MI355X Infinity Cache


def _weight_copies(w, M):
    """Copies of the device weight w that the timed launches cycle through: for weight-streaming shapes
    (up to 256 rows) enough copies to span more than the Infinity Cache, so each launch reads its weight
    from HBM as a model's layers do, not from the cache the previous launch filled."""
    if M > 256:
        return [w]
    n = min(96, -(-(MALL_BYTES + (64 << 20)) // (w.numel() * w.element_size())))
    return [w] + [w.clone() for _ in range(n - 1)]


def _cycling(fn, items):
    it = itertools.cycle(items)
    return lambda: fn(next(it))


def _gemm_case(kind, M, N, K, dev):
    """(timed launch, launch whose result is checked, the CPU's result or None, how to compare, ops)
    for one GEMM shape."""
    g = _gen(M * 31 + N * 7 + K)
    if kind == "i8":
        a = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
        w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
        sx, sw = torch.rand(M, generator=g) + 0.01, torch.rand(N, generator=g) + 0.01
        ag, wg, sxg, swg = a.to(dev), w.to(dev), sx.to(dev), sw.to(dev)
        # what the product runs
        bench = _cycling(lambda wc: kernels.mm_i8_dequant(ag, sxg, wc, swg, None, torch.bfloat16),
                         _weight_copies(wg, M))
        exact = lambda: kernels.mm_i8(ag, wg)
        want = torch._int_mm(a, w.t().contiguous()) if M * N * K <= CPU_CHECK_MACS else None
        return bench, exact, want, "equal", 2 * M * N * K
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    xg, wg = x.to(dev), w.to(dev)
    run = lambda: kernels.mm_bf16(xg, wg, None, torch.float32)
    bench = _cycling(lambda wc: kernels.mm_bf16(xg, wc, None, torch.float32), _weight_copies(wg, M))
    want = x.float() @ w.float().t() if M * N * K <= CPU_CHECK_MACS else None
    return bench, run, want, "norm", 2 * M * N * K


def _conv_case(n, ci, co, h, w, dev):
    from .conv import ConvLayer

    g = _gen(n * 131 + ci * 17 + co + h)
    c_pad = kernels.round_up(ci, 16)
    xq = torch.randint(-127, 128, (n, ci, h, w), generator=g, dtype=torch.int8)
    weight = torch.randn(co, ci, 3, 3, generator=g) * 0.05
    layer = ConvLayer(weight, h, w, True)
    x_nhwc = kernels.nchw_to_nhwc(xq.to(dev), c_pad)
    wq, _ = layer.gpu_weights(dev)
    layer.shift = 8
    run = lambda: kernels.conv3x3(x_nhwc, wq, layer.shift, True)
    want = layer.cpu(xq).permute(0, 2, 3, 1).contiguous() if n * h * w * ci * co * 9 <= CPU_CHECK_MACS else None
    return run, run, want, "equal", 2 * n * h * w * ci * co * 9


def _agrees(got, want, how):
    if how == "equal":
        return torch.equal(got.cpu(), want.cpu())
    got, want = got.float().cpu(), want.float().cpu()
    return bool(torch.isfinite(got).all()) and float((got - want).norm() / want.norm().clamp(min=1e-30)) < 5e-2


def sweep_shape(kind, M, N, K, dev, case, done, out, tiles=None):
    """Every candidate tile of one shape (those in `tiles` if given): JSONL lines appended to `out`
    (skipping those in `done`)."""
    bench, exact, want, how, ops = case
    kernels.tile_set(kind, M, N, K, "auto")
    rule = kernels.tile_get(dev, kind, M, N, K)
    rule_plan = kernels.tile_plan(dev, kind, M, N, K)
    ref_kind = "cpu"
    if want is None:               # too large for the CPU: the rule's tile is the reference
        want, ref_kind = exact(), "rule"
    for tile in candidates(kind, M, N, K):
        if (kind, M, N, K, tile) in done or (tiles is not None and tile not in tiles):
            continue
        rec = {"kind": kind, "M": M, "N": N, "K": K, "tiling": tile, "rule": rule, "rule_plan": list(rule_plan),
               "checked_against": ref_kind}
        try:
            kernels.tile_set(kind, M, N, K, tile)
            # the launch plan the time belongs to: rows [0, m1) with the head tile, the rest with the tail
            rec["plan"] = list(kernels.tile_plan(dev, kind, M, N, K))
            got = exact()
            rec["exact"] = _agrees(got, want, how)
            us = gpu_us(bench)
            rec.update(gpu_us=round(us, 2), tops=round(ops / us / 1e6, 1), status="ok")
        except Exception as e:     # a launch error: recorded, the sweep goes on
            rec.update(exact=False, status=f"{type(e).__name__}: {e}"[:300])
        finally:
            kernels.tile_set(kind, M, N, K, "auto")
        out.write(json.dumps(rec) + "\n")
        out.flush()
        print(json.dumps(rec), flush=True)


def sweep(kind, rows, shapes, convs, out_path, tiles=None):
    assert kernels.available(), kernels.unavailable_reason()
    dev = torch.device("cuda", torch.cuda.current_device())
    done = set()
    if os.path.exists(out_path):
        with open(out_path) as f:
            for line in f:
                r = json.loads(line)
                done.add((r["kind"], r["M"], r["N"], r["K"], r["tiling"]))
    kernels.use_tuned(False)
    with open(out_path, "a") as out:
        if kind == "conv":
            for n, ci, co, h, w in convs:
                case = _conv_case(n, ci, co, h, w, dev)
                sweep_shape("conv", n * h * w, co, 9 * kernels.round_up(ci, 16), dev, case, done, out, tiles)
        else:
            for N, K in shapes:
                for M in rows:
                    Kp = kernels.round_up(K, 16)
                    sweep_shape(kind, M, N, Kp, dev, _gemm_case(kind, M, N, Kp, dev), done, out, tiles)


def summarize(path):
    """{kind: {"MxNxK": {"tiling", "gpu_us", "rule", "rule_us"}}} of the shapes whose fastest exact tile
    beats the rule's by more than 2%."""
    best, rule_us, rule_of = {}, {}, {}
    with open(path) as f:
        for line in f:
            r = json.loads(line)
            if r.get("status") != "ok" or not r.get("exact"):
                continue
            key = (r["kind"], r["M"], r["N"], r["K"])
            rule_of[key] = r["rule"]
            if r["tiling"] == r["rule"]:
                rule_us[key] = r["gpu_us"]
            if key not in best or r["gpu_us"] < best[key][1]:
                best[key] = (r["tiling"], r["gpu_us"])
    table = {}
    for key, (tile, us) in sorted(best.items()):
        ru = rule_us.get(key)
        if ru is None or tile == rule_of[key] or us > 0.98 * ru:
            continue
        kind, M, N, K = key
        table.setdefault(kind, {})[f"{M}x{N}x{K}"] = {"tiling": tile, "gpu_us": us, "rule": rule_of[key],
                                                      "rule_us": ru}
    return table


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--kind", default="i8", choices=["i8", "bf16", "conv"])
    ap.add_argument("--rows", type=int, nargs="*", default=GEMM_ROWS)
    ap.add_argument("--shapes", nargs="*", default=[f"{n}x{k}" for n, k in GEMM_SHAPES])
    ap.add_argument("--convs", nargs="*", default=["x".join(map(str, c)) for c in CONV_SHAPES])
    ap.add_argument("--tiles", nargs="*", choices=[t for t in kernels.TILES if t != "auto"],
                    help="sweep only these tiles (default: every candidate)")
    ap.add_argument("--out", default="sweep.jsonl")
    ap.add_argument("--summary", metavar="JSONL")
    ap.add_argument("--table", metavar="JSON", help="with --summary: merge the result into this tuned table")
    a = ap.parse_args(argv)
    if a.summary:
        table = summarize(a.summary)
        for kind, entries in table.items():
            for key, v in entries.items():
                print(f"{kind:5s} {key:22s} {v['tiling']:11s} {v['gpu_us']:9.2f} us   rule {v['rule']:11s} "
                      f"{v['rule_us']:9.2f} us")
        if a.table:
            doc = {}
            if os.path.exists(a.table):
                with open(a.table) as f:
                    doc = json.load(f)
            for kind, entries in table.items():
                doc.setdefault(kind, {}).update(entries)
            props = torch.cuda.get_device_properties(0) if torch.cuda.is_available() else None
            if props is not None:
                doc["device"] = f"{props.name} {props.gcnArchName} ({props.multi_processor_count} CUs)"
            with open(a.table, "w") as f:
                json.dump(doc, f, indent=1, sort_keys=True)
                f.write("\n")
        return 0
    shapes = [tuple(int(v) for v in s.split("x")) for s in a.shapes]
    convs = [tuple(int(v) for v in s.split("x")) for s in a.convs]
    sweep(a.kind, a.rows, shapes, convs, a.out, set(a.tiles) if a.tiles else None)
    return 0


if __name__ == "__main__":
    sys.exit(main())
