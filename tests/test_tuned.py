"""The tuned tile table (Config.tuned_tilings) and the sweep's summary, on the CPU.

The reference's counterparts are kernels.tuned_table / tiling_for (torch_xdna/kernels.py:123-149),
read from a table written by tools/sweep.py. The GPU side (forcing tiles, the sweep on the device)
is in test_gpu_kernels.py.
"""
import json

import pytest

from torch_xdna import kernels, sweep


@pytest.fixture
def fresh_table(monkeypatch):
    monkeypatch.setattr(kernels, "_tuned", None)
    monkeypatch.setattr(kernels, "_tuned_applied", None)
    yield
    kernels._tuned = None
    kernels._tuned_applied = None


def test_shipped_table_is_valid(fresh_table, monkeypatch):
    """The shipped MI355X table loads, and every entry names a built tile that beat the rule."""
    monkeypatch.delenv("TORCH_XDNA_TUNED", raising=False)
    with open(kernels.TUNED_PATH) as f:
        doc = json.load(f)
    n = 0
    for kind in kernels.KINDS:
        for key, v in doc.get(kind, {}).items():
            assert v["tiling"] in kernels.TILES and v["tiling"] != v["rule"] and v["gpu_us"] < v["rule_us"], (key, v)
            if kind == "conv":
                assert not v["tiling"].startswith(("small", "gemv")), key
            n += 1
    table = kernels.tuned_table()
    assert len(table) == n and n > 0
    (kind, M, N, K), tile = next(iter(table.items()))
    assert kernels.tiling_for(kind, M, N, K) == tile
    assert kernels.tiling_for(kind, M + 1, N, K) is None


def test_env_table_and_use_tuned(fresh_table, monkeypatch, tmp_path):
    """TORCH_XDNA_TUNED overrides the shipped table; use_tuned registers its entries in the library
    once and takes them out again (malformed entries are skipped)."""
    path = tmp_path / "t.json"
    path.write_text(json.dumps({"i8": {"128x4096x1024": {"tiling": "t128x128"}, "bad": {"tiling": "t64x64"},
                                       "16x1024x1024": {"tiling": "no_such_tile"}},
                                "conv": {"4096x256x2304": {"tiling": "t256x128"}}}))
    monkeypatch.setenv("TORCH_XDNA_TUNED", str(path))
    calls = []
    monkeypatch.setattr(kernels, "tile_set", lambda *a: calls.append(a))
    assert kernels.tuned_table() == {("i8", 128, 4096, 1024): "t128x128", ("conv", 4096, 256, 2304): "t256x128"}
    kernels.use_tuned(True)
    kernels.use_tuned(True)
    assert sorted(calls) == [("conv", 4096, 256, 2304, "t256x128"), ("i8", 128, 4096, 1024, "t128x128")]
    calls.clear()
    kernels.use_tuned(False)
    assert sorted(calls) == [("conv", 4096, 256, 2304, "auto"), ("i8", 128, 4096, 1024, "auto")]


def test_summary_keeps_clear_wins(tmp_path):
    """--summary: per shape the fastest exact tile, kept only when it beats the rule's tile by > 2%;
    inexact or failed lines never win."""
    recs = [
        # shape A: t128x128 beats the rule t64x64 by 20%; a faster but inexact tile is ignored
        dict(kind="i8", M=128, N=4096, K=1024, tiling="t64x64", rule="t64x64", exact=True, gpu_us=10.0, status="ok"),
        dict(kind="i8", M=128, N=4096, K=1024, tiling="t128x128", rule="t64x64", exact=True, gpu_us=8.0, status="ok"),
        dict(kind="i8", M=128, N=4096, K=1024, tiling="t256x128", rule="t64x64", exact=False, gpu_us=1.0, status="ok"),
        # shape B: the best is within 2% of the rule: no entry
        dict(kind="i8", M=512, N=4096, K=1024, tiling="t128x128", rule="t128x128", exact=True, gpu_us=10.0,
             status="ok"),
        dict(kind="i8", M=512, N=4096, K=1024, tiling="t128x256", rule="t128x128", exact=True, gpu_us=9.9,
             status="ok"),
        # shape C (conv): a failed launch never wins
        dict(kind="conv", M=4096, N=256, K=2304, tiling="t256x256w8", rule="t256x256w8", exact=True, gpu_us=20.0,
             status="ok"),
        dict(kind="conv", M=4096, N=256, K=2304, tiling="t64x64", rule="t256x256w8", exact=False, gpu_us=0.5,
             status="RuntimeError: x"),
        dict(kind="conv", M=4096, N=256, K=2304, tiling="t128x128", rule="t256x256w8", exact=True, gpu_us=15.0,
             status="ok"),
    ]
    path = tmp_path / "s.jsonl"
    path.write_text("".join(json.dumps(r) + "\n" for r in recs))
    assert sweep.summarize(str(path)) == {
        "i8": {"128x4096x1024": {"tiling": "t128x128", "gpu_us": 8.0, "rule": "t64x64", "rule_us": 10.0}},
        "conv": {"4096x256x2304": {"tiling": "t128x128", "gpu_us": 15.0, "rule": "t256x256w8", "rule_us": 20.0}}}


def test_sweep_candidates():
    assert sweep.candidates("i8", 16) == sweep.ENGINE_TILES + sweep.SMALL_TILES + sweep.SEG4_TILES
    assert sweep.candidates("i8", 17) == sweep.ENGINE_TILES + sweep.SMALL_TILES
    assert sweep.candidates("i8", 1) == sweep.ENGINE_TILES + sweep.SMALL_TILES + sweep.GEMV_TILES + sweep.SEG4_TILES
    assert sweep.candidates("bf16", 1) == sweep.candidates("i8", 1)
    assert sweep.candidates("i8", 3000) == sweep.ENGINE_TILES
    assert sweep.candidates("conv", 1) == sweep.ENGINE_TILES + ["direct"]
    assert sweep.candidates("conv", 1000, 64, 9 * 16) == sweep.ENGINE_TILES + ["direct"]
    assert sweep.candidates("conv", 1000, 40, 9 * 48) == sweep.ENGINE_TILES            # co not a multiple of 32
    assert sweep.candidates("conv", 1000, 64, 9 * 128) == sweep.ENGINE_TILES           # c_pad 128
    assert set(sweep.ENGINE_TILES + sweep.SMALL_TILES + sweep.GEMV_TILES + sweep.SEG4_TILES + sweep.DIRECT_TILES) == \
        set(kernels.TILES) - {"auto"}
