"""The C-ABI library (CPU only): it loads, exports every entry point include/xdna_hip.h declares, and
rejects bad arguments with a status and a message before touching a device."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "xdna_hip.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(xdna_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    from torch_xdna import kernels

    if not os.path.exists(kernels.LIB_PATH):
        pytest.fail(f"{kernels.LIB_PATH} is not built (run __graft_entry__.build())")
    return kernels.lib()


def test_header_declares_entry_points():
    names = declared()
    assert "xdna_gemm_i8_i32" in names and "xdna_conv3x3_i8" in names and len(names) >= 12


def test_library_exports_every_declared_symbol(lib):
    from torch_xdna import kernels

    out = subprocess.run(["nm", "-D", "--defined-only", kernels.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (xdna_\w+)$", out, re.M))
    missing = [n for n in declared() if n not in exported]
    assert not missing, f"declared in xdna_hip.h but not exported: {missing}"
    for n in declared():
        getattr(lib, n)
    assert sorted(kernels.EXPORTS) == declared()


def test_tile_ids_match_header():
    """kernels.TILES lists the tile names by the header's XDNA_TILE_* ids."""
    from torch_xdna import kernels

    ids = {int(v): n for n, v in re.findall(r"^#define XDNA_TILE_(\w+) (\d+)", open(HEADER).read(), re.M)}
    assert sorted(ids) == list(range(len(kernels.TILES)))
    for i, name in ids.items():
        assert kernels.TILES[i].replace("_", "").lower().lstrip("t") == name.replace("_", "").lower().lstrip("t"), (i, name)


def test_abi_version(lib):
    from torch_xdna import kernels

    assert lib.xdna_abi_version() == kernels.ABI_VERSION == 1


def test_argument_validation(lib):
    """Bad arguments return XDNA_EINVAL (-1) and set a message; no device is needed for these."""
    p = ctypes.c_void_p(16)
    assert lib.xdna_gemm_i8_i32(p, 16, p, 16, p, 16, 4, 4, 15, None) == -1
    assert "multiple of 16" in lib.xdna_last_error().decode()
    assert lib.xdna_gemm_i8_dequant(p, 16, p, p, 16, p, None, p, 7, 16, 4, 4, 16, None) == -1
    assert "y_dtype" in lib.xdna_last_error().decode()
    # the workspace forms: the same checks, and a workspace that is not 256-byte aligned
    assert lib.xdna_gemm_i8_i32_ws(p, 16, p, 16, p, 16, 4, 4, 15, None, 0, None) == -1
    assert "multiple of 16" in lib.xdna_last_error().decode()
    assert lib.xdna_gemm_i8_i32_ws(p, 16, p, 16, p, 16, 4, 4, 16, ctypes.c_void_p(272), 4096, None) == -1
    assert "256-byte" in lib.xdna_last_error().decode()
    assert lib.xdna_gemm_i8_dequant_ws(p, 16, p, p, 16, p, None, p, 7, 16, 4, 4, 16, None, 0, None) == -1
    assert lib.xdna_gemm_i8_dequant_ws(p, 16, p, p, 16, p, None, p, 0, 16, 4, 4, 16, p, -1, None) == -1
    assert lib.xdna_gemm_ws_bytes(4, 4, 15) == -1
    assert "bad sizes" in lib.xdna_last_error().decode()
    # the one-row linear: dtypes, k's range and multiple, kx's bytes, leading dimension, pointers
    f = lib.xdna_linear_row
    assert f(p, 9, 16, p, 16, p, None, p, 1, 4, 16, None, None) == -1
    assert "x_dtype" in lib.xdna_last_error().decode()
    assert f(p, 1, 16, p, 16, p, None, p, 7, 4, 16, None, None) == -1
    assert f(p, 1, 16, p, 24, p, None, p, 1, 4, 24, None, None) == -1            # k % 16
    assert f(p, 1, 16, p, 32784, p, None, p, 1, 4, 32784, None, None) == -1      # k > XDNA_LINEAR_ROW_KMAX
    assert "XDNA_LINEAR_ROW_KMAX" in lib.xdna_last_error().decode()
    assert f(p, 1, 12, p, 16, p, None, p, 1, 4, 16, None, None) == -1            # 12 bf16: 24 bytes
    assert "kx" in lib.xdna_last_error().decode()
    assert f(p, 0, 20, p, 16, p, None, p, 1, 4, 16, None, None) == -1            # kx > k
    assert f(p, 1, 16, p, 8, p, None, p, 1, 4, 16, None, None) == -1             # ldw < k
    assert f(ctypes.c_void_p(24), 1, 16, p, 16, p, None, p, 1, 4, 16, None, None) == -1   # x unaligned
    assert f(p, 1, 16, p, 16, None, None, p, 1, 4, 16, None, None) == -1         # no weight scales
    assert f(None, 1, 16, None, 16, None, None, None, 1, 0, 16, None, None) == 0   # n = 0: nothing to do
    assert lib.xdna_quant_rows(p, 9, 4, 16, 16, p, 16, 16, p, None) == -1
    assert lib.xdna_quant_rows(p, 0, 4, 16, 8, p, 16, 16, p, None) == -1          # ld_x < k
    assert lib.xdna_conv3x3_i8(p, 1, 4, 4, 15, p, 8, 3, 0, p, None, None) == -1    # c_pad % 16
    assert lib.xdna_conv3x3_i8(p, 1, 4, 4, 16, p, 8, 0, 0, p, None, None) == -1    # shift 0
    assert "shift" in lib.xdna_last_error().decode()
    assert lib.xdna_conv_quant_nhwc(p, 0, 1, 3, 4, 4, p, 8, p, p, None) == -1     # c_pad % 16
    # empty work is a no-op success
    assert lib.xdna_gemm_i8_i32(None, 16, None, 16, None, 16, 0, 4, 16, None) == 0
    assert lib.xdna_quant_rows(None, 0, 0, 16, 16, None, 16, 16, None, None) == 0
    # the launch-plan query validates its arguments before it needs a device
    out_i, out_l = ctypes.c_int(), ctypes.c_int64()
    assert lib.xdna_tile_plan(7, 4, 4, 16, ctypes.byref(out_i), ctypes.byref(out_l), ctypes.byref(out_i)) == -1
    assert lib.xdna_tile_plan(0, 4, 4, 16, None, ctypes.byref(out_l), ctypes.byref(out_i)) == -1
