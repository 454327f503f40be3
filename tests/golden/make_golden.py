"""Writes tests/golden/golden.npz: small seeded fixtures of the int8 hot path.

The reference commits no golden vectors for this path, so these are produced by this repository's
oracle (oracle/xdna_oracle.py) after it has been pinned by tests/test_oracle.py, and serve as
regression fixtures for the oracle and as cross-language vectors for the GPU tests. The conv case
draws its integers the way the reference's research harnesses do (numpy default_rng(0),
activations in [-60, 60), weights in [-40, 40): npu_kernels/conv3x3_array.py:206-208).

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import xdna_oracle as O  # noqa: E402


def bf16(a):
    return O.to_bf16(np.asarray(a, np.float32))


def main():
    rng = np.random.default_rng(0)
    out = {}
    # quantize: bf16-valued rows with ties (s == 1 and s == 2 rows), a zero row, outliers x20
    x = bf16(rng.standard_normal((8, 64)).astype(np.float32))
    x[0, :8] = [127.0, 2.5, -3.5, 0.5, -0.5, 1.5, 126.5, -126.5]
    x[0, 8:] = np.clip(x[0, 8:], -1, 1)
    x[1, :8] = [254.0, 5.0, -5.0, 7.0, -7.0, 1.0, 3.0, -1.0]
    x[1, 8:] = np.clip(x[1, 8:], -1, 1)
    x[2] = 0.0
    x[5, ::13] *= 20
    out["q_x"] = x
    out["q_xq"], out["q_sx"] = O.quant_rows(x)
    # int32 GEMM and dequant (bf16 output, with bias)
    a = rng.integers(-127, 128, (24, 80), dtype=np.int8)
    w = rng.integers(-127, 128, (40, 80), dtype=np.int8)
    out["g_a"], out["g_w"] = a, w
    out["g_acc"] = O.gemm_i32(a, w)
    out["d_sx"] = (rng.random(24) * 0.05 + 1e-3).astype(np.float32)
    out["d_sw"] = (rng.random(40) * 0.01 + 1e-4).astype(np.float32)
    out["d_bias"] = (rng.standard_normal(40) * 0.01).astype(np.float32)
    out["d_y_bf16"] = O.to_bf16(O.dequant(out["g_acc"], out["d_sx"], out["d_sw"], out["d_bias"]))
    # conv integers, calibration and requant (both relu modes)
    crng = np.random.default_rng(0)
    cx = crng.integers(-60, 60, (2, 16, 6, 9), dtype=np.int8)
    cw = crng.integers(-40, 40, (8, 16, 3, 3), dtype=np.int8)
    acc = O.conv3x3_acc(cx, cw)
    out["c_x"], out["c_w"], out["c_acc"] = cx, cw, acc
    shifts = [O.calibrate_shift(acc[0], False), O.calibrate_shift(acc[0], True)]
    out["c_shift"] = np.array(shifts, np.int32)
    out["c_q0"] = O.requant(acc, shifts[0], False)
    out["c_q1"] = O.requant(acc, shifts[1], True)
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **out)
    print("wrote", os.path.join(HERE, "golden.npz"), {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
