/* Plain-C restatement of the int8 hot path's integer arithmetic -- TEST INFRASTRUCTURE.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library, as the
 * checker. The product never links it. Built by oracle/Makefile into oracle/_build/liboracle.so.
 *
 * Each routine restates the reference's CPU route (paths relative to the reference root):
 *   oracle_quant_rows   torch_xdna/runtime.py:145-148 (and :64-65, :366-368, conv.py:45-46, :58-60)
 *   oracle_gemm_i32     torch_xdna/runtime.py:162-163 (torch._int_mm(xq, w_kn)), w given as [N, K]
 *   oracle_dequant      torch_xdna/runtime.py:350-353, :370-373
 *   oracle_conv3x3_acc  torch_xdna/conv.py:86-87; npu_kernels/conv3x3_array.py:176-182
 *   oracle_requant      torch_xdna/conv.py:89-92
 * It is compiled without fast-math and without FP contraction, so float32 operations round once
 * each, as torch's CPU kernels do.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#define ORACLE_ABI 1

int oracle_abi_version(void) { return ORACLE_ABI; }

/* s[r] = max(amax|x[r,:]|, 1e-8f) / 127; q = rint(x / s) clamped to +-127 (rint: ties to even in
 * the default rounding mode). */
void oracle_quant_rows(const float* x, int64_t rows, int64_t k, int8_t* q, float* s) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * k;
    float amax = 0.0f;
    int nan = 0;
    for (int64_t i = 0; i < k; ++i) {
      float a = fabsf(xr[i]);
      if (a != a) nan = 1;
      if (a > amax) amax = a;
    }
    float sc = (nan ? NAN : (amax > 1e-8f ? amax : 1e-8f)) / 127.0f;
    s[r] = sc;
    for (int64_t i = 0; i < k; ++i) {
      float v = rintf(xr[i] / sc);
      if (v > 127.0f) v = 127.0f;
      if (v < -127.0f) v = -127.0f;
      q[r * k + i] = (int8_t)v;
    }
  }
}

/* c[m, n] = sum_k a[m, k] * w[n, k], exact in int64, stored as int32. */
void oracle_gemm_i32(const int8_t* a, const int8_t* w, int32_t* c, int64_t m, int64_t n, int64_t k) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; ++i) {
    const int8_t* ar = a + i * k;
    for (int64_t j = 0; j < n; ++j) {
      const int8_t* wr = w + j * k;
      int64_t acc = 0;
      for (int64_t t = 0; t < k; ++t) acc += (int64_t)ar[t] * (int64_t)wr[t];
      c[i * n + j] = (int32_t)acc;
    }
  }
}

/* y[m, n] = ((float)acc * sx[m]) * sw[n] (+ bias[n]), each operation rounded to float32. */
void oracle_dequant(const int32_t* acc, const float* sx, const float* sw, const float* bias, float* y,
                    int64_t m, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; ++i) {
    for (int64_t j = 0; j < n; ++j) {
      volatile float t = (float)acc[i * n + j];
      t = t * sx[i];
      t = t * sw[j];
      if (bias) t = t + bias[j];
      y[i * n + j] = t;
    }
  }
}

/* acc[b, o, y, x] = sum_{c, ky, kx} w[o, c, ky, kx] * xin[b, c, y + ky - 1, x + kx - 1] (zero
 * outside the image), NCHW int8 in, int32 out (exact; |acc| <= 127 * 127 * 9 * Ci). */
void oracle_conv3x3_acc(const int8_t* xin, const int8_t* w, int32_t* acc, int64_t nb, int64_t ci,
                        int64_t h, int64_t wd, int64_t co) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < nb; ++b) {
    for (int64_t o = 0; o < co; ++o) {
      int32_t* out = acc + (b * co + o) * h * wd;
      for (int64_t p = 0; p < h * wd; ++p) out[p] = 0;
      for (int64_t c = 0; c < ci; ++c) {
        const int8_t* xc = xin + (b * ci + c) * h * wd;
        const int8_t* wc = w + (o * ci + c) * 9;
        for (int64_t ky = 0; ky < 3; ++ky) {
          for (int64_t kx = 0; kx < 3; ++kx) {
            int32_t wv = wc[ky * 3 + kx];
            if (!wv) continue;
            for (int64_t y = 0; y < h; ++y) {
              int64_t sy = y + ky - 1;
              if (sy < 0 || sy >= h) continue;
              for (int64_t x = 0; x < wd; ++x) {
                int64_t sx = x + kx - 1;
                if (sx < 0 || sx >= wd) continue;
                out[y * wd + x] += wv * (int32_t)xc[sy * wd + sx];
              }
            }
          }
        }
      }
    }
  }
}

/* q = floor((acc + 2^(shift-1)) / 2^shift), saturated to [0, 255] (relu, stored as uint8) or
 * [-128, 127] (int8). Floor division is written out so it does not depend on >> of negatives. */
void oracle_requant(const int32_t* acc, int64_t count, int shift, int relu, void* out) {
  const int64_t half = (int64_t)1 << (shift - 1);
  const int64_t div = (int64_t)1 << shift;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < count; ++i) {
    int64_t num = (int64_t)acc[i] + half;
    int64_t q = num / div;
    if ((num % div != 0) && (num < 0)) q -= 1;
    if (relu) {
      if (q < 0) q = 0;
      if (q > 255) q = 255;
      ((uint8_t*)out)[i] = (uint8_t)q;
    } else {
      if (q < -128) q = -128;
      if (q > 127) q = 127;
      ((int8_t*)out)[i] = (int8_t)q;
    }
  }
}
