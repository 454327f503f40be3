// The pieces of xdna::qwen3_stack that are not GEMMs (the GEMMs run on the tile engine's bf16 path),
// for gfx950 (MI355X). The stack runs on a packed activation: the valid tokens of every sequence one
// after another, T rows; the residual stream is float32, GEMM operands bf16 with float32 sums.
//
//   rmsnorm_bf16   y = bf16(w * (x * rsqrt(mean(x^2) + eps)))           Qwen3RMSNorm on float32 rows
//   qk_norm_rope   per token: q / k heads RMSNorm'd over head_dim with their weights, then rotated by
//                  RoPE at the token's position; V written transposed (dims x tokens) for attention
//   attention      softmax(q k^T * scale) v per sequence and head, bidirectional over the sequence's
//                  tokens, grouped-query (q head h reads kv head h / (nh / nkv)), bf16 MFMA with an
//                  online softmax in float32 (32 queries per wave, keys in blocks of 32)
//   silu_mul       bf16(silu(gate) * up)
//   add_f32        x += y (the residual adds)
#include <hip/hip_runtime.h>

#include <cmath>

#include "xdna_common.h"
#include "xdna_hip.h"

namespace xdna {

typedef float f32x16s __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8s __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x16s mfma_bf16(const i32x4& a, const i32x4& b, const f32x16s& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8s, a), __builtin_bit_cast(bf16x8s, b), c,
                                                 0, 0, 0);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int DT>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
  return load_as_f32<DT>(p, i);
}

// ------------------------------------------------------------------------------ RMSNorm -> bf16
// One 256-thread block per row; d % 256 == 0 and d <= 4096 (the host checks). ADD: the residual add
// that precedes the norm in the layer, x += a, in the same launch (the float32 sums are written back
// and normalized as the separate add and norm would: the same values, one launch fewer).
template <int WDT, bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_bf16_kernel(float* __restrict__ x, const float* __restrict__ a,
                                                           int64_t d, const void* __restrict__ w, float eps,
                                                           uint16_t* __restrict__ y) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  float* xr = x + row * d;
  float v[16];
  float ss = 0.0f;
  const int nper = (int)(d / 256);       // d is a multiple of 256 here, at most 16 per thread
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    v[j] = 0.0f;
    if (j < nper) {
      v[j] = xr[j * 256 + threadIdx.x];
      if constexpr (ADD) {
        v[j] = v[j] + a[row * d + j * 256 + threadIdx.x];
        xr[j * 256 + threadIdx.x] = v[j];
      }
      ss += v[j] * v[j];
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  const float r = 1.0f / sqrtf(tot / (float)d + eps);
#pragma unroll
  for (int j = 0; j < 16; ++j)
    if (j < nper) {
      const int64_t c = j * 256 + threadIdx.x;
      y[row * d + c] = f32_to_bf16_bits(ld<WDT>(w, c) * (v[j] * r));
    }
}

// ------------------------------------------------------------------------------ q / k norm + RoPE
// One wave per (token, slot): slots 0 .. nh-1 are q heads, nh .. nh+nkv-1 k heads, then nkv v heads.
// Lane j holds dims j and j + 64 of a 128-dim head, which RoPE rotates into each other
// (rotate_half), so no lane exchange is needed besides the norm's sum.
template <int WDT>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(const float* __restrict__ qkv, int64_t T, int nh, int nkv,
                                                           const void* __restrict__ qw, const void* __restrict__ kw,
                                                           const float* __restrict__ inv_freq,
                                                           const int32_t* __restrict__ pos,
                                                           const int32_t* __restrict__ vt_col, float eps,
                                                           uint16_t* __restrict__ q, uint16_t* __restrict__ k,
                                                           uint16_t* __restrict__ vt, int64_t ld_vt) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int slots = nh + 2 * nkv;
  if (item >= T * slots) return;
  const int64_t t = item / slots;
  const int slot = (int)(item - t * slots);
  const float* src = qkv + t * (int64_t)slots * 128 + (int64_t)slot * 128;
  float a = src[lane], b = src[lane + 64];
  if (slot >= nh + nkv) {                 // v: transposed copy, vt[kv head][dim][token column]
    const int kvh = slot - nh - nkv;
    const int64_t col = vt_col[t];
    vt[((int64_t)kvh * 128 + lane) * ld_vt + col] = f32_to_bf16_bits(a);
    vt[((int64_t)kvh * 128 + lane + 64) * ld_vt + col] = f32_to_bf16_bits(b);
    return;
  }
  const bool isq = slot < nh;
  const void* w = isq ? qw : kw;
  const float r = 1.0f / sqrtf(wave_sum(a * a + b * b) / 128.0f + eps);
  a = ld<WDT>(w, lane) * (a * r);
  b = ld<WDT>(w, lane + 64) * (b * r);
  const float f = (float)pos[t] * inv_freq[lane];
  const float c = cosf(f), s = sinf(f);
  const float ra = a * c - b * s;         // dim j:      x_j cos - x_{j+64} sin
  const float rb = b * c + a * s;         // dim j + 64: x_{j+64} cos + x_j sin
  uint16_t* dst = isq ? q + (t * nh + slot) * 128 : k + (t * nkv + (slot - nh)) * 128;
  dst[lane] = f32_to_bf16_bits(ra);
  dst[lane + 64] = f32_to_bf16_bits(rb);
}

// ------------------------------------------------------------------------------ attention
// Grid (nseq * qblocks_max, nh); one wave per block: 32 queries of one head of one sequence.
// MFMA (srcA = X, srcB = Y) gives, in lane l, row l % 32 of Y and, in element 4 g + r, row
// 8 g + 4 (l / 32) + r of X. S = K Q^T: lane l <-> query l % 32, elements <-> 16 of 32 keys. The
// softmax statistics of a query are kept identical in lanes l and l ^ 32. O^T = V^T P^T accumulates
// with lane l <-> query l % 32 and elements <-> dims. P's operand needs keys 8 (l / 32) .. +7 of each
// 16-key step in lane l: lanes l and l ^ 32 swap one group of 4 keys per step.
__global__ __launch_bounds__(64) void attention_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                       const uint16_t* __restrict__ vt, int64_t ld_vt,
                                                       const int32_t* __restrict__ seq_start,
                                                       const int32_t* __restrict__ seq_len,
                                                       const int32_t* __restrict__ seq_vt, int qblocks, int nh,
                                                       int nkv, float scale, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x;
  const int seq = blockIdx.x / qblocks;
  const int qb = blockIdx.x - seq * qblocks;
  const int h = blockIdx.y;
  const int n = seq_len[seq];
  if (qb * 32 >= n) return;
  const int64_t start = seq_start[seq];
  const int64_t vt0 = seq_vt[seq];
  const int kvh = h / (nh / nkv);
  const int half = lane >> 5, row = lane & 31;
  // this lane's query and its 8 fragments (16 bytes of dims 16 s + 8 half .. +7)
  const int qi = min(qb * 32 + row, n - 1);
  i32x4 qf[8];
  const uint16_t* qrow = q + ((start + qi) * nh + h) * 128 + 8 * half;
#pragma unroll
  for (int s = 0; s < 8; ++s) qf[s] = *reinterpret_cast<const i32x4*>(qrow + 16 * s);
  f32x16s o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f32x16s{};
  float m = -INFINITY, l = 0.0f;
  for (int kb = 0; kb < n; kb += 32) {
    // S block: keys kb .. kb + 31
    const int ki = min(kb + row, n - 1);
    const uint16_t* krow = k + ((start + ki) * nkv + kvh) * 128 + 8 * half;
    f32x16s sc = f32x16s{};
#pragma unroll
    for (int s = 0; s < 8; ++s) sc = mfma_bf16(*reinterpret_cast<const i32x4*>(krow + 16 * s), qf[s], sc);
    float p[16];
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int key = kb + 8 * (e >> 2) + 4 * half + (e & 3);
      p[e] = key < n ? sc[e] * scale : -INFINITY;
      mx = fmaxf(mx, p[e]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m, mx);        // finite: every block has at least one key < n
    const float alpha = m == -INFINITY ? 0.0f : __expf(m - mn);
    float ps = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      p[e] = __expf(p[e] - mn);           // exp(-inf) = 0 for keys past n
      ps += p[e];
    }
    ps += __shfl_xor(ps, 32, 64);
    l = l * alpha + ps;
    m = mn;
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] *= alpha;
    // P V for the two 16-key steps of this block
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      // own keys 16 st + 4 half + (0..3) (group g = 2 st) and 16 st + 8 + 4 half + (0..3) (g = 2 st + 1);
      // half 0 needs 16 st + 0..7, half 1 needs 16 st + 8..15
      float send[4], recv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) send[r] = half == 0 ? p[4 * (2 * st + 1) + r] : p[4 * (2 * st) + r];
#pragma unroll
      for (int r = 0; r < 4; ++r) recv[r] = __shfl_xor(send[r], 32, 64);
      float lo[4], hi[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        lo[r] = half == 0 ? p[4 * (2 * st) + r] : recv[r];
        hi[r] = half == 0 ? recv[r] : p[4 * (2 * st + 1) + r];
      }
      const i32x4 pf = {(int)f32x2_to_bf16x2_bits(lo[0], lo[1]), (int)f32x2_to_bf16x2_bits(lo[2], lo[3]),
                        (int)f32x2_to_bf16x2_bits(hi[0], hi[1]), (int)f32x2_to_bf16x2_bits(hi[2], hi[3])};
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const uint16_t* vrow = vt + ((int64_t)kvh * 128 + db * 32 + row) * ld_vt + vt0 + kb + 16 * st + 8 * half;
        o[db] = mfma_bf16(*reinterpret_cast<const i32x4*>(vrow), pf, o[db]);
      }
    }
  }
  const int qo = qb * 32 + row;
  if (qo >= n) return;
  const float inv = 1.0f / l;
  uint16_t* orow = out + ((start + qo) * nh + h) * 128;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = db * 32 + 8 * g + 4 * half;
      const uint32_t w0 = f32x2_to_bf16x2_bits(o[db][4 * g] * inv, o[db][4 * g + 1] * inv);
      const uint32_t w1 = f32x2_to_bf16x2_bits(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv);
      *reinterpret_cast<uint2*>(orow + d) = make_uint2(w0, w1);
    }
}

// ------------------------------------------------------------------------------ SiLU * up, residual add
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ gu, int64_t T, int64_t inter,
                                                       uint16_t* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= T * inter) return;
  const int64_t t = i / inter, c = i - t * inter;
  const float g = gu[t * 2 * inter + c], u = gu[t * 2 * inter + inter + c];
  y[i] = f32_to_bf16_bits(g / (1.0f + __expf(-g)) * u);
}

__global__ __launch_bounds__(256) void add_f32_kernel(float* __restrict__ x, const float* __restrict__ y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) x[i] += y[i];
}

}  // namespace xdna

using namespace xdna;

extern "C" {

int xdna_rmsnorm_bf16(const float* x, int64_t rows, int64_t d, const void* w, int w_dtype, float eps, void* y,
                      void* stream) {
  XDNA_REQUIRE(w_dtype == XDNA_F32 || w_dtype == XDNA_BF16 || w_dtype == XDNA_F16, "w_dtype must be F32/BF16/F16");
  XDNA_REQUIRE(rows >= 0 && d >= 256 && d % 256 == 0 && d <= 4096, "d must be a multiple of 256, at most 4096");
  if (rows == 0) return XDNA_OK;
  XDNA_REQUIRE(x && w && y && rows < (1ll << 31), "bad arguments");
  hipStream_t st = as_stream(stream);
  uint16_t* yb = static_cast<uint16_t*>(y);
  float* xm = const_cast<float*>(x);     // read only without ADD
  if (w_dtype == XDNA_F32) rmsnorm_bf16_kernel<XDNA_F32, false><<<(unsigned)rows, 256, 0, st>>>(xm, nullptr, d, w, eps, yb);
  else if (w_dtype == XDNA_BF16) rmsnorm_bf16_kernel<XDNA_BF16, false><<<(unsigned)rows, 256, 0, st>>>(xm, nullptr, d, w, eps, yb);
  else rmsnorm_bf16_kernel<XDNA_F16, false><<<(unsigned)rows, 256, 0, st>>>(xm, nullptr, d, w, eps, yb);
  return launch_status("rmsnorm_bf16");
}

int xdna_add_rmsnorm_bf16(float* x, const float* a, int64_t rows, int64_t d, const void* w, int w_dtype, float eps,
                          void* y, void* stream) {
  XDNA_REQUIRE(w_dtype == XDNA_F32 || w_dtype == XDNA_BF16 || w_dtype == XDNA_F16, "w_dtype must be F32/BF16/F16");
  XDNA_REQUIRE(rows >= 0 && d >= 256 && d % 256 == 0 && d <= 4096, "d must be a multiple of 256, at most 4096");
  if (rows == 0) return XDNA_OK;
  XDNA_REQUIRE(x && a && w && y && rows < (1ll << 31), "bad arguments");
  hipStream_t st = as_stream(stream);
  uint16_t* yb = static_cast<uint16_t*>(y);
  if (w_dtype == XDNA_F32) rmsnorm_bf16_kernel<XDNA_F32, true><<<(unsigned)rows, 256, 0, st>>>(x, a, d, w, eps, yb);
  else if (w_dtype == XDNA_BF16) rmsnorm_bf16_kernel<XDNA_BF16, true><<<(unsigned)rows, 256, 0, st>>>(x, a, d, w, eps, yb);
  else rmsnorm_bf16_kernel<XDNA_F16, true><<<(unsigned)rows, 256, 0, st>>>(x, a, d, w, eps, yb);
  return launch_status("add_rmsnorm_bf16");
}

int xdna_qk_norm_rope(const float* qkv, int64_t T, int nh, int nkv, const void* q_w, const void* k_w, int w_dtype,
                      const float* inv_freq, const int32_t* pos, const int32_t* vt_col, float eps, void* q, void* k,
                      void* vt, int64_t ld_vt, void* stream) {
  XDNA_REQUIRE(w_dtype == XDNA_F32 || w_dtype == XDNA_BF16 || w_dtype == XDNA_F16, "w_dtype must be F32/BF16/F16");
  XDNA_REQUIRE(T >= 0 && nh >= 1 && nkv >= 1 && nh % nkv == 0, "bad head counts");
  if (T == 0) return XDNA_OK;
  XDNA_REQUIRE(qkv && q_w && k_w && inv_freq && pos && vt_col && q && k && vt && ld_vt >= 1, "bad arguments");
  const int64_t items = T * (nh + 2 * nkv);
  XDNA_REQUIRE(cdiv(items, 4) < (1ll << 31), "too many tokens");
  hipStream_t st = as_stream(stream);
  dim3 g((unsigned)cdiv(items, 4));
  uint16_t *qb = static_cast<uint16_t*>(q), *kb = static_cast<uint16_t*>(k), *vb = static_cast<uint16_t*>(vt);
  if (w_dtype == XDNA_F32)
    qk_norm_rope_kernel<XDNA_F32><<<g, 256, 0, st>>>(qkv, T, nh, nkv, q_w, k_w, inv_freq, pos, vt_col, eps, qb, kb, vb, ld_vt);
  else if (w_dtype == XDNA_BF16)
    qk_norm_rope_kernel<XDNA_BF16><<<g, 256, 0, st>>>(qkv, T, nh, nkv, q_w, k_w, inv_freq, pos, vt_col, eps, qb, kb, vb, ld_vt);
  else
    qk_norm_rope_kernel<XDNA_F16><<<g, 256, 0, st>>>(qkv, T, nh, nkv, q_w, k_w, inv_freq, pos, vt_col, eps, qb, kb, vb, ld_vt);
  return launch_status("qk_norm_rope");
}

int xdna_attention_bf16(const void* q, const void* k, const void* vt, int64_t ld_vt, const int32_t* seq_start,
                        const int32_t* seq_len, const int32_t* seq_vt, int64_t nseq, int64_t max_len, int nh, int nkv,
                        float scale, void* out, void* stream) {
  XDNA_REQUIRE(nseq >= 0 && max_len >= 0 && nh >= 1 && nkv >= 1 && nh % nkv == 0 && nh < 65536, "bad sizes");
  if (nseq == 0 || max_len == 0) return XDNA_OK;
  XDNA_REQUIRE(q && k && vt && seq_start && seq_len && seq_vt && out, "null pointer");
  XDNA_REQUIRE(ld_vt % 8 == 0 && aligned(q, 16) && aligned(k, 16) && aligned(vt, 16) && aligned(out, 8),
               "misaligned operands (ld_vt % 8, 16-byte q / k / vt)");
  const int64_t qblocks = cdiv(max_len, 32);
  XDNA_REQUIRE(nseq * qblocks < (1ll << 31), "too many sequences");
  dim3 g((unsigned)(nseq * qblocks), (unsigned)nh);
  attention_kernel<<<g, 64, 0, as_stream(stream)>>>(static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                                                     static_cast<const uint16_t*>(vt), ld_vt, seq_start, seq_len,
                                                     seq_vt, (int)qblocks, nh, nkv, scale, static_cast<uint16_t*>(out));
  return launch_status("attention_bf16");
}

int xdna_silu_mul_bf16(const float* gu, int64_t T, int64_t inter, void* y, void* stream) {
  XDNA_REQUIRE(T >= 0 && inter >= 1, "bad sizes");
  if (T == 0) return XDNA_OK;
  XDNA_REQUIRE(gu && y && cdiv(T * inter, 256) < (1ll << 31), "bad arguments");
  silu_mul_kernel<<<(unsigned)cdiv(T * inter, 256), 256, 0, as_stream(stream)>>>(gu, T, inter,
                                                                                 static_cast<uint16_t*>(y));
  return launch_status("silu_mul_bf16");
}

int xdna_add_f32(float* x, const float* y, int64_t n, void* stream) {
  XDNA_REQUIRE(n >= 0, "bad size");
  if (n == 0) return XDNA_OK;
  XDNA_REQUIRE(x && y && cdiv(n, 256) < (1ll << 31), "bad arguments");
  add_f32_kernel<<<(unsigned)cdiv(n, 256), 256, 0, as_stream(stream)>>>(x, y, n);
  return launch_status("add_f32");
}

}  // extern "C"
