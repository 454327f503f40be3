// int8 MFMA GEMM and implicit-GEMM 3x3 conv for gfx950 (MI355X).
//
// One tile engine serves both ops. A workgroup computes a BM x BN tile of D = A * W^T with
// A [M, K] and W [N, K] int8, both K-contiguous, accumulating in int32 with
// v_mfma_i32_32x32x32_i8 (the full-rate int8 MFMA of gfx950). The MFMA is issued as
// D^T = W * A^T (W fragment in srcA, A fragment in srcB), so each lane holds consecutive output
// columns n of one row m. Tiles: 256x256 with 8 waves (two per SIMD), 256x128 / 128x256 /
// 128x128 with 4 waves, 64x64 with 4 waves; the host picks one per shape.
//
// K is staged through S LDS stages of 64-byte slices by the LDS-DMA form of the raw buffer load:
// each lane's 16 bytes land at M0 + 16 * lane, so no VGPRs carry the tile, and S - 1 slices are in
// flight while one is consumed. LDS rows are 64 bytes; the 16-byte chunk c of row r sits at chunk
// c ^ f(r) with f(r) = (r >> 2) & 3. gfx950's LDS has 64 banks (a 256-byte period) and serves a
// 64-lane ds_read_b128 in 4 cycles when it is conflict-free; a fragment read (32 rows x 2 chunks)
// under this f measured 4.0 cycles per instruction and no SQ_LDS_BANK_CONFLICT cycles, where
// f(r) = ((r >> 1) ^ (r >> 3)) & 3 measured 8 (2-way) and no swizzle 16. f depends only on r & 15,
// so fragment offsets are immediates. Out-of-range rows, K chunks and conv halo pixels are out-of-range buffer loads, which
// read 0.
//
// Integer sums are exact, so the order in which K is split between lanes, MFMAs or waves does not
// change the result: the only requirement is that the A and W fragments of one MFMA pair the same
// k values, which both loaders guarantee by using one lane -> k mapping.
//
// The conv is the same engine with an implicit-im2col A loader: row m is output pixel
// (image, y, x), column k = tap * C_pad + c with tap = ky * 3 + kx, and the 16-byte chunk for
// (m, k) is 16 channels of input pixel (y + ky - 1, x + kx - 1) of the NHWC activation, or zeros
// outside the image (padding 1). C_pad % 16 == 0 keeps every chunk inside one tap.
//
// Epilogues: int32 store (xdna::linear_i8), dequantize + bias + cast (xdna::linear / linear_cat),
// shift / round-half-up / saturate (xdna::conv3x3), and the calibration max (first conv call).
//
// Small M (decode, M <= 64) uses a separate weight-streaming kernel: each workgroup owns 16 output
// columns, its waves (2, or 4 for K above 8 KB) split K, each wave keeps a batch of 16-byte weight loads in flight
// while it runs the MFMAs of the previous batch, and the partial sums meet in LDS. A single row (M = 1)
// has its own kernel that puts 16 K segments where the 16 rows would go (mm_gemv_kernel).
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <atomic>
#include <mutex>
#include <string>
#include <type_traits>
#include <unordered_map>

#include "xdna_common.h"

namespace xdna {

// EPI_DEQUANT_* carry the output dtype in the kernel's type so each epilogue is straight-line code.
// EPI_BF_*: the bf16 GEMM (precision "bf16"): float accumulators, + bias, cast to the output dtype.
enum Epi {
  EPI_I32 = 0, EPI_REQUANT = 2, EPI_CALIB = 3, EPI_DQ_F32 = 4, EPI_DQ_BF16 = 5, EPI_DQ_F16 = 6,
  EPI_BF_F32 = 7, EPI_BF_BF16 = 8, EPI_BF_F16 = 9, EPI_BF_SILU = 10
};
constexpr bool epi_dq(int e) { return e == EPI_DQ_F32 || e == EPI_DQ_BF16 || e == EPI_DQ_F16; }
// EPI_BF_SILU: the bf16 GEMM of a gated MLP's gate|up projection, its weight rows interleaved in pairs
// (gate 2j, gate 2j + 1, up 2j, up 2j + 1): each group of four sums gives two bf16 outputs silu(g) * u,
// column n of the GEMM writing output column n / 2.
constexpr bool epi_bf(int e) { return e == EPI_BF_F32 || e == EPI_BF_BF16 || e == EPI_BF_F16 || e == EPI_BF_SILU; }

struct EpiArgs {
  void* out;            // int32 C, float y, or int8/uint8 q (NHWC); with dq_out float y (NCHW)
  int64_t ldo;          // elements between output rows
  const float* sx;      // [M]; with dq_out per image [nb]
  const float* sw;      // [N]
  const float* bias;    // [N] or null
  int shift;            // EPI_REQUANT
  int relu;             // EPI_REQUANT / EPI_CALIB
  int32_t* acc_max;     // EPI_CALIB
  int vec_ok;           // output 16-byte aligned, row stride a multiple of 8 elements
  int dq_out;           // EPI_REQUANT: 0 writes the integers (NHWC); XDNA_F32 / BF16 / F16 + 1: the
                        // integers dequantized with sw = the conv's weight scales and sx = the per-image
                        // scales (+ bias), written NCHW in that dtype (out, sx not shifted by launch rows)
  int64_t px0;          // with dq_out: global pixel of the conv launch's first image
  // K split across workgroups (int8 GEMM tiles of at most 64 x 64): grid.y workgroups share a tile, each
  // summing a contiguous range of its K slices; ksplit <= 1 or part == null: no split
  int ksplit;
  uint32_t* cnt;        // [tiles * waves] arrival counters, zero before the launch (reset by the last arrival)
  int32_t* part;        // [tiles * waves][ksplit][the wave's int32 accumulators in register order]
  void* ws;             // host side: the caller's workspace (counters, then partial sums), or null
  int64_t ws_bytes;
};

struct ConvGeom {
  int64_t h, w, c_pad;  // NHWC input geometry
  int64_t m0;           // pixel (within the launch's images) of the launch's row 0
};

typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ i32x4 mfma16x16x64(const i32x4& a, const i32x4& b, const i32x4& c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// The tile engine's MFMA: on gfx950 the 32x32x32 int8 form issues at the full int8 rate
// (32768 MACs per 32 cycles per SIMD); the 16x16x64 form issues at half of it.
__device__ __forceinline__ i32x16 mfma32x32x32(const i32x4& a, const i32x4& b, const i32x16& c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// The bf16 forms take the same 16 bytes per lane (8 bf16 values instead of 16 int8) and the same
// lane layouts, so the byte-level staging of the int8 engine carries them unchanged: one MFMA covers
// 16 k-values (32 x 32) or 32 (16 x 16) instead of 32 / 64.
__device__ __forceinline__ f32x16 mfma32x32x16bf(const i32x4& a, const i32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32bf(const i32x4& a, const i32x4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// ------------------------------------------------------------------------------ epilogue
// Per-column values of CW consecutive output columns n .. n+CW-1 (weight scales and bias of the
// dequantize), loaded once per column block and reused for every row.
template <int EPI, int CW = 4>
struct EpiCols {
  float sw[CW], b[CW];
  __device__ __forceinline__ EpiCols() {}
  __device__ __forceinline__ EpiCols(const EpiArgs& e, int64_t n, int64_t N) {
    if constexpr (epi_dq(EPI)) load(e.sw, n, N, sw);
    if constexpr (epi_dq(EPI) || epi_bf(EPI)) {
#pragma unroll
      for (int r = 0; r < CW; ++r) b[r] = 0.0f;
      if (e.bias) load(e.bias, n, N, b);
    }
  }
  // One straight-line path: no per-lane branch merges the loaded values, so nothing waits for them
  // before the epilogue (the tile kernel issues these before its first K slice). Columns past N read
  // column N - 1; their outputs are never stored.
  __device__ __forceinline__ static void load(const float* p, int64_t n, int64_t N, float (&v)[CW]) {
#pragma unroll
    for (int r = 0; r < CW; ++r) v[r] = p[min(n + r, N - 1)];
  }
};

// One lane's CW outputs: row m, columns n .. n+CW-1 (acc[r] is column n + r). FULL: the caller has
// established that the whole tile is in bounds and the output rows take CW-wide vector stores, so
// there are no per-element tests. e.vec_ok: output rows are 16-byte aligned with a row stride that
// is a multiple of 8 elements (CW-wide stores at column multiples of CW are aligned).
template <int EPI, bool FULL, int CW>
__device__ __forceinline__ void epilogue_w(const EpiArgs& e, int64_t m, int64_t n, int64_t M, int64_t N,
                                           const int32_t (&acc)[CW], int& calib, const EpiCols<EPI, CW>& cols,
                                           float sxm) {
  static_assert(CW == 4 || CW == 8, "4 or 8 columns per lane");
  if (!FULL && m >= M) return;
  const bool vec = FULL || (e.vec_ok && n + CW - 1 < N);
  if constexpr (EPI == EPI_CALIB) {
#pragma unroll
    for (int r = 0; r < CW; ++r)
      if (FULL || n + r < N) calib = max(calib, e.relu ? max(acc[r], 0) : abs(acc[r]));
  } else if constexpr (EPI == EPI_I32) {
    int32_t* c = reinterpret_cast<int32_t*>(e.out) + m * e.ldo + n;
    if (vec) {
#pragma unroll
      for (int q = 0; q < CW / 4; ++q)
        *reinterpret_cast<i32x4*>(c + 4 * q) = i32x4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
    } else {
#pragma unroll
      for (int r = 0; r < CW; ++r)
        if (n + r < N) c[r] = acc[r];
    }
  } else if constexpr (EPI == EPI_REQUANT) {
    const int half = 1 << (e.shift - 1);
    uint32_t packed[CW / 4];
    int qv[CW];
#pragma unroll
    for (int r = 0; r < CW; ++r) {
      int q = (acc[r] + half) >> e.shift;      // arithmetic shift: floor, i.e. round half up
      q = e.relu ? min(max(q, 0), 255) : min(max(q, -128), 127);
      qv[r] = q;
    }
#pragma unroll
    for (int g = 0; g < CW / 4; ++g) {
      packed[g] = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) packed[g] |= ((uint32_t)(qv[4 * g + r] & 0xff)) << (8 * r);
    }
    uint8_t* o = reinterpret_cast<uint8_t*>(e.out) + m * e.ldo + n;
    if (vec) {
      if constexpr (CW == 8) *reinterpret_cast<uint2*>(o) = make_uint2(packed[0], packed[1]);
      else *reinterpret_cast<uint32_t*>(o) = packed[0];
    } else {
#pragma unroll
      for (int r = 0; r < CW; ++r)
        if (n + r < N) o[r] = (uint8_t)(qv[r] & 0xff);
    }
  } else if constexpr (EPI == EPI_BF_SILU) {
    // n is a multiple of 4 and N of 4 (the launcher checks): a group of four columns is wholly in or out;
    // silu(g) * u as the separate kernel computes it, g / (1 + exp(-g)) * u
    uint32_t h[CW / 4];
#pragma unroll
    for (int q = 0; q < CW / 4; ++q) {
      float y2[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const float g = __builtin_bit_cast(float, acc[4 * q + r]);
        const float u = __builtin_bit_cast(float, acc[4 * q + 2 + r]);
        y2[r] = g / (1.0f + __expf(-g)) * u;
      }
      h[q] = f32x2_to_bf16x2_bits(y2[0], y2[1]);
    }
    uint16_t* y = reinterpret_cast<uint16_t*>(e.out) + m * e.ldo + n / 2;
    if (vec) {
      if constexpr (CW == 8) *reinterpret_cast<uint2*>(y) = make_uint2(h[0], h[1]);
      else *reinterpret_cast<uint32_t*>(y) = h[0];
    } else {
#pragma unroll
      for (int q = 0; q < CW / 4; ++q)
        if (n + 4 * q < N) *reinterpret_cast<uint32_t*>(y + 2 * q) = h[q];
    }
  } else {
    // EPI_DQ_*: ((float)acc * sx[m]) * sw[n] (+ bias[n]), each step rounded once;
    // EPI_BF_*: the float accumulator (its bits arrive in acc) (+ bias[n])
    float v[CW];
#pragma unroll
    for (int r = 0; r < CW; ++r) {
      float t;
      if constexpr (epi_bf(EPI)) {
        t = __builtin_bit_cast(float, acc[r]);
      } else {
        t = (float)acc[r];
        t = t * sxm;
        t = t * cols.sw[r];
      }
      if (e.bias) t = t + cols.b[r];           // uniform test: the bias pointer is a kernel argument
      v[r] = t;
    }
    const int64_t off = m * e.ldo + n;
    if constexpr (EPI == EPI_DQ_F32 || EPI == EPI_BF_F32) {
      float* y = reinterpret_cast<float*>(e.out) + off;
      if (vec) {
#pragma unroll
        for (int q = 0; q < CW / 4; ++q)
          *reinterpret_cast<f32x4*>(y + 4 * q) = f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
      } else {
#pragma unroll
        for (int r = 0; r < CW; ++r)
          if (n + r < N) y[r] = v[r];
      }
    } else {
      uint32_t h[CW / 2];
#pragma unroll
      for (int q = 0; q < CW / 2; ++q)
        h[q] = (EPI == EPI_DQ_BF16 || EPI == EPI_BF_BF16) ? f32x2_to_bf16x2_bits(v[2 * q], v[2 * q + 1])
                                                          : f32x2_to_f16x2_bits(v[2 * q], v[2 * q + 1]);
      uint16_t* y = reinterpret_cast<uint16_t*>(e.out) + off;
      if (vec) {
        if constexpr (CW == 8) *reinterpret_cast<uint4*>(y) = make_uint4(h[0], h[1], h[2], h[3]);
        else *reinterpret_cast<uint2*>(y) = make_uint2(h[0], h[1]);
      } else {
#pragma unroll
        for (int r = 0; r < CW; ++r)
          if (n + r < N) y[r] = (uint16_t)(h[r / 2] >> (16 * (r & 1)));
      }
    }
  }
}

// Per element: an image boundary, an unaligned run, the end of the launch's rows.
__device__ __forceinline__ void epilogue_rqdq_each(const EpiArgs& e, int64_t hw, int64_t b, int64_t p, int64_t m,
                                                int64_t n, int64_t M, int64_t N, const float (&v)[4], float fo, float bo) {
  const int dt = e.dq_out - 1;
  const int esz = dt == XDNA_F32 ? 4 : 2;
  for (int r = 0; r < 4; ++r) {
    if (m + r >= M) return;
    while (p >= hw) {                        // the next image (several when an image has fewer than 4 pixels)
      p -= hw;
      ++b;
    }
    float t = v[r] * (fo * e.sx[b]);
    if (e.bias) t = t + bo;
    char* o = reinterpret_cast<char*>(e.out) + ((b * N + n) * hw + p) * esz;
    if (dt == XDNA_F32) *reinterpret_cast<float*>(o) = t;
    else if (dt == XDNA_BF16) *reinterpret_cast<uint16_t*>(o) = f32_to_bf16_bits(t);
    else *reinterpret_cast<uint16_t*>(o) = f32_to_f16_bits(t);
    ++p;
  }
}

// Where four consecutive output pixels m .. m+3 (launch rows) of the fused dequantize go: image b and pixel p
// within it, and whether the four lie in one image at an aligned position (then one vector store per channel,
// with the image's scale sx). The same for every channel, so the caller finds it once per four pixels. b_c /
// sx_c: an image index and its scale the caller loaded ahead (the image of the wave's first pixel), used
// instead of a load of e.sx[b] when the pixels lie in that image. Rows past M: fast = false, nothing loaded.
struct RqPix {
  int64_t b, p;
  float sx;
  bool fast;
};

__device__ __forceinline__ RqPix rq_pixel(const EpiArgs& e, const ConvGeom& cg, int64_t m, int64_t M, int64_t b_c,
                                          float sx_c) {
  RqPix r{0, 0, 0.0f, false};
  if (m >= M) return r;
  const int64_t hw = cg.h * cg.w;
  const int64_t gp = e.px0 + cg.m0 + m;  // global pixel of the first of the four
  // a 32-bit division where the pixel index allows (a 64-bit one costs several times the instructions)
  if (gp <= 0xffffffffll && hw <= 0xffffffffll) {
    const uint32_t bb = (uint32_t)gp / (uint32_t)hw;
    r.b = bb;
    r.p = gp - (int64_t)bb * hw;
  } else {
    r.b = gp / hw;
    r.p = gp - r.b * hw;
  }
  r.fast = m + 3 < M && r.p + 3 < hw && (r.p % 4) == 0 && hw % 4 == 0;
  if (r.fast) r.sx = r.b == b_c ? sx_c : e.sx[r.b];
  return r;
}

// The conv's requantize fused with the op's dequantize: four consecutive output pixels m .. m+3 (launch
// rows, placed by rq_pixel) of channel n, int32 sums in a[]. Each is requantized as EPI_REQUANT does, then
// dequantized as the separate dequantize kernel does, y = (float)q * (scale[n] * sx[image]) (+ bias[n]),
// and stored NCHW in dtype e.dq_out - 1: one 16-byte (float32) or 8-byte store when the four pixels lie in
// one image at an aligned position, else per element.
__device__ __forceinline__ void epilogue_rqdq(const EpiArgs& e, const ConvGeom& cg, const RqPix& px, int64_t m,
                                              int64_t n, int64_t M, int64_t N, const int32_t (&a)[4], float fo,
                                              float bo) {
  if (n >= N || m >= M) return;
  const int64_t hw = cg.h * cg.w;
  const int half = 1 << (e.shift - 1);
  float v[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    int q = (a[r] + half) >> e.shift;        // arithmetic shift: floor, i.e. round half up
    q = e.relu ? min(max(q, 0), 255) : min(max(q, -128), 127);
    v[r] = (float)q;
  }
  if (!px.fast) {
    epilogue_rqdq_each(e, hw, px.b, px.p, m, n, M, N, v, fo, bo);
    return;
  }
  const int64_t b = px.b, p = px.p;
  const int dt = e.dq_out - 1;
  const float f = fo * px.sx;
  float t[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    t[r] = v[r] * f;
    if (e.bias) t[r] = t[r] + bo;
  }
  char* o = reinterpret_cast<char*>(e.out) + ((b * N + n) * hw + p) * (dt == XDNA_F32 ? 4 : 2);
  if (dt == XDNA_F32) {
    *reinterpret_cast<f32x4*>(o) = f32x4{t[0], t[1], t[2], t[3]};
  } else if (dt == XDNA_BF16) {
    *reinterpret_cast<uint2*>(o) = make_uint2(f32x2_to_bf16x2_bits(t[0], t[1]), f32x2_to_bf16x2_bits(t[2], t[3]));
  } else {
    *reinterpret_cast<uint2*>(o) = make_uint2(f32x2_to_f16x2_bits(t[0], t[1]), f32x2_to_f16x2_bits(t[2], t[3]));
  }
}

// Four columns held as one i32x4 (the small-M kernel's accumulator).
template <int EPI>
__device__ __forceinline__ void epilogue4(const EpiArgs& e, int64_t m, int64_t n, int64_t M, int64_t N,
                                          const i32x4& acc, int& calib, const EpiCols<EPI, 4>& cols, float sxm) {
  const int32_t a[4] = {acc[0], acc[1], acc[2], acc[3]};
  epilogue_w<EPI, false, 4>(e, m, n, M, N, a, calib, cols, sxm);
}

template <int EPI>
__device__ __forceinline__ void calib_flush(const EpiArgs& e, int calib) {
  if constexpr (EPI == EPI_CALIB) {
    calib = wave_max_i(calib);
    if ((threadIdx.x & 63) == 0) atomicMax(e.acc_max, calib);
  }
}

// ------------------------------------------------------------------------------ tile engine
// XCD-aware order: consecutive workgroup ids go round-robin over the 8 XCDs, so ids are remapped
// to give each XCD a contiguous run of tiles, and runs are walked GROUP_M tile-rows at a time so
// that the workgroups sharing an XCD's L2 share A rows and W columns.
__device__ __forceinline__ void tile_coords(uint32_t pid, uint32_t tiles_m, uint32_t tiles_n, int64_t& tm,
                                            int64_t& tn) {
  // 32-bit arithmetic (the launcher keeps tile counts below 2^31): 64-bit divisions cost thousands
  // of cycles on the scalar unit
  constexpr uint32_t XCDS = 8;
  constexpr uint32_t GROUP_M = 8;
  const uint32_t total = tiles_m * tiles_n;
  const uint32_t q = total / XCDS, r = total % XCDS;
  const uint32_t xcd = pid % XCDS, local = pid / XCDS;
  const uint32_t tile = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + local;
  const uint32_t in_group = GROUP_M * tiles_n;
  const uint32_t g = tile / in_group;
  const uint32_t first_m = g * GROUP_M;
  const uint32_t gsz = min(GROUP_M, tiles_m - first_m);
  const uint32_t rem = tile - g * in_group;
  const uint32_t rdiv = rem / gsz;
  tm = first_m + (rem - rdiv * gsz);
  tn = rdiv;
}

// LDS rows are 64 bytes (one 64-deep K slice of a tile row); the 16-byte chunk c (0..3) of row r sits
// at chunk c ^ f(r) with f(r) = (r >> 2) & 3. A fragment read touches 32 consecutive rows at logical
// chunks 2 ks and 2 ks + 1 (lanes 0-31 and 32-63). Under this f every 16 consecutive lanes cover the 16
// bank groups of a 256-byte line and lanes l, l + 32 never share a 16-byte group within a 4-row block;
// measured on gfx950 (rocprofv3 SQ_LDS_IDX_ACTIVE / SQ_INSTS_LDS) at 4.0 cycles per ds_read_b128,
// the conflict-free minimum. f depends only on r & 15, so fragments 32 rows apart differ by a
// constant offset.
__device__ __forceinline__ int swz_f(int row) { return (row >> 2) & 3; }

// CONVM 3: haloed pixels (a multiple of 16) one halo buffer of a tile with BN columns, S weight stages and
// NW waves holds: what the LDS leaves after the weight stages and the sink, and what the loads can carry
// in the (10 - S) slices of a channel slice that may load the next one (one 16-pixel instruction per wave
// per slice).
__host__ __device__ constexpr int conv_halo_max(int bn, int s, int nw) {
  const int by_lds = ((160 * 1024 - s * bn * 64 - 1024) / (2 * 64)) / 16 * 16;
  const int by_loads = (10 - s) * nw * 16;
  return by_lds < by_loads ? by_lds : by_loads;
}
__device__ __forceinline__ int swz(int row, int chunk) { return (row << 6) + ((chunk ^ swz_f(row)) << 4); }


typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16 bytes per lane from global memory straight into LDS: lane l's bytes land at lds + 16 * l.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t off, int8_t* lds, uint32_t soff = 0) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, (int)off, (int)soff, 0, 0);
}

// s_waitcnt with a compile-time count (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8): wait until at most N vector memory loads of this wave are outstanding (they complete
// in issue order), optionally also for every LDS access.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
template <int N>
__device__ __forceinline__ void wait_vmcnt_lgkm0() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

// Wait for every LDS access of this wave (no vector-memory wait).
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4)); }

// Scheduling groups for __builtin_amdgcn_sched_group_barrier.
constexpr int SG_MFMA = 0x008, SG_VMEM_READ = 0x020, SG_DS_READ = 0x100;

// Emits NX groups "1 instruction of kind X, then its share of NM MFMAs" (shares differ by at most
// one), i.e. spreads NX memory instructions evenly over NM MFMAs in the scheduling region.
template <int X, int NX, int NM, int G>
struct PinGroups {
  __device__ __forceinline__ static void emit() {
    if constexpr (G < NX) {
      __builtin_amdgcn_sched_group_barrier(X, 1, 0);
      constexpr int nm = NM * (G + 1) / NX - NM * G / NX;
      if constexpr (nm > 0) __builtin_amdgcn_sched_group_barrier(SG_MFMA, nm, 0);
      PinGroups<X, NX, NM, G + 1>::emit();
    }
  }
};


// Emits NA groups "1 instruction of kind XA + its share of the first half of NM MFMAs", then NB
// groups "1 instruction of kind XB + its share of the second half".
template <int XA, int NA, int XB, int NB, int NM>
struct PinTwo {
  __device__ __forceinline__ static void emit() {
    PinGroups<XA, NA, NM / 2, 0>::emit();
    PinGroups<XB, NB, NM - NM / 2, 0>::emit();
  }
};

// Tile engine. Each 64-deep K slice of the A and W tiles is brought into LDS by the DMA form of the
// buffer load: one wave instruction fills 16 whole 64-byte LDS rows, and each lane fetches the global
// chunk that belongs at its LDS position under the swizzle. S LDS stages hold slices kt .. kt+S-1, so
// the loads of a slice have S - 1 slices of MFMAs to land. Per slice kt (two 32-deep MFMA steps):
//   step 0: MFMAs of the step-0 fragments, with the reads of the step-1 fragments in between;
//   wait for this wave's DMA of slice kt+1; barrier (every wave has read all of slice kt, and slice
//   kt+1 is complete);
//   step 1: MFMAs of the step-1 fragments, with the DMA of slice kt+S into slice kt's stage and the
//   reads of slice kt+1's step-0 fragments in between.
// Slices past the end of K are loaded as out-of-range (zero) reads, which keeps the wait counts and
// the loop uniform.
// KG > 1 splits K inside the workgroup: KG groups of WM x WN waves each run this pipeline in their own
// LDS stages over every KG-th slice (group g: slices g, g + KG, ...), all groups meeting at the same
// barriers; at the end groups 1 .. KG-1 leave their accumulators in LDS and group 0 adds them before
// the epilogue. It multiplies the loads in flight and the MFMA streams of a tile for shapes with few
// tiles and deep K (integer sums are exact in any order).
// f(std::integral_constant<int, I>{}) for I = I0 .. N - 1, unrolled at compile time
template <int I0, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I0 < N) {
    f(std::integral_constant<int, I0>{});
    static_for<I0 + 1, N>(f);
  }
}

template <int BM, int BN, int WM, int WN, int S, int CONVM, int EPI, bool KFULL, int KG = 1, bool PP = false>
__global__ __launch_bounds__(WM * WN * KG * 64) void mm_tile_kernel(const int8_t* __restrict__ a, int64_t lda,
                                                               const int8_t* __restrict__ w, int64_t ldw, int64_t M,
                                                               int64_t N, int64_t K, ConvGeom cg, EpiArgs e) {
  // CONVM: 0 GEMM, 1 conv with C_pad % 64 == 0, 2 any C_pad, 3 conv from a haloed input tile (below)
  constexpr bool CONV = CONVM != 0;
  constexpr bool HALO = CONVM == 3;
  constexpr int BK = 64;
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;  // 32 x 32 MFMA tiles per wave
  constexpr int IA = BM / 16 / NW;       // DMA instructions per wave per slice (16 rows each)
  constexpr int IW = BN / 16 / NW;
  static_assert(FM >= 1 && FN >= 1, "wave tile below 32 x 32");
  static_assert(IA >= 1 && IW >= 1 && BM % (16 * NW) == 0 && BN % (16 * NW) == 0, "tile / wave mismatch");
  // CONVM 3: the K slices are (64-channel slice, tap) pairs, taps inner. The stages hold only the weight
  // slices; the tile's input pixels plus a one-pixel border ("halo"), one channel slice at a time, sit in
  // two halo buffers after them (the slice being read, the next one being loaded), then a 1 KB sink for
  // the halo loads that carry nothing. Each input byte is loaded once per channel slice instead of once
  // per tap.
  static_assert(!HALO || (KG == 1 && !PP), "the haloed conv runs one K group, no ping-pong");
  constexpr int STAGE = HALO ? BN * BK : (BM + BN) * BK;
  constexpr int HMAX = HALO ? conv_halo_max(BN, S, NW) : 0;   // haloed pixels a buffer holds
  constexpr int LDS_BYTES = HALO ? S * STAGE + 2 * HMAX * BK + 1024 : KG * S * STAGE;
  static_assert(S >= 2 && KG >= 1 && LDS_BYTES <= 160 * 1024, "LDS stages");
  constexpr int NDMA = HALO ? IW + 1 : IA + IW;   // CONVM 3: the weight slice and one halo instruction
  static_assert((S - 1) * NDMA <= 63, "vmcnt range");

  __shared__ __attribute__((aligned(1024))) int8_t lds_all[LDS_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave_all = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: keeps LDS bases scalar
  const int kg = wave_all / NW;          // K group
  const int wave = wave_all - kg * NW;   // wave within the group
  const int wm = wave / WN, wn = wave % WN;
  int8_t* const lds = lds_all + kg * (S * STAGE);

  const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int64_t tm, tn;
  tile_coords(blockIdx.x, (uint32_t)tiles_m, (uint32_t)tiles_n, tm, tn);
  const int64_t m0 = tm * BM, n0 = tn * BN;

  // The epilogue's per-row and per-column scales do not depend on K: load them now, so they arrive
  // during the K loop. Read-back layout: row rr * 8 + (lane >> 3), columns 4 * (lane & 7) .. +3.
  constexpr bool DQ = EPI == EPI_DQ_F32 || EPI == EPI_DQ_BF16 || EPI == EPI_DQ_F16;
  float sx_pre[DQ ? TM / 8 : 1];
  if constexpr (DQ) {
#pragma unroll
    for (int rr = 0; rr < TM / 8; ++rr) {
      const int64_t m = m0 + wm * TM + rr * 8 + (lane >> 3);
      sx_pre[rr] = e.sx[min(m, M - 1)];   // rows past M are never stored
    }
  }
  // Epilogue read-back width: CB 32-column blocks side by side, CW columns per lane (8 lanes per row)
  constexpr int CB = FN % 2 == 0 ? 2 : 1;
  constexpr int CW = 4 * CB;
  EpiCols<EPI, CW> cols_pre[FN / CB];
#pragma unroll
  for (int jp = 0; jp < FN / CB; ++jp)
    cols_pre[jp] = EpiCols<EPI, CW>(e, n0 + wn * TN + jp * 32 * CB + (lane & 7) * CW, N);

  // conv: the launch's rows lie in whole images that start at a; a 3 x 3 window reads past the launch's
  // first and last rows within those images
  const int64_t conv_px = CONV ? (cg.m0 + M + cg.h * cg.w - 1) / (cg.h * cg.w) * (cg.h * cg.w) : 0;
  const __amdgpu_buffer_rsrc_t ra_rsrc = make_rsrc(a, (uint32_t)(CONV ? (conv_px * cg.c_pad) : (M * lda)));
  const __amdgpu_buffer_rsrc_t rw_rsrc = make_rsrc(w, (uint32_t)(N * ldw));

  // This lane's rows: DMA instruction j of this wave covers tile rows r0 = (wave * I + j) * 16 .. +16,
  // and lane l fills LDS chunk l % 4 of row r0 + l / 4, i.e. logical chunk (l % 4) ^ f(row).
  const int lrow = lane >> 2;
  const int pch = lane & 3;
  uint32_t oa[IA], ow[IW];
  int ca[IA], cw[IW];                    // logical chunk per slot
  int py[IA], px[IA];
  (void)py;
  (void)px;
  (void)oa;
  (void)ca;
#pragma unroll
  for (int j = 0; j < (HALO ? 0 : IA); ++j) {
    const int row = (wave * IA + j) * 16 + lrow;
    ca[j] = pch ^ swz_f(row);
    const int64_t m = m0 + row;
    if constexpr (CONV) {
      // 32-bit: M * c_pad stays below 2^30 (the launcher splits larger batches)
      const uint32_t hw = (uint32_t)(cg.h * cg.w);
      const uint32_t mm = m < M ? (uint32_t)(cg.m0 + m) : 0u;
      const uint32_t p = mm % hw;
      const uint32_t yy = p / (uint32_t)cg.w;
      py[j] = m < M ? (int)yy : -1000000;  // an invalid row fails every bounds test
      px[j] = (int)(p - yy * (uint32_t)cg.w);
      oa[j] = mm * (uint32_t)cg.c_pad;
    } else {
      oa[j] = m < M ? (uint32_t)(m * lda + ca[j] * 16) : OOB;
    }
  }
#pragma unroll
  for (int j = 0; j < IW; ++j) {
    const int row = (wave * IW + j) * 16 + lrow;
    cw[j] = pch ^ swz_f(row);
    const int64_t n = n0 + row;
    ow[j] = n < N ? (uint32_t)(n * ldw + cw[j] * 16) : OOB;
  }

  // CONVM 3: the tile is rt whole image rows of wt pixels (or, for rows wider than the tile, a wt-pixel
  // segment of one row) inside one image (the launcher checks); its halo is (rt + 2) x (wt + 2) pixels,
  // haloed pixel hp = (row + 1) * hw_halo + col + 1 for tile pixel (row, col). hp0[i]: the haloed pixel of
  // this lane's fragment row in MFMA row block i, before the tap's offset dy * hw_halo + dx.
  // All of it in 32-bit arithmetic (the launch's bytes stay below 2^31); the slice bookkeeping runs on the
  // scalar unit every slice, where 64-bit divisions would cost more issue slots than the MFMAs leave.
  int h_y0 = 0, h_x0 = 0, hw_halo = 0, hp_n = 0, h_nq = 0;
  uint32_t h_px0 = 0, h_ncs = 0;           // first pixel of the tile's image; channel slices
  int hp0[HALO ? FM : 1];
  (void)h_y0;
  (void)h_x0;
  (void)hw_halo;
  (void)hp_n;
  (void)h_nq;
  (void)h_px0;
  (void)h_ncs;
  (void)hp0;
  if constexpr (HALO) {
    const uint32_t ipx = (uint32_t)(cg.h * cg.w);
    const uint32_t gp0 = (uint32_t)(cg.m0 + m0);
    const uint32_t img = gp0 / ipx;
    h_px0 = img * ipx;
    const uint32_t p0 = gp0 - h_px0;
    h_y0 = (int)(p0 / (uint32_t)cg.w);
    h_x0 = (int)(p0 - (uint32_t)h_y0 * (uint32_t)cg.w);
    const int wt = (int)min<int64_t>(cg.w, BM);
    hw_halo = wt + 2;
    hp_n = (BM / wt + 2) * hw_halo;
    h_nq = (hp_n + 15) / 16;
    h_ncs = (uint32_t)(cg.c_pad / BK);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int p = wm * TM + i * 32 + (lane & 31);
      const int prow = p / wt;
      hp0[i] = (prow + 1) * hw_halo + (p - prow * wt) + 1;
    }
  }
  int8_t* const halo = lds_all + S * STAGE;          // CONVM 3: buffer b at halo + b * HMAX * BK
  int8_t* const halo_sink = halo + 2 * HMAX * BK;
  (void)halo;
  (void)halo_sink;
  // CONVM 3: halo slot jj of this wave is load instruction q = jj * NW + wave of a channel slice's halo: lane l
  // fills physical chunk l % 4 of haloed pixel 16 q + l / 4 with its logical chunk (l % 4) ^ f(pixel).
  // hsrc[jj]: that lane's source byte offset less the channel slice's, OOB for pixels outside the image (the
  // conv's zero padding) or past the halo (an offset past OOB is still past the buffer's end).
  uint32_t hsrc[HALO ? 10 - S : 1];
  (void)hsrc;
  if constexpr (HALO) {
#pragma unroll
    for (int jj = 0; jj < 10 - S; ++jj) {
      const int hp = 16 * (jj * NW + wave) + lrow;
      const int hy = hp / hw_halo;
      const int y = h_y0 - 1 + hy, x = h_x0 - 1 + (hp - hy * hw_halo);
      const bool ok = hp < hp_n && (uint32_t)y < (uint32_t)cg.h && (uint32_t)x < (uint32_t)cg.w;
      hsrc[jj] = ok ? (h_px0 + (uint32_t)(y * (int)cg.w + x)) * (uint32_t)cg.c_pad + (uint32_t)((pch ^ swz_f(hp)) * 16)
                    : OOB;
    }
  }

  // The cross-workgroup K split (int8 GEMM tiles of at most 64 x 64): workgroup blockIdx.y of the tile
  // sums slices [kbase, kbase + nk) of its nk_all
  constexpr bool CAN_SPLIT = CONVM == 0 && !PP && (EPI == EPI_I32 || epi_dq(EPI)) && BM * BN <= 64 * 64;
  const int64_t nk_all = (K + BK - 1) / BK;
  int64_t kbase = 0, nk = nk_all;
  if constexpr (CAN_SPLIT) {
    if (e.ksplit > 1) {
      const int64_t per = (nk_all + e.ksplit - 1) / e.ksplit;
      kbase = (int64_t)blockIdx.y * per;
      nk = max<int64_t>(0, min(nk_all, kbase + per) - kbase);
    }
  }
  // CONVM 1: a group's slices are issued in order, KG slices apart, so the tap and channel offset of
  // its next slice are kept as running counters instead of being divided out of k (the launcher takes
  // CONVM 1 with KG > 1 only when c_pad is a multiple of KG * 64, so each step wraps at most once).
  int dtap = 0, dc0 = 0;
  if constexpr (CONVM == 1) {
    dtap = (kg * BK) / (int)cg.c_pad;
    dc0 = (kg * BK) - dtap * (int)cg.c_pad;
  }
  (void)dtap;
  (void)dc0;
  auto dma_slice = [&](int64_t kt, int8_t* stage) {
    const int64_t k0 = (kbase + kt) * BK;
    const bool live = kt < nk;           // uniform; dead slices read zeros without memory traffic
    int8_t* sa = stage;
    int8_t* sw = stage + BM * BK;
    if constexpr (CONVM == 1) {
      // C_pad % 64 == 0: the whole slice is one tap
      const int dy = (dtap >= 3) + (dtap >= 6) - 1;
      const int dx = dtap - 3 * (dy + 1) - 1;
      const int64_t delta = ((int64_t)dy * cg.w + dx) * cg.c_pad + dc0;
#pragma unroll
      for (int j = 0; j < IA; ++j) {
        const int sy = py[j] + dy, sx = px[j] + dx;
        const bool ok = live && sy >= 0 && sy < cg.h && sx >= 0 && sx < cg.w;
        dma16(ra_rsrc, ok ? (uint32_t)(oa[j] + delta + ca[j] * 16) : OOB, sa + ((wave * IA + j) << 10));
      }
      dc0 += BK * KG;
      if (dc0 >= cg.c_pad) {
        dc0 -= (int)cg.c_pad;
        ++dtap;
      }
    } else if constexpr (CONVM == 2) {
#pragma unroll
      for (int j = 0; j < IA; ++j) {
        const uint32_t kb = (uint32_t)k0 + ca[j] * 16;
        const uint32_t tap = kb / (uint32_t)cg.c_pad;
        const uint32_t c = kb - tap * (uint32_t)cg.c_pad;
        const int dy = (int)(tap / 3) - 1, dx = (int)(tap % 3) - 1;
        const int sy = py[j] + dy, sx = px[j] + dx;
        const bool ok = kb < K && sy >= 0 && sy < cg.h && sx >= 0 && sx < cg.w;
        const int64_t delta = ((int64_t)dy * cg.w + dx) * cg.c_pad + c;
        dma16(ra_rsrc, ok ? (uint32_t)(oa[j] + delta) : OOB, sa + ((wave * IA + j) << 10));
      }
    } else {
      if (KFULL) {                         // K % 64 == 0: the per-slot offsets are constant
#pragma unroll
        for (int j = 0; j < IA; ++j)
          dma16(ra_rsrc, live ? oa[j] : OOB, sa + ((wave * IA + j) << 10), live ? (uint32_t)k0 : 0u);
      } else {
#pragma unroll
        for (int j = 0; j < IA; ++j) {
          // live: with a K split, a slice past this workgroup's range still lies inside K
          const bool ok = live && oa[j] != OOB && k0 + ca[j] * 16 < K;
          dma16(ra_rsrc, ok ? oa[j] + (uint32_t)k0 : OOB, sa + ((wave * IA + j) << 10));
        }
      }
    }
    if (KFULL) {
#pragma unroll
      for (int j = 0; j < IW; ++j)
        dma16(rw_rsrc, live ? ow[j] : OOB, sw + ((wave * IW + j) << 10), live ? (uint32_t)k0 : 0u);
    } else {
#pragma unroll
      for (int j = 0; j < IW; ++j) {
        const bool ok = live && ow[j] != OOB && k0 + cw[j] * 16 < K;
        dma16(rw_rsrc, ok ? ow[j] + (uint32_t)k0 : OOB, sw + ((wave * IW + j) << 10));
      }
    }
  };

  // Fragments of one 32-deep k step ks (2 per slice): lane l holds 16 bytes of row
  // (frag base + l % 32) at logical chunk 2 * ks + l / 32. Two register sets alternate: while the
  // MFMAs of one step run, the fragments of the next are read into the other set.
  const int frow = lane & 31;
  const int fk = lane >> 5;
  i32x4 fa[2][FM], fw[2][FN];
  auto read_frags = [&](const int8_t* stage, int ks, int set) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
      fa[set][i] = *reinterpret_cast<const i32x4*>(stage + swz(wm * TM + i * 32 + frow, ks * 2 + fk));
#pragma unroll
    for (int j = 0; j < FN; ++j)
      fw[set][j] = *reinterpret_cast<const i32x4*>(stage + BM * BK + swz(wn * TN + j * 32 + frow, ks * 2 + fk));
  };
  // CONVM 3: the input fragment of a slice comes from its channel slice's halo buffer hb, each row at its
  // haloed pixel moved by the tap (dy, dx): toff = dy * hw_halo + dx
  auto read_halo = [&](const int8_t* stage, const int8_t* hb, int ks, int set, int toff) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
      fa[set][i] = *reinterpret_cast<const i32x4*>(hb + swz(hp0[i] + toff, ks * 2 + fk));
#pragma unroll
    for (int j = 0; j < FN; ++j)
      fw[set][j] = *reinterpret_cast<const i32x4*>(stage + swz(wn * TN + j * 32 + frow, ks * 2 + fk));
  };
  // CONVM 3: the weight slice of (channel slice cs, tap) into a stage (zeros past the last channel slice)
  auto dma_w_tap = [&](int8_t* stage, uint32_t cs, int tap) {
    const bool live = cs < h_ncs;
    const uint32_t k0 = live ? (uint32_t)tap * (uint32_t)cg.c_pad + cs * BK : 0u;
#pragma unroll
    for (int j = 0; j < IW; ++j) dma16(rw_rsrc, live ? ow[j] : OOB, stage + ((wave * IW + j) << 10), k0);
  };

  constexpr bool BFE = epi_bf(EPI);       // bf16 operands, float accumulators
  using AccT = std::conditional_t<BFE, f32x16, i32x16>;
  AccT acc[FN][FM];
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int i = 0; i < FM; ++i) acc[j][i] = AccT{};
  auto mfmas = [&](int set) {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        if constexpr (BFE) acc[j][i] = mfma32x32x16bf(fw[set][j], fa[set][i], acc[j][i]);
        else acc[j][i] = mfma32x32x32(fw[set][j], fa[set][i], acc[j][i]);
      }
  };

  if constexpr (PP) {
    // Ping-pong schedule: the 8 waves form two groups of 4 (group = wm: waves 0-3 own rows [0, BM/2),
    // waves 4-7 rows [BM/2, BM)); wave w runs on SIMD w % 4, so every SIMD holds one wave of each
    // group. The workgroup steps through phases separated by barriers; in each phase one group runs a
    // memory phase (its share of the DMA of slice t + S - 1, then all 2 x (FM + FN) fragments of slice
    // t from LDS) while the other runs the 2 x FM x FN MFMAs of the slice it read in the phase before,
    // as one uninterrupted stream. Group 1 runs one phase behind group 0, so each SIMD's MFMA pipe
    // always has one wave feeding it while the other waits on memory.
    //   phase 2t:     group 0 memory (slice t)   group 1 MFMAs (slice t - 1)
    //   phase 2t + 1: group 0 MFMAs (slice t)    group 1 memory (slice t)
    // Slice t + S - 1 goes into the stage of slice t - 1, which both groups finished reading by the end
    // of phase 2t - 1. Before the barrier that ends phase 2t + 1 every wave has waited for its share of
    // slice t + 1 (issued at least S - 2 slices earlier), so group 0 reads a complete slice in phase
    // 2t + 2. Every wave passes 2 nk + 2 barriers.
    static_assert(NW == 8 && WM == 2 && KG == 1, "ping-pong: two groups of four waves");
    const int grp = wm;
#pragma unroll
    for (int s = 0; s < S - 1; ++s) dma_slice(s, lds + s * STAGE);
    wait_vmcnt<(S - 2) * NDMA>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (grp == 1) {
      __builtin_amdgcn_s_barrier();      // group 1 starts one phase behind
      __builtin_amdgcn_sched_barrier(0);
    }
    int cur_s = 0;
    for (int64_t t = 0; t < nk; ++t) {
      const int prev_s = cur_s == 0 ? S - 1 : cur_s - 1;
      dma_slice(t + S - 1, lds + prev_s * STAGE);
      const int8_t* cur = lds + cur_s * STAGE;
      read_frags(cur, 0, 0);
      read_frags(cur, 1, 1);
      if (grp == 1) wait_vmcnt_lgkm0<(S - 2) * NDMA>();
      else wait_lgkm0();
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      mfmas(0);
      mfmas(1);
      __builtin_amdgcn_sched_barrier(0);
      if (grp == 0) wait_vmcnt<(S - 2) * NDMA>();
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      cur_s = cur_s + 1 == S ? 0 : cur_s + 1;
    }
    if (grp == 0) __builtin_amdgcn_s_barrier();
  } else if constexpr (HALO) {
    // The schedule of the loop below, one channel slice c per iteration with its nine taps unrolled, so the
    // tap's offsets and the halo slot each tap carries are compile-time constants. In tap t of channel slice
    // c (slice 9 c + t) the DMA issues slice 9 c + t + S's weights and, for t <= 9 - S, halo slot t of
    // channel slice c + 1 into buffer (c + 1) & 1 (last read by channel slice c - 1, whose reads every wave
    // finished before the first barrier of channel slice c); other taps issue one load into the sink, so
    // every slice issues NDMA loads. The last slot rides on slice 9 c + 9's DMA, so the wait before that
    // slice's first read covers the whole halo.
    constexpr int NMF = FM * FN, NRD = FM + FN;
    const int8_t* const hb0 = halo;
    const int8_t* const hb1 = halo + HMAX * BK;
    // prologue: the halo of channel slice 0, then taps 0 .. S-1 into stages 0 .. S-1; wait for tap 0
#pragma unroll
    for (int jj = 0; jj < 10 - S; ++jj) {
      const int q = jj * NW + wave;
      if (q < h_nq) dma16(ra_rsrc, hsrc[jj], halo + (q << 10));
    }
#pragma unroll
    for (int s = 0; s < S; ++s) {
      dma_w_tap(lds + s * STAGE, 0u, s);
      dma16(ra_rsrc, OOB, halo_sink);
    }
    wait_vmcnt<(S - 1) * NDMA>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    read_halo(lds, hb0, 0, 0, -hw_halo - 1);
    int cur_s = 0;
    for (uint32_t c = 0; c < h_ncs; ++c) {
      const int8_t* const hb = (c & 1u) ? hb1 : hb0;
      const int8_t* const hbn = (c & 1u) ? hb0 : hb1;
      // 256-row tiles: hw_halo through an empty asm each iteration, so the nine taps' fragment addresses are
      // computed where they are read instead of being kept live across the loop (9 x FM registers more than
      // such a tile has left); smaller tiles keep them
      int hw = hw_halo;
      if constexpr (FM * FN >= 8) asm volatile("" : "+s"(hw));
      static_for<0, 9>([&](auto tc) {
        constexpr int t = decltype(tc)::value;
        constexpr int tn = (t + S) % 9, cn = (t + S) / 9;   // the slice this tap's DMA issues
        constexpr int t1 = (t + 1) % 9;                      // the next slice's tap
        int8_t* cur = lds + cur_s * STAGE;
        const int nxt_s = cur_s + 1 == S ? 0 : cur_s + 1;
        const int8_t* nxt = lds + nxt_s * STAGE;
        // step 0
        read_halo(cur, hb, 1, 1, (t / 3 - 1) * hw + (t % 3 - 1));
        mfmas(0);
        PinGroups<SG_DS_READ, NRD, NMF, 0>::emit();
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt_lgkm0<(S - 2) * NDMA>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // step 1
        dma_w_tap(cur, c + cn, tn);
        if constexpr (t <= 9 - S) {
          const int q = t * NW + wave;
          const bool on = c + 1u < h_ncs && q < h_nq;
          dma16(ra_rsrc, on ? hsrc[t] + (c + 1u) * BK : OOB, on ? (int8_t*)hbn + (q << 10) : halo_sink);
        } else {
          dma16(ra_rsrc, OOB, halo_sink);
        }
        read_halo(nxt, t == 8 ? hbn : hb, 0, 0, (t1 / 3 - 1) * hw + (t1 % 3 - 1));
        mfmas(1);
        PinTwo<SG_VMEM_READ, NDMA, SG_DS_READ, NRD, NMF>::emit();
        __builtin_amdgcn_sched_barrier(0);
        cur_s = nxt_s;
      });
    }
  } else {
  // prologue: the group's slices 0 .. S-1 into stages 0 .. S-1, then wait for slice 0
#pragma unroll
  for (int s = 0; s < S; ++s) dma_slice(kg + (int64_t)KG * s, lds + s * STAGE);
  // bare barrier: __syncthreads() would also fence, i.e. wait for every load of the prologue
  wait_vmcnt<(S - 1) * NDMA>();
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  read_frags(lds, 0, 0);

  constexpr int NMF = FM * FN, NRD = FM + FN;
  int cur_s = 0;
  const int64_t nkg = (nk + KG - 1) / KG;   // slices per group (past nk: zero slices)
  for (int64_t it = 0; it < nkg; ++it) {
    const int64_t kt = kg + KG * it;
    int8_t* cur = lds + cur_s * STAGE;
    const int nxt_s = cur_s + 1 == S ? 0 : cur_s + 1;
    const int8_t* nxt = lds + nxt_s * STAGE;
    // step 0
    read_frags(cur, 1, 1);
    mfmas(0);
    PinGroups<SG_DS_READ, NRD, NMF, 0>::emit();
    __builtin_amdgcn_sched_barrier(0);
    // slice kt+1 landed (this wave's part), this wave's reads of slice kt done; then all waves
    wait_vmcnt_lgkm0<(S - 2) * NDMA>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // step 1
    dma_slice(kt + (int64_t)KG * S, cur);
    read_frags(nxt, 0, 0);
    mfmas(1);
    PinTwo<SG_VMEM_READ, NDMA, SG_DS_READ, NRD, NMF>::emit();
    __builtin_amdgcn_sched_barrier(0);
    cur_s = nxt_s;
  }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Epilogue through LDS. The 32x32 accumulator of tile (j, i) holds, in lane l, output row
  // m = i * 32 + l % 32 of the wave tile and, in element 4 * g + r, column 8 * g + 4 * (l / 32) + r of
  // column block j. CB accumulator blocks of one row block go to a per-wave LDS staging area as 32
  // int32 rows of 32 * CB columns (pitch 32 * CB * 4 + 16 bytes: conflict-free 16-byte writes and
  // reads), read back CW consecutive columns per lane, eight lanes per row: each store instruction
  // writes whole 8-row pieces of 32 * CB contiguous columns (full 128-byte lines for bf16 with CB 2).
  constexpr int PITCH = 32 * CB * 4 + 16;
  static_assert(NW * 32 * PITCH <= (HALO ? LDS_BYTES : S * STAGE), "staging does not fit in LDS");
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();                       // every wave is done with the K-loop's LDS stages
  if constexpr (KG > 1) {
    // groups 1 .. KG-1 hand their accumulators to group 0 through LDS, past group 0's staging area
    constexpr int ACCB = FN * FM * 64 * 64;            // bytes of one wave's accumulators
    constexpr int RED0 = ((NW * 32 * PITCH + 1023) / 1024) * 1024;
    static_assert(RED0 + (KG - 1) * NW * ACCB <= KG * S * STAGE, "reduction does not fit in LDS");
    if (kg > 0) {
      int8_t* r = lds_all + RED0 + ((kg - 1) * NW + wave) * ACCB;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const i32x16 c = __builtin_bit_cast(i32x16, acc[j][i]);
#pragma unroll
          for (int g = 0; g < 4; ++g)
            *reinterpret_cast<i32x4*>(r + ((j * FM + i) * 4 + g) * 1024 + lane * 16) =
                i32x4{c[4 * g], c[4 * g + 1], c[4 * g + 2], c[4 * g + 3]};
        }
    }
    __syncthreads();
    if (kg > 0) return;                  // no barrier follows
#pragma unroll
    for (int u = 1; u < KG; ++u) {
      const int8_t* r = lds_all + RED0 + ((u - 1) * NW + wave) * ACCB;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            // the partner's values in their own type (float sums for bf16 operands): no bit casts of
            // vector elements
            using V4 = std::conditional_t<BFE, f32x4, i32x4>;
            const V4 t = *reinterpret_cast<const V4*>(r + ((j * FM + i) * 4 + g) * 1024 + lane * 16);
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[j][i][4 * g + q] += t[q];
          }
    }
  }
  if constexpr (CAN_SPLIT) {
    if (e.ksplit > 1) {
      // Every wave (of group 0) stores its partial sums; the wave that arrives last for its (tile, wave)
      // slot adds the others' and runs the epilogue. The workgroups of a tile may run on different XCDs,
      // whose L2 caches are not coherent with each other: the partials go out as agent-scope atomic
      // stores and come back as agent-scope atomic loads, which are coherent across XCDs by themselves,
      // and the arrival count is an agent-scope atomic issued after every partial store has completed
      // (vmcnt 0). Fences would write back and invalidate the whole L2 of the XCD instead, for every
      // wave. Integer sums are exact in any order: the result does not depend on which wave is last.
      constexpr int WORDS = FN * FM * 16;                   // int32 accumulators per lane
      const int64_t slot = (int64_t)blockIdx.x * NW + wave;
      const int ks = (int)blockIdx.y;
      int32_t* const base = e.part + slot * e.ksplit * WORDS * 64;
      {
        int32_t* mine = base + ks * WORDS * 64;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int i = 0; i < FM; ++i) {
            const i32x16 c = __builtin_bit_cast(i32x16, acc[j][i]);
#pragma unroll
            for (int r = 0; r < 16; ++r)
              __hip_atomic_store(mine + ((j * FM + i) * 16 + r) * 64 + lane, c[r], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
          }
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      uint32_t prev = 0;
      if (lane == 0) prev = __hip_atomic_fetch_add(e.cnt + slot, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      prev = (uint32_t)__builtin_amdgcn_readfirstlane((int)prev);
      if (prev + 1 < (uint32_t)e.ksplit) return;          // wave-uniform; no barrier follows
      for (int u = 0; u < e.ksplit; ++u) {
        if (u == ks) continue;
        const int32_t* p = base + u * WORDS * 64;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              acc[j][i][r] += __hip_atomic_load(p + ((j * FM + i) * 16 + r) * 64 + lane, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
      }
      if (lane == 0) __hip_atomic_store(e.cnt + slot, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // for the next launch
    }
  }
  int8_t* stg = lds + wave * 32 * PITCH;     // group 0: lds == lds_all
  int calib = 0;
  // uniform: the whole tile is inside M x N and the output rows take CW-wide vector stores
  const bool full = m0 + BM <= M && n0 + BN <= N && (EPI == EPI_CALIB || e.vec_ok);
  const int rsub = lane >> 3;            // read-back: row rr * 8 + rsub, columns CW * (lane & 7) ..
  const int cq = lane & 7;
  // the conv's fused dequantize (EPI_REQUANT with e.dq_out, uniform): the staged block (32 pixels x COLS
  // channels) is read back transposed, eight lanes per channel with four consecutive pixels each, so every
  // store instruction writes whole 128-byte runs of eight channels of the NCHW output
  constexpr int COLS = 32 * CB;          // staged columns per block
  // not for three column blocks per wave (256 x 192): that epilogue would outgrow full unrolling, and the
  // launcher runs such launches with another tile
  constexpr bool RQDQ = EPI == EPI_REQUANT && FN != 3;
  const bool rqdq = RQDQ && e.dq_out != 0;
  const int dquad = lane & 7;            // the lane's four pixels: 4 * dquad .. + 3 of the block
  const int dch = lane >> 3;             // the lane's channel within each group of eight
  // the fused dequantize's per-image scale of the wave's first pixel (its last rows may lie past M: the
  // first pixel is clamped into the launch), loaded once instead of once per four outputs
  int64_t rq_b = 0;
  float rq_sx = 0.0f;
  if constexpr (RQDQ) {
    if (rqdq) {
      const int64_t hw = cg.h * cg.w;
      rq_b = (e.px0 + cg.m0 + min(m0 + wm * TM, M - 1)) / hw;
      rq_sx = e.sx[rq_b];
    }
  }
  (void)rq_b;
  (void)rq_sx;
#pragma unroll
  for (int jp = 0; jp < FN / CB; ++jp) {
    const int64_t n = n0 + wn * TN + jp * 32 * CB + cq * CW;
    // the fused dequantize's weight scale and bias of column block jp: lane l holds those of channel l % COLS
    // (all loaded at once); the rolled loop below takes its channel's from the holding lane
    float rq_fo = 0.0f, rq_bo = 0.0f;
    if constexpr (RQDQ) {
      if (rqdq) {
        const int64_t nl = min<int64_t>(n0 + wn * TN + jp * COLS + (lane % COLS), N - 1);
        rq_fo = e.sw[nl];
        rq_bo = e.bias ? e.bias[nl] : 0.0f;
      }
    }
    (void)rq_fo;
    (void)rq_bo;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int jj = 0; jj < CB; ++jj) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const i32x16 c = __builtin_bit_cast(i32x16, acc[jp * CB + jj][i]);   // float bits for BFE
          *reinterpret_cast<i32x4*>(stg + (lane & 31) * PITCH + (jj * 32 + 8 * g + 4 * (lane >> 5)) * 4) =
              i32x4{c[4 * g], c[4 * g + 1], c[4 * g + 2], c[4 * g + 3]};
        }
      }
      if (rqdq) {
        if constexpr (RQDQ) {
          // unrolled by four, not fully: four channels' LDS reads and shuffles go out together (a rolled loop
          // waited on them once per channel), and fully unrolled (with every tile's blocks) the epilogue would
          // outgrow full unrolling of the accumulator loops
          const int64_t mq = m0 + wm * TM + i * 32 + 4 * dquad;   // the lane's four pixels
          const RqPix px = rq_pixel(e, cg, mq, M, rq_b, rq_sx);
#pragma unroll 4
          for (int g8 = 0; g8 < COLS / 8; ++g8) {
            const int col = 8 * g8 + dch;
            const int64_t nd = n0 + wn * TN + jp * COLS + col;
            const float fo = __shfl(rq_fo, col, 64);    // e.sw[min(nd, N - 1)]
            const float bo = __shfl(rq_bo, col, 64);
            int32_t a4[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) a4[r] = *reinterpret_cast<const int32_t*>(stg + (4 * dquad + r) * PITCH + col * 4);
            epilogue_rqdq(e, cg, px, mq, nd, M, N, a4, fo, bo);
          }
        }
      } else {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int row = rr * 8 + rsub;
          int32_t v[CW];
#pragma unroll
          for (int q = 0; q < CB; ++q) {
            const i32x4 t = *reinterpret_cast<const i32x4*>(stg + row * PITCH + cq * CW * 4 + q * 16);
            v[4 * q] = t[0], v[4 * q + 1] = t[1], v[4 * q + 2] = t[2], v[4 * q + 3] = t[3];
          }
          const int64_t m = m0 + wm * TM + i * 32 + row;
          const float sxm = sx_pre[DQ ? i * 4 + rr : 0];
          if (full) epilogue_w<EPI, true, CW>(e, m, n, M, N, v, calib, cols_pre[jp], sxm);
          else epilogue_w<EPI, false, CW>(e, m, n, M, N, v, calib, cols_pre[jp], sxm);
        }
      }
    }
  }
  calib_flush<EPI>(e, calib);
}

// ------------------------------------------------------------------------------ small M
// Weight streaming for M <= 64 (decode): a workgroup of WAVES waves owns output columns
// [n0, n0 + 16) and rows [m0, m0 + 16); wave v sums k over its own range [kbeg, kend) (a multiple of
// 64 bytes). Per 64-deep step a lane loads 16 bytes of weight row n0 + (lane & 15) and of activation
// row m0 + (lane & 15) at k + 16 * (lane >> 4), and one 16x16x64 MFMA consumes them. Steps go in
// batches of U with two register sets, so the loads of the next batch are in flight while the MFMAs of
// this one run. Rows past M / N and bytes past the wave's range read as zeros (out-of-range buffer
// loads). The waves' partial sums meet in LDS; wave 0 runs the epilogue.
__device__ __forceinline__ i32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return i32x4{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
}

template <int WAVES, int U, int EPI>
__global__ __launch_bounds__(WAVES * 64) void mm_small_kernel(const int8_t* __restrict__ a, int64_t lda,
                                                              const int8_t* __restrict__ w, int64_t ldw, int64_t M,
                                                              int64_t N, int64_t K, int64_t kper, EpiArgs e) {
  constexpr bool BFE = epi_bf(EPI);       // bf16 operands, float accumulators
  using Acc4 = std::conditional_t<BFE, f32x4, i32x4>;
  __shared__ Acc4 red[WAVES][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int64_t m0 = (int64_t)blockIdx.y * 16;
  const int64_t n = n0 + (lane & 15);
  const int64_t m = m0 + (lane & 15);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)(N * ldw));
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(a, (uint32_t)(M * lda));
  const uint32_t wrow = n < N ? (uint32_t)(n * ldw) : OOB;
  const uint32_t arow = m < M ? (uint32_t)(m * lda) : OOB;
  const int64_t kbeg = (int64_t)wave * kper;
  const int64_t kend = min(K, kbeg + kper);
  const int cq = (lane >> 4) * 16;

  auto load = [&](int64_t kb, i32x4 (&wv)[U], i32x4 (&av)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k = kb + u * 64 + cq;
      const bool kin = k < kend;
      wv[u] = buf_load16(rw, kin && wrow != OOB ? wrow + (uint32_t)k : OOB);
      av[u] = buf_load16(ra, kin && arow != OOB ? arow + (uint32_t)k : OOB);
    }
  };
  // two accumulators alternate so consecutive MFMAs do not wait on each other
  Acc4 acc0 = {}, acc1 = {};
  auto mfma = [&](const i32x4& w_, const i32x4& a_, Acc4& c) {
    if constexpr (BFE) c = mfma16x16x32bf(w_, a_, c);
    else c = mfma16x16x64(w_, a_, c);
  };
  auto mfmas = [&](const i32x4 (&wv)[U], const i32x4 (&av)[U]) {
#pragma unroll
    for (int u = 0; u < U; u += 2) {
      mfma(wv[u], av[u], acc0);
      if (u + 1 < U) mfma(wv[u + 1], av[u + 1], acc1);
    }
  };
  // the epilogue's operands (wave 0 runs it) go out ahead of the K loop where the 9 registers they hold
  // through it cost no occupancy (up to 4 waves; 8 and 16 waves load them after the loop)
  constexpr bool PRE = WAVES <= 4;
  const int64_t mrow = m0 + (lane & 15);
  EpiCols<EPI> cols;
  float sxm = 0.0f;
  auto load_epi = [&]() {
    cols = EpiCols<EPI>(e, n0 + 4 * (lane >> 4), N);
    if constexpr (epi_dq(EPI)) sxm = e.sx[min(mrow, M - 1)];
  };
  if constexpr (PRE) load_epi();
  i32x4 w0[U], a0[U], w1[U], a1[U];
  load(kbeg, w0, a0);
  for (int64_t kb = kbeg; kb < kend; kb += 2 * U * 64) {
    load(kb + U * 64, w1, a1);
    mfmas(w0, a0);
    if (kb + U * 64 >= kend) break;
    load(kb + 2 * U * 64, w0, a0);
    mfmas(w1, a1);
  }
  Acc4 acc = acc0 + acc1;
  red[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int v = 1; v < WAVES; ++v) acc += red[v][lane];
  int calib = 0;
  if constexpr (!PRE) load_epi();
  epilogue4<EPI>(e, mrow, n0 + 4 * (lane >> 4), M, N, __builtin_bit_cast(i32x4, acc), calib, cols, sxm);
  calib_flush<EPI>(e, calib);
}

// ------------------------------------------------------------------------------ one row (M = 1)
// GEMV for a single activation row. The 16 columns of the 16x16x64 MFMA carry 16 K segments of the
// one row instead of 16 rows: in a 1 KB step at byte kb, lane l (A row and B column i = l % 16, k chunk
// c = l / 16) holds bytes kb + 16 l .. +15 of both the weight row and the activation, so D[i][i] sums
// exactly the bytes kb + 16 (i + 16 c) + q over c and q, and the trace of D over the steps is the dot
// product (the off-diagonal sums are discarded; integer sums are exact in any order). Every weight
// load is one contiguous KB of one row and every activation byte is loaded once per wave, where the
// 16-row layout of mm_small_kernel spends a mostly-empty activation load per weight load. A wave owns
// one output column; KS steps (KS KB of K) are loaded before their MFMAs, longer K in rounds.
// The scale and bias operands of one output element (row m, column n), loaded by the kernel ahead of its
// K loop so that their latency hides under the weight stream instead of following it. m and n must be
// in range (callers clamp them).
template <int EPI>
struct Epi1Ops {
  float sx = 0.0f, sw = 0.0f, b = 0.0f;
  __device__ __forceinline__ Epi1Ops() {}
  __device__ __forceinline__ Epi1Ops(const EpiArgs& e, int64_t m, int64_t n) {
    if constexpr (epi_dq(EPI)) {
      sx = e.sx[m];
      sw = e.sw[n];
    }
    if constexpr (epi_dq(EPI) || epi_bf(EPI)) {
      if (e.bias) b = e.bias[n];
    }
  }
};

// One output element (row m, column n) of a GEMM epilogue, with the arithmetic of epilogue_w.
template <int EPI, typename T>
__device__ __forceinline__ void epilogue1(const EpiArgs& e, int64_t m, int64_t n, T v, const Epi1Ops<EPI>& o) {
  static_assert(EPI != EPI_REQUANT && EPI != EPI_CALIB, "GEMM epilogues only");
  const int64_t off = m * e.ldo + n;
  if constexpr (EPI == EPI_I32) {
    reinterpret_cast<int32_t*>(e.out)[off] = v;
  } else {
    // ((float)acc * sx) * sw (+ bias), or the float sum (+ bias); no bias adds nothing (not +0.0,
    // which would turn a -0.0 into +0.0)
    float t;
    if constexpr (epi_bf(EPI)) {
      t = v;
    } else {
      t = (float)v;
      t = t * o.sx;
      t = t * o.sw;
    }
    if (e.bias) t = t + o.b;
    if constexpr (EPI == EPI_DQ_F32 || EPI == EPI_BF_F32) reinterpret_cast<float*>(e.out)[off] = t;
    else if constexpr (EPI == EPI_DQ_BF16 || EPI == EPI_BF_BF16) reinterpret_cast<uint16_t*>(e.out)[off] = f32_to_bf16_bits(t);
    else reinterpret_cast<uint16_t*>(e.out)[off] = f32_to_f16_bits(t);
  }
}

template <int W, int KS, int EPI>
__global__ __launch_bounds__(W * 64) void mm_gemv_kernel(const int8_t* __restrict__ a, const int8_t* __restrict__ w,
                                                         int64_t ldw, int64_t N, int64_t K, EpiArgs e) {
  constexpr bool BFE = epi_bf(EPI);       // bf16 operands, float accumulators
  using Acc4 = std::conditional_t<BFE, f32x4, i32x4>;
  using T = std::conditional_t<BFE, float, int32_t>;
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * W + (threadIdx.x >> 6);
  if (n >= N) return;                     // wave-uniform, and the kernel has no barrier
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)(N * ldw));
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(a, (uint32_t)K);
  const uint32_t wrow = (uint32_t)(n * ldw);
  auto mfma = [&](const i32x4& w_, const i32x4& a_, Acc4& c) {
    if constexpr (BFE) c = mfma16x16x32bf(w_, a_, c);
    else c = mfma16x16x64(w_, a_, c);
  };
  const Epi1Ops<EPI> ops(e, 0, n);
  Acc4 acc0 = {}, acc1 = {};
  for (int64_t kc = 0; kc < K; kc += KS * 1024) {
    i32x4 wv[KS], xv[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int64_t k = kc + s * 1024 + 16 * lane;
      if (kc + s * 1024 < K) {            // uniform: steps wholly past K issue no loads
        wv[s] = buf_load16(rw, k < K ? wrow + (uint32_t)k : OOB);
        xv[s] = buf_load16(ra, k < K ? (uint32_t)k : OOB);
      } else {
        wv[s] = i32x4{0, 0, 0, 0};
        xv[s] = i32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int s = 0; s < KS; s += 2) {     // two accumulators: consecutive MFMAs do not wait on each other
      mfma(wv[s], xv[s], acc0);
      if (s + 1 < KS) mfma(wv[s + 1], xv[s + 1], acc1);
    }
  }
  const Acc4 acc = acc0 + acc1;
  // lane l holds D[4 (l / 16) + j][l % 16] in element j: the diagonal is in lanes with
  // (l % 16) / 4 == l / 16, element l % 4
  const int i = lane & 15;
  const int j = lane & 3;
  const T d = j == 0 ? acc[0] : j == 1 ? acc[1] : j == 2 ? acc[2] : acc[3];
  T v = (i >> 2) == (lane >> 4) ? d : T(0);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  if (lane == 0) epilogue1<EPI>(e, 0, n, v, ops);
}

// ------------------------------------------------------------------------------ a few rows (M <= 16)
// The segment trick with 4 segments of 4 rows: the 16 rows of the MFMA's A operand are 4 weight rows x 4
// segments and its 16 columns 4 activation rows x 4 segments. In a 256-byte step at byte kb, lane l
// (row / column i = l % 16, k chunk c = l / 16) holds bytes kb + 16 (i % 4 + 4 c) .. +15 of weight row
// i / 4 (A) and of activation row i / 4 (B), so D[i][m] with i % 4 == m % 4 sums segment i % 4 of the
// step for weight row i / 4 and activation row m / 4, and the four segments together cover the step.
// In the accumulator, lane l's element l % 4 is that segment's sum for weight row l / 16 and activation
// row (l % 16) / 4; the sum over the lane's quad is the dot product over the step. Every load is 4 rows x
// 256 contiguous bytes. The activation comes in XG groups of 4 rows, each loaded once per step and used
// for the R weight-row groups of the workgroup; the W waves split K into multiples of 256 bytes and
// their sums meet in LDS.
template <int W, int R, int XG, int EPI>
__global__ __launch_bounds__(W * 64) void mm_seg4_kernel(const int8_t* __restrict__ a, int64_t lda,
                                                         const int8_t* __restrict__ w, int64_t ldw, int64_t M,
                                                         int64_t N, int64_t K, int64_t kper, EpiArgs e) {
  constexpr bool BFE = epi_bf(EPI);       // bf16 operands, float accumulators
  using Acc4 = std::conditional_t<BFE, f32x4, i32x4>;
  using T = std::conditional_t<BFE, float, int32_t>;
  constexpr int KS = 4;                   // 256-byte steps loaded before their MFMAs
  __shared__ T red[W][R][XG][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t n0 = (int64_t)blockIdx.x * (4 * R);
  const int rsub = (lane & 15) >> 2;      // this lane's row within a group of 4 (A and B alike)
  const uint32_t koff = 16 * ((lane & 3) + 4 * (lane >> 4));
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)(N * ldw));
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(a, (uint32_t)(M * lda));
  uint32_t wrow[R], arow[XG];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t n = n0 + 4 * r + rsub;
    wrow[r] = n < N ? (uint32_t)(n * ldw) : OOB;
  }
#pragma unroll
  for (int q = 0; q < XG; ++q) {
    const int64_t m = 4 * q + rsub;
    arow[q] = m < M ? (uint32_t)(m * lda) : OOB;
  }
  const int64_t kbeg = (int64_t)wave * kper;
  const int64_t kend = min(K, kbeg + kper);
  auto mfma = [&](const i32x4& w_, const i32x4& a_, Acc4& c) {
    if constexpr (BFE) c = mfma16x16x32bf(w_, a_, c);
    else c = mfma16x16x64(w_, a_, c);
  };
  // the epilogue's operands for this lane's outputs (row 4 q + rsub, column n0 + 4 r + lane / 16) go out
  // ahead of the K loop where the 3 R XG registers they hold through it cost no occupancy
  constexpr bool PRE = R * XG <= 2;
  Epi1Ops<EPI> ops[PRE ? R : 1][PRE ? XG : 1];
  if constexpr (PRE) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int q = 0; q < XG; ++q)
        ops[r][q] = Epi1Ops<EPI>(e, min<int64_t>(4 * q + rsub, M - 1), min<int64_t>(n0 + 4 * r + (lane >> 4), N - 1));
  }
  Acc4 acc[R][XG];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int q = 0; q < XG; ++q) acc[r][q] = Acc4{};
  for (int64_t kc = kbeg; kc < kend; kc += KS * 256) {
    i32x4 wv[R][KS], xv[XG][KS];
#pragma unroll
    for (int st = 0; st < KS; ++st) {
      const int64_t k = kc + st * 256 + koff;
      const bool in = k < kend;
      if (kc + st * 256 < kend) {         // uniform: steps wholly past the range issue no loads
#pragma unroll
        for (int q = 0; q < XG; ++q) xv[q][st] = buf_load16(ra, in && arow[q] != OOB ? arow[q] + (uint32_t)k : OOB);
#pragma unroll
        for (int r = 0; r < R; ++r) wv[r][st] = buf_load16(rw, in && wrow[r] != OOB ? wrow[r] + (uint32_t)k : OOB);
      } else {
#pragma unroll
        for (int q = 0; q < XG; ++q) xv[q][st] = i32x4{0, 0, 0, 0};
#pragma unroll
        for (int r = 0; r < R; ++r) wv[r][st] = i32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int st = 0; st < KS; ++st)
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int q = 0; q < XG; ++q) mfma(wv[r][st], xv[q][st], acc[r][q]);
  }
  const int j = lane & 3;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int q = 0; q < XG; ++q) {
      const Acc4& c = acc[r][q];
      T v = j == 0 ? c[0] : j == 1 ? c[1] : j == 2 ? c[2] : c[3];
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      red[wave][r][q][lane] = v;
    }
  __syncthreads();
  if (wave != 0 || j != 0) return;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int q = 0; q < XG; ++q) {
      T v = red[0][r][q][lane];
#pragma unroll
      for (int u = 1; u < W; ++u) v += red[u][r][q][lane];
      const int64_t m = 4 * q + rsub;
      const int64_t n = n0 + 4 * r + (lane >> 4);
      if (m < M && n < N) {
        if constexpr (PRE) epilogue1<EPI>(e, m, n, v, ops[r][q]);
        else epilogue1<EPI>(e, m, n, v, Epi1Ops<EPI>(e, m, n));
      }
    }
}

// ------------------------------------------------------------------------------ one row, quantize in the launch
// The W8A8 linear of a single activation row (decode, M = 1) as one launch: every workgroup quantizes the
// whole row itself (max |x|, scale, quant_pack: the arithmetic of the quantize kernels, so the int8 row and
// its scale are bit for bit theirs), with no flag or wait between workgroups, then streams its weight rows
// against it as mm_gemv_kernel does. Workgroup of 8 waves:
//   - each wave issues its first D - 1 weight rounds (4 KB of one row per round, 16 bytes per lane per 1 KB
//     step), so the weight stream is in flight while the row is reduced;
//   - the 512 threads load the row (16-byte loads, zeros past its end), agree on its max through LDS, and
//     write its int8 values to LDS (zeros up to the end of the last 4 KB round);
//   - each wave takes C consecutive output columns, streaming their weight rows round by round through a
//     ring of D register sets that runs across its columns; a step's activation is one conflict-free
//     ds_read_b128 (lane l: bytes 16 l .. +15 of the KB), and one 16x16x64 MFMA puts the step's 16 K
//     segments on the diagonal, as in mm_gemv_kernel.
// Every workgroup quantizes the K elements again (about 8 vector instructions each), so C grows with N to
// keep the number of workgroups near 1.75 per CU. Rows whose scale is NaN quantize their zero padding to
// -127 rather than 0; their outputs are NaN either way.
template <int DT, int C, int D, int JM, int EPI>
__global__ __launch_bounds__(512) void mm_rowq_kernel(const void* __restrict__ x, int64_t kx,
                                                      const int8_t* __restrict__ w, int64_t ldw, int64_t N, int64_t K,
                                                      float* __restrict__ sx_out, EpiArgs e) {
  static_assert(epi_dq(EPI), "the dequantizing epilogues");
  constexpr int W = 8, KS = 4;
  using V = Vec16<DT>;
  constexpr int ESZ = DT == XDNA_F32 ? 4 : 2;
  constexpr int LPG = 16 / V::N;          // 16-byte loads per group of 16 elements
  extern __shared__ __attribute__((aligned(16))) int8_t xq[];   // the int8 row, rounds * 4 KB
  __shared__ int red[W];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int rounds = (int)((K + KS * 1024 - 1) / (KS * 1024));
  const int items = C * rounds;           // (column, round) pairs of this wave
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)(N * ldw));
  const int64_t ncol0 = ((int64_t)blockIdx.x * W + wave) * C;
  i32x4 ring[D][KS];
  int ic = 0, ir = 0;                     // the next item to issue: column ic, round ir
  auto issue = [&](i32x4 (&dst)[KS]) {
    const int64_t n = ncol0 + ic;
    const bool live = ic < C && n < N;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int64_t k = (int64_t)ir * (KS * 1024) + s * 1024 + 16 * lane;
      dst[s] = buf_load16(rw, live && k < K ? (uint32_t)(n * ldw + k) : OOB);
    }
    if (++ir == rounds) {
      ir = 0;
      ++ic;
    }
  };
  static_for<0, D - 1>([&](auto d) { issue(ring[decltype(d)::value]); });

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)(kx * ESZ));
  V v[JM][LPG];
#pragma unroll
  for (int j = 0; j < JM; ++j) {
    const uint32_t g = (uint32_t)(t + j * W * 64);
#pragma unroll
    for (int l = 0; l < LPG; ++l) v[j][l].raw = buf_load_u4(rx, g * (16 * ESZ) + l * 16);
  }
  AbsMaxBits<DT> am;
#pragma unroll
  for (int j = 0; j < JM; ++j)
#pragma unroll
    for (int l = 0; l < LPG; ++l) am.add(v[j][l]);
  const int wmax = wave_max_i(am.lane_bits());
  if (lane == 0) red[wave] = wmax;
  __syncthreads();
  int mb = red[0];
#pragma unroll
  for (int u = 1; u < W; ++u) mb = max(mb, red[u]);
  const float sc = scale_from_amax(bits_to_abs<DT>(mb));
  const float rc = 1.0f / sc;
  if (sx_out && blockIdx.x == 0 && t == 0) *sx_out = sc;
  const int ngr = rounds * KS * 64;       // 16-byte groups of the LDS row
#pragma unroll
  for (int j = 0; j < JM; ++j) {
    const int g = t + j * W * 64;
    if (g < ngr) {
      float f[16];
#pragma unroll
      for (int l = 0; l < LPG; ++l)
#pragma unroll
        for (int q = 0; q < V::N; ++q) f[l * V::N + q] = v[j][l].get(q);
      uint32_t b[4];
      quant_pack<16>(f, sc, rc, b);
      *reinterpret_cast<u32x4*>(xq + g * 16) = u32x4{b[0], b[1], b[2], b[3]};
    }
  }
  __syncthreads();                        // the last barrier: waves past N run on with zero loads

  Epi1Ops<EPI> ops;
  ops.sx = sc;
  auto column_ops = [&](int64_t n) {
    const int64_t nc = min(n, N - 1);
    ops.sw = e.sw[nc];
    ops.b = e.bias ? e.bias[nc] : 0.0f;
  };
  column_ops(ncol0);
  int cc = 0, rr = 0;                     // the item being consumed
  i32x4 acc0 = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
  for (int i0 = 0; i0 < items; i0 += D) {
    static_for<0, D>([&](auto dc) {
      constexpr int d = decltype(dc)::value;
      if (i0 + d < items) {
        issue(ring[(d + D - 1) % D]);     // the set item i0 + d - 1 used
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const i32x4 xv = *reinterpret_cast<const i32x4*>(xq + rr * (KS * 1024) + s * 1024 + 16 * lane);
          if (s & 1) acc1 = mfma16x16x64(ring[d][s], xv, acc1);
          else acc0 = mfma16x16x64(ring[d][s], xv, acc0);
        }
        if (++rr == rounds) {
          // lane l holds D[4 (l / 16) + j][l % 16] in element j: the diagonal is in lanes with
          // (l % 16) / 4 == l / 16, element l % 4
          const i32x4 acc = acc0 + acc1;
          const int i = lane & 15, j = lane & 3;
          const int32_t dv = j == 0 ? acc[0] : j == 1 ? acc[1] : j == 2 ? acc[2] : acc[3];
          int32_t sum = (i >> 2) == (lane >> 4) ? dv : 0;
#pragma unroll
          for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
          const int64_t n = ncol0 + cc;
          if (lane == 0 && n < N) epilogue1<EPI>(e, 0, n, sum, ops);
          rr = 0;
          ++cc;
          acc0 = i32x4{0, 0, 0, 0};
          acc1 = i32x4{0, 0, 0, 0};
          if (cc < C) column_ops(ncol0 + cc);
        }
      }
    });
  }
}

// ------------------------------------------------------------------------------ dispatch
struct TileCfg {
  int bm, bn, waves, kg;   // kg: K groups of `waves` waves each
};

// Tile ids (XDNA_TILE_* in the header): the tile engine's shapes, then the small-M kernel by waves.
constexpr int T_AUTO = 0, T_256x256W8 = 1, T_256x256W4 = 2, T_256x128 = 3, T_128x256 = 4, T_128x128 = 5,
              T_64x64 = 6, T_SMALL1 = 7, T_SMALL2 = 8, T_SMALL4 = 9, T_SMALL8 = 10, T_SMALL16 = 11,
              T_192x256 = 12, T_256x192 = 13, T_64x32 = 14, T_32x64 = 15, T_32x32 = 16, T_GEMV4 = 17,
              T_GEMV2 = 18, T_GEMV8 = 19, T_SEG4R2 = 20, T_SEG4R4 = 21, T_64x64K2 = 22, T_64x64K4 = 23,
              T_32x64K4 = 24, T_32x32K4 = 25, T_128x128K2 = 26, T_128x256W8 = 27, T_256x128W8 = 28,
              T_256x256PP = 29, T_256x64 = 30, T_DIRECT = 31, T_COUNT = 32;

static_assert(T_SMALL2 == T_SMALL1 + 1 && T_SMALL4 == T_SMALL1 + 2 && T_SMALL8 == T_SMALL1 + 3 &&
                  T_SMALL16 == T_SMALL1 + 4,
              "small-M ids count waves as powers of two");
inline bool is_small(int t) { return t >= T_SMALL1 && t <= T_SMALL16; }
inline int small_waves(int t) { return 1 << (t - T_SMALL1); }
inline bool is_gemv(int t) { return t >= T_GEMV4 && t <= T_GEMV8; }
inline int gemv_waves(int t) { return t == T_GEMV2 ? 2 : t == T_GEMV8 ? 8 : 4; }
inline bool is_seg4(int t) { return t == T_SEG4R2 || t == T_SEG4R4; }
// T_DIRECT: the conv kernels with register operands (conv16_kernel for c_pad 16, convd_kernel for c_pad 32,
// 48, 64), for co a multiple of 32 up to 128; a conv of K = 9 c_pad, N = co they take
inline bool direct_ok(int64_t n, int64_t k) {
  const int64_t c_pad = k / 9;
  return k % 9 == 0 && (c_pad == 16 || c_pad == 32 || c_pad == 48 || c_pad == 64) && n % 32 == 0 && n <= 128;
}

inline TileCfg tile_cfg(int t) {
  switch (t) {
    case T_256x256W8: return {256, 256, 8, 1};
    case T_256x256W4: return {256, 256, 4, 1};
    case T_256x128: return {256, 128, 4, 1};
    case T_128x256: return {128, 256, 4, 1};
    case T_128x128: return {128, 128, 4, 1};
    case T_192x256: return {192, 256, 4, 1};
    case T_256x192: return {256, 192, 4, 1};
    case T_64x32: return {64, 32, 2, 1};
    case T_32x64: return {32, 64, 2, 1};
    case T_32x32: return {32, 32, 1, 1};
    case T_64x64K2: return {64, 64, 4, 2};
    case T_64x64K4: return {64, 64, 4, 4};
    case T_32x64K4: return {32, 64, 2, 4};
    case T_32x32K4: return {32, 32, 1, 4};
    case T_128x128K2: return {128, 128, 4, 2};
    case T_128x256W8: return {128, 256, 8, 1};
    case T_256x128W8: return {256, 128, 8, 1};
    case T_256x256PP: return {256, 256, 8, 1};
    case T_256x64: return {256, 64, 4, 1};
    default: return {64, 64, 4, 1};
  }
}

// Per-shape tile choices registered by the host (a tuned table, or a sweep forcing each tile in
// turn), keyed by (kind, m, n, k) in the caller's units; consulted before the rule below.
struct TileKey {
  int kind;
  int64_t m, n, k;
  bool operator==(const TileKey& o) const { return kind == o.kind && m == o.m && n == o.n && k == o.k; }
};
struct TileKeyHash {
  size_t operator()(const TileKey& t) const {
    uint64_t h = (uint64_t)t.kind * 0x9E3779B97F4A7C15ull;
    h ^= (uint64_t)t.m + 0x9E3779B97F4A7C15ull + (h << 6) + (h >> 2);
    h ^= (uint64_t)t.n + 0x9E3779B97F4A7C15ull + (h << 6) + (h >> 2);
    h ^= (uint64_t)t.k + 0x9E3779B97F4A7C15ull + (h << 6) + (h >> 2);
    return (size_t)h;
  }
};
std::mutex g_tile_mu;
std::unordered_map<TileKey, int, TileKeyHash> g_tiles;
std::atomic<int> g_tile_count{0};

int tile_lookup(int kind, int64_t m, int64_t n, int64_t k) {
  if (g_tile_count.load(std::memory_order_acquire) == 0) return T_AUTO;
  std::lock_guard<std::mutex> lock(g_tile_mu);
  const auto it = g_tiles.find(TileKey{kind, m, n, k});
  return it == g_tiles.end() ? T_AUTO : it->second;
}

// The built-in rule, from back-to-back timed sweeps of every tile shape over the BASELINE GEMM and
// conv shapes on MI355X (t128 / t256: tiles of that size the problem needs; kbytes: K in bytes):
//   * M == 1: the one-row kernel, 4 waves (one output column each) per workgroup;
//   * 2 <= M <= 8 with K of at least 2 KB: the few-row kernel, 8 output columns per workgroup;
//   * M <= 64 (decode): the small-M kernel, 2 waves per workgroup, 4 once K exceeds 8 KB;
//   * 64 x 64 for N <= 64; for N <= 128 no 256-wide tile (half of it would be idle);
//   * 256 x 256 with 8 waves (one workgroup per CU) from 1.5 rounds of such tiles, or from three
//     quarters of a round for deep K (>= 4096 bytes), where its lower LDS traffic per MAC outweighs
//     the idle CUs;
//   * otherwise, once 128 x 128 tiles fill three quarters of the CUs: 128 x 256 (four waves) for deep K
//     when there are at least half a round of 256-wide tiles, else 128 x 128 (three workgroups per CU);
//   * smaller problems with deep K (at least 2 KB): tiles whose workgroups split K between wave groups,
//     32 x 32 x 4 groups below an eighth of a round of 64 x 64 tiles, 32 x 64 x 4 groups up to half a
//     round, 64 x 64 x 2 groups up to a round;
//   * 64 x 64 otherwise.
// A shape the tuned table lists uses the table's tile instead.
int rule_tile(int64_t M, int64_t N, int64_t kbytes, bool small_ok) {
  if (small_ok && M == 1) return T_GEMV4;
  if (small_ok && M <= 8 && kbytes >= 2048) return T_SEG4R2;
  if (small_ok && M <= 64) return (kbytes + 63) / 64 > 128 ? T_SMALL4 : T_SMALL2;
  const int64_t cus = device_cus();
  // narrow outputs with rows for at least two rounds of 256 x 64 tiles (the VGG-16 224 x 224 convs): a
  // quarter of the 64 x 64 tiles, each paying its fixed prologue / epilogue cost once for four times the work
  if (N <= 64 && ((M + 255) / 256) * ((N + 63) / 64) >= 2 * cus) return T_256x64;
  if (M <= 64 || N <= 64) return T_64x64;
  const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256);
  const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
  const bool deep = kbytes >= 4096;
  if (N > 128 && (2 * t256 >= 3 * cus || (deep && 4 * t256 >= 3 * cus))) return T_256x256W8;
  if (4 * t128 >= 3 * cus) return (N > 128 && deep && 2 * t256 >= cus) ? T_128x256 : T_128x128;
  if (kbytes >= 2048) {
    const int64_t t64 = ((M + 63) / 64) * ((N + 63) / 64);
    if (8 * t64 < cus) return T_32x32K4;
    if (2 * t64 <= cus) return T_32x64K4;
    if (t64 <= cus) return T_64x64K2;
  }
  return T_64x64;
}

// kind / (m, n, k): the table key; kbytes: K as the engine counts it (bytes of an operand row).
int choose_tile(int kind, int64_t m, int64_t n, int64_t k, int64_t kbytes) {
  int t = tile_lookup(kind, m, n, k);
  if (t == T_DIRECT && !(kind == XDNA_KIND_CONV && direct_ok(n, k))) t = T_AUTO;   // not a shape it takes
  if (t != T_AUTO) return t;
  if (kind == XDNA_KIND_CONV && direct_ok(n, k)) return T_DIRECT;
  return rule_tile(m, n, kbytes, kind != XDNA_KIND_CONV);
}

// Buffer resources address at most 2 GB; larger operands are processed in row chunks.
constexpr int64_t MAX_BUF = 0x40000000;   // 1 GB per resource

// Output pointer of row block m0 / column block n0 of an epilogue.
inline EpiArgs shift_epi(const EpiArgs& e, int out_bytes, int64_t m0, int64_t n0) {
  EpiArgs r = e;
  if (r.out) r.out = reinterpret_cast<char*>(r.out) + (m0 * e.ldo + n0) * out_bytes;
  if (r.sx) r.sx += m0;
  if (r.sw) r.sw += n0;
  if (r.bias) r.bias += n0;
  return r;
}

// Bytes of one output element: int32 sums and float32 results 4, bf16 / fp16 2, requantized int8 1.
template <int EPI>
constexpr int out_bytes() {
  return (EPI == EPI_I32 || EPI == EPI_DQ_F32 || EPI == EPI_BF_F32) ? 4
         : (EPI == EPI_DQ_BF16 || EPI == EPI_DQ_F16 || EPI == EPI_BF_BF16 || EPI == EPI_BF_F16 ||
            EPI == EPI_BF_SILU) ? 2     // EPI_BF_SILU: per output row; its calls make no column chunks
                                                                                               : 1;
}

// The cross-workgroup K split of the int8 GEMM tiles up to 64 x 64 (the kernel's CAN_SPLIT). A launch
// whose tiles would leave more than half of the CUs idle gives each tile up to CUs / tiles workgroups
// along K (at most 16, each with at least 16 slices of 64 per K group: measured, shorter splits cost
// more in partial sums than they gain, e.g. 128 x 1024 x 3072 in 32 x 32 tiles with 4 K groups takes
// 5.7 us unsplit and 6.3 us in two splits of 6 slices per group); 1: no split. Its workspace is
// WS_CNT_BYTES of arrival counters (a launch uses tiles x waves of them) and then the partial sums,
// tiles x bm x bn int32 per split.
constexpr int64_t WS_CNT_BYTES = XDNA_GEMM_WS_COUNTER_BYTES;

int ksplit_for(const TileCfg& t, int64_t tiles, int64_t K) {
  const int64_t cus = device_cus();
  if (t.bm * t.bn > 64 * 64 || 2 * tiles > cus || tiles * t.waves * 4 > WS_CNT_BYTES) return 1;
  const int64_t nk = (K + 63) / 64;
  const int64_t ks = std::min<int64_t>({cus / tiles, nk / (16 * t.kg), 16});
  if (ks < 2) return 1;
  const int64_t per = (nk + ks - 1) / ks;
  return (int)((nk + per - 1) / per);     // no split without slices
}

int64_t split_ws_bytes(const TileCfg& t, int64_t tiles, int ks) {
  return ks > 1 ? WS_CNT_BYTES + tiles * t.bm * t.bn * 4 * ks : 0;
}

template <int CONVM, int EPI>
int launch_tiles_once(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K,
                      ConvGeom cg, const EpiArgs& e_in, int tile, hipStream_t st) {
  if (e_in.dq_out && tile == T_256x192) tile = T_256x256W8;   // no fused dequantize in that tile (same results)
  const TileCfg t = tile_cfg(tile);
  const int64_t tiles = ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
  if (tiles >= (1ll << 31)) {
    set_error("launch_mm: too many tiles");
    return XDNA_EINVAL;
  }
  dim3 grid((unsigned)tiles, 1, 1);
  EpiArgs e = e_in;
  e.ksplit = 1;
  if constexpr (CONVM == 0 && (EPI == EPI_I32 || epi_dq(EPI))) {
    // split only where the caller's workspace holds it (else the same sums in one workgroup per tile)
    const int ks = e.ws ? ksplit_for(t, tiles, K) : 1;
    if (ks > 1 && split_ws_bytes(t, tiles, ks) <= e.ws_bytes) {
      e.ksplit = ks;
      e.cnt = static_cast<uint32_t*>(e.ws);
      e.part = reinterpret_cast<int32_t*>(static_cast<char*>(e.ws) + WS_CNT_BYTES);
      grid.y = (unsigned)ks;
    }
  }
  const bool kfull = K % 64 == 0;
  // LDS stages per tile shape, from a measured sweep of 3 / 4 / 5 (and 4 / 8 / 12 for 64 x 64): 3 for
  // the large tiles (96 KB at 256 x 256; 48 KB at 128 x 128, three workgroups per CU), 4 for 64 x 64
#define XDNA_TILE_WK(BM_, BN_, WM_, WN_, S_, KG_)                                                             \
  if (kfull) mm_tile_kernel<BM_, BN_, WM_, WN_, S_, CONVM, EPI, true, KG_><<<grid, WM_ * WN_ * KG_ * 64, 0, st>>>(a, lda, w, ldw, M, N, K, cg, e); \
  else mm_tile_kernel<BM_, BN_, WM_, WN_, S_, CONVM, EPI, false, KG_><<<grid, WM_ * WN_ * KG_ * 64, 0, st>>>(a, lda, w, ldw, M, N, K, cg, e);
#define XDNA_TILE_W(BM_, BN_, WM_, WN_, S_) XDNA_TILE_WK(BM_, BN_, WM_, WN_, S_, 1)
#define XDNA_TILE(BM_, BN_, S_) XDNA_TILE_W(BM_, BN_, 2, 2, S_)
  if constexpr (CONVM == 3) {
    // the haloed conv: the 8-wave 256 x 256 tile (3 stages) and, for tails, the 8-wave 128 x 256 (4 stages)
    if (tile == T_256x256W8) {
      XDNA_TILE_W(256, 256, 2, 4, 3)
    } else {
      XDNA_TILE_W(128, 256, 2, 4, 4)
    }
  } else if (tile == T_256x256PP) {
    // the ping-pong schedule: 4 stages (S - 2 = 2 slices between a DMA and its use)
    if (kfull) mm_tile_kernel<256, 256, 2, 4, 4, CONVM, EPI, true, 1, true><<<grid, 512, 0, st>>>(a, lda, w, ldw, M, N, K, cg, e);
    else mm_tile_kernel<256, 256, 2, 4, 4, CONVM, EPI, false, 1, true><<<grid, 512, 0, st>>>(a, lda, w, ldw, M, N, K, cg, e);
  } else if (t.kg > 1) {
    // K groups (in-workgroup split-K) for tiles with few tiles and deep K
    if (t.bm == 128) {
      XDNA_TILE_WK(128, 128, 2, 2, 4, 2)
    } else if (t.bm == 64 && t.kg == 2) {
      XDNA_TILE_WK(64, 64, 2, 2, 4, 2)
    } else if (t.bm == 64) {
      XDNA_TILE_WK(64, 64, 2, 2, 4, 4)
    } else if (t.bn == 64) {
      XDNA_TILE_WK(32, 64, 1, 2, 4, 4)
    } else {
      XDNA_TILE_WK(32, 32, 1, 1, 4, 4)
    }
  } else if (t.waves == 8 && t.bm == 128) {
    XDNA_TILE_W(128, 256, 2, 4, 4)
  } else if (t.waves == 8 && t.bn == 128) {
    XDNA_TILE_W(256, 128, 4, 2, 4)
  } else if (t.bm == 256 && t.bn == 64) {
    XDNA_TILE_W(256, 64, 4, 1, 4)
  } else if (t.bm == 256 && t.bn == 256 && t.waves == 8) {
    XDNA_TILE_W(256, 256, 2, 4, 3)
  } else if (t.bm == 256 && t.bn == 256) {
    XDNA_TILE(256, 256, 4)
  } else if (t.bm == 192) {
    XDNA_TILE(192, 256, 4)
  } else if (t.bn == 192) {
    XDNA_TILE(256, 192, 4)
  } else if (t.bm == 256) {
    XDNA_TILE(256, 128, 4)
  } else if (t.bn == 256) {
    XDNA_TILE(128, 256, 4)
  } else if (t.bm == 128) {
    XDNA_TILE(128, 128, 3)
  } else if (t.bn == 32 && t.bm == 64) {
    XDNA_TILE_W(64, 32, 2, 1, 4)
  } else if (t.bm == 32 && t.bn == 64) {
    XDNA_TILE_W(32, 64, 1, 2, 4)
  } else if (t.bm == 32) {
    XDNA_TILE_W(32, 32, 1, 1, 4)
  } else {
    XDNA_TILE(64, 64, 4)
  }
#undef XDNA_TILE
#undef XDNA_TILE_W
#undef XDNA_TILE_WK
  return launch_status("mm_tile");
}

// Tiles whose LDS (or registers) allow one workgroup per CU run in rounds of one tile per CU. When the
// last round would leave more than half of the CUs idle, the whole rounds run with the chosen tile and
// the rows left over as a second launch with a smaller tile: e.g. C4's conv (384 tiles of 256 x 256 on
// 256 CUs) as 256 of them plus 256 tiles of 128 x 256 over the last third of the rows. Row r of the tail
// launch is row m1 + r of the problem; for the conv that is a pixel offset (ConvGeom::m0) into the same
// images.
struct TilePlan {
  int head;       // tile of rows [0, m1) (all rows when m1 == 0)
  int64_t m1;     // first row of the tail launch; 0: one launch
  int tail;       // tile of rows [m1, M) when m1 > 0
};

// kind: the table's kind of the launch; kbytes: K as the engine counts it (bytes of an operand row);
// ktab: K as the table keys it (bf16 elements for the bf16 GEMM).
TilePlan plan_tiles(int kind, int64_t M, int64_t N, int64_t kbytes, int64_t ktab, int tile) {
  const TilePlan one{tile, 0, T_AUTO};
  if (is_small(tile) || is_gemv(tile) || is_seg4(tile) || tile == T_DIRECT) return one;
  const TileCfg t = tile_cfg(tile);
  const bool one_per_cu = t.kg == 1 && t.bm >= 128 && t.bn >= 128 && !(t.bm == 128 && t.bn == 128);
  if (!one_per_cu) return one;
  const int64_t cus = device_cus();
  const int64_t tm = (M + t.bm - 1) / t.bm, tn = (N + t.bn - 1) / t.bn;
  const int64_t rounds = (tm * tn) / cus, rem = (tm * tn) % cus;
  const int64_t tm_head = rounds * cus / tn;
  if (!(rounds >= 1 && rem > 0 && 2 * rem <= cus && tm_head >= 1 && tm_head < tm)) return one;
  const int64_t m1 = tm_head * t.bm;
  // the tail's tile: the table's entry for the tail's own shape if it lists an engine tile; else after
  // 256 x 256 tiles the 8-wave 128 x 256 tile, else the rule. C4 (1 x 256 x 1536 x 64) measured 79.8 us
  // unsplit, 72.7 us with a 128 x 128 tail (the rule's) and 69.4 us with the 128 x 256 one.
  int tail = tile_lookup(kind, M - m1, N, ktab);
  if (is_small(tail) || is_gemv(tail) || is_seg4(tail) || tail == T_DIRECT) tail = T_AUTO;
  if (tail == T_AUTO)
    tail = (tile == T_256x256W8 || tile == T_256x256PP) ? T_128x256W8 : rule_tile(M - m1, N, kbytes, false);
  // only when the leftover rows fit one round of the tail's tiles (8192 x 3072 in 256 x 256 tiles leaves
  // 2816 rows, 264 tiles of 128 x 256: measured slower split than not)
  const TileCfg tt = tile_cfg(tail);
  if (((M - m1 + tt.bm - 1) / tt.bm) * ((N + tt.bn - 1) / tt.bn) > cus) return one;
  return TilePlan{tile, m1, tail};
}

// The conv's loader for a tile: 3 (haloed input tile) for the 8-wave 256 x 256 and 128 x 256 tiles when a
// tile is whole image rows (or a segment of one row) inside one image and its halo fits a buffer; else 1
// (one tap per K slice: C_pad a multiple of the tile's K groups' 64-channel slices), else 2.
int conv_mode(int tile, int64_t h, int64_t w, int64_t c_pad) {
  const TileCfg t = tile_cfg(tile);
  const int s = tile == T_256x256W8 ? 3 : tile == T_128x256W8 ? 4 : 0;
  if (s != 0 && c_pad % 64 == 0 && (w <= t.bm ? (t.bm % w == 0 && h % (t.bm / w) == 0) : (w % t.bm == 0))) {
    const int64_t wt = std::min<int64_t>(w, t.bm);
    if ((t.bm / wt + 2) * (wt + 2) <= conv_halo_max(t.bn, s, t.waves)) return 3;
  }
  return c_pad % (64 * t.kg) == 0 ? 1 : 2;
}

template <int CONVM, int EPI>
int launch_tiles(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K,
                 ConvGeom cg, const EpiArgs& e, int tile, hipStream_t st) {
  const int kind = CONVM != 0 ? XDNA_KIND_CONV : epi_bf(EPI) ? XDNA_KIND_BF16 : XDNA_KIND_I8;
  const TilePlan p = plan_tiles(kind, M, N, K, epi_bf(EPI) ? K / 2 : K, tile);
  if (p.m1 == 0) return launch_tiles_once<CONVM, EPI>(a, lda, w, ldw, M, N, K, cg, e, tile, st);
  const int64_t m1 = p.m1;
  int rc = launch_tiles_once<CONVM, EPI>(a, lda, w, ldw, m1, N, K, cg, e, tile, st);
  if (rc) return rc;
  ConvGeom ct = cg;
  const int8_t* at = a;
  if constexpr (CONVM != 0) ct.m0 += m1;
  else at += m1 * lda;
  // the conv's NCHW dequantized output is addressed by the pixel offset in its geometry (ct.m0)
  const EpiArgs et = (CONVM != 0 && e.dq_out) ? e : shift_epi(e, out_bytes<EPI>(), m1, 0);
  // the tail's tile has its own conv loader (it may split K over groups, or not take the halo)
  if constexpr (CONVM != 0) {
    switch (conv_mode(p.tail, cg.h, cg.w, cg.c_pad)) {
      case 3: return launch_tiles_once<3, EPI>(at, lda, w, ldw, M - m1, N, K, ct, et, p.tail, st);
      case 1: return launch_tiles_once<1, EPI>(at, lda, w, ldw, M - m1, N, K, ct, et, p.tail, st);
      default: return launch_tiles_once<2, EPI>(at, lda, w, ldw, M - m1, N, K, ct, et, p.tail, st);
    }
  }
  return launch_tiles_once<CONVM, EPI>(at, lda, w, ldw, M - m1, N, K, ct, et, p.tail, st);
}

template <int EPI>
int launch_gemm(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K,
                const EpiArgs& e, int tile, hipStream_t st) {
  // the one-row kernel takes one row; the small-M kernel addresses the whole activation with one buffer
  // resource, 16 rows per grid row
  if (is_gemv(tile) && M != 1) tile = rule_tile(M, N, K, M > 1);
  if (is_seg4(tile) && M > 16) tile = rule_tile(M, N, K, true);
  // the one-row and few-row kernels write one column per lane: the fused SiLU needs a column's partner
  if (EPI == EPI_BF_SILU && (is_gemv(tile) || is_seg4(tile))) tile = T_SMALL2;
  if (is_small(tile) && (M * lda > MAX_BUF || (M + 15) / 16 >= 65536)) tile = rule_tile(M, N, K, false);
  if constexpr (EPI != EPI_BF_SILU) {
  if (is_seg4(tile)) {
    // four rows per segment group; the workgroup's 4 waves split K into multiples of 256 bytes
    constexpr int W = 4;
    const int64_t steps = (K + 255) / 256;
    const int64_t kper = ((steps + W - 1) / W) * 256;
    const int R = tile == T_SEG4R2 ? 2 : 4;
    const int64_t nrows = std::max<int64_t>(4 * R, (MAX_BUF / ldw) / (4 * R) * (4 * R));
    for (int64_t n0 = 0; n0 < N; n0 += nrows) {
      const int64_t nc = std::min(nrows, N - n0);
      dim3 grid((unsigned)((nc + 4 * R - 1) / (4 * R)), 1, 1);
      const EpiArgs en = shift_epi(e, out_bytes<EPI>(), 0, n0);
      const int8_t* wn = w + n0 * ldw;
#define XDNA_SEG4(R_, XG_) mm_seg4_kernel<W, R_, XG_, EPI><<<grid, W * 64, 0, st>>>(a, lda, wn, ldw, M, nc, K, kper, en)
      if (R == 2) {
        if (M <= 4) XDNA_SEG4(2, 1);
        else if (M <= 8) XDNA_SEG4(2, 2);
        else XDNA_SEG4(2, 4);
      } else {
        if (M <= 4) XDNA_SEG4(4, 1);
        else if (M <= 8) XDNA_SEG4(4, 2);
        else XDNA_SEG4(4, 4);
      }
#undef XDNA_SEG4
      const int rc = launch_status("mm_seg4");
      if (rc) return rc;
    }
    return XDNA_OK;
  }
  if (is_gemv(tile)) {
    // one wave per output column, the weight in row chunks one buffer resource can address; K in
    // rounds of 4 KB (K <= 4 KB) or 16 KB
    const int64_t nrows = std::max<int64_t>(1, MAX_BUF / ldw);
    const int waves = gemv_waves(tile);
    for (int64_t n0 = 0; n0 < N; n0 += nrows) {
      const int64_t nc = std::min(nrows, N - n0);
      dim3 grid((unsigned)((nc + waves - 1) / waves), 1, 1);
      const EpiArgs en = shift_epi(e, out_bytes<EPI>(), 0, n0);
      const int8_t* wn = w + n0 * ldw;
#define XDNA_GEMV(W_)                                                                                      \
  if (K <= 4096) mm_gemv_kernel<W_, 4, EPI><<<grid, W_ * 64, 0, st>>>(a, wn, ldw, nc, K, en);              \
  else mm_gemv_kernel<W_, 16, EPI><<<grid, W_ * 64, 0, st>>>(a, wn, ldw, nc, K, en);
      if (waves == 2) {
        XDNA_GEMV(2)
      } else if (waves == 8) {
        XDNA_GEMV(8)
      } else {
        XDNA_GEMV(4)
      }
#undef XDNA_GEMV
      const int rc = launch_status("mm_gemv");
      if (rc) return rc;
    }
    return XDNA_OK;
  }
  }
  if (is_small(tile)) {
    // weight streaming: the waves of a workgroup split K into multiples of 64 bytes; the weight is
    // processed in row chunks that one buffer resource can address. Waves per workgroup, from a
    // measured sweep of 1 / 2 / 4 / 8 / 16 over the decode shapes: long per-wave streams through the
    // double-buffered loop beat wide workgroups (the rule takes 2, or 4 once K exceeds 8 KB).
    constexpr int U = 8;
    const int64_t steps = (K + 63) / 64;
    const int waves = small_waves(tile);
    const int64_t kper = ((steps + waves - 1) / waves) * 64;
    const int64_t nrows = std::max<int64_t>(16, (MAX_BUF / ldw) / 16 * 16);
    for (int64_t n0 = 0; n0 < N; n0 += nrows) {
      const int64_t nc = std::min(nrows, N - n0);
      dim3 grid((unsigned)((nc + 15) / 16), (unsigned)((M + 15) / 16), 1);
      const EpiArgs en = shift_epi(e, out_bytes<EPI>(), 0, n0);
      if (waves == 16) mm_small_kernel<16, U, EPI><<<grid, 16 * 64, 0, st>>>(a, lda, w + n0 * ldw, ldw, M, nc, K, kper, en);
      else if (waves == 8) mm_small_kernel<8, U, EPI><<<grid, 8 * 64, 0, st>>>(a, lda, w + n0 * ldw, ldw, M, nc, K, kper, en);
      else if (waves == 4) mm_small_kernel<4, U, EPI><<<grid, 4 * 64, 0, st>>>(a, lda, w + n0 * ldw, ldw, M, nc, K, kper, en);
      else if (waves == 2) mm_small_kernel<2, U, EPI><<<grid, 2 * 64, 0, st>>>(a, lda, w + n0 * ldw, ldw, M, nc, K, kper, en);
      else mm_small_kernel<1, U, EPI><<<grid, 64, 0, st>>>(a, lda, w + n0 * ldw, ldw, M, nc, K, kper, en);
      const int rc = launch_status("mm_small");
      if (rc) return rc;
    }
    return XDNA_OK;
  }
  const int64_t mrows = std::max<int64_t>(256, (MAX_BUF / lda) / 256 * 256);
  const int64_t nrows = std::max<int64_t>(256, (MAX_BUF / ldw) / 256 * 256);
  for (int64_t m0 = 0; m0 < M; m0 += mrows) {
    for (int64_t n0 = 0; n0 < N; n0 += nrows) {
      const int64_t mc = std::min(mrows, M - m0), nc = std::min(nrows, N - n0);
      int rc = launch_tiles<0, EPI>(a + m0 * lda, lda, w + n0 * ldw, ldw, mc, nc, K, ConvGeom{},
                                    shift_epi(e, out_bytes<EPI>(), m0, n0), tile, st);
      if (rc) return rc;
    }
  }
  return XDNA_OK;
}

// xdna_linear_row's launches. Columns per wave: 4 (with a 3-deep ring) once that still leaves 1.75 workgroups
// per CU, else 1 (2-deep), from a sweep of 1 / 2 / 4 columns with 2- to 4-deep rings over the C5 decode
// shapes (bf16, rotating weights): 14336 x 4096 12.6 us with 4 columns against 14.6 with 1, 4096 x 14336 and
// 4096 x 4096 13.0 / 6.4 us with 1 against 16.5 / 7.2 with 4. The weight goes in row chunks one buffer
// resource can address, each chunk a launch of its own.
template <int DT, int EPI>
int launch_rowq(const void* x, int64_t kx, const int8_t* w, int64_t ldw, int64_t N, int64_t K, float* sx,
                const EpiArgs& e, hipStream_t st) {
  const int64_t rounds = cdiv(K, 4096);
  const int jm = (int)cdiv(rounds * 256, 512);   // 16-element groups of the row per thread
  const size_t lds = (size_t)rounds * 4096;
  const bool c4 = N >= 32 * (7 * (int64_t)device_cus() / 4);
  const int64_t cols = c4 ? 32 : 8;              // output columns per workgroup
  const int64_t nrows = std::max<int64_t>(cols, (MAX_BUF / ldw) / cols * cols);
  for (int64_t n0 = 0; n0 < N; n0 += nrows) {
    const int64_t nc = std::min(nrows, N - n0);
    dim3 grid((unsigned)cdiv(nc, cols), 1, 1);
    const EpiArgs en = shift_epi(e, out_bytes<EPI>(), 0, n0);
    const int8_t* wn = w + n0 * ldw;
    float* s = n0 == 0 ? sx : nullptr;
#define XDNA_ROWQ(C_, D_, JM_) \
  mm_rowq_kernel<DT, C_, D_, JM_, EPI><<<grid, 512, lds, st>>>(x, kx, wn, ldw, nc, K, s, en)
    if (c4) {
      if (jm <= 1) XDNA_ROWQ(4, 3, 1);
      else if (jm <= 2) XDNA_ROWQ(4, 3, 2);
      else XDNA_ROWQ(4, 3, 4);
    } else {
      if (jm <= 1) XDNA_ROWQ(1, 2, 1);
      else if (jm <= 2) XDNA_ROWQ(1, 2, 2);
      else XDNA_ROWQ(1, 2, 4);
    }
#undef XDNA_ROWQ
    const int rc = launch_status("mm_rowq");
    if (rc) return rc;
  }
  return XDNA_OK;
}

template <int EPI>
int launch_rowq_dt(const void* x, int x_dtype, int64_t kx, const int8_t* w, int64_t ldw, int64_t N, int64_t K,
                   float* sx, const EpiArgs& e, hipStream_t st) {
  if (x_dtype == XDNA_F32) return launch_rowq<XDNA_F32, EPI>(x, kx, w, ldw, N, K, sx, e, st);
  if (x_dtype == XDNA_BF16) return launch_rowq<XDNA_BF16, EPI>(x, kx, w, ldw, N, K, sx, e, st);
  return launch_rowq<XDNA_F16, EPI>(x, kx, w, ldw, N, K, sx, e, st);
}

// Conv of 16-channel inputs (c_pad == 16: RGB or gray images padded to 16 channels, narrow early layers).
// With 16-byte pixels a 32-deep K step of the MFMA is exactly two taps x 16 channels: lanes 0-31 carry
// K chunk 2 s (tap 2 s) and lanes 32-63 chunk 2 s + 1, so a lane's activation operand is one 16-byte load
// of its pixel's tap-shifted neighbour (a zero load outside the image: the padding) and its weight operand
// 16 contiguous bytes of wq. No LDS stages and no barriers: K = 9 taps in 5 steps (chunk 9 is zero). Each
// wave holds the weight fragments of all NB = co / 32 column blocks (loaded once) and takes runs of BPW
// consecutive 32-pixel blocks, a grid stride of runs apart, every activation load of a run issued before
// its first MFMA and the next run's loads issued before this run's MFMAs (one run per wave measured best:
// VGG-16's 8x3x224x224 -> 64 in 14.0 us, 16.3 us with runs of four, 30 us on the tile engine). Lane l
// holds pixel l % 32 and channels 32 j + 8 g + 4 (l / 32) + t (t < 4) of column
// block j; the requantized bytes go through a wave-private LDS tile [32 pixels][co] (pitch co + 16: the
// 4-byte writes of 32 pixels fall on 16 bank groups) and leave as 16-byte stores, consecutive lanes
// covering consecutive 16-byte pieces of the block's 32 * co contiguous output bytes (4-byte stores
// straight from the accumulators split every instruction into partial lines of 16 pixel rows).
// EPI_REQUANT (int8 / uint8 NHWC rows of co bytes) or EPI_CALIB.
template <int EPI, int NB, int BPW>
__global__ __launch_bounds__(256) void conv16_kernel(const int8_t* __restrict__ x, uint32_t M, uint32_t h,
                                                     uint32_t w, const int8_t* __restrict__ wq, EpiArgs e) {
  static_assert(EPI == EPI_REQUANT || EPI == EPI_CALIB, "requantize or calibrate");
  constexpr int PITCH = NB * 32 + 16, CPP = NB * 2;       // tile pitch; 16-byte pieces per pixel
  __shared__ __attribute__((aligned(16))) uint8_t tiles[EPI == EPI_REQUANT ? 4 : 1][EPI == EPI_REQUANT ? 32 * PITCH : 16];
  const int lane = threadIdx.x & 63;
  const int hl = lane >> 5, r32 = lane & 31;
  const uint32_t nwaves = gridDim.x * 4;
  const uint32_t nrun = (M + 32 * BPW - 1) / (32 * BPW);
  const uint32_t hw = h * w;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(wq, NB * 32 * 9 * 16);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, M * 16);
  uint8_t* const tile = tiles[EPI == EPI_REQUANT ? (threadIdx.x >> 6) : 0];
  i32x4 wf[5][NB];
#pragma unroll
  for (int s = 0; s < 5; ++s) {
    const int tap = 2 * s + hl;
#pragma unroll
    for (int j = 0; j < NB; ++j)
      wf[s][j] = __builtin_bit_cast(i32x4, buf_load_u4(rw, tap < 9 ? (uint32_t)(((32 * j + r32) * 9 + tap) * 16) : OOB));
  }
  const int qlo = e.relu ? 0 : -128, qhi = e.relu ? 255 : 127;
  int calib = 0;
  // the 5 activation chunks of each block's pixel for this lane (zeros past M, outside the image, tap 9)
  auto load_run = [&](uint32_t run, i32x4 (&a)[BPW][5]) {
#pragma unroll
    for (int b = 0; b < BPW; ++b) {
      const uint32_t m = (run * BPW + b) * 32 + r32;
      const uint32_t img = m / hw, p = m - img * hw, y = p / w, xx = p - y * w;
#pragma unroll
      for (int s = 0; s < 5; ++s) {
        const int tap = 2 * s + hl;
        const uint32_t yy = y + (uint32_t)(tap / 3) - 1u, xs = xx + (uint32_t)(tap % 3) - 1u;
        const bool ok = m < M && tap < 9 && yy < h && xs < w;
        a[b][s] = __builtin_bit_cast(i32x4, buf_load_u4(rx, ok ? (img * hw + yy * w + xs) * 16u : OOB));
      }
    }
  };
  uint32_t run = (blockIdx.x * 256 + threadIdx.x) >> 6;
  i32x4 a[BPW][5];
  load_run(run, a);
  for (; run < nrun; run += nwaves) {
    i32x4 an[BPW][5];
    load_run(run + nwaves, an);
#pragma unroll
    for (int b = 0; b < BPW; ++b) {
      i32x16 acc[NB];
#pragma unroll
      for (int j = 0; j < NB; ++j) acc[j] = i32x16{};
#pragma unroll
      for (int s = 0; s < 5; ++s)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[j] = mfma32x32x32(wf[s][j], a[b][s], acc[j]);
      const uint32_t m0 = (run * BPW + b) * 32;
      if constexpr (EPI == EPI_CALIB) {
        if (m0 + r32 < M) {
#pragma unroll
          for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) calib = max(calib, e.relu ? max(acc[j][r], 0) : abs(acc[j][r]));
        }
      } else {
        const int rnd = 1 << (e.shift - 1);
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            uint32_t packed = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const int q = min(max((acc[j][4 * g + t] + rnd) >> e.shift, qlo), qhi);   // round half up
              packed |= ((uint32_t)(q & 0xff)) << (8 * t);
            }
            *reinterpret_cast<uint32_t*>(tile + r32 * PITCH + 32 * j + 8 * g + 4 * hl) = packed;
          }
        uint8_t* const out = reinterpret_cast<uint8_t*>(e.out) + (int64_t)m0 * e.ldo;
#pragma unroll
        for (int k = 0; k < CPP / 2; ++k) {
          const int idx = 64 * k + lane, px = idx / CPP, pc = idx - px * CPP;
          const uint4 v = *reinterpret_cast<const uint4*>(tile + px * PITCH + pc * 16);
          if (m0 + px < M) *reinterpret_cast<uint4*>(out + (int64_t)px * e.ldo + pc * 16) = v;
        }
      }
    }
#pragma unroll
    for (int b = 0; b < BPW; ++b)
#pragma unroll
      for (int s = 0; s < 5; ++s) a[b][s] = an[b][s];
  }
  calib_flush<EPI>(e, calib);
}

// Conv of 32-, 48- and 64-channel inputs (c_pad = 16 CP) with the weights resident in LDS and the
// activations loaded straight into registers. Row k of the implicit GEMM is KC = 9 CP chunks of 16 bytes
// (chunk c: tap c / CP, channels 16 (c % CP) ..), so as in conv16_kernel a lane's activation operand of K
// step s is one 16-byte load: chunk 2 s + (l / 32) of its pixel's tap-shifted neighbour. The whole weight
// [co][KC][16] sits in LDS for the workgroup's life (loaded once by its 8 waves; row pitch KC * 16 + 16, so
// the 16 rows one 16-lane phase of a fragment read touches fall on distinct bank groups; the pad chunk is
// zero and serves the odd KC's last step), and only those weight fragments are read from LDS: 16 bytes per
// lane per MFMA, half of what the tile engine's fragment reads of both operands cost for the same MACs.
// Each wave walks 32-pixel blocks a grid stride apart, all NS activation loads of a block issued before
// its first MFMA; epilogue as conv16_kernel (requantize into a wave-private LDS tile, 16-byte stores).
template <int EPI, int NB, int CP>
__global__ __launch_bounds__(512) void convd_kernel(const int8_t* __restrict__ x, uint32_t M, uint32_t h,
                                                    uint32_t w, const int8_t* __restrict__ wq, EpiArgs e) {
  static_assert(EPI == EPI_REQUANT || EPI == EPI_CALIB, "requantize or calibrate");
  constexpr int KC = 9 * CP, NS = (KC + 1) / 2;
  constexpr int WP = KC * 16 + 16;                          // weight row pitch (bytes)
  constexpr int PITCH = NB * 32 + 16, CPP = NB * 2;          // epilogue tile pitch; 16-byte pieces per pixel
  constexpr int TILE = EPI == EPI_REQUANT ? 32 * PITCH : 0;
  __shared__ __attribute__((aligned(16))) uint8_t lds[NB * 32 * WP + 8 * TILE];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hl = lane >> 5, r32 = lane & 31;
  const uint32_t nwaves = gridDim.x * 8;
  const uint32_t nblk = (M + 31) / 32;
  const uint32_t hw = h * w;
  // the weights, chunk i of the flat [co][KC] array to row i / KC, chunk i % KC; the pad chunks zero
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(wq, NB * 32 * KC * 16);
  for (int i = threadIdx.x; i < NB * 32 * (KC + 1); i += 512) {
    const int n = i / (KC + 1), c = i - n * (KC + 1);
    const uint4 v = buf_load_u4(rw, c < KC ? (uint32_t)((n * KC + c) * 16) : OOB);
    *reinterpret_cast<uint4*>(lds + n * WP + c * 16) = v;
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, M * CP * 16);
  uint8_t* const tile = lds + NB * 32 * WP + wave * TILE;
  const int qlo = e.relu ? 0 : -128, qhi = e.relu ? 255 : 127;
  int calib = 0;
  for (uint32_t blk = blockIdx.x * 8 + wave; blk < nblk; blk += nwaves) {
    const uint32_t m = blk * 32 + r32;
    const uint32_t img = m / hw, p = m - img * hw, y = p / w, xx = p - y * w;
    i32x4 a[NS];
    if constexpr (CP % 2 == 0) {
      // even CP: step s covers chunks 2 s, 2 s + 1 of one tap (s / (CP / 2)), so each tap's bounds and
      // offset are worked out once and its CP / 2 loads differ by a constant
      const uint32_t pix = (img * hw + y * w + xx) * (CP * 16) + 16 * hl;
#pragma unroll
      for (int tap = 0; tap < 9; ++tap) {
        const int dy = tap / 3 - 1, dx = tap % 3 - 1;
        const bool ok = m < M && y + (uint32_t)dy < h && xx + (uint32_t)dx < w;
        const uint32_t off = pix + (uint32_t)((dy * (int)w + dx) * CP * 16);
#pragma unroll
        for (int uu = 0; uu < CP / 2; ++uu)
          a[tap * (CP / 2) + uu] = __builtin_bit_cast(i32x4, buf_load_u4(rx, ok ? off + 32u * uu : OOB));
      }
    } else {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int c = 2 * s + hl, tap = c / CP, u = c - tap * CP;
        const uint32_t yy = y + (uint32_t)(tap / 3) - 1u, xs = xx + (uint32_t)(tap % 3) - 1u;
        const bool ok = m < M && c < KC && yy < h && xs < w;
        a[s] = __builtin_bit_cast(i32x4, buf_load_u4(rx, ok ? ((img * hw + yy * w + xs) * CP + u) * 16u : OOB));
      }
    }
    i32x16 acc[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[j] = i32x16{};
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const i32x4 b = *reinterpret_cast<const i32x4*>(lds + (32 * j + r32) * WP + (2 * s + hl) * 16);
        acc[j] = mfma32x32x32(b, a[s], acc[j]);
      }
    const uint32_t m0 = blk * 32;
    if constexpr (EPI == EPI_CALIB) {
      if (m < M) {
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) calib = max(calib, e.relu ? max(acc[j][r], 0) : abs(acc[j][r]));
      }
    } else {
      const int rnd = 1 << (e.shift - 1);
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          uint32_t packed = 0;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int q = min(max((acc[j][4 * g + t] + rnd) >> e.shift, qlo), qhi);   // round half up
            packed |= ((uint32_t)(q & 0xff)) << (8 * t);
          }
          *reinterpret_cast<uint32_t*>(tile + r32 * PITCH + 32 * j + 8 * g + 4 * hl) = packed;
        }
      uint8_t* const out = reinterpret_cast<uint8_t*>(e.out) + (int64_t)m0 * e.ldo;
#pragma unroll
      for (int k = 0; k < CPP / 2; ++k) {
        const int idx = 64 * k + lane, px = idx / CPP, pc = idx - px * CPP;
        const uint4 v = *reinterpret_cast<const uint4*>(tile + px * PITCH + pc * 16);
        if (m0 + px < M) *reinterpret_cast<uint4*>(out + (int64_t)px * e.ldo + pc * 16) = v;
      }
    }
  }
  calib_flush<EPI>(e, calib);
}

// The direct conv's launch (c_pad 32, 48 or 64), XDNA_EUNSUPPORTED for shapes it does not take.
template <int EPI>
int launch_convd(const int8_t* x, int64_t m, int64_t h, int64_t w, int64_t c_pad, const int8_t* wq, int64_t co,
                 const EpiArgs& e, hipStream_t st) {
  if (co % 32 != 0 || co > 128 || m * c_pad >= (int64_t(1) << 31) || m * co >= (int64_t(1) << 31)) return XDNA_EUNSUPPORTED;
  if constexpr (EPI == EPI_REQUANT) {
    if (e.dq_out) return XDNA_EUNSUPPORTED;
  }
  const int64_t wgs = std::min<int64_t>(cdiv(cdiv(m, 32), 8), (int64_t)device_cus() * (co <= 64 ? 2 : 1));
  const dim3 grid((unsigned)wgs);
  const uint32_t um = (uint32_t)m, uh = (uint32_t)h, uw = (uint32_t)w;
#define XDNA_CD(NB_, CP_) convd_kernel<EPI, NB_, CP_><<<grid, 512, 0, st>>>(x, um, uh, uw, wq, e)
#define XDNA_CD_NB(CP_)                      \
  switch (co / 32) {                         \
    case 1: XDNA_CD(1, CP_); break;          \
    case 2: XDNA_CD(2, CP_); break;          \
    case 3: XDNA_CD(3, CP_); break;          \
    default: XDNA_CD(4, CP_);                \
  }
  switch (c_pad) {
    case 32: XDNA_CD_NB(2) break;
    case 48: XDNA_CD_NB(3) break;
    case 64: XDNA_CD_NB(4) break;
    default: return XDNA_EUNSUPPORTED;
  }
#undef XDNA_CD_NB
#undef XDNA_CD
  return launch_status("conv3x3 (resident weights)");
}

// The 16-channel conv's launch, or XDNA_EUNSUPPORTED when the shape is not one it takes (co a multiple
// of 32 up to 128, no fused dequantize, the launch's bytes addressable in 32 bits).
template <int EPI>
int launch_conv16(const int8_t* x, int64_t m, int64_t h, int64_t w, const int8_t* wq, int64_t co, const EpiArgs& e,
                  hipStream_t st) {
  if (co % 32 != 0 || co > 128 || m * 16 >= (int64_t(1) << 31) || m * co >= (int64_t(1) << 31)) return XDNA_EUNSUPPORTED;
  if constexpr (EPI == EPI_REQUANT) {
    if (e.dq_out) return XDNA_EUNSUPPORTED;
  }
  constexpr int BPW = 1;                  // blocks of 32 pixels per run of a wave
  const int64_t waves = std::min<int64_t>(cdiv(m, 32 * BPW), (int64_t)device_cus() * 12);
  const dim3 grid((unsigned)cdiv(waves, 4));
  switch (co / 32) {
    case 1: conv16_kernel<EPI, 1, BPW><<<grid, 256, 0, st>>>(x, (uint32_t)m, (uint32_t)h, (uint32_t)w, wq, e); break;
    case 2: conv16_kernel<EPI, 2, BPW><<<grid, 256, 0, st>>>(x, (uint32_t)m, (uint32_t)h, (uint32_t)w, wq, e); break;
    case 3: conv16_kernel<EPI, 3, BPW><<<grid, 256, 0, st>>>(x, (uint32_t)m, (uint32_t)h, (uint32_t)w, wq, e); break;
    default: conv16_kernel<EPI, 4, BPW><<<grid, 256, 0, st>>>(x, (uint32_t)m, (uint32_t)h, (uint32_t)w, wq, e);
  }
  return launch_status("conv3x3 (16 channels)");
}

template <int EPI>
int launch_conv(const int8_t* x, int64_t nb, int64_t h, int64_t w, int64_t c_pad, const int8_t* wq, int64_t co,
                const EpiArgs& e, hipStream_t st) {
  const int64_t per_img = h * w * c_pad;
  const int64_t imgs = std::max<int64_t>(1, MAX_BUF / per_img);
  if (per_img > MAX_BUF || co * 9 * c_pad > MAX_BUF) {
    set_error("conv3x3: one image or the weight exceeds 1 GB");
    return XDNA_EUNSUPPORTED;
  }
  const int64_t K = 9 * c_pad;
  const int tile = choose_tile(XDNA_KIND_CONV, nb * h * w, co, K, K);
  ConvGeom cg{h, w, c_pad};
  for (int64_t b0 = 0; b0 < nb; b0 += imgs) {
    const int64_t bc = std::min(imgs, nb - b0);
    EpiArgs eb = e;
    if (e.dq_out) eb.px0 = e.px0 + b0 * h * w;   // NCHW output: addressed by global pixel, not by row
    else eb = shift_epi(e, 1, b0 * h * w, 0);
    const int8_t* xb = x + b0 * per_img;
    // the direct kernels (register operands) for the shapes and epilogues they take, else the tile engine
    // with the rule's tile (the fused dequantize, launches past their 32-bit sizes)
    if (tile == T_DIRECT) {
      int rc = XDNA_EUNSUPPORTED;
      if constexpr (EPI == EPI_REQUANT || EPI == EPI_CALIB) {
        rc = c_pad == 16 ? launch_conv16<EPI>(xb, bc * h * w, h, w, wq, co, eb, st)
                         : launch_convd<EPI>(xb, bc * h * w, h, w, c_pad, wq, co, eb, st);
      }
      if (rc != XDNA_EUNSUPPORTED) {
        if (rc) return rc;
        continue;
      }
    }
    const int etile = tile == T_DIRECT ? rule_tile(nb * h * w, co, K, false) : tile;
    // the haloed input tile where the tile allows it; the running tap counters of CONVM 1 step by KG
    // slices of 64 channels
    const int mode = conv_mode(etile, h, w, c_pad);
    int rc = mode == 3   ? launch_tiles<3, EPI>(xb, c_pad, wq, K, bc * h * w, co, K, cg, eb, etile, st)
             : mode == 1 ? launch_tiles<1, EPI>(xb, c_pad, wq, K, bc * h * w, co, K, cg, eb, etile, st)
                         : launch_tiles<2, EPI>(xb, c_pad, wq, K, bc * h * w, co, K, cg, eb, etile, st);
    if (rc) return rc;
  }
  return XDNA_OK;
}

__global__ void zero_i32_kernel(int32_t* p) { *p = 0; }

}  // namespace xdna

using namespace xdna;

extern "C" {

int xdna_gemm_i8_i32_ws(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int32_t* c, int64_t ldc,
                        int64_t m, int64_t n, int64_t k, void* ws, int64_t ws_bytes, void* stream) {
  XDNA_REQUIRE(m >= 0 && n >= 0 && k >= 0, "negative size");
  if (m == 0 || n == 0) return XDNA_OK;
  XDNA_REQUIRE(k % 16 == 0 && k >= 16, "k must be a positive multiple of 16 (pad with xdna_pad_rows_i8)");
  XDNA_REQUIRE(lda >= k && ldw >= k && lda % 16 == 0 && ldw % 16 == 0 && ldc >= n, "bad leading dimensions");
  XDNA_REQUIRE(a && w && c && aligned(a, 16) && aligned(w, 16), "operands must be 16-byte aligned device pointers");
  XDNA_REQUIRE(ws_bytes >= 0 && (ws == nullptr || aligned(ws, 256)), "workspace must be 256-byte aligned");
  EpiArgs e{};
  e.out = c;
  e.ldo = ldc;
  e.vec_ok = (ldc % 8 == 0) && aligned(c, 16);
  e.ws = ws;
  e.ws_bytes = ws ? ws_bytes : 0;
  const int tile = choose_tile(XDNA_KIND_I8, m, n, k, k);
  return launch_gemm<EPI_I32>(a, lda, w, ldw, m, n, k, e, tile, as_stream(stream));
}

int xdna_gemm_i8_i32(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int32_t* c, int64_t ldc, int64_t m,
                     int64_t n, int64_t k, void* stream) {
  return xdna_gemm_i8_i32_ws(a, lda, w, ldw, c, ldc, m, n, k, nullptr, 0, stream);
}

int xdna_gemm_i8_dequant_ws(const int8_t* a, int64_t lda, const float* sx, const int8_t* w, int64_t ldw,
                            const float* sw, const float* bias, void* y, int y_dtype, int64_t ldy, int64_t m,
                            int64_t n, int64_t k, void* ws, int64_t ws_bytes, void* stream) {
  XDNA_REQUIRE(y_dtype == XDNA_F32 || y_dtype == XDNA_BF16 || y_dtype == XDNA_F16, "y_dtype must be F32/BF16/F16");
  XDNA_REQUIRE(m >= 0 && n >= 0 && k >= 0, "negative size");
  if (m == 0 || n == 0) return XDNA_OK;
  XDNA_REQUIRE(k % 16 == 0 && k >= 16, "k must be a positive multiple of 16 (pad with xdna_pad_rows_i8)");
  XDNA_REQUIRE(lda >= k && ldw >= k && lda % 16 == 0 && ldw % 16 == 0 && ldy >= n, "bad leading dimensions");
  XDNA_REQUIRE(a && w && y && sx && sw && aligned(a, 16) && aligned(w, 16), "bad pointers");
  XDNA_REQUIRE(ws_bytes >= 0 && (ws == nullptr || aligned(ws, 256)), "workspace must be 256-byte aligned");
  EpiArgs e{};
  e.out = y;
  e.ldo = ldy;
  e.sx = sx;
  e.sw = sw;
  e.bias = bias;
  e.vec_ok = (ldy % 8 == 0) && aligned(y, 16);
  e.ws = ws;
  e.ws_bytes = ws ? ws_bytes : 0;
  hipStream_t st = as_stream(stream);
  const int tile = choose_tile(XDNA_KIND_I8, m, n, k, k);
  if (y_dtype == XDNA_F32) return launch_gemm<EPI_DQ_F32>(a, lda, w, ldw, m, n, k, e, tile, st);
  if (y_dtype == XDNA_BF16) return launch_gemm<EPI_DQ_BF16>(a, lda, w, ldw, m, n, k, e, tile, st);
  return launch_gemm<EPI_DQ_F16>(a, lda, w, ldw, m, n, k, e, tile, st);
}

int xdna_gemm_i8_dequant(const int8_t* a, int64_t lda, const float* sx, const int8_t* w, int64_t ldw, const float* sw,
                         const float* bias, void* y, int y_dtype, int64_t ldy, int64_t m, int64_t n, int64_t k,
                         void* stream) {
  return xdna_gemm_i8_dequant_ws(a, lda, sx, w, ldw, sw, bias, y, y_dtype, ldy, m, n, k, nullptr, 0, stream);
}

int xdna_linear_row(const void* x, int x_dtype, int64_t kx, const int8_t* w, int64_t ldw, const float* sw,
                    const float* bias, void* y, int y_dtype, int64_t n, int64_t k, float* sx, void* stream) {
  XDNA_REQUIRE(x_dtype == XDNA_F32 || x_dtype == XDNA_BF16 || x_dtype == XDNA_F16, "x_dtype must be F32/BF16/F16");
  XDNA_REQUIRE(y_dtype == XDNA_F32 || y_dtype == XDNA_BF16 || y_dtype == XDNA_F16, "y_dtype must be F32/BF16/F16");
  XDNA_REQUIRE(n >= 0 && k >= 0 && kx >= 0, "negative size");
  if (n == 0) return XDNA_OK;
  XDNA_REQUIRE(k % 16 == 0 && k >= 16 && k <= XDNA_LINEAR_ROW_KMAX,
               "k must be a multiple of 16 in [16, XDNA_LINEAR_ROW_KMAX]");
  const int64_t esz = x_dtype == XDNA_F32 ? 4 : 2;
  XDNA_REQUIRE(kx >= 1 && kx <= k && (kx * esz) % 16 == 0, "kx must lie in [1, k] with kx elements a multiple of 16 bytes");
  XDNA_REQUIRE(ldw >= k && ldw % 16 == 0, "bad leading dimension");
  XDNA_REQUIRE(x && w && sw && y && aligned(x, 16) && aligned(w, 16), "bad pointers");
  EpiArgs e{};
  e.out = y;
  e.ldo = n;
  e.sw = sw;
  e.bias = bias;
  hipStream_t st = as_stream(stream);
  if (y_dtype == XDNA_F32) return launch_rowq_dt<EPI_DQ_F32>(x, x_dtype, kx, w, ldw, n, k, sx, e, st);
  if (y_dtype == XDNA_BF16) return launch_rowq_dt<EPI_DQ_BF16>(x, x_dtype, kx, w, ldw, n, k, sx, e, st);
  return launch_rowq_dt<EPI_DQ_F16>(x, x_dtype, kx, w, ldw, n, k, sx, e, st);
}

int xdna_gemm_bf16(const void* a, int64_t lda, const void* w, int64_t ldw, const float* bias, void* y, int y_dtype,
                   int64_t ldy, int64_t m, int64_t n, int64_t k, void* stream) {
  XDNA_REQUIRE(y_dtype == XDNA_F32 || y_dtype == XDNA_BF16 || y_dtype == XDNA_F16, "y_dtype must be F32/BF16/F16");
  XDNA_REQUIRE(m >= 0 && n >= 0 && k >= 0, "negative size");
  if (m == 0 || n == 0) return XDNA_OK;
  XDNA_REQUIRE(k % 8 == 0 && k >= 8, "k must be a positive multiple of 8 (16-byte bf16 rows; pad with zeros)");
  XDNA_REQUIRE(lda >= k && ldw >= k && lda % 8 == 0 && ldw % 8 == 0 && ldy >= n, "bad leading dimensions");
  XDNA_REQUIRE(a && w && y && aligned(a, 16) && aligned(w, 16), "operands must be 16-byte aligned device pointers");
  EpiArgs e{};
  e.out = y;
  e.ldo = ldy;
  e.bias = bias;
  e.vec_ok = (ldy % 8 == 0) && aligned(y, 16);
  // the engine stages bytes: a bf16 row of k values is 2 * k bytes
  const int8_t* ab = static_cast<const int8_t*>(a);
  const int8_t* wb = static_cast<const int8_t*>(w);
  hipStream_t st = as_stream(stream);
  const int tile = choose_tile(XDNA_KIND_BF16, m, n, k, 2 * k);
  if (y_dtype == XDNA_F32) return launch_gemm<EPI_BF_F32>(ab, 2 * lda, wb, 2 * ldw, m, n, 2 * k, e, tile, st);
  if (y_dtype == XDNA_BF16) return launch_gemm<EPI_BF_BF16>(ab, 2 * lda, wb, 2 * ldw, m, n, 2 * k, e, tile, st);
  return launch_gemm<EPI_BF_F16>(ab, 2 * lda, wb, 2 * ldw, m, n, 2 * k, e, tile, st);
}

int xdna_gemm_bf16_silu(const void* a, int64_t lda, const void* w, int64_t ldw, void* y, int64_t ldy, int64_t m,
                        int64_t n2, int64_t k, void* stream) {
  XDNA_REQUIRE(m >= 0 && n2 >= 0 && k >= 0, "negative size");
  if (m == 0 || n2 == 0) return XDNA_OK;
  XDNA_REQUIRE(n2 % 4 == 0, "n2 (gate and up rows together) must be a multiple of 4");
  XDNA_REQUIRE(k % 8 == 0 && k >= 8, "k must be a positive multiple of 8 (16-byte bf16 rows; pad with zeros)");
  XDNA_REQUIRE(lda >= k && ldw >= k && lda % 8 == 0 && ldw % 8 == 0 && ldy >= n2 / 2 && ldy % 2 == 0,
               "bad leading dimensions");
  XDNA_REQUIRE(a && w && y && aligned(a, 16) && aligned(w, 16) && aligned(y, 4), "misaligned operands");
  XDNA_REQUIRE(n2 * ldw * 2 <= MAX_BUF, "the gate|up weight must be at most 1 GB");   // no column chunks
  EpiArgs e{};
  e.out = y;
  e.ldo = ldy;
  e.vec_ok = (ldy % 4 == 0) && aligned(y, 8);
  const int8_t* ab = static_cast<const int8_t*>(a);
  const int8_t* wb = static_cast<const int8_t*>(w);
  const int tile = choose_tile(XDNA_KIND_BF16, m, n2, k, 2 * k);
  return launch_gemm<EPI_BF_SILU>(ab, 2 * lda, wb, 2 * ldw, m, n2, 2 * k, e, tile, as_stream(stream));
}

int xdna_conv3x3_i8(const int8_t* x, int64_t nb, int64_t h, int64_t w, int64_t c_pad, const int8_t* wq, int64_t co,
                    int shift, int relu, void* y, int32_t* acc_max, void* stream) {
  XDNA_REQUIRE(nb >= 0 && h >= 1 && w >= 1 && co >= 1, "bad sizes");
  XDNA_REQUIRE(c_pad >= 16 && c_pad % 16 == 0, "c_pad must be a positive multiple of 16");
  if (nb == 0) return XDNA_OK;
  XDNA_REQUIRE(x && wq && aligned(x, 16) && aligned(wq, 16), "operands must be 16-byte aligned device pointers");
  hipStream_t st = as_stream(stream);
  EpiArgs e{};
  e.relu = relu ? 1 : 0;
  if (acc_max) {
    zero_i32_kernel<<<1, 1, 0, st>>>(acc_max);
    e.acc_max = acc_max;
    return launch_conv<EPI_CALIB>(x, nb, h, w, c_pad, wq, co, e, st);
  }
  XDNA_REQUIRE(y != nullptr, "y is null");
  XDNA_REQUIRE(shift >= 1 && shift <= 31, "shift must be in [1, 31]");
  e.out = y;
  e.ldo = co;
  e.shift = shift;
  e.vec_ok = (co % 8 == 0) && aligned(y, 16);
  return launch_conv<EPI_REQUANT>(x, nb, h, w, c_pad, wq, co, e, st);
}

int xdna_conv3x3_dequant(const int8_t* x, int64_t nb, int64_t h, int64_t w, int64_t c_pad, const int8_t* wq,
                         int64_t co, int shift, int relu, const float* scale, const float* sx, const float* bias,
                         void* y, int y_dtype, void* stream) {
  XDNA_REQUIRE(nb >= 0 && h >= 1 && w >= 1 && co >= 1, "bad sizes");
  XDNA_REQUIRE(c_pad >= 16 && c_pad % 16 == 0, "c_pad must be a positive multiple of 16");
  XDNA_REQUIRE(y_dtype == XDNA_F32 || y_dtype == XDNA_BF16 || y_dtype == XDNA_F16,
               "y_dtype must be XDNA_F32, XDNA_BF16 or XDNA_F16");
  if (nb == 0) return XDNA_OK;
  XDNA_REQUIRE(x && wq && aligned(x, 16) && aligned(wq, 16), "operands must be 16-byte aligned device pointers");
  XDNA_REQUIRE(scale && sx && y, "null pointer");
  XDNA_REQUIRE(shift >= 1 && shift <= 31, "shift must be in [1, 31]");
  XDNA_REQUIRE(aligned(y, 16), "y must be 16-byte aligned");
  EpiArgs e{};
  e.out = y;
  e.ldo = co;
  e.shift = shift;
  e.relu = relu ? 1 : 0;
  e.sw = scale;
  e.sx = sx;
  e.bias = bias;
  e.dq_out = y_dtype + 1;
  e.px0 = 0;
  return launch_conv<EPI_REQUANT>(x, nb, h, w, c_pad, wq, co, e, as_stream(stream));
}

int xdna_tile_set(int kind, int64_t m, int64_t n, int64_t k, int tile) {
  XDNA_REQUIRE(kind == XDNA_KIND_I8 || kind == XDNA_KIND_BF16 || kind == XDNA_KIND_CONV, "unknown kind");
  XDNA_REQUIRE(m >= 1 && n >= 1 && k >= 1, "bad sizes");
  XDNA_REQUIRE(tile >= T_AUTO && tile < T_COUNT, "unknown tile id");
  XDNA_REQUIRE(!(kind == XDNA_KIND_CONV && (is_small(tile) || is_gemv(tile) || is_seg4(tile))),
               "the small-M, one-row and few-row kernels do not run convs");
  XDNA_REQUIRE(!(kind != XDNA_KIND_CONV && tile == T_DIRECT), "the direct conv kernels run only convs");
  std::lock_guard<std::mutex> lock(g_tile_mu);
  const TileKey key{kind, m, n, k};
  if (tile == T_AUTO) g_tiles.erase(key);
  else g_tiles[key] = tile;
  g_tile_count.store((int)g_tiles.size(), std::memory_order_release);
  return XDNA_OK;
}

int xdna_tile_get(int kind, int64_t m, int64_t n, int64_t k) {
  XDNA_REQUIRE(kind == XDNA_KIND_I8 || kind == XDNA_KIND_BF16 || kind == XDNA_KIND_CONV, "unknown kind");
  XDNA_REQUIRE(m >= 1 && n >= 1 && k >= 1, "bad sizes");
  return choose_tile(kind, m, n, k, kind == XDNA_KIND_BF16 ? 2 * k : k);
}

int xdna_tile_plan(int kind, int64_t m, int64_t n, int64_t k, int* head, int64_t* m1, int* tail) {
  XDNA_REQUIRE(kind == XDNA_KIND_I8 || kind == XDNA_KIND_BF16 || kind == XDNA_KIND_CONV, "unknown kind");
  XDNA_REQUIRE(m >= 1 && n >= 1 && k >= 1, "bad sizes");
  XDNA_REQUIRE(head && m1 && tail, "null output pointer");
  const int64_t kbytes = kind == XDNA_KIND_BF16 ? 2 * k : k;
  int t = choose_tile(kind, m, n, k, kbytes);
  // the launchers' own substitutions: the one-row and few-row kernels take only their row counts, and
  // the small-M kernel addresses the whole activation with one buffer resource
  if (kind != XDNA_KIND_CONV) {
    if (is_gemv(t) && m != 1) t = rule_tile(m, n, kbytes, m > 1);
    if (is_seg4(t) && m > 16) t = rule_tile(m, n, kbytes, true);
    if (is_small(t) && (m * kbytes > MAX_BUF || (m + 15) / 16 >= 65536)) t = rule_tile(m, n, kbytes, false);
  }
  // GEMM operands above one buffer resource run in row chunks (with dense rows, lda = k): the plan of
  // the first chunk
  int64_t mc = m;
  if (kind != XDNA_KIND_CONV && !(is_small(t) || is_gemv(t) || is_seg4(t)))
    mc = std::min(m, std::max<int64_t>(256, (MAX_BUF / kbytes) / 256 * 256));
  const TilePlan p = plan_tiles(kind, mc, n, kbytes, k, t);
  *head = p.head;
  *m1 = p.m1;
  *tail = p.tail;
  return XDNA_OK;
}

int64_t xdna_gemm_ws_bytes(int64_t m, int64_t n, int64_t k) {
  XDNA_REQUIRE(m >= 1 && n >= 1 && k >= 16 && k % 16 == 0, "bad sizes");
  int head = 0, tail = 0;
  int64_t m1 = 0;
  if (xdna_tile_plan(XDNA_KIND_I8, m, n, k, &head, &m1, &tail) != XDNA_OK) return -1;
  if (is_small(head) || is_gemv(head) || is_seg4(head)) return 0;
  auto can_split = [](int tile) {
    const TileCfg t = tile_cfg(tile);
    return t.bm * t.bn <= 64 * 64;
  };
  if (!can_split(head) && !(m1 > 0 && can_split(tail))) return 0;
  // a split launch has at most as many workgroups as CUs (tiles x splits <= CUs), each holding at most a
  // 64 x 64 int32 tile of partial sums: one bound for every launch of the call
  return WS_CNT_BYTES + device_cus() * 64 * 64 * 4;
}

int xdna_gemm_ksplit(int64_t m, int64_t n, int64_t k, int* head_ks, int* tail_ks) {
  XDNA_REQUIRE(head_ks && tail_ks, "null output pointer");
  *head_ks = *tail_ks = 1;
  int head = 0, tail = 0;
  int64_t m1 = 0;
  const int rc = xdna_tile_plan(XDNA_KIND_I8, m, n, k, &head, &m1, &tail);
  if (rc != XDNA_OK) return rc;
  if (is_small(head) || is_gemv(head) || is_seg4(head)) return XDNA_OK;
  // the first row and column chunk's launches, as launch_gemm / launch_tiles make them (dense rows)
  const int64_t mc = std::min(m, std::max<int64_t>(256, (MAX_BUF / k) / 256 * 256));
  const int64_t nc = std::min(n, std::max<int64_t>(256, (MAX_BUF / k) / 256 * 256));
  auto ks_of = [&](int tile, int64_t rows) {
    const TileCfg t = tile_cfg(tile);
    return ksplit_for(t, ((rows + t.bm - 1) / t.bm) * ((nc + t.bn - 1) / t.bn), k);
  };
  *head_ks = ks_of(head, m1 ? m1 : mc);
  if (m1) *tail_ks = ks_of(tail, mc - m1);
  return XDNA_OK;
}

int xdna_tile_clear(void) {
  std::lock_guard<std::mutex> lock(g_tile_mu);
  g_tiles.clear();
  g_tile_count.store(0, std::memory_order_release);
  return XDNA_OK;
}

}  // extern "C"
