// int8 MFMA GEMM and implicit-GEMM 3x3 conv for gfx950 (MI355X).
//
// One tile engine serves both ops. A workgroup computes a BM x BN tile of D = A * W^T with
// A [M, K] and W [N, K] int8, both K-contiguous, accumulating in int32 with
// v_mfma_i32_16x16x64_i8. The MFMA is issued as D^T = W * A^T (W fragment in srcA, A fragment in
// srcB), so each lane ends up holding four consecutive output columns n of one row m, and the
// epilogue writes 16-byte (int32 / fp32) or 8-byte (bf16) pieces of output rows.
//
// K is staged through LDS in 128-byte slices, double-buffered: while the waves run the MFMAs of
// slice kt from one LDS buffer, the next slice's global loads are in flight in registers and are
// written to the other buffer afterwards (one barrier per slice). LDS rows are 128 bytes; the
// 16-byte chunk c of row r is stored at chunk c ^ (r & 7), so the eight rows a fragment read
// touches in one pass land in eight different bank groups.
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
// columns, its waves split K, each lane streams 32 contiguous weight bytes per step (so every
// weight row is read as whole 128-byte lines), and the partial sums meet in LDS.
#include <algorithm>
#include <string>

#include "xdna_common.h"

namespace xdna {

// EPI_DEQUANT_* carry the output dtype in the kernel's type so each epilogue is straight-line code.
enum Epi { EPI_I32 = 0, EPI_REQUANT = 2, EPI_CALIB = 3, EPI_DQ_F32 = 4, EPI_DQ_BF16 = 5, EPI_DQ_F16 = 6 };

struct EpiArgs {
  void* out;            // int32 C, float y, or int8/uint8 q (NHWC)
  int64_t ldo;          // elements between output rows
  const float* sx;      // [M]
  const float* sw;      // [N]
  const float* bias;    // [N] or null
  int shift;            // EPI_REQUANT
  int relu;             // EPI_REQUANT / EPI_CALIB
  int32_t* acc_max;     // EPI_CALIB
  int vec_ok;           // output rows allow 4-wide vector stores
};

struct ConvGeom {
  int64_t h, w, c_pad;  // NHWC input geometry
};

__device__ __forceinline__ i32x4 mfma16x16x64(const i32x4& a, const i32x4& b, const i32x4& c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------------------ epilogue
// One lane's four outputs: row m, columns n .. n+3 (acc[r] is column n + r).
template <int EPI>
__device__ __forceinline__ void epilogue4(const EpiArgs& e, int64_t m, int64_t n, int64_t M, int64_t N,
                                          const i32x4& acc, int& calib) {
  if (m >= M) return;
  if constexpr (EPI == EPI_CALIB) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (n + r < N) {
        int v = acc[r];
        v = e.relu ? max(v, 0) : abs(v);
        calib = max(calib, v);
      }
    }
  } else if constexpr (EPI == EPI_I32) {
    int32_t* c = reinterpret_cast<int32_t*>(e.out) + m * e.ldo + n;
    if (e.vec_ok && n + 3 < N) {
      *reinterpret_cast<i32x4*>(c) = acc;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (n + r < N) c[r] = acc[r];
    }
  } else if constexpr (EPI == EPI_REQUANT) {
    const int half = 1 << (e.shift - 1);
    uint32_t packed = 0;
    int qv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int q = (acc[r] + half) >> e.shift;      // arithmetic shift: floor, i.e. round half up
      q = e.relu ? min(max(q, 0), 255) : min(max(q, -128), 127);
      qv[r] = q;
      packed |= ((uint32_t)(q & 0xff)) << (8 * r);
    }
    uint8_t* o = reinterpret_cast<uint8_t*>(e.out) + m * e.ldo + n;
    if (e.vec_ok && n + 3 < N) {
      *reinterpret_cast<uint32_t*>(o) = packed;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (n + r < N) o[r] = (uint8_t)(qv[r] & 0xff);
    }
  } else {  // EPI_DQ_*: ((float)acc * sx[m]) * sw[n] (+ bias[n]), each step rounded once
    const float sxm = e.sx[m];
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (n + r < N) {
        float t = (float)acc[r];
        t = t * sxm;
        t = t * e.sw[n + r];
        if (e.bias) t = t + e.bias[n + r];
        v[r] = t;
      } else {
        v[r] = 0.0f;
      }
    }
    const int64_t off = m * e.ldo + n;
    if constexpr (EPI == EPI_DQ_F32) {
      float* y = reinterpret_cast<float*>(e.out) + off;
      if (e.vec_ok && n + 3 < N) {
        *reinterpret_cast<f32x4*>(y) = f32x4{v[0], v[1], v[2], v[3]};
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < N) y[r] = v[r];
      }
    } else {
      uint16_t h[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) h[r] = EPI == EPI_DQ_BF16 ? f32_to_bf16_bits(v[r]) : f32_to_f16_bits(v[r]);
      uint16_t* y = reinterpret_cast<uint16_t*>(e.out) + off;
      if (e.vec_ok && n + 3 < N) {
        *reinterpret_cast<uint2*>(y) = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16),
                                                  (uint32_t)h[2] | ((uint32_t)h[3] << 16));
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < N) y[r] = h[r];
      }
    }
  }
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
__device__ __forceinline__ void tile_coords(int64_t pid, int64_t tiles_m, int64_t tiles_n, int64_t& tm, int64_t& tn) {
  constexpr int XCDS = 8;
  constexpr int GROUP_M = 8;
  const int64_t total = tiles_m * tiles_n;
  const int64_t q = total / XCDS, r = total % XCDS;
  const int64_t xcd = pid % XCDS, local = pid / XCDS;
  const int64_t tile = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + local;
  const int64_t in_group = (int64_t)GROUP_M * tiles_n;
  const int64_t g = tile / in_group;
  const int64_t first_m = g * GROUP_M;
  const int64_t gsz = min((int64_t)GROUP_M, tiles_m - first_m);
  const int64_t rem = tile % in_group;
  tm = first_m + rem % gsz;
  tn = rem / gsz;
}

__device__ __forceinline__ int swz(int row, int chunk) { return (row << 7) + ((chunk ^ (row & 7)) << 4); }

template <int BM, int BN, int WM, int WN, bool CONV, int EPI>
__global__ __launch_bounds__(WM * WN * 64) void mm_tile_kernel(const int8_t* __restrict__ a, int64_t lda,
                                                               const int8_t* __restrict__ w, int64_t ldw, int64_t M,
                                                               int64_t N, int64_t K, ConvGeom cg, EpiArgs e) {
  constexpr int BK = 128;
  constexpr int T = WM * WN * 64;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16;
  constexpr int AC = BM * 8 / T;   // A chunks (16 B) per thread per K slice
  constexpr int WC = BN * 8 / T;
  static_assert(AC >= 1 && WC >= 1 && BM * 8 % T == 0 && BN * 8 % T == 0, "tile / thread mismatch");

  __shared__ __attribute__((aligned(16))) int8_t lds[2 * (BM + BN) * BK];
  // buffer b: A slice at lds + b * STAGE, W slice right after it
  constexpr int STAGE = (BM + BN) * BK;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int64_t tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = tm * BM, n0 = tn * BN;

  // Per-thread load slots: chunk index is fixed per thread, rows step by T/8.
  const int chunk = tid & 7;
  const int row0 = tid >> 3;
  constexpr int RSTEP = T / 8;

  const int8_t* pa[AC];
  bool va[AC];
  int py[AC], px[AC];
  (void)py;
  (void)px;
#pragma unroll
  for (int i = 0; i < AC; ++i) {
    const int64_t m = m0 + row0 + i * RSTEP;
    va[i] = m < M;
    if constexpr (CONV) {
      const int64_t hw = cg.h * cg.w;
      const int64_t mm = va[i] ? m : 0;
      const int64_t img = mm / hw, p = mm - img * hw;
      py[i] = (int)(p / cg.w);
      px[i] = (int)(p - (int64_t)py[i] * cg.w);
      pa[i] = a + mm * cg.c_pad + chunk * 16;   // pixel (img, y, x), channel chunk
    } else {
      pa[i] = a + (va[i] ? m : 0) * lda + chunk * 16;
    }
  }
  const int8_t* pw[WC];
  bool vw[WC];
#pragma unroll
  for (int i = 0; i < WC; ++i) {
    const int64_t n = n0 + row0 + i * RSTEP;
    vw[i] = n < N;
    pw[i] = w + (vw[i] ? n : 0) * ldw + chunk * 16;
  }

  i32x4 ra[AC], rw[WC];
  auto gload = [&](int64_t kt) {
    const int64_t kb = kt * BK + chunk * 16;
    const bool kin = kb < K;
    if constexpr (CONV) {
      const int64_t tap = kb / cg.c_pad;
      const int64_t c = kb - tap * cg.c_pad;
      const int dy = (int)(tap / 3) - 1, dx = (int)(tap % 3) - 1;
      const int64_t delta = ((int64_t)dy * cg.w + dx) * cg.c_pad + c - chunk * 16;
#pragma unroll
      for (int i = 0; i < AC; ++i) {
        const int sy = py[i] + dy, sx = px[i] + dx;
        const bool ok = kin && va[i] && sy >= 0 && sy < cg.h && sx >= 0 && sx < cg.w;
        ra[i] = ok ? *reinterpret_cast<const i32x4*>(pa[i] + delta) : i32x4{0, 0, 0, 0};
      }
    } else {
#pragma unroll
      for (int i = 0; i < AC; ++i)
        ra[i] = (kin && va[i]) ? *reinterpret_cast<const i32x4*>(pa[i] + kt * BK) : i32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < WC; ++i)
      rw[i] = (kin && vw[i]) ? *reinterpret_cast<const i32x4*>(pw[i] + kt * BK) : i32x4{0, 0, 0, 0};
  };
  auto lstore = [&](int buf) {
    int8_t* sa = lds + buf * STAGE;
    int8_t* sw = sa + BM * BK;
#pragma unroll
    for (int i = 0; i < AC; ++i) *reinterpret_cast<i32x4*>(sa + swz(row0 + i * RSTEP, chunk)) = ra[i];
#pragma unroll
    for (int i = 0; i < WC; ++i) *reinterpret_cast<i32x4*>(sw + swz(row0 + i * RSTEP, chunk)) = rw[i];
  };

  i32x4 acc[FN][FM];
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int i = 0; i < FM; ++i) acc[j][i] = i32x4{0, 0, 0, 0};

  const int64_t nk = (K + BK - 1) / BK;
  gload(0);
  lstore(0);
  __syncthreads();

  const int frow = lane & 15;
  const int fk = lane >> 4;
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const int8_t* sa = lds + cur * STAGE;
    const int8_t* sw = sa + BM * BK;
    if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      i32x4 fa[FM], fw[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        fa[i] = *reinterpret_cast<const i32x4*>(sa + swz(wm * TM + i * 16 + frow, kk * 4 + fk));
#pragma unroll
      for (int j = 0; j < FN; ++j)
        fw[j] = *reinterpret_cast<const i32x4*>(sw + swz(wn * TN + j * 16 + frow, kk * 4 + fk));
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int i = 0; i < FM; ++i) acc[j][i] = mfma16x16x64(fw[j], fa[i], acc[j][i]);
    }
    if (kt + 1 < nk) lstore(cur ^ 1);
    __syncthreads();
  }

  int calib = 0;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int64_t m = m0 + wm * TM + i * 16 + (lane & 15);
      const int64_t n = n0 + wn * TN + j * 16 + 4 * (lane >> 4);
      epilogue4<EPI>(e, m, n, M, N, acc[j][i], calib);
      // keep each fragment's epilogue loads next to its stores (no hoisting of all of them)
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  calib_flush<EPI>(e, calib);
}

// ------------------------------------------------------------------------------ small M
// Workgroup = WAVES waves owning output columns [n0, n0+16) and rows [m0, m0+16); wave v sums
// k in its own K range. Per step a lane loads 32 bytes of weight row n0 + (lane & 15) at
// k = kb + (lane >> 4) * 32 and the matching 32 bytes of activation row m0 + (lane & 15), and
// issues two MFMAs (bytes 0..15 and 16..31).
template <int WAVES, int U, int EPI>
__global__ __launch_bounds__(WAVES * 64) void mm_small_kernel(const int8_t* __restrict__ a, int64_t lda,
                                                              const int8_t* __restrict__ w, int64_t ldw, int64_t M,
                                                              int64_t N, int64_t K, int64_t kper, EpiArgs e) {
  __shared__ i32x4 red[WAVES][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int64_t m0 = (int64_t)blockIdx.y * 16;
  const int64_t n = n0 + (lane & 15);
  const int64_t m = m0 + (lane & 15);
  const bool nv = n < N, mv = m < M;
  const int8_t* pw = w + (nv ? n : 0) * ldw + (lane >> 4) * 32;
  const int8_t* pa = a + (mv ? m : 0) * lda + (lane >> 4) * 32;
  const int64_t kbeg = (int64_t)wave * kper;
  const int64_t kend = min(K, kbeg + kper);

  i32x4 acc = {0, 0, 0, 0};
  for (int64_t kb = kbeg; kb < kend; kb += 128 * U) {
    i32x4 wv[U][2], av[U][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k = kb + u * 128 + (lane >> 4) * 32;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const bool kin = k + h * 16 < kend;
        wv[u][h] = (nv && kin) ? *reinterpret_cast<const i32x4*>(pw + kb + u * 128 + h * 16) : i32x4{0, 0, 0, 0};
        av[u][h] = (mv && kin) ? *reinterpret_cast<const i32x4*>(pa + kb + u * 128 + h * 16) : i32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      acc = mfma16x16x64(wv[u][0], av[u][0], acc);
      acc = mfma16x16x64(wv[u][1], av[u][1], acc);
    }
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int v = 1; v < WAVES; ++v) acc += red[v][lane];
  int calib = 0;
  epilogue4<EPI>(e, m0 + (lane & 15), n0 + 4 * (lane >> 4), M, N, acc, calib);
  calib_flush<EPI>(e, calib);
}

// ------------------------------------------------------------------------------ dispatch
struct TileCfg {
  int bm, bn;
};

int g_num_cus = 0;

int num_cus() {
  if (g_num_cus == 0) {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
      g_num_cus = prop.multiProcessorCount;
    else
      g_num_cus = 256;
  }
  return g_num_cus;
}

// Pick the largest tile that still gives every CU work; a 256x256 tile needs 128 KB of LDS and
// runs one workgroup per CU, a 128x128 tile two to three, a 64x64 tile up to eight.
TileCfg pick_tile(int64_t M, int64_t N) {
  const int64_t cus = num_cus();
  auto tiles = [&](int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  if (M >= 256 && N >= 256 && tiles(256, 256) >= cus) return {256, 256};
  if (M >= 128 && N >= 128 && tiles(128, 128) >= cus) return {128, 128};
  return {64, 64};
}

template <bool CONV, int EPI>
int launch_mm(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K,
              ConvGeom cg, const EpiArgs& e, hipStream_t st) {
  if (!CONV && M <= 64) {
    // weight streaming: waves split K into 128-byte multiples
    constexpr int WAVES = 8, U = 2;
    const int64_t slices = (K + 127) / 128;
    const int64_t kper = ((slices + WAVES - 1) / WAVES) * 128;
    dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + 15) / 16), 1);
    mm_small_kernel<WAVES, U, EPI><<<grid, WAVES * 64, 0, st>>>(a, lda, w, ldw, M, N, K, kper, e);
    return launch_status("mm_small");
  }
  const TileCfg t = pick_tile(M, N);
  const int64_t tiles = ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
  if (tiles >= (1ll << 31)) {
    set_error("launch_mm: too many tiles");
    return XDNA_EINVAL;
  }
  dim3 grid((unsigned)tiles, 1, 1);
  if (t.bm == 256) mm_tile_kernel<256, 256, 2, 2, CONV, EPI><<<grid, 256, 0, st>>>(a, lda, w, ldw, M, N, K, cg, e);
  else if (t.bm == 128) mm_tile_kernel<128, 128, 2, 2, CONV, EPI><<<grid, 256, 0, st>>>(a, lda, w, ldw, M, N, K, cg, e);
  else mm_tile_kernel<64, 64, 2, 2, CONV, EPI><<<grid, 256, 0, st>>>(a, lda, w, ldw, M, N, K, cg, e);
  return launch_status("mm_tile");
}

__global__ void zero_i32_kernel(int32_t* p) { *p = 0; }

}  // namespace xdna

using namespace xdna;

extern "C" {

int xdna_gemm_i8_i32(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int32_t* c, int64_t ldc, int64_t m,
                     int64_t n, int64_t k, void* stream) {
  XDNA_REQUIRE(m >= 0 && n >= 0 && k >= 0, "negative size");
  if (m == 0 || n == 0) return XDNA_OK;
  XDNA_REQUIRE(k % 16 == 0 && k >= 16, "k must be a positive multiple of 16 (pad with xdna_pad_rows_i8)");
  XDNA_REQUIRE(lda >= k && ldw >= k && lda % 16 == 0 && ldw % 16 == 0 && ldc >= n, "bad leading dimensions");
  XDNA_REQUIRE(a && w && c && aligned(a, 16) && aligned(w, 16), "operands must be 16-byte aligned device pointers");
  EpiArgs e{};
  e.out = c;
  e.ldo = ldc;
  e.vec_ok = (ldc % 4 == 0) && aligned(c, 16);
  return launch_mm<false, EPI_I32>(a, lda, w, ldw, m, n, k, ConvGeom{}, e, as_stream(stream));
}

int xdna_gemm_i8_dequant(const int8_t* a, int64_t lda, const float* sx, const int8_t* w, int64_t ldw, const float* sw,
                         const float* bias, void* y, int y_dtype, int64_t ldy, int64_t m, int64_t n, int64_t k,
                         void* stream) {
  XDNA_REQUIRE(y_dtype == XDNA_F32 || y_dtype == XDNA_BF16 || y_dtype == XDNA_F16, "y_dtype must be F32/BF16/F16");
  XDNA_REQUIRE(m >= 0 && n >= 0 && k >= 0, "negative size");
  if (m == 0 || n == 0) return XDNA_OK;
  XDNA_REQUIRE(k % 16 == 0 && k >= 16, "k must be a positive multiple of 16 (pad with xdna_pad_rows_i8)");
  XDNA_REQUIRE(lda >= k && ldw >= k && lda % 16 == 0 && ldw % 16 == 0 && ldy >= n, "bad leading dimensions");
  XDNA_REQUIRE(a && w && y && sx && sw && aligned(a, 16) && aligned(w, 16), "bad pointers");
  EpiArgs e{};
  e.out = y;
  e.ldo = ldy;
  e.sx = sx;
  e.sw = sw;
  e.bias = bias;
  const int esz = y_dtype == XDNA_F32 ? 4 : 2;
  e.vec_ok = (ldy % 4 == 0) && aligned(y, 4 * esz);
  hipStream_t st = as_stream(stream);
  if (y_dtype == XDNA_F32) return launch_mm<false, EPI_DQ_F32>(a, lda, w, ldw, m, n, k, ConvGeom{}, e, st);
  if (y_dtype == XDNA_BF16) return launch_mm<false, EPI_DQ_BF16>(a, lda, w, ldw, m, n, k, ConvGeom{}, e, st);
  return launch_mm<false, EPI_DQ_F16>(a, lda, w, ldw, m, n, k, ConvGeom{}, e, st);
}

int xdna_conv3x3_i8(const int8_t* x, int64_t nb, int64_t h, int64_t w, int64_t c_pad, const int8_t* wq, int64_t co,
                    int shift, int relu, void* y, int32_t* acc_max, void* stream) {
  XDNA_REQUIRE(nb >= 0 && h >= 1 && w >= 1 && co >= 1, "bad sizes");
  XDNA_REQUIRE(c_pad >= 16 && c_pad % 16 == 0, "c_pad must be a positive multiple of 16");
  if (nb == 0) return XDNA_OK;
  XDNA_REQUIRE(x && wq && aligned(x, 16) && aligned(wq, 16), "operands must be 16-byte aligned device pointers");
  hipStream_t st = as_stream(stream);
  const int64_t M = nb * h * w, K = 9 * c_pad;
  ConvGeom cg{h, w, c_pad};
  EpiArgs e{};
  e.relu = relu ? 1 : 0;
  if (acc_max) {
    zero_i32_kernel<<<1, 1, 0, st>>>(acc_max);
    e.acc_max = acc_max;
    return launch_mm<true, EPI_CALIB>(x, c_pad, wq, K, M, co, K, cg, e, st);
  }
  XDNA_REQUIRE(y != nullptr, "y is null");
  XDNA_REQUIRE(shift >= 1 && shift <= 31, "shift must be in [1, 31]");
  e.out = y;
  e.ldo = co;
  e.shift = shift;
  e.vec_ok = (co % 4 == 0) && aligned(y, 4);
  return launch_mm<true, EPI_REQUANT>(x, c_pad, wq, K, M, co, K, cg, e, st);
}

}  // extern "C"
