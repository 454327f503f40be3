// int8 MFMA GEMM and implicit-GEMM 3x3 conv for gfx950 (MI355X).
//
// One tile engine serves both ops. A workgroup computes a BM x BN tile of D = A * W^T with
// A [M, K] and W [N, K] int8, both K-contiguous, accumulating in int32 with
// v_mfma_i32_32x32x32_i8 (the full-rate int8 MFMA of gfx950). The MFMA is issued as
// D^T = W * A^T (W fragment in srcA, A fragment in srcB), so each lane holds consecutive output
// columns n of one row m. Tiles: 256x256 with 8 waves (two per SIMD), 256x128 / 128x256 /
// 128x128 with 4 waves, 64x64 with 4 waves; the host picks one per shape.
//
// K is staged through LDS in 128-byte slices, two stages deep, by the LDS-DMA form of the raw
// buffer load: each lane's 16 bytes land at M0 + 16 * lane, so no VGPRs carry the tile. The DMA
// of slice kt + 2 is issued after the one barrier per slice and overlaps the MFMAs of kt + 1.
// LDS rows are 128 bytes; the 16-byte chunk c of row r sits at chunk c ^ f(r) with
// f(r) = (r & 7) ^ ((r >> 3) & 1), which keeps the 8- and 16-lane phases of a fragment read on
// distinct bank groups and is periodic in 16 rows, so fragment offsets are immediates.
// Out-of-range rows, K chunks and conv halo pixels are out-of-range buffer loads, which read 0.
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
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <type_traits>

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

typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ i32x4 mfma16x16x64(const i32x4& a, const i32x4& b, const i32x4& c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// The tile engine's MFMA: on gfx950 the 32x32x32 int8 form issues at the full int8 rate
// (32768 MACs per 32 cycles per SIMD); the 16x16x64 form issues at half of it.
__device__ __forceinline__ i32x16 mfma32x32x32(const i32x4& a, const i32x4& b, const i32x16& c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------------------ epilogue
// Per-column values of four consecutive output columns n .. n+3 (weight scales and bias of the
// dequantize), loaded once per column block and reused for every row.
template <int EPI>
struct EpiCols {
  float sw[4], b[4];
  __device__ __forceinline__ EpiCols() {}
  __device__ __forceinline__ EpiCols(const EpiArgs& e, int64_t n, int64_t N) {
    if constexpr (EPI == EPI_DQ_F32 || EPI == EPI_DQ_BF16 || EPI == EPI_DQ_F16) {
      if (n + 3 < N && (reinterpret_cast<uintptr_t>(e.sw + n) & 15) == 0) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(e.sw + n);
        sw[0] = v[0], sw[1] = v[1], sw[2] = v[2], sw[3] = v[3];
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) sw[r] = n + r < N ? e.sw[n + r] : 0.0f;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) b[r] = 0.0f;
      if (e.bias) {
        if (n + 3 < N && (reinterpret_cast<uintptr_t>(e.bias + n) & 15) == 0) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(e.bias + n);
          b[0] = v[0], b[1] = v[1], b[2] = v[2], b[3] = v[3];
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) b[r] = n + r < N ? e.bias[n + r] : 0.0f;
        }
      }
    }
  }
};

// One lane's four outputs: row m, columns n .. n+3 (acc[r] is column n + r). FULL: the caller has
// established that the whole tile is in bounds and vector stores are allowed (no per-element tests).
template <int EPI, bool FULL = false>
__device__ __forceinline__ void epilogue4(const EpiArgs& e, int64_t m, int64_t n, int64_t M, int64_t N,
                                          const i32x4& acc, int& calib, const EpiCols<EPI>& cols, float sxm) {
  if constexpr (FULL) {
    if constexpr (EPI == EPI_CALIB) {
#pragma unroll
      for (int r = 0; r < 4; ++r) calib = max(calib, e.relu ? max(acc[r], 0) : abs(acc[r]));
    } else if constexpr (EPI == EPI_I32) {
      *reinterpret_cast<i32x4*>(reinterpret_cast<int32_t*>(e.out) + m * e.ldo + n) = acc;
    } else if constexpr (EPI == EPI_REQUANT) {
      const int half = 1 << (e.shift - 1);
      uint32_t packed = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int q = (acc[r] + half) >> e.shift;    // arithmetic shift: floor, i.e. round half up
        q = e.relu ? min(max(q, 0), 255) : min(max(q, -128), 127);
        packed |= ((uint32_t)(q & 0xff)) << (8 * r);
      }
      *reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(e.out) + m * e.ldo + n) = packed;
    } else {
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float t = (float)acc[r];
        t = t * sxm;
        t = t * cols.sw[r];
        if (e.bias) t = t + cols.b[r];         // uniform test: the bias pointer is a kernel argument
        v[r] = t;
      }
      const int64_t off = m * e.ldo + n;
      if constexpr (EPI == EPI_DQ_F32) {
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(e.out) + off) = f32x4{v[0], v[1], v[2], v[3]};
      } else {
        uint16_t h[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) h[r] = EPI == EPI_DQ_BF16 ? f32_to_bf16_bits(v[r]) : f32_to_f16_bits(v[r]);
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(e.out) + off) =
            make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
      }
    }
    return;
  }
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
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (n + r < N) {
        float t = (float)acc[r];
        t = t * sxm;
        t = t * cols.sw[r];
        if (e.bias) t = t + cols.b[r];
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

// LDS rows are 128 bytes (one K slice of a row); chunk c of row r sits at chunk c ^ f(r) with
// f(r) = (r & 7) ^ ((r >> 3) & 1). A fragment read touches 16 consecutive rows at one logical chunk:
// rows r..r+7 land in 8 distinct 16-byte bank groups (LDS serving 8 lanes of 16 bytes per pass), and
// the 8 rows of equal parity among r..r+15 land in 8 distinct groups of a 256-byte line (16 lanes per
// pass). f depends only on r & 15, so fragments 16 rows apart differ by a constant LDS offset.
__device__ __forceinline__ int swz_f(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int swz(int row, int chunk) { return (row << 7) + ((chunk ^ swz_f(row)) << 4); }

// Raw buffer loads: a 16-byte load at a byte offset >= the resource's size returns zeros, which is how
// rows past M / N, chunks past K and conv taps outside the image read as zero without a branch.
constexpr uint32_t OOB = 0x7ffffff0u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16 bytes per lane from global memory straight into LDS: lane l's bytes land at lds + 16 * l.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t off, int8_t* lds, uint32_t soff = 0) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, (int)off, (int)soff, 0, 0);
}

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


// Tile engine. Each K slice (128 bytes of K) of the A and W tiles is brought into LDS by the DMA
// form of the buffer load: one wave instruction fills 8 whole 128-byte LDS rows, and each lane
// fetches the global chunk that belongs at its LDS position under the swizzle. Two LDS stages; per
// slice kt (two 64-deep MFMA steps):
//   step 0: MFMAs of the step-0 fragments, with the step-1 fragment reads in between;
//   step 1, first half of the MFMAs; wait for this wave's DMA of slice kt+1; barrier;
//   step 1, second half, with the DMA of slice kt+2 (into the stage just freed) and the reads of
//   slice kt+1's step-0 fragments in between.
// One barrier per slice; the DMA has a whole slice of MFMAs to land.
template <int BM, int BN, int WM, int WN, int CONVM, int EPI, bool KFULL>
__global__ __launch_bounds__(WM * WN * 64) void mm_tile_kernel(const int8_t* __restrict__ a, int64_t lda,
                                                               const int8_t* __restrict__ w, int64_t ldw, int64_t M,
                                                               int64_t N, int64_t K, ConvGeom cg, EpiArgs e) {
  constexpr bool CONV = CONVM != 0;      // CONVM: 0 GEMM, 1 conv with C_pad % 128 == 0, 2 any C_pad
  constexpr int BK = 128;
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;  // 32 x 32 MFMA tiles per wave
  constexpr int IA = BM / 8 / NW;        // DMA instructions per wave per slice (8 rows each)
  constexpr int IW = BN / 8 / NW;
  static_assert(FM >= 1 && FN >= 1, "wave tile below 32 x 32");
  static_assert(IA >= 1 && IW >= 1 && BM % (8 * NW) == 0 && BN % (8 * NW) == 0, "tile / wave mismatch");
  constexpr int STAGE = (BM + BN) * BK;

  __shared__ __attribute__((aligned(1024))) int8_t lds[2 * STAGE];
  int8_t* const lds0 = lds;
  int8_t* const lds1 = lds + STAGE;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: keeps LDS bases scalar
  const int wm = wave / WN, wn = wave % WN;

  const int64_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  int64_t tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = tm * BM, n0 = tn * BN;

  // The epilogue's per-row and per-column scales do not depend on K: load them now, so they arrive
  // during the K loop. Read-back layout: row rr * 8 + (lane >> 3), columns 4 * (lane & 7) .. +3.
  constexpr bool DQ = EPI == EPI_DQ_F32 || EPI == EPI_DQ_BF16 || EPI == EPI_DQ_F16;
  float sx_pre[DQ ? TM / 8 : 1];
  if constexpr (DQ) {
#pragma unroll
    for (int rr = 0; rr < TM / 8; ++rr) {
      const int64_t m = m0 + wm * TM + rr * 8 + (lane >> 3);
      sx_pre[rr] = m < M ? e.sx[m] : 0.0f;
    }
  }
  EpiCols<EPI> cols_pre[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) cols_pre[j] = EpiCols<EPI>(e, n0 + wn * TN + j * 32 + (lane & 7) * 4, N);

  const __amdgpu_buffer_rsrc_t ra_rsrc = make_rsrc(a, (uint32_t)(CONV ? (M * cg.c_pad) : (M * lda)));
  const __amdgpu_buffer_rsrc_t rw_rsrc = make_rsrc(w, (uint32_t)(N * ldw));

  // This lane's rows: DMA instruction j of this wave covers tile rows r0 = (wave * I + j) * 8 .. +8,
  // and lane l fills LDS chunk l % 8 of row r0 + l / 8, i.e. logical chunk (l % 8) ^ f(row).
  const int lrow = lane >> 3;
  const int pch = lane & 7;
  uint32_t oa[IA], ow[IW];
  int ca[IA], cw[IW];                    // logical chunk per slot
  int py[IA], px[IA];
  (void)py;
  (void)px;
#pragma unroll
  for (int j = 0; j < IA; ++j) {
    const int row = (wave * IA + j) * 8 + lrow;
    ca[j] = pch ^ swz_f(row);
    const int64_t m = m0 + row;
    if constexpr (CONV) {
      const int64_t hw = cg.h * cg.w;
      const int64_t mm = m < M ? m : 0;
      const int64_t img = mm / hw, p = mm - img * hw;
      const int yy = (int)(p / cg.w);
      py[j] = m < M ? yy : -1000000;       // an invalid row fails every bounds test
      px[j] = (int)(p - (int64_t)yy * cg.w);
      oa[j] = (uint32_t)(mm * cg.c_pad);
    } else {
      oa[j] = m < M ? (uint32_t)(m * lda + ca[j] * 16) : OOB;
    }
  }
#pragma unroll
  for (int j = 0; j < IW; ++j) {
    const int row = (wave * IW + j) * 8 + lrow;
    cw[j] = pch ^ swz_f(row);
    const int64_t n = n0 + row;
    ow[j] = n < N ? (uint32_t)(n * ldw + cw[j] * 16) : OOB;
  }

  auto dma_slice = [&](int64_t kt, int8_t* stage) {
    const int64_t k0 = kt * BK;
    int8_t* sa = stage;
    int8_t* sw = stage + BM * BK;
    if constexpr (CONVM == 1) {
      // C_pad % 128 == 0: the whole slice is one tap
      const int64_t tap = k0 / cg.c_pad;
      const int64_t c0 = k0 - tap * cg.c_pad;
      const int dy = (int)(tap / 3) - 1, dx = (int)(tap % 3) - 1;
      const int64_t delta = ((int64_t)dy * cg.w + dx) * cg.c_pad + c0;
      const bool kin = k0 < K;
#pragma unroll
      for (int j = 0; j < IA; ++j) {
        const int sy = py[j] + dy, sx = px[j] + dx;
        const bool ok = kin && sy >= 0 && sy < cg.h && sx >= 0 && sx < cg.w;
        dma16(ra_rsrc, ok ? (uint32_t)(oa[j] + delta + ca[j] * 16) : OOB, sa + ((wave * IA + j) << 10));
      }
    } else if constexpr (CONVM == 2) {
#pragma unroll
      for (int j = 0; j < IA; ++j) {
        const int64_t kb = k0 + ca[j] * 16;
        const int64_t tap = kb / cg.c_pad;
        const int64_t c = kb - tap * cg.c_pad;
        const int dy = (int)(tap / 3) - 1, dx = (int)(tap % 3) - 1;
        const int sy = py[j] + dy, sx = px[j] + dx;
        const bool ok = kb < K && sy >= 0 && sy < cg.h && sx >= 0 && sx < cg.w;
        const int64_t delta = ((int64_t)dy * cg.w + dx) * cg.c_pad + c;
        dma16(ra_rsrc, ok ? (uint32_t)(oa[j] + delta) : OOB, sa + ((wave * IA + j) << 10));
      }
    } else {
      if (KFULL) {                         // K % 128 == 0: the per-slot offsets are constant
#pragma unroll
        for (int j = 0; j < IA; ++j) dma16(ra_rsrc, oa[j], sa + ((wave * IA + j) << 10), (uint32_t)k0);
      } else {
#pragma unroll
        for (int j = 0; j < IA; ++j) {
          const bool ok = oa[j] != OOB && k0 + ca[j] * 16 < K;
          dma16(ra_rsrc, ok ? oa[j] + (uint32_t)k0 : OOB, sa + ((wave * IA + j) << 10));
        }
      }
    }
    if (KFULL) {
#pragma unroll
      for (int j = 0; j < IW; ++j) dma16(rw_rsrc, ow[j], sw + ((wave * IW + j) << 10), (uint32_t)k0);
    } else {
#pragma unroll
      for (int j = 0; j < IW; ++j) {
        const bool ok = ow[j] != OOB && k0 + cw[j] * 16 < K;
        dma16(rw_rsrc, ok ? ow[j] + (uint32_t)k0 : OOB, sw + ((wave * IW + j) << 10));
      }
    }
  };

  // Fragments of one 32-deep k sub-step ks (4 per slice): lane l holds 16 bytes of row
  // (frag base + l % 32) at logical chunk 2 * ks + l / 32. Two register sets alternate: while the
  // MFMAs of sub-step ks run, the fragments of sub-step ks + 1 are read into the other set.
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

  i32x16 acc[FN][FM];
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int i = 0; i < FM; ++i) acc[j][i] = i32x16{};
  auto mfmas = [&](int set) {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int i = 0; i < FM; ++i) acc[j][i] = mfma32x32x32(fw[set][j], fa[set][i], acc[j][i]);
  };

  const int64_t nk = (K + BK - 1) / BK;
  dma_slice(0, lds0);
  if (nk > 1) dma_slice(1, lds1);
  if (nk > 1) {
    // slice 0 landed (the DMA completes in order): wait for all but slice 1's loads
    if constexpr (IA + IW == 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    else if constexpr (IA + IW == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else if constexpr (IA + IW == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  __syncthreads();
  read_frags(lds0, 0, 0);

  // Pinned order inside each sub-step: the next sub-step's fragment reads are spread between this
  // sub-step's MFMAs (one read per NMF / NRD MFMAs), so no MFMA waits on LDS.
  constexpr int NMF = FM * FN, NRD = FM + FN, NDMA = IA + IW;
  auto pin_reads = [&]() { PinGroups<SG_DS_READ, NRD, NMF, 0>::emit(); };
  auto substep = [&](const int8_t* stage, int ks_next, int set_next, int set) {
    read_frags(stage, ks_next, set_next);
    mfmas(set);
    pin_reads();
    __builtin_amdgcn_sched_barrier(0);
  };

  // One slice = sub-steps 0..3 (sets 0,1,0,1). The barrier sits between sub-steps 2 and 3: by then
  // every wave has read all of this slice's fragments, so its stage can take the DMA of slice kt+2,
  // and slice kt+1 (waited for just before) is complete for the reads during sub-step 3. The loop
  // body is branch-free; the last two slices (no DMA left to issue) are peeled.
  auto slice = [&](int64_t kt, auto dma_tag, auto next_tag) {
    constexpr bool DMA = decltype(dma_tag)::value, NEXT = decltype(next_tag)::value;
    int8_t* cur = lds + (kt & 1) * STAGE;
    const int8_t* nxt = lds + ((kt + 1) & 1) * STAGE;
    substep(cur, 1, 1, 0);
    substep(cur, 2, 0, 1);
    substep(cur, 3, 1, 0);
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (DMA) dma_slice(kt + 2, cur);
    if constexpr (NEXT) read_frags(nxt, 0, 0);
    mfmas(1);
    // DMA issue spread over the last sub-step's MFMAs
    if constexpr (DMA) PinGroups<SG_VMEM_READ, NDMA, NMF, 0>::emit();
    __builtin_amdgcn_sched_barrier(0);
  };
  using T_ = std::integral_constant<bool, true>;
  using F_ = std::integral_constant<bool, false>;
  int64_t kt = 0;
  for (; kt + 2 < nk; ++kt) slice(kt, T_{}, T_{});
  if (kt + 1 < nk) slice(kt++, F_{}, T_{});
  slice(kt, F_{}, F_{});
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Epilogue through LDS. The 32x32 accumulator of tile (j, i) holds, in lane l, output row
  // m = i * 32 + l % 32 of the wave tile and, in element 4 * g + r, column 8 * g + 4 * (l / 32) + r of
  // column block j. Each accumulator block goes to a per-wave LDS staging area as 32 int32 rows of
  // 32 columns (pitch 144 bytes: conflict-free for these 16-byte writes and reads), and is read back
  // four consecutive columns per lane, eight lanes per row, for the epilogue: every store instruction
  // writes whole contiguous row pieces instead of 4 columns of 64 different rows.
  constexpr int PITCH = 144;
  static_assert(NW * 32 * PITCH <= 2 * STAGE, "staging does not fit in LDS");
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();                       // every wave is done with the K-loop's LDS stages
  int8_t* stg = lds0 + wave * 32 * PITCH;
  int calib = 0;
  // uniform: the whole tile is inside M x N and the output rows take 4-wide vector stores
  const bool full = m0 + BM <= M && n0 + BN <= N && (EPI == EPI_CALIB || e.vec_ok);
  const int rsub = lane >> 3;            // read-back: row rr * 8 + rsub, columns 4 * (lane & 7) .. +3
  const int cq = lane & 7;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t n = n0 + wn * TN + j * 32 + cq * 4;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const i32x4 v = {acc[j][i][4 * g], acc[j][i][4 * g + 1], acc[j][i][4 * g + 2], acc[j][i][4 * g + 3]};
        *reinterpret_cast<i32x4*>(stg + (lane & 31) * PITCH + (8 * g + 4 * (lane >> 5)) * 4) = v;
      }
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int row = rr * 8 + rsub;
        const i32x4 v = *reinterpret_cast<const i32x4*>(stg + row * PITCH + cq * 16);
        const int64_t m = m0 + wm * TM + i * 32 + row;
        const float sxm = sx_pre[DQ ? i * 4 + rr : 0];
        if (full) epilogue4<EPI, true>(e, m, n, M, N, v, calib, cols_pre[j], sxm);
        else epilogue4<EPI, false>(e, m, n, M, N, v, calib, cols_pre[j], sxm);
      }
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
  const EpiCols<EPI> cols(e, n0 + 4 * (lane >> 4), N);
  const int64_t mrow = m0 + (lane & 15);
  float sxm = 0.0f;
  if constexpr (EPI == EPI_DQ_F32 || EPI == EPI_DQ_BF16 || EPI == EPI_DQ_F16) sxm = mrow < M ? e.sx[mrow] : 0.0f;
  epilogue4<EPI>(e, mrow, n0 + 4 * (lane >> 4), M, N, acc, calib, cols, sxm);
  calib_flush<EPI>(e, calib);
}

// ------------------------------------------------------------------------------ dispatch
struct TileCfg {
  int bm, bn, waves;
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

// Tile choice, from a sweep of every tile shape over the BASELINE shapes on MI355X: 256 x 256 tiles
// with 8 waves (two per SIMD, one workgroup per CU) win from about 1.75 rounds of such tiles; 128 x 128
// tiles (two workgroups per CU) win whenever they fill the CUs once; 64 x 64 tiles win for smaller
// problems and for N <= 64.
TileCfg pick_tile(int64_t M, int64_t N) {
  // XDNA_GEMM_TILE=<bm>x<bn> forces a tile shape (tile sweeps); ignored unless it names a built one
  if (const char* env = std::getenv("XDNA_GEMM_TILE")) {
    int bm = 0, bn = 0, waves = 4;
    const int got = std::sscanf(env, "%dx%dw%d", &bm, &bn, &waves);
    if (got >= 2 && ((bm == 256 && bn == 256 && (waves == 4 || waves == 8)) ||
                     (waves == 4 && ((bm == 256 && bn == 128) || (bm == 128 && (bn == 256 || bn == 128)) ||
                                     (bm == 64 && bn == 64)))))
      return {bm, bn, waves};
  }
  const int64_t cus = num_cus();
  if (M <= 64 || N <= 64) return {64, 64, 4};
  const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256);
  const int64_t t128 = ((M + 127) / 128) * ((N + 127) / 128);
  if (4 * t256 >= 7 * cus) return {256, 256, 8};
  if (t128 >= cus) return {128, 128, 4};
  return {64, 64, 4};
}

// Buffer resources address at most 2 GB; larger operands are processed in row chunks.
constexpr int64_t MAX_BUF = 0x40000000;   // 1 GB per resource

template <int CONVM, int EPI>
int launch_tiles(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K,
                 ConvGeom cg, const EpiArgs& e, hipStream_t st) {
  const TileCfg t = pick_tile(M, N);
  const int64_t tiles = ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
  if (tiles >= (1ll << 31)) {
    set_error("launch_mm: too many tiles");
    return XDNA_EINVAL;
  }
  dim3 grid((unsigned)tiles, 1, 1);
  const bool kfull = K % 128 == 0;
#define XDNA_TILE_W(BM_, BN_, WM_, WN_)                                                                       \
  if (kfull) mm_tile_kernel<BM_, BN_, WM_, WN_, CONVM, EPI, true><<<grid, WM_ * WN_ * 64, 0, st>>>(a, lda, w, ldw, M, N, K, cg, e); \
  else mm_tile_kernel<BM_, BN_, WM_, WN_, CONVM, EPI, false><<<grid, WM_ * WN_ * 64, 0, st>>>(a, lda, w, ldw, M, N, K, cg, e);
#define XDNA_TILE(BM_, BN_) XDNA_TILE_W(BM_, BN_, 2, 2)
  if (t.bm == 256 && t.bn == 256 && t.waves == 8) {
    XDNA_TILE_W(256, 256, 2, 4)
  } else if (t.bm == 256 && t.bn == 256) {
    XDNA_TILE(256, 256)
  } else if (t.bm == 256) {
    XDNA_TILE(256, 128)
  } else if (t.bn == 256) {
    XDNA_TILE(128, 256)
  } else if (t.bm == 128) {
    XDNA_TILE(128, 128)
  } else {
    XDNA_TILE(64, 64)
  }
#undef XDNA_TILE
#undef XDNA_TILE_W
  return launch_status("mm_tile");
}

// Output pointer of row block m0 / column block n0 of an epilogue.
inline EpiArgs shift_epi(const EpiArgs& e, int out_bytes, int64_t m0, int64_t n0) {
  EpiArgs r = e;
  if (r.out) r.out = reinterpret_cast<char*>(r.out) + (m0 * e.ldo + n0) * out_bytes;
  if (r.sx) r.sx += m0;
  if (r.sw) r.sw += n0;
  if (r.bias) r.bias += n0;
  return r;
}

template <int EPI>
constexpr int out_bytes() {
  return EPI == EPI_I32 ? 4 : EPI == EPI_DQ_F32 ? 4 : (EPI == EPI_DQ_BF16 || EPI == EPI_DQ_F16) ? 2 : 1;
}

template <int EPI>
int launch_gemm(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int64_t M, int64_t N, int64_t K,
                const EpiArgs& e, hipStream_t st) {
  if (M <= 64) {
    // weight streaming: waves split K into 128-byte multiples
    constexpr int WAVES = 8, U = 2;
    const int64_t slices = (K + 127) / 128;
    const int64_t kper = ((slices + WAVES - 1) / WAVES) * 128;
    dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + 15) / 16), 1);
    mm_small_kernel<WAVES, U, EPI><<<grid, WAVES * 64, 0, st>>>(a, lda, w, ldw, M, N, K, kper, e);
    return launch_status("mm_small");
  }
  const int64_t mrows = std::max<int64_t>(256, (MAX_BUF / lda) / 256 * 256);
  const int64_t nrows = std::max<int64_t>(256, (MAX_BUF / ldw) / 256 * 256);
  for (int64_t m0 = 0; m0 < M; m0 += mrows) {
    for (int64_t n0 = 0; n0 < N; n0 += nrows) {
      const int64_t mc = std::min(mrows, M - m0), nc = std::min(nrows, N - n0);
      int rc = launch_tiles<0, EPI>(a + m0 * lda, lda, w + n0 * ldw, ldw, mc, nc, K, ConvGeom{},
                                    shift_epi(e, out_bytes<EPI>(), m0, n0), st);
      if (rc) return rc;
    }
  }
  return XDNA_OK;
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
  ConvGeom cg{h, w, c_pad};
  for (int64_t b0 = 0; b0 < nb; b0 += imgs) {
    const int64_t bc = std::min(imgs, nb - b0);
    const EpiArgs eb = shift_epi(e, 1, b0 * h * w, 0);
    const int8_t* xb = x + b0 * per_img;
    int rc = (c_pad % 128 == 0) ? launch_tiles<1, EPI>(xb, c_pad, wq, K, bc * h * w, co, K, cg, eb, st)
                                : launch_tiles<2, EPI>(xb, c_pad, wq, K, bc * h * w, co, K, cg, eb, st);
    if (rc) return rc;
  }
  return XDNA_OK;
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
  return launch_gemm<EPI_I32>(a, lda, w, ldw, m, n, k, e, as_stream(stream));
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
  if (y_dtype == XDNA_F32) return launch_gemm<EPI_DQ_F32>(a, lda, w, ldw, m, n, k, e, st);
  if (y_dtype == XDNA_BF16) return launch_gemm<EPI_DQ_BF16>(a, lda, w, ldw, m, n, k, e, st);
  return launch_gemm<EPI_DQ_F16>(a, lda, w, ldw, m, n, k, e, st);
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
  e.vec_ok = (co % 4 == 0) && aligned(y, 4);
  return launch_conv<EPI_REQUANT>(x, nb, h, w, c_pad, wq, co, e, st);
}

}  // extern "C"
