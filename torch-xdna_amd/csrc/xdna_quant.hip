// Quantize, dequantize and layout kernels of the int8 hot path (gfx950).
//
//  * quant_rows: per-row symmetric int8 (torch_xdna/runtime.py:145-148, :366-368, :64-65). One
//    group of TPR threads per row keeps the row in registers, so the row is read from HBM once:
//    a coalesced 16-byte-per-lane load, a wavefront max reduction, then the divide/round/clamp.
//  * conv_quant_nhwc: per-image amax (conv.py:45) as a grid-wide reduction, then the quantize
//    fused with the NCHW -> NHWC transpose through LDS, so the int8 conv input is written once in
//    the layout the implicit GEMM reads.
//  * conv_weight_pack: quantize-once of a conv weight into [Co][9][Ci_pad] (conv.py:58-60).
//  * conv_dequant: NHWC int8 -> NCHW float with q * (scale[o] * sx[b]) + bias (conv.py:48-50).
//
// All floating-point arithmetic here is compiled without contraction (-ffp-contract=off), so
// every product and sum rounds once as in torch's CPU kernels.
#include <algorithm>
#include <mutex>
#include <string>

#include "xdna_common.h"

namespace xdna {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

int device_cus() {
  static int cache[64] = {0};              // per device; concurrent first calls store the same value
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    hipDeviceProp_t prop;
    cache[dev] = hipGetDeviceProperties(&prop, dev) == hipSuccess ? prop.multiProcessorCount : 256;
  }
  return cache[dev];
}

int launch_status(const char* where) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string(where) + ": " + hipGetErrorString(e));
    return static_cast<int>(e);
  }
  return XDNA_OK;
}

// ------------------------------------------------------------------------------ quant_rows
// The larger of two magnitudes (values with the sign bit clear: |x|, or maxima of them) as their bit
// patterns order: a NaN (above +inf) wins, so it propagates as torch.amax propagates it (fmaxf would drop it).
__device__ __forceinline__ float mag_max(float a, float b) {
  return __uint_as_float(max(__float_as_uint(a), __float_as_uint(b)));
}

// Masks that keep the first `valid` bytes of a packed 16-byte group (0..16): padding channels read as 0.0 quantize
// to 0 only while the scale is finite (0 * (1 / NaN) would give -127), so their bytes are cleared instead.
__device__ __forceinline__ void valid_masks(int valid, uint32_t (&m)[4]) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int k = valid - 4 * g;
    m[g] = k >= 4 ? 0xffffffffu : k <= 0 ? 0u : (0xffffffffu >> (32 - 8 * k));
  }
}

// Max of the magnitudes v over the group's TPR threads (one wave, or the whole block through LDS); NaN wins.
template <int TPR>
__device__ __forceinline__ float group_max(float v, float* red) {
  v = __int_as_float(wave_max_i(__float_as_int(v)));      // magnitudes order as their (non-negative) bits
  if constexpr (TPR == 64) {
    return v;
  } else {
    constexpr int W = TPR / 64;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;          // TPR == blockDim.x for TPR > 64
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int i = 1; i < W; ++i) m = mag_max(m, red[i]);
    return m;
  }
}

// max |x| over the row's TPR threads (one wave, or the whole block through LDS), as a float.
template <int DT, int TPR>
__device__ __forceinline__ float group_absmax(const AbsMaxBits<DT>& a, int* red) {
  int v = wave_max_i(a.lane_bits());
  if constexpr (TPR > 64) {
    constexpr int W = TPR / 64;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;          // TPR == blockDim.x for TPR > 64
    if (lane == 0) red[wave] = v;
    __syncthreads();
    v = red[0];
#pragma unroll
    for (int i = 1; i < W; ++i) v = max(v, red[i]);
  }
  return bits_to_abs<DT>(v);
}

// Vector path: k % VEC == 0, ld_x % VEC == 0, x 16-byte aligned, ld_q % 16 == 0, q aligned.
// Rows of up to TPR * MAXV vectors stay in registers; longer rows are read twice.
template <int DT, int TPR, int MAXV>
__global__ __launch_bounds__(256) void quant_rows_vec_kernel(const void* __restrict__ x, int64_t rows, int64_t k,
                                                             int64_t ld_x, int8_t* __restrict__ q, int64_t ld_q,
                                                             int64_t k_pad, float* __restrict__ s) {
  using V = Vec16<DT>;
  constexpr int VEC = V::N;
  constexpr int ESZ = (DT == XDNA_F32) ? 4 : 2;
  __shared__ int red[4];
  const int groups = 256 / TPR;
  const int64_t row = (int64_t)blockIdx.x * groups + threadIdx.x / TPR;
  const int t = threadIdx.x % TPR;
  const bool active = row < rows;
  const int64_t nvec = k / VEC;
  const char* xr = reinterpret_cast<const char*>(x) + (active ? row : 0) * ld_x * ESZ;
  int8_t* qr = q + (active ? row : 0) * ld_q;

  V v[MAXV];
  AbsMaxBits<DT> am;
  const bool cached = nvec <= (int64_t)TPR * MAXV;
  if (active) {
    if (cached) {
#pragma unroll
      for (int j = 0; j < MAXV; ++j) {
        int64_t iv = t + (int64_t)j * TPR;
        if (iv < nvec) v[j].raw = *reinterpret_cast<const uint4*>(xr + iv * 16);
        else v[j].raw = make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < MAXV; ++j) am.add(v[j]);
    } else {
      for (int64_t iv = t; iv < nvec; iv += TPR) {
        V u;
        u.raw = *reinterpret_cast<const uint4*>(xr + iv * 16);
        am.add(u);
      }
    }
  }
  const float amax = group_absmax<DT, TPR>(am, red);
  if (!active) return;
  const float sc = scale_from_amax(amax);
  const float rc = 1.0f / sc;
  if (t == 0) s[row] = sc;

  auto emit = [&](const V& u, int64_t iv) {
    float f[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) f[e] = u.get(e);
    uint32_t w[VEC / 4];
    quant_pack<VEC>(f, sc, rc, w);
    if constexpr (VEC == 8) *reinterpret_cast<uint2*>(qr + iv * VEC) = make_uint2(w[0], w[1]);
    else *reinterpret_cast<uint32_t*>(qr + iv * VEC) = w[0];
  };
  if (cached) {
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
      int64_t iv = t + (int64_t)j * TPR;
      if (iv < nvec) emit(v[j], iv);
    }
  } else {
    for (int64_t iv = t; iv < nvec; iv += TPR) {
      V u;
      u.raw = *reinterpret_cast<const uint4*>(xr + iv * 16);
      emit(u, iv);
    }
  }
  for (int64_t c = k + t; c < k_pad; c += TPR) qr[c] = 0;
}

// Rows of up to 1024 * G elements with k % 16 == 0: one wavefront per row (four rows per block), the
// row in registers. Lane t owns groups t, t + 64, ... of 16 consecutive elements (two or four 16-byte
// loads), so each quantized group leaves as one 16-byte store; no barrier, the row max is a wave
// reduction. NT: the input is read with non-temporal loads, for inputs too large to stay in the
// 256 MB Infinity Cache (measured on MI355X: 64 us instead of 70 us for 8192 x 14336 bf16; on inputs
// that fit, the cached loads win).
template <int DT, int G, bool NT>
__global__ __launch_bounds__(256) void quant_rows_wave_kernel(const void* __restrict__ x, int64_t rows, int64_t k,
                                                              int64_t ld_x, int8_t* __restrict__ q, int64_t ld_q,
                                                              int64_t k_pad, float* __restrict__ s) {
  using V = Vec16<DT>;
  constexpr int VEC = V::N;
  constexpr int ESZ = (DT == XDNA_F32) ? 4 : 2;
  constexpr int LPG = 16 / VEC;          // 16-byte loads per group of 16 elements
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;               // wave-uniform, no barrier below
  const int t = threadIdx.x & 63;
  const int ng = (int)(k / 16);          // k < 2^31 (checked by the launcher)
  const char* xr = reinterpret_cast<const char*>(x) + row * ld_x * ESZ;
  int8_t* qr = q + row * ld_q;
  // the row as a buffer resource: groups past its end read zeros without a branch, so every load of
  // the row is in flight before the first use
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(xr, (uint32_t)(k * ESZ));
  V v[G][LPG];
  AbsMaxBits<DT> am;
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const uint32_t off = (uint32_t)(t + j * 64) * (16 * ESZ);
#pragma unroll
    for (int l = 0; l < LPG; ++l) v[j][l].raw = buf_load_u4<NT>(rr, off + l * 16);
  }
#pragma unroll
  for (int j = 0; j < G; ++j)
#pragma unroll
    for (int l = 0; l < LPG; ++l) am.add(v[j][l]);
  const float amax = bits_to_abs<DT>(wave_max_i(am.lane_bits()));
  const float sc = scale_from_amax(amax);
  const float rc = 1.0f / sc;
  if (t == 0) s[row] = sc;
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const int gi = t + j * 64;
    if (gi < ng) {
      float f[16];
#pragma unroll
      for (int l = 0; l < LPG; ++l)
#pragma unroll
        for (int e = 0; e < VEC; ++e) f[l * VEC + e] = v[j][l].get(e);
      uint32_t w[4];
      quant_pack<16>(f, sc, rc, w);
      *reinterpret_cast<uint4*>(qr + (int64_t)gi * 16) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
  for (int64_t c = k + t; c < k_pad; c += 64) qr[c] = 0;
}

// Rows of more than 2048 (up to 16 * 256 * G) elements with k % 16 == 0: one block of 256 threads per row;
// thread t owns groups t, t + 256, ... of 16 consecutive elements, read as raw buffer loads (past the row's
// end they read zeros; non-temporal under NT) and written as one 16-byte store each; the four waves' maxima
// meet in LDS (one barrier). Many small blocks in flight keep HBM busier than persistent blocks that
// prefetch their next row: with one row per block the registers of a second row are not needed, so more
// blocks are resident (bf16, G 4: 8192 x 14336 64.2 us against 67.2 us persistent, 8192 x 4096 20.0-21.1
// against 21.4, 3000 x 3072 8.5 against 8.8; float32 2000 x 8192 16.2 against 16.9, all before the second
// buffer was dropped). (A wave per row holds such a row in up to 224 registers.) NTS: the int8 rows leave as
// non-temporal stores, for outputs that do not stay in the caches anyway (at least 16 MB): the kernel then reads
// and writes HBM like a plain stream of its bytes (bf16 8192 x 4096 measured 16.5 against 20.0 us, 0.76 of
// 8 TB/s; 8192 x 14336 with non-temporal loads 62.3 against 64.3 us, where a copy-like stream of the same
// bytes with no arithmetic takes 62.2 us).
template <int DT, int G, bool NT, bool NTS>
__global__ __launch_bounds__(256) void quant_rows_block_kernel(const void* __restrict__ x, int64_t k, int64_t ld_x,
                                                               int8_t* __restrict__ q, int64_t ld_q, int64_t k_pad,
                                                               float* __restrict__ s) {
  using V = Vec16<DT>;
  constexpr int VEC = V::N;
  constexpr int ESZ = (DT == XDNA_F32) ? 4 : 2;
  constexpr int LPG = 16 / VEC;
  __shared__ int red[4];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int64_t row = blockIdx.x;
  const int ng = (int)(k / 16);          // at most 256 * G (checked by the launcher)
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(reinterpret_cast<const char*>(x) + row * ld_x * ESZ, (uint32_t)(k * ESZ));
  V v[G][LPG];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const uint32_t off = (uint32_t)(t + j * 256) * (16 * ESZ);
#pragma unroll
    for (int l = 0; l < LPG; ++l) v[j][l].raw = buf_load_u4<NT>(rr, off + l * 16);
  }
  AbsMaxBits<DT> am;
#pragma unroll
  for (int j = 0; j < G; ++j)
#pragma unroll
    for (int l = 0; l < LPG; ++l) am.add(v[j][l]);
  const int wm = wave_max_i(am.lane_bits());
  if (lane == 0) red[wave] = wm;
  __syncthreads();
  const float amax = bits_to_abs<DT>(max(max(red[0], red[1]), max(red[2], red[3])));
  const float sc = scale_from_amax(amax);
  const float rc = 1.0f / sc;
  if (t == 0) s[row] = sc;
  int8_t* qr = q + row * ld_q;
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const int gi = t + j * 256;
    if (gi < ng) {
      float f[16];
#pragma unroll
      for (int l = 0; l < LPG; ++l)
#pragma unroll
        for (int e = 0; e < VEC; ++e) f[l * VEC + e] = v[j][l].get(e);
      uint32_t w[4];
      quant_pack<16>(f, sc, rc, w);
      const u32x4 word = {w[0], w[1], w[2], w[3]};
      if constexpr (NTS) __builtin_nontemporal_store(word, reinterpret_cast<u32x4*>(qr + (int64_t)gi * 16));
      else *reinterpret_cast<u32x4*>(qr + (int64_t)gi * 16) = word;
    }
  }
  for (int64_t c = k + t; c < k_pad; c += 256) qr[c] = 0;
}

// Long rows (more than 512 vectors): persistent blocks of 256 threads walk rows with a grid stride;
// each thread holds up to MAXV 16-byte vectors of a row, and the loads of the block's next row are
// issued before this row's reduction and quantize, so HBM sees a continuous stream. The partial
// maxima go through a double-buffered LDS slot: one barrier per row.
template <int DT, int MAXV>
__global__ __launch_bounds__(256) void quant_rows_stream_kernel(const void* __restrict__ x, int64_t rows, int64_t k,
                                                                int64_t ld_x, int8_t* __restrict__ q, int64_t ld_q,
                                                                int64_t k_pad, float* __restrict__ s) {
  using V = Vec16<DT>;
  constexpr int VEC = V::N;
  constexpr int ESZ = (DT == XDNA_F32) ? 4 : 2;
  __shared__ int red[2][4];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int64_t nvec = k / VEC;
  const int64_t stride = gridDim.x;

  auto load = [&](int64_t row, V (&v)[MAXV]) {
    const char* xr = reinterpret_cast<const char*>(x) + (row < rows ? row : 0) * ld_x * ESZ;
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
      const int64_t iv = t + (int64_t)j * 256;
      v[j].raw = (row < rows && iv < nvec) ? *reinterpret_cast<const uint4*>(xr + iv * 16) : make_uint4(0, 0, 0, 0);
    }
  };
  auto process = [&](int64_t row, const V (&v)[MAXV], int buf) {
    AbsMaxBits<DT> am;
#pragma unroll
    for (int j = 0; j < MAXV; ++j) am.add(v[j]);   // vectors past the row hold zeros
    const int wm = wave_max_i(am.lane_bits());
    if (lane == 0) red[buf][wave] = wm;
    __syncthreads();
    const float amax = bits_to_abs<DT>(max(max(red[buf][0], red[buf][1]), max(red[buf][2], red[buf][3])));
    const float sc = scale_from_amax(amax);
    const float rc = 1.0f / sc;
    if (t == 0) s[row] = sc;
    int8_t* qr = q + row * ld_q;
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
      const int64_t iv = t + (int64_t)j * 256;
      if (iv < nvec) {
        float f[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) f[e] = v[j].get(e);
        uint32_t w[VEC / 4];
        quant_pack<VEC>(f, sc, rc, w);
        if constexpr (VEC == 8) *reinterpret_cast<uint2*>(qr + iv * VEC) = make_uint2(w[0], w[1]);
        else *reinterpret_cast<uint32_t*>(qr + iv * VEC) = w[0];
      }
    }
    for (int64_t c = k + t; c < k_pad; c += 256) qr[c] = 0;
  };

  V va[MAXV], vb[MAXV];
  int64_t row = blockIdx.x;
  load(row, va);
  while (row < rows) {
    load(row + stride, vb);
    process(row, va, 0);
    row += stride;
    if (row >= rows) break;
    load(row + stride, va);
    process(row, vb, 1);
    row += stride;
  }
}

// Scalar path for any k / stride / alignment: one block per row, the row read twice.
template <int DT>
__global__ __launch_bounds__(256) void quant_rows_scalar_kernel(const void* __restrict__ x, int64_t rows, int64_t k,
                                                                int64_t ld_x, int8_t* __restrict__ q, int64_t ld_q,
                                                                int64_t k_pad, float* __restrict__ s) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t base = row * ld_x;
  float amax = 0.0f;
  for (int64_t i = threadIdx.x; i < k; i += 256) amax = mag_max(amax, fabsf(load_as_f32<DT>(x, base + i)));
  amax = group_max<256>(amax, red);
  const float sc = scale_from_amax(amax);
  const float rc = 1.0f / sc;
  if (threadIdx.x == 0) s[row] = sc;
  int8_t* qr = q + row * ld_q;
  for (int64_t i = threadIdx.x; i < k; i += 256) qr[i] = (int8_t)quant1(load_as_f32<DT>(x, base + i), sc, rc);
  for (int64_t i = k + threadIdx.x; i < k_pad; i += 256) qr[i] = 0;
}

// Blocks of a persistent streaming kernel: as many as are resident at once (the runtime's occupancy
// for 256 threads, cached per kernel and device), at most `rows`.
template <auto KERNEL, int THREADS = 256>
unsigned stream_blocks(int64_t rows) {
  static int per_cu[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (per_cu[dev] == 0) {
    int n = 0;
    per_cu[dev] = (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, KERNEL, THREADS, 0) == hipSuccess && n > 0) ? n : 1;
  }
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(rows, (int64_t)per_cu[dev] * device_cus()));
}

template <int DT>
int launch_quant_rows(const void* x, int64_t rows, int64_t k, int64_t ld_x, int8_t* q, int64_t ld_q, int64_t k_pad,
                      float* s, hipStream_t st) {
  constexpr int VEC = (DT == XDNA_F32) ? 4 : 8;
  const bool vec_ok = (k % VEC == 0) && (ld_x % VEC == 0) && aligned(x, 16) && aligned(q, 16) && (ld_q % 16 == 0);
  if (!vec_ok) {
    quant_rows_scalar_kernel<DT><<<dim3((unsigned)rows), 256, 0, st>>>(x, rows, k, ld_x, q, ld_q, k_pad, s);
    return launch_status("quant_rows_scalar");
  }
  const int64_t nvec = k / VEC;
  constexpr int ESZ = (DT == XDNA_F32) ? 4 : 2;
  // One wavefront per row with 16-element groups for rows of up to 2048 elements; longer rows take one
  // 256-thread block per row (quant_rows_block_kernel; the figures below were measured with its earlier
  // persistent form, which one block per row beats).
  // Measured on MI355X, bf16, against a wave per row: 8192 x 14336 67.4 us against 74.9, 8192 x 4096 21.6
  // against 24.6, 3000 x 3072 8.8 against 10.7, 1024 x 3072 4.8 against 6.3, the decode rows (1 and 16 of
  // 4096 and 14336) 4.0 against 4.3 and 11.2 us; at 2048 elements the wave per row wins (14.0 against 15.9
  // us on 8192 rows).
  const int64_t gpl = cdiv(k / 16, 64);  // groups per lane of a wave
  const int64_t ngr = k / 16;            // groups of the row
  const bool few = rows < 512;
  if (k % 16 == 0 && gpl > 2 && ngr <= 256 * (DT == XDNA_F32 ? 4 : 8) && rows < (int64_t(1) << 31)) {
    const bool nt = rows * k * ESZ >= (int64_t(128) << 20);   // half the Infinity Cache
    const bool nts = rows * k_pad >= (int64_t(16) << 20);       // an output well beyond the L2 caches
    const dim3 bg((unsigned)rows);                              // one block per row
#define XDNA_QB(G_)                                                                                           \
  {                                                                                                           \
    if (nt) quant_rows_block_kernel<DT, G_, true, true><<<bg, 256, 0, st>>>(x, k, ld_x, q, ld_q, k_pad, s);   \
    else if (nts) quant_rows_block_kernel<DT, G_, false, true><<<bg, 256, 0, st>>>(x, k, ld_x, q, ld_q, k_pad, s); \
    else quant_rows_block_kernel<DT, G_, false, false><<<bg, 256, 0, st>>>(x, k, ld_x, q, ld_q, k_pad, s);    \
  }
    if (ngr <= 256) {
      XDNA_QB(1)
    } else if (ngr <= 512) {
      XDNA_QB(2)
    } else if (ngr <= 1024) {
      XDNA_QB(4)
    } else if constexpr (DT != XDNA_F32) {
      XDNA_QB(8)
    }
#undef XDNA_QB
    return launch_status("quant_rows");
  }
  if (k % 16 == 0 && k < (int64_t(1) << 31) && gpl <= 2) {
    const bool nt = rows * k * (DT == XDNA_F32 ? 4 : 2) >= (int64_t(128) << 20);   // half the Infinity Cache
    // one wave per row at any row count: a grid of many more waves than are resident keeps more loads in
    // flight than persistent waves that prefetch their next row (measured against such a kernel, bf16:
    // 3000 x 1024 4.9 against 5.1 us, 8192 x 2048 12.6 against 13.8 us, 8192 x 1024 8.2 against 8.5 us;
    // float32 4096 x 2048 10.9 against 11.7 us)
    const dim3 grid((unsigned)cdiv(rows, 4));
#define XDNA_QW(G_)                                                                                     \
  if (nt) quant_rows_wave_kernel<DT, G_, true><<<grid, 256, 0, st>>>(x, rows, k, ld_x, q, ld_q, k_pad, s); \
  else quant_rows_wave_kernel<DT, G_, false><<<grid, 256, 0, st>>>(x, rows, k, ld_x, q, ld_q, k_pad, s);
    if (gpl <= 1) {
      XDNA_QW(1)
    } else {
      XDNA_QW(2)
    }
#undef XDNA_QW
    return launch_status("quant_rows");
  }
  if (nvec <= 64 * 8 && !few) {  // one wavefront per row, four rows per block
    quant_rows_vec_kernel<DT, 64, 8><<<dim3((unsigned)cdiv(rows, 4)), 256, 0, st>>>(x, rows, k, ld_x, q, ld_q, k_pad, s);
  } else if (nvec <= 256 * 8) {
    quant_rows_stream_kernel<DT, 8><<<dim3(stream_blocks<quant_rows_stream_kernel<DT, 8>>(rows)), 256, 0, st>>>(
        x, rows, k, ld_x, q, ld_q, k_pad, s);
  } else if (nvec <= 256 * 16) {
    quant_rows_stream_kernel<DT, 16><<<dim3(stream_blocks<quant_rows_stream_kernel<DT, 16>>(rows)), 256, 0, st>>>(
        x, rows, k, ld_x, q, ld_q, k_pad, s);
  } else {               // one block per row, the row read twice
    quant_rows_vec_kernel<DT, 256, 16><<<dim3((unsigned)rows), 256, 0, st>>>(x, rows, k, ld_x, q, ld_q, k_pad, s);
  }
  return launch_status("quant_rows");
}

// ------------------------------------------------------------------------------ fills / pads
__global__ void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t v) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ void pad_rows_i8_kernel(const int8_t* __restrict__ src, int64_t rows, int64_t cols, int64_t ld_src,
                                   int8_t* __restrict__ dst, int64_t ld_dst, int64_t cols_pad) {
  const int64_t row = blockIdx.y;
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < cols_pad; c += (int64_t)gridDim.x * blockDim.x)
    dst[row * ld_dst + c] = c < cols ? src[row * ld_src + c] : (int8_t)0;
}

// ------------------------------------------------------------------------------ conv quantize
// Per-image max |x| in two steps without atomics: a first kernel with grid (parts, nb), parts <=
// AMAX_PARTS, writes each block's max to parts_out[b * AMAX_PARTS + block]; the kernel that needs
// the image's max reduces those `parts` values (image_amax). The caller's scratch holds nb *
// AMAX_PARTS floats.
constexpr int AMAX_PARTS = XDNA_AMAX_WS_PER_IMAGE;

__device__ __forceinline__ float image_amax(const float* __restrict__ parts, int64_t b, int nparts, float* red) {
  const float m = threadIdx.x < nparts ? parts[b * AMAX_PARTS + threadIdx.x] : 0.0f;
  return group_max<256>(m, red);
}

// Grid (parts, nb) of 1024-thread blocks (16 waves per CU at one block per CU), parts chosen by the launcher
// so that the whole grid is one round of resident blocks (a second, partial round leaves most CUs idle:
// 2048 blocks of 256 threads read 537 MB at 3.8 TB/s). Each lane keeps U 16-byte loads in flight per step
// (a branch-free buffer resource over the image: past its end they read zeros; non-temporal under NT);
// magnitude bits keep a NaN as torch.amax does.
template <int DT, bool NT>
__global__ __launch_bounds__(1024) void image_absmax_kernel(const void* __restrict__ x, int64_t per,
                                                            float* __restrict__ parts) {
  __shared__ float red[16];
  const int64_t b = blockIdx.y;
  constexpr int ESZ = (DT == XDNA_F32) ? 4 : 2;
  const char* xb = reinterpret_cast<const char*>(x) + b * per * ESZ;
  const int t = threadIdx.x;
  float m = 0.0f;
  const bool vec_ok = ((per * ESZ) % 16 == 0) && aligned(x, 16) && per * ESZ < (int64_t(1) << 31);
  if (vec_ok) {
    constexpr int U = 8;
    using V = Vec16<DT>;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(xb, (uint32_t)(per * ESZ));
    // 32-bit: nvec < 2^27, so every offset below stays under 2^32
    const uint32_t nvec = (uint32_t)(per * ESZ / 16);
    const uint32_t step = gridDim.x * 1024u * U;
    AbsMaxBits<DT> am;
    for (uint32_t base = blockIdx.x * 1024u * U + t; base < nvec; base += step) {
      V u[U];
#pragma unroll
      for (int j = 0; j < U; ++j) u[j].raw = buf_load_u4<NT>(r, (base + j * 1024u) * 16u);
#pragma unroll
      for (int j = 0; j < U; ++j) am.add(u[j]);
    }
    m = bits_to_abs<DT>(am.lane_bits());
  } else {
    for (int64_t i = (int64_t)blockIdx.x * 1024 + t; i < per; i += (int64_t)gridDim.x * 1024)
      m = mag_max(m, fabsf(load_as_f32<DT>(xb, i)));
  }
  m = group_max<1024>(m, red);
  if (t == 0) parts[b * AMAX_PARTS + blockIdx.x] = m;
}

// Quantize + NCHW -> NHWC with 16-byte accesses on both sides: a block (256 threads) covers 256
// channels x TP = 16 * PPL pixels (PPL = pixels per 16-byte load: 4 float32, 8 bf16 / fp16). Wave w owns
// channels c0 + 64 w .. + 63; in load i lane l reads channel c0 + 64 w + 16 (l / 16) + i at pixels
// PPL (l % 16) .. + PPL (16 lanes read a channel's 16 PPL contiguous pixels), so each lane ends with 16
// consecutive channels of PPL pixels, quantizes each pixel's 16 channels into one 16-byte LDS word of the
// tile [TP][256] and the tile leaves as 16-byte stores, 256 contiguous channel bytes per pixel.
// Channels past ch read as zeros (quantized 0); needs hw % PPL == 0 and an image below 2 GB.
template <int DT, bool NT>
__global__ __launch_bounds__(256) void conv_quant_nhwc_vec_kernel(const void* __restrict__ x, int64_t ch, int64_t hw,
                                                                  const float* __restrict__ parts, int nparts,
                                                                  int8_t* __restrict__ q, int64_t c_pad,
                                                                  float* __restrict__ sx) {
  constexpr int ESZ = (DT == XDNA_F32) ? 4 : 2;
  constexpr int PPL = 16 / ESZ, TP = 16 * PPL;
  // tile [TP][256] bytes; 16-byte chunk c of row p at chunk c ^ ((p / PPL) % 16): the 16 rows one write
  // instruction spans (PPL apart) and the 16 chunks of a row one read spans hit distinct bank groups
  __shared__ __attribute__((aligned(16))) uint8_t tile[TP * 256];
  __shared__ float red[4];
  using V = Vec16<DT>;
  const int64_t b = blockIdx.z;
  const int64_t p0 = (int64_t)blockIdx.x * TP;
  const int64_t c0 = (int64_t)blockIdx.y * 256;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cl = 64 * wave + 16 * (lane >> 4);             // the lane's first channel within the tile
  const int pl = PPL * (lane & 15);                        // the lane's first pixel within the tile
  const __amdgpu_buffer_rsrc_t r = make_rsrc(reinterpret_cast<const char*>(x) + b * ch * hw * ESZ,
                                             (uint32_t)(ch * hw * ESZ));
  // the tile's loads go out first: they do not depend on the image's scale, whose reduction (a load of
  // the block maxima and a barrier) then overlaps them
  V v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t c = c0 + cl + i;
    v[i].raw = buf_load_u4<NT>(r, c < ch ? (uint32_t)((c * hw + p0 + pl) * ESZ) : OOB);
  }
  const float sc = scale_from_amax(image_amax(parts, b, nparts, red));
  const float rc = 1.0f / sc;
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) sx[b] = sc;
  uint32_t keep[4];
  valid_masks((int)max<int64_t>(0, min<int64_t>(16, ch - (c0 + cl))), keep);
#pragma unroll
  for (int j = 0; j < PPL; ++j) {
    float f[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) f[i] = v[i].get(j);
    uint32_t w[4];
    quant_pack<16>(f, sc, rc, w);
    *reinterpret_cast<uint4*>(&tile[(pl + j) * 256 + (((cl >> 4) ^ (lane & 15)) << 4)]) =
        make_uint4(w[0] & keep[0], w[1] & keep[1], w[2] & keep[2], w[3] & keep[3]);
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < TP / 16; ++j) {
    const int k = threadIdx.x + 256 * j;                    // 16-byte chunk of the tile
    const int pix = k >> 4, part = k & 15;
    const int64_t p = p0 + pix, c = c0 + part * 16;
    if (p < hw && c < c_pad)
      *reinterpret_cast<uint4*>(q + (b * hw + p) * c_pad + c) =
          *reinterpret_cast<const uint4*>(&tile[pix * 256 + ((part ^ ((pix / PPL) & 15)) << 4)]);
  }
}

// Quantize + NCHW -> NHWC for narrow images (c_pad <= 48: RGB inputs, early layers), pixel-major with no
// channel tile: lane i of the block owns PPL consecutive pixels, and per group of 16 channels it reads
// each real channel's PPL pixels with one 16-byte load (channels past ch are not read: they quantize to
// 0), quantizes each pixel's 16 channels and writes them as one 16-byte store. Lanes read consecutive 16
// bytes of a channel and write consecutive pixels. Grid (cdiv(hw, 256 PPL), nb); needs hw % PPL == 0 and
// an image below 2 GB.
template <int DT, bool NT>
__global__ __launch_bounds__(256) void conv_quant_nhwc_narrow_kernel(const void* __restrict__ x, int64_t ch,
                                                                     int64_t hw, const float* __restrict__ parts,
                                                                     int nparts, int8_t* __restrict__ q,
                                                                     int64_t c_pad, float* __restrict__ sx) {
  constexpr int ESZ = (DT == XDNA_F32) ? 4 : 2;
  constexpr int PPL = 16 / ESZ;
  __shared__ float red[4];
  using V = Vec16<DT>;
  const int64_t b = blockIdx.y;
  const int64_t p = ((int64_t)blockIdx.x * 256 + threadIdx.x) * PPL;     // the lane's first pixel
  const __amdgpu_buffer_rsrc_t r = make_rsrc(reinterpret_cast<const char*>(x) + b * ch * hw * ESZ,
                                             (uint32_t)(ch * hw * ESZ));
  const int groups = (int)(c_pad / 16);
  // the first group's loads go out before the image's scale is reduced
  V v[16];
  int nc = (int)min<int64_t>(16, ch);
#pragma unroll
  for (int i = 0; i < 16; ++i)
    v[i].raw = i < nc ? buf_load_u4<NT>(r, (uint32_t)((i * hw + p) * ESZ)) : make_uint4(0, 0, 0, 0);
  const float sc = scale_from_amax(image_amax(parts, b, nparts, red));
  const float rc = 1.0f / sc;
  if (blockIdx.x == 0 && threadIdx.x == 0) sx[b] = sc;
  int8_t* qp = q + (b * hw + p) * c_pad;
  for (int g = 0; g < groups; ++g) {
    if (g > 0) {
      nc = (int)max<int64_t>(0, min<int64_t>(16, ch - 16 * g));
#pragma unroll
      for (int i = 0; i < 16; ++i)
        v[i].raw = i < nc ? buf_load_u4<NT>(r, (uint32_t)(((16 * g + i) * hw + p) * ESZ)) : make_uint4(0, 0, 0, 0);
    }
    uint32_t keep[4];
    valid_masks(nc, keep);
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
      float f[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) f[i] = v[i].get(j);
      uint32_t w[4];
      quant_pack<16>(f, sc, rc, w);
      if (p < hw)
        *reinterpret_cast<uint4*>(qp + j * c_pad + 16 * g) =
            make_uint4(w[0] & keep[0], w[1] & keep[1], w[2] & keep[2], w[3] & keep[3]);
    }
  }
}

// Quantize + NCHW -> NHWC: tile of 64 channels x 64 pixels per block (256 threads). Wave w
// reads channels [w*16, w*16+16) of the tile, lane = pixel, so every global read is 64
// consecutive pixels of one channel; four channels pack into one LDS word per pixel. The
// write-out gives each thread 16 channels of one pixel (a 16-byte store).
template <int DT>
__global__ __launch_bounds__(256) void conv_quant_nhwc_kernel(const void* __restrict__ x, int64_t ch, int64_t hw,
                                                              const float* __restrict__ parts, int nparts,
                                                              int8_t* __restrict__ q, int64_t c_pad,
                                                              float* __restrict__ sx) {
  __shared__ uint32_t tile[64][17];
  __shared__ float red[4];
  const int64_t b = blockIdx.z;
  const int64_t p0 = (int64_t)blockIdx.x * 64;
  const int64_t c0 = (int64_t)blockIdx.y * 64;
  const float sc = scale_from_amax(image_amax(parts, b, nparts, red));
  const float rc = 1.0f / sc;
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) sx[b] = sc;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t p = p0 + lane;
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4) {
    uint32_t packed = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t c = c0 + wave * 16 + c4 * 4 + e;
      int qv = 0;
      if (c < ch && p < hw) qv = quant1(load_as_f32<DT>(x, (b * ch + c) * hw + p), sc, rc);
      packed |= ((uint32_t)(uint8_t)(int8_t)qv) << (8 * e);
    }
    tile[lane][wave * 4 + c4] = packed;
  }
  __syncthreads();
  const int pix = threadIdx.x >> 2;
  const int part = threadIdx.x & 3;
  const int64_t po = p0 + pix;
  const int64_t co = c0 + part * 16;
  if (po < hw && co < c_pad) {
    uint4 v = make_uint4(tile[pix][part * 4 + 0], tile[pix][part * 4 + 1], tile[pix][part * 4 + 2],
                         tile[pix][part * 4 + 3]);
    *reinterpret_cast<uint4*>(q + (b * hw + po) * c_pad + co) = v;
  }
}

// Conv weight quantize-once: one block per output channel.
template <int DT>
__global__ __launch_bounds__(256) void conv_weight_pack_kernel(const void* __restrict__ w, int64_t ci,
                                                               int8_t* __restrict__ wq, int64_t ci_pad,
                                                               float* __restrict__ sw) {
  __shared__ float red[4];
  const int64_t o = blockIdx.x;
  const int64_t per = ci * 9;
  const int64_t base = o * per;
  float m = 0.0f;
  for (int64_t i = threadIdx.x; i < per; i += 256) m = mag_max(m, fabsf(load_as_f32<DT>(w, base + i)));
  m = group_max<256>(m, red);
  const float sc = scale_from_amax(m);
  const float rc = 1.0f / sc;
  if (threadIdx.x == 0) sw[o] = sc;
  int8_t* out = wq + o * 9 * ci_pad;
  for (int64_t i = threadIdx.x; i < 9 * ci_pad; i += 256) {
    const int64_t tap = i / ci_pad, c = i % ci_pad;
    out[i] = c < ci ? (int8_t)quant1(load_as_f32<DT>(w, base + c * 9 + tap), sc, rc) : (int8_t)0;
  }
}

// NHWC q (int8 / uint8) -> NCHW float with 16-byte accesses on both sides: a block covers 256 channels x
// TP = 16 * PPL pixels (PPL = output pixels per 16-byte store: 4 float32, 8 bf16 / fp16). The tile's NHWC
// bytes come in as 16-byte loads into LDS [TP][256]; lane l of wave w then takes channels
// 64 w + 16 (l / 16) .. + 15 of pixels PPL (l % 16) .. + PPL (PPL 16-byte LDS reads) and writes, per
// channel, PPL contiguous outputs as one 16-byte store: y = (float)q * (scale[o] * sx[b]) (+ bias[o]).
// Needs hw % PPL == 0.
template <int DT, bool RELU, bool NT>
__global__ __launch_bounds__(256) void conv_dequant_vec_kernel(const void* __restrict__ qv, int64_t hw, int64_t co,
                                                               const float* __restrict__ scale,
                                                               const float* __restrict__ sx,
                                                               const float* __restrict__ bias, void* __restrict__ y) {
  constexpr int ESZ = (DT == XDNA_F32) ? 4 : 2;
  constexpr int PPL = 16 / ESZ, TP = 16 * PPL;
  __shared__ __attribute__((aligned(16))) uint8_t tile[TP * 256];   // swizzled as in conv_quant_nhwc_vec_kernel
  const int64_t b = blockIdx.z;
  const int64_t p0 = (int64_t)blockIdx.x * TP;
  const int64_t c0 = (int64_t)blockIdx.y * 256;
  const __amdgpu_buffer_rsrc_t r = make_rsrc(reinterpret_cast<const uint8_t*>(qv) + b * hw * co, (uint32_t)(hw * co));
  const bool co16 = co % 16 == 0;
#pragma unroll
  for (int j = 0; j < TP / 16; ++j) {
    const int k = threadIdx.x + 256 * j;
    const int pix = k >> 4, part = k & 15;
    const int64_t p = p0 + pix, c = c0 + part * 16;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (co16) {
      v = buf_load_u4<NT>(r, (p < hw && c < co) ? (uint32_t)(p * co + c) : OOB);
    } else if (p < hw) {        // rows not 16-byte aligned: bytes
      uint8_t by[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) by[e] = c + e < co ? reinterpret_cast<const uint8_t*>(qv)[(b * hw + p) * co + c + e] : 0;
      v = *reinterpret_cast<const uint4*>(by);
    }
    *reinterpret_cast<uint4*>(&tile[pix * 256 + ((part ^ ((pix / PPL) & 15)) << 4)]) = v;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cl = 64 * wave + 16 * (lane >> 4);
  const int pl = PPL * (lane & 15);
  const float sxb = sx[b];
  uint4 bytes[PPL];
#pragma unroll
  for (int j = 0; j < PPL; ++j) bytes[j] = *reinterpret_cast<const uint4*>(&tile[(pl + j) * 256 + (((cl >> 4) ^ (lane & 15)) << 4)]);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t o = c0 + cl + i;
    if (o >= co) break;
    const float f = scale[o] * sxb;
    const float bo = bias ? bias[o] : 0.0f;
    float v[PPL];
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
      const uint8_t raw = reinterpret_cast<const uint8_t*>(&bytes[j])[i];
      const float qf = RELU ? (float)raw : (float)(int8_t)raw;
      float t = qf * f;
      if (bias) t = t + bo;
      v[j] = t;
    }
    const int64_t p = p0 + pl;
    if (p >= hw) continue;
    char* out = reinterpret_cast<char*>(y) + ((b * co + o) * hw + p) * ESZ;
    u32x4 word;
    if constexpr (DT == XDNA_F32) {
      word = __builtin_bit_cast(u32x4, f32x4{v[0], v[1], v[2], v[3]});
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        word[e] = DT == XDNA_BF16 ? f32x2_to_bf16x2_bits(v[2 * e], v[2 * e + 1]) : f32x2_to_f16x2_bits(v[2 * e], v[2 * e + 1]);
    }
    // outputs above 128 MB (NT) do not fit the Infinity Cache: written past it
    if constexpr (NT) __builtin_nontemporal_store(word, reinterpret_cast<u32x4*>(out));
    else *reinterpret_cast<u32x4*>(out) = word;
  }
}

// NHWC q (int8 / uint8) -> NCHW float: y[b, o, p] = (float)q * (scale[o] * sx[b]) (+ bias[o]).
// Tile of 64 pixels x 64 channels; reads 64 contiguous channel bytes per pixel, writes 64
// contiguous pixels per channel.
template <int DT, bool RELU>
__global__ __launch_bounds__(256) void conv_dequant_kernel(const void* __restrict__ qv, int64_t hw, int64_t co,
                                                           const float* __restrict__ scale,
                                                           const float* __restrict__ sx,
                                                           const float* __restrict__ bias, void* __restrict__ y) {
  __shared__ uint8_t tile[64][68];
  const int64_t b = blockIdx.z;
  const int64_t p0 = (int64_t)blockIdx.x * 64;
  const int64_t o0 = (int64_t)blockIdx.y * 64;
  const uint8_t* q = reinterpret_cast<const uint8_t*>(qv);
  // load: thread -> (pixel t/4, 16 channels)
  {
    const int pix = threadIdx.x >> 2;
    const int part = threadIdx.x & 3;
    const int64_t p = p0 + pix;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int64_t o = o0 + part * 16 + e;
      tile[pix][part * 16 + e] = (p < hw && o < co) ? q[(b * hw + p) * co + o] : 0;
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t p = p0 + lane;
  const float sxb = sx[b];
  for (int j = 0; j < 16; ++j) {
    const int oi = wave * 16 + j;
    const int64_t o = o0 + oi;
    if (o >= co || p >= hw) continue;
    const uint8_t raw = tile[lane][oi];
    const float qf = RELU ? (float)raw : (float)(int8_t)raw;
    const float f = scale[o] * sxb;
    float v = qf * f;
    if (bias) v = v + bias[o];
    store_from_f32<DT>(y, (b * co + o) * hw + p, v);
  }
}

// ------------------------------------------------------------------------------ conv chaining
// Between two convs of a chain: the previous conv's NHWC int8 output q (uint8 with ReLU) is
// dequantized as conv_dequant does (q * (scale[o] * sx[b]) (+ bias[o]), cast to the activation
// dtype), optionally 2x2 max-pooled, and quantized per image for the next conv, straight into its
// NHWC int8 layout: the float activation is never written. Dequantize and cast are non-decreasing
// in q (scale * sx > 0), so pooling the integers first gives the same values as pooling the floats.
// relu_y applies a ReLU to the dequantized value (a graph ReLU after a biased conv); a ReLU before
// or after the cast gives the same quantized integers (the cast is monotone and keeps 0).
// Item: one output pixel, 16 channels (item = pixel * ng + group, ng = c_pad / 16); indices within
// an image are 32-bit (the host checks the sizes). PASS 0 (grid (parts, nb), grid-stride over the
// items) writes each block's max |x| to parts_ws; PASS 1 (one item per thread) reduces the image's
// parts, then quantizes (scale as conv_quant_nhwc), channels >= co written as 0.
// PASS 0 keeps, per channel, only the min and max of the (pooled) integers: the dequantize is
// non-decreasing in q, so max |x| over a channel is max(|x(q_min)|, |x(q_max)|). This needs each
// thread's items to share one channel group (grid stride a multiple of ng); otherwise PASS 0
// dequantizes every value.
struct ChainArgs {
  const uint8_t* q;
  uint32_t h, w, co, ho, wo, ng;
  const float* scale;
  const float* bias;
  int relu_y, vec_f;
};

// The (pooled) integers of channels c0 .. c0+15 of output pixel pix of image b (int domain: uint8
// with ReLU, else int8); channels >= co read as the domain's minimum.
template <bool RELU, bool POOL>
__device__ __forceinline__ void chain_q(const ChainArgs& a, int64_t b, uint32_t pix, uint32_t c0, int (&qv)[16]) {
  const uint32_t y = pix / a.wo, x = pix - y * a.wo;
  const uint8_t* img = a.q + (uint64_t)b * a.h * a.w * a.co;
#pragma unroll
  for (int e = 0; e < 16; ++e) qv[e] = RELU ? 0 : -128;
  const bool vec = (a.co % 16 == 0) && (c0 + 16 <= a.co);
#pragma unroll
  for (int d = 0; d < (POOL ? 4 : 1); ++d) {
    const uint32_t sy = POOL ? 2 * y + (d >> 1) : y, sxp = POOL ? 2 * x + (d & 1) : x;
    const uint8_t* src = img + (sy * a.w + sxp) * a.co + c0;
    if (vec) {
      const uint4 raw = *reinterpret_cast<const uint4*>(src);
      const uint32_t words[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t byte = (words[e >> 2] >> (8 * (e & 3))) & 0xffu;
        qv[e] = max(qv[e], RELU ? (int)byte : (int)(int8_t)byte);
      }
    } else if (c0 < a.co) {
      const uint32_t last = a.co - 1 - c0;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint8_t byte = src[min((uint32_t)e, last)];
        if ((uint32_t)e <= last) qv[e] = max(qv[e], RELU ? (int)byte : (int)(int8_t)byte);
      }
    }
  }
}

// scale * sx and bias of channels c0 .. c0+15 (0 past co).
__device__ __forceinline__ void chain_factors(const ChainArgs& a, uint32_t c0, float sxb, float (&f)[16],
                                              float (&bv)[16]) {
  if (a.vec_f && c0 + 16 <= a.co) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float4 s4 = reinterpret_cast<const float4*>(a.scale + c0)[k];
      f[4 * k] = s4.x * sxb; f[4 * k + 1] = s4.y * sxb; f[4 * k + 2] = s4.z * sxb; f[4 * k + 3] = s4.w * sxb;
      float4 b4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (a.bias) b4 = reinterpret_cast<const float4*>(a.bias + c0)[k];
      bv[4 * k] = b4.x; bv[4 * k + 1] = b4.y; bv[4 * k + 2] = b4.z; bv[4 * k + 3] = b4.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const uint32_t o = min(c0 + e, a.co - 1);
      const bool in = c0 + e < a.co;
      f[e] = in ? a.scale[o] * sxb : 0.0f;
      bv[e] = (in && a.bias) ? a.bias[o] : 0.0f;
    }
  }
}

// The raw scale and bias of channels c0 .. c0+15 (0 past co), loaded without the image's factor so the
// loads can go out before anything they would wait for; chain_scale then forms chain_factors' values.
__device__ __forceinline__ void chain_factors_raw(const ChainArgs& a, uint32_t c0, float (&sr)[16], float (&bv)[16]) {
  if (a.vec_f && c0 + 16 <= a.co) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float4 s4 = reinterpret_cast<const float4*>(a.scale + c0)[k];
      sr[4 * k] = s4.x; sr[4 * k + 1] = s4.y; sr[4 * k + 2] = s4.z; sr[4 * k + 3] = s4.w;
      float4 b4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (a.bias) b4 = reinterpret_cast<const float4*>(a.bias + c0)[k];
      bv[4 * k] = b4.x; bv[4 * k + 1] = b4.y; bv[4 * k + 2] = b4.z; bv[4 * k + 3] = b4.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const uint32_t o = min(c0 + e, a.co - 1);
      const bool in = c0 + e < a.co;
      sr[e] = in ? a.scale[o] : 0.0f;
      bv[e] = (in && a.bias) ? a.bias[o] : 0.0f;
    }
  }
}
__device__ __forceinline__ void chain_scale(const ChainArgs& a, uint32_t c0, float sxb, const float (&sr)[16],
                                            float (&f)[16]) {
#pragma unroll
  for (int e = 0; e < 16; ++e) f[e] = c0 + e < a.co ? sr[e] * sxb : 0.0f;
}

// The activation value of integer q: q * f (+ bias), ReLU'd with relu_y, cast to DT (as a float).
template <int DT>
__device__ __forceinline__ float chain_value(int q, float f, float bias, bool has_bias, int relu_y) {
  float t = (float)q * f;
  if (has_bias) t = t + bias;
  if (relu_y) t = __builtin_elementwise_maximum(t, 0.0f);   // IEEE maximum: a NaN stays NaN, as torch.relu keeps it
  if constexpr (DT == XDNA_BF16) t = bf16_bits_to_f32(f32_to_bf16_bits(t));
  if constexpr (DT == XDNA_F16) t = f16_bits_to_f32(f32_to_f16_bits(t));
  return t;
}

// Chaining for channels in whole 16-byte groups whose group count divides 64 (co % 16 == 0, c_pad_next / 16
// a power of two <= 64: every VGG-16 and C3 boundary). A block covers U * 256 consecutive items (pixel,
// channel group) of one image, wave w the U * 64 from w * U * 64, and lane l item k * 64 + l of its wave's
// range: every load and store instruction covers 64 consecutive items, and a lane keeps one channel group
// (l % ng), so its factors are read once and its extremes are per channel. A lane's U items are all loaded
// before any is used. Loads are buffer loads over the image's bytes.

// The source bytes of item pixel pix, channels c0 .. c0+15: the pixel's (1) or its 2x2 window's (4) 16 bytes.
template <bool POOL>
__device__ __forceinline__ void chain_load(__amdgpu_buffer_rsrc_t r, const ChainArgs& a, uint32_t pix, uint32_t c0,
                                           uint4 (&raw)[POOL ? 4 : 1]) {
  if constexpr (POOL) {
    const uint32_t y = pix / a.wo, x = pix - y * a.wo;
#pragma unroll
    for (int d = 0; d < 4; ++d)
      raw[d] = buf_load_u4(r, ((2 * y + (d >> 1)) * a.w + 2 * x + (d & 1)) * a.co + c0);
  } else {
    raw[0] = buf_load_u4(r, pix * a.co + c0);
  }
}

// The (window max of the) 16 integers in raw: uint8 with RELU, else int8.
template <bool RELU, bool POOL>
__device__ __forceinline__ void chain_decode(const uint4 (&raw)[POOL ? 4 : 1], int (&qv)[16]) {
#pragma unroll
  for (int d = 0; d < (POOL ? 4 : 1); ++d) {
    const uint32_t words[4] = {raw[d].x, raw[d].y, raw[d].z, raw[d].w};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const uint32_t byte = (words[e >> 2] >> (8 * (e & 3))) & 0xffu;
      const int v = RELU ? (int)byte : (int)(int8_t)byte;
      qv[e] = d == 0 ? v : max(qv[e], v);
    }
  }
}

template <int DT, bool RELU, bool POOL, int PASS, int U>
__global__ __launch_bounds__(256) void conv_chain_wide_kernel(ChainArgs a, const float* __restrict__ sx,
                                                              float* __restrict__ parts, int nparts,
                                                              int8_t* __restrict__ xq, float* __restrict__ sx_next) {
  constexpr int ND = POOL ? 4 : 1;
  __shared__ float red[4];
  const int64_t b = blockIdx.y;
  const uint32_t items = a.ho * a.wo * a.ng;
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t sh = (uint32_t)__builtin_ctz(a.ng);              // ng is a power of two
  const uint32_t c0 = (lane & (a.ng - 1)) * 16;
  const float sxb = sx[b];
  const bool has_bias = a.bias != nullptr;
  const __amdgpu_buffer_rsrc_t r = make_rsrc(a.q + (uint64_t)b * a.h * a.w * a.co, a.h * a.w * a.co);
  const uint32_t span = 256u * U;
  // the channel group's scale and bias go out first: nothing they feed waits on them before the end
  float sr[16], f[16], bv[16];
  chain_factors_raw(a, c0, sr, bv);
  if constexpr (PASS == 0) {
    // per-channel integer extremes over the lane's items; an item past the end is replaced by item `lane`
    // (the same channel group), which exists whenever lane < items
    int hi[16], lo[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) { hi[e] = -1024; lo[e] = 1024; }
    for (uint32_t t0 = blockIdx.x * span; t0 < items; t0 += gridDim.x * span) {
      uint4 raw[U][ND];
#pragma unroll
      for (int k = 0; k < U; ++k) {
        uint32_t it = t0 + wave * 64u * U + 64u * k + lane;
        if (it >= items) it = lane;
        chain_load<POOL>(r, a, it >> sh, c0, raw[k]);
      }
#pragma unroll
      for (int k = 0; k < U; ++k) {
        int qv[16];
        chain_decode<RELU, POOL>(raw[k], qv);
#pragma unroll
        for (int e = 0; e < 16; ++e) { hi[e] = max(hi[e], qv[e]); lo[e] = min(lo[e], qv[e]); }
      }
    }
    float m = 0.0f;
    if (lane < items && blockIdx.x * span < items) {
      chain_scale(a, c0, sxb, sr, f);
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (c0 + e < a.co)
          m = mag_max(m, mag_max(fabsf(chain_value<DT>(hi[e], f[e], bv[e], has_bias, a.relu_y)),
                             fabsf(chain_value<DT>(lo[e], f[e], bv[e], has_bias, a.relu_y))));
    }
    m = group_max<256>(m, red);
    if (threadIdx.x == 0) parts[b * AMAX_PARTS + blockIdx.x] = m;
  } else {
    // items past the end are loaded (in bounds or zeros) but never stored; the loads go out before the
    // image's scale is reduced
    const uint32_t t0 = blockIdx.x * span + wave * 64u * U + lane;
    uint4 raw[U][ND];
#pragma unroll
    for (int k = 0; k < U; ++k) chain_load<POOL>(r, a, (t0 + 64u * k) >> sh, c0, raw[k]);
    const float sc = scale_from_amax(image_amax(parts, b, nparts, red));
    const float rc = 1.0f / sc;
    if (blockIdx.x == 0 && threadIdx.x == 0) sx_next[b] = sc;
    chain_scale(a, c0, sxb, sr, f);
    uint32_t keep[4];
    valid_masks((int)min<uint32_t>(16u, a.co > c0 ? a.co - c0 : 0u), keep);
    int8_t* out = xq + (uint64_t)b * items * 16;
#pragma unroll
    for (int k = 0; k < U; ++k) {
      int qv[16];
      chain_decode<RELU, POOL>(raw[k], qv);
      float v[16];
#pragma unroll
      for (int e = 0; e < 16; ++e)
        v[e] = c0 + e < a.co ? chain_value<DT>(qv[e], f[e], bv[e], has_bias, a.relu_y) : 0.0f;
      uint32_t wds[4];
      quant_pack<16>(v, sc, rc, wds);
      const uint32_t it = t0 + 64u * k;
      if (it < items)
        *reinterpret_cast<uint4*>(out + (uint64_t)it * 16) =
            make_uint4(wds[0] & keep[0], wds[1] & keep[1], wds[2] & keep[2], wds[3] & keep[3]);
    }
  }
}

template <int DT, bool RELU, bool POOL, int PASS>
__global__ __launch_bounds__(256) void conv_chain_kernel(ChainArgs a, const float* __restrict__ sx,
                                                         float* __restrict__ parts, int nparts,
                                                         int8_t* __restrict__ xq, float* __restrict__ sx_next) {
  __shared__ float red[4];
  const int64_t b = blockIdx.y;
  const uint32_t items = a.ho * a.wo * a.ng;
  const float sxb = sx[b];
  const bool has_bias = a.bias != nullptr;
  int qv[16];
  float f[16], bv[16];
  if constexpr (PASS == 0) {
    float m = 0.0f;
    const uint32_t stride = gridDim.x * 256u;
    uint32_t item = blockIdx.x * 256u + threadIdx.x;
    if (stride % a.ng == 0) {
      int hi[16], lo[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) { hi[e] = -1024; lo[e] = 1024; }
      const uint32_t c0 = (item % a.ng) * 16;
      const bool any = item < items;
      for (; item < items; item += stride) {
        chain_q<RELU, POOL>(a, b, item / a.ng, c0, qv);
#pragma unroll
        for (int e = 0; e < 16; ++e) { hi[e] = max(hi[e], qv[e]); lo[e] = min(lo[e], qv[e]); }
      }
      if (any) {
        chain_factors(a, c0, sxb, f, bv);
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (c0 + e < a.co)
            m = mag_max(m, mag_max(fabsf(chain_value<DT>(hi[e], f[e], bv[e], has_bias, a.relu_y)),
                               fabsf(chain_value<DT>(lo[e], f[e], bv[e], has_bias, a.relu_y))));
      }
    } else {
      for (; item < items; item += stride) {
        const uint32_t pix = item / a.ng, c0 = (item - pix * a.ng) * 16;
        chain_q<RELU, POOL>(a, b, pix, c0, qv);
        chain_factors(a, c0, sxb, f, bv);
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (c0 + e < a.co) m = mag_max(m, fabsf(chain_value<DT>(qv[e], f[e], bv[e], has_bias, a.relu_y)));
      }
    }
    m = group_max<256>(m, red);
    if (threadIdx.x == 0) parts[b * AMAX_PARTS + blockIdx.x] = m;
  } else {
    const float sc = scale_from_amax(image_amax(parts, b, nparts, red));
    const float rc = 1.0f / sc;
    const uint32_t item = blockIdx.x * 256u + threadIdx.x;
    if (item == 0) sx_next[b] = sc;
    if (item < items) {
      const uint32_t pix = item / a.ng, c0 = (item - pix * a.ng) * 16;
      chain_q<RELU, POOL>(a, b, pix, c0, qv);
      chain_factors(a, c0, sxb, f, bv);
      float v[16];
#pragma unroll
      for (int e = 0; e < 16; ++e)
        v[e] = c0 + e < a.co ? chain_value<DT>(qv[e], f[e], bv[e], has_bias, a.relu_y) : 0.0f;
      uint32_t wds[4], keep[4];
      quant_pack<16>(v, sc, rc, wds);
      valid_masks((int)min<uint32_t>(16u, a.co > c0 ? a.co - c0 : 0u), keep);
      *reinterpret_cast<uint4*>(xq + (uint64_t)b * items * 16 + (uint64_t)item * 16) =
          make_uint4(wds[0] & keep[0], wds[1] & keep[1], wds[2] & keep[2], wds[3] & keep[3]);
    }
  }
}

// int8 NCHW -> NHWC with channel padding (tile 64 channels x 64 pixels).
__global__ __launch_bounds__(256) void nchw_to_nhwc_i8_kernel(const int8_t* __restrict__ src, int64_t ch, int64_t hw,
                                                              int8_t* __restrict__ dst, int64_t c_pad) {
  __shared__ int8_t tile[64][80];
  const int64_t b = blockIdx.z;
  const int64_t p0 = (int64_t)blockIdx.x * 64;
  const int64_t c0 = (int64_t)blockIdx.y * 64;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (int j = 0; j < 16; ++j) {
    const int ci = wave * 16 + j;
    const int64_t c = c0 + ci, p = p0 + lane;
    tile[lane][ci] = (c < ch && p < hw) ? src[(b * ch + c) * hw + p] : (int8_t)0;
  }
  __syncthreads();
  const int pix = threadIdx.x >> 2, part = threadIdx.x & 3;
  const int64_t p = p0 + pix, c = c0 + part * 16;
  if (p < hw && c < c_pad) {
    for (int e = 0; e < 16; ++e) dst[(b * hw + p) * c_pad + c + e] = tile[pix][part * 16 + e];
  }
}

// int8 NHWC (ch channels, unpadded) -> NCHW.
__global__ __launch_bounds__(256) void nhwc_to_nchw_i8_kernel(const int8_t* __restrict__ src, int64_t ch, int64_t hw,
                                                              int8_t* __restrict__ dst) {
  __shared__ int8_t tile[64][68];
  const int64_t b = blockIdx.z;
  const int64_t p0 = (int64_t)blockIdx.x * 64;
  const int64_t c0 = (int64_t)blockIdx.y * 64;
  {
    const int pix = threadIdx.x >> 2, part = threadIdx.x & 3;
    const int64_t p = p0 + pix;
    for (int e = 0; e < 16; ++e) {
      const int64_t c = c0 + part * 16 + e;
      tile[pix][part * 16 + e] = (p < hw && c < ch) ? src[(b * hw + p) * ch + c] : (int8_t)0;
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t p = p0 + lane;
  for (int j = 0; j < 16; ++j) {
    const int ci = wave * 16 + j;
    const int64_t c = c0 + ci;
    if (c < ch && p < hw) dst[(b * ch + c) * hw + p] = tile[lane][ci];
  }
}

inline bool float_dtype(int dt) { return dt == XDNA_F32 || dt == XDNA_BF16 || dt == XDNA_F16; }

// ------------------------------------------------------------------------------ no-allocation scratch
// The per-image block maxima of xdna_conv_quant_nhwc_noalloc live in this file-scope device array instead
// of a caller workspace: XDNA_NOALLOC_MAX_IMAGES images x XDNA_AMAX_WS_PER_IMAGE floats (1 MB), held on
// every device the library runs on until the process ends. Host code never passes the array's name (a
// host-side stand-in): it passes the device address hipGetSymbolAddress returns, looked up once per
// device with that device current. The kernels write every slot they read, so nothing is cleared.
static __device__ __align__(256) float scratch[XDNA_NOALLOC_MAX_IMAGES * XDNA_AMAX_WS_PER_IMAGE];

namespace {
std::mutex g_scratch_mu;
float* g_scratch_ptr[64] = {nullptr};
}  // namespace

// The current device's address of `scratch`, or nullptr with the error set.
float* scratch_ptr() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    set_error("no-alloc scratch: no current device (or a device index above 63)");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (rc != hipSuccess || ptr == nullptr) {
      set_error(std::string("no-alloc scratch: hipGetSymbolAddress failed: ") + hipGetErrorString(rc));
      return nullptr;
    }
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  return g_scratch_ptr[dev];
}

}  // namespace xdna

using namespace xdna;

extern "C" {

int xdna_abi_version(void) { return XDNA_ABI_VERSION; }

const char* xdna_last_error(void) { return g_last_error.c_str(); }

int xdna_device_info(int* num_cus, int* gfx_major, int* gfx_minor) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error(std::string("xdna_device_info: ") + hipGetErrorString(e));
    return XDNA_ENODEV;
  }
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) {
    set_error(std::string("xdna_device_info: ") + hipGetErrorString(e));
    return static_cast<int>(e);
  }
  if (num_cus) *num_cus = prop.multiProcessorCount;
  if (gfx_major) *gfx_major = prop.major;
  if (gfx_minor) *gfx_minor = prop.minor;
  return XDNA_OK;
}

int xdna_quant_rows(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ld_x, int8_t* q, int64_t ld_q,
                    int64_t k_pad, float* s, void* stream) {
  XDNA_REQUIRE(float_dtype(x_dtype), "x_dtype must be XDNA_F32, XDNA_BF16 or XDNA_F16");
  XDNA_REQUIRE(rows >= 0 && k >= 1 && ld_x >= k && k_pad >= k && ld_q >= k_pad, "bad sizes");
  XDNA_REQUIRE(rows < (1ll << 31), "rows must be < 2^31");
  if (rows == 0) return XDNA_OK;
  XDNA_REQUIRE(x && q && s, "null pointer");
  hipStream_t st = as_stream(stream);
  switch (x_dtype) {
    case XDNA_F32: return launch_quant_rows<XDNA_F32>(x, rows, k, ld_x, q, ld_q, k_pad, s, st);
    case XDNA_BF16: return launch_quant_rows<XDNA_BF16>(x, rows, k, ld_x, q, ld_q, k_pad, s, st);
    default: return launch_quant_rows<XDNA_F16>(x, rows, k, ld_x, q, ld_q, k_pad, s, st);
  }
}

int xdna_pad_rows_i8(const int8_t* src, int64_t rows, int64_t cols, int64_t ld_src, int8_t* dst, int64_t ld_dst,
                     int64_t cols_pad, void* stream) {
  XDNA_REQUIRE(rows >= 0 && cols >= 0 && ld_src >= cols && cols_pad >= cols && ld_dst >= cols_pad, "bad sizes");
  XDNA_REQUIRE(rows < 65536 * 1024ll, "too many rows");
  if (rows == 0 || cols_pad == 0) return XDNA_OK;
  unsigned bx = (unsigned)std::min<int64_t>(cdiv(cols_pad, 256), 64);
  dim3 grid(bx, 1, 1);
  for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
    const int64_t r = std::min<int64_t>(65535, rows - r0);
    grid.y = (unsigned)r;
    pad_rows_i8_kernel<<<grid, 256, 0, as_stream(stream)>>>(src + r0 * ld_src, r, cols, ld_src, dst + r0 * ld_dst,
                                                           ld_dst, cols_pad);
  }
  return launch_status("pad_rows_i8");
}

int xdna_conv_quant_nhwc(const void* x, int x_dtype, int64_t nb, int64_t ch, int64_t h, int64_t w, int8_t* q,
                         int64_t c_pad, float* sx, float* amax_ws, void* stream) {
  XDNA_REQUIRE(float_dtype(x_dtype), "x_dtype must be XDNA_F32, XDNA_BF16 or XDNA_F16");
  XDNA_REQUIRE(nb >= 0 && ch >= 1 && h >= 1 && w >= 1 && c_pad >= ch && c_pad % 16 == 0, "bad sizes");
  XDNA_REQUIRE(nb < 65536, "batch must be < 65536");
  if (nb == 0) return XDNA_OK;
  XDNA_REQUIRE(x && q && sx && amax_ws, "null pointer");
  XDNA_REQUIRE(aligned(q, 16), "q must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  const int64_t hw = h * w, per = ch * hw;
  const int esz = x_dtype == XDNA_F32 ? 4 : 2;
  // per-image max: at least 8 loads of 16 bytes per thread per block, and one round of resident blocks
  const bool nt = nb * per * esz >= (int64_t(128) << 20);   // half the Infinity Cache
  const int64_t resident = x_dtype == XDNA_F32 ? stream_blocks<image_absmax_kernel<XDNA_F32, false>, 1024>(INT64_MAX)
                                               : stream_blocks<image_absmax_kernel<XDNA_BF16, false>, 1024>(INT64_MAX);
  const int parts = (int)std::max<int64_t>(
      1, std::min<int64_t>({cdiv(per * esz, 1024 * 8 * 16), (int64_t)AMAX_PARTS, std::max<int64_t>(1, resident / nb)}));
  dim3 g1((unsigned)parts, (unsigned)nb, 1);
  dim3 g2((unsigned)cdiv(hw, 64), (unsigned)cdiv(c_pad, 64), (unsigned)nb);
  XDNA_REQUIRE(cdiv(hw, 64) < (1ll << 31) && cdiv(c_pad, 64) < 65536, "image too large");
  // the 16-byte path: pixel rows in whole 16-byte loads, an image's bytes addressable by one buffer resource
  const bool vec = hw % (16 / esz) == 0 && aligned(x, 16) && per * esz < (int64_t(1) << 31);
  const dim3 gv((unsigned)cdiv(hw, 16 * (16 / esz)), (unsigned)cdiv(c_pad, 256), (unsigned)nb);
  // narrow images: the pixel-major kernel reads only the real channels (a 256-channel tile spends most of its
  // loads past ch: 8x3x448x448 float32 took 114 us, 20 us this way); at c_pad 64 the tile is faster again
  const bool narrow = vec && c_pad <= 48;
  const dim3 gn((unsigned)cdiv(hw, 256 * (16 / esz)), (unsigned)nb, 1);
#define XDNA_CQ(DT)                                                                                        \
  if (nt) image_absmax_kernel<DT, true><<<g1, 1024, 0, st>>>(x, per, amax_ws);                              \
  else image_absmax_kernel<DT, false><<<g1, 1024, 0, st>>>(x, per, amax_ws);                                \
  if (narrow && nt) conv_quant_nhwc_narrow_kernel<DT, true><<<gn, 256, 0, st>>>(x, ch, hw, amax_ws, parts, q, c_pad, sx); \
  else if (narrow) conv_quant_nhwc_narrow_kernel<DT, false><<<gn, 256, 0, st>>>(x, ch, hw, amax_ws, parts, q, c_pad, sx); \
  else if (vec && nt) conv_quant_nhwc_vec_kernel<DT, true><<<gv, 256, 0, st>>>(x, ch, hw, amax_ws, parts, q, c_pad, sx); \
  else if (vec) conv_quant_nhwc_vec_kernel<DT, false><<<gv, 256, 0, st>>>(x, ch, hw, amax_ws, parts, q, c_pad, sx); \
  else conv_quant_nhwc_kernel<DT><<<g2, 256, 0, st>>>(x, ch, hw, amax_ws, parts, q, c_pad, sx);
  switch (x_dtype) {
    case XDNA_F32: XDNA_CQ(XDNA_F32) break;
    case XDNA_BF16: XDNA_CQ(XDNA_BF16) break;
    default: XDNA_CQ(XDNA_F16)
  }
#undef XDNA_CQ
  return launch_status("conv_quant_nhwc");
}

int xdna_conv_quant_nhwc_noalloc(const void* x, int x_dtype, int64_t nb, int64_t ch, int64_t h, int64_t w, int8_t* q,
                                 int64_t c_pad, float* sx, void* stream) {
  XDNA_REQUIRE(nb >= 0 && nb <= XDNA_NOALLOC_MAX_IMAGES,
               "xdna_conv_quant_nhwc_noalloc takes at most XDNA_NOALLOC_MAX_IMAGES (1024) images per call");
  if (nb == 0) return XDNA_OK;
  float* ws = scratch_ptr();
  if (ws == nullptr) return XDNA_ENODEV;
  return xdna_conv_quant_nhwc(x, x_dtype, nb, ch, h, w, q, c_pad, sx, ws, stream);
}

int xdna_conv_weight_pack(const void* w, int w_dtype, int64_t co, int64_t ci, int8_t* wq, int64_t ci_pad, float* sw,
                          void* stream) {
  XDNA_REQUIRE(float_dtype(w_dtype), "w_dtype must be XDNA_F32, XDNA_BF16 or XDNA_F16");
  XDNA_REQUIRE(co >= 1 && ci >= 1 && ci_pad >= ci && ci_pad % 16 == 0 && co < (1ll << 31), "bad sizes");
  XDNA_REQUIRE(w && wq && sw, "null pointer");
  hipStream_t st = as_stream(stream);
  switch (w_dtype) {
    case XDNA_F32: conv_weight_pack_kernel<XDNA_F32><<<dim3((unsigned)co), 256, 0, st>>>(w, ci, wq, ci_pad, sw); break;
    case XDNA_BF16: conv_weight_pack_kernel<XDNA_BF16><<<dim3((unsigned)co), 256, 0, st>>>(w, ci, wq, ci_pad, sw); break;
    default: conv_weight_pack_kernel<XDNA_F16><<<dim3((unsigned)co), 256, 0, st>>>(w, ci, wq, ci_pad, sw);
  }
  return launch_status("conv_weight_pack");
}

int xdna_conv_dequant(const void* q, int relu, int64_t nb, int64_t h, int64_t w, int64_t co, const float* scale,
                      const float* sx, const float* bias, void* y, int y_dtype, void* stream) {
  XDNA_REQUIRE(float_dtype(y_dtype), "y_dtype must be XDNA_F32, XDNA_BF16 or XDNA_F16");
  XDNA_REQUIRE(nb >= 0 && h >= 1 && w >= 1 && co >= 1 && nb < 65536, "bad sizes");
  if (nb == 0) return XDNA_OK;
  XDNA_REQUIRE(q && scale && sx && y, "null pointer");
  const int64_t hw = h * w;
  XDNA_REQUIRE(cdiv(co, 64) < 65536, "too many channels");
  dim3 g((unsigned)cdiv(hw, 64), (unsigned)cdiv(co, 64), (unsigned)nb);
  hipStream_t st = as_stream(stream);
  const int esz = y_dtype == XDNA_F32 ? 4 : 2;
  // the 16-byte path: output rows in whole 16-byte stores, an image's int8 addressable by one resource
  const bool vec = hw % (16 / esz) == 0 && aligned(y, 16) && hw * co < (int64_t(1) << 31);
  const bool nt = nb * hw * co * esz >= (int64_t(128) << 20);   // output above half the Infinity Cache
  const dim3 gv((unsigned)cdiv(hw, 16 * (16 / esz)), (unsigned)cdiv(co, 256), (unsigned)nb);
#define XDNA_DQ(DT)                                                                                   \
  if (vec && relu && nt) conv_dequant_vec_kernel<DT, true, true><<<gv, 256, 0, st>>>(q, hw, co, scale, sx, bias, y); \
  else if (vec && relu) conv_dequant_vec_kernel<DT, true, false><<<gv, 256, 0, st>>>(q, hw, co, scale, sx, bias, y); \
  else if (vec && nt) conv_dequant_vec_kernel<DT, false, true><<<gv, 256, 0, st>>>(q, hw, co, scale, sx, bias, y); \
  else if (vec) conv_dequant_vec_kernel<DT, false, false><<<gv, 256, 0, st>>>(q, hw, co, scale, sx, bias, y); \
  else if (relu) conv_dequant_kernel<DT, true><<<g, 256, 0, st>>>(q, hw, co, scale, sx, bias, y);       \
  else conv_dequant_kernel<DT, false><<<g, 256, 0, st>>>(q, hw, co, scale, sx, bias, y);
  switch (y_dtype) {
    case XDNA_F32: XDNA_DQ(XDNA_F32) break;
    case XDNA_BF16: XDNA_DQ(XDNA_BF16) break;
    default: XDNA_DQ(XDNA_F16)
  }
#undef XDNA_DQ
  return launch_status("conv_dequant");
}

int xdna_conv_requant_next(const void* q, int relu, int relu_y, int pool, int64_t nb, int64_t h, int64_t w, int64_t co,
                           const float* scale, const float* sx, const float* bias, int x_dtype, int8_t* xq_next,
                           int64_t c_pad_next, float* sx_next, float* amax_ws, void* stream) {
  XDNA_REQUIRE(float_dtype(x_dtype), "x_dtype must be XDNA_F32, XDNA_BF16 or XDNA_F16");
  XDNA_REQUIRE(nb >= 0 && h >= 1 && w >= 1 && co >= 1 && nb < 65536, "bad sizes");
  XDNA_REQUIRE(c_pad_next >= co && c_pad_next % 16 == 0, "c_pad_next must be a multiple of 16 and >= co");
  XDNA_REQUIRE(!pool || (h >= 2 && w >= 2), "a 2x2 pool needs h, w >= 2");
  if (nb == 0) return XDNA_OK;
  XDNA_REQUIRE(q && scale && sx && xq_next && sx_next && amax_ws, "null pointer");
  XDNA_REQUIRE(aligned(xq_next, 16) && (co % 16 != 0 || aligned(q, 16)), "misaligned buffers");
  const int64_t ho = pool ? h / 2 : h, wo = pool ? w / 2 : w;
  const int64_t items = ho * wo * (c_pad_next / 16);
  XDNA_REQUIRE(h * w * co < (1ll << 31) && items * 16 < (1ll << 31), "image too large");
  hipStream_t st = as_stream(stream);
  // whole 16-byte channel groups, a power-of-two group count <= 64: the wide kernels, 4 items a lane where
  // that still gives two blocks per CU, else 1 (small boundaries are latency-bound: more blocks)
  const int64_t ng = c_pad_next / 16;
  const bool wide = co % 16 == 0 && ng <= 64 && (ng & (ng - 1)) == 0;
  const int u = wide && cdiv(items, 1024) * nb >= 2 * device_cus() ? 4 : 1;
  const int64_t per_block = 256 * u;
  const int parts = (int)std::max<int64_t>(1, std::min<int64_t>(cdiv(items, per_block), AMAX_PARTS));
  dim3 g0((unsigned)parts, (unsigned)nb), g1((unsigned)cdiv(items, per_block), (unsigned)nb);
  ChainArgs ca{static_cast<const uint8_t*>(q), (uint32_t)h, (uint32_t)w, (uint32_t)co, (uint32_t)ho, (uint32_t)wo,
               (uint32_t)ng, scale, bias, relu_y ? 1 : 0,
               (aligned(scale, 16) && (!bias || aligned(bias, 16))) ? 1 : 0};
#define XDNA_CH(DT, R, P)                                                                                 \
  if (wide && u == 4) {                                                                                   \
    conv_chain_wide_kernel<DT, R, P, 0, 4><<<g0, 256, 0, st>>>(ca, sx, amax_ws, parts, xq_next, sx_next); \
    conv_chain_wide_kernel<DT, R, P, 1, 4><<<g1, 256, 0, st>>>(ca, sx, amax_ws, parts, xq_next, sx_next); \
  } else if (wide) {                                                                                      \
    conv_chain_wide_kernel<DT, R, P, 0, 1><<<g0, 256, 0, st>>>(ca, sx, amax_ws, parts, xq_next, sx_next); \
    conv_chain_wide_kernel<DT, R, P, 1, 1><<<g1, 256, 0, st>>>(ca, sx, amax_ws, parts, xq_next, sx_next); \
  } else {                                                                                                \
    conv_chain_kernel<DT, R, P, 0><<<g0, 256, 0, st>>>(ca, sx, amax_ws, parts, xq_next, sx_next);        \
    conv_chain_kernel<DT, R, P, 1><<<g1, 256, 0, st>>>(ca, sx, amax_ws, parts, xq_next, sx_next);        \
  }
#define XDNA_CH_RP(DT)                 \
  if (relu && pool) { XDNA_CH(DT, true, true) }        \
  else if (relu) { XDNA_CH(DT, true, false) }          \
  else if (pool) { XDNA_CH(DT, false, true) }          \
  else { XDNA_CH(DT, false, false) }
  switch (x_dtype) {
    case XDNA_F32: XDNA_CH_RP(XDNA_F32) break;
    case XDNA_BF16: XDNA_CH_RP(XDNA_BF16) break;
    default: XDNA_CH_RP(XDNA_F16)
  }
#undef XDNA_CH_RP
#undef XDNA_CH
  return launch_status("conv_requant_next");
}

int xdna_nchw_to_nhwc_i8(const int8_t* src, int64_t nb, int64_t ch, int64_t h, int64_t w, int8_t* dst, int64_t c_pad,
                         void* stream) {
  XDNA_REQUIRE(nb >= 0 && ch >= 1 && h >= 1 && w >= 1 && c_pad >= ch && c_pad % 16 == 0 && nb < 65536, "bad sizes");
  if (nb == 0) return XDNA_OK;
  XDNA_REQUIRE(src && dst, "null pointer");
  const int64_t hw = h * w;
  dim3 g((unsigned)cdiv(hw, 64), (unsigned)cdiv(c_pad, 64), (unsigned)nb);
  nchw_to_nhwc_i8_kernel<<<g, 256, 0, as_stream(stream)>>>(src, ch, hw, dst, c_pad);
  return launch_status("nchw_to_nhwc_i8");
}

int xdna_nhwc_to_nchw_i8(const void* src, int64_t nb, int64_t ch, int64_t h, int64_t w, void* dst, void* stream) {
  XDNA_REQUIRE(nb >= 0 && ch >= 1 && h >= 1 && w >= 1 && nb < 65536, "bad sizes");
  if (nb == 0) return XDNA_OK;
  XDNA_REQUIRE(src && dst, "null pointer");
  const int64_t hw = h * w;
  dim3 g((unsigned)cdiv(hw, 64), (unsigned)cdiv(ch, 64), (unsigned)nb);
  nhwc_to_nchw_i8_kernel<<<g, 256, 0, as_stream(stream)>>>(reinterpret_cast<const int8_t*>(src), ch, hw,
                                                           reinterpret_cast<int8_t*>(dst));
  return launch_status("nhwc_to_nchw_i8");
}

}  // extern "C"
