// Shared device helpers and host-side error plumbing for the xdna HIP library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "xdna_hip.h"

namespace xdna {

// ------------------------------------------------------------------------------ host errors
// The last failure's message for xdna_last_error(); one per host thread.
void set_error(const std::string& msg);

#define XDNA_REQUIRE(cond, msg)                                  \
  do {                                                           \
    if (!(cond)) {                                               \
      ::xdna::set_error(std::string(__func__) + ": " + (msg));   \
      return XDNA_EINVAL;                                        \
    }                                                            \
  } while (0)

// Status of the launches just made on this thread (hipGetLastError), as an ABI status.
int launch_status(const char* where);
// Compute units of the current device (cached per device).
int device_cus();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

__host__ __device__ inline bool aligned(const void* p, int64_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// ------------------------------------------------------------------------------ device types
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// float32 -> bfloat16 bits, round to nearest even (NaN stays a quiet NaN), the rounding torch's
// `.to(torch.bfloat16)` applies.
// Branch-free: both results are computed and selected.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);   // v_cvt_pk_bf16_f32: round to nearest even
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Two float32 -> two bfloat16 / float16 (round to nearest even) in one instruction, lo | hi << 16.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}
__device__ __forceinline__ uint32_t f32x2_to_f16x2_bits(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, f16x2_t));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// float32 -> float16 bits with round to nearest even (v_cvt_f16_f32 under the default mode).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// Element loads of the floating-point input dtypes as float32 (exact widening).
template <int DT>
__device__ __forceinline__ float load_as_f32(const void* base, int64_t i);

template <>
__device__ __forceinline__ float load_as_f32<XDNA_F32>(const void* base, int64_t i) {
  return reinterpret_cast<const float*>(base)[i];
}
template <>
__device__ __forceinline__ float load_as_f32<XDNA_BF16>(const void* base, int64_t i) {
  return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[i]);
}
template <>
__device__ __forceinline__ float load_as_f32<XDNA_F16>(const void* base, int64_t i) {
  return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[i]);
}

template <int DT>
__device__ __forceinline__ void store_from_f32(void* base, int64_t i, float v);

template <>
__device__ __forceinline__ void store_from_f32<XDNA_F32>(void* base, int64_t i, float v) {
  reinterpret_cast<float*>(base)[i] = v;
}
template <>
__device__ __forceinline__ void store_from_f32<XDNA_BF16>(void* base, int64_t i, float v) {
  reinterpret_cast<uint16_t*>(base)[i] = f32_to_bf16_bits(v);
}
template <>
__device__ __forceinline__ void store_from_f32<XDNA_F16>(void* base, int64_t i, float v) {
  reinterpret_cast<uint16_t*>(base)[i] = f32_to_f16_bits(v);
}

// round_half_even(x / s) for |x / s| <= 128, equal to rintf of the correctly rounded float32
// quotient (what torch.round(x / s) computes). The product with the reciprocal is within 2^-15 of
// the rounded quotient for these magnitudes, so the two round to the same integer unless the
// product lies within 2^-14 of a half-integer; only then is the IEEE division done.
__device__ __forceinline__ float round_div(float x, float s, float r) {
  float t = x * r;
  const float f = __builtin_amdgcn_fractf(t);   // t - floor(t) in one instruction (v_fract_f32)
  if (fabsf(f - 0.5f) < 6.103515625e-05f) t = x / s;
  return rintf(t);
}

// Quantized value of x for a row scale s (with r = 1 / s): clamp(round(x / s), -127, 127).
__device__ __forceinline__ float quantf(float x, float s, float r) {
  return fminf(fmaxf(round_div(x, s, r), -127.0f), 127.0f);
}
__device__ __forceinline__ int quant1(float x, float s, float r) { return (int)quantf(x, s, r); }

// N values quantized and packed as N int8 bytes (value e in byte e % 4 of word e / 4), the vector form
// of quant1; the integer is round_half_even(fl(x / s)), the correctly rounded quotient rounded again, as
// torch.round(x / s) computes it. With r = fl(1 / s), t = fl(x * r) is within 127 * 2^-23 * (1 + 2^-24)
// < 1.52e-5 of the exact quotient (two roundings of relative size 2^-24, |x / s| <= 127), and fl(x / s)
// within a further 2^-18, so when t is at least 2^-15 (3.05e-5) from a half-integer, fl(x / s) lies on
// the same side of it and both round alike. v_cvt_pk_u8_f32 rounds to nearest even and saturates to
// [0, 255] (checked on gfx950 over every float in [-2, 258] at 2^-12 spacing and the neighbours of every
// half-integer), so the byte q + 128 is that conversion of t + 128: the sum's rounding (at most 2^-17)
// cannot carry it across the boundary either. Within 2^-15 of a half-integer (rare) the IEEE division
// computes fl(x / s) itself; that branch is taken when some lane of the wave holds such a value, so it
// is wave-uniform and the divisions are not computed speculatively for every element. |x / s| <= 127,
// so the only clamp needed is the lower bound for -inf, which also maps NaN to -127 (max returns the
// non-NaN operand); +inf saturates to 127. Flipping bit 7 of every byte then gives the two's-complement
// int8.
template <int N>
__device__ __forceinline__ void quant_pack(const float (&x)[N], float s, float r, uint32_t (&w)[N / 4]) {
  constexpr float NEAR = 3.0517578125e-05f;   // 2^-15
  float t[N], b[N];
  bool near = false;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    t[i] = x[i] * r;
    near |= fabsf(__builtin_amdgcn_fractf(t[i]) - 0.5f) < NEAR;
    b[i] = t[i] + 128.0f;
  }
  if (__builtin_amdgcn_ballot_w64(near)) {
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (fabsf(__builtin_amdgcn_fractf(t[i]) - 0.5f) < NEAR) b[i] = rintf(x[i] / s) + 128.0f;
  }
#pragma unroll
  for (int g = 0; g < N / 4; ++g) {
    uint32_t v = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) v = __builtin_amdgcn_cvt_pk_u8_f32(fmaxf(b[4 * g + e], 1.0f), e, v);
    w[g] = v ^ 0x80808080u;
  }
}

// The row scale from the row's max |x|: max(amax, 1e-8f) / 127 with IEEE division.
__device__ __forceinline__ float scale_from_amax(float amax) {
  float a = amax > 1e-8f ? amax : 1e-8f;
  if (amax != amax) a = amax;   // NaN propagates as torch.clamp does
  return a / 127.0f;
}

// 16-byte vector of input elements: 8 x 16-bit or 4 x float32.
template <int DT>
struct Vec16 {
  static constexpr int N = (DT == XDNA_F32) ? 4 : 8;
  uint4 raw;
  __device__ __forceinline__ float get(int i) const {
    if constexpr (DT == XDNA_F32) {
      const float* f = reinterpret_cast<const float*>(&raw);
      return f[i];
    } else {
      const uint16_t* h = reinterpret_cast<const uint16_t*>(&raw);
      if constexpr (DT == XDNA_BF16) return bf16_bits_to_f32(h[i]);
      else return f16_bits_to_f32(h[i]);
    }
  }
};

// Row max |x| kept as magnitude bits: a float's magnitude orders like its bit pattern with the sign bit
// cleared, NaN patterns above +inf, so an unsigned max finds max |x| and lets a NaN through (torch's
// amax propagates NaN; a float max would drop it). bf16 / fp16 words hold two elements, which one
// packed 16-bit max (v_pk_max_u16) compares at once; the float is formed once per row.
template <int DT>
struct AbsMaxBits {
  uint32_t m = 0;                       // 16-bit types: two packed 16-bit maxima; float32: one
  __device__ __forceinline__ void add(const Vec16<DT>& v) {
    const uint32_t w[4] = {v.raw.x, v.raw.y, v.raw.z, v.raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DT == XDNA_F32) {
        m = max(m, w[i] & 0x7fffffffu);
      } else {
        typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
        m = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, m),
                                                                   __builtin_bit_cast(u16x2, w[i] & 0x7fff7fffu)));
      }
    }
  }
  // this lane's magnitude bits (below 2^31: usable as int)
  __device__ __forceinline__ int lane_bits() const {
    if constexpr (DT == XDNA_F32) return (int)m;
    else return (int)max(m & 0xffffu, m >> 16);
  }
};

template <int DT>
__device__ __forceinline__ float bits_to_abs(int b) {
  if constexpr (DT == XDNA_F32) return __uint_as_float((uint32_t)b);
  else if constexpr (DT == XDNA_BF16) return bf16_bits_to_f32((uint16_t)b);
  else return f16_bits_to_f32((uint16_t)b);
}

// Raw buffer loads: a 16-byte load at a byte offset >= the resource's size returns zeros, which is how
// rows past M / N, chunks past K and conv taps outside the image read as zero without a branch.
constexpr uint32_t OOB = 0x7ffffff0u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// 16 bytes at byte offset off of a buffer resource (zeros past its end). NT: the non-temporal (slc)
// form, for data read once that should not displace cached data.
template <bool NT = false>
__device__ __forceinline__ uint4 buf_load_u4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, NT ? 2 : 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Wavefront (64 lanes) max reduction.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
  return v;
}

}  // namespace xdna
