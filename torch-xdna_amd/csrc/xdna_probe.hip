// Measurement probe, not part of the hot path's C ABI: the int8 MFMA issue ceiling of the device.
//
// Each wave runs `iters` rounds of 16 back-to-back v_mfma_i32_32x32x32_i8 on registers only (four
// independent accumulators, no memory traffic inside the loop) and records the shader-clock cycles
// of its loop (s_memtime). With constant operands the MFMA datapath barely toggles; with 16
// registers of random bytes every MFMA sees different data, which is what a GEMM's power draw looks
// like. The ratio of MFMAs issued to elapsed time gives the achievable int8 rate, and cycles / time
// the shader clock the device held while doing it. Built as its own library (libxdna_probe.so),
// loaded only by bench.py's `mfma` workload.
#include <hip/hip_runtime.h>
#include <cstdint>

namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

template <bool RANDOM>
__global__ __launch_bounds__(512) void mfma_ceiling_kernel(int iters, uint32_t seed, int32_t* out, uint64_t* cycles) {
  uint32_t x = 0x9E3779B9u * (threadIdx.x + 1) ^ (seed * 0x85EBCA6Bu) ^ (blockIdx.x * 0xC2B2AE35u);
  i32x4 r[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    i32x4 v;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      x ^= x << 13;                       // xorshift32
      x ^= x >> 17;
      x ^= x << 5;
      v[q] = RANDOM ? (int32_t)x : (int32_t)(0x01010101u * (uint32_t)(k + 1));
    }
    r[k] = v;
  }
  i32x16 c[4] = {};
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int k = 0; k < 16; ++k)
      c[k & 3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(r[k], r[(k * 7 + 3) & 15], c[k & 3], 0, 0, 0);
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  int32_t s = 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) s ^= c[0][j] ^ c[1][j] ^ c[2][j] ^ c[3][j];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;   // keeps the MFMAs live
  if (threadIdx.x == 0) cycles[blockIdx.x] = t1 - t0;
}

}  // namespace

extern "C" {

// blocks workgroups of 256 threads (one wave per SIMD); out: blocks * 256 int32; cycles: blocks uint64.
// MFMAs issued: blocks * 4 * iters * 16, each 32 x 32 x 32 int8 multiply-adds. Returns 0 or a HIP error.
int xdna_probe_mfma_i8(int blocks, int iters, int random_operands, uint32_t seed, int32_t* out, uint64_t* cycles,
                       hipStream_t stream) {
  if (blocks <= 0 || iters <= 0 || !out || !cycles) return (int)hipErrorInvalidValue;
  if (random_operands)
    mfma_ceiling_kernel<true><<<blocks, 256, 0, stream>>>(iters, seed, out, cycles);
  else
    mfma_ceiling_kernel<false><<<blocks, 256, 0, stream>>>(iters, seed, out, cycles);
  return (int)hipGetLastError();
}

}  // extern "C"
