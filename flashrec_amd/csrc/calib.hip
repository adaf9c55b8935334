// Measurement only: the sustained rate of the fp8 MFMA this library's GEMM
// issues (v_mfma_scale_f32_32x32x64_f8f6f4), with every operand in
// registers and no memory traffic in the timed loop.  Used to put the GEMM's
// TFLOP/s next to what the matrix cores reach on this board under the same
// power management: the vendor peak (2.4 GHz) is reached only when the
// operand bits barely toggle; with random e4m3 operands the shader clock
// settles lower.  No counterpart in the reference.
#include "fr_common.h"

namespace fr {

typedef int v8i_c __attribute__((ext_vector_type(8)));
typedef float v16f_c __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint32_t lcg(uint32_t& x) {
  x = x * 1664525u + 1013904223u;
  return x;
}

// A random e4m3 byte with no NaN code and an exponent of at most 11
// (|x| < 16): the products and sums stay finite.
__device__ __forceinline__ uint32_t rand_e4m3x4(uint32_t& x) {
  uint32_t w = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t b = lcg(x) >> 24;
    if ((b & 0x78u) > 0x58u) b &= 0xD7u;
    w |= b << (8 * i);
  }
  return w;
}

// Four independent accumulator chains, four operand pairs cycled, so every
// MFMA's inputs differ from the previous one's (random) or not (constant).
__global__ __launch_bounds__(256) void mfma_ceiling(int64_t iters, int random_operands, uint64_t* clocks,
                                                    float* sink) {
  uint32_t seed = 0x9E3779B9u * (threadIdx.x + 1) + blockIdx.x;
  v8i_c a[4], b[4];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[u][e] = random_operands ? static_cast<int>(rand_e4m3x4(seed)) : 0x11111111;
      b[u][e] = random_operands ? static_cast<int>(rand_e4m3x4(seed)) : 0x11111111;
    }
  v16f_c acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[c][v] = 0.0f;
  const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      acc[c] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[c], b[c], acc[c], 0, 0, 0, 0, 0, 0);
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int v = 0; v < 16; ++v) s += acc[c][v];
  if (s == 12345.678f) sink[threadIdx.x] = s;  // keeps the chains live
  if (threadIdx.x == 0) {
    clocks[2 * blockIdx.x] = t1 - t0;
    clocks[2 * blockIdx.x + 1] = r1 - r0;
  }
}

}  // namespace fr

extern "C" int fr_calib_mfma_ceiling(int64_t blocks, int64_t iters, int random_operands, uint64_t* clocks,
                                     float* sink, void* stream) {
  if (blocks <= 0 || blocks > 65536 || iters < 0 || !clocks || !sink) return FR_EINVAL;
  hipLaunchKernelGGL(fr::mfma_ceiling, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), iters, random_operands, clocks, sink);
  return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
}
