// Row-wise log_softmax over fp32 logits, for the SID-restricted lm_head.
// Replaces the `F.log_softmax(logits.float(), dim=-1)` of
// python/flashrec/logits.py:118-120 and :136-137.
//
// Rows of N = 1024 * NCH (the SID head: 8192): one 256-thread workgroup per
// row holds the row in registers (NCH float4 per thread, read once with
// streaming loads), reduces max and sum of exp over the workgroup, and
// writes x - max - log(sum) once: HBM-bound, 8 bytes per element.
// Other widths: one wave64 per row, an online (max, sum of exp) pass, then a
// second read for the output.  In place is allowed (out == x).  A NaN in a
// row, or a row of -inf, gives NaN everywhere, as torch's log_softmax.
#include "fr_common.h"

namespace fr {

__global__ __launch_bounds__(256) void log_softmax_rows(const float* x, int64_t ldx, float* out,
                                                         int64_t ldo, int64_t M, int64_t N) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const float* xr = x + row * ldx;
  float m = -__builtin_inff(), s = 0.0f;
  for (int64_t e = lane; e < N; e += 64) {
    const float v = xr[e];
    if (v > m) {
      s = s * expf(m - v) + 1.0f;
      m = v;
    } else {
      s += expf(v - m);
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float m2 = __shfl_xor(m, o, 64);
    const float s2 = __shfl_xor(s, o, 64);
    const float mm = __builtin_fmaxf(m, m2);
    const float a = (m == -__builtin_inff()) ? 0.0f : s * expf(m - mm);
    const float b = (m2 == -__builtin_inff()) ? 0.0f : s2 * expf(m2 - mm);
    m = mm;
    s = a + b;
  }
  const float lse = m + logf(s);
  float* orow = out + row * ldo;
  for (int64_t e = lane; e < N; e += 64) orow[e] = xr[e] - lse;
}

template <int NCH>
__global__ __launch_bounds__(256) void log_softmax_rows_block(const float* x, int64_t ldx, float* out,
                                                              int64_t ldo) {
  __shared__ float red[8];
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  const f32x4* xr = reinterpret_cast<const f32x4*>(x + row * ldx);
  f32x4 v[NCH];
#pragma unroll
  for (int j = 0; j < NCH; ++j) v[j] = ldkeep(xr + t + 256 * j);
  const float lse = block_row_lse<NCH>(v, red);
  f32x4* orow = reinterpret_cast<f32x4*>(out + row * ldo);
#pragma unroll
  for (int j = 0; j < NCH; ++j) stnt(orow + t + 256 * j, v[j] - lse);
}

}  // namespace fr

extern "C" int fr_log_softmax_f32(const float* x, int64_t ldx, float* out, int64_t ldo, int64_t M,
                                  int64_t N, void* stream) {
  if (M < 0 || N < 0) return FR_EINVAL;
  if (M == 0 || N == 0) return FR_OK;
  if (!x || !out || ldx < N || ldo < N) return FR_EINVAL;
  const bool aligned = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) & 15) == 0 &&
                       (ldx & 3) == 0 && (ldo & 3) == 0 && M <= 0x7FFFFFFF;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (aligned && N == 8192) {
    hipLaunchKernelGGL(fr::log_softmax_rows_block<8>, dim3(static_cast<unsigned>(M)), dim3(256), 0, st, x, ldx,
                       out, ldo);
    return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
  }
  if (aligned && N == 4096) {
    hipLaunchKernelGGL(fr::log_softmax_rows_block<4>, dim3(static_cast<unsigned>(M)), dim3(256), 0, st, x, ldx,
                       out, ldo);
    return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
  }
  hipLaunchKernelGGL(fr::log_softmax_rows, dim3(static_cast<unsigned>((M + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, ldx, out, ldo, M, N);
  return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
}

extern "C" int fr_abi_version(void) { return 1; }
