// Row-wise bandwidth-bound kernels of the FP8 path: per-token e4m3 quant,
// RMSNorm (+ residual add) and SiLU-and-mul, each either quantized to
// e4m3 + a per-row fp32 scale or written back as bf16.
//
// Layout: one wave64 owns one row.  The row is read once with 16-byte
// loads (8 bf16 per lane per vector), kept in VGPRs, reduced with
// cross-lane shuffles (no LDS, no barriers), and written once with
// coalesced 8-byte (e4m3) or 16-byte (bf16) stores.  Rows wider than the
// register budget, or with unaligned widths/strides, take a generic
// three-pass kernel with the same arithmetic.
//
// Arithmetic (bit-for-bit the torch CPU composition of the reference's
// fallback path):
//   quant   python/flashrec/kernel/sglops.py:92-96
//           amax = max|x| clamped to 1e-12; scale = amax / 448;
//           q = e4m3(clamp(x / scale, +-448))
//   rmsnorm sglops.py:35-39   h = bf16((x * rsqrt(mean(x^2) + eps)) * w)
//   add     sglops.py:53-55   residual = bf16(residual + x)
//   silu    sglops.py:151 with torch's silu: s = bf16(g / (1 + exp(-g)));
//           y = bf16(s * u)
#include "fr_common.h"

namespace fr {

enum RowMode { kQuant = 0, kRms = 1, kAddRms = 2, kSilu = 3 };

struct RowArgs {
  const uint16_t* x;   // bf16 input rows (silu: [g | u], 2*K wide)
  int64_t ldx;
  uint16_t* res;       // residual (kAddRms), updated in place
  int64_t ldr;
  const uint16_t* w;   // RMSNorm weight [K]
  uint8_t* q;          // e4m3 codes (quant output) or bf16 rows (bf16 output)
  int64_t ldq;         // in elements of the output dtype
  float* s;            // per-row scales
  int64_t M, K;
  float eps;
};

__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(v[i] << 16);
    f[2 * i + 1] = __uint_as_float(v[i] & 0xFFFF0000u);
  }
}

__device__ __forceinline__ float silu_bf16(float g) {
  // torch CPU silu: x / (1 + exp(-x)) in fp32, then the bf16 store.
  return round_bf16(g / (1.0f + expf(-g)));
}

// Same value in the vector kernel: the divisor 1 + exp(-g) >= 1 is always
// finite-positive or +inf, so one reciprocal plus a correction step gives the
// quotient to within an ulp of the IEEE result before the bf16 rounding.
__device__ __forceinline__ float silu_bf16_fast(float g) {
  const float d = 1.0f + expf(-g);
  const float r = __builtin_amdgcn_rcpf(d);
  const float y = g * r;
  const float e = __builtin_fmaf(-y, d, g);
  return round_bf16(__builtin_copysignf(__builtin_fmaf(e, r, y), g));
}

// Pairs of bf16 roundings with one v_cvt_pk_bf16_f32.
__device__ __forceinline__ void round_bf16x2(float& a, float& b) {
  const uint32_t w = pack_bf16x2(a, b);
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xFFFF0000u);
}

// NaN-propagating max (v_maximum3_f32): torch's amax propagates NaN.
__device__ __forceinline__ float maxnan(float a, float b) { return __builtin_elementwise_maximum(a, b); }

__device__ __forceinline__ float wave_maxnan(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = maxnan(v, __shfl_xor(v, o, 64));
  return v;
}

// One wave per row, NV vectors of 8 elements per lane held in registers.
template <int MODE, int NV, bool QOUT>
__global__ __launch_bounds__(256) void row_kernel_vec(RowArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= a.M) return;
  const int64_t K = a.K;
  float v[NV][8];

  const uint16_t* xr = a.x + row * a.ldx;
  u32x4 xv[NV], uv[NV], wv[NV];
  // issue every load of the row (and the norm weight) first
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t e = (static_cast<int64_t>(j) * 64 + lane) * 8;
    if (e < K) {
      xv[j] = *reinterpret_cast<const u32x4*>(xr + e);
      if (MODE == kRms || MODE == kAddRms) wv[j] = *reinterpret_cast<const u32x4*>(a.w + e);
      if (MODE == kSilu) uv[j] = *reinterpret_cast<const u32x4*>(xr + K + e);
      if (MODE == kAddRms) uv[j] = *reinterpret_cast<const u32x4*>(a.res + row * a.ldr + e);
    }
  }
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t e = (static_cast<int64_t>(j) * 64 + lane) * 8;
    if (e < K) {
      unpack8(xv[j], v[j]);
      if (MODE == kSilu) {
        float u[8];
        unpack8(uv[j], u);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[j][i] = silu_bf16_fast(v[j][i]) * u[i];
#pragma unroll
        for (int i = 0; i < 8; i += 2) round_bf16x2(v[j][i], v[j][i + 1]);
      }
      if (MODE == kAddRms) {
        float r[8];
        unpack8(uv[j], r);
        u32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[j][2 * i] = r[2 * i] + v[j][2 * i];
          v[j][2 * i + 1] = r[2 * i + 1] + v[j][2 * i + 1];
          o[i] = pack_bf16x2(v[j][2 * i], v[j][2 * i + 1]);
          v[j][2 * i] = __uint_as_float(o[i] << 16);
          v[j][2 * i + 1] = __uint_as_float(o[i] & 0xFFFF0000u);
        }
        *reinterpret_cast<u32x4*>(a.res + row * a.ldr + e) = o;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[j][i] = 0.0f;
    }
  }

  if (MODE == kRms || MODE == kAddRms) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += v[j][i] * v[j][i];
    ss = wave_sum(ss);
    const float var = ss / static_cast<float>(K);
    const float rstd = 1.0f / __builtin_sqrtf(var + a.eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t e = (static_cast<int64_t>(j) * 64 + lane) * 8;
      if (e < K) {
        float w[8];
        unpack8(wv[j], w);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[j][i] = (v[j][i] * rstd) * w[i];
#pragma unroll
        for (int i = 0; i < 8; i += 2) round_bf16x2(v[j][i], v[j][i + 1]);
      }
    }
  }

  if (!QOUT) {
    uint16_t* orow = reinterpret_cast<uint16_t*>(a.q) + row * a.ldq;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t e = (static_cast<int64_t>(j) * 64 + lane) * 8;
      if (e < K) {
        u32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = pack_bf16x2(v[j][2 * i], v[j][2 * i + 1]);
        *reinterpret_cast<u32x4*>(orow + e) = o;
      }
    }
    return;
  }

  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = maxnan(amax, __builtin_fabsf(v[j][i]));
  amax = maxnan(wave_maxnan(amax), kAmaxFloor);
  const float scale = amax / kFp8Max;
  if (lane == 0) a.s[row] = scale;

  uint8_t* qrow = a.q + row * a.ldq;
  if (amax < 3.0e38f) {
    // Finite row: |x / scale| <= 448 (within rounding), where the hardware
    // conversion equals torch's clamp + convert; the quotient is correctly
    // rounded (Markstein correction with the row's reciprocal).
    const float r = 1.0f / scale;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t e = (static_cast<int64_t>(j) * 64 + lane) * 8;
      if (e < K) {
        float t[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = div_rn_shared(v[j][i], scale, r);
        u32x2 o;
        o[0] = cvt_pk_e4m3<true>(t[2], t[3], cvt_pk_e4m3<false>(t[0], t[1], 0u));
        o[1] = cvt_pk_e4m3<true>(t[6], t[7], cvt_pk_e4m3<false>(t[4], t[5], 0u));
        *reinterpret_cast<u32x2*>(qrow + e) = o;
      }
    }
  } else {
    // NaN or inf in the row: plain IEEE division and torch's NaN codes.
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t e = (static_cast<int64_t>(j) * 64 + lane) * 8;
      if (e < K) {
        float t[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] = v[j][i] / scale;
        u32x2 o;
        o[0] = e4m3x4_clamped(t[0], t[1], t[2], t[3]);
        o[1] = e4m3x4_clamped(t[4], t[5], t[6], t[7]);
        *reinterpret_cast<u32x2*>(qrow + e) = o;
      }
    }
  }
}

// Generic path: any width, any stride, any input dtype.  One wave per row,
// lane-strided elements, re-reading the row from global memory per pass.
template <int MODE, int DT, bool QOUT>
__global__ __launch_bounds__(256) void row_kernel_generic(RowArgs a) {
  using E = Elem<DT>;
  using T = typename E::T;
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= a.M) return;
  const int64_t K = a.K;
  const T* xr = reinterpret_cast<const T*>(a.x) + row * a.ldx;
  uint16_t* rr = (MODE == kAddRms) ? a.res + row * a.ldr : nullptr;

  // Pass 1: the pre-normalisation value of each element (and the residual
  // update), plus the sum of squares.
  float ss = 0.0f;
  if (MODE == kRms || MODE == kAddRms) for (int64_t e = lane; e < K; e += 64) {
    float val = E::load(xr + e);
    if (MODE == kAddRms) {
      val = round_bf16(bf16_to_f32(rr[e]) + val);
      rr[e] = static_cast<uint16_t>(pack_bf16x2(val, 0.0f) & 0xFFFFu);
    }
    ss += val * val;
  }
  float rstd = 0.0f;
  if (MODE == kRms || MODE == kAddRms) {
    ss = wave_sum(ss);
    rstd = 1.0f / __builtin_sqrtf(ss / static_cast<float>(K) + a.eps);
  }
  auto value = [&](int64_t e) -> float {
    float val;
    if (MODE == kAddRms) {
      val = bf16_to_f32(rr[e]);
    } else {
      val = E::load(xr + e);
    }
    if (MODE == kSilu) val = round_bf16(silu_bf16(val) * E::load(xr + K + e));
    if (MODE == kRms || MODE == kAddRms) val = round_bf16((val * rstd) * bf16_to_f32(a.w[e]));
    return val;
  };

  if (!QOUT) {
    uint16_t* orow = reinterpret_cast<uint16_t*>(a.q) + row * a.ldq;
    for (int64_t e = lane; e < K; e += 64)
      orow[e] = static_cast<uint16_t>(pack_bf16x2(value(e), 0.0f) & 0xFFFFu);
    return;
  }
  float amax = 0.0f;
  for (int64_t e = lane; e < K; e += 64) amax = maxnan(amax, __builtin_fabsf(value(e)));
  amax = maxnan(wave_maxnan(amax), kAmaxFloor);
  const float scale = amax / kFp8Max;
  if (lane == 0) a.s[row] = scale;
  uint8_t* qrow = a.q + row * a.ldq;
  for (int64_t e = lane; e < K; e += 64)
    qrow[e] = static_cast<uint8_t>(e4m3_clamped_byte(value(e) / scale));
}

template <int MODE, bool QOUT, int NV>
static hipError_t launch_vec(const RowArgs& a, hipStream_t st) {
  dim3 grid(static_cast<unsigned>((a.M + 3) / 4));
  hipLaunchKernelGGL((row_kernel_vec<MODE, NV, QOUT>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

template <int MODE, bool QOUT>
static int launch_rows(RowArgs a, int dtype, hipStream_t st) {
  if (a.M < 0 || a.K < 0) return FR_EINVAL;
  if (a.M == 0 || a.K == 0) {
    // torch: amax over an empty row is an error; an empty batch is a no-op.
    return a.M == 0 ? FR_OK : FR_EUNSUPPORTED;
  }
  if (a.M > (int64_t)4 * 0x7FFFFFFF) return FR_EUNSUPPORTED;
  const int64_t K = a.K;
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  bool vec = dtype == FR_DTYPE_BF16 && K % 8 == 0 && a.ldx % 8 == 0 && al16(a.x) &&
             K <= 8192;
  if (MODE == kSilu) vec = vec && al16(a.x + K);
  if (MODE == kAddRms) vec = vec && a.ldr % 8 == 0 && al16(a.res);
  if (MODE == kRms || MODE == kAddRms) vec = vec && al16(a.w);
  if (QOUT) vec = vec && a.ldq % 8 == 0 && (reinterpret_cast<uintptr_t>(a.q) & 7u) == 0;
  else vec = vec && a.ldq % 8 == 0 && al16(a.q);
  hipError_t err;
  if (vec) {
    const int64_t nv = (K + 511) / 512;
    if (nv <= 1) err = launch_vec<MODE, QOUT, 1>(a, st);
    else if (nv <= 2) err = launch_vec<MODE, QOUT, 2>(a, st);
    else if (nv <= 3) err = launch_vec<MODE, QOUT, 3>(a, st);
    else if (nv <= 4) err = launch_vec<MODE, QOUT, 4>(a, st);
    else if (nv <= 6) err = launch_vec<MODE, QOUT, 6>(a, st);
    else if (nv <= 8) err = launch_vec<MODE, QOUT, 8>(a, st);
    else if (nv <= 12) err = launch_vec<MODE, QOUT, 12>(a, st);
    else err = launch_vec<MODE, QOUT, 16>(a, st);
  } else {
    dim3 grid(static_cast<unsigned>((a.M + 3) / 4));
    switch (dtype) {
      case FR_DTYPE_BF16:
        hipLaunchKernelGGL((row_kernel_generic<MODE, FR_DTYPE_BF16, QOUT>), grid, dim3(256), 0, st, a);
        break;
      case FR_DTYPE_FP16:
        if (MODE != kQuant) return FR_EUNSUPPORTED;
        hipLaunchKernelGGL((row_kernel_generic<MODE, FR_DTYPE_FP16, QOUT>), grid, dim3(256), 0, st, a);
        break;
      case FR_DTYPE_FP32:
        if (MODE != kQuant) return FR_EUNSUPPORTED;
        hipLaunchKernelGGL((row_kernel_generic<MODE, FR_DTYPE_FP32, QOUT>), grid, dim3(256), 0, st, a);
        break;
      default:
        return FR_EINVAL;
    }
    err = hipGetLastError();
  }
  return err == hipSuccess ? FR_OK : FR_ELAUNCH;
}

}  // namespace fr

using namespace fr;

extern "C" {

int fr_per_token_quant_fp8(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                           void* q, float* s, void* stream) {
  if ((M > 0 && K > 0) && (!x || !q || !s)) return FR_EINVAL;
  RowArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.q = static_cast<uint8_t*>(q);
  a.ldq = K;
  a.s = s;
  a.M = M;
  a.K = K;
  return launch_rows<kQuant, true>(a, x_dtype, static_cast<hipStream_t>(stream));
}

int fr_quantize_weight_fp8(const void* w, int w_dtype, int64_t N, int64_t K, int64_t ldw,
                           void* q, float* s, void* stream) {
  return fr_per_token_quant_fp8(w, w_dtype, N, K, ldw, q, s, stream);
}

int fr_rms_quant_fp8(const void* x, int64_t ldx, void* residual, int64_t ldr, const void* w,
                     int64_t M, int64_t H, float eps, void* q, float* s, void* stream) {
  if ((M > 0 && H > 0) && (!x || !w || !q || !s)) return FR_EINVAL;
  RowArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.res = static_cast<uint16_t*>(residual);
  a.ldr = ldr;
  a.w = static_cast<const uint16_t*>(w);
  a.q = static_cast<uint8_t*>(q);
  a.ldq = H;
  a.s = s;
  a.M = M;
  a.K = H;
  a.eps = eps;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return residual ? launch_rows<kAddRms, true>(a, FR_DTYPE_BF16, st)
                  : launch_rows<kRms, true>(a, FR_DTYPE_BF16, st);
}

int fr_rmsnorm(const void* x, int64_t ldx, void* residual, int64_t ldr, const void* w,
               void* out, int64_t ldo, int64_t M, int64_t H, float eps, void* stream) {
  if ((M > 0 && H > 0) && (!x || !w || !out)) return FR_EINVAL;
  RowArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.res = static_cast<uint16_t*>(residual);
  a.ldr = ldr;
  a.w = static_cast<const uint16_t*>(w);
  a.q = static_cast<uint8_t*>(out);
  a.ldq = ldo;
  a.M = M;
  a.K = H;
  a.eps = eps;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return residual ? launch_rows<kAddRms, false>(a, FR_DTYPE_BF16, st)
                  : launch_rows<kRms, false>(a, FR_DTYPE_BF16, st);
}

int fr_silu_quant_fp8(const void* x, int64_t ldx, int64_t M, int64_t d, void* q, float* s,
                      void* stream) {
  if ((M > 0 && d > 0) && (!x || !q || !s)) return FR_EINVAL;
  RowArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.q = static_cast<uint8_t*>(q);
  a.ldq = d;
  a.s = s;
  a.M = M;
  a.K = d;
  return launch_rows<kSilu, true>(a, FR_DTYPE_BF16, static_cast<hipStream_t>(stream));
}

int fr_silu_and_mul(const void* x, int64_t ldx, void* out, int64_t ldo, int64_t M, int64_t d,
                    void* stream) {
  if ((M > 0 && d > 0) && (!x || !out)) return FR_EINVAL;
  RowArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.q = static_cast<uint8_t*>(out);
  a.ldq = ldo;
  a.M = M;
  a.K = d;
  return launch_rows<kSilu, false>(a, FR_DTYPE_BF16, static_cast<hipStream_t>(stream));
}

}  // extern "C"
