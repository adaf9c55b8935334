// Shared device helpers for the FlashRec FP8 path on MI355X (gfx950, CDNA4).
//
// Numeric conventions follow the torch CPU arithmetic of the reference's
// fallback path (python/flashrec/kernel/sglops.py:33-151):
//   * bf16 <-> fp32 conversions are exact widening / round-to-nearest-even;
//   * float -> float8_e4m3fn follows torch's c10 conversion: round to nearest
//     even, |x| > 464 (and NaN/inf) -> NaN code 0x7F | sign;
//   * divisions and square roots are IEEE correctly rounded.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define FR_OK 0
#define FR_EINVAL 1      // bad pointer / size / stride
#define FR_EUNSUPPORTED 2  // shape the kernels do not handle (caller falls back)
#define FR_ELAUNCH 3     // HIP launch error
#define FR_ETOOLARGE 4   // request exceeds a fixed capacity (no-allocation entry points)

// static device scratch of fr_genrec_mask_topk_expand_noalloc, per GPU
#define FR_GENREC_NOALLOC_SCRATCH_BYTES (4 << 20)

namespace fr {
constexpr int kMaxDevices = 64;  // per-device tables of host-side state
}  // namespace fr

#define FR_DTYPE_BF16 0
#define FR_DTYPE_FP16 1
#define FR_DTYPE_FP32 2
#define FR_DTYPE_E4M3 3

namespace fr {

constexpr float kFp8Max = 448.0f;

// Streaming (nontemporal) global accesses for data read or written once:
// on MI355X a copy kernel moves 6.0-6.2 TB/s with them against 5.5 TB/s with
// plain loads and stores.
template <typename T>
__device__ __forceinline__ T ldnt(const T* p) {
  return __builtin_nontemporal_load(p);
}
template <typename T>
__device__ __forceinline__ void stnt(T* p, T v) {
  __builtin_nontemporal_store(v, p);
}
// Plain load for input that a later kernel of the decode step reads again
// (the residual stream, the queries rotated in place, the head's logits):
// a nontemporal load leaves the lines out of the caches, so the next reader
// goes to HBM; a plain one keeps them (the config-4 decode step: 1.3 % faster).
template <typename T>
__device__ __forceinline__ T ldkeep(const T* p) {
  return *p;
}
constexpr float kAmaxFloor = 1e-12f;

// ---------------------------------------------------------------- bf16 / fp16
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (gfx950 v_cvt_pk_bf16_f32; NaN stays NaN).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  bf2 v;
  v[0] = static_cast<__bf16>(lo);
  v[1] = static_cast<__bf16>(hi);
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float round_bf16(float x) {
  return bf16_to_f32(static_cast<uint16_t>(pack_bf16x2(x, 0.0f) & 0xFFFFu));
}

// Pairs of bf16 roundings with one v_cvt_pk_bf16_f32.
__device__ __forceinline__ void round_bf16x2(float& a, float& b) {
  const uint32_t w = pack_bf16x2(a, b);
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xFFFF0000u);
}

// silu(g) = g / (1 + exp(-g)) for |g| <= 80 (the result is rounded to bf16
// next).  exp(-g) = 2^a with a = fl(-g * log2(e)); the quotient by
// d = 1 + 2^a is corrected as in div_rn_shared.  The one inexact step left is
// the rounding of a, which moves 2^a by at most |a| * 2^-24 * ln 2 relative:
// with the hardware exp2, under 3 fp32 ulps for |g| <= 4; for g < -4 up to
// |g| * 6e-8 relative, on results below 0.08 in magnitude.  Against the reference's bf16 results this
// flipped no output on N(0, s^2) rows with s = 1, 4 and 20 (the variant that
// also carries a's rounding error, 4 more operations per element, agrees
// bit for bit and is 7 % slower).  In range, 2^a and d are finite and
// positive.
__device__ __forceinline__ float silu_in_range(float g) {
  const float d = 1.0f + __builtin_amdgcn_exp2f(g * -1.4426950216293335f);
  const float r = __builtin_amdgcn_rcpf(d);
  const float y = g * r;
  return __builtin_fmaf(-__builtin_fmaf(y, d, -g), r, y);
}

__device__ __forceinline__ float fp16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// fp32 -> fp16, round to nearest even, of a value already rounded to fp32,
// as one v_cvt_f16_f32 written as asm (fp16 bits in the low half, high half
// zero): a plain cast lets the compiler fold the multiply that produced x
// into the conversion (v_fma_mixlo_f16 with a zero addend: one rounding of
// the exact product), while torch rounds the fp32 product and then converts
// it; the two differ where the fp32 rounding lands on an fp16 halfway point.
__device__ __forceinline__ uint32_t fp16_bits(float x) {
  uint32_t r;
  asm("v_cvt_f16_f32 %0, %1" : "=v"(r) : "v"(x));
  return r & 0xFFFFu;
}
__device__ __forceinline__ _Float16 to_fp16(float x) {
  return __builtin_bit_cast(_Float16, static_cast<uint16_t>(fp16_bits(x)));
}

__device__ __forceinline__ uint32_t pack_fp16x2(float lo, float hi) {
  return fp16_bits(lo) | (fp16_bits(hi) << 16);
}

// Element loader: the activation dtype is a template parameter so the row
// kernels read bf16, fp16 or fp32 without a runtime branch.
template <int DT>
struct Elem;
template <>
struct Elem<FR_DTYPE_BF16> {
  using T = uint16_t;
  static __device__ __forceinline__ float load(const T* p) { return bf16_to_f32(*p); }
  // round to this dtype (RNE) and the rounded value's bit pattern
  static __device__ __forceinline__ float round(float x) { return round_bf16(x); }
  static __device__ __forceinline__ uint16_t bits(float x) {
    return static_cast<uint16_t>(pack_bf16x2(x, 0.0f) & 0xFFFFu);
  }
};
template <>
struct Elem<FR_DTYPE_FP16> {
  using T = uint16_t;
  static __device__ __forceinline__ float load(const T* p) { return fp16_to_f32(*p); }
  static __device__ __forceinline__ float round(float x) { return static_cast<float>(to_fp16(x)); }
  static __device__ __forceinline__ uint16_t bits(float x) { return __builtin_bit_cast(uint16_t, to_fp16(x)); }
};
template <>
struct Elem<FR_DTYPE_FP32> {
  using T = float;
  static __device__ __forceinline__ float load(const T* p) { return *p; }
  // fp32 activations keep their intermediates in fp32 (torch's `.to(x.dtype)`
  // is then the identity)
  static __device__ __forceinline__ float round(float x) { return x; }
  static __device__ __forceinline__ float bits(float x) { return x; }
};

// ---------------------------------------------------------------- e4m3
// Hardware pack of two fp32 values already inside [-448, 448] into e4m3
// (v_cvt_pk_fp8_f32, OCP e4m3 on gfx950, round to nearest even).
template <bool HI>
__device__ __forceinline__ uint32_t cvt_pk_e4m3(float a, float b, uint32_t old) {
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, static_cast<int>(old), HI));
}

__device__ __forceinline__ float sat448(float x) {
  return __builtin_fminf(__builtin_fmaxf(x, -kFp8Max), kFp8Max);
}

// The gfx950 conversion (v_cvt_pk_fp8_f32, no clamp) matches torch's
// `.to(float8_e4m3fn)` on every input except NaN: it always writes 0xFF,
// torch writes 0x7F | sign.  (Verified over all 65536 bf16 bit patterns and
// the over-range / inf / signed-zero / subnormal cases.)
__device__ __forceinline__ uint32_t e4m3_nan_byte(float x) {
  return (__float_as_uint(x) >> 24 & 0x80u) | 0x7Fu;
}

__device__ __forceinline__ uint32_t nan_fix4(uint32_t w, float a, float b, float c, float d) {
  if (__builtin_expect((a != a) | (b != b) | (c != c) | (d != d), 0)) {
    float v[4] = {a, b, c, d};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (v[i] != v[i]) w = (w & ~(0xFFu << (8 * i))) | (e4m3_nan_byte(v[i]) << (8 * i));
  }
  return w;
}

// Four values -> four e4m3 bytes packed little-endian, torch `.to(e4m3)`
// semantics (no prior clamp): |x| > 464, inf and NaN become NaN codes.
__device__ __forceinline__ uint32_t e4m3x4_torch(float a, float b, float c, float d) {
  uint32_t w = cvt_pk_e4m3<true>(c, d, cvt_pk_e4m3<false>(a, b, 0u));
  return nan_fix4(w, a, b, c, d);
}

// Four values that went through torch's `.clamp(-448, 448)` first (a NaN
// survives a torch clamp and becomes 0x7F | sign).
__device__ __forceinline__ uint32_t e4m3x4_clamped(float a, float b, float c, float d) {
  uint32_t w = cvt_pk_e4m3<false>(sat448(a), sat448(b), 0u);
  w = cvt_pk_e4m3<true>(sat448(c), sat448(d), w);
  return nan_fix4(w, a, b, c, d);
}

__device__ __forceinline__ uint32_t e4m3_torch_byte(float x) {
  return e4m3x4_torch(x, 0.f, 0.f, 0.f) & 0xFFu;
}
__device__ __forceinline__ uint32_t e4m3_clamped_byte(float x) {
  return e4m3x4_clamped(x, 0.f, 0.f, 0.f) & 0xFFu;
}

// ---------------------------------------------------------------- division
// Correctly rounded x / s for a divisor shared by a whole row, with r the
// correctly rounded reciprocal 1/s.  One mul + two fma (Markstein's
// correction step: with y faithful and r = RN(1/s), RN(y + r*(x - s*y)) is
// RN(x/s) barring under/overflow).  The row kernels only call this when s is
// finite and normal; otherwise they use the plain IEEE division.
// The residual is formed as y*s - x and subtracted, so both negations are
// free source modifiers and a zero quotient keeps the sign of x (-0 / s gives
// -0, as IEEE division does; s > 0 here): three VALU ops per element.
__device__ __forceinline__ float div_rn_shared(float x, float s, float r) {
  const float y = x * r;
  const float e = __builtin_fmaf(y, s, -x);
  return __builtin_fmaf(-e, r, y);
}

// ---------------------------------------------------------------- wave64 reductions
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// Reduction over aligned groups of G lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = G / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Lane i of each 16-lane row reads lane (i + N) mod 16 of the same row
// (DPP row_ror:N, a VALU operand modifier, no LDS round trip).  With N = 8
// this is lane i ^ 8.
template <int N>
__device__ __forceinline__ uint32_t row_ror(uint32_t v) {
  static_assert(N >= 1 && N <= 15, "row_ror range");
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x120 + N, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_ror8f(float v) { return __uint_as_float(row_ror<8>(__float_as_uint(v))); }

// Sum over each 16-lane row, every lane of the row gets the total.
__device__ __forceinline__ float row16_sum(float v) {
  v += __uint_as_float(row_ror<8>(__float_as_uint(v)));
  v += __uint_as_float(row_ror<4>(__float_as_uint(v)));
  v += __uint_as_float(row_ror<2>(__float_as_uint(v)));
  v += __uint_as_float(row_ror<1>(__float_as_uint(v)));
  return v;
}

// 16-byte vector type for coalesced loads/stores.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// log(sum(exp(x))) of one row held by a 256-thread workgroup, thread t owning
// the float4 chunks t + 256 j (j < NCH): the row max (wave, then the four
// wave maxima), the sum of exp(x - max) in a fixed order (per thread the
// chunks in order, each as (e0 + e1) + (e2 + e3); the wave sum; then
// (w0 + w1) + (w2 + w3)), and max + log(sum).  One definition for the
// log-softmax kernel and the top-k that folds the log-softmax in, so the two
// agree to the bit.  A NaN anywhere, or a row of -inf, gives NaN.  red: 8
// floats of LDS; every thread of the workgroup must call it.
template <int NCH>
__device__ __forceinline__ float block_row_lse(const f32x4 (&v)[NCH], float* red) {
  const int t = threadIdx.x;
  const int lane = t & 63, w = t >> 6;
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < NCH; ++j)
    m = __builtin_fmaxf(__builtin_fmaxf(m, __builtin_fmaxf(v[j].x, v[j].y)), __builtin_fmaxf(v[j].z, v[j].w));
  m = wave_max(m);
  if (lane == 0) red[w] = m;
  __syncthreads();
  m = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) s += (expf(v[j].x - m) + expf(v[j].y - m)) + (expf(v[j].z - m) + expf(v[j].w - m));
  s = wave_sum(s);
  if (lane == 0) red[4 + w] = s;
  __syncthreads();
  s = (red[4] + red[5]) + (red[6] + red[7]);
  return m + logf(s);
}

// ---------------------------------------------------------------- per-token quant
// NaN-propagating max (v_maximum3_f32): torch's amax propagates NaN.
__device__ __forceinline__ float maxnan(float a, float b) { return __builtin_elementwise_maximum(a, b); }

__device__ __forceinline__ float wave_maxnan(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = maxnan(v, __shfl_xor(v, o, 64));
  return v;
}

// Max of a 32-bit word's two bf16 magnitudes (and m), as bf16 bits.  For
// |bf16| bit patterns the unsigned order is the float order with NaN above
// inf above every finite value, so the max propagates NaN as torch's amax.
__device__ __forceinline__ uint32_t absmax_bits(uint32_t m, uint32_t w) {
  return __builtin_elementwise_max(m, __builtin_elementwise_max(w & 0x7FFFu, (w >> 16) & 0x7FFFu));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1)
    v = __builtin_elementwise_max(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), o, 64)));
  return v;
}

// e4m3 codes of 8 values of a row whose scale is amax / 448 (r = 1 / scale),
// torch's `(x / scale).clamp(-448, 448).to(e4m3)` (sglops.py:92-96).  A
// finite row (amax < 3e38) has |x / scale| <= 448 within rounding, where the
// hardware conversion equals clamp + convert, and the quotient is correctly
// rounded (div_rn_shared); a row holding NaN or inf takes the plain IEEE
// division and torch's NaN codes.
__device__ __forceinline__ u32x2 quant8_e4m3(const float* v, float scale, float r, bool finite) {
  float t[8];
  u32x2 o;
  if (finite) {
#pragma unroll
    for (int i = 0; i < 8; ++i) t[i] = div_rn_shared(v[i], scale, r);
    o[0] = cvt_pk_e4m3<true>(t[2], t[3], cvt_pk_e4m3<false>(t[0], t[1], 0u));
    o[1] = cvt_pk_e4m3<true>(t[6], t[7], cvt_pk_e4m3<false>(t[4], t[5], 0u));
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) t[i] = v[i] / scale;
    o[0] = e4m3x4_clamped(t[0], t[1], t[2], t[3]);
    o[1] = e4m3x4_clamped(t[4], t[5], t[6], t[7]);
  }
  return o;
}

}  // namespace fr
