// Row-wise bandwidth-bound kernels of the FP8 path: per-token e4m3 quant,
// RMSNorm (+ residual add) and SiLU-and-mul, each either quantized to
// e4m3 + a per-row fp32 scale or written back as bf16.
//
// Layout: one wave64 owns one row at a time and walks rows with a grid
// stride.  The row is read once with 16-byte loads (8 bf16 per lane per
// vector), kept in VGPRs, reduced with cross-lane shuffles (no LDS, no
// barriers), and written once with coalesced 8-byte (e4m3) or 16-byte (bf16)
// stores.  Rows wider than the register budget, or with unaligned
// widths/strides, take a generic three-pass kernel with the same arithmetic.
//
// These kernels issue more VALU work per byte than the HBM can deliver
// bytes at a wave64 op per 4 clocks per SIMD, so the per-element
// instruction count is what bounds them next to bandwidth: the row kernel
// spends about 10 ops per element for RMSNorm->e4m3 and 16 for SiLU->e4m3.
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

// Grid-stride over rows, one wave per row at a time, NV vectors of 8
// elements per lane held in registers as fp32.  FULL: K == NV * 512, no
// per-vector bounds.  The kernels are VALU-issue bound (a wave64 op takes 4
// clocks on a SIMD), so the arithmetic is counted per element: unpack 1,
// norm 2 muls + bf16 round 1.5, square-sum 1 fma, amax 0.5 (maximum3 with
// |.|), quotient 3, e4m3 pack 0.5.
// Generic row: any width, any stride, any input dtype.  One wave per row,
// lane-strided elements, re-reading the row from global memory per pass.
// A loop, not unrolled, so the vector kernel can also fall back to it for a
// rare row without paying for it in registers.
//
// The RMS and SiLU modes round their intermediates to the activation dtype
// (bf16 or fp16: torch's CPU ops compute in fp32 and store in that dtype;
// fp32 rows keep them unrounded); the residual, the norm weight and the
// unquantized output rows are in that dtype too.
//
// SiLU of bf16 rows: the same arithmetic as the vector kernel and the GEMM's
// SiLU epilogue (silu_in_range for |g| <= 80, torch's formula beyond), so a
// bf16 row gives the same bits whichever kernel takes it (aligned or not,
// GEMM epilogue or row kernel).  fp16 and fp32 rows only ever take this
// kernel and keep torch's formula: their finer roundings (fp16 subnormals,
// unrounded fp32) show the last-ulp differences of the in-range form.
template <int DT>
__device__ __forceinline__ float silu_any(float g) {
  if constexpr (DT == FR_DTYPE_BF16)
    return __builtin_fabsf(g) <= 80.0f ? silu_in_range(g) : g / (1.0f + expf(-g));
  else
    return g / (1.0f + expf(-g));
}

template <int MODE, int DT, bool QOUT>
__device__ __forceinline__ void generic_row(const RowArgs& a, int64_t row, int lane) {
  using E = Elem<DT>;
  using T = typename E::T;
  using H = E;  // dtype of the RMS/SiLU intermediates
  const int64_t K = a.K;
  const T* xr = reinterpret_cast<const T*>(a.x) + row * a.ldx;
  T* rr = (MODE == kAddRms) ? reinterpret_cast<T*>(a.res) + row * a.ldr : nullptr;
  const T* wr = reinterpret_cast<const T*>(a.w);

  // Pass 1: the pre-normalisation value of each element (and the residual
  // update), plus the sum of squares.
  float ss = 0.0f;
  if (MODE == kRms || MODE == kAddRms) for (int64_t e = lane; e < K; e += 64) {
    float val = E::load(xr + e);
    if (MODE == kAddRms) {
      val = H::round(H::load(rr + e) + val);
      rr[e] = H::bits(val);
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
      val = H::load(rr + e);
    } else {
      val = E::load(xr + e);
    }
    if (MODE == kSilu) val = H::round(H::round(silu_any<DT>(val)) * E::load(xr + K + e));
    if (MODE == kRms || MODE == kAddRms) val = H::round((val * rstd) * H::load(wr + e));
    return val;
  };

  if (!QOUT) {
    T* orow = reinterpret_cast<T*>(a.q) + row * a.ldq;
    for (int64_t e = lane; e < K; e += 64) orow[e] = H::bits(value(e));
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

// Out-of-line copy for the vector kernel's rare fallback rows, so the
// fallback's registers do not count against the vector kernel's hot path.
template <int MODE, int DT, bool QOUT>
__device__ __attribute__((noinline)) void generic_row_call(RowArgs a, int64_t row, int lane) {
  generic_row<MODE, DT, QOUT>(a, row, lane);
}

template <int MODE, int DT, bool QOUT>
__global__ __launch_bounds__(256) void row_kernel_generic(RowArgs a) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= a.M) return;
  generic_row<MODE, DT, QOUT>(a, row, threadIdx.x & 63);
}

template <int MODE, int NV, bool QOUT, bool FULL>
__global__ __launch_bounds__(256) void row_kernel_vec(RowArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t K = a.K;
  auto col = [&](int j) __attribute__((always_inline)) {
    return (static_cast<int64_t>(j) * 64 + lane) * 8;
  };
  auto in = [&](int j) __attribute__((always_inline)) { return FULL || col(j) < K; };
  constexpr bool kNorm = MODE == kRms || MODE == kAddRms;
  // norm weight, loaded once per wave (kept unpacked for narrow rows)
  constexpr bool kWUnpacked = NV <= 4;
  u32x4 wp[kNorm ? NV : 1];
  float wf[kNorm && kWUnpacked ? NV : 1][8];
  if (kNorm) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      wp[j] = in(j) ? *reinterpret_cast<const u32x4*>(a.w + col(j)) : u32x4{0, 0, 0, 0};
      if (kWUnpacked) unpack8(wp[j], wf[j]);
    }
  }
  // SiLU rows: each 8-element chunk is turned into bf16(bf16(silu(g)) * u)
  // and packed back into the gate's registers as it is computed, so a row
  // costs 2 NV VGPR quads.  |g| is tracked on the way; a row holding a gate
  // beyond 80 (or inf / NaN) is redone by generic_row with torch's formula
  // literally (the in-range form's residual step does not hold there).
  auto silu_row = [&](int64_t row) __attribute__((always_inline)) {
    const uint16_t* xr = a.x + row * a.ldx;
    u32x4 p[NV], uv[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      p[j] = in(j) ? ldnt(reinterpret_cast<const u32x4*>(xr + col(j))) : u32x4{0, 0, 0, 0};
      uv[j] = in(j) ? ldnt(reinterpret_cast<const u32x4*>(xr + K + col(j))) : u32x4{0, 0, 0, 0};
    }
    auto chunk = [&](int j) __attribute__((always_inline)) {
      float g[8], u[8];
      unpack8(p[j], g);
      unpack8(uv[j], u);
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        float s0 = silu_in_range(g[i]), s1 = silu_in_range(g[i + 1]);
        round_bf16x2(s0, s1);
        p[j][i / 2] = pack_bf16x2(s0 * u[i], s1 * u[i + 1]);
      }
    };
    float gmax = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      float g[8];
      unpack8(p[j], g);
#pragma unroll
      for (int i = 0; i < 8; ++i) gmax = maxnan(gmax, __builtin_fabsf(g[i]));
      chunk(j);
    }
    if (!(wave_maxnan(gmax) <= 80.0f)) {
      generic_row_call<kSilu, FR_DTYPE_BF16, QOUT>(a, row, lane);
      return;
    }
    if (!QOUT) {
      uint16_t* orow = reinterpret_cast<uint16_t*>(a.q) + row * a.ldq;
#pragma unroll
      for (int j = 0; j < NV; ++j)
        if (in(j)) stnt(reinterpret_cast<u32x4*>(orow + col(j)), p[j]);
      return;
    }
    uint32_t mb = 0;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) mb = absmax_bits(mb, p[j][i]);
    const float amax = maxnan(__uint_as_float(wave_max_u32(mb) << 16), kAmaxFloor);
    const float scale = amax / kFp8Max;
    if (lane == 0) a.s[row] = scale;
    uint8_t* qrow = a.q + row * a.ldq;
    const bool finite = amax < 3.0e38f;
    const float r = 1.0f / scale;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      float v[8];
      unpack8(p[j], v);
      const u32x2 o = quant8_e4m3(v, scale, r, finite);
      if (in(j)) stnt(reinterpret_cast<u32x2*>(qrow + col(j)), o);
    }
  };

  const int64_t stride = static_cast<int64_t>(gridDim.x) * 4;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); row < a.M;
       row += stride) {
    if constexpr (MODE == kSilu) {
      silu_row(row);
      continue;
    }
    float v[NV][8];
    const uint16_t* xr = a.x + row * a.ldx;
    u32x4 xv[NV], uv[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (in(j)) {
        xv[j] = kNorm ? ldkeep(reinterpret_cast<const u32x4*>(xr + col(j)))
                      : ldnt(reinterpret_cast<const u32x4*>(xr + col(j)));
        if (MODE == kAddRms) uv[j] = ldkeep(reinterpret_cast<const u32x4*>(a.res + row * a.ldr + col(j)));
      } else {
        xv[j] = u32x4{0, 0, 0, 0};
        uv[j] = u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      unpack8(xv[j], v[j]);

      if (MODE == kAddRms) {
        float r[8];
        unpack8(uv[j], r);
        u32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          o[i] = pack_bf16x2(r[2 * i] + v[j][2 * i], r[2 * i + 1] + v[j][2 * i + 1]);
          v[j][2 * i] = __uint_as_float(o[i] << 16);
          v[j][2 * i + 1] = __uint_as_float(o[i] & 0xFFFF0000u);
        }
        if (in(j)) stnt(reinterpret_cast<u32x4*>(a.res + row * a.ldr + col(j)), o);
      }
    }

    if (kNorm) {
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(v[j][i], v[j][i], ss);
      ss = wave_sum(ss);
      const float var = ss / static_cast<float>(K);
      const float rstd = 1.0f / __builtin_sqrtf(var + a.eps);
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        float w[8];
        if (kWUnpacked) {
#pragma unroll
          for (int i = 0; i < 8; ++i) w[i] = wf[j][i];
        } else {
          unpack8(wp[j], w);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) v[j][i] = (v[j][i] * rstd) * w[i];
#pragma unroll
        for (int i = 0; i < 8; i += 2) round_bf16x2(v[j][i], v[j][i + 1]);
      }
    }

    if (!QOUT) {
      uint16_t* orow = reinterpret_cast<uint16_t*>(a.q) + row * a.ldq;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        if (in(j)) {
          u32x4 o;
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = pack_bf16x2(v[j][2 * i], v[j][2 * i + 1]);
          stnt(reinterpret_cast<u32x4*>(orow + col(j)), o);
        }
      }
      continue;
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
    const bool finite = amax < 3.0e38f;
    const float r = 1.0f / scale;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const u32x2 o = quant8_e4m3(v[j], scale, r, finite);
      if (in(j)) stnt(reinterpret_cast<u32x2*>(qrow + col(j)), o);
    }
  }
}

// Few rows (M up to a few per SIMD): one 256-thread workgroup per row, each
// lane with NC chunks of 8 elements (chunk c at column (256 c + tid) * 8), the
// row's sum of squares and amax reduced through LDS (wave partials summed in
// wave order).  With one wave per row the per-lane arithmetic of a whole row
// (about 10 ops per element) sits in a single wave's latency; here it is
// spread over four.  Same arithmetic as row_kernel_vec but for the order of
// the sum of squares.  quant, RMSNorm and add + RMSNorm; bf16 rows.
template <int MODE, int NC, bool QOUT>
__global__ __launch_bounds__(256) void row_kernel_split(RowArgs a) {
  static_assert(MODE != kSilu, "split rows: quant and norm modes");
  constexpr bool kNorm = MODE == kRms || MODE == kAddRms;
  __shared__ float red[2][4];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const int64_t K = a.K;
  auto col = [&](int c) __attribute__((always_inline)) { return (static_cast<int64_t>(c) * 256 + tid) * 8; };
  auto in = [&](int c) __attribute__((always_inline)) { return col(c) < K; };
  const uint16_t* xr = a.x + row * a.ldx;
  u32x4 xv[NC], uv[NC], wv[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    xv[c] = !in(c) ? u32x4{0, 0, 0, 0}
            : kNorm ? ldkeep(reinterpret_cast<const u32x4*>(xr + col(c)))
                    : ldnt(reinterpret_cast<const u32x4*>(xr + col(c)));
    if (MODE == kAddRms)
      uv[c] = in(c) ? ldkeep(reinterpret_cast<const u32x4*>(a.res + row * a.ldr + col(c))) : u32x4{0, 0, 0, 0};
    if (kNorm) wv[c] = in(c) ? *reinterpret_cast<const u32x4*>(a.w + col(c)) : u32x4{0, 0, 0, 0};
  }
  float v[NC][8];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    unpack8(xv[c], v[c]);
    if (MODE == kAddRms) {
      float r[8];
      unpack8(uv[c], r);
      u32x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[i] = pack_bf16x2(r[2 * i] + v[c][2 * i], r[2 * i + 1] + v[c][2 * i + 1]);
        v[c][2 * i] = __uint_as_float(o[i] << 16);
        v[c][2 * i + 1] = __uint_as_float(o[i] & 0xFFFF0000u);
      }
      if (in(c)) stnt(reinterpret_cast<u32x4*>(a.res + row * a.ldr + col(c)), o);
    }
  }
  if (kNorm) {
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(v[c][i], v[c][i], ss);
    ss = wave_sum(ss);
    if (lane == 0) red[0][wave] = ss;
    __syncthreads();
    ss = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
    const float var = ss / static_cast<float>(K);
    const float rstd = 1.0f / __builtin_sqrtf(var + a.eps);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float w[8];
      unpack8(wv[c], w);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[c][i] = (v[c][i] * rstd) * w[i];
#pragma unroll
      for (int i = 0; i < 8; i += 2) round_bf16x2(v[c][i], v[c][i + 1]);
    }
  }
  if (!QOUT) {
    uint16_t* orow = reinterpret_cast<uint16_t*>(a.q) + row * a.ldq;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (in(c)) {
        u32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = pack_bf16x2(v[c][2 * i], v[c][2 * i + 1]);
        stnt(reinterpret_cast<u32x4*>(orow + col(c)), o);
      }
    }
    return;
  }
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = maxnan(amax, __builtin_fabsf(v[c][i]));
  amax = wave_maxnan(amax);
  if (lane == 0) red[1][wave] = amax;
  __syncthreads();
  amax = maxnan(maxnan(maxnan(red[1][0], red[1][1]), maxnan(red[1][2], red[1][3])), kAmaxFloor);
  const float scale = amax / kFp8Max;
  if (tid == 0) a.s[row] = scale;
  uint8_t* qrow = a.q + row * a.ldq;
  const bool finite = amax < 3.0e38f;
  const float r = 1.0f / scale;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const u32x2 o = quant8_e4m3(v[c], scale, r, finite);
    if (in(c)) stnt(reinterpret_cast<u32x2*>(qrow + col(c)), o);
  }
}

template <int MODE, bool QOUT>
static hipError_t launch_split(const RowArgs& a, hipStream_t st) {
  const int64_t nc = (a.K + 2047) / 2048;
  const dim3 grid(static_cast<unsigned>(a.M));
  if (nc <= 1) hipLaunchKernelGGL((row_kernel_split<MODE, 1, QOUT>), grid, dim3(256), 0, st, a);
  else if (nc <= 2) hipLaunchKernelGGL((row_kernel_split<MODE, 2, QOUT>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((row_kernel_split<MODE, 4, QOUT>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

// Several workgroups per CU; each wave walks rows with a grid stride (the
// norm weight is unpacked once per wave).
template <int MODE, bool QOUT, int NV>
static hipError_t launch_vec(const RowArgs& a, hipStream_t st) {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  const int64_t need = (a.M + 3) / 4;
  const int64_t cap = static_cast<int64_t>(cus) * 32;  // measured best of 8, 16, 32, unbounded
  dim3 grid(static_cast<unsigned>(need < cap ? need : cap));
  if (a.K == static_cast<int64_t>(NV) * 512)
    hipLaunchKernelGGL((row_kernel_vec<MODE, NV, QOUT, true>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((row_kernel_vec<MODE, NV, QOUT, false>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

// Row counts up to which a workgroup per row beats a wave per row (RMS->e4m3
// at K = 2048, graph-replayed launches: 64 rows 3.48 -> 3.18 us, 256 rows
// 3.99 -> 3.61, 512 rows 4.16 -> 3.97; 1024 rows 4.48 -> 4.66, slower).
constexpr int64_t kSplitRowsMax = 512;

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
  if (vec && MODE != kSilu && a.M <= kSplitRowsMax) {
    err = launch_split<MODE == kSilu ? kQuant : MODE, QOUT>(a, st);
  } else if (vec) {
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
        hipLaunchKernelGGL((row_kernel_generic<MODE, FR_DTYPE_FP16, QOUT>), grid, dim3(256), 0, st, a);
        break;
      case FR_DTYPE_FP32:
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

int fr_rms_quant_fp8(const void* x, int x_dtype, int64_t ldx, void* residual, int64_t ldr,
                     const void* w, int64_t M, int64_t H, float eps, void* q, float* s, void* stream) {
  if (x_dtype != FR_DTYPE_BF16 && x_dtype != FR_DTYPE_FP16 && x_dtype != FR_DTYPE_FP32) return FR_EUNSUPPORTED;
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
  return residual ? launch_rows<kAddRms, true>(a, x_dtype, st) : launch_rows<kRms, true>(a, x_dtype, st);
}

int fr_rmsnorm(const void* x, int x_dtype, int64_t ldx, void* residual, int64_t ldr, const void* w,
               void* out, int64_t ldo, int64_t M, int64_t H, float eps, void* stream) {
  if (x_dtype != FR_DTYPE_BF16 && x_dtype != FR_DTYPE_FP16 && x_dtype != FR_DTYPE_FP32) return FR_EUNSUPPORTED;
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
  return residual ? launch_rows<kAddRms, false>(a, x_dtype, st) : launch_rows<kRms, false>(a, x_dtype, st);
}

int fr_silu_quant_fp8(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t d, void* q, float* s,
                      void* stream) {
  if (x_dtype != FR_DTYPE_BF16 && x_dtype != FR_DTYPE_FP16 && x_dtype != FR_DTYPE_FP32) return FR_EUNSUPPORTED;
  if ((M > 0 && d > 0) && (!x || !q || !s)) return FR_EINVAL;
  RowArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.q = static_cast<uint8_t*>(q);
  a.ldq = d;
  a.s = s;
  a.M = M;
  a.K = d;
  return launch_rows<kSilu, true>(a, x_dtype, static_cast<hipStream_t>(stream));
}

int fr_silu_and_mul(const void* x, int x_dtype, int64_t ldx, void* out, int64_t ldo, int64_t M, int64_t d,
                    void* stream) {
  if (x_dtype != FR_DTYPE_BF16 && x_dtype != FR_DTYPE_FP16 && x_dtype != FR_DTYPE_FP32) return FR_EUNSUPPORTED;
  if ((M > 0 && d > 0) && (!x || !out)) return FR_EINVAL;
  RowArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.q = static_cast<uint8_t*>(out);
  a.ldq = ldo;
  a.M = M;
  a.K = d;
  return launch_rows<kSilu, false>(a, x_dtype, static_cast<hipStream_t>(stream));
}

}  // extern "C"
