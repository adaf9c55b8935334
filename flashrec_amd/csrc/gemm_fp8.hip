// W8A8 fp8 GEMM on CDNA4 OCP-FP8 MFMA:
//   out[m, n] = (sum_k a[m, k] * b[k, n]) * sa[m] * sb[n] (+ bias[n])
// a: [M, K] e4m3 row-major (activations, per-row scale sa)
// b: [K, N] e4m3 column-major, i.e. N rows of K contiguous bytes
//    (weights, per-output-channel scale sb)
// Replaces python/flashrec/kernel/sglops.py:99-140 (fp8_scaled_mm), called
// from python/flashrec/layers/linear.py:153-172.
//
// Design (gfx950):
//  * 256 threads = 4 wave64 in a 2x2 grid; each wave owns a
//    (BN/2) x (BM/2) sub-tile built from 32x32 blocks of
//    v_mfma_f32_32x32x64_f8f6f4 (A-operand = weight rows, B-operand =
//    activation rows, so every lane ends up holding 4 consecutive output
//    columns and stores 8 bytes at a time).
//  * K is consumed in 128-byte tiles staged through LDS, double buffered:
//    the next tile's global loads are in flight while the current one feeds
//    the MFMAs, one barrier per K tile.
//  * LDS rows are 128 bytes (8 chunks of 16 B); chunk c of row r lives at
//    chunk slot c ^ (r & 7), so the 16-byte fragment reads of 8 consecutive
//    rows hit 8 distinct bank groups (conflict free) and the 16-byte writes
//    of one row stay conflict free as well.
//  * The MFMA's K ordering inside one instruction is irrelevant as long as
//    both operands use the same (lane group, byte) -> k assignment: lane l
//    supplies row l%32 and the 32 contiguous bytes k0 + (l/32)*32 .. +31 of
//    the current 64-byte K chunk for both operands.
//  * Workgroup -> tile mapping is XCD aware: dispatch places workgroup i on
//    XCD i % 8, so consecutive tiles (which share weight/activation panels)
//    are given to workgroups on the same XCD and its L2.
#include "fr_common.h"

namespace fr {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

struct GemmArgs {
  const uint8_t* a;
  int64_t lda;
  const uint8_t* b;
  int64_t ldb;
  const float* sa;
  int64_t sa_stride;  // 1: per-row, 0: per-tensor
  const float* sb;
  int64_t sb_stride;  // 1: per-channel, 0: per-tensor
  const void* bias;   // out dtype, [N] or null
  void* out;
  int64_t ldo;
  int64_t M, N, K;
};

constexpr int kBK = 128;  // bytes of K per LDS tile

__device__ __forceinline__ int swz(int r, int c) { return (r * 8 + (c ^ (r & 7))) * 16; }

template <int OUT>
__device__ __forceinline__ void store4(void* out, int64_t ldo, int64_t m, int64_t n, int64_t N,
                                       const float* v, const void* bias) {
  float t[4] = {v[0], v[1], v[2], v[3]};
  if (OUT == FR_DTYPE_FP32) {
    float* o = static_cast<float*>(out) + m * ldo + n;
    if (bias) {
      const float* bb = static_cast<const float*>(bias) + n;
      for (int i = 0; i < 4; ++i)
        if (n + i < N) t[i] += bb[i];
    }
    if (n + 3 < N && (ldo & 3) == 0) {
      *reinterpret_cast<float4*>(o) = make_float4(t[0], t[1], t[2], t[3]);
    } else {
      for (int i = 0; i < 4; ++i)
        if (n + i < N) o[i] = t[i];
    }
    return;
  }
  uint16_t* o = static_cast<uint16_t*>(out) + m * ldo + n;
  if (bias) {
    const uint16_t* bb = static_cast<const uint16_t*>(bias) + n;
    for (int i = 0; i < 4; ++i)
      if (n + i < N) t[i] += (OUT == FR_DTYPE_BF16) ? bf16_to_f32(bb[i]) : fp16_to_f32(bb[i]);
  }
  uint32_t lo, hi;
  if (OUT == FR_DTYPE_BF16) {
    lo = pack_bf16x2(t[0], t[1]);
    hi = pack_bf16x2(t[2], t[3]);
  } else {
    lo = pack_fp16x2(t[0], t[1]);
    hi = pack_fp16x2(t[2], t[3]);
  }
  if (n + 3 < N && (ldo & 3) == 0) {
    u32x2 w;
    w[0] = lo;
    w[1] = hi;
    *reinterpret_cast<u32x2*>(o) = w;
  } else {
    uint16_t h[4] = {(uint16_t)(lo & 0xFFFF), (uint16_t)(lo >> 16), (uint16_t)(hi & 0xFFFF),
                     (uint16_t)(hi >> 16)};
    for (int i = 0; i < 4; ++i)
      if (n + i < N) o[i] = h[i];
  }
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Raw buffer resource over [base, base + bytes): loads past the end return 0,
// which zero-fills rows beyond M / N and the K tail without branches.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// BN: weight rows (output columns) per tile, BM: activation rows per tile.
// KTAIL: K is not a multiple of the 128-byte K tile (last tile zero-filled).
template <int BN, int BM, int OUT, bool KTAIL>
__global__ __launch_bounds__(256, 1) void gemm_fp8_mfma(GemmArgs g) {
  // The host pass only needs the kernel's signature (for its launch stub);
  // the body uses device-only buffer-resource builtins.
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int FN = BN / 64;  // 32-row blocks per wave along n
  constexpr int FM = BM / 64;  // 32-row blocks per wave along m
  constexpr int IB = BN / 32;  // 1 KB direct-to-LDS loads per wave per K tile (weights)
  constexpr int IA = BM / 32;
  constexpr int STAGE = (BN + BM) * kBK;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wn = wave & 1, wm = wave >> 1;

  // ---- tile index: XCD-aware remap, then grouped ordering along m.
  const int64_t tilesN = (g.N + BN - 1) / BN;
  const int64_t tilesM = (g.M + BM - 1) / BM;
  const int64_t nt = tilesN * tilesM;
  int64_t pid = blockIdx.x;
  if ((nt & 7) == 0) pid = (pid & 7) * (nt >> 3) + (pid >> 3);
  constexpr int64_t kGroupM = 8;
  const int64_t width = kGroupM * tilesN;
  const int64_t gid = pid / width;
  const int64_t first_m = gid * kGroupM;
  const int64_t gsz = (tilesM - first_m) < kGroupM ? (tilesM - first_m) : kGroupM;
  const int64_t tm = first_m + (pid % width) % gsz;
  const int64_t tn = (pid % width) / gsz;
  const int64_t n0 = tn * BN, m0 = tm * BM;

  // ---- direct-to-LDS loads.  One wave instruction fills 1 KB = 8 rows of
  // 128 B; lane L lands in row L/8, chunk slot L%8, and therefore fetches the
  // global chunk (L%8) ^ (L/8), which realises the XOR swizzle in LDS.
  const __amdgpu_buffer_rsrc_t rb =
      make_rsrc(g.b, static_cast<uint32_t>((g.N - 1) * g.ldb + g.K));
  const __amdgpu_buffer_rsrc_t ra =
      make_rsrc(g.a, static_cast<uint32_t>((g.M - 1) * g.lda + g.K));
  const int lrow = lane >> 3;
  const int lchunk = (lane & 7) ^ lrow;
  uint32_t vob[IB], voa[IA];
#pragma unroll
  for (int i = 0; i < IB; ++i) {
    const int64_t row = n0 + (i * 4 + wave) * 8 + lrow;
    vob[i] = static_cast<uint32_t>(row * g.ldb + lchunk * 16);
  }
#pragma unroll
  for (int i = 0; i < IA; ++i) {
    const int64_t row = m0 + (i * 4 + wave) * 8 + lrow;
    voa[i] = static_cast<uint32_t>(row * g.lda + lchunk * 16);
  }
  auto issue = [&](int stage, uint32_t k0) {
    uint8_t* sb = smem + stage * STAGE;
    uint8_t* sa = sb + BN * kBK;
    const bool kin = !KTAIL || (k0 + lchunk * 16 < static_cast<uint64_t>(g.K));
#pragma unroll
    for (int i = 0; i < IB; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rb, (lds_ptr_t)(sb + (i * 4 + wave) * 1024), 16, kin ? vob[i] : 0x80000000u, k0, 0, 0);
#pragma unroll
    for (int i = 0; i < IA; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ra, (lds_ptr_t)(sa + (i * 4 + wave) * 1024), 16, kin ? voa[i] : 0x80000000u, k0, 0, 0);
  };

  v16f acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int KT = static_cast<int>((g.K + kBK - 1) / kBK);
  issue(0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const int fr = lane & 31;        // fragment row inside a 32-row block
  const int fk = (lane >> 5) * 2;  // first 16-byte chunk inside a 64-byte K chunk

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) issue(cur ^ 1, static_cast<uint32_t>(kt + 1) * kBK);
    const uint8_t* sb = smem + cur * STAGE;
    const uint8_t* sa = sb + BN * kBK;
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      v8i fb[FN], fa[FM];
      const int c0 = kc * 4 + fk;
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        const int r = wn * (BN / 2) + i * 32 + fr;
        u32x4 x0 = *reinterpret_cast<const u32x4*>(sb + swz(r, c0));
        u32x4 x1 = *reinterpret_cast<const u32x4*>(sb + swz(r, c0 + 1));
        fb[i] = v8i{(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3],
                    (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
      }
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int r = wm * (BM / 2) + j * 32 + fr;
        u32x4 x0 = *reinterpret_cast<const u32x4*>(sa + swz(r, c0));
        u32x4 x1 = *reinterpret_cast<const u32x4*>(sa + swz(r, c0 + 1));
        fa[j] = v8i{(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3],
                    (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
      }
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[i], fa[j], acc[i][j], 0, 0,
                                                                     0, 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of the next tile have landed
    __syncthreads();                 // ... and everyone's; the current tile is free
  }

  // ---- epilogue: lane holds, per block (i, j), column m = l%32 and the
  // four consecutive rows n = 8*q + 4*(l/32) + 0..3 for q = 0..3.
  const bool full = m0 + BM <= g.M && n0 + BN <= g.N && (g.ldo & 3) == 0 && g.bias == nullptr;
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int64_t m = m0 + wm * (BM / 2) + j * 32 + (lane & 31);
    if (!full && m >= g.M) continue;
    const float sam = g.sa[m * g.sa_stride];
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t n = n0 + wn * (BN / 2) + i * 32 + 8 * q + 4 * (lane >> 5);
        float v[4];
        if (full) {
          if (g.sb_stride) {
            const float4 sbv = *reinterpret_cast<const float4*>(g.sb + n);
            v[0] = (acc[i][j][4 * q + 0] * sam) * sbv.x;
            v[1] = (acc[i][j][4 * q + 1] * sam) * sbv.y;
            v[2] = (acc[i][j][4 * q + 2] * sam) * sbv.z;
            v[3] = (acc[i][j][4 * q + 3] * sam) * sbv.w;
          } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] = (acc[i][j][4 * q + t] * sam) * g.sb[0];
          }
          if (OUT == FR_DTYPE_FP32) {
            *reinterpret_cast<float4*>(static_cast<float*>(g.out) + m * g.ldo + n) =
                make_float4(v[0], v[1], v[2], v[3]);
          } else {
            u32x2 w;
            w[0] = OUT == FR_DTYPE_BF16 ? pack_bf16x2(v[0], v[1]) : pack_fp16x2(v[0], v[1]);
            w[1] = OUT == FR_DTYPE_BF16 ? pack_bf16x2(v[2], v[3]) : pack_fp16x2(v[2], v[3]);
            *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(g.out) + m * g.ldo + n) = w;
          }
          continue;
        }
        if (n >= g.N) continue;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int64_t nn = n + t < g.N ? n + t : g.N - 1;
          v[t] = (acc[i][j][4 * q + t] * sam) * g.sb[nn * g.sb_stride];
        }
        store4<OUT>(g.out, g.ldo, m, n, g.N, v, g.bias);
      }
    }
  }
#endif  // __HIP_DEVICE_COMPILE__
}

// Scalar fallback for shapes/strides the MFMA kernel does not take
// (K not a multiple of 16, unaligned operands).  One thread per output.
template <int OUT>
__global__ __launch_bounds__(256) void gemm_fp8_scalar(GemmArgs g) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= g.M * g.N) return;
  const int64_t m = idx / g.N, n = idx % g.N;
  const uint8_t* ar = g.a + m * g.lda;
  const uint8_t* br = g.b + n * g.ldb;
  float acc = 0.0f;
  for (int64_t k = 0; k < g.K; ++k)
    acc += __builtin_amdgcn_cvt_f32_fp8(ar[k], 0) * __builtin_amdgcn_cvt_f32_fp8(br[k], 0);
  float v[4] = {(acc * g.sa[m * g.sa_stride]) * g.sb[n * g.sb_stride], 0.f, 0.f, 0.f};
  // store one element through the 4-wide helper with N clipped to n + 1
  store4<OUT>(g.out, g.ldo, m, n, n + 1, v, g.bias);
}

template <int BN, int BM, int OUT>
static hipError_t launch_mfma(const GemmArgs& g, hipStream_t st) {
  const int64_t nt = ((g.N + BN - 1) / BN) * ((g.M + BM - 1) / BM);
  if (g.K % kBK == 0)
    hipLaunchKernelGGL((gemm_fp8_mfma<BN, BM, OUT, false>), dim3(static_cast<unsigned>(nt)),
                       dim3(256), 0, st, g);
  else
    hipLaunchKernelGGL((gemm_fp8_mfma<BN, BM, OUT, true>), dim3(static_cast<unsigned>(nt)),
                       dim3(256), 0, st, g);
  return hipGetLastError();
}

template <int OUT>
static hipError_t dispatch(const GemmArgs& g, hipStream_t st) {
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  // Buffer offsets are 32-bit: each operand must span < 2 GiB; the K == 0
  // case has nothing to load.
  const bool mfma_ok = g.K > 0 && g.K % 16 == 0 && g.lda % 16 == 0 && g.ldb % 16 == 0 &&
                       al16(g.a) && al16(g.b) && (g.M - 1) * g.lda + g.K < (int64_t(1) << 31) &&
                       (g.N - 1) * g.ldb + g.K < (int64_t(1) << 31);
  if (!mfma_ok) {
    const int64_t total = g.M * g.N;
    hipLaunchKernelGGL((gemm_fp8_scalar<OUT>), dim3(static_cast<unsigned>((total + 255) / 256)),
                       dim3(256), 0, st, g);
    return hipGetLastError();
  }
  // Tile choice: the largest tile that still gives at least one full wave of
  // workgroups over the 256 CUs.
  auto tiles = [&](int bn, int bm) { return ((g.N + bn - 1) / bn) * ((g.M + bm - 1) / bm); };
  if (tiles(256, 256) >= 256) return launch_mfma<256, 256, OUT>(g, st);
  if (tiles(256, 128) >= 256) return launch_mfma<256, 128, OUT>(g, st);
  return launch_mfma<128, 128, OUT>(g, st);
}

}  // namespace fr

using namespace fr;

extern "C" int fr_fp8_scaled_mm(const void* a, int64_t lda, const void* b, int64_t ldb,
                                const float* scale_a, int64_t scale_a_numel,
                                const float* scale_b, int64_t scale_b_numel, const void* bias,
                                void* out, int64_t ldo, int64_t M, int64_t N, int64_t K,
                                int out_dtype, void* stream) {
  if (M < 0 || N < 0 || K < 0) return FR_EINVAL;
  if (M == 0 || N == 0) return FR_OK;
  if (!a || !b || !scale_a || !scale_b || !out) return FR_EINVAL;
  if (lda < K || ldb < K || ldo < N) return FR_EINVAL;
  if (!(scale_a_numel == 1 || scale_a_numel == M)) return FR_EINVAL;
  if (!(scale_b_numel == 1 || scale_b_numel == N)) return FR_EINVAL;
  if (M * N > (int64_t)0x7FFFFFFF * 256) return FR_EUNSUPPORTED;
  GemmArgs g{};
  g.a = static_cast<const uint8_t*>(a);
  g.lda = lda;
  g.b = static_cast<const uint8_t*>(b);
  g.ldb = ldb;
  g.sa = scale_a;
  g.sa_stride = scale_a_numel == 1 && M != 1 ? 0 : 1;
  g.sb = scale_b;
  g.sb_stride = scale_b_numel == 1 && N != 1 ? 0 : 1;
  g.bias = bias;
  g.out = out;
  g.ldo = ldo;
  g.M = M;
  g.N = N;
  g.K = K;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t err;
  switch (out_dtype) {
    case FR_DTYPE_BF16: err = dispatch<FR_DTYPE_BF16>(g, st); break;
    case FR_DTYPE_FP16: err = dispatch<FR_DTYPE_FP16>(g, st); break;
    case FR_DTYPE_FP32: err = dispatch<FR_DTYPE_FP32>(g, st); break;
    default: return FR_EINVAL;
  }
  return err == hipSuccess ? FR_OK : FR_ELAUNCH;
}
