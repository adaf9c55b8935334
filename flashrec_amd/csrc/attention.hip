// Paged attention over the e4m3 KV pool (page size 1): every query token
// attends to its own ragged list of slots.
//
// Reference: python/flashrec/attention/flashinfer.py:380-431 (_sdpa, the
// fallback that defines the result: gather k/v rows by slot, cast to the
// query dtype, scaled_dot_product_attention with scale D^-0.5, grouped-query
// heads repeated) and :240-378 (paged KV view and the decode / prefill plans:
// kv_indptr / kv_indices, page size 1, kv heads in NHD layout).  A query token t sees the slots
// kv_indices[kv_start[t] .. kv_start[t] + kv_len[t]) — one token per row in
// decode; in causal prefill, token j of a row with prefix P sees P + j + 1.
//
// Layout: one wave per (query token, kv head) computes the NREP query heads
// that share that kv head.  Lanes form 8 key groups of 8 lanes; a lane holds
// 16 of the 128 dims, so one key's K (or V) row for the head is one 128-byte
// gather per group (16 bytes per lane).  Keys go in chunks of 8 * NP: scores
// of a chunk stay in registers (pass 1, K), then the chunk is folded into a
// running max / sum / accumulator (pass 2, V) in the exp2 domain (q carries
// scale * log2(e)).  Partial sums are merged across the 8 key groups once at
// the end.  Arithmetic in fp32 (e4m3 and bf16 convert exactly), output bf16.
#include "fr_common.h"

namespace fr {

struct AttnArgs {
  const uint16_t* q;  // [T, Hq, 128] bf16
  int64_t sqt, sqh;
  const uint8_t* kc;  // [slots, Hk, 128] e4m3
  const uint8_t* vc;
  int64_t skp, skh, svp, svh;
  const int32_t* kv_indices;
  const int32_t* kv_start;  // [T]
  const int32_t* kv_len;    // [T]
  uint16_t* out;            // [T, Hq, 128] bf16
  int64_t sot, soh;
  int64_t T, Hq, Hk, num_slots;
  float qscale;  // softmax scale * log2(e)
};

// Sum over the 8 lanes of each aligned group of 8 (DPP: half-row mirror,
// then quad swaps); every lane of the group gets the total.
__device__ __forceinline__ float group8_sum(float v) {
  v += __uint_as_float(static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(__float_as_uint(v)), 0x141, 0xF, 0xF, false)));
  v += __uint_as_float(static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(__float_as_uint(v)), 0xB1, 0xF, 0xF, false)));
  v += __uint_as_float(static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(__float_as_uint(v)), 0x4E, 0xF, 0xF, false)));
  return v;
}

// e4m3 x 16 (one 16-byte load) -> fp32, exact.
__device__ __forceinline__ void e4m3x16_to_f32(const u32x4& w, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[i]), false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w[i]), true);
    f[4 * i + 0] = lo[0];
    f[4 * i + 1] = lo[1];
    f[4 * i + 2] = hi[0];
    f[4 * i + 3] = hi[1];
  }
}

template <int NREP, int NP>
__global__ __launch_bounds__(256) void paged_attn_d128(AttnArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t item =
      static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t = item / a.Hk;
  if (t >= a.T) return;
  const int kh = static_cast<int>(item - t * a.Hk);
  const int kg = lane >> 3;       // key group
  const int d0 = (lane & 7) * 16;  // first of this lane's 16 dims

  // queries of the NREP heads sharing kv head kh, pre-scaled into the exp2 domain
  float q[NREP][16];
#pragma unroll
  for (int r = 0; r < NREP; ++r) {
    const uint16_t* qp = a.q + t * a.sqt + (kh * NREP + r) * a.sqh + d0;
    const u32x4 w0 = *reinterpret_cast<const u32x4*>(qp);
    const u32x4 w1 = *reinterpret_cast<const u32x4*>(qp + 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      q[r][2 * i] = __uint_as_float(w0[i] << 16) * a.qscale;
      q[r][2 * i + 1] = __uint_as_float(w0[i] & 0xFFFF0000u) * a.qscale;
      q[r][8 + 2 * i] = __uint_as_float(w1[i] << 16) * a.qscale;
      q[r][8 + 2 * i + 1] = __uint_as_float(w1[i] & 0xFFFF0000u) * a.qscale;
    }
  }

  const int32_t len = a.kv_len[t];
  const int32_t* idx = a.kv_indices + a.kv_start[t];
  float m[NREP], l[NREP], acc[NREP][16];
#pragma unroll
  for (int r = 0; r < NREP; ++r) {
    m[r] = -__builtin_inff();
    l[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[r][i] = 0.0f;
  }

  constexpr int CH = 8 * NP;  // keys per chunk
  for (int c0 = 0; c0 < len; c0 += CH) {
    // pass 1: scores of the chunk's keys (key c0 + 8p + kg in s[p])
    int32_t slot[NP];
    float s[NP][NREP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int key = c0 + 8 * p + kg;
      int32_t sl = key < len ? idx[key] : -1;
      if (sl >= a.num_slots) sl = -1;  // outside the pool: contributes nothing
      slot[p] = sl;
    }
    u32x4 kw[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p)
      kw[p] = slot[p] >= 0 ? *reinterpret_cast<const u32x4*>(a.kc + static_cast<int64_t>(slot[p]) * a.skp + kh * a.skh + d0)
                           : u32x4{0, 0, 0, 0};
    float cm[NREP];
#pragma unroll
    for (int r = 0; r < NREP; ++r) cm[r] = -__builtin_inff();
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      float k[16];
      e4m3x16_to_f32(kw[p], k);
#pragma unroll
      for (int r = 0; r < NREP; ++r) {
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) d = __builtin_fmaf(q[r][i], k[i], d);
        d = group8_sum(d);
        s[p][r] = slot[p] >= 0 ? d : -__builtin_inff();
        cm[r] = __builtin_fmaxf(cm[r], s[p][r]);
      }
    }
    // chunk max over the 8 key groups (lanes 8 apart)
#pragma unroll
    for (int r = 0; r < NREP; ++r) {
      cm[r] = __builtin_fmaxf(cm[r], __shfl_xor(cm[r], 8, 64));
      cm[r] = __builtin_fmaxf(cm[r], __shfl_xor(cm[r], 16, 64));
      cm[r] = __builtin_fmaxf(cm[r], __shfl_xor(cm[r], 32, 64));
    }
    // fold: rescale the running state to the new max
    float mn[NREP];
#pragma unroll
    for (int r = 0; r < NREP; ++r) {
      mn[r] = __builtin_fmaxf(m[r], cm[r]);
      // mn is -inf only while every key so far is masked: keep the state zero
      const float alpha = mn[r] == -__builtin_inff() ? 1.0f : __builtin_amdgcn_exp2f(m[r] - mn[r]);
      l[r] *= alpha;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[r][i] *= alpha;
      m[r] = mn[r];
    }
    // pass 2: probabilities and V
    u32x4 vw[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p)
      vw[p] = slot[p] >= 0 ? *reinterpret_cast<const u32x4*>(a.vc + static_cast<int64_t>(slot[p]) * a.svp + kh * a.svh + d0)
                           : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      float v[16];
      e4m3x16_to_f32(vw[p], v);
#pragma unroll
      for (int r = 0; r < NREP; ++r) {
        const float pr = slot[p] >= 0 ? __builtin_amdgcn_exp2f(s[p][r] - m[r]) : 0.0f;
        l[r] += pr;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[r][i] = __builtin_fmaf(pr, v[i], acc[r][i]);
      }
    }
  }

  // merge the 8 key groups: sums over lanes 8, 16, 32 apart (each group's
  // l counts its own keys once per lane of the group, identically)
#pragma unroll
  for (int r = 0; r < NREP; ++r) {
    l[r] += __shfl_xor(l[r], 8, 64);
    l[r] += __shfl_xor(l[r], 16, 64);
    l[r] += __shfl_xor(l[r], 32, 64);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc[r][i] += __shfl_xor(acc[r][i], 8, 64);
      acc[r][i] += __shfl_xor(acc[r][i], 16, 64);
      acc[r][i] += __shfl_xor(acc[r][i], 32, 64);
    }
  }
  if (kg != 0) return;
#pragma unroll
  for (int r = 0; r < NREP; ++r) {
    // no visible key: zeros (the softmax of an empty row is undefined)
    const float inv = l[r] > 0.0f ? 1.0f / l[r] : 0.0f;
    u32x4 o0, o1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o0[i] = pack_bf16x2(acc[r][2 * i] * inv, acc[r][2 * i + 1] * inv);
      o1[i] = pack_bf16x2(acc[r][8 + 2 * i] * inv, acc[r][8 + 2 * i + 1] * inv);
    }
    uint16_t* op = a.out + t * a.sot + (kh * NREP + r) * a.soh + d0;
    *reinterpret_cast<u32x4*>(op) = o0;
    *reinterpret_cast<u32x4*>(op + 8) = o1;
  }
}

template <int NREP>
static hipError_t launch_attn(const AttnArgs& a, hipStream_t st) {
  const int64_t items = a.T * a.Hk;
  // keys per chunk 8 * NP: the chunk's scores and K/V loads stay within the
  // register budget at every group width
  constexpr int NP = NREP >= 8 ? 1 : 16 / NREP;
  hipLaunchKernelGGL((paged_attn_d128<NREP, NP>), dim3(static_cast<unsigned>((items + 3) / 4)),
                     dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace fr

using namespace fr;

extern "C" int fr_paged_attention_fp8(const void* q, int64_t sqt, int64_t sqh, const void* k_cache,
                                      int64_t skp, int64_t skh, const void* v_cache, int64_t svp,
                                      int64_t svh, int64_t num_slots, const int32_t* kv_indices,
                                      const int32_t* kv_start, const int32_t* kv_len, void* out,
                                      int64_t sot, int64_t soh, int64_t T, int64_t Hq, int64_t Hk,
                                      int64_t D, float scale, void* stream) {
  if (T < 0 || Hq <= 0 || Hk <= 0 || D <= 0) return FR_EINVAL;
  if (T == 0) return FR_OK;
  if (!q || !k_cache || !v_cache || !kv_indices || !kv_start || !kv_len || !out) return FR_EINVAL;
  if (D != 128 || Hq % Hk != 0) return FR_EUNSUPPORTED;
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  // 16-byte vector access: row and head strides in whole 16-byte units
  if (!al16(q) || !al16(k_cache) || !al16(v_cache) || !al16(out) || sqt % 8 || sqh % 8 || sot % 8 ||
      soh % 8 || skp % 16 || skh % 16 || svp % 16 || svh % 16)
    return FR_EUNSUPPORTED;
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.sqt = sqt;
  a.sqh = sqh;
  a.kc = static_cast<const uint8_t*>(k_cache);
  a.vc = static_cast<const uint8_t*>(v_cache);
  a.skp = skp;
  a.skh = skh;
  a.svp = svp;
  a.svh = svh;
  a.kv_indices = kv_indices;
  a.kv_start = kv_start;
  a.kv_len = kv_len;
  a.out = static_cast<uint16_t*>(out);
  a.sot = sot;
  a.soh = soh;
  a.T = T;
  a.Hq = Hq;
  a.Hk = Hk;
  a.num_slots = num_slots;
  a.qscale = scale * 1.4426950408889634f;
  hipError_t e;
  switch (Hq / Hk) {
    case 1: e = launch_attn<1>(a, static_cast<hipStream_t>(stream)); break;
    case 2: e = launch_attn<2>(a, static_cast<hipStream_t>(stream)); break;
    case 4: e = launch_attn<4>(a, static_cast<hipStream_t>(stream)); break;
    case 8: e = launch_attn<8>(a, static_cast<hipStream_t>(stream)); break;
    default: return FR_EUNSUPPORTED;
  }
  return e == hipSuccess ? FR_OK : FR_ELAUNCH;
}
