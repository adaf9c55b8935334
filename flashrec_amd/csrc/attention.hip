// Paged attention over the e4m3 KV pool (page size 1): every query token
// attends to its own ragged list of slots.
//
// Reference: python/flashrec/attention/flashinfer.py:380-431 (_sdpa, the
// fallback that defines the result: gather k/v rows by slot, cast to the
// query dtype, scaled_dot_product_attention with scale D^-0.5, grouped-query
// heads repeated) and :240-378 (paged KV view and the decode / prefill
// plans: kv_indptr / kv_indices, page size 1, kv heads in NHD layout).  A
// query token t sees the slots kv_indices[kv_start[t] .. + kv_len[t]) — one
// token per row in decode; in causal prefill, token j of a row with prefix P
// sees P + j + 1.
//
// The work of one call goes in whole groups of 32 / NREP consecutive query
// tokens (32 query rows):
//  * paged_attn_grouped_d128 (bf16 MFMA) takes the groups whose tokens all
//    see the same first 32 slots — beams of one request decoding over their
//    shared prompt, the common case — and multiplies their shared slot
//    prefix once for all 32 queries;
//  * every other group is attended token by token on the VALU (attend_token):
//    inside the same kernel for NREP < 8, by paged_attn_tokens_d128 (a
//    second launch, more registers per wave) for NREP >= 8.
// Arithmetic in fp32 (e4m3 and bf16 convert exactly; the MFMA path rounds the
// probabilities to bf16, as the reference's bf16 SDPA does), output bf16.
#include <type_traits>

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
  const int32_t* gp;  // [groups] shared prefix rounded down to 32 (0: none), or null
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

// One (query token t, kv head kh) on the whole wave, VALU arithmetic, for
// the NREP query heads that share kv head kh.  Lanes form 8 key groups of 8
// lanes; a lane holds 16 of the 128 dims, so one key's K (or V) row for the
// head is one 128-byte gather per group (16 bytes per lane).  Keys go in
// chunks of 8 * NP: scores of a chunk stay in registers (pass 1, K), then the
// chunk is folded into a running max / sum / accumulator (pass 2, V) in the
// exp2 domain (q carries scale * log2(e)); the 8 key groups' partial sums
// are merged once at the end.  Head kh * NREP + r's output row goes to
// op0 + r * ohs (global memory, or the LDS staging of the quantizing kernel).
template <int NREP, int NP>
__device__ __forceinline__ void attend_token(const AttnArgs& a, int64_t t, int kh, int lane, uint16_t* op0,
                                             int64_t ohs) {
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
    uint16_t* op = op0 + r * ohs + d0;
    *reinterpret_cast<u32x4*>(op) = o0;
    *reinterpret_cast<u32x4*>(op + 8) = o1;
  }
}

// Whether every token of the group t0 .. t0 + ntok - 1 sees at least 32
// slots and the same first 32 of them: the grouped kernel takes exactly
// these groups (its shared prefix then has at least one 32-key block), the
// per-token kernel all others.  Wave-uniform; both kernels call this.
template <int TOK>
__device__ __forceinline__ bool group_shares_block(const AttnArgs& a, int64_t t0, int lane) {
  const int ntok = static_cast<int>(min<int64_t>(TOK, a.T - t0));
  int32_t my_start = 0, my_len = 0x7FFFFFFF;
  if (lane < ntok) {
    my_start = a.kv_start[t0 + lane];
    my_len = a.kv_len[t0 + lane];
  }
  int32_t lenmin = my_len;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) lenmin = min(lenmin, __shfl_xor(lenmin, o, 64));
  if (lenmin < 32) return false;
  // lane p compares position p % 32 of tokens p / 32, p / 32 + 2, ...
  const int pos = lane & 31;
  const int32_t s0 = a.kv_indices[__builtin_amdgcn_readlane(my_start, 0) + pos];
  bool ok = true;
  for (int tt = 1 + (lane >> 5); tt < ntok; tt += 2)
    ok = ok && a.kv_indices[__shfl(my_start, tt, 64) + pos] == s0;
  return __ballot(!ok) == 0;
}

// Longest slot prefix shared by every token of the group starting at t0,
// rounded down to a multiple of 32 (0 when the tokens do not share 32
// slots).  Lanes 0 .. TOK-1 fetch the tokens' (start, length) in one load;
// every comparison load of a 64-position chunk is issued before any is used.
template <int TOK>
__device__ __forceinline__ int32_t group_prefix32(const AttnArgs& a, int64_t t0, int lane) {
  const int ntok = static_cast<int>(min<int64_t>(TOK, a.T - t0));
  int32_t my_start = 0, my_len = 0x7FFFFFFF;
  if (lane < ntok) {
    my_start = a.kv_start[t0 + lane];
    my_len = a.kv_len[t0 + lane];
  }
  int32_t lenmin = my_len;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) lenmin = min(lenmin, __shfl_xor(lenmin, o, 64));
  int32_t starts[TOK];
#pragma unroll
  for (int tt = 0; tt < TOK; ++tt) starts[tt] = __builtin_amdgcn_readlane(my_start, tt);
  const int32_t* i0 = a.kv_indices + starts[0];
  int32_t P = 0;
  for (int32_t c = 0; c < lenmin; c += 64) {
    const int32_t pos = c + lane;
    const bool in = pos < lenmin;
    const int32_t s0 = in ? i0[pos] : 0;
    int32_t sv[TOK];
#pragma unroll
    for (int tt = 1; tt < TOK; ++tt) sv[tt] = (in && tt < ntok) ? a.kv_indices[starts[tt] + pos] : s0;
    bool ok = in;
#pragma unroll
    for (int tt = 1; tt < TOK; ++tt) ok = ok && sv[tt] == s0;
    const uint64_t bad = __ballot(!ok);
    if (bad) {
      P = c + __builtin_ctzll(bad);
      break;
    }
    P = c + 64;
  }
  P = min(P, lenmin);
  return P & ~31;
}

// The plan: one wave per group, the group's shared prefix for every layer.
template <int TOK>
__global__ __launch_bounds__(256) void attn_group_plan(AttnArgs a, int32_t* gp, int64_t groups) {
  const int lane = threadIdx.x & 63;
  const int64_t group = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (group >= groups) return;
  const int32_t p = group_prefix32<TOK>(a, group * TOK, lane);
  if (lane == 0) gp[group] = p;
}

// ---------------------------------------------------------------------------
// Grouped kernel (the default): one wave per (group of 32 / NREP consecutive
// query tokens, kv head), i.e. 32 query rows, on bf16 MFMA.
//
// Beams of one request share their prompt's slots, so consecutive decode
// rows usually attend to a common slot prefix.  The wave finds the longest
// prefix P shared by every token of its group (one ballot per 64 positions)
// and runs it in blocks of 32 keys for all 32 queries at once:
//   S^T[32 keys x 32 queries] = K . Q^T   (8 x mfma_f32_32x32x16_bf16; each
//       lane gathers 64 bytes of one key row and converts them to bf16 with
//       one op per two bytes; dims are taken in the order 64h + 8s + t on
//       both operands, which leaves the dot products unchanged)
//   online softmax per query: a lane owns one query column and 16 key rows,
//       so the block max takes one cross-lane step
//   O^T[128 x 32] += V^T . P^T  (8 MFMAs; V is staged in LDS as bf16
//       [key][dim] and read back transposed with ds_read_b64_tr_b16; the keys
//       of each 16-key chunk are taken in the order the score layout holds
//       them, so P^T feeds the B operand without a lane exchange)
// The keys past the shared prefix run through the same block with each
// token's own keys (NREP per token per block) and every query masked to its
// own token's keys.  A shared 128-slot prefix is thus read and multiplied
// once for all 32 queries (config-4 decode, 4096 beams: 25-29 us a layer,
// against 189 us token by token).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t* lds_s16x4_t;

// e4m3 x 8 (two dwords, little-endian) -> bf16 x 8, exact
__device__ __forceinline__ bf16x8_t e4m3x8_to_bf16(uint32_t w0, uint32_t w1) {
  const bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false);
  const bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true);
  const bf16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false);
  const bf16x2_t d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true);
  // each pair is one dword: the vector is the four dwords as they are
  return __builtin_bit_cast(bf16x8_t, u32x4{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                            __builtin_bit_cast(uint32_t, c), __builtin_bit_cast(uint32_t, d)});
}

constexpr int kVRow = 288;  // LDS bytes per staged V row: 256 + 32 (bank spread)

template <int NREP>
constexpr bool kSeparateTokenKernel = NREP >= 8;

// One (group, kv head kh) item on one wave; vs is the wave's 32 x kVRow
// bytes of LDS.  STAGE: the 32 query rows' outputs go to vs (row n = query
// column n, bf16 at byte 2 * dim) instead of a.out, for the quantizing
// kernel below.
template <int NREP, bool STAGE>
__device__ __forceinline__ void grouped_item(const AttnArgs& a, uint8_t* vs, int64_t group, int kh, int lane) {
  constexpr int TOK = 32 / NREP;  // tokens per group
  const int64_t t0 = group * TOK;
  const int n = lane & 31;  // query column (and key row when loading)
  const int h = lane >> 5;  // half: dims 64h .. 64h + 63
  // this lane's query and key token: t0 + n / NREP (head kh * NREP + n % NREP).
  // Its row bounds and query are fetched before the plan entry is examined,
  // so those loads share one latency with it.
  const int64_t tq = t0 + n / NREP;
  const bool qok = tq < a.T;
  const int32_t qlen = qok ? a.kv_len[tq] : 0;
  const int32_t* ik = a.kv_indices + (qok ? a.kv_start[tq] : 0);
  const int32_t* i0 = a.kv_indices + a.kv_start[t0];
  u32x4 qb[8];
  {
    const uint16_t* qp = a.q + (qok ? tq : 0) * a.sqt + (kh * NREP + n % NREP) * a.sqh + 64 * h;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      qb[s] = qok ? *reinterpret_cast<const u32x4*>(qp + 8 * s) : u32x4{0, 0, 0, 0};
  }
  // A group without a shared 32-slot block is attended token by token on
  // the VALU: here, by this wave for its kv head, when the per-token
  // registers fit two waves per SIMD (NREP < 8); otherwise by
  // paged_attn_tokens_d128, a launch of its own.
  if (a.gp ? a.gp[group] == 0 : !group_shares_block<TOK>(a, t0, lane)) {
    if constexpr (!kSeparateTokenKernel<NREP>) {
      const int ntok = static_cast<int>(min<int64_t>(TOK, a.T - t0));
      for (int tt = 0; tt < ntok; ++tt) {
        if constexpr (STAGE)
          attend_token<NREP, 16 / NREP>(a, t0 + tt, kh, lane, reinterpret_cast<uint16_t*>(vs + tt * NREP * kVRow),
                                        kVRow / 2);
        else
          attend_token<NREP, 16 / NREP>(a, t0 + tt, kh, lane, a.out + (t0 + tt) * a.sot + kh * NREP * a.soh,
                                        a.soh);
      }
    }
    return;
  }

  // ---- shared slot prefix of the group's tokens: from the plan, or found here
  const int32_t P32 = a.gp ? a.gp[group] : group_prefix32<TOK>(a, t0, lane);

  // ---- running softmax state of this lane's query (the two halves hold the
  // same m; l and O are per half: O^T rows 32mt + 8(v/4) + 4h + v%4)
  float m = -__builtin_inff(), l = 0.0f;
  f32x16_t O[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int v = 0; v < 16; ++v) O[mt][v] = 0.0f;

  // Blocks of 32 key rows.  Block b < nshared: row n is the shared slot
  // i0[32b + n] for every query; after that, row r holds position
  // P32 + j * NREP + r % NREP (j = b - nshared) of token t0 + r / NREP and
  // each query only sees its own token's rows.
  const int32_t klen = qlen;
  int32_t rest = klen - P32;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) rest = max(rest, __shfl_xor(rest, o, 64));
  const int32_t nshared = P32 / 32;
  const int32_t nblocks = nshared + (rest > 0 ? (rest + NREP - 1) / NREP : 0);

  struct Loaded {
    u32x4 kw[4], vw[4];
    bool ok;
  };
  // Gathers are unconditional (an invalid row reads slot 0's bytes); scores
  // of invalid rows are masked below and their V rows zeroed, so nothing
  // from them (not even a NaN pattern) reaches the sums.
  // Slot of this lane's key row in block bi (-1: none).  Fetched one block
  // ahead, so its load latency overlaps the previous block's work (holding
  // the next block's row gathers in registers as well measured no faster).
  auto slot_of = [&](int32_t bi) __attribute__((always_inline)) -> int32_t {
    if (bi < nshared) return i0[32 * bi + n];
    const int32_t pos = P32 + (bi - nshared) * NREP + n % NREP;
    return (bi < nblocks && pos < klen) ? ik[pos] : -1;
  };
  auto load = [&](int32_t slot, Loaded& L) __attribute__((always_inline)) {
    L.ok = slot >= 0 && slot < a.num_slots;
    const int64_t sl = L.ok ? slot : 0;
    const uint8_t* kp = a.kc + sl * a.skp + kh * a.skh + 64 * h;
    const uint8_t* vp = a.vc + sl * a.svp + kh * a.svh + 64 * h;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      L.kw[i] = *reinterpret_cast<const u32x4*>(kp + 16 * i);
      L.vw[i] = *reinterpret_cast<const u32x4*>(vp + 16 * i);
    }
  };

  auto compute = [&](int32_t bi, Loaded& L, auto own_c) __attribute__((always_inline)) {
    constexpr bool OWN = decltype(own_c)::value;
    const int32_t pos_base = P32 + (bi - nshared) * NREP;
    // bit r: key row r usable (lanes 32-63 load the same rows as 0-31)
    const uint32_t rows_ok = static_cast<uint32_t>(__ballot(L.ok));
    const bool all_rows = rows_ok == 0xFFFFFFFFu;
    if (!all_rows) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int w = 0; w < 4; ++w) L.vw[i][w] = L.ok ? L.vw[i][w] : 0u;
    }
    // S^T = K . Q^T
    f32x16_t S;
#pragma unroll
    for (int v = 0; v < 16; ++v) S[v] = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const bf16x8_t ka = e4m3x8_to_bf16(L.kw[s / 2][(s % 2) * 2], L.kw[s / 2][(s % 2) * 2 + 1]);
      S = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, __builtin_bit_cast(bf16x8_t, qb[s]), S, 0, 0, 0);
    }
    // V rows -> LDS as bf16 [key][dim]
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bf16x8_t lo = e4m3x8_to_bf16(L.vw[i][0], L.vw[i][1]);
      const bf16x8_t hi = e4m3x8_to_bf16(L.vw[i][2], L.vw[i][3]);
      *reinterpret_cast<bf16x8_t*>(vs + n * kVRow + 128 * h + 32 * i) = lo;
      *reinterpret_cast<bf16x8_t*>(vs + n * kVRow + 128 * h + 32 * i + 16) = hi;
    }
    // scores of this lane's query against key rows r = 8(v/4) + 4h + v%4,
    // unscaled (the scale is positive: the block max scales with them, and
    // each probability takes the scale in one fma)
    float x[16];
    if (!OWN && all_rows) {
#pragma unroll
      for (int v = 0; v < 16; ++v) x[v] = S[v];
    } else {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = 8 * (v / 4) + 4 * h + (v % 4);
        bool ok = (rows_ok >> r) & 1u;
        if (OWN) ok = ok && (r / NREP == n / NREP) && (pos_base + r % NREP < qlen);
        x[v] = ok ? S[v] : -__builtin_inff();
      }
    }
    float mb = x[0];
#pragma unroll
    for (int v = 1; v < 16; ++v) mb = __builtin_fmaxf(mb, x[v]);
    mb = __builtin_fmaxf(mb, __shfl_xor(mb, 32, 64)) * a.qscale;
    // Lazy rescale: probabilities are taken against the reference max m and
    // may reach 2^8; the accumulators are rescaled only when some query's
    // block max passes m + 8 (wave-uniform, so O is touched rarely).
    const bool grow = mb > m + 8.0f;
    if (__ballot(grow)) {
      const float mn = grow ? mb : m;
      const float alpha = (m == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
      m = mn;
      l *= alpha;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int v = 0; v < 16; ++v) O[mt][v] *= alpha;
    }
    // m stays -inf only while every row this query saw was masked; then
    // every x is -inf and the probabilities must be 0, not exp2(NaN)
    const float mref = m == -__builtin_inff() ? 0.0f : m;
    float pr[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      pr[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[v], a.qscale, -mref));  // x = -inf gives 0
      l += pr[v];
    }
    bf16x8_t pb[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      u32x4 w;
#pragma unroll
      for (int t = 0; t < 4; ++t) w[t] = pack_bf16x2(pr[8 * c + 2 * t], pr[8 * c + 2 * t + 1]);
      pb[c] = __builtin_bit_cast(bf16x8_t, w);
    }
    // O^T += V^T . P^T; A[dim][k] through the transposing LDS read
    const int g = lane >> 4, i16 = lane & 15;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int col = 32 * mt + 16 * (g & 1) + 4 * (i16 & 3);
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int r0 = 16 * c + 4 * h + (i16 >> 2);
        const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t)(vs + r0 * kVRow + 2 * col));
        const s16x4_t hi =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t)(vs + (r0 + 8) * kVRow + 2 * col));
        const bf16x8_t av = __builtin_bit_cast(
            bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        O[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, pb[c], O[mt], 0, 0, 0);
      }
    }
  };

  // One block's gathers at a time: holding a second block's gathers in
  // registers (as a prefetch) needs 329 registers and one wave per SIMD;
  // without it the kernel fits two waves per SIMD (launch bound below), and
  // the other wave hides the gather latency (config-4 decode 62 -> 44 us).
  Loaded LA;
  int32_t bi = 0;
  int32_t slot = nblocks > 0 ? slot_of(0) : -1;
  for (; bi < nshared; ++bi) {
    load(slot, LA);
    if (bi + 1 < nblocks) slot = slot_of(bi + 1);
    compute(bi, LA, std::false_type{});
  }
  for (; bi < nblocks; ++bi) {
    load(slot, LA);
    if (bi + 1 < nblocks) slot = slot_of(bi + 1);
    compute(bi, LA, std::true_type{});
  }

  // ---- normalise and store this lane's query (64 of its 128 dims)
  const float lt = l + __shfl_xor(l, 32, 64);
  if (!qok) return;
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  uint16_t* op = STAGE ? reinterpret_cast<uint16_t*>(vs + n * kVRow)
                       : a.out + tq * a.sot + (kh * NREP + n % NREP) * a.soh;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x2 w;
      w[0] = pack_bf16x2(O[mt][4 * j] * inv, O[mt][4 * j + 1] * inv);
      w[1] = pack_bf16x2(O[mt][4 * j + 2] * inv, O[mt][4 * j + 3] * inv);
      *reinterpret_cast<u32x2*>(op + 32 * mt + 8 * j + 4 * h) = w;
    }
}

template <int NREP>
__global__ __launch_bounds__(256, 2) void paged_attn_grouped_d128(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[4 * 32 * kVRow];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  const int64_t group = item / a.Hk;
  const int kh = static_cast<int>(item - group * a.Hk);
  if (group * (32 / NREP) >= a.T) return;
  grouped_item<NREP, false>(a, lds + wave * (32 * kVRow), group, kh, lane);
}

// Attention fused with the per-token e4m3 quant of its output (the o_proj
// input, linear.py:118-151 -> sglops.py:84-96): one workgroup per group of
// 32 / NREP tokens, wave w on kv head w (Hk <= 8, NREP < 8).  Each wave
// stages its 32 bf16 output rows in its LDS region; after a barrier, wave w
// takes tokens w, w + 8, ...: the token's Hq x 128 bf16 values (4 heads per
// pass, 8 dims per lane), row amax, scale = amax / 448 and the codes, in the
// row kernels' arithmetic (quant8_e4m3).  The codes are bit-for-bit what
// paged_attn_grouped_d128 followed by the per-token quant writes.
template <int NREP>
__global__ __launch_bounds__(512, 1) void paged_attn_grouped_quant_d128(AttnArgs a, uint8_t* qout, int64_t ldq,
                                                                        float* qscale) {
  constexpr int TOK = 32 / NREP;
  __shared__ __attribute__((aligned(16))) uint8_t lds[8 * 32 * kVRow];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t group = blockIdx.x;
  const int64_t t0 = group * TOK;
  if (t0 >= a.T) return;
  if (wave < a.Hk) grouped_item<NREP, true>(a, lds + wave * (32 * kVRow), group, wave, lane);
  __syncthreads();
  const int ntok = static_cast<int>(min<int64_t>(TOK, a.T - t0));
  const int hq = static_cast<int>(a.Hq);
  const int hl = lane >> 4;       // head inside a pass of 4
  const int dl = (lane & 15) * 8;  // first of this lane's 8 dims
  for (int tt = wave; tt < ntok; tt += 8) {
    u32x4 w[8];
    float amax = 0.0f;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int head = 4 * p + hl;
      w[p] = u32x4{0, 0, 0, 0};
      if (head < hq) {
        const uint8_t* src = lds + (head / NREP) * (32 * kVRow) + (tt * NREP + head % NREP) * kVRow + 2 * dl;
        w[p] = *reinterpret_cast<const u32x4*>(src);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        amax = maxnan(amax, __builtin_fabsf(__uint_as_float(w[p][i] << 16)));
        amax = maxnan(amax, __builtin_fabsf(__uint_as_float(w[p][i] & 0xFFFF0000u)));
      }
    }
    amax = maxnan(wave_maxnan(amax), kAmaxFloor);
    const float scale = amax / kFp8Max;
    const int64_t t = t0 + tt;
    if (lane == 0) qscale[t] = scale;
    const bool finite = amax < 3.0e38f;
    const float r = 1.0f / scale;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int head = 4 * p + hl;
      if (head < hq) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[2 * i] = __uint_as_float(w[p][i] << 16);
          v[2 * i + 1] = __uint_as_float(w[p][i] & 0xFFFF0000u);
        }
        *reinterpret_cast<u32x2*>(qout + t * ldq + head * 128 + dl) = quant8_e4m3(v, scale, r, finite);
      }
    }
  }
}

// The groups grouped_d128 leaves: one workgroup per group; its waves (8, or
// 4 for 8-wide query groups, whose per-token registers need a whole SIMD
// half) take the group's (token, kv head) pairs in turn, each on the VALU.
template <int NREP>
constexpr int token_waves() { return NREP >= 8 ? 4 : 8; }

template <int NREP>
__global__ __launch_bounds__(64 * token_waves<NREP>()) void paged_attn_tokens_d128(AttnArgs a) {
  constexpr int TOK = 32 / NREP;
  constexpr int NP = NREP >= 8 ? 1 : 16 / NREP;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * TOK;
  if (t0 >= a.T) return;
  if (a.gp ? a.gp[blockIdx.x] != 0 : group_shares_block<TOK>(a, t0, lane)) return;
  const int ntok = static_cast<int>(min<int64_t>(TOK, a.T - t0));
  const int pairs = ntok * static_cast<int>(a.Hk);
  for (int p = wave; p < pairs; p += token_waves<NREP>())
  {
    const int64_t t = t0 + p / a.Hk;
    const int kh = static_cast<int>(p % a.Hk);
    attend_token<NREP, NP>(a, t, kh, lane, a.out + t * a.sot + kh * NREP * a.soh, a.soh);
  }
}

// One launch, or two for NREP >= 8 (the token path in a kernel of its own):
// every group is taken by exactly one wave set.
template <int NREP>
static hipError_t launch_grouped(const AttnArgs& a, hipStream_t st) {
  const int64_t groups = (a.T + 32 / NREP - 1) / (32 / NREP);
  const int64_t items = groups * a.Hk;
  hipLaunchKernelGGL((paged_attn_grouped_d128<NREP>), dim3(static_cast<unsigned>((items + 3) / 4)),
                     dim3(256), 0, st, a);
  if (kSeparateTokenKernel<NREP>)
    hipLaunchKernelGGL((paged_attn_tokens_d128<NREP>), dim3(static_cast<unsigned>(groups)),
                       dim3(64 * token_waves<NREP>()), 0, st, a);
  return hipGetLastError();
}

}  // namespace fr

using namespace fr;

template <int NREP>
static hipError_t launch_grouped_quant(const AttnArgs& a, uint8_t* qout, int64_t ldq, float* qs, hipStream_t st) {
  const int64_t groups = (a.T + 32 / NREP - 1) / (32 / NREP);
  hipLaunchKernelGGL((paged_attn_grouped_quant_d128<NREP>), dim3(static_cast<unsigned>(groups)), dim3(512), 0, st,
                     a, qout, ldq, qs);
  return hipGetLastError();
}

// Checks shared by both entry points; fills `a` (output fields left unset).
static int attn_args(AttnArgs& a, const void* q, int64_t sqt, int64_t sqh, const void* k_cache, int64_t skp,
                     int64_t skh, const void* v_cache, int64_t svp, int64_t svh, int64_t num_slots,
                     const int32_t* kv_indices, const int32_t* kv_start, const int32_t* kv_len, int64_t T,
                     int64_t Hq, int64_t Hk, int64_t D, float scale, const int32_t* group_prefix) {
  if (T < 0 || Hq <= 0 || Hk <= 0 || D <= 0) return FR_EINVAL;
  if (T > 0 && (!q || !k_cache || !v_cache || !kv_indices || !kv_start || !kv_len)) return FR_EINVAL;
  if (D != 128 || Hq % Hk != 0) return FR_EUNSUPPORTED;
  const int64_t nrep = Hq / Hk;
  if (nrep != 1 && nrep != 2 && nrep != 4 && nrep != 8) return FR_EUNSUPPORTED;
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  // 16-byte vector access: row and head strides in whole 16-byte units
  if (!al16(q) || !al16(k_cache) || !al16(v_cache) || sqt % 8 || sqh % 8 || skp % 16 || skh % 16 || svp % 16 ||
      svh % 16)
    return FR_EUNSUPPORTED;
  a = AttnArgs{};
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
  a.T = T;
  a.Hq = Hq;
  a.Hk = Hk;
  a.num_slots = num_slots;
  a.qscale = scale * 1.4426950408889634f;
  a.gp = group_prefix;
  return FR_OK;
}

extern "C" int fr_paged_attention_fp8(const void* q, int64_t sqt, int64_t sqh, const void* k_cache,
                                      int64_t skp, int64_t skh, const void* v_cache, int64_t svp,
                                      int64_t svh, int64_t num_slots, const int32_t* kv_indices,
                                      const int32_t* kv_start, const int32_t* kv_len, void* out,
                                      int64_t sot, int64_t soh, int64_t T, int64_t Hq, int64_t Hk,
                                      int64_t D, float scale, const int32_t* group_prefix,
                                      void* stream) {
  AttnArgs a;
  const int rc = attn_args(a, q, sqt, sqh, k_cache, skp, skh, v_cache, svp, svh, num_slots, kv_indices, kv_start,
                           kv_len, T, Hq, Hk, D, scale, group_prefix);
  if (rc != FR_OK) return rc;
  if (T == 0) return FR_OK;
  if (!out) return FR_EINVAL;
  if ((reinterpret_cast<uintptr_t>(out) & 15u) || sot % 8 || soh % 8) return FR_EUNSUPPORTED;
  a.out = static_cast<uint16_t*>(out);
  a.sot = sot;
  a.soh = soh;
  hipError_t e;
  switch (Hq / Hk) {
    case 1: e = launch_grouped<1>(a, static_cast<hipStream_t>(stream)); break;
    case 2: e = launch_grouped<2>(a, static_cast<hipStream_t>(stream)); break;
    case 4: e = launch_grouped<4>(a, static_cast<hipStream_t>(stream)); break;
    default: e = launch_grouped<8>(a, static_cast<hipStream_t>(stream)); break;
  }
  return e == hipSuccess ? FR_OK : FR_ELAUNCH;
}

extern "C" int fr_paged_attention_quant_fp8(const void* q, int64_t sqt, int64_t sqh, const void* k_cache,
                                            int64_t skp, int64_t skh, const void* v_cache, int64_t svp,
                                            int64_t svh, int64_t num_slots, const int32_t* kv_indices,
                                            const int32_t* kv_start, const int32_t* kv_len, void* out_q,
                                            int64_t ldq, float* out_scale, int64_t T, int64_t Hq, int64_t Hk,
                                            int64_t D, float scale, const int32_t* group_prefix, void* stream) {
  AttnArgs a;
  const int rc = attn_args(a, q, sqt, sqh, k_cache, skp, skh, v_cache, svp, svh, num_slots, kv_indices, kv_start,
                           kv_len, T, Hq, Hk, D, scale, group_prefix);
  if (rc != FR_OK) return rc;
  // one wave per kv head in a workgroup of 8; 8-wide query groups take the
  // token path in a kernel of their own, which this fusion does not cover
  if (Hk > 8 || Hq / Hk == 8) return FR_EUNSUPPORTED;
  if (T == 0) return FR_OK;
  if (!out_q || !out_scale || ldq < Hq * D) return FR_EINVAL;
  if ((reinterpret_cast<uintptr_t>(out_q) & 7u) || ldq % 8) return FR_EUNSUPPORTED;  // 8-byte code stores
  uint8_t* qo = static_cast<uint8_t*>(out_q);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (Hq / Hk) {
    case 1: e = launch_grouped_quant<1>(a, qo, ldq, out_scale, st); break;
    case 2: e = launch_grouped_quant<2>(a, qo, ldq, out_scale, st); break;
    default: e = launch_grouped_quant<4>(a, qo, ldq, out_scale, st); break;
  }
  return e == hipSuccess ? FR_OK : FR_ELAUNCH;
}

extern "C" int64_t fr_paged_attention_plan_size(int64_t T, int64_t Hq, int64_t Hk) {
  if (T < 0 || Hq <= 0 || Hk <= 0 || Hq % Hk != 0) return -1;
  const int64_t nrep = Hq / Hk;
  if (nrep != 1 && nrep != 2 && nrep != 4 && nrep != 8) return -1;
  const int64_t tok = 32 / nrep;
  return (T + tok - 1) / tok;
}

extern "C" int fr_paged_attention_plan(const int32_t* kv_indices, const int32_t* kv_start,
                                       const int32_t* kv_len, int64_t T, int64_t Hq, int64_t Hk,
                                       int32_t* group_prefix, void* stream) {
  const int64_t groups = fr_paged_attention_plan_size(T, Hq, Hk);
  if (groups < 0) return FR_EUNSUPPORTED;
  if (groups == 0) return FR_OK;
  if (!kv_indices || !kv_start || !kv_len || !group_prefix) return FR_EINVAL;
  AttnArgs a{};
  a.kv_indices = kv_indices;
  a.kv_start = kv_start;
  a.kv_len = kv_len;
  a.T = T;
  a.Hq = Hq;
  a.Hk = Hk;
  const dim3 grid(static_cast<unsigned>((groups + 3) / 4)), block(256);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (Hq / Hk) {
    case 1: hipLaunchKernelGGL((attn_group_plan<32>), grid, block, 0, st, a, group_prefix, groups); break;
    case 2: hipLaunchKernelGGL((attn_group_plan<16>), grid, block, 0, st, a, group_prefix, groups); break;
    case 4: hipLaunchKernelGGL((attn_group_plan<8>), grid, block, 0, st, a, group_prefix, groups); break;
    default: hipLaunchKernelGGL((attn_group_plan<4>), grid, block, 0, st, a, group_prefix, groups); break;
  }
  return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
}
