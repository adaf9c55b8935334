// Fused per-head Q/K RMSNorm + NeoX (rotate-half) RoPE + e4m3 paged-KV
// scatter, and the plain KV-store scatter.
//
// Replaces python/flashrec/kernel/qk_rope_kv.py:164-250 (fused op) and
// python/flashrec/kvcache/pool.py:121-139 + kernel/sglops.py:207-222
// (TokenToKVPool.store / store_kv_cache).
//
// Arithmetic: the sequential composition the reference runs when the fused
// op is off (python/flashrec/models/qwen3.py:108-128):
//   n   = bf16((x * rsqrt(mean(x^2) + eps)) * w)             per head of D
//   lo  = bf16(fl(n[i] * cos[i]) - fl(n[i+D/2] * sin[i]))     i <  D/2
//   hi  = bf16(fl(n[i+D/2] * cos[i]) + fl(n[i] * sin[i]))
//   q  <- (lo | hi) in place;  k_cache[loc, h] = e4m3(lo | hi);
//   v_cache[loc, h] = e4m3(v)     (unscaled, torch `.to(float8_e4m3fn)`)
// with cos[i] = cos_sin_cache[pos, i], sin[i] = cos_sin_cache[pos, D/2 + i].
//
// Layout: one wave64 per (token, group of 4 heads) for D = 128: 16 lanes per
// head, 8 contiguous elements (16 bytes) per lane; the rotate-half partner
// lives 8 lanes away and is fetched with a lane swap.  Each K/V head lands
// as a 128-byte contiguous run in its slot.
#include "fr_common.h"

namespace fr {

struct RopeArgs {
  uint16_t* q;
  int64_t sqt, sqh;
  const uint16_t* k;
  int64_t skt, skh;
  const uint16_t* v;
  int64_t svt, svh;
  const int64_t* pos;
  const int64_t* loc;
  const uint16_t* qw;
  const uint16_t* kw;
  float eps;
  const float* cs;
  int64_t cs_rows;
  uint8_t* kc;
  int64_t sckp, sckh;
  uint8_t* vc;
  int64_t scvp, scvh;
  int64_t num_slots;
  int64_t T;
  int Hq, Hk, D;
};

__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(v[i] << 16);
    f[2 * i + 1] = __uint_as_float(v[i] & 0xFFFF0000u);
  }
}

// D = 128, Hq % HPW == 0, Hk % HPW == 0, all head rows 16-byte aligned.
// One wave per (token, group of HPW heads of one of q / k / v): 16 lanes per
// head, HPW / 4 heads per lane, 8 contiguous elements (16 bytes) per lane per
// head.  All of a wave's loads are issued before any arithmetic so each wave
// keeps HPW / 4 KB in flight.
// MODE kRope: RoPE of q and k in place (python/flashrec/kernel/sglops.py:64-81,
// apply_rope_inplace); kNormRopeFp8: per-head norm + RoPE, q in place, K/V
// as e4m3 into the pool (the fused op); kRopeBf16: RoPE of q and k in place
// plus K/V rows copied into a bf16 pool (sglops.py:154-204,
// apply_rope_and_store_kv with matching dtypes).
enum RopeMode { kRope = 0, kNormRopeFp8 = 1, kRopeBf16 = 2 };

template <int MODE, int HPW>
__global__ __launch_bounds__(256) void qk_rope_kv_d128(RopeArgs a) {
  constexpr bool FUSED = MODE == kNormRopeFp8;  // per-head norm
  constexpr bool STORE = MODE != kRope;         // K/V go to the pool
  constexpr int R = HPW / 4;  // heads per lane
  const int lane = threadIdx.x & 63;
  const int64_t item =
      static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int qg = a.Hq / HPW, kg = a.Hk / HPW;
  const int per_tok = STORE ? qg + 2 * kg : qg + kg;
  const int64_t t = item / per_tok;
  if (t >= a.T) return;
  const int g = static_cast<int>(item - t * per_tok);
  const int hs = lane >> 4;  // head slot inside a group of 4
  const int j = lane & 15;   // 8-element chunk inside the head
  const int e0 = j * 8;

  // a token whose position has no cos/sin row writes neither its K nor its
  // V row (the slot keeps its old contents rather than a new V beside an
  // old K)
  const int64_t slot = STORE ? a.loc[t] : 0;
  const int64_t tpos = a.pos[t];
  const bool slot_ok = slot >= 0 && slot < a.num_slots && tpos >= 0 && tpos < a.cs_rows;

  if (STORE && g >= qg + kg) {  // V: e4m3 conversion or bf16 copy into the slot
    if (!slot_ok) return;
    const int h0 = (g - qg - kg) * HPW + hs;
    u32x4 xv[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
      xv[r] = ldnt(reinterpret_cast<const u32x4*>(a.v + t * a.svt + (h0 + 4 * r) * a.svh + e0));
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (MODE == kRopeBf16) {
        stnt(reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(a.vc) + slot * a.scvp +
                                      (h0 + 4 * r) * a.scvh + e0),
             xv[r]);
        continue;
      }
      float x[8];
      unpack8(xv[r], x);
      u32x2 o;
      o[0] = e4m3x4_torch(x[0], x[1], x[2], x[3]);
      o[1] = e4m3x4_torch(x[4], x[5], x[6], x[7]);
      stnt(reinterpret_cast<u32x2*>(a.vc + slot * a.scvp + (h0 + 4 * r) * a.scvh + e0), o);
    }
    return;
  }
  const bool is_q = g < qg;
  const int h0 = (is_q ? g : g - qg) * HPW + hs;
  const uint16_t* src = is_q ? a.q + t * a.sqt + h0 * a.sqh : a.k + t * a.skt + h0 * a.skh;
  const int64_t hstride = is_q ? a.sqh : a.skh;
  const uint16_t* wp = is_q ? a.qw : a.kw;
  const int64_t pos = a.pos[t];

  u32x4 xv[R];
#pragma unroll
  for (int r = 0; r < R; ++r) xv[r] = ldkeep(reinterpret_cast<const u32x4*>(src + 4 * r * hstride + e0));
  u32x4 wv;
  if (FUSED) wv = *reinterpret_cast<const u32x4*>(wp + e0);
  if (pos < 0 || pos >= a.cs_rows) return;  // no cache row: leave q / slot untouched
  const float* csr = a.cs + pos * 128;
  const int c0 = e0 & 63;
  const float4 ca = *reinterpret_cast<const float4*>(csr + c0);
  const float4 cb = *reinterpret_cast<const float4*>(csr + c0 + 4);
  const float4 sa = *reinterpret_cast<const float4*>(csr + 64 + c0);
  const float4 sb = *reinterpret_cast<const float4*>(csr + 64 + c0 + 4);
  const float cv[8] = {ca.x, ca.y, ca.z, ca.w, cb.x, cb.y, cb.z, cb.w};
  // rotate-half: the first half subtracts the partner's sin term, the second
  // adds it; the sign goes into sin once per token (negation is exact)
  const float sg = j < 8 ? -1.0f : 1.0f;
  const float sv[8] = {sa.x * sg, sa.y * sg, sa.z * sg, sa.w * sg,
                       sb.x * sg, sb.y * sg, sb.z * sg, sb.w * sg};
  float w[8];
  if (FUSED) unpack8(wv, w);

#pragma unroll
  for (int r = 0; r < R; ++r) {
    // the normed head as packed bf16 (the reference rounds it to bf16)
    u32x4 nb;
    if (FUSED) {
      float x[8];
      unpack8(xv[r], x);
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(x[i], x[i], ss);
      ss = row16_sum(ss);
      // mean over D = 128: the power-of-two scale is exact
      const float rstd = 1.0f / __builtin_sqrtf(ss * (1.0f / 128.0f) + a.eps);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        nb[i] = pack_bf16x2((x[2 * i] * rstd) * w[2 * i], (x[2 * i + 1] * rstd) * w[2 * i + 1]);
    } else {
      nb = xv[r];
    }
    // partner half: lane j ^ 8 holds elements e0 +- 64
    float n[8], p[8];
    unpack8(nb, n);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t other = row_ror<8>(nb[i]);
      p[2 * i] = __uint_as_float(other << 16);
      p[2 * i + 1] = __uint_as_float(other & 0xFFFF0000u);
    }
    // y packed to bf16 once (the reference's bf16 result)
    u32x4 yb;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      yb[i] = pack_bf16x2(n[2 * i] * cv[2 * i] + p[2 * i] * sv[2 * i],
                          n[2 * i + 1] * cv[2 * i + 1] + p[2 * i + 1] * sv[2 * i + 1]);
    const int h = h0 + 4 * r;
    if (is_q || !FUSED) {
      const u32x4 o = yb;
      uint16_t* dst = is_q ? a.q + t * a.sqt + h * a.sqh : const_cast<uint16_t*>(a.k + t * a.skt + h * a.skh);
      stnt(reinterpret_cast<u32x4*>(dst + e0), o);
      if (MODE == kRopeBf16 && !is_q && slot_ok)
        stnt(reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(a.kc) + slot * a.sckp + h * a.sckh + e0), o);
    } else if (slot_ok) {
      float y[8];
      unpack8(yb, y);
      u32x2 o;
      o[0] = e4m3x4_torch(y[0], y[1], y[2], y[3]);
      o[1] = e4m3x4_torch(y[4], y[5], y[6], y[7]);
      stnt(reinterpret_cast<u32x2*>(a.kc + slot * a.sckp + h * a.sckh + e0), o);
    }
  }
}

// Any even D <= 128, any head counts / element alignment: one wave per
// (token, head); lane i < D/2 owns the rotate-half pair (i, i + D/2).
template <int MODE>
__global__ __launch_bounds__(256) void qk_rope_kv_generic(RopeArgs a) {
  constexpr bool FUSED = MODE == kNormRopeFp8;
  constexpr bool STORE = MODE != kRope;
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int per_tok = STORE ? a.Hq + 2 * a.Hk : a.Hq + a.Hk;
  const int64_t t = item / per_tok;
  if (t >= a.T) return;
  const int hh = static_cast<int>(item - t * per_tok);
  const int half = a.D >> 1;
  const bool active = lane < half;
  const int64_t slot = STORE ? a.loc[t] : 0;
  const int64_t tpos = a.pos[t];
  const bool slot_ok = slot >= 0 && slot < a.num_slots && tpos >= 0 && tpos < a.cs_rows;
  if (STORE && hh >= a.Hq + a.Hk) {
    const int h = hh - a.Hq - a.Hk;
    if (!slot_ok || !active) return;
    const uint16_t* src = a.v + t * a.svt + h * a.svh;
    if (MODE == kRopeBf16) {
      uint16_t* dst = reinterpret_cast<uint16_t*>(a.vc) + slot * a.scvp + h * a.scvh;
      dst[lane] = src[lane];
      dst[lane + half] = src[lane + half];
      return;
    }
    uint8_t* dst = a.vc + slot * a.scvp + h * a.scvh;
    dst[lane] = static_cast<uint8_t>(e4m3_torch_byte(bf16_to_f32(src[lane])));
    dst[lane + half] = static_cast<uint8_t>(e4m3_torch_byte(bf16_to_f32(src[lane + half])));
    return;
  }
  const bool is_q = hh < a.Hq;
  const int h = is_q ? hh : hh - a.Hq;
  const uint16_t* src = is_q ? a.q + t * a.sqt + h * a.sqh : a.k + t * a.skt + h * a.skh;
  const uint16_t* wp = is_q ? a.qw : a.kw;
  const float x1 = active ? bf16_to_f32(src[lane]) : 0.0f;
  const float x2 = active ? bf16_to_f32(src[lane + half]) : 0.0f;
  float n1 = x1, n2 = x2;
  if (FUSED) {
    const float ss = wave_sum(x1 * x1 + x2 * x2);
    const float rstd = 1.0f / __builtin_sqrtf(ss / static_cast<float>(a.D) + a.eps);
    if (!active) return;
    n1 = round_bf16((x1 * rstd) * bf16_to_f32(wp[lane]));
    n2 = round_bf16((x2 * rstd) * bf16_to_f32(wp[lane + half]));
  }
  if (!active) return;
  const int64_t pos = a.pos[t];
  if (pos < 0 || pos >= a.cs_rows) return;
  const float c = a.cs[pos * a.D + lane];
  const float s = a.cs[pos * a.D + half + lane];
  const float y1 = round_bf16(n1 * c - n2 * s);
  const float y2 = round_bf16(n2 * c + n1 * s);
  if (is_q || !FUSED) {
    uint16_t* dq = is_q ? a.q + t * a.sqt + h * a.sqh : const_cast<uint16_t*>(src);
    const uint16_t b1 = static_cast<uint16_t>(pack_bf16x2(y1, 0.f) & 0xFFFFu);
    const uint16_t b2 = static_cast<uint16_t>(pack_bf16x2(y2, 0.f) & 0xFFFFu);
    dq[lane] = b1;
    dq[lane + half] = b2;
    if (MODE == kRopeBf16 && !is_q && slot_ok) {
      uint16_t* dk = reinterpret_cast<uint16_t*>(a.kc) + slot * a.sckp + h * a.sckh;
      dk[lane] = b1;
      dk[lane + half] = b2;
    }
  } else if (slot_ok) {
    uint8_t* dst = a.kc + slot * a.sckp + h * a.sckh;
    dst[lane] = static_cast<uint8_t>(e4m3_torch_byte(y1));
    dst[lane + half] = static_cast<uint8_t>(e4m3_torch_byte(y2));
  }
}

// NeoX rotate-half RoPE in place for layouts the kernels above do not take:
// bf16, fp16 or fp32 heads, any even D, any element strides.  One wave per
// (token, head), lane i walking the rotate-half pairs (i, i + D/2) with a
// stride of 64.  The arithmetic is torch's for a head of that dtype times
// the fp32 cos/sin rows: y1 = x1*c - x2*s, y2 = x2*c + x1*s in fp32, then one
// rounding to the head's dtype (none for fp32).
struct RopeAnyArgs {
  void* q;
  int64_t sqt, sqh, sqd;
  void* k;
  int64_t skt, skh, skd;
  const int64_t* pos;
  const float* cs;
  int64_t cs_rows;
  int64_t T;
  int Hq, Hk, D;
};

template <int DT>
__global__ __launch_bounds__(256) void rope_inplace_any(RopeAnyArgs a) {
  using E = Elem<DT>;
  using T = typename E::T;
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int per_tok = a.Hq + a.Hk;
  const int64_t t = item / per_tok;
  if (t >= a.T) return;
  const int hh = static_cast<int>(item - t * per_tok);
  const int64_t pos = a.pos[t];
  if (pos < 0 || pos >= a.cs_rows) return;
  const bool is_q = hh < a.Hq;
  const int h = is_q ? hh : hh - a.Hq;
  T* x = is_q ? static_cast<T*>(a.q) + t * a.sqt + h * a.sqh : static_cast<T*>(a.k) + t * a.skt + h * a.skh;
  const int64_t sd = is_q ? a.sqd : a.skd;
  const int half = a.D >> 1;
  const float* csr = a.cs + pos * a.D;
  for (int i = lane; i < half; i += 64) {
    const float x1 = E::load(x + i * sd), x2 = E::load(x + (i + half) * sd);
    const float c = csr[i], s = csr[half + i];
    const float y1 = x1 * c - x2 * s;
    const float y2 = x2 * c + x1 * s;
    x[i * sd] = E::bits(y1);
    x[(i + half) * sd] = E::bits(y2);
  }
}

// k/v rows [T, row_dim] (bf16 or e4m3) -> k_cache/v_cache rows at loc[t].
template <bool SRC_BF16>
__global__ __launch_bounds__(256) void store_kv_kernel(const void* k, int64_t skt, const void* v,
                                                       int64_t svt, const int64_t* loc,
                                                       uint8_t* kc, int64_t sck, uint8_t* vc,
                                                       int64_t scv, int64_t num_slots, int64_t T,
                                                       int64_t row_dim, bool vec) {
  const int64_t per_row = vec ? row_dim / 8 : row_dim;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= 2 * T * per_row) return;
  const int which = static_cast<int>(idx / (T * per_row));  // 0 = K, 1 = V
  const int64_t r = idx - which * T * per_row;
  const int64_t t = r / per_row;
  const int64_t c = r - t * per_row;
  const int64_t slot = loc[t];
  if (slot < 0 || slot >= num_slots) return;
  const int64_t st = which ? svt : skt;
  uint8_t* dst = (which ? vc : kc) + slot * (which ? scv : sck);
  if (SRC_BF16) {
    const uint16_t* src = static_cast<const uint16_t*>(which ? v : k) + t * st;
    if (vec) {
      u32x4 xv = *reinterpret_cast<const u32x4*>(src + c * 8);
      float x[8];
      unpack8(xv, x);
      u32x2 o;
      o[0] = e4m3x4_torch(x[0], x[1], x[2], x[3]);
      o[1] = e4m3x4_torch(x[4], x[5], x[6], x[7]);
      *reinterpret_cast<u32x2*>(dst + c * 8) = o;
    } else {
      dst[c] = static_cast<uint8_t>(e4m3_torch_byte(bf16_to_f32(src[c])));
    }
  } else {
    const uint8_t* src = static_cast<const uint8_t*>(which ? v : k) + t * st;
    if (vec) {
      *reinterpret_cast<u32x2*>(dst + c * 8) = *reinterpret_cast<const u32x2*>(src + c * 8);
    } else {
      dst[c] = src[c];
    }
  }
}

// bf16 K/V rows -> a bf16 pool (plain row copy to loc[t]); 16-byte pieces
// when every row and stride allows it.
__global__ __launch_bounds__(256) void store_kv_bf16_kernel(const uint16_t* k, int64_t skt,
                                                            const uint16_t* v, int64_t svt,
                                                            const int64_t* loc, uint16_t* kc,
                                                            int64_t sck, uint16_t* vc, int64_t scv,
                                                            int64_t num_slots, int64_t T,
                                                            int64_t row_dim, bool vec) {
  const int64_t per_row = vec ? row_dim / 8 : row_dim;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= 2 * T * per_row) return;
  const int which = static_cast<int>(idx / (T * per_row));  // 0 = K, 1 = V
  const int64_t r = idx - which * T * per_row;
  const int64_t t = r / per_row;
  const int64_t c = r - t * per_row;
  const int64_t slot = loc[t];
  if (slot < 0 || slot >= num_slots) return;
  const uint16_t* src = (which ? v : k) + t * (which ? svt : skt);
  uint16_t* dst = (which ? vc : kc) + slot * (which ? scv : sck);
  if (vec)
    *reinterpret_cast<u32x4*>(dst + c * 8) = *reinterpret_cast<const u32x4*>(src + c * 8);
  else
    dst[c] = src[c];
}

}  // namespace fr

using namespace fr;

extern "C" {

int fr_qk_norm_rope_store_fp8(void* q, int64_t sqt, int64_t sqh, const void* k, int64_t skt,
                              int64_t skh, const void* v, int64_t svt, int64_t svh,
                              const int64_t* positions, const int64_t* loc, const void* q_weight,
                              const void* k_weight, float eps, const float* cos_sin_cache,
                              int64_t cache_rows, void* k_cache, int64_t sckp, int64_t sckh,
                              void* v_cache, int64_t scvp, int64_t scvh, int64_t num_slots,
                              int64_t T, int64_t Hq, int64_t Hk, int64_t D, void* stream) {
  if (T < 0 || Hq < 0 || Hk < 0) return FR_EINVAL;
  if (D <= 0 || D > 128 || (D & 1)) return FR_EUNSUPPORTED;
  if (T == 0) return FR_OK;
  if (!q || !k || !v || !positions || !loc || !q_weight || !k_weight || !cos_sin_cache ||
      !k_cache || !v_cache)
    return FR_EINVAL;
  RopeArgs a{};
  a.q = static_cast<uint16_t*>(q);
  a.sqt = sqt; a.sqh = sqh;
  a.k = static_cast<const uint16_t*>(k);
  a.skt = skt; a.skh = skh;
  a.v = static_cast<const uint16_t*>(v);
  a.svt = svt; a.svh = svh;
  a.pos = positions;
  a.loc = loc;
  a.qw = static_cast<const uint16_t*>(q_weight);
  a.kw = static_cast<const uint16_t*>(k_weight);
  a.eps = eps;
  a.cs = cos_sin_cache;
  a.cs_rows = cache_rows;
  a.kc = static_cast<uint8_t*>(k_cache);
  a.sckp = sckp; a.sckh = sckh;
  a.vc = static_cast<uint8_t*>(v_cache);
  a.scvp = scvp; a.scvh = scvh;
  a.num_slots = num_slots;
  a.T = T;
  a.Hq = static_cast<int>(Hq);
  a.Hk = static_cast<int>(Hk);
  a.D = static_cast<int>(D);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto al = [](const void* p, unsigned m) { return (reinterpret_cast<uintptr_t>(p) & (m - 1)) == 0; };
  const bool fast = D == 128 && Hq % 4 == 0 && Hk % 4 == 0 && al(q, 16) && al(k, 16) && al(v, 16) &&
                    sqt % 8 == 0 && sqh % 8 == 0 && skt % 8 == 0 && skh % 8 == 0 &&
                    svt % 8 == 0 && svh % 8 == 0 && al(q_weight, 16) && al(k_weight, 16) &&
                    al(cos_sin_cache, 16) && al(k_cache, 8) && al(v_cache, 8) && sckp % 8 == 0 &&
                    sckh % 8 == 0 && scvp % 8 == 0 && scvh % 8 == 0;
  if (fast && Hq % 8 == 0 && Hk % 8 == 0) {
    const int64_t items = T * (Hq / 8 + 2 * (Hk / 8));
    hipLaunchKernelGGL((qk_rope_kv_d128<kNormRopeFp8, 8>), dim3(static_cast<unsigned>((items + 3) / 4)),
                       dim3(256), 0, st, a);
  } else if (fast) {
    const int64_t items = T * (Hq / 4 + 2 * (Hk / 4));
    hipLaunchKernelGGL((qk_rope_kv_d128<kNormRopeFp8, 4>), dim3(static_cast<unsigned>((items + 3) / 4)),
                       dim3(256), 0, st, a);
  } else {
    const int64_t items = T * (Hq + 2 * Hk);
    hipLaunchKernelGGL(qk_rope_kv_generic<kNormRopeFp8>, dim3(static_cast<unsigned>((items + 3) / 4)), dim3(256),
                       0, st, a);
  }
  return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
}

int fr_rope_inplace(void* q, int64_t sqt, int64_t sqh, void* k, int64_t skt, int64_t skh,
                    const int64_t* positions, const float* cos_sin_cache, int64_t cache_rows,
                    int64_t T, int64_t Hq, int64_t Hk, int64_t D, void* stream) {
  if (T < 0 || Hq < 0 || Hk < 0) return FR_EINVAL;
  if (D <= 0 || D > 128 || (D & 1)) return FR_EUNSUPPORTED;
  if (T == 0) return FR_OK;
  if (!q || !k || !positions || !cos_sin_cache) return FR_EINVAL;
  RopeArgs a{};
  a.q = static_cast<uint16_t*>(q);
  a.sqt = sqt; a.sqh = sqh;
  a.k = static_cast<const uint16_t*>(k);
  a.skt = skt; a.skh = skh;
  a.pos = positions;
  a.cs = cos_sin_cache;
  a.cs_rows = cache_rows;
  a.num_slots = 1;
  a.T = T;
  a.Hq = static_cast<int>(Hq);
  a.Hk = static_cast<int>(Hk);
  a.D = static_cast<int>(D);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto al = [](const void* p, unsigned m) { return (reinterpret_cast<uintptr_t>(p) & (m - 1)) == 0; };
  const bool fast = D == 128 && Hq % 4 == 0 && Hk % 4 == 0 && al(q, 16) && al(k, 16) &&
                    sqt % 8 == 0 && sqh % 8 == 0 && skt % 8 == 0 && skh % 8 == 0 &&
                    al(cos_sin_cache, 16);
  if (fast) {
    const int64_t items = T * (Hq / 4 + Hk / 4);
    hipLaunchKernelGGL((qk_rope_kv_d128<kRope, 4>), dim3(static_cast<unsigned>((items + 3) / 4)),
                       dim3(256), 0, st, a);
  } else {
    const int64_t items = T * (Hq + Hk);
    hipLaunchKernelGGL(qk_rope_kv_generic<kRope>, dim3(static_cast<unsigned>((items + 3) / 4)),
                       dim3(256), 0, st, a);
  }
  return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
}

int fr_rope_inplace_any(void* q, int64_t sqt, int64_t sqh, int64_t sqd, void* k, int64_t skt, int64_t skh,
                        int64_t skd, int dtype, const int64_t* positions, const float* cos_sin_cache,
                        int64_t cache_rows, int64_t T, int64_t Hq, int64_t Hk, int64_t D, void* stream) {
  if (T < 0 || Hq < 0 || Hk < 0 || D <= 0 || (D & 1)) return FR_EINVAL;
  if (dtype != FR_DTYPE_BF16 && dtype != FR_DTYPE_FP16 && dtype != FR_DTYPE_FP32) return FR_EUNSUPPORTED;
  if (T == 0 || Hq + Hk == 0) return FR_OK;
  if (!q || !k || !positions || !cos_sin_cache) return FR_EINVAL;
  // grid of items / 4 workgroups (< 2^31)
  if (Hq + Hk > 0x7FFFFFFF || T > (int64_t(1) << 33) / (Hq + Hk)) return FR_EUNSUPPORTED;
  RopeAnyArgs a{};
  a.q = q;
  a.sqt = sqt; a.sqh = sqh; a.sqd = sqd;
  a.k = k;
  a.skt = skt; a.skh = skh; a.skd = skd;
  a.pos = positions;
  a.cs = cos_sin_cache;
  a.cs_rows = cache_rows;
  a.T = T;
  a.Hq = static_cast<int>(Hq);
  a.Hk = static_cast<int>(Hk);
  a.D = static_cast<int>(D);
  const int64_t items = T * (Hq + Hk);
  const dim3 grid(static_cast<unsigned>((items + 3) / 4));
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case FR_DTYPE_BF16: hipLaunchKernelGGL(rope_inplace_any<FR_DTYPE_BF16>, grid, dim3(256), 0, st, a); break;
    case FR_DTYPE_FP16: hipLaunchKernelGGL(rope_inplace_any<FR_DTYPE_FP16>, grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL(rope_inplace_any<FR_DTYPE_FP32>, grid, dim3(256), 0, st, a); break;
  }
  return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
}

int fr_store_kv_fp8(const void* k, int64_t skt, const void* v, int64_t svt, int src_dtype,
                    const int64_t* loc, void* k_cache, int64_t sck, void* v_cache, int64_t scv,
                    int64_t num_slots, int64_t T, int64_t row_dim, void* stream) {
  if (T < 0 || row_dim < 0) return FR_EINVAL;
  if (T == 0 || row_dim == 0) return FR_OK;
  if (!k || !v || !loc || !k_cache || !v_cache) return FR_EINVAL;
  if (src_dtype != FR_DTYPE_BF16 && src_dtype != FR_DTYPE_E4M3) return FR_EUNSUPPORTED;
  auto al = [](const void* p, unsigned m) { return (reinterpret_cast<uintptr_t>(p) & (m - 1)) == 0; };
  const unsigned sal = src_dtype == FR_DTYPE_BF16 ? 16 : 8;
  const bool vec = row_dim % 8 == 0 && skt % 8 == 0 && svt % 8 == 0 && sck % 8 == 0 &&
                   scv % 8 == 0 && al(k, sal) && al(v, sal) && al(k_cache, 8) && al(v_cache, 8);
  const int64_t per_row = vec ? row_dim / 8 : row_dim;
  const int64_t total = 2 * T * per_row;
  dim3 grid(static_cast<unsigned>((total + 255) / 256));
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint8_t* kc = static_cast<uint8_t*>(k_cache);
  uint8_t* vc = static_cast<uint8_t*>(v_cache);
  if (src_dtype == FR_DTYPE_BF16)
    hipLaunchKernelGGL(store_kv_kernel<true>, grid, dim3(256), 0, st, k, skt, v, svt, loc, kc, sck,
                       vc, scv, num_slots, T, row_dim, vec);
  else
    hipLaunchKernelGGL(store_kv_kernel<false>, grid, dim3(256), 0, st, k, skt, v, svt, loc, kc, sck,
                       vc, scv, num_slots, T, row_dim, vec);
  return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
}

int fr_store_kv_bf16(const void* k, int64_t skt, const void* v, int64_t svt, const int64_t* loc,
                     void* k_cache, int64_t sck, void* v_cache, int64_t scv, int64_t num_slots,
                     int64_t T, int64_t row_dim, void* stream) {
  if (T < 0 || row_dim < 0) return FR_EINVAL;
  if (T == 0 || row_dim == 0) return FR_OK;
  if (!k || !v || !loc || !k_cache || !v_cache) return FR_EINVAL;
  auto al = [](const void* p, unsigned m) { return (reinterpret_cast<uintptr_t>(p) & (m - 1)) == 0; };
  const bool vec = row_dim % 8 == 0 && skt % 8 == 0 && svt % 8 == 0 && sck % 8 == 0 &&
                   scv % 8 == 0 && al(k, 16) && al(v, 16) && al(k_cache, 16) && al(v_cache, 16);
  const int64_t per_row = vec ? row_dim / 8 : row_dim;
  const int64_t total = 2 * T * per_row;
  hipLaunchKernelGGL(store_kv_bf16_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(k), skt,
                     static_cast<const uint16_t*>(v), svt, loc, static_cast<uint16_t*>(k_cache), sck,
                     static_cast<uint16_t*>(v_cache), scv, num_slots, T, row_dim, vec);
  return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
}

int fr_rope_store_kv_bf16(void* q, int64_t sqt, int64_t sqh, void* k, int64_t skt, int64_t skh,
                          const void* v, int64_t svt, int64_t svh, const int64_t* positions,
                          const int64_t* loc, const float* cos_sin_cache, int64_t cache_rows,
                          void* k_cache, int64_t sckp, int64_t sckh, void* v_cache, int64_t scvp,
                          int64_t scvh, int64_t num_slots, int64_t T, int64_t Hq, int64_t Hk,
                          int64_t D, void* stream) {
  if (T < 0 || Hq < 0 || Hk < 0) return FR_EINVAL;
  if (D <= 0 || D > 128 || (D & 1)) return FR_EUNSUPPORTED;
  if (T == 0) return FR_OK;
  if (!q || !k || !v || !positions || !loc || !cos_sin_cache || !k_cache || !v_cache) return FR_EINVAL;
  RopeArgs a{};
  a.q = static_cast<uint16_t*>(q);
  a.sqt = sqt; a.sqh = sqh;
  a.k = static_cast<const uint16_t*>(k);
  a.skt = skt; a.skh = skh;
  a.v = static_cast<const uint16_t*>(v);
  a.svt = svt; a.svh = svh;
  a.pos = positions;
  a.loc = loc;
  a.cs = cos_sin_cache;
  a.cs_rows = cache_rows;
  a.kc = static_cast<uint8_t*>(k_cache);
  a.sckp = sckp; a.sckh = sckh;
  a.vc = static_cast<uint8_t*>(v_cache);
  a.scvp = scvp; a.scvh = scvh;
  a.num_slots = num_slots;
  a.T = T;
  a.Hq = static_cast<int>(Hq);
  a.Hk = static_cast<int>(Hk);
  a.D = static_cast<int>(D);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto al = [](const void* p, unsigned m) { return (reinterpret_cast<uintptr_t>(p) & (m - 1)) == 0; };
  const bool fast = D == 128 && Hq % 4 == 0 && Hk % 4 == 0 && al(q, 16) && al(k, 16) && al(v, 16) &&
                    sqt % 8 == 0 && sqh % 8 == 0 && skt % 8 == 0 && skh % 8 == 0 && svt % 8 == 0 &&
                    svh % 8 == 0 && al(cos_sin_cache, 16) && al(k_cache, 16) && al(v_cache, 16) &&
                    sckp % 8 == 0 && sckh % 8 == 0 && scvp % 8 == 0 && scvh % 8 == 0;
  if (fast) {
    const int64_t items = T * (Hq / 4 + 2 * (Hk / 4));
    hipLaunchKernelGGL((qk_rope_kv_d128<kRopeBf16, 4>), dim3(static_cast<unsigned>((items + 3) / 4)),
                       dim3(256), 0, st, a);
  } else {
    const int64_t items = T * (Hq + 2 * Hk);
    hipLaunchKernelGGL(qk_rope_kv_generic<kRopeBf16>, dim3(static_cast<unsigned>((items + 3) / 4)),
                       dim3(256), 0, st, a);
  }
  return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
}

}  // extern "C"
