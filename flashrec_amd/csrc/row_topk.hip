// Per-row top-C of fp32 scores with the candidate-token gather: the
// "torch.topk(logprobs.view(n, bw, V), C, sorted=True) + cand_ids[idx]" that
// feeds the fused beam step (python/flashrec/scheduler/scheduler.py:1476-1481,
// python/flashrec/engine/graph.py:33-43 and :186-193).
//
// One 256-thread workgroup per row.  The row is read once into registers as
// 48-bit composite keys (order-preserving score bits << 16 | (0xFFFF - index))
// so that every key is distinct and equal scores rank by ascending index.
// A coarse pass bins the keys into 2048 integer ranges spanning the row's
// finite key range (LDS histogram + block scan): keys in bins above the C-th
// key's bin are taken outright and scattered bin by bin into LDS, and the few
// keys of that bin are ranked exactly by one wave.  Bins are in rank order,
// so each taken key's final place is its bin's start plus its rank among the
// (few) keys of its bin.  Rows that defeat the binning (more than 64 keys in
// the boundary bin or in any taken bin: heavy ties, degenerate ranges) fall
// back to an exact radix select over the keys and a bitonic sort whose short
// strides run in registers and across lanes and whose long strides go
// through LDS.
// Scores are rebuilt from their keys; zeros and NaNs are re-read from the row
// so that signed zeros and NaN payloads come out as stored.  NaN ranks above
// +inf and -0 equals +0, as in torch's sort and topk.
//
// Bytes per row: V*4 read + C*(4 + 8 [+ 8]) written; HBM-bound when the row
// count fills the chip.

#include "fr_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxC = 1024;
constexpr int kMaxV = 16384;
constexpr int kBinBits = 11;
constexpr uint32_t kBins = 1u << kBinBits;  // coarse-pass histogram
constexpr uint32_t kSegMax = 64;  // longest bin ordered by counting
constexpr uint32_t kKeyNegInf = 0x007FFFFFu;  // score_bits(-inf)
constexpr uint32_t kKeyPosInf = 0xFF800000u;  // score_bits(+inf)

__device__ __forceinline__ uint32_t score_bits(float v) {
  uint32_t b = __float_as_uint(v);
  if (v != v) return 0xFFFFFFFFu;
  if (b == 0x80000000u) b = 0;  // -0 ties with +0, as the float compare has it
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ uint64_t comp_key(uint32_t bits, uint32_t idx) {
  return (static_cast<uint64_t>(bits) << 16) | static_cast<uint64_t>(0xFFFFu - idx);
}

struct TopkArgs {
  const float* x;
  int64_t ldx;
  const int64_t* cand_ids;
  float* out_vals;
  int64_t* out_idx;
  int64_t* out_tok;
  int R, V, C;
  int vec;
};

// Inclusive scan of one value per thread over the block (thread order).
__device__ __forceinline__ uint32_t block_scan(uint32_t v, uint32_t* wsum) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  if (lane == 63) wsum[w] = v;
  __syncthreads();
  uint32_t base = 0;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i)
    if (i < w) base += wsum[i];
  __syncthreads();
  return v + base;
}

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), m, 64);
  const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), m, 64);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ __forceinline__ uint32_t uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// Hides a value from the optimiser so that what is derived from it per
// element is recomputed where used instead of being held in 32 registers
// across the row's passes (registers set how many rows a CU works on at once).
__device__ __forceinline__ uint32_t fresh(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ uint32_t fresh_s(uint32_t v) {
  asm volatile("" : "+s"(v));
  return v;
}

// LSM: the scores are log_softmax(x) of the row, x - lse with lse from
// block_row_lse (the log-softmax kernel's own arithmetic), formed in
// registers and never written; FULL rows only.
template <int NCH, int PT, bool FULL, bool LSM>
__global__ __launch_bounds__(kThreads) void row_topk_kernel(TopkArgs a) {
  static_assert(FULL || !LSM, "the folded log-softmax takes whole aligned rows");
  constexpr int NK = NCH * 4;
  constexpr int N = kThreads * PT;  // sort network width
  __shared__ uint32_t hist[kBins];
  __shared__ uint32_t wsum[kThreads / 64];
  __shared__ uint32_t red[3 * (kThreads / 64)];
  __shared__ uint32_t sel[4];
  __shared__ uint64_t sk[N];
  __shared__ uint64_t cl[64];
  __shared__ float lred[8];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int w = t >> 6;
  const int row = blockIdx.x;
  const float* xr = a.x + static_cast<int64_t>(row) * a.ldx;
  const uint32_t t4 = 4 * t;
  auto index_of = [&](int q) -> uint32_t { return fresh(t4) + (4 * kThreads * (q >> 2) + (q & 3)); };
  auto valid = [&](int q) -> bool { return FULL || index_of(q) < static_cast<uint32_t>(a.V); };

  // ---- the row, as order-preserving bits; element q is index 4*(t + 256*(q/4)) + q%4
  uint32_t key[NK];
  float lse = 0.0f;
  if constexpr (LSM) {
    fr::f32x4 v[NCH];
#pragma unroll
    for (int j = 0; j < NCH; ++j) v[j] = *reinterpret_cast<const fr::f32x4*>(xr + 4 * (t + kThreads * j));
    lse = fr::block_row_lse<NCH>(v, lred);
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const fr::f32x4 y = v[j] - lse;
      key[4 * j + 0] = score_bits(y.x);
      key[4 * j + 1] = score_bits(y.y);
      key[4 * j + 2] = score_bits(y.z);
      key[4 * j + 3] = score_bits(y.w);
    }
  }
#pragma unroll
  for (int j = 0; j < NCH && !LSM; ++j) {
    const int i0 = 4 * (t + kThreads * j);
    if (FULL || (a.vec && i0 + 3 < a.V)) {
      const float4 f = *reinterpret_cast<const float4*>(xr + i0);
      key[4 * j + 0] = score_bits(f.x);
      key[4 * j + 1] = score_bits(f.y);
      key[4 * j + 2] = score_bits(f.z);
      key[4 * j + 3] = score_bits(f.w);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) key[4 * j + e] = (i0 + e < a.V) ? score_bits(xr[i0 + e]) : 0u;
    }
  }

  // ---- key range: the maximum over all keys, and the range of the finite
  // scores (NaN and +-inf keys would stretch it to the whole bit space)
  uint32_t mx = 0, fmx = 0, fmn = 0xFFFFFFFFu;
#pragma unroll
  for (int q = 0; q < NK; ++q)
    if (valid(q)) {
      const uint32_t k = key[q];
      mx = k > mx ? k : mx;
      const bool fin = k > kKeyNegInf && k < kKeyPosInf;
      fmx = fin && k > fmx ? k : fmx;
      fmn = fin && k < fmn ? k : fmn;
    }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t a1 = __shfl_xor(mx, o, 64), a2 = __shfl_xor(fmx, o, 64), a3 = __shfl_xor(fmn, o, 64);
    mx = a1 > mx ? a1 : mx;
    fmx = a2 > fmx ? a2 : fmx;
    fmn = a3 < fmn ? a3 : fmn;
  }
  if (lane == 0) {
    red[w] = mx;
    red[4 + w] = fmx;
    red[8 + w] = fmn;
  }
  __syncthreads();
  uint32_t kmax = red[0], kfmax = red[4], kfmin = red[8];
#pragma unroll
  for (int i = 1; i < kThreads / 64; ++i) {
    kmax = red[i] > kmax ? red[i] : kmax;
    kfmax = red[4 + i] > kfmax ? red[4 + i] : kfmax;
    kfmin = red[8 + i] < kfmin ? red[8 + i] : kfmin;
  }
  kmax = uni(kmax);
  if (kfmin > kfmax) kfmin = kfmax = kmax;  // no finite score
  kfmax = uni(kfmax);
  kfmin = uni(kfmin);

  // ---- coarse pass: 2048 bins of the distance below the finite maximum,
  // scaled to the finite range.  bin() is non-decreasing in the distance
  // (saturating below, clamped above), so every key of a lower bin outranks
  // every key of a higher one: the C-th key's bin b* splits the row into the
  // keys surely taken (bins < b*) and the few candidates of bin b*.
  const uint32_t span = kfmax - kfmin;
  const int s0 = span < kBins ? 0 : (32 - __builtin_clz(span)) - kBinBits;
  auto bin = [&](uint32_t k) -> uint32_t {
    const uint32_t top = fresh_s(kfmax);  // recomputed per pass, not held
    const uint32_t b = (k >= top ? 0u : top - k) >> s0;
    return b < kBins - 1 ? b : kBins - 1;
  };
#pragma unroll
  for (int i = 0; i < kBins / kThreads; ++i) hist[t * (kBins / kThreads) + i] = 0;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < NK; ++q)
    if (valid(q)) atomicAdd(&hist[bin(key[q])], 1u);
  __syncthreads();
  constexpr int BPT = kBins / kThreads;  // bins per thread, ascending
  uint32_t c[BPT];
  {
    uint32_t tot = 0;
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      c[i] = hist[t * BPT + i];
      tot += c[i];
    }
    const uint32_t incl = block_scan(tot, wsum);
    uint32_t run = incl - tot;
    const uint32_t C = static_cast<uint32_t>(a.C);
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      if (run < C && C <= run + c[i]) {
        sel[0] = t * BPT + i;
        sel[1] = C - run;  // keys still needed from bin b*
        sel[2] = c[i];
        sel[3] = run;      // keys surely taken
      }
      hist[t * BPT + i] = run;  // bin start; a cursor below
      run += c[i];
    }
  }
  __syncthreads();
  const uint32_t bstar = uni(sel[0]), need0 = uni(sel[1]), cntb = uni(sel[2]), sure = uni(sel[3]);
  // longest bin among those taken outright
  uint32_t lmax = 0;
#pragma unroll
  for (int i = 0; i < BPT; ++i)
    if (static_cast<uint32_t>(t * BPT + i) < bstar) lmax = c[i] > lmax ? c[i] : lmax;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t x = __shfl_xor(lmax, o, 64);
    lmax = x > lmax ? x : lmax;
  }
  if (lane == 0) red[w] = lmax;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) lmax = red[i] > lmax ? red[i] : lmax;
  // sure keys are placed bin by bin (bins are already in rank order), so
  // only each bin's few keys need ordering among themselves (bin b*'s keys
  // come out of the one-wave ranking in order)
  const bool bin_sort = uni(lmax) <= kSegMax && cntb <= 64;

  // ---- compaction: sure keys into their bin's range of the sort buffer;
  // candidates of bin b* into a short list when they fit one wave (else the
  // exact radix pass below resolves them)
  const bool short_list = cntb <= 64;
  // slots are claimed eight keys at a time so the atomics' round trips overlap
  constexpr int SB = NK < 8 ? NK : 8;
#pragma unroll
  for (int q0 = 0; q0 < NK; q0 += SB) {
    uint32_t slot[SB];
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int q = q0 + u;
      const uint32_t b = bin(key[q]);
      const bool take = valid(q) && (b < bstar || (short_list && b == bstar));
      slot[u] = take ? atomicAdd(&hist[b], 1u) : 0xFFFFFFFFu;
    }
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int q = q0 + u;
      if (slot[u] < sure) sk[slot[u]] = comp_key(key[q], index_of(q));
      else if (slot[u] != 0xFFFFFFFFu) cl[slot[u] - sure] = comp_key(key[q], index_of(q));
    }
  }
  __syncthreads();

  if (short_list) {
    // exact rank of each candidate among the candidates (keys are distinct)
    if (w == 0) {
      const uint64_t mine = lane < static_cast<int>(cntb) ? cl[lane] : 0;
      uint32_t rank = 0;
      for (uint32_t m = 0; m < cntb; ++m) rank += cl[m] > mine ? 1u : 0u;
      if (lane < static_cast<int>(cntb) && rank < need0) sk[sure + rank] = mine;
    }
  } else {
    // ---- exact radix select of the need0-th best key of bin b*: 8-bit
    // digits of d = kmax - key (smaller is better), then of the index
    uint32_t need = need0;
    int sh = 24;
    bool ip = false;
    uint32_t P = 0, D = 0, Pi = 0;
    int ish = 8;
    for (;;) {
      hist[t] = 0;
      __syncthreads();
#pragma unroll
      for (int q = 0; q < NK; ++q) {
        if (valid(q) && bin(key[q]) == bstar) {
          const uint32_t d = kmax - key[q];
          const uint32_t idx = index_of(q);
          bool match;
          uint32_t digit;
          if (!ip) {
            match = sh == 24 || (d >> (sh + 8)) == P;
            digit = (d >> sh) & 255u;
          } else {
            match = d == D && (ish == 8 || (idx >> 8) == Pi);
            digit = (idx >> ish) & 255u;
          }
          if (match) atomicAdd(&hist[digit], 1u);
        }
      }
      __syncthreads();
      const uint32_t cnt = hist[t];
      const uint32_t incl = block_scan(cnt, wsum);
      const uint32_t excl = incl - cnt;
      if (excl < need && need <= incl) {
        sel[0] = t;
        sel[1] = need - excl;
        sel[2] = (cnt == need - excl) ? 1u : 0u;
      }
      __syncthreads();
      const uint32_t digit = uni(sel[0]);
      need = uni(sel[1]);
      const bool whole = uni(sel[2]) != 0;
      __syncthreads();
      if (!ip) {
        P = sh == 24 ? digit : ((P << 8) | digit);
        if (whole) break;
        if (sh == 0) {  // equal scores: order by index
          ip = true;
          D = P;
        } else {
          sh -= 8;
        }
      } else {
        Pi = ish == 8 ? digit : ((Pi << 8) | digit);
        if (whole || ish == 0) break;
        ish = 0;
      }
    }
    uint32_t mine = 0;
    auto admitted = [&](int q) -> bool {
      if (!valid(q) || bin(key[q]) != bstar) return false;
      const uint32_t d = kmax - key[q];
      if (!ip) return (d >> sh) <= P;
      return d < D || (d == D && (index_of(q) >> ish) <= Pi);
    };
#pragma unroll
    for (int q = 0; q < NK; ++q) mine += admitted(q) ? 1u : 0u;
    uint32_t pos = sure + block_scan(mine, wsum) - mine;
#pragma unroll
    for (int q = 0; q < NK; ++q)
      if (admitted(q)) sk[pos++] = comp_key(key[q], index_of(q));
  }
  for (int i = a.C + t; i < N; i += kThreads) sk[i] = 0;
  __syncthreads();

  const int64_t ob = static_cast<int64_t>(row) * a.C;
  auto emit = [&](int i, uint64_t kk) {
    const int64_t idx = 0xFFFF - static_cast<int64_t>(kk & 0xFFFFu);
    // the score from its key; zeros (either sign) and NaNs are re-read so
    // that their bits come out as stored
    const uint32_t kb = static_cast<uint32_t>(kk >> 16);
    const float val = (kb == 0x80000000u || kb == 0xFFFFFFFFu)
                          ? (LSM ? xr[idx] - lse : xr[idx])
                          : __uint_as_float((kb & 0x80000000u) ? (kb & 0x7FFFFFFFu) : ~kb);
    a.out_vals[ob + i] = val;
    if (a.out_idx) a.out_idx[ob + i] = idx;
    if (a.out_tok) a.out_tok[ob + i] = a.cand_ids ? a.cand_ids[idx] : idx;
  };
  if (bin_sort) {
    // after the scatter, hist[b] is the end of bin b (= start of b + 1):
    // a sure key's final place is its bin's start plus the number of keys of
    // its bin above it; keys of bin b* are already in order
    for (int i = t; i < a.C; i += kThreads) {
      const uint64_t kk = sk[i];
      int f = i;
      if (static_cast<uint32_t>(i) < sure) {
        const uint32_t b = bin(static_cast<uint32_t>(kk >> 16));
        const uint32_t s = b == 0 ? 0u : hist[b - 1], e = hist[b];
        uint32_t r = 0;
        for (uint32_t m = s; m < e; ++m) r += sk[m] > kk ? 1u : 0u;
        f = static_cast<int>(s + r);
      }
      emit(f, kk);
    }
    return;
  }

  // ---- bitonic sort, descending; element i = t*PT + s
  uint64_t v[PT];
#pragma unroll
  for (int s = 0; s < PT; ++s) v[s] = sk[t * PT + s];
#pragma unroll
  for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j < PT) {
#pragma unroll
        for (int s = 0; s < PT; ++s) {
          const int p = s ^ j;
          if (s < p) {
            const bool up = ((t * PT + s) & k) == 0;
            const uint64_t lo = v[s] < v[p] ? v[s] : v[p];
            const uint64_t hi = v[s] < v[p] ? v[p] : v[s];
            v[s] = up ? hi : lo;
            v[p] = up ? lo : hi;
          }
        }
      } else if (j < 64 * PT) {
#pragma unroll
        for (int s = 0; s < PT; ++s) {
          const int i = t * PT + s;
          const uint64_t o = shfl_xor64(v[s], j / PT);
          const bool want_max = (((i & j) == 0) == ((i & k) == 0));
          const uint64_t mx = v[s] < o ? o : v[s];
          const uint64_t mn = v[s] < o ? v[s] : o;
          v[s] = want_max ? mx : mn;
        }
      } else {
        __syncthreads();
#pragma unroll
        for (int s = 0; s < PT; ++s) sk[t * PT + s] = v[s];
        __syncthreads();
#pragma unroll
        for (int s = 0; s < PT; ++s) {
          const int i = t * PT + s;
          const uint64_t o = sk[i ^ j];
          const bool want_max = (((i & j) == 0) == ((i & k) == 0));
          const uint64_t mx = v[s] < o ? o : v[s];
          const uint64_t mn = v[s] < o ? v[s] : o;
          v[s] = want_max ? mx : mn;
        }
      }
    }
  }

  // ---- outputs
#pragma unroll
  for (int s = 0; s < PT; ++s) {
    const int i = t * PT + s;
    if (i < a.C) emit(i, v[s]);
  }
}

template <int NCH, bool FULL, bool LSM = false>
void launch_pt(const TopkArgs& a, int pt, hipStream_t stream) {
  const dim3 grid(a.R), block(kThreads);
  switch (pt) {
    case 1: hipLaunchKernelGGL((row_topk_kernel<NCH, 1, FULL, LSM>), grid, block, 0, stream, a); break;
    case 2: hipLaunchKernelGGL((row_topk_kernel<NCH, 2, FULL, LSM>), grid, block, 0, stream, a); break;
    default: hipLaunchKernelGGL((row_topk_kernel<NCH, 4, FULL, LSM>), grid, block, 0, stream, a); break;
  }
}

template <int NCH>
int launch_nch(const TopkArgs& a, int pt, hipStream_t stream) {
  // FULL: every thread's chunks are in range and 16-byte aligned
  if (a.vec && a.V == NCH * 4 * kThreads) launch_pt<NCH, true>(a, pt, stream);
  else launch_pt<NCH, false>(a, pt, stream);
  return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
}

}  // namespace

extern "C" int fr_row_topk(const float* x, int64_t ldx, int64_t R, int64_t V, int64_t C,
                           const int64_t* cand_ids, float* out_vals, int64_t* out_idx,
                           int64_t* out_tokens, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (R < 0 || V <= 0 || C <= 0 || ldx < V) return FR_EINVAL;
  if (R == 0) return FR_OK;
  if (!x || !out_vals) return FR_EINVAL;
  if (C > V || C > kMaxC || V > kMaxV || R > 0x7FFFFFFF) return FR_EUNSUPPORTED;
  TopkArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.cand_ids = cand_ids;
  a.out_vals = out_vals;
  a.out_idx = out_idx;
  a.out_tok = out_tokens;
  a.R = static_cast<int>(R);
  a.V = static_cast<int>(V);
  a.C = static_cast<int>(C);
  a.vec = ((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (ldx & 3) == 0) ? 1 : 0;
  const int pt = C <= 256 ? 1 : (C <= 512 ? 2 : 4);
  const int64_t chunks = (V + 4 * kThreads - 1) / (4 * kThreads);
  if (chunks <= 1) return launch_nch<1>(a, pt, stream);
  if (chunks <= 2) return launch_nch<2>(a, pt, stream);
  if (chunks <= 4) return launch_nch<4>(a, pt, stream);
  if (chunks <= 8) return launch_nch<8>(a, pt, stream);
  return launch_nch<16>(a, pt, stream);
}

extern "C" int fr_log_softmax_row_topk(const float* logits, int64_t ldx, int64_t R, int64_t V, int64_t C,
                                       const int64_t* cand_ids, float* out_vals, int64_t* out_idx,
                                       int64_t* out_tokens, void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (R < 0 || V <= 0 || C <= 0 || ldx < V) return FR_EINVAL;
  if (R == 0) return FR_OK;
  if (!logits || !out_vals) return FR_EINVAL;
  // the widths fr_log_softmax_f32 runs as one workgroup per row (whose
  // arithmetic block_row_lse is), whole aligned rows
  const bool aligned = (reinterpret_cast<uintptr_t>(logits) & 15) == 0 && (ldx & 3) == 0;
  if (!aligned || (V != 4096 && V != 8192) || C > V || C > kMaxC || R > 0x7FFFFFFF) return FR_EUNSUPPORTED;
  TopkArgs a{};
  a.x = logits;
  a.ldx = ldx;
  a.cand_ids = cand_ids;
  a.out_vals = out_vals;
  a.out_idx = out_idx;
  a.out_tok = out_tokens;
  a.R = static_cast<int>(R);
  a.V = static_cast<int>(V);
  a.C = static_cast<int>(C);
  a.vec = 1;
  const int pt = C <= 256 ? 1 : (C <= 512 ? 2 : 4);
  if (V == 4096) launch_pt<4, true, true>(a, pt, stream);
  else launch_pt<8, true, true>(a, pt, stream);
  return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
}
