// Fused beam-search step over trie-constrained candidates: mask -> top-K ->
// expand token rows -> advance trie nodes.
//
// Reference: python/flashrec/kernel/beam_trie.py:536-633
// (genrec_mask_topk_expand, whose PyTorch branch defines the result) and its
// CUDA kernel python/flashrec/kernel/csrc/beam_trie.cuh:548-757, whose
// choices for what the PyTorch branch leaves open are kept: candidates are
// ranked by score descending, then flat index (b * C + c) ascending; with
// masking on, masked candidates (and -inf scores) are never picked, and when
// fewer than K remain the missing picks are (-inf, index 0, parent 0,
// token top_tokens[n][0][0]); rows b >= K of the token / node planes are
// copied unchanged; with expansion off nothing is advanced either.
// Candidate rule (beam_trie.cuh:37-49): node < 0 accepts every token,
// otherwise allow[node][tok - token_base] with tok outside the table refused;
// transition (:51-64): node < 0 stays, tok outside the table -> invalid_node,
// else next_node[node][tok - token_base].  NaN scores are treated as masked.
//
// Layout for MI355X.  Per request the candidates are BW beams x C columns,
// each beam's C already sorted descending (they come from a per-row sorted
// top-k), so the top K is a merge.  A candidate is one 64-bit key: the
// orderable bits of its score in the high word, the complement of its flat
// index in the low word, so "larger key" is exactly the ranking above and
// every merge is exact.
//   kernel 1, one workgroup per (request, slice of BS beams): each wave
//     compacts its beams' valid candidates into per-beam sorted lists of at
//     most K keys (ballot prefix sums; stops at K), then the BS lists are
//     merged pairwise in LDS (merge path: each output finds its split by a
//     binary search, all outputs in parallel, one barrier per tree level)
//     into the slice's top K, written to the caller's scratch;
//   kernel 2, one workgroup per request: merges the slices' lists the same
//     way (in groups that fit LDS, each folded into a running top K), writes
//     vals / parents / tokens / indices, then the expanded token rows and the
//     advanced trie nodes.
#include <mutex>

#include "fr_common.h"

namespace fr {

struct GenrecArgs {
  float* out_vals;        // [N, K]
  int64_t* out_parents;   // [N, K]
  int64_t* out_tokens;    // [N, K]
  int64_t* out_indices;   // [N, K]
  uint64_t* scratch;      // [N, S, 1 + K]
  const float* cum;       // [N, BW]
  const float* lp;        // [N, BW, C]
  const int64_t* tok;     // [N, BW, C]
  const int64_t* nodes;   // [N, BW] or null
  const uint8_t* allow;   // [n_nodes, vsz] or null
  const int64_t* tin;     // [N, BW, L] or null
  int64_t* tout;          // [N, BW, L] or null
  const void* next;       // [n_nodes, vsz] int64 or int32 (next_i32), or null
  int next_i32;
  int64_t* nout;          // [N, BW] or null
  const uint8_t* do_exp;  // [N] or null (all)
  const int32_t* col;     // [N]
  int64_t token_base, n_nodes, vsz, invalid_node;
  float neg_inf;
  int N, BW, C, K, L, S, BS;
  int apply_mask, apply_expand, apply_advance;
};

constexpr int kListKeys = 8192;  // keys per LDS list buffer (64 KB)

__device__ __forceinline__ uint32_t order_bits(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_order_bits(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}
__device__ __forceinline__ uint64_t make_key(float v, uint32_t idx) {
  return (static_cast<uint64_t>(order_bits(v)) << 32) | static_cast<uint64_t>(~idx);
}
__device__ __forceinline__ float key_val(uint64_t k) { return from_order_bits(static_cast<uint32_t>(k >> 32)); }
__device__ __forceinline__ uint32_t key_idx(uint64_t k) { return ~static_cast<uint32_t>(k); }

__device__ __forceinline__ bool cand_ok(const GenrecArgs& a, int64_t node, int64_t t) {
  if (node < 0) return true;
  const int64_t rel = t - a.token_base;
  if (rel < 0 || rel >= a.vsz || a.n_nodes <= 0) return false;
  const int64_t safe = node < 0 ? 0 : (node > a.n_nodes - 1 ? a.n_nodes - 1 : node);
  return a.allow[safe * a.vsz + rel] != 0;
}

// Outputs i0 .. i0 + count - 1 of merge(A[0..na), B[0..nb)), both
// descending, into dst[i0 ..]: one
// binary search for where output i0 splits A and B (merge path), then a
// sequential walk, one comparison per output with the two heads in
// registers.
__device__ __forceinline__ void merge_run(const uint64_t* A, int na, const uint64_t* B, int nb, int i0, int count,
                                          uint64_t* dst) {
  int lo = i0 - nb > 0 ? i0 - nb : 0;
  int hi = i0 < na ? i0 : na;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (A[mid] > B[i0 - mid - 1]) lo = mid + 1;
    else hi = mid;
  }
  int ia = lo, ib = i0 - lo;
  uint64_t ha = ia < na ? A[ia] : 0, hb = ib < nb ? B[ib] : 0;
  for (int k = 0; k < count; ++k) {
    const bool take_a = ia < na && (ib >= nb || ha > hb);
    if (take_a) {
      dst[i0 + k] = ha;
      ++ia;
      ha = ia < na ? A[ia] : 0;
    } else {
      dst[i0 + k] = hb;
      ++ib;
      hb = ib < nb ? B[ib] : 0;
    }
  }
}

constexpr int kRun = 8;  // outputs per thread per merge_run

// Merge `n` lists (list l at src + l * K, length len[l]) pairwise down to
// one, ping-ponging between src and dst; returns the buffer holding it (at
// offset 0) and its length in len[0].  All threads of the block call this.
__device__ uint64_t* merge_tree(uint64_t* src, uint64_t* dst, int* len, int n, int K) {
  while (n > 1) {
    const int pairs = n >> 1;
    const int runs = (K + kRun - 1) / kRun;  // per pair
    for (int t = threadIdx.x; t < pairs * runs; t += blockDim.x) {
      const int p = t / runs, i0 = (t - p * runs) * kRun;
      const int la = len[2 * p], lb = len[2 * p + 1];
      const int lim = la + lb < K ? la + lb : K;
      if (i0 < lim)
        merge_run(src + 2 * p * K, la, src + (2 * p + 1) * K, lb, i0, lim - i0 < kRun ? lim - i0 : kRun,
                  dst + p * K);
    }
    // an odd list out is carried over unchanged
    if (n & 1)
      for (int i = threadIdx.x; i < len[n - 1]; i += blockDim.x) dst[pairs * K + i] = src[(n - 1) * K + i];
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int p = 0; p < pairs; ++p) {
        const int s = len[2 * p] + len[2 * p + 1];
        len[p] = s < K ? s : K;
      }
      if (n & 1) len[pairs] = len[n - 1];
    }
    __syncthreads();
    uint64_t* t = src;
    src = dst;
    dst = t;
    n = pairs + (n & 1);
  }
  return src;
}

constexpr int kSliceWaves = 16;  // one wave per beam of a slice (BS <= 16)

__global__ __launch_bounds__(64 * kSliceWaves) void genrec_slice_topk(GenrecArgs a) {
  __shared__ uint64_t bufA[kListKeys];
  __shared__ uint64_t bufB[kListKeys];
  __shared__ int len[64];
  const int n = blockIdx.x / a.S, s = blockIdx.x - (blockIdx.x / a.S) * a.S;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b0 = s * a.BS;
  const int nb = a.BW - b0 < a.BS ? a.BW - b0 : a.BS;
  const bool mask = a.apply_mask && a.allow != nullptr && a.nodes != nullptr;
  // each wave compacts beams wave, wave + kSliceWaves, ... (one each when
  // BS <= kSliceWaves): list of beam j at bufA + j * K.
  // A beam's candidates go in groups of kPre chunks of 64: the scores and
  // tokens of the whole group are loaded, then all of its trie lookups are
  // issued, then the chunks are compacted in order (ballot prefix sums,
  // stopping at K): two memory round trips per group instead of two per
  // chunk.  Which candidates are taken, and where, is unchanged.
  constexpr int kPre = 16;
  for (int j = wave; j < nb; j += kSliceWaves) {
    const int b = b0 + j;
    const float cb = a.cum[static_cast<int64_t>(n) * a.BW + b];
    const int64_t node = mask ? a.nodes[static_cast<int64_t>(n) * a.BW + b] : -1;
    const float* lpb = a.lp + (static_cast<int64_t>(n) * a.BW + b) * a.C;
    const int64_t* tkb = a.tok + (static_cast<int64_t>(n) * a.BW + b) * a.C;
    int count = 0;
    for (int g0 = 0; g0 < a.C && count < a.K; g0 += 64 * kPre) {
      float v[kPre];
      int64_t tk[kPre];
#pragma unroll
      for (int u = 0; u < kPre; ++u) {
        const int c = g0 + 64 * u + lane;
        v[u] = c < a.C ? cb + lpb[c] : 0.0f;
        tk[u] = c < a.C && mask ? tkb[c] : 0;
      }
      bool okv[kPre];
#pragma unroll
      for (int u = 0; u < kPre; ++u) {
        const int c = g0 + 64 * u + lane;
        bool ok = c < a.C && v[u] == v[u];  // NaN: never picked
        if (mask) ok = ok && v[u] != a.neg_inf && cand_ok(a, node, tk[u]);
        okv[u] = ok;
      }
#pragma unroll
      for (int u = 0; u < kPre; ++u) {
        if (count >= a.K) break;
        const int c = g0 + 64 * u + lane;
        const uint64_t bal = __ballot(okv[u]);
        const int pos = count + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                    static_cast<uint32_t>(bal >> 32),
                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u)));
        if (okv[u] && pos < a.K) bufA[j * a.K + pos] = make_key(v[u], static_cast<uint32_t>(b * a.C + c));
        count += __builtin_popcountll(bal);
      }
    }
    if (lane == 0) len[j] = count < a.K ? count : a.K;
  }
  __syncthreads();
  uint64_t* res = merge_tree(bufA, bufB, len, nb, a.K);
  uint64_t* out = a.scratch + (static_cast<int64_t>(n) * a.S + s) * (1 + a.K);
  for (int i = threadIdx.x; i < len[0]; i += blockDim.x) out[1 + i] = res[i];
  if (threadIdx.x == 0) out[0] = static_cast<uint64_t>(len[0]);
}

__global__ __launch_bounds__(1024) void genrec_request_topk_expand(GenrecArgs a) {
  __shared__ uint64_t bufA[kListKeys];
  __shared__ uint64_t bufB[kListKeys];
  __shared__ uint64_t acc[1024];  // running top K of the groups merged so far
  __shared__ int len[64];
  __shared__ int acc_len;
  __shared__ int64_t sel_parent[1024];
  __shared__ int64_t sel_token[1024];
  const int n = blockIdx.x;
  const int K = a.K;
  const uint64_t* lists = a.scratch + static_cast<int64_t>(n) * a.S * (1 + K);
  // The slice lists go in groups of G that fill an LDS buffer: a group is
  // copied in (coalesced, one memory round trip), merged down to one list
  // in LDS and folded into acc.  (Merging straight from the scratch would
  // put a dependent global read at every step of every binary search.)
  const int G = kListKeys / K < 64 ? kListKeys / K : 64;  // (len[] holds 64)
  if (threadIdx.x == 0) acc_len = 0;
  for (int g0 = 0; g0 < a.S; g0 += G) {
    const int gs = a.S - g0 < G ? a.S - g0 : G;
    const uint64_t* gl = lists + static_cast<int64_t>(g0) * (1 + K);
    if (threadIdx.x < gs) len[threadIdx.x] = static_cast<int>(gl[static_cast<int64_t>(threadIdx.x) * (1 + K)]);
    __syncthreads();
    // the keys of every list of the group (gs * K <= kListKeys = 8 per
    // thread of 1024): all loads issued before any is stored
    constexpr int kPer = kListKeys / 1024;
    uint64_t key[kPer];
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
      const int t = threadIdx.x + r * 1024;
      const int l = t / K, i = t - l * K;
      key[r] = (l < gs && i < len[l]) ? gl[static_cast<int64_t>(l) * (1 + K) + 1 + i] : 0;
    }
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
      const int t = threadIdx.x + r * 1024;
      const int l = t / K, i = t - l * K;
      if (l < gs && i < len[l]) bufA[l * K + i] = key[r];
    }
    __syncthreads();
    uint64_t* res = merge_tree(bufA, bufB, len, gs, K);
    uint64_t* other = res == bufA ? bufB : bufA;
    const int lr = len[0], la = acc_len;
    const int lt = la + lr < K ? la + lr : K;
    for (int i0 = threadIdx.x * kRun; i0 < lt; i0 += blockDim.x * kRun)
      merge_run(acc, la, res, lr, i0, lt - i0 < kRun ? lt - i0 : kRun, other);
    __syncthreads();
    for (int i = threadIdx.x; i < lt; i += blockDim.x) acc[i] = other[i];
    if (threadIdx.x == 0) acc_len = lt;
    __syncthreads();
  }
  const uint64_t* res = acc;
  const int got = acc_len;
  const int64_t* tkn = a.tok + static_cast<int64_t>(n) * a.BW * a.C;
  for (int k = threadIdx.x; k < K; k += blockDim.x) {
    float v = a.neg_inf;
    uint32_t idx = 0;
    if (k < got) {
      v = key_val(res[k]);
      idx = key_idx(res[k]);
    }
    const int64_t parent = k < got ? static_cast<int64_t>(idx / static_cast<uint32_t>(a.C)) : 0;
    const int64_t token = tkn[idx];
    const int64_t o = static_cast<int64_t>(n) * K + k;
    a.out_vals[o] = v;
    a.out_parents[o] = parent;
    a.out_tokens[o] = token;
    a.out_indices[o] = static_cast<int64_t>(idx);
    sel_parent[k] = parent;
    sel_token[k] = token;
  }
  const bool expand = a.apply_expand && a.tin != nullptr && a.tout != nullptr &&
                      (a.do_exp == nullptr || a.do_exp[n] != 0);
  if (!expand) return;
  __syncthreads();
  const int col = a.col[n] < 0 ? 0 : a.col[n];
  const int64_t* tin = a.tin + static_cast<int64_t>(n) * a.BW * a.L;
  int64_t* tout = a.tout + static_cast<int64_t>(n) * a.BW * a.L;
  for (int64_t e = threadIdx.x; e < static_cast<int64_t>(a.BW) * a.L; e += blockDim.x) {
    const int b = static_cast<int>(e / a.L), c = static_cast<int>(e - static_cast<int64_t>(b) * a.L);
    if (b >= K) {
      tout[e] = tin[e];
    } else if (c == col) {
      tout[e] = sel_token[b];
    } else {
      int64_t p = sel_parent[b];
      p = p < 0 ? 0 : (p > a.BW - 1 ? a.BW - 1 : p);
      tout[e] = tin[p * a.L + c];
    }
  }
  if (a.apply_advance && a.next != nullptr && a.nodes != nullptr && a.nout != nullptr) {
    const int64_t* nin = a.nodes + static_cast<int64_t>(n) * a.BW;
    int64_t* nout = a.nout + static_cast<int64_t>(n) * a.BW;
    for (int b = threadIdx.x; b < a.BW; b += blockDim.x) {
      if (b >= K) {
        nout[b] = nin[b];
        continue;
      }
      int64_t p = sel_parent[b];
      p = p < 0 ? 0 : (p > a.BW - 1 ? a.BW - 1 : p);
      const int64_t old = nin[p];
      int64_t nx;
      if (old < 0) {
        nx = old;
      } else {
        const int64_t rel = sel_token[b] - a.token_base;
        if (rel < 0 || rel >= a.vsz || a.n_nodes <= 0) {
          nx = a.invalid_node;
        } else {
          const int64_t safe = old > a.n_nodes - 1 ? a.n_nodes - 1 : old;
          const int64_t cell = safe * a.vsz + rel;
          nx = a.next_i32 ? static_cast<int64_t>(static_cast<const int32_t*>(a.next)[cell])
                          : static_cast<const int64_t*>(a.next)[cell];
        }
      }
      nout[b] = nx;
    }
  }
}

}  // namespace fr

using namespace fr;

extern "C" int fr_genrec_scratch_bytes(int64_t N, int64_t BW, int64_t K) {
  if (N <= 0 || BW <= 0 || K <= 0 || K > 1024) return -1;
  const int64_t BS = kListKeys / K < 16 ? kListKeys / K : 16;
  const int64_t S = (BW + BS - 1) / BS;
  const int64_t bytes = N * S * (1 + K) * 8;
  return bytes > 0x7FFFFFFF ? -1 : static_cast<int>(bytes);
}

// Argument checks shared by both entry points; the scratch is checked by
// each (caller's buffer, or the library's static one).
static int genrec_check(float* out_vals, int64_t* out_parents, int64_t* out_tokens, int64_t* out_indices,
                        const float* cum, const float* top_logprobs, const int64_t* top_tokens,
                        const int32_t* col, int64_t N, int64_t BW, int64_t C, int64_t K, int64_t L) {
  if (N < 0 || BW <= 0 || C <= 0 || K <= 0 || L < 0) return FR_EINVAL;
  if (N == 0) return FR_OK;
  if (!out_vals || !out_parents || !out_tokens || !out_indices || !cum || !top_logprobs || !top_tokens ||
      !col)
    return FR_EINVAL;
  if (K > 1024 || K > BW * C || BW * C > 0x7FFFFFFF) return FR_EUNSUPPORTED;
  return FR_OK;
}

static int genrec_launch(
    float* out_vals, int64_t* out_parents, int64_t* out_tokens, int64_t* out_indices, void* scratch,
    const float* cum, const float* top_logprobs, const int64_t* top_tokens,
    const int64_t* node_ids, const uint8_t* allow_table, const int64_t* token_ids_in,
    int64_t* token_ids_out, const void* next_node, int64_t* node_ids_out, const uint8_t* do_expand,
    const int32_t* col, int64_t token_base, int64_t n_nodes, int64_t vsz, int64_t invalid_node,
    int64_t N, int64_t BW, int64_t C, int64_t K, int64_t L, int apply_mask, int apply_expand,
    int apply_advance, int next_i32, void* stream) {
  if (apply_mask && node_ids && allow_table && n_nodes > 0 && vsz <= 0) return FR_EINVAL;
  if (apply_expand && (!token_ids_in || !token_ids_out || L <= 0)) return FR_EINVAL;
  if (apply_expand && token_ids_in == token_ids_out) return FR_EINVAL;  // rows gather from other rows
  GenrecArgs a{};
  a.out_vals = out_vals;
  a.out_parents = out_parents;
  a.out_tokens = out_tokens;
  a.out_indices = out_indices;
  a.scratch = static_cast<uint64_t*>(scratch);
  a.cum = cum;
  a.lp = top_logprobs;
  a.tok = top_tokens;
  a.nodes = node_ids;
  a.allow = allow_table;
  a.tin = token_ids_in;
  a.tout = token_ids_out;
  a.next = next_node;
  a.next_i32 = next_i32 ? 1 : 0;
  a.nout = node_ids_out;
  a.do_exp = do_expand;
  a.col = col;
  a.token_base = token_base;
  a.n_nodes = n_nodes;
  a.vsz = vsz;
  a.invalid_node = invalid_node;
  a.neg_inf = -__builtin_inff();
  a.N = static_cast<int>(N);
  a.BW = static_cast<int>(BW);
  a.C = static_cast<int>(C);
  a.K = static_cast<int>(K);
  a.L = static_cast<int>(L);
  a.BS = kListKeys / a.K < 16 ? kListKeys / a.K : 16;
  a.S = (a.BW + a.BS - 1) / a.BS;
  a.apply_mask = apply_mask;
  a.apply_expand = apply_expand;
  a.apply_advance = apply_advance;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(genrec_slice_topk, dim3(static_cast<unsigned>(N * a.S)), dim3(64 * kSliceWaves), 0, st, a);
  hipLaunchKernelGGL(genrec_request_topk_expand, dim3(static_cast<unsigned>(N)), dim3(1024), 0, st, a);
  return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
}

extern "C" int fr_genrec_mask_topk_expand(
    float* out_vals, int64_t* out_parents, int64_t* out_tokens, int64_t* out_indices, void* scratch,
    int64_t scratch_bytes, const float* cum, const float* top_logprobs, const int64_t* top_tokens,
    const int64_t* node_ids, const uint8_t* allow_table, const int64_t* token_ids_in,
    int64_t* token_ids_out, const void* next_node, int64_t* node_ids_out, const uint8_t* do_expand,
    const int32_t* col, int64_t token_base, int64_t n_nodes, int64_t vsz, int64_t invalid_node,
    int64_t N, int64_t BW, int64_t C, int64_t K, int64_t L, int apply_mask, int apply_expand,
    int apply_advance, int next_i32, void* stream) {
  const int rc = genrec_check(out_vals, out_parents, out_tokens, out_indices, cum, top_logprobs, top_tokens,
                              col, N, BW, C, K, L);
  if (rc != FR_OK || N == 0) return rc;
  if (!scratch) return FR_EINVAL;
  const int need = fr_genrec_scratch_bytes(N, BW, K);
  if (need < 0 || scratch_bytes < need) return FR_EINVAL;
  return genrec_launch(out_vals, out_parents, out_tokens, out_indices, scratch, cum, top_logprobs,
                       top_tokens, node_ids, allow_table, token_ids_in, token_ids_out, next_node,
                       node_ids_out, do_expand, col, token_base, n_nodes, vsz, invalid_node, N, BW, C, K, L,
                       apply_mask, apply_expand, apply_advance, next_i32, stream);
}

// ---- The same step with no allocation anywhere: the slice lists live in a
// static device array of FR_GENREC_NOALLOC_SCRATCH_BYTES (every GPU the
// library runs on holds its own copy until the process ends).  Its device
// address is looked up once per device, with that device current; host code
// never passes the array's name to a kernel (on the host that name is a
// stand-in, not a device address).  The slice kernel writes every list entry
// the request kernel reads, so nothing needs clearing between calls.  All
// calls on one GPU share the array: calls that overlap on one GPU (other
// streams, other threads) race.
static __device__ __align__(256) uint64_t genrec_static_scratch[FR_GENREC_NOALLOC_SCRATCH_BYTES / 8];

static void* genrec_static_scratch_ptr() {
  static std::mutex mu;
  static void* ptrs[kMaxDevices] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (ptrs[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(genrec_static_scratch)) != hipSuccess) return nullptr;
    ptrs[dev] = p;
  }
  return ptrs[dev];
}

extern "C" int fr_genrec_mask_topk_expand_noalloc(
    float* out_vals, int64_t* out_parents, int64_t* out_tokens, int64_t* out_indices, const float* cum,
    const float* top_logprobs, const int64_t* top_tokens, const int64_t* node_ids,
    const uint8_t* allow_table, const int64_t* token_ids_in, int64_t* token_ids_out,
    const void* next_node, int64_t* node_ids_out, const uint8_t* do_expand, const int32_t* col,
    int64_t token_base, int64_t n_nodes, int64_t vsz, int64_t invalid_node, int64_t N, int64_t BW,
    int64_t C, int64_t K, int64_t L, int apply_mask, int apply_expand, int apply_advance, int next_i32,
    void* stream) {
  const int rc = genrec_check(out_vals, out_parents, out_tokens, out_indices, cum, top_logprobs, top_tokens,
                              col, N, BW, C, K, L);
  if (rc != FR_OK || N == 0) return rc;
  const int need = fr_genrec_scratch_bytes(N, BW, K);
  if (need < 0 || need > FR_GENREC_NOALLOC_SCRATCH_BYTES) return FR_ETOOLARGE;
  void* scratch = genrec_static_scratch_ptr();
  if (scratch == nullptr) return FR_ELAUNCH;
  return genrec_launch(out_vals, out_parents, out_tokens, out_indices, scratch, cum, top_logprobs,
                       top_tokens, node_ids, allow_table, token_ids_in, token_ids_out, next_node,
                       node_ids_out, do_expand, col, token_base, n_nodes, vsz, invalid_node, N, BW, C, K, L,
                       apply_mask, apply_expand, apply_advance, next_i32, stream);
}
