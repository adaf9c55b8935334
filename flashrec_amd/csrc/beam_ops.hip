// The beam-search trie steps one at a time (the unfused path):
//   trie_mask_candidates  -- mask candidate scores through the dense allow table
//   trie_advance_nodes    -- gather each pick's parent node and step it on the token
//   beam_expand_token_ids -- gather each pick's parent token row and set one column
// Reference: python/flashrec/kernel/beam_trie.py:82-229 (the PyTorch branches,
// which define the results; the CUDA kernels in csrc/beam_trie.cuh:66-460
// agree with them).  Used by python/flashrec/search/trie.py:480-580 and
// search/state.py when the fused step (beam_trie.hip) is not taken.
//
// The candidate rule and the transition are the fused kernel's
// (beam_trie.hip): node < 0 accepts every token and stays; a token outside
// [token_base, token_base + vsz) is refused / leads to invalid_node; nodes
// are clamped into the table.  Parents are clamped into [0, rows).  All of
// it is integer selection: results are bit-exact.  Elementwise work, one
// lane per output element, grid-stride loops over int64 indices.
#include "fr_common.h"

namespace fr {

__device__ __forceinline__ int64_t clampi(int64_t x, int64_t lo, int64_t hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}

__device__ __forceinline__ bool allowed(int64_t node, int64_t tok, const uint8_t* allow, int64_t token_base,
                                        int64_t n_nodes, int64_t vsz) {
  if (node < 0) return true;
  const int64_t rel = tok - token_base;
  if (rel < 0 || rel >= vsz || n_nodes <= 0) return false;
  return allow[clampi(node, 0, n_nodes - 1) * vsz + rel] != 0;
}

template <bool NEXT_I32>
__device__ __forceinline__ int64_t step_node(int64_t old, int64_t tok, const void* next, int64_t token_base,
                                             int64_t n_nodes, int64_t vsz, int64_t invalid) {
  if (old < 0) return old;
  const int64_t rel = tok - token_base;
  if (rel < 0 || rel >= vsz || n_nodes <= 0) return invalid;
  const int64_t at = clampi(old, 0, n_nodes - 1) * vsz + rel;
  return NEXT_I32 ? static_cast<int64_t>(static_cast<const int32_t*>(next)[at])
                  : static_cast<const int64_t*>(next)[at];
}

__global__ __launch_bounds__(256) void mask_kernel(float* out, const float* scores, const int64_t* toks,
                                                   const int64_t* nodes, const uint8_t* allow,
                                                   int64_t token_base, int64_t n_nodes, int64_t vsz,
                                                   float neg_inf, int64_t rows, int64_t cols) {
  const int64_t total = rows * cols;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t r = i / cols;
    out[i] = allowed(nodes[r], toks[i], allow, token_base, n_nodes, vsz) ? scores[i] : neg_inf;
  }
}

// batch b: out[b, i] = step(nodes[b, clamp(parents[b, i])], tokens[b, i])
template <bool NEXT_I32>
__global__ __launch_bounds__(256) void advance_kernel(int64_t* out, const int64_t* nodes, const int64_t* parents,
                                                      const int64_t* toks, const void* next, int64_t token_base,
                                                      int64_t n_nodes, int64_t vsz, int64_t invalid,
                                                      int64_t batch, int64_t rows, int64_t picks) {
  const int64_t total = batch * picks;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t b = i / picks;
    const int64_t old = nodes[b * rows + clampi(parents[i], 0, rows - 1)];
    out[i] = step_node<NEXT_I32>(old, toks[i], next, token_base, n_nodes, vsz, invalid);
  }
}

// out[p, c] = token_ids[clamp(parents[p]), c] for c < width, new_tokens[p] at c == col
// (out has out_width = max(width, col + 1) columns; the extra column is new)
__global__ __launch_bounds__(256) void expand_kernel(int64_t* out, const int64_t* token_ids, const int64_t* parents,
                                                     const int64_t* new_tokens, int64_t rows, int64_t width,
                                                     int64_t picks, int64_t out_width, int64_t col) {
  const int64_t total = picks * out_width;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t p = i / out_width;
    const int64_t c = i - p * out_width;
    out[i] = c == col ? new_tokens[p] : token_ids[clampi(parents[p], 0, rows - 1) * width + c];
  }
}

static dim3 grid_for(int64_t total) {
  const int64_t blocks = (total + 255) / 256;
  return dim3(static_cast<unsigned>(blocks < 65536 ? blocks : 65536));
}

}  // namespace fr

using namespace fr;

extern "C" {

int fr_trie_mask_candidates(float* out, const float* scores, const int64_t* cand_tokens, const int64_t* node_ids,
                            const uint8_t* allow_table, int64_t rows, int64_t cols, int64_t n_nodes, int64_t vsz,
                            int64_t token_base, float neg_inf, void* stream) {
  if (rows < 0 || cols < 0 || n_nodes < 0 || vsz < 0) return FR_EINVAL;
  if (rows == 0 || cols == 0) return FR_OK;
  if (!out || !scores || !cand_tokens || !node_ids || (n_nodes > 0 && vsz > 0 && !allow_table))
    return FR_EINVAL;
  hipLaunchKernelGGL(mask_kernel, grid_for(rows * cols), dim3(256), 0, static_cast<hipStream_t>(stream), out,
                     scores, cand_tokens, node_ids, allow_table, token_base, n_nodes, vsz, neg_inf, rows, cols);
  return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
}

int fr_trie_advance_nodes(int64_t* out, const int64_t* node_ids, const int64_t* parents, const int64_t* tokens,
                          const void* next_node, int next_i32, int64_t batch, int64_t rows, int64_t picks,
                          int64_t n_nodes, int64_t vsz, int64_t token_base, int64_t invalid_node,
                          void* stream) {
  if (batch < 0 || rows < 0 || picks < 0 || n_nodes < 0 || vsz < 0) return FR_EINVAL;
  if (batch == 0 || picks == 0) return FR_OK;
  if (rows == 0 || !out || !node_ids || !parents || !tokens || (n_nodes > 0 && vsz > 0 && !next_node))
    return FR_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (next_i32)
    hipLaunchKernelGGL(advance_kernel<true>, grid_for(batch * picks), dim3(256), 0, st, out, node_ids, parents,
                       tokens, next_node, token_base, n_nodes, vsz, invalid_node, batch, rows, picks);
  else
    hipLaunchKernelGGL(advance_kernel<false>, grid_for(batch * picks), dim3(256), 0, st, out, node_ids, parents,
                       tokens, next_node, token_base, n_nodes, vsz, invalid_node, batch, rows, picks);
  return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
}

int fr_beam_expand_token_ids(int64_t* out, const int64_t* token_ids, const int64_t* parents,
                             const int64_t* new_tokens, int64_t rows, int64_t width, int64_t picks, int64_t col,
                             void* stream) {
  if (rows < 0 || width < 0 || picks < 0 || col < 0) return FR_EINVAL;
  if (picks == 0) return FR_OK;
  if (rows == 0 || !out || !token_ids || !parents || !new_tokens) return FR_EINVAL;
  const int64_t out_width = col < width ? width : col + 1;
  if (col > width) return FR_EINVAL;  // at most one new column
  hipLaunchKernelGGL(expand_kernel, grid_for(picks * out_width), dim3(256), 0, static_cast<hipStream_t>(stream),
                     out, token_ids, parents, new_tokens, rows, width, picks, out_width, col);
  return hipGetLastError() == hipSuccess ? FR_OK : FR_ELAUNCH;
}

}  // extern "C"
