/*
 * flashrec_amd: C ABI of the MI355X (gfx950) FP8 quantized compute path.
 *
 * Every entry point takes raw device pointers, element strides and a
 * hipStream_t (passed as void*), launches on that stream, never allocates,
 * never synchronises and never reads device memory from the host, so all of
 * them are safe to record into a HIP graph.  Return value: FR_OK (0) or one
 * of the FR_E* codes below.  Dtype codes: 0 bf16, 1 fp16, 2 fp32, 3 e4m3fn.
 *
 * Each declaration cites the reference interface it replaces
 * (paths relative to the sohu-mptc/FlashRec tree).
 */
#ifndef FLASHREC_AMD_H
#define FLASHREC_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FR_OK 0
#define FR_EINVAL 1        /* null pointer, negative size, bad stride/scale size */
#define FR_EUNSUPPORTED 2  /* valid request the kernels do not handle; caller falls back */
#define FR_ELAUNCH 3       /* HIP reported a launch error */
#define FR_ETOOLARGE 4     /* request exceeds a fixed capacity (no-allocation entry points) */

#define FR_DTYPE_BF16 0
#define FR_DTYPE_FP16 1
#define FR_DTYPE_FP32 2
#define FR_DTYPE_E4M3 3

/* ABI revision of this header (1). */
int fr_abi_version(void);

/* Per-token (per-row) e4m3 quantisation.
 * x: [M, K] of x_dtype (bf16/fp16/fp32) with row stride ldx (elements);
 * q: [M, K] e4m3 contiguous; s: [M] fp32, s = max(amax|x|, 1e-12) / 448,
 * q = e4m3(clamp(x / s, -448, 448)).
 * Replaces python/flashrec/kernel/sglops.py:84-96 (per_token_quant_fp8). */
int fr_per_token_quant_fp8(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                           void* q, float* s, void* stream);

/* Per-output-channel weight quantisation: w [N, K] -> q [N, K] e4m3, s [N].
 * Same arithmetic as fr_per_token_quant_fp8 along the rows of W.
 * Replaces python/flashrec/layers/linear.py:26-32 (quantize_weight_fp8). */
int fr_quantize_weight_fp8(const void* w, int w_dtype, int64_t N, int64_t K, int64_t ldw,
                           void* q, float* s, void* stream);

/* RMSNorm (optionally after `residual += x`, residual updated in place)
 * fused with per-token e4m3 quantisation.  x, residual, w: all of x_dtype
 * (FR_DTYPE_BF16, FR_DTYPE_FP16 or FR_DTYPE_FP32; intermediates rounded to
 * it as torch does, fp32 ones unrounded); residual may be NULL.  q: [M, H] e4m3 contiguous, s: [M] fp32.
 * Replaces python/flashrec/kernel/rms_fp8.py:120-145
 * (rmsnorm_per_token_quant_fp8, fused_add_rmsnorm_per_token_quant_fp8). */
int fr_rms_quant_fp8(const void* x, int x_dtype, int64_t ldx, void* residual, int64_t ldr,
                     const void* w, int64_t M, int64_t H, float eps, void* q, float* s, void* stream);

/* RMSNorm with x_dtype output (out may alias x); with residual != NULL it is
 * fused_add_rmsnorm: residual = round(residual + x), out = rmsnorm(residual).
 * x_dtype: FR_DTYPE_BF16, FR_DTYPE_FP16 or FR_DTYPE_FP32 (x, residual, w and out).
 * Replaces python/flashrec/kernel/sglops.py:33-45 (rmsnorm) and :48-61
 * (fused_add_rmsnorm). */
int fr_rmsnorm(const void* x, int x_dtype, int64_t ldx, void* residual, int64_t ldr,
               const void* w, void* out, int64_t ldo, int64_t M, int64_t H, float eps, void* stream);

/* SiLU-and-mul over [M, 2d] rows of x_dtype (FR_DTYPE_BF16, FR_DTYPE_FP16 or
 * FR_DTYPE_FP32; gate half first) fused with per-token
 * e4m3 quantisation: q [M, d] e4m3 contiguous, s [M] fp32.
 * Replaces python/flashrec/kernel/silu_fp8.py:85-119
 * (silu_and_mul_per_token_quant_fp8). */
int fr_silu_quant_fp8(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t d, void* q,
                      float* s, void* stream);

/* SiLU-and-mul with x_dtype output [M, d] (row stride ldo).
 * Replaces python/flashrec/kernel/sglops.py:143-151 (silu_and_mul). */
int fr_silu_and_mul(const void* x, int x_dtype, int64_t ldx, void* out, int64_t ldo, int64_t M,
                    int64_t d, void* stream);

/* W8A8 GEMM: out[m, n] = (sum_k a[m, k] b[k, n]) * scale_a[m] * scale_b[n]
 * (+ bias[n]).  a: [M, K] e4m3 row-major (row stride lda bytes);
 * b: [K, N] e4m3 column-major (column n at b + n * ldb); scale_a numel 1 or
 * M, scale_b numel 1 or N (fp32); bias: out_dtype [N] or NULL, bias_numel its
 * length (must be N when bias is given, else FR_EINVAL); out: [M, N]
 * of out_dtype (bf16, fp16 or fp32) with row stride ldo (elements).
 * Fast (MFMA) path: K, lda and ldb multiples of 16, a and b 16-byte aligned,
 * each operand spanning < 2 GiB; anything else runs a scalar kernel, one
 * thread per output, orders of magnitude slower (the Python wrapper repacks
 * such operands, zero-padding K, so it never takes that path).
 * Replaces python/flashrec/kernel/sglops.py:99-140 (fp8_scaled_mm). */
int fr_fp8_scaled_mm(const void* a, int64_t lda, const void* b, int64_t ldb,
                     const float* scale_a, int64_t scale_a_numel, const float* scale_b,
                     int64_t scale_b_numel, const void* bias, int64_t bias_numel, void* out,
                     int64_t ldo, int64_t M, int64_t N, int64_t K, int out_dtype, void* stream);

/* fr_fp8_scaled_mm with the residual add of the next RMSNorm folded into
 * its epilogue: out[m, n] = rnd(rnd(product[m, n]) + residual[m, n]) for
 * 16-bit out_dtype (bf16 or fp16; fp32 gives FR_EUNSUPPORTED), rnd the
 * rounding to out_dtype; residual [M, N] of out_dtype with row stride ldr.
 * out may be residual itself (then ldr must equal ldo): the residual
 * stream updated in place.  No bias.  Bit-for-bit fr_fp8_scaled_mm followed
 * by the residual update of fused_add_rmsnorm (python/flashrec/kernel/
 * sglops.py:53-55, residual = residual + x in the activation dtype), so the
 * RMSNorm that follows runs without its add.  Replaces, in the decoder layer
 * (python/flashrec/models/qwen3.py:197-210), o_proj / down_proj followed by
 * the add half of the next fused add + RMSNorm. */
int fr_fp8_scaled_mm_residual(const void* a, int64_t lda, const void* b, int64_t ldb, const float* scale_a,
                              int64_t scale_a_numel, const float* scale_b, int64_t scale_b_numel,
                              const void* residual, int64_t ldr, void* out, int64_t ldo, int64_t M, int64_t N,
                              int64_t K, int out_dtype, void* stream);

/* fr_fp8_scaled_mm with SiLU-and-mul in its epilogue (bf16 only): the N
 * weight rows of b come in chunks of 16, the 8 gate rows of a chunk followed
 * by the 8 up rows of the same output columns; with p the bf16-rounded
 * scaled product, out[m, 8k + c] = bf16(bf16(silu(p[m, 16k + c])) *
 * p[m, 16k + 8 + c]) for c < 8, out [M, N / 2] bf16 with row stride ldo.
 * N must be a multiple of 16.  Bit-for-bit fr_fp8_scaled_mm followed by
 * fr_silu_and_mul on the de-interleaved product (torch's silu in fp32, the
 * bf16 rounding after silu and after the product).  Replaces, in the MLP
 * (python/flashrec/models/qwen3.py:144-172), gate_up_proj followed by the
 * SiLU-and-mul half of silu_and_mul_per_token_quant_fp8
 * (python/flashrec/kernel/silu_fp8.py:79-82): the per-token quant of out
 * (fr_per_token_quant_fp8) completes that call.  Operands the MFMA kernel
 * cannot take (K % 16, unaligned rows) give FR_EUNSUPPORTED. */
int fr_fp8_scaled_mm_silu(const void* a, int64_t lda, const void* b, int64_t ldb, const float* scale_a,
                          int64_t scale_a_numel, const float* scale_b, int64_t scale_b_numel, void* out,
                          int64_t ldo, int64_t M, int64_t N, int64_t K, void* stream);

/* Weights rearranged once for the prearranged GEMM below: the [N, K] e4m3
 * rows w (row stride ldw bytes) as blocks of 32 rows x 64 bytes of K, each
 * block the two 1 KB halves a wave's MFMA operand registers hold:
 *   out[((n/32)*KT + k/64)*2048 + h*1024 + l*16 + b]
 *     = w[32*(n/32) + l%32][64*(k/64) + 32*(l/32) + 16*h + b]
 * (KT = ceil(K / 64) rounded up to a multiple of 4; rows past N and bytes
 * past K are zero).  out holds fr_fp8_weight_prearranged_bytes(N, K) bytes,
 * 16-byte aligned.  A layout step of the weight-load path (the reference
 * keeps weights as [K, N] column-major views, python/flashrec/layers/
 * linear.py:104-109); it has no counterpart of its own in the reference. */
int64_t fr_fp8_weight_prearranged_bytes(int64_t N, int64_t K);
int fr_fp8_weight_prearrange(const void* w, int64_t ldw, int64_t N, int64_t K, void* out, void* stream);

/* fr_fp8_scaled_mm with the weight given prearranged (w_pre, for this N and
 * K): the same results bit for bit, the weights streamed as contiguous
 * 1 KB runs straight into registers.  residual (bf16/fp16 out_dtype, [M, N],
 * row stride ldr, may alias out) or NULL: as fr_fp8_scaled_mm_residual.
 * silu != 0: as fr_fp8_scaled_mm_silu (bf16, N a multiple of 16, gate/up
 * interleaved weight rows, out [M, N/2]).  No bias.  a: K a multiple of 16,
 * lda a multiple of 16, 16-byte aligned (else FR_EUNSUPPORTED).
 * Replaces python/flashrec/kernel/sglops.py:99-140 (fp8_scaled_mm) for
 * weights the Linear layer owns. */
int fr_fp8_scaled_mm_prearranged(const void* a, int64_t lda, const void* w_pre, const float* scale_a,
                                 int64_t scale_a_numel, const float* scale_b, int64_t scale_b_numel,
                                 const void* residual, int64_t ldr, void* out, int64_t ldo, int64_t M, int64_t N,
                                 int64_t K, int out_dtype, int silu, void* stream);

/* Per-head RMSNorm of q and k (weights q_weight, k_weight: bf16 [D]),
 * NeoX rotate-half RoPE from cos_sin_cache ([cache_rows, D] fp32: cos for
 * i < D/2, sin after), q rotated in place (bf16), rotated k and raw v
 * written unscaled as e4m3 into k_cache[loc[t], h, :] / v_cache[loc[t], h, :].
 * q: [T, Hq, D], k/v: [T, Hk, D] bf16 with (token, head) strides in
 * elements; positions/loc: int64 [T]; cache strides in bytes (e4m3).
 * Slots outside [0, num_slots) and positions outside [0, cache_rows) are
 * skipped.  D must be even and <= 128 (else FR_EUNSUPPORTED).
 * Replaces python/flashrec/kernel/qk_rope_kv.py:164-250
 * (fused_qk_norm_rope_store_fp8). */
int fr_qk_norm_rope_store_fp8(void* q, int64_t sqt, int64_t sqh, const void* k, int64_t skt,
                              int64_t skh, const void* v, int64_t svt, int64_t svh,
                              const int64_t* positions, const int64_t* loc, const void* q_weight,
                              const void* k_weight, float eps, const float* cos_sin_cache,
                              int64_t cache_rows, void* k_cache, int64_t sckp, int64_t sckh,
                              void* v_cache, int64_t scvp, int64_t scvh, int64_t num_slots,
                              int64_t T, int64_t Hq, int64_t Hk, int64_t D, void* stream);

/* NeoX rotate-half RoPE of q [T, Hq, D] and k [T, Hk, D] (bf16) in place,
 * no normalisation, no KV store; same cos_sin_cache layout and rounding as
 * fr_qk_norm_rope_store_fp8.
 * Replaces python/flashrec/kernel/sglops.py:64-81 (apply_rope_inplace). */
int fr_rope_inplace(void* q, int64_t sqt, int64_t sqh, void* k, int64_t skt, int64_t skh,
                    const int64_t* positions, const float* cos_sin_cache, int64_t cache_rows,
                    int64_t T, int64_t Hq, int64_t Hk, int64_t D, void* stream);

/* NeoX rotate-half RoPE in place for the layouts fr_rope_inplace does not
 * take: q [T, Hq, D] / k [T, Hk, D] of dtype (FR_DTYPE_BF16, FR_DTYPE_FP16
 * or FR_DTYPE_FP32) with element strides (token, head, dim), any even D.
 * y1 = x1*cos - x2*sin, y2 = x2*cos + x1*sin in fp32, rounded once to the
 * dtype; tokens whose position has no cache row are left as they are.
 * Replaces the torch branch of python/flashrec/layers/rotary.py:55-71
 * (RotaryEmbedding.forward when neither fused backend takes the layout). */
int fr_rope_inplace_any(void* q, int64_t sqt, int64_t sqh, int64_t sqd, void* k, int64_t skt, int64_t skh,
                        int64_t skd, int dtype, const int64_t* positions, const float* cos_sin_cache,
                        int64_t cache_rows, int64_t T, int64_t Hq, int64_t Hk, int64_t D, void* stream);

/* KV store: k/v rows [T, row_dim] (bf16 -> e4m3 with torch conversion
 * semantics, or e4m3 copied as bytes) scattered to k_cache/v_cache rows
 * loc[t] (row strides sck/scv bytes).  Slots outside [0, num_slots) are
 * skipped.
 * Replaces python/flashrec/kvcache/pool.py:121-139 (TokenToKVPool.store)
 * and python/flashrec/kernel/sglops.py:207-222 (store_kv_cache). */
int fr_store_kv_fp8(const void* k, int64_t skt, const void* v, int64_t svt, int src_dtype,
                    const int64_t* loc, void* k_cache, int64_t sck, void* v_cache, int64_t scv,
                    int64_t num_slots, int64_t T, int64_t row_dim, void* stream);

/* KV store into a bf16 pool: bf16 k/v rows [T, row_dim] copied to
 * k_cache/v_cache rows loc[t] (row strides in elements).  Slots outside
 * [0, num_slots) are skipped.
 * Replaces python/flashrec/kernel/sglops.py:207-222 (store_kv_cache) and
 * python/flashrec/kvcache/pool.py:121-139 for a pool whose dtype matches the
 * activations. */
int fr_store_kv_bf16(const void* k, int64_t skt, const void* v, int64_t svt, const int64_t* loc,
                     void* k_cache, int64_t sck, void* v_cache, int64_t scv, int64_t num_slots,
                     int64_t T, int64_t row_dim, void* stream);

/* RoPE + KV store for a bf16 pool: q [T, Hq, D] and k [T, Hk, D] rotated in
 * place (as fr_rope_inplace), then the rotated k and the unchanged v written
 * to k_cache/v_cache [slots, Hk, D] at loc[t] (strides in elements).  Slots
 * outside [0, num_slots) and positions outside the cache are skipped.
 * Replaces python/flashrec/kernel/sglops.py:154-204 (apply_rope_and_store_kv,
 * the matching-dtype case). */
int fr_rope_store_kv_bf16(void* q, int64_t sqt, int64_t sqh, void* k, int64_t skt, int64_t skh,
                          const void* v, int64_t svt, int64_t svh, const int64_t* positions,
                          const int64_t* loc, const float* cos_sin_cache, int64_t cache_rows,
                          void* k_cache, int64_t sckp, int64_t sckh, void* v_cache, int64_t scvp,
                          int64_t scvh, int64_t num_slots, int64_t T, int64_t Hq, int64_t Hk,
                          int64_t D, void* stream);

/* Paged attention over the e4m3 KV pool, page size 1, head dim 128.
 * q: [T, Hq, 128] bf16 (token / head strides sqt, sqh in elements);
 * k_cache, v_cache: [num_slots, Hk, 128] e4m3 (slot / head strides in bytes);
 * query token t attends to slots kv_indices[kv_start[t] .. + kv_len[t])
 * (int32; slots outside [0, num_slots) are skipped) with query head h using
 * kv head h / (Hq / Hk); out: [T, Hq, 128] bf16 = softmax(q k^T * scale) v,
 * fp32 arithmetic; a token with no visible slot gets zeros.  Decode passes one
 * token per row (kv_start = kv_indptr[row], kv_len = seq_len); causal
 * prefill passes, for token j of a row with prefix P, kv_len = P + j + 1.
 * Replaces the decode / prefill run of python/flashrec/attention/flashinfer.py
 * :212-238 (AttentionBackend.forward over the plans of :262-378), whose
 * semantics are those of its _sdpa fallback (:380-431). */
int fr_paged_attention_fp8(const void* q, int64_t sqt, int64_t sqh, const void* k_cache,
                           int64_t skp, int64_t skh, const void* v_cache, int64_t svp, int64_t svh,
                           int64_t num_slots, const int32_t* kv_indices, const int32_t* kv_start,
                           const int32_t* kv_len, void* out, int64_t sot, int64_t soh, int64_t T,
                           int64_t Hq, int64_t Hk, int64_t D, float scale,
                           const int32_t* group_prefix, void* stream);

/* fr_paged_attention_fp8 fused with the per-token e4m3 quant of its output,
 * the input of the o projection: out_q [T, Hq * 128] e4m3 (row stride ldq
 * bytes, a multiple of 8), out_scale [T] fp32, bit-for-bit the codes and
 * scales of fr_paged_attention_fp8 followed by fr_per_token_quant_fp8 on its
 * bf16 output (no bf16 output is written).  Takes Hk <= 8 and Hq / Hk in
 * {1, 2, 4}; FR_EUNSUPPORTED otherwise (the caller then runs the two steps).
 * Replaces the reference's attention output -> o_proj input pair,
 * python/flashrec/models/qwen3.py:131-134 -> layers/linear.py:118-151 ->
 * kernel/sglops.py:84-96 (per_token_quant_fp8). */
int fr_paged_attention_quant_fp8(const void* q, int64_t sqt, int64_t sqh, const void* k_cache,
                                 int64_t skp, int64_t skh, const void* v_cache, int64_t svp, int64_t svh,
                                 int64_t num_slots, const int32_t* kv_indices, const int32_t* kv_start,
                                 const int32_t* kv_len, void* out_q, int64_t ldq, float* out_scale, int64_t T,
                                 int64_t Hq, int64_t Hk, int64_t D, float scale,
                                 const int32_t* group_prefix, void* stream);

/* The per-batch attention plan, computed once for all layers that attend
 * over the same kv_indices / kv_start / kv_len: for each group of 32 / (Hq /
 * Hk) consecutive query tokens, the slot prefix all of them share, rounded
 * down to 32 (0: none).  fr_paged_attention_plan_size gives the entry count
 * (-1 for an unsupported head ratio).  Passing the plan as group_prefix to
 * fr_paged_attention_fp8 skips that detection in every call (null: each call
 * detects it).  No counterpart in the reference: flashinfer plans its own
 * decode batches (python/flashrec/attention/flashinfer.py:262-349). */
int64_t fr_paged_attention_plan_size(int64_t T, int64_t Hq, int64_t Hk);
int fr_paged_attention_plan(const int32_t* kv_indices, const int32_t* kv_start, const int32_t* kv_len,
                            int64_t T, int64_t Hq, int64_t Hk, int32_t* group_prefix, void* stream);

/* Scratch bytes fr_genrec_mask_topk_expand needs for N requests of BW beams
 * and K picks (-1 when K is outside 1..1024).  No counterpart in the
 * reference, whose kernel sizes its own scratch (beam_trie.py:462). */
int fr_genrec_scratch_bytes(int64_t N, int64_t BW, int64_t K);

/* Fused beam step over trie-constrained candidates, per request n < N:
 * scores = cum[n, b] + top_logprobs[n, b, c] (each beam's C columns sorted
 * descending, as a sorted per-row top-k gives them), masked by
 * allow_table[node_ids[n, b]][top_tokens - token_base] when apply_mask
 * (node < 0 accepts all); top K by score descending then flat index b*C+c
 * ascending -> out_vals / out_parents (b) / out_tokens / out_indices [N, K];
 * with apply_expand: token_ids_out[n, b] = token_ids_in[n, parent_b] with
 * column col[n] set to the picked token (rows b >= K copied); with
 * apply_advance: node_ids_out[n, b] = next_node[node of parent_b][tok -
 * token_base] (node < 0 kept, token outside the table -> invalid_node);
 * next_node is int32 when next_i32 (the trie's own table dtype,
 * python/flashrec/search/trie.py:220), else int64.
 * Fewer than K valid candidates: the missing picks are (-inf, 0, top_tokens[n,
 * 0, 0], 0).  token_ids_in and token_ids_out must not alias.  K <= 1024.
 * Replaces python/flashrec/kernel/beam_trie.py:536-633
 * (genrec_mask_topk_expand; kernel csrc/beam_trie.cuh:548-757). */
int fr_genrec_mask_topk_expand(float* out_vals, int64_t* out_parents, int64_t* out_tokens,
                               int64_t* out_indices, void* scratch, int64_t scratch_bytes,
                               const float* cum, const float* top_logprobs, const int64_t* top_tokens,
                               const int64_t* node_ids, const uint8_t* allow_table,
                               const int64_t* token_ids_in, int64_t* token_ids_out,
                               const void* next_node, int64_t* node_ids_out,
                               const uint8_t* do_expand, const int32_t* col, int64_t token_base,
                               int64_t n_nodes, int64_t vsz, int64_t invalid_node, int64_t N,
                               int64_t BW, int64_t C, int64_t K, int64_t L, int apply_mask,
                               int apply_expand, int apply_advance, int next_i32, void* stream);

/* The beam-search trie steps one at a time (the unfused path of
 * python/flashrec/search/trie.py:480-580 and search/state.py).  Candidate
 * rule and transition as in fr_genrec_mask_topk_expand; integer selection,
 * bit-exact.
 *
 * fr_trie_mask_candidates: out[r, c] = scores[r, c] if the token
 * cand_tokens[r, c] is allowed under node_ids[r] (allow_table [n_nodes, vsz]
 * uint8, tokens relative to token_base), else neg_inf; scores, out [rows,
 * cols] fp32 (out may alias scores).
 * Replaces python/flashrec/kernel/beam_trie.py:82-117 (trie_mask_candidates). */
int fr_trie_mask_candidates(float* out, const float* scores, const int64_t* cand_tokens, const int64_t* node_ids,
                            const uint8_t* allow_table, int64_t rows, int64_t cols, int64_t n_nodes, int64_t vsz,
                            int64_t token_base, float neg_inf, void* stream);

/* fr_trie_advance_nodes: for each of `batch` planes, out[b, i] =
 * step(node_ids[b, clamp(parents[b, i], 0, rows - 1)], tokens[b, i]) over
 * next_node [n_nodes, vsz] (int32 when next_i32, else int64); node_ids [batch,
 * rows], parents / tokens / out [batch, picks] int64.
 * Replaces python/flashrec/kernel/beam_trie.py:120-162 (trie_advance_nodes,
 * batch = 1) and :165-192 (trie_advance_nodes_batched). */
int fr_trie_advance_nodes(int64_t* out, const int64_t* node_ids, const int64_t* parents, const int64_t* tokens,
                          const void* next_node, int next_i32, int64_t batch, int64_t rows, int64_t picks,
                          int64_t n_nodes, int64_t vsz, int64_t token_base, int64_t invalid_node,
                          void* stream);

/* fr_beam_expand_token_ids: out[p, :] = token_ids[clamp(parents[p], 0, rows -
 * 1), :] with column col set to new_tokens[p]; token_ids [rows, width], out
 * [picks, max(width, col + 1)] int64 (col == width appends one column, col >
 * width is FR_EINVAL).
 * Replaces python/flashrec/kernel/beam_trie.py:195-228 (beam_expand_token_ids). */
int fr_beam_expand_token_ids(int64_t* out, const int64_t* token_ids, const int64_t* parents,
                             const int64_t* new_tokens, int64_t rows, int64_t width, int64_t picks, int64_t col,
                             void* stream);

/* fr_genrec_mask_topk_expand with no allocation anywhere, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid hipMalloc).  No counterpart in the reference.  Same arguments
 * and results without the scratch buffer: the slice lists go to a static
 * device array of FR_GENREC_NOALLOC_SCRATCH_BYTES per GPU, held until the
 * process ends (its address is looked up on the first call on each device).
 * Returns FR_ETOOLARGE when fr_genrec_scratch_bytes(N, BW, K) exceeds that
 * size (config 4, 8 x 512 beams with K = 512, needs 1.05 MB).  All calls on
 * one GPU share the array: calls that overlap on one GPU race. */
#define FR_GENREC_NOALLOC_SCRATCH_BYTES (4 << 20)
int fr_genrec_mask_topk_expand_noalloc(float* out_vals, int64_t* out_parents, int64_t* out_tokens,
                                       int64_t* out_indices, const float* cum, const float* top_logprobs,
                                       const int64_t* top_tokens, const int64_t* node_ids,
                                       const uint8_t* allow_table, const int64_t* token_ids_in,
                                       int64_t* token_ids_out, const void* next_node, int64_t* node_ids_out,
                                       const uint8_t* do_expand, const int32_t* col, int64_t token_base,
                                       int64_t n_nodes, int64_t vsz, int64_t invalid_node, int64_t N,
                                       int64_t BW, int64_t C, int64_t K, int64_t L, int apply_mask,
                                       int apply_expand, int apply_advance, int next_i32, void* stream);

/* Per-row top-C of fp32 scores x [R, V] (row stride ldx): out_vals [R, C]
 * sorted descending (NaN above +inf, equal scores by ascending index),
 * out_idx [R, C] int64 column indices (may be null), out_tokens [R, C] int64
 * = cand_ids[idx] (or idx when cand_ids is null; out_tokens may be null).
 * C <= min(V, 1024), V <= 16384.  Replaces the sorted torch.topk over the
 * stacked beam log-probs and the candidate-id gather that feed the fused beam
 * step (python/flashrec/scheduler/scheduler.py:1476-1481,
 * python/flashrec/engine/graph.py:33-43, :186-193). */
int fr_row_topk(const float* x, int64_t ldx, int64_t R, int64_t V, int64_t C,
                const int64_t* cand_ids, float* out_vals, int64_t* out_idx, int64_t* out_tokens,
                void* stream);

/* Row-wise log_softmax of fp32 logits [M, N] (out may alias x).
 * Replaces the log_softmax of python/flashrec/logits.py:118-120, :136-137. */
int fr_log_softmax_f32(const float* x, int64_t ldx, float* out, int64_t ldo, int64_t M,
                       int64_t N, void* stream);

/* fr_row_topk over log_softmax(logits) without writing the log-probs: the
 * decode step's "log_softmax of the SID head (python/flashrec/logits.py:118-120),
 * then torch.topk + the candidate gather (scheduler.py:1476-1481)".  Outputs
 * are bit-identical to fr_log_softmax_f32 followed by fr_row_topk.  Takes
 * V = 4096 or 8192 with 16-byte aligned rows (ldx % 4 == 0), else
 * FR_EUNSUPPORTED (run the two calls). */
int fr_log_softmax_row_topk(const float* logits, int64_t ldx, int64_t R, int64_t V, int64_t C,
                            const int64_t* cand_ids, float* out_vals, int64_t* out_idx,
                            int64_t* out_tokens, void* stream);

/* Measurement only, no counterpart in the reference: `blocks` workgroups of
 * four waves each run `iters` rounds of four v_mfma_scale_f32_32x32x64_f8f6f4
 * (2 * 32 * 32 * 64 flops each) on register operands, random e4m3 bytes when
 * random_operands is nonzero, else one constant byte; clocks[2 * b] and
 * clocks[2 * b + 1] receive workgroup b's s_memtime and s_memrealtime
 * (100 MHz) spans of the loop.  sink ([256] fp32) is never written in
 * practice.  bench.py --mfma-ceiling reports the sustained rate and clock. */
int fr_calib_mfma_ceiling(int64_t blocks, int64_t iters, int random_operands, uint64_t* clocks, float* sink,
                          void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHREC_AMD_H */
