/*
 * sva_hip.h -- C ABI of the MI355X (gfx950) SVA summon -> verify decode path.
 *
 * The reference (asystemoffields/sva) is pure Python on PyTorch and has no FFI;
 * each entry point below replaces the torch ops of one stage of its decode
 * path, cited as file:line.  A ctypes binding (sva_amd/_lib.py) is the host
 * side.
 *
 * Conventions
 *  - Pointers are device pointers unless stated.  Nothing here allocates,
 *    frees or synchronizes; work is enqueued on `stream` (a hipStream_t).
 *  - Returns sva_status; on failure sva_last_error() (thread-local) explains.
 *  - Query items: item = (seq * H + head) * Q + token.  Per-item buffers are
 *    laid out [n_seq, H, Q, ...] row-major.
 *  - Key rows: key n of sequence b lives at row seq_offsets[b] + n of the
 *    packed cache.  seq_offsets / seq_lens are device int64 arrays of length
 *    n_seq, or both NULL for one sequence of n_keys keys at row 0.
 *  - Element (h, row, x) of a per-head catalog lives at h * head_stride +
 *    row * row_stride + x (strides in elements).
 *  - Selection rule: top-k by (score desc, key index asc).
 */
#ifndef SVA_HIP_H
#define SVA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  SVA_OK = 0,
  SVA_ERR_INVALID_ARGUMENT = 1,
  SVA_ERR_HIP = 2,
  SVA_ERR_UNSUPPORTED = 3
} sva_status;

typedef enum { SVA_DTYPE_F32 = 0, SVA_DTYPE_BF16 = 1, SVA_DTYPE_F16 = 2 } sva_dtype;
typedef enum { SVA_CODE_U8 = 0, SVA_CODE_I16 = 1, SVA_CODE_I32 = 2, SVA_CODE_I64 = 3 } sva_code_type;
typedef enum {
  SVA_MASK_NONE = 0, /* causal rule: key n allowed for token t iff n <= len - Q + t */
  SVA_MASK_F32 = 1,  /* additive mask: allowed iff mask > -1e4                     */
  SVA_MASK_BF16 = 2,
  SVA_MASK_F16 = 3,
  SVA_MASK_BOOL = 4 /* bool mask: the reference's `mask > -1e4` allows every key */
} sva_mask_type;

/* Message for the last failed call on this thread ("" if none). */
const char *sva_last_error(void);
/* ABI version of this library. */
int sva_abi_version(void);

/*
 * Write path: low-rank keys and PQ codes of cache rows [row_begin,
 * row_begin + n_rows) for every query head (fresh catalog: all rows; append:
 * the new rows only).
 * Replaces sva/llama.py:597-616 (k_low = einsum(K, k_proj) on the repeat_kv
 * expanded keys; encode_product_keys) and sva/ops.py:10-47
 * (assign_to_centroids: argmin of |x|^2 - 2 x.c + |c|^2, first index on ties).
 *   keys      (g, row, d) at g*kv_head_stride + row*kv_row_stride + d; query
 *             head h reads KV head h / (H / G)
 *   k_proj    [H, D, R] fp32; codebooks [H, S, C, R/S] fp32 (16-byte aligned)
 *   k_low     (h, row, r) at h*k_low_head_stride + row*R + r, fp32 out
 *   codes     (h, row, s) at h*code_head_stride + row*S + s, code_type out;
 *             NULL: k_low only (the reference's lazy static tail, :604-610)
 *   D, R <= 256.  Rows keep no state: writing a row twice gives the same
 *   result.  (R, R/S multiples of 4 and 16-byte aligned fp32 buffers take the
 *   tiled path; other shapes an elementwise one with the same arithmetic.)
 */
int sva_write_encode(const void *keys, int kv_dtype, int64_t kv_head_stride, int64_t kv_row_stride,
                     int64_t row_begin, int64_t n_rows, int64_t H, int64_t G, int64_t D, int64_t R, int64_t S,
                     int64_t C, const float *k_proj, const float *codebooks, float *k_low, int64_t k_low_head_stride,
                     void *codes, int code_type, int64_t code_head_stride, void *stream);

/*
 * sva_write_encode for a batch of n_seq equal-layout caches (sva/llama.py:597-616
 * per sequence of a batch; the reference decodes batch 1): sequence b's K rows
 * start kv_seq_stride elements after sequence b - 1's, its catalog rows
 * catalog_seq_rows rows after (k_low row b * catalog_seq_rows + row of head h).
 * An append of at most four rows per sequence is one launch for the batch.
 */
int sva_write_encode_batch(const void *keys, int kv_dtype, int64_t kv_seq_stride, int64_t kv_head_stride,
                           int64_t kv_row_stride, int64_t n_seq, int64_t row_begin, int64_t n_rows, int64_t H,
                           int64_t G, int64_t D, int64_t R, int64_t S, int64_t C, const float *k_proj,
                           const float *codebooks, float *k_low, int64_t k_low_head_stride, int64_t catalog_seq_rows,
                           void *codes, int code_type, int64_t code_head_stride, void *stream);

/*
 * Learned query map and per-query PQ lookup table.
 * Replaces sva/llama.py:211 (q_low = einsum(q, q_proj) * scale) and the table
 * of sva/ops.py:66-68.
 *   q        (b, h, t, d) at b*q_seq_stride + h*q_head_stride + t*q_tok_stride + d
 *   q_proj   [H, D, R] fp32, scale [H] fp32, codebooks [H, S, C, R/S] fp32
 *            (both 16-byte aligned)
 *   codes    optional (may be NULL): the cache's codes (h, row, s) at
 *            h*code_head_stride + row*S + s, n_keys rows, used for one query
 *            token of one sequence to sample a shortlist-threshold estimate
 *   q_low    [n_seq, H, Q, R] fp32 out
 *   lut      [n_seq, H, Q, S, C] fp32 out (unscaled dot products)
 *   score_range [n_seq, H, Q, 4] fp32 out: lower and upper bound of any scan
 *            sum before the 1/sqrt(R) scale, the sampled estimate (or -inf),
 *            and 0.  Only a performance hint for sva_summon, never a result.
 */
int sva_query_lut(const void *q, int q_dtype, int64_t q_seq_stride, int64_t q_head_stride, int64_t q_tok_stride,
                  int64_t n_seq, int64_t H, int64_t Q, int64_t D, int64_t R, int64_t S, int64_t C,
                  const float *q_proj, const float *scale, const float *codebooks, const void *codes,
                  int code_type, int64_t code_head_stride, int64_t n_keys, int64_t shortlist, float *q_low,
                  float *lut, float *score_range, void *stream);

/*
 * PQ scan scores for every key (sva/ops.py:50-71, product_quantized_scores):
 * scores[item, n] = (((0 + T0[c0]) + T1[c1]) + ...) / sqrt(R).
 *   codes    (h, row, s) at h*code_head_stride + row*S + s
 *   scores   [n_seq, H, Q, n_keys] fp32 out (entries past a sequence's length untouched)
 */
int sva_pq_scores(const float *lut, const void *codes, int code_type, int64_t code_head_stride,
                  const int64_t *seq_offsets, const int64_t *seq_lens, int64_t n_seq, int64_t H, int64_t Q,
                  int64_t n_keys, int64_t R, int64_t S, int64_t C, float *scores, void *stream);

/*
 * Summon: PQ scan + shortlist select + exact low-rank rescore.
 * Replaces sva/llama.py:270-292 (product_quantized_scores, masked topk(L),
 * candidate_counts, gather of k_low and the rank-score sum).
 *   k_low    (h, row, r) at h*k_low_head_stride + row*R + r, fp32
 *   mask     (t, n) at t*mask_tok_stride + n with n the sequence-local key, the same
 *            rows for every sequence (equal-length batches), or NULL
 *   sl_idx   [items, L] key indices of the shortlist (first sl_count[item] valid)
 *   sl_rank  [items, L] their rank scores sum(k_low * q_low) / sqrt(R)
 *   sl_count [items] = min(L, #allowed keys)
 * workspace: sva_summon_workspace_bytes(...) bytes, 256-byte aligned.
 */
size_t sva_summon_workspace_bytes(int64_t n_seq, int64_t H, int64_t Q, int64_t n_keys, int64_t L);
int sva_summon(const float *lut, const float *score_range, const float *q_low, const void *codes, int code_type,
               int64_t code_head_stride, const float *k_low, int64_t k_low_head_stride, const int64_t *seq_offsets,
               const int64_t *seq_lens, int64_t n_seq, int64_t H, int64_t Q, int64_t n_keys, int64_t R, int64_t S,
               int64_t C, int64_t L, const void *mask, int mask_type, int64_t mask_tok_stride, int32_t *sl_idx,
               float *sl_rank, int32_t *sl_count, void *workspace, size_t workspace_bytes, void *stream);

/*
 * Summon followed by the budget select, in one call: sva_summon's outputs,
 * plus fin_idx / fin_count exactly as sva_budget_select writes them.
 * Replaces sva/llama.py:262-302 (scan, masked topk(L), rescore, topk(B),
 * counts).  On the wide path (q = 1 over a long cache) the shortlist and
 * budget selects and the rescore run in one kernel per query item.
 *   fin_idx [items, B] chosen key indices sorted ascending; fin_count[item] = min(B, sl_count[item]).
 * workspace: sva_summon_workspace_bytes(...) bytes, 256-byte aligned.
 * sl_idx and sl_rank may both be null where sva_summon_strategy is 3 (the
 * shortlist then stays inside the kernel, as in the reference's prefill,
 * which keeps only the budget); elsewhere a null pair is SVA_ERR_UNSUPPORTED.
 */
int sva_summon_select(const float *lut, const float *score_range, const float *q_low, const void *codes,
                      int code_type, int64_t code_head_stride, const float *k_low, int64_t k_low_head_stride,
                      const int64_t *seq_offsets, const int64_t *seq_lens, int64_t n_seq, int64_t H, int64_t Q,
                      int64_t n_keys, int64_t R, int64_t S, int64_t C, int64_t L, const void *mask, int mask_type,
                      int64_t mask_tok_stride, int32_t *sl_idx, float *sl_rank, int32_t *sl_count, int64_t B,
                      int32_t *fin_idx, int32_t *fin_count, void *workspace, size_t workspace_bytes, void *stream);

/*
 * Decode lookup of one token of one sequence, query side and summon in one
 * call: the results of sva_query_lut (q_low [H, R], lut [H, S, C],
 * score_range [H, 4]) followed by sva_summon_select (shortlist and budget)
 * on the same arguments.  Replaces sva/llama.py:211 (q_low), sva/ops.py:50-71
 * (table and scan) and sva/llama.py:276-302 (shortlist, rescore, budget) for
 * q_len = 1.  workspace: sva_summon_workspace_bytes(1, H, 1, n_keys, L).
 */
int sva_lookup_select(const void *q, int q_dtype, int64_t q_head_stride, int64_t H, int64_t D, int64_t R, int64_t S,
                      int64_t C, const float *q_proj, const float *scale, const float *codebooks, const void *codes,
                      int code_type, int64_t code_head_stride, const float *k_low, int64_t k_low_head_stride,
                      int64_t n_keys, int64_t L, const void *mask, int mask_type, int64_t mask_tok_stride,
                      float *q_low, float *lut, float *score_range, int32_t *sl_idx, float *sl_rank,
                      int32_t *sl_count, int64_t B, int32_t *fin_idx, int32_t *fin_count, void *workspace,
                      size_t workspace_bytes, void *stream);

/*
 * The whole decode step of one token of one sequence: sva_lookup_select
 * followed by sva_verify on its budget lists, writing the attention output
 * out [H, D] (head stride out_head_stride) besides every lookup output.
 * Replaces sva/llama.py:211-317 for q_len = 1 (q_low, scan, shortlist,
 * rescore, budget, exact verifier).  On the wide path (sva_summon_strategy
 * 1) with D = 64 or 128 the verifier runs inside the finish kernel, each
 * item's workgroup over the list it has just selected; otherwise
 * sva_verify runs after the lookup with verify_workspace
 * (sva_verify_workspace_bytes(1, H, G, 1, D, B)).  One subspace of at most
 * 256 codewords selects by code class (count, boundary class, ordered
 * extraction, budget) with the verifier inside its budget kernel.  K / V rows
 * of KV head g at g * kv_head_stride + n * kv_row_stride elements; query head
 * h reads KV head h / (H / G).  floor_overshoot (optional, int32 [H]): 1 for
 * a head whose sampled shortlist floor overshot (fewer than L keys above
 * it), so that the finish selected over every key; 0 otherwise.
 */
int sva_lookup_verify(const void *q, int q_dtype, int64_t q_head_stride, int64_t H, int64_t D, int64_t R, int64_t S,
                      int64_t C, const float *q_proj, const float *scale, const float *codebooks, const void *codes,
                      int code_type, int64_t code_head_stride, const float *k_low, int64_t k_low_head_stride,
                      int64_t n_keys, int64_t L, const void *mask, int mask_type, int64_t mask_tok_stride,
                      float *q_low, float *lut, float *score_range, int32_t *sl_idx, float *sl_rank,
                      int32_t *sl_count, int64_t B, int32_t *fin_idx, int32_t *fin_count, void *workspace,
                      size_t workspace_bytes, const void *keys, const void *values, int kv_dtype,
                      int64_t kv_head_stride, int64_t kv_row_stride, int64_t G, float scaling, void *out,
                      int out_dtype, int64_t out_head_stride, void *verify_workspace, size_t verify_workspace_bytes,
                      int32_t *floor_overshoot, void *stream);

/*
 * Which summon strategy a call with these shapes takes (16-byte aligned
 * catalogs assumed): 0 = one workgroup per query item, 1 = wide path (q = 1
 * over a long cache: many workgroups per item, one pass over the codes),
 * 2 = code-class path (the wide path's shapes with one subspace of at most
 * 256 codewords: the shortlist taken by code class from per-chunk code
 * counts), 3 = one workgroup per query item that selects, rescores and
 * budgets in registers (R = 64, L <= 2048, at most 16384 keys; the
 * sva_summon_select form; sva_summon on these shapes takes strategy 0).
 */
int sva_summon_strategy(int64_t n_seq, int64_t H, int64_t Q, int64_t n_keys, int64_t R, int64_t S, int64_t C,
                        int64_t L, int code_type, int mask_type);

/*
 * Budget select: top-B of each shortlist by (rank desc, key index asc).
 * Replaces sva/llama.py:293-302 (masked topk(B), gather, verified counts).
 *   fin_idx [items, B] chosen key indices sorted ascending; fin_count[item] = min(B, sl_count[item]).
 */
int sva_budget_select(const int32_t *sl_idx, const float *sl_rank, const int32_t *sl_count, int64_t n_items,
                      int64_t L, int64_t B, int32_t *fin_idx, int32_t *fin_count, void *stream);

/*
 * Exact verifier, GQA-aware: for each KV head g and token, the union of the
 * budget lists of its H/G query heads is read once (each selected K and V row
 * is fetched by exactly one workgroup); each row is scored against every query
 * head that selected it (fp32, times `scaling`), then a softmax and the
 * weighted V sum per head, merged across workgroups by a second kernel.
 * Replaces sva/llama.py:304-317 (scan path) and :532-553 (static path).
 *   keys/values (g, row, d) at g*kv_head_stride + row*kv_row_stride + d
 *   fin_idx [items, B] sorted ascending (as sva_budget_select writes them),
 *   fin_count [items]; indices outside [0, len) of their sequence are
 *   skipped, so every read stays in bounds
 *   out (b, h, t, d) at b*out_seq_stride + h*out_head_stride + t*out_tok_stride + d
 *   head_dim <= 256 (multiples of 16 take the vectorized path).
 * workspace: sva_verify_workspace_bytes(...) bytes (no state between calls).
 */
size_t sva_verify_workspace_bytes(int64_t n_seq, int64_t H, int64_t G, int64_t Q, int64_t D, int64_t B);
int sva_verify(const void *q, int q_dtype, int64_t q_seq_stride, int64_t q_head_stride, int64_t q_tok_stride,
               const void *keys, const void *values, int kv_dtype, int64_t kv_head_stride, int64_t kv_row_stride,
               const int64_t *seq_offsets, const int64_t *seq_lens, int64_t n_keys, const int32_t *fin_idx,
               const int32_t *fin_count, int64_t n_seq, int64_t H, int64_t G, int64_t Q, int64_t D, int64_t B,
               float scaling, void *out, int out_dtype, int64_t out_seq_stride, int64_t out_head_stride,
               int64_t out_tok_stride, void *workspace, size_t workspace_bytes, void *stream);

/*
 * sva_verify without a workspace argument; it allocates nothing.  No
 * counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The slice partials live in a static device array of
 * SVA_VERIFY_NOALLOC_SCRATCH_BYTES that the library holds on every GPU it
 * runs on until the process ends; a call whose sva_verify_workspace_bytes()
 * exceeds it fails with SVA_ERR_UNSUPPORTED (use sva_verify then).  Every
 * call on one GPU shares that GPU's array, so calls that overlap on one GPU
 * (concurrent streams or host threads) race: the caller serializes them.
 * Nothing in the array needs to start at zero: each call writes every
 * partial it reads.  Results equal sva_verify's on the same arguments.
 */
#define SVA_VERIFY_NOALLOC_SCRATCH_BYTES (4u << 20)
int sva_verify_noalloc(const void *q, int q_dtype, int64_t q_seq_stride, int64_t q_head_stride,
                       int64_t q_tok_stride, const void *keys, const void *values, int kv_dtype,
                       int64_t kv_head_stride, int64_t kv_row_stride, const int64_t *seq_offsets,
                       const int64_t *seq_lens, int64_t n_keys, const int32_t *fin_idx, const int32_t *fin_count,
                       int64_t n_seq, int64_t H, int64_t G, int64_t Q, int64_t D, int64_t B, float scaling, void *out,
                       int out_dtype, int64_t out_seq_stride, int64_t out_head_stride, int64_t out_tok_stride,
                       void *stream);

/*
 * A patched layer's scan-mode decode step (one token of one sequence) behind
 * a handle, so that a decode loop pays one short call per layer: the catalog
 * append of the KV cache's new rows, the lookup with its verifier and the
 * step's statistics.  Replaces, for q_len = 1, the per-call work of
 * SVALlamaAttention.forward after the KV-cache update: the catalog append
 * (sva/llama.py:597-616), the lookup and exact verifier (sva/llama.py:211-317)
 * and the stats accounting (sva/llama.py:319-326).
 *
 * sva_decode_layer_create keeps the layer's sizes and weights (q_proj
 * [H, D, R], scale [H] = clamp(exp(logit_scale), 0.01, 100), codebooks
 * [H, S, C, R/S], k_proj [H, D, R], all fp32 on the device; the pointers must
 * stay valid for the handle's life), the shortlist L and budget B, and the
 * verifier's scaling.
 *
 * sva_decode_layer_bind points the handle at its buffers: the catalog
 * (k_low [H, capacity, R] fp32 and codes [H, capacity, S], as sva_write_encode
 * writes them), the lookup outputs of sva_lookup_verify (q_low [H, R], lut
 * [H, S, C], score_range [H, 4], sl_idx [H, L], sl_rank [H, L], counts
 * int32 [3, H] = shortlist sizes, budget sizes and floor overshoots (the
 * last row written only by steps whose path has a sampled floor,
 * sva_summon_strategy 1 or 2), fin_idx [H, B]), its two workspaces and
 * stats (int64 [4] on the device, or NULL): every step adds the sums of its
 * shortlist sizes, budget sizes and overshoots, and H, to stats[0..3].  Bind
 * again when a buffer moves.
 *
 * sva_decode_layer_step encodes cache rows [row_begin, n_keys) into the
 * catalog (keys [G, rows, D] at g * kv_head_stride + n * kv_row_stride), then
 * runs sva_lookup_verify over the first n_keys rows (no mask: the causal
 * decode token sees every key) and writes out [H, D] (head stride
 * out_head_stride).  Stream-ordered; calls on one handle must not overlap.
 */
typedef struct sva_decode_layer sva_decode_layer;
int sva_decode_layer_create(int64_t H, int64_t G, int64_t D, int64_t R, int64_t S, int64_t C, int64_t L, int64_t B,
                            const float *q_proj, const float *scale, const float *codebooks, const float *k_proj,
                            float scaling, sva_decode_layer **out);
int sva_decode_layer_bind(sva_decode_layer *layer, float *k_low, int64_t k_low_head_stride, void *codes,
                          int code_type, int64_t code_head_stride, int64_t capacity, float *q_low, float *lut,
                          float *score_range, int32_t *sl_idx, float *sl_rank, int32_t *counts, int32_t *fin_idx,
                          void *workspace, size_t workspace_bytes, void *verify_workspace,
                          size_t verify_workspace_bytes, int64_t *stats);
int sva_decode_layer_step(sva_decode_layer *layer, const void *q, int q_dtype, int64_t q_head_stride,
                          const void *keys, const void *values, int kv_dtype, int64_t kv_head_stride,
                          int64_t kv_row_stride, int64_t row_begin, int64_t n_keys, void *out, int out_dtype,
                          int64_t out_head_stride, void *stream);
void sva_decode_layer_destroy(sva_decode_layer *layer);

/* ---------------------------------------------------------------------------
 * Inverted-index summon for q = 1 decode (summon_mode "inverted" and
 * "inverted_static").
 */

/*
 * CSR postings of the first n_rows rows: for every (head h, subspace s) and
 * cell c, the key ids with code c, ascending.
 * Replaces sva/llama.py:626-657 (_rebuild_postings; the dense table
 * [H, S, C, max_bucket] becomes offsets + ids).
 *   codes      (h, row, s) at h*code_head_stride + row*S + s
 *   offsets    [H, S, C + 1] int32 out; ids [H, S, n_rows] int32 out
 *   max_count  [H, S] int32 out: the largest cell of each (h, s)
 * C <= 1024.
 */
int sva_postings_build(const void *codes, int code_type, int64_t code_head_stride, int64_t H, int64_t n_rows,
                       int64_t S, int64_t C, int32_t *offsets, int32_t *ids, int32_t *max_count, void *stream);

/* Candidate slots per head of sva_inverted_candidates. */
int64_t sva_inverted_slots(int64_t S, int64_t postings_len, int64_t k_len, int64_t tail_start);

/*
 * Candidates of one decode token per head: the top `cells` cells of every
 * subspace by LUT / sqrt(R) (ties: lower cell index), the postings of those
 * cells (rows < postings_len, one entry per list holding a key), the rows
 * [tail_start, k_len) (static: every row; adaptive: rows whose code is in a
 * chosen cell), and one extra slot (static without a tail: the current row
 * k_len - 1; adaptive: the current row if allowed, else the last allowed row
 * as a fallback).  Each entry gets its rank score (k_low . q_low) / sqrt(R)
 * in torch's order.
 * Replaces sva/llama.py:359-392 (adaptive) and :451-495 (static).
 *   lut [H, S, C] (sva_query_lut, one token), q_low [H, R]
 *   mask: NULL / SVA_MASK_NONE / SVA_MASK_BOOL (every row allowed) or the
 *         token's additive mask row [k_len] (allowed iff > -1e4)
 *   comp [H, slots] uint64 out: (order-preserving key of the masked score
 *         << 32) | (0xFFFFFFFF - key), 0 for an empty slot
 *   flag [H, slots] uint8 out: bit 0 allowed, bit 1 fallback entry
 *   slots = sva_inverted_slots(S, postings_len, k_len, tail_start)
 */
int sva_inverted_candidates(const float *lut, const float *q_low, const float *k_low, int64_t k_low_head_stride,
                            const void *codes, int code_type, int64_t code_head_stride, const int32_t *offsets,
                            const int32_t *ids, int64_t postings_len, int64_t tail_start, int64_t k_len, int64_t H,
                            int64_t S, int64_t C, int64_t R, int64_t cells, const void *mask, int mask_type,
                            int adaptive, uint64_t *comp, uint8_t *flag, int64_t slots, void *stream);

/*
 * Selection over the candidates of each head, the reference's rules:
 *   mode 0 (static, sva/llama.py:83-116 and :497-526): refill window of the
 *     best min(width, max(B, refill_factor * B)) entries counted with
 *     multiplicity, width = S * cells * max(max_count) + (tail_len or 1) as
 *     in the dense layout; first occurrence per key; margin-adaptive budget
 *     over the min(B, refill) selected slots (fp32 comparisons);
 *   mode 1 (adaptive, sva/llama.py:383-404): distinct allowed candidates,
 *     rank_count = min(B, their number), margin-adaptive budget (the margin
 *     compared as a double), the fallback entry when no candidate is allowed.
 *   fin_idx [H, B] chosen keys ascending (for sva_verify), fin_count [H]
 *   stats [H, 4] float out: summoned, refill pool, verified, selected slots
 * workspace: sva_unique_select_workspace_bytes(H, B, refill_factor, slots).
 */
size_t sva_unique_select_workspace_bytes(int64_t H, int64_t B, int64_t refill_factor, int64_t slots);
int sva_unique_refill_select(const uint64_t *comp, const uint8_t *flag, int64_t slots, int64_t H, int mode, int64_t B,
                             int64_t min_budget, int64_t mid_budget, double low_margin, double high_margin,
                             int64_t refill_factor, const int32_t *max_count, int64_t S, int64_t cells,
                             int64_t tail_len, int32_t *fin_idx, int32_t *fin_count, float *stats, void *workspace,
                             size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------------
 * Ragged static inverted decode: the static mode above for a packed batch of
 * n_seq sequences, one launch per stage (the reference decodes batch 1 only,
 * sva/llama.py:182-183; each sequence gets sva/llama.py:427-576).  Sequence b
 * owns packed rows [seq_offsets[b], seq_offsets[b] + k_lens[b]) of codes,
 * k_low, K and V; its postings cover its first postings_lens[b] rows and its
 * tail is [postings_lens[b], k_lens[b]).  Key indices are sequence-local.
 * Items are b * H + h.  No attention mask (every row allowed).
 */

/*
 * Postings of every sequence: offsets [n_seq, H, S, C + 1], max_count
 * [n_seq, H, S], ids [H, S, rows] with sequence b's ids (local, ascending
 * within a cell) at its packed rows.  C <= 1024.
 */
int sva_postings_build_ragged(const void *codes, int code_type, int64_t code_head_stride, const int64_t *seq_offsets,
                              const int64_t *postings_lens, int64_t n_seq, int64_t H, int64_t rows, int64_t S,
                              int64_t C, int32_t *offsets, int32_t *ids, int32_t *max_count, void *stream);

/* Candidate slots per item: lists of the longest postings, the longest tail, one extra slot. */
int64_t sva_inverted_slots_ragged(int64_t S, int64_t max_postings_len, int64_t max_tail);

/*
 * Candidates of every item (sva_inverted_candidates, static mode, per
 * sequence): lut [n_seq, H, S, C] and q_low [n_seq, H, R] from sva_query_lut
 * (one token per sequence); comp / flag [n_seq * H, slots]: the item's list
 * entries in slots [0, list_counts[item]) (later list slots are not
 * written), its tail from slot S * max_postings_len, the extra slot last.
 * max_postings_len >= every postings_lens[b], max_tail >= every
 * k_lens[b] - postings_lens[b] (larger lists or tails are cut at the slots).
 * R = 64, n_seq * H <= 8192.  Two launches: lists per item, then the
 * scoring of every item's live slots spread evenly over the CUs.
 */
int sva_inverted_candidates_ragged(const float *lut, const float *q_low, const float *k_low,
                                   int64_t k_low_head_stride, const void *codes, int code_type,
                                   int64_t code_head_stride, const int32_t *offsets, const int32_t *ids, int64_t rows,
                                   const int64_t *seq_offsets, const int64_t *postings_lens, const int64_t *k_lens,
                                   int64_t n_seq, int64_t max_postings_len, int64_t max_tail, int64_t H, int64_t S,
                                   int64_t C, int64_t R, int64_t cells, uint64_t *comp, uint8_t *flag,
                                   int32_t *list_counts, int64_t slots, void *stream);

/*
 * Static-mode selection of every item (sva_unique_refill_select, mode 0):
 * sequence b's budgets are min(budget, k_lens[b]) and the adaptive minimum
 * and middle budgets derived from it as in sva/llama.py:443-445 (0: the
 * reference's defaults); its refill width uses its own largest cell and tail.
 * Only the slots sva_inverted_candidates_ragged wrote are read (list_counts).
 *   fin_idx [n_seq * H, budget] ascending local keys, fin_count, stats [.., 4]
 * workspace: sva_unique_select_workspace_bytes(n_seq * H, budget, refill_factor, slots).
 */
int sva_unique_refill_select_ragged(const uint64_t *comp, const uint8_t *flag, int64_t slots, int64_t n_seq,
                                    int64_t H, int64_t budget, int64_t adaptive_min_budget,
                                    int64_t adaptive_mid_budget, double low_margin, double high_margin,
                                    int64_t refill_factor, const int32_t *max_count, int64_t S, int64_t cells,
                                    const int64_t *postings_lens, const int64_t *k_lens, const int32_t *list_counts,
                                    int64_t max_postings_len, int32_t *fin_idx, int32_t *fin_count, float *stats,
                                    void *workspace, size_t workspace_bytes, void *stream);

/*
 * Residual output adapter of the late-layer socket, one fused launch for T
 * tokens: out = attn + (up(gelu(down([hidden, attn]))) * scale).to(attn
 * dtype), with down [rank, 2 * hidden] and up [hidden, rank] fp32 and the
 * exact (erf) GELU.
 * Replaces experiments/sva_late4_logit_distill.py:47-51
 * (SVAResidualOutputAdapter.forward after the attention).
 *   hidden / attn / out: token t's row at t * row_stride (contiguous rows)
 *   rank <= 64
 */
int sva_residual_adapter(const void *hidden, int hidden_dtype, int64_t hidden_row_stride, const void *attn,
                         int attn_dtype, int64_t attn_row_stride, const float *down_w, const float *up_w, float scale,
                         int64_t n_tokens, int64_t hidden_size, int64_t rank, void *out, int out_dtype,
                         int64_t out_row_stride, void *stream);

/*
 * k-means centroid update of the product-codebook fit, per (head, subspace,
 * cell): the mean of the cell's rows (weighted: sum of w * x over sum of w),
 * summed in ascending key order; empty cells keep their centroid.  The
 * cells are sva_postings_build's CSR of the current labels.
 * Replaces the update step of experiments/sva_pq_lookup_test.py:92-100 and
 * experiments/sva_supervised_coarse_pq_test.py:117-126.
 *   x [H, n_rows, R] fp32 (head stride x_head_stride), weights [H, n_rows] or NULL
 *   offsets [H, S, C + 1], ids [H, S, n_rows]; centroids / next [H, S, C, R / S]
 *   R / S <= 64
 */
int sva_centroid_update(const float *x, int64_t x_head_stride, int64_t n_rows, int64_t H, int64_t R, int64_t S,
                        int64_t C, const float *weights, const int32_t *offsets, const int32_t *ids,
                        const float *centroids, float *next_centroids, void *stream);

/*
 * Attention-weighted key weights of the codebook refresh: weights[h, n] =
 * 1 + boost added once per valid top-k hit of key n in head h (indices
 * clamped into [0, n_keys)), each addition rounded in turn, as index_add_
 * gives.  Replaces topk_key_weights,
 * experiments/sva_codebook_refresh_benchmark.py:136-153.
 *   top_idx [H, per_head] int64, top_valid [H, per_head] bool (uint8)
 *   weights [H, n_keys] fp32 (written; also the hit counter between passes)
 */
int sva_key_weights(const int64_t *top_idx, const uint8_t *top_valid, int64_t H, int64_t per_head, int64_t n_keys,
                    float boost, float *weights, void *stream);

/*
 * Unique refill selection over arbitrary rows of candidates
 * (SVALlamaAttention._top_unique_candidates, sva/llama.py:83-116): per row,
 * the best min(W, max(budget, refill_factor * budget)) entries by masked
 * score, the best-scored occurrence of each key, then the best
 * min(budget, refill) of those by (score desc, key asc); slots past the valid
 * ones are invalid (score -FLT_MAX).
 *   idx [H, W] int64, scores [H, W] fp32, valid [H, W] uint8
 *   sel_idx [H, cap] int32, sel_scores [H, cap] fp32, sel_valid [H, cap] uint8
 *   out, cap = min(budget, refill)
 */
size_t sva_top_unique_workspace_bytes(int64_t H, int64_t W, int64_t budget, int64_t refill_factor);
int sva_top_unique(const int64_t *idx, const float *scores, const uint8_t *valid, int64_t H, int64_t W, int64_t budget,
                   int64_t refill_factor, int32_t *sel_idx, float *sel_scores, uint8_t *sel_valid, void *workspace,
                   size_t workspace_bytes, void *stream);

/*
 * A plain streaming read of `bytes` (a positive multiple of 16, the buffer
 * 16-byte aligned): each wave reads 8 KB of consecutive 16-byte words, the
 * code scan's access pattern, and the words are folded by XOR into `sink`
 * (the XOR of all sink words is the XOR of all 32-bit words of the buffer).
 * No counterpart in the reference: a measurement helper, the time a read of
 * the scan's bytes takes on its own, which the scan is priced against.
 *   sink: sva_stream_read_sink_words(bytes) uint32 words
 */
int64_t sva_stream_read_sink_words(int64_t bytes);
int sva_stream_read(const void *src, int64_t bytes, uint32_t *sink, int64_t sink_words, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SVA_HIP_H */
