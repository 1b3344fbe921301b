/*
 * nvx_spec.h -- C ABI of libnvx_spec.so, the MI355X (gfx950) speculative-decoding
 * verify path: n-gram drafter, paged tree attention, temperature softmax + tree /
 * chain rejection sampling (also fused, without materialising the probabilities),
 * KV-cache slot scatter and accepted-path compaction;
 * beside them, the fused model layers the verify step runs around the attention
 * and the EAGLE-3 draft head's top-k of log-probabilities.
 *
 * Conventions
 *   - Plain pointers to device memory, sizes in elements unless a name says
 *     _bytes.  The caller owns every buffer; no entry point allocates device
 *     memory.  Work is enqueued on `stream` (a hipStream_t; NULL = legacy
 *     default stream) and never synchronises the host.
 *   - Return 0 on success, a negative NVX_E* code otherwise; nvx_last_error()
 *     returns a message for the calling thread's last failure.
 *   - The reference (nano-vllm 0.2.0) exposes these as Python modules, not a C
 *     ABI; each declaration cites the reference interface it replaces or feeds.
 *     The Python host mirror (nano-vllm-x_amd/nanovllm) binds them with ctypes.
 */
#ifndef NVX_SPEC_H
#define NVX_SPEC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NVX_OK 0
#define NVX_EINVAL -1 /* bad argument (shape, dtype, alignment, range) */
#define NVX_EHIP -2   /* HIP runtime error (launch, event) */

#define NVX_DTYPE_F32 0
#define NVX_DTYPE_BF16 1
#define NVX_DTYPE_F16 2

/* Library version (major*10000 + minor*100 + patch). */
int nvx_version(void);

/* Message for the calling thread's most recent failure ("" if none). */
const char* nvx_last_error(void);

/* ------------------------------------------------------------------ drafter --
 * N-gram prompt-lookup drafting over a packed batch of token histories.
 * Feeds from Sequence.token_ids (reference nanovllm/engine/sequence.py:21,
 * :67-70); the reference has no drafter.  Semantics of transformers'
 * PromptLookupCandidateGenerator.get_candidates: for n = min(max_ngram, L-1)
 * down to min_ngram, the left-most earlier occurrence of the last n tokens whose
 * continuation is non-empty wins; propose up to num_draft following tokens.
 *   tokens  int32 [offsets[num_seqs]]     offsets int64 [num_seqs + 1]
 *   draft   int32 [num_seqs, num_draft]   (-1 padded)   draft_len int32 [num_seqs]
 * Limits: 1 <= min_ngram <= max_ngram <= 8, num_draft >= 1.
 */
int nvx_ngram_propose(const int32_t* tokens, const int64_t* offsets, int32_t num_seqs,
                      int32_t min_ngram, int32_t max_ngram, int32_t num_draft,
                      int32_t* draft, int32_t* draft_len, void* stream);

/* ------------------------------------------------------------ KV slot scatter --
 * Replaces store_kvcache / store_kvcache_kernel (reference
 * nanovllm/layers/attention.py:10-40): for i < num_tokens with
 * slot_mapping[i] != -1, copy row_bytes bytes from key + i*key_stride_bytes to
 * k_cache + slot*row_bytes, and likewise value -> v_cache.
 */
int nvx_store_kvcache(const void* key, int64_t key_stride_bytes, const void* value,
                      int64_t value_stride_bytes, void* k_cache, void* v_cache,
                      const int32_t* slot_mapping, int32_t num_tokens, int32_t row_bytes,
                      void* stream);

/* ------------------------------------------------------------- KV compaction --
 * Moves the accepted path of each verified draft tree into contiguous cache
 * positions, for num_layers layers of K and V: row(ctx + d) <- row(ctx + path[d])
 * for d = 1..accepted_len[b], where row(pos) is slot
 * block_tables[b][pos / block_size] * block_size + pos % block_size (reference slot
 * formula, nanovllm/engine/model_runner.py:151-161, :181; cache layout :115).
 * Generalises store_kvcache (attention.py:21-30) to a cache-resident source; the
 * reference has no compaction.  Layer l of K lives at k_cache + l*layer_stride_bytes.
 *   block_tables int32 [num_seqs, block_table_stride]   ctx_lens int32 [num_seqs]
 *   path int32 [num_seqs, path_stride]                    accepted_len int32 [num_seqs]
 */
int nvx_kv_compact(void* k_cache, void* v_cache, int64_t layer_stride_bytes,
                   int32_t num_layers, int32_t row_bytes, int32_t block_size,
                   const int32_t* block_tables, int32_t block_table_stride,
                   const int32_t* ctx_lens, const int32_t* path, int32_t path_stride,
                   const int32_t* accepted_len, int32_t num_seqs, void* stream);

/* ----------------------------------------------------------- tree attention --
 * Paged attention of q_len query rows per sequence against the paged KV cache,
 * with an ancestor mask over the sequence's last q_len cached positions.  Replaces
 * the decode call flash_attn_with_kvcache(..., cache_seqlens=context_lens,
 * block_table=block_tables, softmax_scale=scale, causal=True) (reference
 * nanovllm/layers/attention.py:71-74) and, with tree_mask = NULL, the prefill call
 * flash_attn_varlen_func(..., causal=True, block_table=...) (:64-70) once the
 * prompt's K/V are in the cache.
 *   q, o          bf16 [cu_seqlens_q[num_seqs], num_heads, 128]
 *   k/v_cache     bf16 [*, block_size, num_kv_heads, 128]   (model_runner.py:115)
 *   block_tables  int32 [num_seqs, block_table_stride]
 *   cu_seqlens_q  int32 [num_seqs + 1]      context_lens int32 [num_seqs] (includes q rows,
 *                 each <= max_context_len, which sizes the launch)
 *   max_seqlen_q  >= every q_len (it sizes the q-row chunks of the launch)
 *   tree_mask     uint64 [total q rows] or NULL: bit m of row i's mask makes key
 *                 (context_len - q_len + m) visible; NULL = causal (m <= i).
 *                 With a mask, q_len <= 64.
 *   workspace     device scratch of nvx_tree_attention_workspace_size() bytes
 *                 (may be NULL when that size is 0).
 * Limits: head_dim == 128, block_size % 64 == 0, num_heads % num_kv_heads == 0.
 */
size_t nvx_tree_attention_workspace_size(int32_t num_seqs, int32_t total_q, int32_t max_seqlen_q,
                                         int32_t max_context_len, int32_t num_heads,
                                         int32_t num_kv_heads, int32_t head_dim);

int nvx_tree_attention(const void* q, void* o, const void* k_cache, const void* v_cache,
                       const int32_t* block_tables, int32_t block_table_stride,
                       const int32_t* cu_seqlens_q, const int32_t* context_lens,
                       const uint64_t* tree_mask, int32_t num_seqs, int32_t total_q,
                       int32_t max_seqlen_q, int32_t max_context_len, int32_t num_heads,
                       int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                       float scale, void* workspace, size_t workspace_bytes, void* stream);

/* nvx_tree_attention_noalloc: no counterpart in the reference.  For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): nvx_tree_attention without the workspace
 * argument.  Split-KV partials go to a static device array of
 * nvx_tree_attention_noalloc_scratch_bytes() bytes (64 MiB) that the library holds
 * on every GPU it runs on until the process ends; a launch whose partials need more
 * (nvx_tree_attention_workspace_size) is refused with NVX_EINVAL.  The entry point
 * calls no allocating routine (no hipMalloc / hipFree, no timing events).  All calls
 * on one GPU share that GPU's array: calls that overlap in time on one GPU (two
 * streams, or two threads) race on it and must be serialised by the caller.  The
 * current device must be the stream's device.  Other arguments, results and errors
 * as nvx_tree_attention.
 */
size_t nvx_tree_attention_noalloc_scratch_bytes(void);
int nvx_tree_attention_noalloc(const void* q, void* o, const void* k_cache, const void* v_cache,
                               const int32_t* block_tables, int32_t block_table_stride,
                               const int32_t* cu_seqlens_q, const int32_t* context_lens,
                               const uint64_t* tree_mask, int32_t num_seqs, int32_t total_q,
                               int32_t max_seqlen_q, int32_t max_context_len, int32_t num_heads,
                               int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                               float scale, void* stream);

/* ------------------------------------------------------- temperature softmax --
 * probs[r] = softmax(float(logits[r]) / temperatures[r]) in fp32 (reference
 * nanovllm/layers/sampler.py:9-10).  Rows with temperature 0 are greedy: the fp32
 * logits are written unchanged (only their argmax is used downstream).
 *   logits  [num_rows, logits_row_stride] of logits_dtype (F32 or BF16)
 *   probs   fp32 [num_rows, vocab] (contiguous)
 */
int nvx_temperature_softmax(const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                            const float* temperatures, float* probs, int32_t num_rows,
                            int32_t vocab, void* stream);

/* -------------------------------------------------- tree rejection sampling --
 * Verifies one draft tree per sequence and emits the accepted path plus one
 * recovered/bonus token.  Sits beside Sampler.forward (reference
 * nanovllm/layers/sampler.py:5-12), whose categorical draw it generalises; the
 * reference has no rejection sampler.  Node 0 is the root (the last committed
 * token); parents[b][0] = -1 and parents[b][i] < i.  From the root, the children
 * of the current node are tested in ascending node order:
 *   accept child c (token x) iff  U[c] * q[x] <= cur[x]  and  cur[x] > 0,
 *   q = draft row of the current node (draft_mode 0) or a point mass on x
 *   (draft_mode 1); a rejection replaces cur by norm(max(cur - q, 0)).
 * When no child is accepted (or the node is a leaf) the next token is drawn from
 * cur by inverse CDF with final_uniforms[b].  Greedy rows (greedy[b] != 0): accept
 * the first child whose token is the row argmax; else next = argmax.
 *   target_probs  fp32, row (b, i) at  b*p_seq_stride + i*vocab   (rows are vocab long)
 *   draft_probs   fp32, row (b, i) at  b*q_seq_stride + i*vocab   (NULL in draft_mode 1)
 *   tokens, parents int32 [num_seqs, node_stride]; num_nodes int32 [num_seqs] or NULL
 *   uniforms fp32 [num_seqs, node_stride] in [0,1); final_uniforms fp32 [num_seqs]
 *   greedy uint8 [num_seqs] or NULL (all sampled)
 * Outputs: path int32 [num_seqs, node_stride] (accepted node ids from the root,
 * -1 padded), accepted_len int32 [num_seqs] (accepted draft nodes), out_tokens
 * int32 [num_seqs, node_stride] (accepted tokens then the next token, -1 padded),
 * next_token int32 [num_seqs].  Limits: 1 <= node_stride <= 64, vocab <= 2,097,152.
 *
 * Workspace (caller-owned, device memory): with a workspace of at least
 * nvx_rejection_walk_workspace_size(num_seqs) bytes (8-byte aligned), each sequence
 * is walked by 16, 8, 4 or 2 workgroups (the most for which the whole grid fits on
 * the GPU at once; 1 under stream capture), which meet through exchange slots in
 * the workspace.  It must be zero-filled before its first use and is then kept by
 * the library from call to call (it holds each sequence's exchange counter), so do
 * not reuse it for anything else.  Walks that overlap in time (different streams)
 * need different workspaces, and together must fit on the GPU at once.  With
 * workspace = NULL each sequence is walked by one workgroup and no state is shared:
 * any number of such calls may overlap.  If a sequence's workgroups fail to meet
 * within about a second (a device shared with a kernel that never ends), its
 * outputs are all -1 (accepted_len = next_token = -1): callers must check
 * accepted_len >= 0.  Outputs do not depend on the number of workgroups.
 */
int nvx_rejection_sample_tree(const float* target_probs, int64_t p_seq_stride,
                              const float* draft_probs, int64_t q_seq_stride, int32_t vocab,
                              const int32_t* tokens, const int32_t* parents,
                              const int32_t* num_nodes, int32_t node_stride,
                              const float* uniforms, const float* final_uniforms,
                              const uint8_t* greedy, int32_t draft_mode, int32_t num_seqs,
                              int32_t* path, int32_t* accepted_len, int32_t* out_tokens,
                              int32_t* next_token, void* workspace, size_t workspace_bytes,
                              void* stream);

/* nvx_rejection_walk_workspace_size: no counterpart in the reference.  Bytes of the
 * exchange workspace a tree / chain rejection walk of num_seqs sequences needs
 * (1,280 per sequence; 0 for num_seqs <= 0).  Sequence b always uses the same
 * 1,280 bytes, so one workspace serves walks of any batch size up to the one it was
 * sized for.
 */
size_t nvx_rejection_walk_workspace_size(int32_t num_seqs);

/* nvx_rejection_walk_max_width: no counterpart in the reference.  Bounds the
 * workgroups per sequence of later tree / chain rejection walks in this process
 * (1, 2, 4, 8 or 16; other values in [1, 16] round down to one of those) and returns
 * the previous bound, or -1 for a value outside [1, 16].  Width 1 needs no
 * cross-workgroup exchange (as a NULL workspace).  The default is 16.
 */
int nvx_rejection_walk_max_width(int32_t max_width);

/* ------------------------------------ fused softmax + tree rejection sampling --
 * Tree verification from the target logits without writing fp32 probabilities: one
 * streaming pass reads every logits row for its statistics, then the walk reads only
 * the rows it visits and recomputes each probability it needs.  No counterpart in
 * the reference; it fuses the softmax of Sampler.forward (reference
 * nanovllm/layers/sampler.py:9-10) into the walk.
 *
 * nvx_softmax_stats: per logits row r (temperature T = temperatures[r]), one online
 *   pass gives stats[2r] = max_y(logit[y]) * log2(e)/T and stats[2r+1] = 1 / sum_y
 *   exp2(logit[y] * log2(e)/T - stats[2r]) (fp32, within 1e-5 relative of the exact
 *   values); T == 0 rows get (0, 0).  Logits rows must be 16-byte aligned with vocab
 *   and row stride multiples of 8 (bf16) or 4 (fp32).  stats is [num_rows, 2] fp32,
 *   8-byte aligned (all three entry points check this).
 * nvx_softmax_from_stats: probs[r][y] = exp2(fma(logit[y], log2(e)/T, -stats[2r])) *
 *   stats[2r+1], or logit[y] when T == 0: the probabilities the fused walk uses (same
 *   alignment rules; probs 16-byte aligned, [num_rows, vocab] contiguous).
 * nvx_rejection_sample_tree_logits: nvx_rejection_sample_tree with target row (b, i)
 *   given as logits row b*node_stride + i (logits_row_stride elements apart), its
 *   temperature and its stats.  Its outputs are bit for bit those of
 *   nvx_rejection_sample_tree on the rows nvx_softmax_from_stats writes.  Other
 *   arguments and outputs as nvx_rejection_sample_tree.
 */
int nvx_softmax_stats(const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                      const float* temperatures, float* stats, int32_t num_rows, int32_t vocab,
                      void* stream);
int nvx_softmax_from_stats(const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                           const float* temperatures, const float* stats, float* probs,
                           int32_t num_rows, int32_t vocab, void* stream);
int nvx_rejection_sample_tree_logits(const void* logits, int32_t logits_dtype,
                                     int64_t logits_row_stride, const float* temperatures,
                                     const float* stats, const float* draft_probs,
                                     int64_t q_seq_stride, int32_t vocab, const int32_t* tokens,
                                     const int32_t* parents, const int32_t* num_nodes,
                                     int32_t node_stride, const float* uniforms,
                                     const float* final_uniforms, const uint8_t* greedy,
                                     int32_t draft_mode, int32_t num_seqs, int32_t* path,
                                     int32_t* accepted_len, int32_t* out_tokens,
                                     int32_t* next_token, void* workspace,
                                     size_t workspace_bytes, void* stream);

/* nvx_rejection_sample_tree_logits_lazy: the fused walk without the statistics pass.
 * On reaching a node the walk computes its row's statistics itself, only for the rows
 * it visits: stats[2r] = max_y(logit[y]) * log2(e)/T (exact), then stats[2r+1] = 1 / the
 * sum of exp2(fma(logit[y], log2(e)/T, -stats[2r])) in the walk's canonical order (the
 * same bits for every number of workgroups per sequence).  stats_out ([num_rows, 2]
 * fp32, 8-byte aligned, or NULL) receives them for the visited rows; other rows are
 * left as they were.  Rows at temperature 0 (greedy sequences) need no statistics.
 * Outputs are bit for bit those of nvx_rejection_sample_tree on the rows
 * nvx_softmax_from_stats writes from any stats that hold stats_out's values on the
 * visited rows.  It replaces nvx_softmax_stats + nvx_rejection_sample_tree_logits
 * where only the walk's outputs are needed (the verify step).  Other arguments and
 * outputs as nvx_rejection_sample_tree_logits.
 */
int nvx_rejection_sample_tree_logits_lazy(const void* logits, int32_t logits_dtype,
                                          int64_t logits_row_stride, const float* temperatures,
                                          float* stats_out, const float* draft_probs,
                                          int64_t q_seq_stride, int32_t vocab,
                                          const int32_t* tokens, const int32_t* parents,
                                          const int32_t* num_nodes, int32_t node_stride,
                                          const float* uniforms, const float* final_uniforms,
                                          const uint8_t* greedy, int32_t draft_mode,
                                          int32_t num_seqs, int32_t* path, int32_t* accepted_len,
                                          int32_t* out_tokens, int32_t* next_token,
                                          void* workspace, size_t workspace_bytes, void* stream);

/* -------------------------------------------------- fused model layers --
 * Elementwise layers of the target model around the verify-path attention, each
 * one pass over HBM (bf16 in/out, fp32 math).  Not part of the four verify-path
 * kernels; they replace chains of eager torch kernels.
 *
 * nvx_rmsnorm: RMSNorm / add+RMSNorm (reference nanovllm/layers/layernorm.py:16-40):
 *   s = x (+ residual); residual_out = bf16(s); out = bf16(bf16(s*rsqrt(mean(s^2)+eps))*w).
 *   residual and residual_out are both NULL (plain) or both set.  hidden % 8 == 0,
 *   hidden <= 8192, 16-byte aligned rows.
 * nvx_qk_norm_rope: per-head RMSNorm of the q and k heads of a fused qkv row
 *   [q (Hq heads) | k (Hkv) | v (Hkv)], then NeoX rotary embedding at positions[n]
 *   with cos_sin_cache [cache_positions, 128] fp32 (64 cos then 64 sin) (reference
 *   qwen3.py:82-85, rotary_embedding.py:6-14).  Writes contiguous q_out [N, Hq, 128];
 *   k goes to k_out [N, Hkv, 128] (may be NULL) and, when k_cache / v_cache /
 *   slot_mapping are given, k and the raw v are stored at cache row
 *   slot_mapping[n] (rows of Hkv*128 bf16; slot -1 skips the token): the fused form
 *   of store_kvcache (attention.py:62-63) for the step's new rows.  Norm weights both
 *   NULL: RoPE only (Llama-style heads without q/k norm).  A position outside
 *   [0, cache_positions) writes NaN for that token instead of reading past the
 *   table.  head_dim 128.
 * nvx_silu_mul: out[n, i] = bf16(silu(gate_up[n, i]) * gate_up[n, inter + i])
 *   (reference nanovllm/layers/activation.py:8-11).
 */
int nvx_rmsnorm(const void* x, int64_t x_row_stride, const void* residual, void* residual_out,
                const void* weight, void* out, int32_t num_rows, int32_t hidden, float eps,
                void* stream);
int nvx_qk_norm_rope(const void* qkv, int64_t qkv_row_stride, int32_t num_q_heads,
                     int32_t num_kv_heads, int32_t head_dim, const void* q_norm_weight,
                     const void* k_norm_weight, const int64_t* positions,
                     const float* cos_sin_cache, int64_t cache_positions, int32_t num_tokens,
                     void* q_out, void* k_out, void* k_cache, void* v_cache,
                     const int32_t* slot_mapping, float eps, void* stream);
int nvx_silu_mul(const void* gate_up, int64_t row_stride, void* out, int32_t num_rows,
                 int32_t inter, void* stream);

/* ------------------------------------------------------- draft-head top-k --
 * Top-k of log_softmax(logits[r]) for every row, in one pass over the logits.
 * No counterpart in the reference (nano-vllm has no draft model); it serves the
 * EAGLE-2/3 draft-tree expansion (arXiv:2406.16858), replacing
 * torch.log_softmax(logits.float()) followed by torch.topk.
 *   logits   [num_rows, logits_row_stride] of logits_dtype (BF16 or F32), 16-byte
 *            aligned; vocab and the stride are multiples of 8 (bf16) or 4 (fp32)
 *   out_tokens    int32 [num_rows, k]  token ids, by descending log-probability,
 *                 equal values ordered by the lower token id
 *   out_logprobs  fp32  [num_rows, k]  (x - max) - ln(sum exp(x - max))
 * Limits: 1 <= k <= min(64, vocab); rows free of NaN.
 */
int nvx_topk_logprobs(const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                      int32_t num_rows, int32_t vocab, int32_t k, int32_t* out_tokens,
                      float* out_logprobs, void* stream);

/* ------------------------------------------------------------------ timing --
 * Optional per-entry-point HIP-event timing on the launch stream (used by the
 * benchmark to measure kernel durations in its timed region).
 * kernel ids: 0 ngram, 1 store_kvcache, 2 kv_compact, 3 tree_attention,
 *             4 temperature_softmax, 5 rejection_sample_tree, 6 topk_logprobs.
 */
#define NVX_TIMER_NGRAM 0
#define NVX_TIMER_STORE_KV 1
#define NVX_TIMER_KV_COMPACT 2
#define NVX_TIMER_TREE_ATTENTION 3
#define NVX_TIMER_SOFTMAX 4
#define NVX_TIMER_REJECTION 5
#define NVX_TIMER_TOPK 6
#define NVX_TIMER_COUNT 7

int nvx_timing_enable(int on);
/* Synchronises the recorded events and returns the accumulated milliseconds and
 * launch count for one kernel id since the last reset. */
int nvx_timing_read(int32_t kernel_id, double* total_ms, int64_t* count);
int nvx_timing_reset(void);

#ifdef __cplusplus
}
#endif

#endif /* NVX_SPEC_H */
