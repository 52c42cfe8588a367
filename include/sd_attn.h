/*
 * C ABI of the MI355X (gfx950) spec-decode attention hot path.
 *
 * Plain pointers and sizes only: every pointer is a device address (HIP), every
 * `stream` is a hipStream_t passed as void*. Entry points enqueue work on that
 * stream, never synchronize the host, never allocate device memory (scratch comes
 * from the caller's `workspace`), and keep launch geometry a function of the
 * shape arguments only (not of device-resident lengths), so they can be captured
 * into a hipGraph. All return 0 on success and a non-zero SD_STATUS_* code
 * otherwise; sd_last_error() describes the last failure on the calling thread.
 * A workspace holds one call's intermediate data (and, for the planned entry
 * points, the plan): calls that use one workspace must run in one stream's order,
 * never overlapped.
 *
 * Layouts (row-major, element strides):
 *   KV cache    [num_blocks, block_size, num_kv_heads, head_dim] bf16, one tensor for K and one for V
 *               (nanovllm/engine/model_runner.py:260-266 per-layer views).
 *   q / out     [tokens, num_heads, head_dim] bf16, token stride given, head stride = head_dim.
 *   block table [seqs, table_width] int32, -1 padded; entries past ceil(len / block_size) are never read.
 */
#ifndef SD_ATTN_H
#define SD_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SD_ABI_VERSION 2

#define SD_STATUS_OK 0
#define SD_STATUS_BAD_ARGUMENT 1
#define SD_STATUS_UNSUPPORTED 2
#define SD_STATUS_WORKSPACE_TOO_SMALL 3
#define SD_STATUS_LAUNCH_FAILED 4

#define SD_DTYPE_BF16 0
#define SD_DTYPE_F32 1

int sd_abi_version(void);
const char* sd_last_error(void);

/*
 * KV-cache scatter. Replaces the Triton store_kvcache_kernel and its wrapper,
 * nanovllm/layers/attention.py:10-40.
 * For idx in [0, num_tokens): slot = slot_mapping[idx]; slot == -1 (any negative) skips the row
 * (graph padding, attention.py:23); otherwise row idx of key / value (num_kv_heads*head_dim contiguous
 * bf16 elements, row stride key_row_stride / value_row_stride elements) is copied to slot `slot` of
 * k_cache / v_cache viewed as [num_slots, num_kv_heads*head_dim]. Slots >= num_slots are skipped.
 */
int sd_store_kvcache(const void* key, int64_t key_row_stride, const void* value, int64_t value_row_stride,
                     void* k_cache, void* v_cache, int64_t num_slots, const int32_t* slot_mapping,
                     int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim, void* stream);

/*
 * q/k RMSNorm + rotary embedding + KV store in one pass over a layer's qkv rows. Replaces, after the qkv
 * split of Qwen3Attention.pre_attn (nanovllm/models/qwen3.py:89-96):
 *   q_norm / k_norm  RMSNorm.rms_forward, nanovllm/layers/layernorm.py:16-26 (skipped when both weights are
 *                    NULL: models with a qkv bias, qwen3.py:93);
 *   rotary_emb       RotaryEmbedding.forward + apply_rotary_emb, nanovllm/layers/rotary_embedding.py:37-48,
 *                    6-14 (neox halves, fp32 cos / sin);
 *   store_kvcache    nanovllm/layers/attention.py:33-40 as Attention.forward calls it (:62-63), when the
 *                    caches are given (then Attention.forward must not store again).
 * q [tokens, num_heads, head_dim], k / v [tokens, num_kv_heads, head_dim] bf16 with the given row strides
 * (views of one qkv row work); positions int64 [tokens]; norm weights bf16 [head_dim]; cos_sin_cache fp32
 * [max_position, head_dim] (cos of the head_dim/2 frequencies, then sin: the reference's cos_sin_cache
 * buffer). Writes q_out (may be q itself) and, if k_out is not NULL, k_out (may be k). With k_cache /
 * v_cache (both or neither, [num_slots, num_kv_heads*head_dim] bf16) the rotated k and the unchanged v
 * rows go to slot slot_mapping[t]; negative slots and slots >= num_slots are skipped.
 * Arithmetic: fp32, correctly rounded 1/sqrt(mean(x^2) + eps), bf16 rounding after the normalisation,
 * after the weight and after the rotation, as the reference's eager operations. A position outside
 * [0, max_position) gives NaN rows for that token. head_dim 128 only.
 */
int sd_qk_norm_rope_store(const void* q, int64_t q_row_stride, const void* k, int64_t k_row_stride,
                          const void* v, int64_t v_row_stride, const int64_t* positions, const void* q_norm_weight,
                          const void* k_norm_weight, float eps, const float* cos_sin_cache, int64_t max_position,
                          void* q_out, int64_t q_out_row_stride, void* k_out, int64_t k_out_row_stride,
                          void* k_cache, void* v_cache, int64_t num_slots, const int32_t* slot_mapping,
                          int32_t num_tokens, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                          void* stream);

/*
 * Decode / speculative-verify attention over the paged cache. Replaces
 * flash_attn_with_kvcache(q, k_cache, v_cache, cache_seqlens=context_lens, block_table=block_tables,
 * softmax_scale=scale, causal=True), nanovllm/layers/attention.py:71-78.
 * q holds num_seqs * num_query_tokens tokens (sequence-major). context_lens[b] counts the cached keys
 * including the sequence's num_query_tokens new ones; query i sees keys 0 .. context_lens[b]-n+i
 * (bottom-right causal). context_lens[b] == 0 (padding sequence) writes zeros.
 * Keys are cut into 32-key tiles; tile t belongs to residue t % 8, each residue is reduced with an online
 * softmax in increasing tile order and the eight residue partials are merged in residue order with a fixed
 * fma chain. That reduction depends only on key positions, so a row's result does not depend on num_seqs,
 * num_query_tokens or the other rows (bitwise), and equals the row's result from sd_varlen_attention.
 * sd_paged_decode needs the workspace only when the call has too few (sequence, KV head) pairs to merge
 * inside one workgroup (residue partials); sd_paged_decode_workspace_size also counts the sequence order
 * of the planned variant below.
 */
size_t sd_paged_decode_workspace_size(int32_t num_seqs, int32_t num_query_tokens, int32_t num_heads,
                                      int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                      int32_t table_width);
int sd_paged_decode(const void* q, int64_t q_token_stride, const void* k_cache, const void* v_cache,
                    int64_t num_blocks, int32_t block_size, const int32_t* context_lens,
                    const int32_t* block_tables, int32_t table_width, int32_t num_seqs,
                    int32_t num_query_tokens, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                    float scale, void* out, int64_t out_token_stride, void* workspace,
                    size_t workspace_bytes, void* stream);

/*
 * Decode / verify dispatch order, for callers that run many layers on one step's context lengths.
 * sd_paged_decode takes the sequences in index order. sd_paged_decode_plan writes into `workspace` (sized by
 * sd_paged_decode_workspace_size) the sequences sorted by context length, longest first (up to 1024
 * sequences; index order beyond), and sd_paged_decode_planned (same arguments as sd_paged_decode) launches
 * the workgroups in that order, so that long sequences do not end the call alone. The plan also picks the
 * K / V load policy of the planned calls: non-temporal when the contexts are balanced (longest at most twice
 * the mean), the default policy otherwise; sd_paged_decode always loads non-temporal. Order and policy only
 * decide which workgroup computes which sequence and how it loads: results are bitwise those of
 * sd_paged_decode even when the plan was made for other context lengths, as long as it was made for the
 * same num_seqs. No counterpart
 * in the reference; it serves the per-layer loop of a decode step (nanovllm/engine/model_runner.py:476-485).
 */
int sd_paged_decode_plan(const int32_t* context_lens, int32_t num_seqs, int32_t num_query_tokens, int32_t num_heads,
                         int32_t num_kv_heads, void* workspace, size_t workspace_bytes, void* stream);
int sd_paged_decode_planned(const void* q, int64_t q_token_stride, const void* k_cache, const void* v_cache,
                            int64_t num_blocks, int32_t block_size, const int32_t* context_lens,
                            const int32_t* block_tables, int32_t table_width, int32_t num_seqs,
                            int32_t num_query_tokens, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                            float scale, void* out, int64_t out_token_stride, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * Varlen prefill / mixed prefill+decode attention. Replaces
 * flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
 * softmax_scale=scale, causal=True, block_table=block_tables), nanovllm/layers/attention.py:64-70.
 * Sequence s has Lq = cu_seqlens_q[s+1]-cu_seqlens_q[s] queries (rows cu_seqlens_q[s].. of q) and
 * Lk = cu_seqlens_k[s+1]-cu_seqlens_k[s] keys; query i sees keys 0 .. Lk-Lq+i.
 * With table_width > 0, k / v are the paged caches (k_token_stride = v_token_stride = num_kv_heads*head_dim)
 * and key j of sequence s is at block block_tables[s*table_width + j/block_size]; with table_width == 0
 * key j is row cu_seqlens_k[s]+j of the fresh k / v ([total_k, num_kv_heads, head_dim], given token
 * strides; sequences whose keys would fall outside total_k rows are skipped).
 * total_q = cu_seqlens_q[num_seqs]; max_seqlen_q / max_seqlen_k bound the per-sequence lengths.
 */
size_t sd_varlen_workspace_size(int32_t num_seqs, int32_t total_q, int32_t max_seqlen_k, int32_t num_heads,
                                int32_t num_kv_heads, int32_t head_dim);
int sd_varlen_attention(const void* q, int64_t q_token_stride, const void* k, int64_t k_token_stride,
                        const void* v, int64_t v_token_stride, int64_t total_k, int64_t num_blocks, int32_t block_size,
                        const int32_t* block_tables, int32_t table_width, const int32_t* cu_seqlens_q,
                        const int32_t* cu_seqlens_k, int32_t num_seqs, int32_t total_q, int32_t max_seqlen_q,
                        int32_t max_seqlen_k, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                        float scale, void* out, int64_t out_token_stride, void* workspace,
                        size_t workspace_bytes, void* stream);

/*
 * Varlen work planning, for callers that run many layers on the same step metadata. sd_varlen_attention
 * derives its work lists from cu_seqlens_q / cu_seqlens_k on the device at every call; sd_varlen_plan writes
 * them into `workspace` once (they depend only on cu_seqlens_q, cu_seqlens_k, num_seqs, total_q,
 * max_seqlen_q and the head counts), and sd_varlen_attention_planned (same arguments as sd_varlen_attention)
 * then skips that step. The workspace must hold the plan of exactly these arguments and must not have been
 * written by any other call in between. The lists put the sequences with the most keys first (up to 1024
 * sequences; index order beyond), which changes the order work is dispatched in, never a row's result.
 * No counterpart in the reference (flash-attn plans on the host from max_seqlen alone); it serves the
 * per-layer loop of nanovllm/engine/model_runner.py:565-589.
 */
int sd_varlen_plan(const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t num_seqs, int32_t total_q,
                   int32_t max_seqlen_q, int32_t num_heads, int32_t num_kv_heads, void* workspace,
                   size_t workspace_bytes, void* stream);
int sd_varlen_attention_planned(const void* q, int64_t q_token_stride, const void* k, int64_t k_token_stride,
                                const void* v, int64_t v_token_stride, int64_t total_k, int64_t num_blocks,
                                int32_t block_size, const int32_t* block_tables, int32_t table_width,
                                const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t num_seqs,
                                int32_t total_q, int32_t max_seqlen_q, int32_t max_seqlen_k, int32_t num_heads,
                                int32_t num_kv_heads, int32_t head_dim, float scale, void* out,
                                int64_t out_token_stride, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Speculative-decoding verifier. Replaces verify_drafts(logits, draft_token_ids, num_drafts,
 * temperatures, draft_logits), nanovllm/layers/sampler.py:28-103, with the reference's internal
 * torch.rand(S, K) and exponential_(1) [S, V] passed in as `uniforms` and `exp_noise`.
 * logits: [S*(K+1), vocab] rows (row stride in elements), dtype SD_DTYPE_BF16 or SD_DTYPE_F32.
 * draft_token_ids int64 [S, K]; num_drafts int64 [S]; temperatures fp32 [S] (0 = greedy), or NULL when
 * every row is greedy: then only the argmax pass and the decision run (two launches instead of four).
 * draft_logits: [S*K, vocab] rows or NULL (n-gram: q is one-hot on the guess).
 * uniforms fp32 [S, K] and exp_noise fp32 [S, vocab] are read only for rows with temperature != 0
 * (may be NULL when every temperature is 0; a NULL one reads as u = 1 / E = 1).
 * Logsumexp and softmax statistics follow torch.logsumexp's rule (shift by the row maximum, 0 when that is
 * infinite); every exponential is computed to about 1.5 ulp.
 * Outputs num_accepted int64 [S] and next_token int64 [S].
 */
size_t sd_verify_workspace_size(int32_t num_seqs, int32_t num_draft_slots, int32_t vocab,
                                int32_t has_draft_logits);
int sd_verify_drafts(const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                     const int64_t* draft_token_ids, const int64_t* num_drafts, const float* temperatures,
                     const void* draft_logits, int32_t draft_dtype, int64_t draft_row_stride,
                     const float* uniforms, const float* exp_noise, int32_t num_seqs, int32_t num_draft_slots,
                     int32_t vocab, int64_t* num_accepted, int64_t* next_token, void* workspace,
                     size_t workspace_bytes, void* stream);

/*
 * LM head + verifier in one call. Replaces logits = compute_logits(hidden_states) (ParallelLMHead.forward,
 * nanovllm/layers/embed_head.py:56-68: the logits_indices gather and F.linear) followed by verify_drafts
 * (nanovllm/layers/sampler.py:28-103), as ModelRunner.run_verify calls them (nanovllm/engine/model_runner.py:
 * 482-483). hidden: bf16 [hidden_rows, hidden_dim] rows with row stride hidden_row_stride (16-byte aligned rows);
 * token row m = s*(K+1)+j of the verifier reads hidden row logits_indices[m], or row m when logits_indices is
 * NULL; a sequence with an index outside [0, hidden_rows) gets num_accepted = next_token = -1 (where the
 * reference's gather raises). packed_weight: the LM head weight (bf16 [vocab, hidden_dim], rows contiguous) in
 * the tile layout sd_lm_head_pack_weight writes, once per model (sd_lm_head_packed_weight_size bytes);
 * hidden_dim a multiple of 32. logits[m, n] = bf16(fp32 sum over hidden_dim) as the library GEMM rounds them.
 * With temperatures == NULL (every row greedy) the logits are never written unless logits_out is given: the
 * GEMM's epilogue takes each row's first argmax. With temperatures, logits_out ([S*(K+1), vocab] bf16, row
 * stride >= vocab) is required and the sampled rows are decided by sd_verify_drafts's passes over it. The
 * other arguments and the outputs are sd_verify_drafts's. No counterpart in the reference for the packing (the
 * reference's F.linear reads the weight as stored). A token row's logits depend on its hidden row, the weight and
 * (vocab, hidden_dim) only, never on the call's row count (num_seqs * (K+1)) or the device's CU count: the
 * vocabulary tiles of the GEMM's last round are split along hidden_dim by a rule of (vocab, hidden_dim) alone and
 * their fp32 sums added in a fixed order in the workspace. K = 0 is plain sampling (Sampler.forward,
 * sampler.py:7-16, on compute_logits' rows), so plain decode and verify steps read the same logits.
 */
size_t sd_lm_head_packed_weight_size(int32_t vocab, int32_t hidden_dim);
int sd_lm_head_pack_weight(const void* weight, int32_t vocab, int32_t hidden_dim, void* packed_weight, void* stream);
size_t sd_lm_head_verify_workspace_size(int32_t num_seqs, int32_t num_draft_slots, int32_t vocab, int32_t hidden_dim,
                                        int32_t has_draft_logits);
int sd_lm_head_verify(const void* hidden, int64_t hidden_row_stride, int32_t hidden_rows,
                      const int64_t* logits_indices, const void* packed_weight, int32_t vocab, int32_t hidden_dim,
                      const int64_t* draft_token_ids, const int64_t* num_drafts, const float* temperatures,
                      const void* draft_logits, int32_t draft_dtype, int64_t draft_row_stride, const float* uniforms,
                      const float* exp_noise, int32_t num_seqs, int32_t num_draft_slots, void* logits_out,
                      int64_t logits_out_row_stride, int64_t* num_accepted, int64_t* next_token, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * Linear layer with row-invariant results: out[m, n] = bf16(fp32 sum_k x[m, k] * w[n, k]), as F.linear in bf16
 * computes the projections of nanovllm/layers/linear.py (the reference's qkv_proj, o_proj, gate_up_proj and
 * down_proj, nanovllm/models/qwen3.py:47-63,115-126). It is the LM head's GEMM without the argmax: packed_weight
 * is w [out_features, in_features] bf16 in sd_lm_head_pack_weight's layout (in_features a multiple of 32); x bf16
 * with 16-byte aligned rows (row stride a multiple of 8 elements), out bf16 with any row stride >= out_features. Each output row depends on its
 * input row and the weight only, never on `rows`: the library GEMM picks kernels (and summation orders) by the
 * row count, which changes a model's greedy tokens with the batch; reference counterpart of the property:
 * scripts/check_padding.py:46-52 (GEMMs, padded vs alone). The workspace size is not monotonic in `rows` (a
 * call of at most 320 rows may hold fp32 range sums that a longer call keeps in registers): size it for each
 * row count a caller uses.
 */
size_t sd_linear_workspace_size(int32_t rows, int32_t out_features, int32_t in_features);
int sd_linear(const void* x, int64_t x_row_stride, int32_t rows, const void* packed_weight, int32_t out_features,
              int32_t in_features, void* out, int64_t out_row_stride, void* workspace, size_t workspace_bytes,
              void* stream);

/*
 * RMSNorm over rows of `hidden` bf16 elements. Replaces RMSNorm.forward, nanovllm/layers/layernorm.py:16-38:
 * residual == NULL: out = rms_forward(x); else s = x + residual (fp32), residual_out = bf16(s) and
 * out = add_rms_forward's normalised s. weight bf16 [hidden]; hidden a multiple of 8, at most 16384; rows
 * 16-byte aligned. out may be x and residual_out may be residual (in place). A row's result does not depend on
 * `rows` (fixed summation order), unlike the library's reductions.
 */
int sd_rms_norm(const void* x, int64_t x_row_stride, const void* residual, int64_t residual_row_stride,
                const void* weight, float eps, int32_t rows, int32_t hidden, void* out, int64_t out_row_stride,
                void* residual_out, int64_t residual_out_row_stride, void* stream);

/*
 * sd_verify_drafts without a workspace argument, for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * Same arguments, rule and results as sd_verify_drafts; the per-row statistics go to a scratch array of
 * SD_VERIFY_NOALLOC_SCRATCH_BYTES that the library holds on each GPU it runs on until the process ends
 * (looked up on the current device at its first call there). Calls that need more scratch than that
 * (sd_verify_workspace_size of the same sizes) fail with SD_STATUS_UNSUPPORTED: about 1024 sequences x 15
 * draft slots with draft logits fit. Every call on one GPU shares that GPU's scratch, so calls that overlap
 * on one GPU (concurrent streams or threads) race; calls in one stream's order are safe.
 */
#define SD_VERIFY_NOALLOC_SCRATCH_BYTES (8u << 20)
int sd_verify_drafts_noalloc(const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                             const int64_t* draft_token_ids, const int64_t* num_drafts, const float* temperatures,
                             const void* draft_logits, int32_t draft_dtype, int64_t draft_row_stride,
                             const float* uniforms, const float* exp_noise, int32_t num_seqs, int32_t num_draft_slots,
                             int32_t vocab, int64_t* num_accepted, int64_t* next_token, void* stream);

/*
 * Inputs of one later draft step. Replaces the tensor operations of ModelRunner.run_draft's loop,
 * nanovllm/engine/model_runner.py:443-452 (steps j = 1 .. k-1). For every sequence b < num_seqs:
 *   real = real_lens[b] > 0 (the first draft step's context_lens; 0 marks a padding sequence)
 *   positions[b]    = real ? last_positions[b] + step : 0
 *   slot_mapping[b] = real ? block_tables[b, pos / block_size] * block_size + pos % block_size : -1
 *   context_lens[b] = real ? pos + 1 : 0
 *   input_ids[b]    = b < num_tokens ? tokens[b] : 0   (tokens: the last sampled draft tokens, int64 [S])
 * Integer results equal the reference's (int64 arithmetic, int32 outputs truncated as torch's casts do).
 * Where the reference's gather would index past the block table (pos / block_size >= table_width), the
 * slot is -1 instead of a device fault. One launch; every output element is written.
 */
int sd_draft_step_inputs(const int32_t* real_lens, const int64_t* last_positions, const int32_t* block_tables,
                         int32_t table_width, int32_t block_size, const int64_t* tokens, int32_t num_tokens,
                         int32_t step, int32_t num_seqs, int64_t* input_ids, int64_t* positions,
                         int32_t* slot_mapping, int32_t* context_lens, void* stream);

/*
 * Token sampler. Replaces Sampler.forward(logits, temperatures), nanovllm/layers/sampler.py:5-16, with
 * the internal exponential_(1) noise passed in as exp_noise fp32 [S, vocab] (NULL if all greedy).
 * Greedy rows (temperature 0) take the first argmax; the others argmax(softmax(l/T) / max(E, 1e-10)).
 * temperatures may be NULL when every row is greedy (argmax pass only).
 */
int sd_sample(const void* logits, int32_t logits_dtype, int64_t logits_row_stride, const float* temperatures,
              const float* exp_noise, int32_t num_seqs, int32_t vocab, int64_t* next_token, void* workspace,
              size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SD_ATTN_H */
