/*
 * speech_kv.h — C ABI of the MI355X (gfx950) decoder KV-cache hot path.
 *
 * One shared library (libspeechkv.so) exports these entry points. They replace
 * the PyTorch tensor ops the reference engine runs on its decoder KV-cache path:
 *
 *   skv_append            paged KV append (slot_mapping scatter into BlockManager
 *                         blocks). Replaces `key_pool[l][blk, off] = new_k` at
 *                         speech_serving/phase_aware_scheduler.py:1001-1010 and the
 *                         prefill write at :678-690 (graph analogue: the scatter_ at
 *                         speech_serving/models.py:449-454; TTS: tts_engine.py:197-204).
 *   skv_gather            block-table gather into a zero-padded contiguous batch.
 *                         Replaces `pool[l][table].view(-1,H,D)[:T].permute(1,0,2)`
 *                         at speech_serving/tts_engine.py:177-185,
 *                         speech_serving/encoder_attention.py:50-59 and
 *                         speech_serving/phase_aware_scheduler.py:617-623, 860-882,
 *                         plus the zero-padded batching at :818-830.
 *   skv_paged_attention   fused paged self-attention decode over the block table.
 *                         Replaces matmul/mask/softmax/matmul at
 *                         speech_serving/models.py:126-165 (eager) and :444-466
 *                         (graph) together with the working-KV cat/pad at
 *                         speech_serving/phase_aware_scheduler.py:795-846,1012-1018.
 *                         Same computation as the Triton kernel at
 *                         scripts/evaluate_paging_variants.py:56-133.
 *   skv_dense_attention   attention over contiguous K/V with per-row valid length
 *                         (cross-attention against the encoder K/V handed off by
 *                         graph_direct_encoder_kv, and causal prompt attention over
 *                         contiguous K/V). Replaces speech_serving/models.py:167-203
 *                         (eager) and :468-479 (graph), with the masks of
 *                         phase_aware_scheduler.py:884-887,964-970 and
 *                         graph_decode_buffers.py:529,537 expressed as lengths.
 *   skv_copy_cross_kv     one launch that copies a request's encoder K/V for every
 *                         decoder layer into its decode slot of the slot-major
 *                         cross-attention buffer. Replaces the per-layer copy_ loop
 *                         of GraphDecodeBuffers.assign_slot at
 *                         speech_serving/graph_decode_buffers.py:317-327.
 *   skv_codebook_embed_sum  the summed per-codebook embedding rows of a multi-codebook
 *                         frame (speech_serving/models.py:39-52) in one launch.
 *   skv_argmax            greedy sampling (first maximum) with optional on-device
 *                         token feedback per decode slot. Replaces argmax +
 *                         copy_ at speech_serving/models.py:486-487 and
 *                         graph_decode_buffers.py:463.
 *
 * Conventions
 *   - Every pointer argument is a device pointer owned by the caller (PyTorch).
 *     The library never allocates, frees or synchronises; every launch is
 *     ordered on `stream` (a hipStream_t; NULL = the null stream) and is safe to
 *     record into a HIP graph.
 *   - Strides are in elements of the tensor's dtype. The innermost (head_dim)
 *     dimension must be contiguous, and every row start must be 16-byte aligned.
 *   - dtype codes: SKV_F32, SKV_F16, SKV_BF16. K/V, Q and the output share one dtype.
 *   - Return value: SKV_OK (0) on success, a negative SKV_E* code for an invalid
 *     argument, or a positive hipError_t from the launch. skv_last_error() gives
 *     a message for the last failing call on the calling thread.
 *   - Index robustness: rows whose slot (append) or block id (gather, attention)
 *     is negative or >= the pool size are skipped (append), zero-filled (gather) or
 *     excluded from the softmax (attention); no out-of-bounds access is made.
 */
#ifndef SPEECH_KV_H_
#define SPEECH_KV_H_

#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define SKV_API __attribute__((visibility("default")))
#else
#define SKV_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

enum skv_dtype { SKV_F32 = 0, SKV_F16 = 1, SKV_BF16 = 2 };

/* Bits of the attention entry points' `causal` argument (0 / 1 keep their meaning). */
enum skv_attn_flags {
  SKV_ATTN_CAUSAL = 1,             /* query qi sees ctx_lens[b] - (q_len - 1 - qi) keys */
  SKV_ATTN_ROWS_LONGEST_FIRST = 2  /* skv_paged_attention: the rows come in non-increasing ctx_lens
                                      order, so the launch need not rank them itself */
};

enum skv_status {
  SKV_OK = 0,
  SKV_EINVAL = -1,     /* bad size / null pointer / unsupported head_dim */
  SKV_EDTYPE = -2,     /* unknown dtype code */
  SKV_EALIGN = -3,     /* pointer or stride not 16-byte aligned */
  SKV_EWORKSPACE = -4, /* workspace missing or smaller than skv_attention_workspace_bytes */
  SKV_EUNSUPPORTED = -5 /* skv_linear: no workspace-free hipBLASLt algorithm for the shape */
};

/* Library version string, e.g. "speechkv 0.3.0 gfx950 src:0123456789abcdef"; the
 * src field is a hash of the sources, headers and code flags the library was
 * built from. */
SKV_API const char* skv_version(void);

/* Message describing the last non-OK return on the calling thread. */
SKV_API const char* skv_last_error(void);

/*
 * skv_append — scatter N new token rows of K and V into the paged pools.
 *   k_new, v_new : [N, H, D] rows (row stride new_stride_n, head stride new_stride_h)
 *   k_pool,v_pool: [num_blocks, block_size, H, D], contiguous
 *   slot_mapping : int64 [N] device; slot = block_id * block_size + offset;
 *                  a negative slot, or one at or past num_slots, skips that row.
 * Either v_new/v_pool pair may be NULL to append K only.
 * Rows that name the same slot in one call race (the slot ends up holding one of
 * them, not necessarily the last); the reference's writes name distinct slots
 * (each request its own next positions).
 * Reference: phase_aware_scheduler.py:1004-1010 (decode), :681-690 (prefill).
 */
SKV_API int skv_append(const void* k_new, const void* v_new,
               int64_t new_stride_n, int64_t new_stride_h,
               void* k_pool, void* v_pool,
               const int64_t* slot_mapping,
               int32_t n_tokens, int32_t num_heads, int32_t head_dim,
               int64_t num_slots, int32_t dtype, void* stream);

/*
 * skv_gather — materialise paged K/V as a zero-padded contiguous batch.
 *   block_tables : int32 [B, table_stride] device
 *   lens         : int32 [B] device, valid tokens per row (<= max_len)
 *   k_out, v_out : [B, H, max_len, D] contiguous; positions >= lens[b] are zeroed.
 * v_pool/v_out may be NULL to gather K only.
 * Reference: tts_engine.py:177-185; phase_aware_scheduler.py:617-623, 818-830.
 */
SKV_API int skv_gather(const void* k_pool, const void* v_pool,
               const int32_t* block_tables, int32_t table_stride,
               const int32_t* lens,
               void* k_out, void* v_out,
               int32_t batch, int32_t num_heads, int32_t head_dim,
               int32_t block_size, int32_t num_blocks, int32_t max_len,
               int32_t dtype, void* stream);

/*
 * skv_copy_cross_kv — encoder K/V of every decoder layer into one decode slot.
 *   For l < n_layers, kv in {K, V}, h < num_heads, t < n_tokens:
 *     dst[l*dst_stride_l + kv*dst_stride_kv + h*dst_stride_h + t*dst_stride_t + d]
 *       = src_{l,kv}[h*src_stride_h + t*src_stride_t + d]
 *   k_srcs, v_srcs : HOST arrays of n_layers device pointers (1 <= n_layers <= 64);
 *                    every source is [num_heads, >= n_tokens, head_dim] with the
 *                    same strides
 *   dst            : the slot's [n_layers, 2, num_heads, >= n_tokens, head_dim] region
 *                    (e.g. g_cross_kv[slot]); positions >= n_tokens are left as they are
 *   head_dim * element bytes must be a power-of-two multiple of 16.
 * Reference: graph_decode_buffers.py:317-327 (assign_slot's per-layer copies).
 */
SKV_API int skv_copy_cross_kv(const void* const* k_srcs, const void* const* v_srcs, int32_t n_layers,
                              int64_t src_stride_h, int64_t src_stride_t,
                              void* dst, int64_t dst_stride_l, int64_t dst_stride_kv,
                              int64_t dst_stride_h, int64_t dst_stride_t,
                              int32_t num_heads, int32_t n_tokens, int32_t head_dim,
                              int32_t dtype, void* stream);

/*
 * skv_argmax — greedy token per row: the first index of the maximum of
 * logits[r, 0:vocab] (a NaN counts as the maximum), as torch.argmax(dim=-1).
 *   logits     : [rows, row_stride] of dtype, row_stride >= vocab
 *   out_tokens : int64 [rows]
 *   row_slots  : int32 [rows] (optional) — the decode slot of each row; rows
 *                whose slot is outside [0, num_slots) get no per-slot output.
 *                Required by, and only used with, the two options below.
 *   slot_tokens: int64 [num_slots] (optional) — slot_tokens[row_slots[r]] = token,
 *                the on-device token feedback of a graph decode step.
 *   slot_eos, slot_finished, finished_count (optional, all or none):
 *                int64 [num_slots] EOS id per slot (< 0: none), int32 [num_slots]
 *                finished flags, int64 [1] counter. When a row's token is its
 *                slot's EOS id and the slot's flag is 0, the flag becomes 1 and
 *                the counter grows by 1. A host that copies the counter back
 *                with the step's tokens learns of a finished request without
 *                reading every token. Rows of one launch must name distinct
 *                slots, except slots whose EOS id is negative.
 * Reference: speech_serving/models.py:486-487; phase_aware_scheduler.py:693,
 * 997, 1026 (greedy); the EOS stop at :739-766 and the unused g_finished /
 * g_lengths state at graph_decode_buffers.py:209-211, 556-558.
 */
SKV_API int skv_argmax(const void* logits, int64_t row_stride, int32_t rows, int32_t vocab,
                       int32_t dtype, int64_t* out_tokens, const int32_t* row_slots,
                       int32_t num_slots, int64_t* slot_tokens, const int64_t* slot_eos,
                       int32_t* slot_finished, int64_t* finished_count, void* stream);

/*
 * Workspace bytes needed by skv_paged_attention / skv_dense_attention for a
 * call with `rows` = batch * q_len query rows and `num_heads` heads whose keys
 * (up to `max_len`) are split into chunks of `chunk_tokens` (0 = library
 * default for `dtype`). The workspace holds one (max, sum, acc[head_dim])
 * fp32 partial per (row, head, chunk); any content is fine on entry. Returns 0
 * when every row fits one chunk (then the workspace may be NULL).
 */
SKV_API int64_t skv_attention_workspace_bytes(int32_t rows, int32_t num_heads, int32_t head_dim,
                                      int32_t max_len, int32_t chunk_tokens, int32_t dtype);

/* Chunk size skv_dense_attention uses when chunk_tokens == 0. */
SKV_API int32_t skv_default_chunk_tokens(int32_t rows, int32_t num_heads, int32_t head_dim,
                                 int32_t max_len, int32_t dtype);

/*
 * Chunk size skv_paged_attention uses when chunk_tokens == 0 for pools of num_blocks
 * blocks of block_size tokens: skv_default_chunk_tokens, except that pools read
 * through staged block ids (a block size that is not a power of two of at least
 * 64 * (16 / element bytes) / head_dim keys, or a pool past 2 GiB) keep a chunk
 * within 254 blocks. Pass it to skv_attention_workspace_bytes to size the
 * workspace of such a call.
 * Reference: the block-table walk of scripts/evaluate_paging_variants.py:56-133
 * (one block id per BLOCK_SIZE keys).
 */
SKV_API int32_t skv_paged_chunk_tokens(int32_t rows, int32_t num_heads, int32_t num_kv_heads,
                                       int32_t head_dim, int32_t max_ctx, int32_t dtype,
                                       int32_t block_size, int32_t num_blocks);

/*
 * skv_paged_attention — softmax(q K^T * scale) V over the paged K/V of each row.
 *   q   : [B, Q, H, D] with strides (q_stride_b, q_stride_q, q_stride_h)
 *   out : [B, Q, H, D] with strides (o_stride_b, o_stride_q, o_stride_h)
 *   k_pool, v_pool : [num_blocks, block_size, num_kv_heads, D] contiguous
 *   block_tables   : int32 [*, table_stride]; row b uses table row
 *                    table_rows ? table_rows[b] : b
 *   ctx_lens : int32 [B] keys visible to the LAST query of row b (new token
 *              included). With SKV_ATTN_CAUSAL in `causal`, query qi sees
 *              ctx_lens[b] - (Q-1-qi) keys; otherwise every query sees ctx_lens[b].
 *   causal   : SKV_ATTN_CAUSAL | SKV_ATTN_ROWS_LONGEST_FIRST bits (skv_attn_flags).
 *   max_ctx  : upper bound of ctx_lens (sizes the launch grid).
 *   k_new, v_new (optional, both or neither): [B, Q, num_kv_heads, D] rows of
 *              the Q newest keys of each row, i.e. positions
 *              ctx_lens[b]-Q .. ctx_lens[b]-1. The call appends them into the
 *              pools at pool[table[pos / block_size], pos % block_size] (the
 *              reference's slot-mapping scatter, phase_aware_scheduler.py:
 *              1004-1010 and :681-690) and attends over them in the same launch.
 * A row with 0 visible keys gets a zero output. Non-causal calls with q_len >= 2 and
 * no fused append (attention over an encoder table), head_dim 64, fp16/bf16 and a
 * power-of-two block size of at least 8 run every 16 queries of a row against one
 * read of its blocks, with both products on the matrix cores; with 64 or more
 * queries per row and (row, head, 64-query) workgroups for at least three quarters
 * of the GPU's compute units, every 64 queries share one read of the blocks staged
 * in LDS.
 * Row order: the launch spreads (row, head) items over the compute units in an order that
 * balances their bytes when the items go longest row first. A decode launch (q_len 1, one
 * key chunk per row, at most 128 rows) ranks its rows by length class itself (the top 4
 * bits of the length), so rows may come in any order; results do not depend on the order.
 * A caller whose rows already come longest-first (as the graph decode lays out its batch)
 * sets SKV_ATTN_ROWS_LONGEST_FIRST in `causal` to skip the ranking (Whisper-large-v3 shape,
 * batch 64: 14.5 us with the flag, 14.9 us without it, 15.2 us for rows in random order,
 * against 17.5 us for random order without any ranking; batch 128: 27.4 us for rows in
 * random order against 29.0 us without the ranking, 25.6 us with the flag).
 * Reference: models.py:126-165, :444-466; scripts/evaluate_paging_variants.py:56-133.
 */
SKV_API int skv_paged_attention(const void* q, int64_t q_stride_b, int64_t q_stride_q, int64_t q_stride_h,
                        void* k_pool, void* v_pool,
                        const int32_t* block_tables, int32_t table_stride,
                        const int32_t* table_rows,
                        const int32_t* ctx_lens,
                        const void* k_new, const void* v_new,
                        int64_t new_stride_b, int64_t new_stride_q, int64_t new_stride_h,
                        void* out, int64_t o_stride_b, int64_t o_stride_q, int64_t o_stride_h,
                        int32_t batch, int32_t q_len, int32_t num_heads, int32_t num_kv_heads,
                        int32_t head_dim, int32_t block_size, int32_t num_blocks,
                        int32_t max_ctx, float scale, int32_t causal, int32_t dtype,
                        int32_t chunk_tokens, void* workspace, int64_t workspace_bytes,
                        void* stream);

/*
 * skv_paged_attention_noalloc — skv_paged_attention without a workspace argument.
 * No counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, hosts that forbid
 * hipMalloc). Arguments and results are those of skv_paged_attention; the split-K
 * partials live in a fixed 4 MiB device array inside the library (one per device,
 * held until the process ends), so the call allocates nothing. A call whose
 * partials (skv_attention_workspace_bytes) exceed 4 MiB returns SKV_EWORKSPACE.
 * Every call on one device shares that array: calls that overlap in time on one
 * device (different streams) race. The first call on a device looks the array's
 * address up (hipGetSymbolAddress).
 */
SKV_API int skv_paged_attention_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_q, int64_t q_stride_h,
                        void* k_pool, void* v_pool,
                        const int32_t* block_tables, int32_t table_stride,
                        const int32_t* table_rows,
                        const int32_t* ctx_lens,
                        const void* k_new, const void* v_new,
                        int64_t new_stride_b, int64_t new_stride_q, int64_t new_stride_h,
                        void* out, int64_t o_stride_b, int64_t o_stride_q, int64_t o_stride_h,
                        int32_t batch, int32_t q_len, int32_t num_heads, int32_t num_kv_heads,
                        int32_t head_dim, int32_t block_size, int32_t num_blocks,
                        int32_t max_ctx, float scale, int32_t causal, int32_t dtype,
                        int32_t chunk_tokens, void* stream);

/*
 * skv_dense_attention — attention over contiguous K/V.
 *   K/V element (slot s, kv head h, position t, dim d) is at
 *   k[s*kv_stride_s + h*kv_stride_h + t*kv_stride_t + d] (same strides for v).
 *   Row b reads slot slot_ids ? slot_ids[b] : b.
 *   lens  : int32 [B] keys visible to the last query of row b (causal as above).
 * Used for cross-attention over g_cross_kv [S, L, 2, H, T_enc, D] slices and for
 * causal attention over contiguous prompt K/V. Non-causal calls with q_len >= 2
 * (a prompt's cross-attention), head_dim 64 and fp16/bf16 run every 16 queries of
 * a row against one read of its K/V, with both products on the matrix cores (every
 * 64 queries, staged in LDS, when rows carry 64 or more queries and the
 * (row, head, 64-query) workgroups cover at least three quarters of the GPU).
 * Reference: models.py:167-203, :468-479, :126-165 (contiguous past).
 */
SKV_API int skv_dense_attention(const void* q, int64_t q_stride_b, int64_t q_stride_q, int64_t q_stride_h,
                        const void* k, const void* v,
                        int64_t kv_stride_s, int64_t kv_stride_h, int64_t kv_stride_t,
                        const int32_t* slot_ids,
                        const int32_t* lens,
                        void* out, int64_t o_stride_b, int64_t o_stride_q, int64_t o_stride_h,
                        int32_t batch, int32_t q_len, int32_t num_heads, int32_t num_kv_heads,
                        int32_t head_dim, int32_t max_len, float scale, int32_t causal,
                        int32_t dtype, int32_t chunk_tokens,
                        void* workspace, int64_t workspace_bytes, void* stream);

/*
 * skv_add_layernorm — residual add + LayerNorm of a decode batch.
 *   x, y : [rows, hidden] at row strides ldx, ldy (y NULL: no add, sum unused)
 *   sum  : x + y rounded to dtype (may be x itself; NULL: not stored)
 *   norm : LayerNorm(sum) * gamma + beta, fp32 statistics with the population
 *          variance and eps, as torch.nn.LayerNorm; gamma, beta [hidden].
 *   hidden a multiple of the 16-byte vector (8 fp16/bf16, 4 fp32), at most 64*8
 *   vectors; rows 16-byte aligned.
 * Replaces the pre-LN residual step `x = x + f(x)` followed by `norm(x)` of the
 * decoder layers, speech_serving/models.py:126-208 (norm1/norm2/norm3 and the
 * final decoder norm), each pair in one launch.
 */
SKV_API int skv_add_layernorm(const void* x, int64_t ldx, const void* y, int64_t ldy,
                              const void* gamma, const void* beta, float eps,
                              void* sum, int64_t lds, void* norm, int64_t ldn,
                              int32_t rows, int32_t hidden, int32_t dtype, void* stream);

/*
 * skv_codebook_embed_sum — the frame input of a multi-codebook model.
 *   out[r*out_stride + d] = T_0[c_r0][d] + T_1[c_r1][d] + ... + T_{K-1}[c_r(K-1)][d],
 *   added left to right with each partial sum rounded to dtype, so the result has
 *   the bits of the sequential `embeds = embeds + emb_k(codes[..., k])` in that dtype.
 *   c_rk = codes[r*codes_stride + k] (int64); a code outside [0, vocab) adds a zero row.
 *   tables : HOST array of num_codebooks (1..16) device pointers, each [vocab, dim]
 *            contiguous and 16-byte aligned
 *   out    : [rows, dim] at row stride out_stride (elements); dim a multiple of the
 *            16-byte vector.
 * Replaces MultiCodebookEmbedding.forward, speech_serving/models.py:39-52 (one
 * gather per codebook and K-1 adds) with one launch.
 */
SKV_API int skv_codebook_embed_sum(const int64_t* codes, int64_t codes_stride, int32_t rows,
                                   const void* const* tables, int32_t num_codebooks, int32_t vocab,
                                   int32_t dim, void* out, int64_t out_stride, int32_t dtype, void* stream);

/*
 * skv_linear — a decode-batch projection through hipBLASLt with one plan cached per shape.
 *   y[r*ldy + j] = sum_i x[r*ldx + i] * w[j*ldw + i] (+ bias[j]) for r < m, j < n, i < k:
 *   row-major x [m, k], w [n, k] and y [m, n], fp32 accumulation, the result in dtype;
 *   bias : [n] in dtype, or NULL.
 *   The first call on a device creates its hipBLASLt handle and the first call of a shape
 *   builds its plan (host work: make them outside graph capture). Plans use algorithms that
 *   need no workspace, so a call allocates no device memory. SKV_EUNSUPPORTED: hipBLASLt has
 *   no such algorithm for the shape (the caller runs its own GEMM). Calls are serialised by
 *   a lock.
 * Replaces the nn.Linear calls of the decoder step, speech_serving/models.py:127-207 (q/k/v,
 * output, cross-attention and MLP projections) and :416, :486 (the LM head), whose torch
 * dispatch rebuilds the matmul descriptors and reruns the algorithm heuristic on every call.
 */
SKV_API int skv_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, const void* bias, void* y,
                       int64_t ldy, int32_t m, int32_t n, int32_t k, int32_t dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPEECH_KV_H_ */
