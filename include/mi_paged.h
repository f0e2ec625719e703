/*
 * mi_paged.h -- C ABI of the MI355X paged-KV data plane (libmi_paged.so).
 *
 * Every entry point takes plain device pointers, element strides and sizes,
 * and a HIP stream handle passed as `void*` (0 = the default stream).  No entry
 * point allocates or frees device memory: the caller owns pools, metadata,
 * outputs and workspaces.  Work is enqueued asynchronously on `stream`; nothing
 * here synchronises the device.
 *
 * Return value: MI_OK (0) on success, a negative MI_ERR_* code otherwise.  The
 * message for the last failure on the calling thread is `mi_last_error()`.
 *
 * Pool layout (identical to the reference's PagedKVCachePool tensors, which the
 * reference's tests index directly): one key pool and one value pool per layer,
 * each `[num_blocks, block_size, num_kv_heads, head_dim]`, row-major.  A slot is
 * `block_id * block_size + offset`, i.e. the row number of the pool viewed as
 * `[num_blocks * block_size, num_kv_heads, head_dim]`.  Block 0 is the null
 * block used to right-pad block tables.
 *
 * Index metadata is int64, as the reference packs it on the host.
 *
 * Out-of-range indices, one rule for every entry point (the kernels never fault on them and never
 * touch memory outside the pools): a block id outside [0, num_blocks) *read* through a block
 * table or id list (attention histories, gather, pack) reads the null block 0; a *write* to a slot
 * outside [0, num_blocks * block_size) or to a block id outside [0, num_blocks) (scatter, the
 * decode appends, unpack) is skipped.  The reference's tensor indexing raises instead on ids >=
 * num_blocks; the Python layer can do the same before each launch (data_plane.set_index_checks).
 */
#ifndef MI_PAGED_H
#define MI_PAGED_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI_PAGED_ABI_VERSION 4  /* 2: mi_paged_decode_workspace_bytes takes num_kv_heads;
                                   3: mi_paged_decode_attention_exact takes a workspace;
                                   4: mi_mixed_paged_attention[_exact] take ragged chunk rows */

#define MI_OK 0
#define MI_ERR_INVALID_ARGUMENT (-1) /* null pointer, negative size, bad stride  */
#define MI_ERR_UNSUPPORTED (-2)      /* shape or alignment the kernels do not cover */
#define MI_ERR_WORKSPACE (-3)        /* workspace missing or too small            */
#define MI_ERR_DEVICE (-4)           /* HIP launch / runtime error                */

/* ABI version of the loaded library (MI_PAGED_ABI_VERSION it was built with). */
int32_t mi_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* mi_last_error(void);

/*
 * Kernel 1 -- reshape-and-cache scatter of new K/V rows into pool slots.
 *
 * Replaces PagedKVCachePool.write_prefill
 *   (src/mini_infra/worker/paged_kv_cache.py:74-95): per layer
 *   `pool.view(-1, H, D).index_copy_(0, slot_mapping, src[token_rows, :, token_positions, :])`
 * and the decode-time append in Qwen3Attention._apply_paged_kv_pool
 *   (src/mini_infra/model/qwen3.py:282-283): `pool.view(-1, H, D).index_copy_(0, slot_mapping, key.squeeze(2))`.
 *
 * For token i and every layer l:
 *   key_pools[l][slot_mapping[i], h, :] = key_src[l][token_rows[i], h, token_positions[i], :]   (h < num_kv_heads)
 * and the same for values.  Source element (r, h, p, d) is at
 *   r * row_stride + h * head_stride + p * pos_stride + d     (element strides, d contiguous).
 * token_rows == NULL means row i; token_positions == NULL means position 0 (the
 * decode form, source `[B, H, 1, D]`).  The three index arrays share the
 * element stride `index_stride` (the reference's decode slot_mapping is a
 * column of a packed [B, 4 + max_blocks] tensor).
 *
 * Slots must be unique (as in the reference).  A token whose slot is outside
 * [0, num_slots), row outside [0, num_src_rows) or position outside
 * [0, num_src_positions) is skipped: nothing is read or written for it.  The copy
 * is bit-exact for any element type of `elem_bytes` bytes (2 for bf16/fp16, 4 for fp32).
 */
int32_t mi_reshape_and_cache(const void* const* key_src, const void* const* value_src,
                             int64_t key_row_stride, int64_t key_head_stride, int64_t key_pos_stride,
                             int64_t value_row_stride, int64_t value_head_stride, int64_t value_pos_stride,
                             const int64_t* token_rows, const int64_t* token_positions,
                             const int64_t* slot_mapping, int64_t index_stride, int64_t num_tokens,
                             int64_t num_src_rows, int64_t num_src_positions,
                             void* const* key_pools, void* const* value_pools, int32_t num_layers,
                             int64_t num_slots, int32_t num_kv_heads, int32_t head_dim, int32_t elem_bytes,
                             void* stream);

/*
 * Kernel 2 -- block-table gather of whole physical blocks.
 *
 * Replaces PagedKVCachePool.gather_blocks (src/mini_infra/worker/paged_kv_cache.py:54-72),
 *   `key_pool[block_ids].view(B, nb * block_size, H, D)` per layer (the reference then
 *   returns `.transpose(1, 2)` views of it),
 * and the history gather of Qwen3Attention._apply_paged_kv_pool (src/mini_infra/model/qwen3.py:288-291).
 *
 * For every layer l, row b < batch and j < num_gathered_blocks:
 *   key_out[l][b, j, :] = key_pools[l][block_ids[b * block_id_stride + j], :]
 * where one block is `block_bytes` bytes (block_size * num_kv_heads * head_dim * elem_bytes).
 * Outputs are contiguous `[batch, num_gathered_blocks, block_bytes]`.  Whole blocks are
 * copied, including null block 0 and stale tails of recycled blocks, so the result is
 * bit-identical to the reference's advanced-index gather.  A block id outside
 * [0, num_blocks) reads the null block 0.
 */
int32_t mi_gather_blocks(const void* const* key_pools, const void* const* value_pools, int64_t num_blocks,
                         const int64_t* block_ids, int64_t block_id_stride, int32_t batch,
                         int32_t num_gathered_blocks, void* const* key_out, void* const* value_out,
                         int32_t num_layers, int64_t block_bytes, void* stream);

/*
 * Workspace for mi_paged_decode_attention: bytes of float scratch for the partial
 * results of sequences cut between two of the launch's equal block ranges -- two slots
 * per range per query head, (128 + 2) floats each.  It depends on the device's CU count and,
 * for small launches, on batch * max_blocks; never on the context lengths.  0 when
 * batch or max_blocks is 0.  No initialisation needed.
 */
int64_t mi_paged_decode_workspace_bytes(int32_t batch, int32_t max_blocks, int32_t num_heads,
                                        int32_t num_kv_heads, int32_t head_dim, int32_t block_size);

/*
 * Kernel 3 -- paged GQA decode attention (one query token per sequence).
 *
 * Replaces the decode branch of Qwen3Attention: the pool gather of
 * _apply_paged_kv_pool (src/mini_infra/model/qwen3.py:285-292), the additive
 * context-length bias of Qwen3Model._build_paged_inputs (:513-528) and
 * _attend with _repeat_key_value (:219-255, :147-156).
 *
 * For sequence b and query head h (kv head g = h / (num_heads / num_kv_heads),
 * the reference's repeat_interleave mapping), with n = min(context_lens[b], max_blocks * block_size):
 *   s_t = bf16(bf16(q[b,h,:] . K_t) * scale),  K_t = key_pool[block_tables[b, t / bs], t % bs, g, :]
 *   out[b, h*D : (h+1)*D] = bf16( sum_{t<n} softmax(s)_t * V_t )
 * Softmax and accumulation run in fp32.  Positions t >= n are excluded (the
 * reference adds finfo(bf16).min there, which underflows to exactly zero weight).
 * n <= 0 writes a zero output row.
 *
 * query: `[batch, num_heads, head_dim]` bf16 with row/head element strides, head_dim contiguous.
 * out:   `[batch, num_heads * head_dim]` bf16 with row element stride.
 * block_tables: `[batch, max_blocks]` int64 with row element stride; ids outside
 *   [0, num_blocks) read the null block 0 instead.  context_lens: int64 with element stride.
 * workspace: at least mi_paged_decode_workspace_bytes(...) bytes (may be null when
 *   max_blocks is 0).  The launch's blocks are cut into equal ranges, one per workgroup
 *   (and head group); sequences cut between ranges leave partials that a second, small
 *   launch merges (it also writes the zero rows).  Launches of at most one (sequence, KV
 *   head) per CU with max_blocks <= 512 run a single per-sequence kernel instead, which
 *   leaves the workspace untouched; the environment variable MI_DECODE_PATH=stream or =seq
 *   forces either kernel where both apply.
 * Specialised for head_dim 128, block_size 16, num_kv_heads in {1, 2, 4, 8} and GQA groups
 * num_heads / num_kv_heads in {1, 2, 4, 5, 8} (query head h reads KV head h / group, as
 * _repeat_key_value does, src/mini_infra/model/qwen3.py:147-156); other shapes return
 * MI_ERR_UNSUPPORTED.
 */
int32_t mi_paged_decode_attention(void* out, int64_t out_row_stride, const void* query,
                                  int64_t query_row_stride, int64_t query_head_stride,
                                  const void* key_pool, const void* value_pool, int64_t num_blocks,
                                  const int64_t* block_tables, int64_t block_table_stride, int32_t max_blocks,
                                  const int64_t* context_lens, int64_t context_lens_stride, int32_t batch,
                                  int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                  float scale, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * mi_paged_decode_attention_fused -- mi_qk_norm_rope's decode form (q/k RMSNorm + RoPE of the new
 * tokens, K/V rows into their slots: qwen3.py:182-217 with _apply_paged_kv_pool's append :282-283)
 * followed by mi_paged_decode_attention (qwen3.py:219-292), with the same results bit for bit.
 * Where the per-sequence kernel serves the launch (batch * num_kv_heads <= CUs, max_blocks <= 512)
 * it is one launch whose workgroups rotate their own q heads and append their own K/V head;
 * otherwise it runs the two entry points, rotating q into q_scratch.
 * q: [batch] rows of num_heads * 128 (q_row_stride), k / v: rows of num_kv_heads * 128;
 * cos / sin: [batch, 128]; q_scratch: [batch, num_heads, 128] bf16 (always required).
 * The remaining arguments are those of mi_qk_norm_rope and mi_paged_decode_attention.  Each row's
 * slot must lie in one of its own blocks (decode packing puts it at position context - 1): in the
 * one-launch form only the row's own workgroups are ordered after its append.
 */
int32_t mi_paged_decode_attention_fused(void* out, int64_t out_row_stride, const void* q, int64_t q_row_stride,
                                        const void* k, int64_t k_row_stride, const void* v, int64_t v_row_stride,
                                        const void* q_weight, const void* k_weight, const void* cos,
                                        const void* sin, float eps, const int64_t* slot_mapping,
                                        int64_t slot_stride, void* key_pool, void* value_pool, int64_t num_blocks,
                                        const int64_t* block_tables, int64_t block_table_stride,
                                        int32_t max_blocks, const int64_t* context_lens,
                                        int64_t context_lens_stride, int32_t batch, int32_t num_heads,
                                        int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                                        void* q_scratch, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * mi_paged_decode_attention_noalloc -- mi_paged_decode_attention without a workspace argument: a
 * variant that allocates nothing and takes no caller scratch.  It has no counterpart in the
 * reference; it is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).
 *
 * Same arguments, results and errors as mi_paged_decode_attention, bit for bit.  The partials of
 * sequences cut between block ranges go to a fixed device array of the library,
 * MI_PAGED_NOALLOC_SCRATCH_BYTES bytes per GPU, held from the first call on a device until the
 * process ends.  A launch that needs more (mi_paged_decode_workspace_bytes above it; 4.3 MB at
 * 16 query / 8 KV heads on 256 CUs) returns MI_ERR_WORKSPACE before any launch, copy or scratch
 * lookup; the size check itself only queries the current device and its CU count (hipGetDevice,
 * and hipDeviceGetAttribute once per device).  The array
 * needs no clearing, but it is shared by every call on one GPU: calls that overlap on one GPU
 * (two streams, or two threads) race on it and must be serialised by the caller.
 */
#define MI_PAGED_NOALLOC_SCRATCH_BYTES (8ll << 20)
int32_t mi_paged_decode_attention_noalloc(void* out, int64_t out_row_stride, const void* query,
                                          int64_t query_row_stride, int64_t query_head_stride,
                                          const void* key_pool, const void* value_pool, int64_t num_blocks,
                                          const int64_t* block_tables, int64_t block_table_stride,
                                          int32_t max_blocks, const int64_t* context_lens,
                                          int64_t context_lens_stride, int32_t batch, int32_t num_heads,
                                          int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                                          void* stream);

/*
 * Kernel 4 -- chunked-prefill attention on MFMA with the history read from the pool.
 *
 * Replaces, for one layer of PagedRunner.run_prefill_chunk_step
 * (src/mini_infra/worker/paged_runner.py:32-102): the history gather
 * PagedKVCachePool.gather_blocks (src/mini_infra/worker/paged_kv_cache.py:54-72), the
 * history/chunk concat of Qwen3Attention.forward (src/mini_infra/model/qwen3.py:325-330), the
 * visibility mask (paged_runner.py:83-89 with the causal mask of qwen3.py:477-484) and
 * Qwen3Attention._attend (qwen3.py:219-255).
 *
 * Row b of the batch is a chunk of padded_len positions whose last chunk_lens[b] are real
 * tokens (left padding).  With pad = padded_len - chunk_lens[b] and
 * nh = min(start_lens[b], 16 * max_history_blocks), query position i >= pad sees
 *   - history slot k < nh: key_pool/value_pool row (history_blocks[b, k / 16] * 16 + k % 16, g)
 *   - chunk position j with pad <= j <= i: key/value[b, g, j, :]
 * for kv head g = h / 2 of query head h; scores as in kernel 3 (bf16 product, bf16 scale),
 * fp32 softmax and accumulation, bf16 output.  Rows i < pad get zeros.
 *
 * out:   [batch, padded_len, num_heads * head_dim] bf16 (row / token element strides).
 * query: [batch, num_heads, padded_len, head_dim]; key / value: [batch, num_kv_heads,
 *   padded_len, head_dim] (row / head / token element strides, head_dim contiguous).
 * history_blocks: [batch, max_history_blocks] int64, row stride history_stride; ids outside
 *   [0, num_blocks) read block 0.  start_lens / chunk_lens: int64 with element stride lens_stride.
 * Specialised for head_dim 128, block_size 16, num_kv_heads in {1, 2, 4, 8} and num_heads any
 * multiple of num_kv_heads (query head h reads KV head h / group); strides multiples of 8 elements, key / value token strides below 2^24 elements,
 * and 16-byte aligned tensors.
 */
int32_t mi_chunked_prefill_attention(void* out, int64_t out_row_stride, int64_t out_tok_stride, const void* query,
                                     int64_t query_row_stride, int64_t query_head_stride, int64_t query_tok_stride,
                                     const void* key, int64_t key_row_stride, int64_t key_head_stride,
                                     int64_t key_tok_stride, const void* value, int64_t value_row_stride,
                                     int64_t value_head_stride, int64_t value_tok_stride, const void* key_pool,
                                     const void* value_pool, int64_t num_blocks, const int64_t* history_blocks,
                                     int64_t history_stride, int32_t max_history_blocks, const int64_t* start_lens,
                                     const int64_t* chunk_lens, int64_t lens_stride, int32_t batch,
                                     int32_t padded_len, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                     int32_t block_size, float scale, void* stream);

/*
 * Reference numerics -- attention at the reference's rounding points with exactly accumulated
 * sums, for callers that need results independent of reduction order (a model forward that must
 * reproduce its reference bit for bit).  Replaces the same reference code as kernels 3 and 4
 * (src/mini_infra/model/qwen3.py:219-255 with the paged gather :257-292 and the chunk mask
 * :438-485).  Per query row and visible key t (same visibility as kernels 3 and 4):
 *   s_t = bf16(bf16(fp32(sum_d q_d k_td)) * scale)     (exact dot product)
 *   m = max_t s_t,  e_t = fp32(exp(fp32(s_t - m))),  l = fp32(sum_t e_t)   (exp in fp64, exact sum)
 *   p_t = bf16(fp32(e_t / l)),  out_d = bf16(fp32(sum_t p_t v_td))          (exact sum)
 * i.e. the reference's bf16 scores, fp32 softmax cast to bf16 before P V, and bf16 output, with
 * every sum exact instead of an fp32 sum in an implementation-defined order.  fp64 arithmetic,
 * scores held in LDS: meant for latency-bound launches (decode steps, prompt-sized prefill).
 *
 * mi_paged_decode_attention_exact -- decode.  With q_weight == NULL, `q` holds the rotated
 * queries ([batch, num_heads, 128], row / head strides) and k, v, k_weight, cos, sin, eps and
 * slot_mapping are ignored: the arguments and outputs of mi_paged_decode_attention.  With
 * q_weight != NULL the prologue of mi_paged_decode_attention_fused runs first
 * (q / k RMSNorm + RoPE of the raw projection rows q / k, K/V rows into their slots; the q head
 * stride is then 128), bit-identical to mi_qk_norm_rope; as in the mixed form's decode rows,
 * context 0 marks a padding row, which appends nothing.  Out-of-range table ids read block 0.
 * Any context length (contexts longer than the LDS cache recompute their scores per pass).
 * workspace (optional, 256-byte aligned): with at least mi_paged_decode_exact_workspace_bytes(...)
 * bytes, a batch too small to fill the GPU with one workgroup per (sequence, KV head) runs split
 * over each sequence's blocks (three launches: scores, then the softmax statistics and P V per
 * split, then the merge), with the same results bit for bit.  NULL, or a batch that needs no
 * split (the size query returns 0), runs one launch; a non-NULL workspace smaller than the split
 * needs is MI_ERR_WORKSPACE.
 *
 * mi_chunked_prefill_attention_exact -- chunked prefill: the arguments and layout of
 * mi_chunked_prefill_attention.  Padding rows get zeros.
 *
 * Specialised for head_dim 128, block_size 16 and 1, 2, 4, 5 or 8 query heads per KV head.
 */
int32_t mi_paged_decode_attention_exact(void* out, int64_t out_row_stride, const void* q, int64_t q_row_stride,
                                        int64_t q_head_stride, const void* k, int64_t k_row_stride, const void* v,
                                        int64_t v_row_stride, const void* q_weight, const void* k_weight,
                                        const void* cos, const void* sin, float eps, const int64_t* slot_mapping,
                                        int64_t slot_stride, void* key_pool, void* value_pool, int64_t num_blocks,
                                        const int64_t* block_tables, int64_t block_table_stride, int32_t max_blocks,
                                        const int64_t* context_lens, int64_t context_lens_stride, int32_t batch,
                                        int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                        int32_t block_size, float scale, void* workspace, int64_t workspace_bytes,
                                        void* stream);
/* Workspace bytes of mi_paged_decode_attention_exact's split form for this launch shape; 0 when
 * the launch runs unsplit.  No reference counterpart (the reference has no workspace). */
int64_t mi_paged_decode_exact_workspace_bytes(int32_t batch, int32_t max_blocks, int32_t num_heads,
                                              int32_t num_kv_heads);
int32_t mi_chunked_prefill_attention_exact(void* out, int64_t out_row_stride, int64_t out_tok_stride,
                                           const void* query, int64_t query_row_stride, int64_t query_head_stride,
                                           int64_t query_tok_stride, const void* key, int64_t key_row_stride,
                                           int64_t key_head_stride, int64_t key_tok_stride, const void* value,
                                           int64_t value_row_stride, int64_t value_head_stride,
                                           int64_t value_tok_stride, const void* key_pool, const void* value_pool,
                                           int64_t num_blocks, const int64_t* history_blocks, int64_t history_stride,
                                           int32_t max_history_blocks, const int64_t* start_lens,
                                           const int64_t* chunk_lens, int64_t lens_stride, int32_t batch,
                                           int32_t padded_len, int32_t num_heads, int32_t num_kv_heads,
                                           int32_t head_dim, int32_t block_size, float scale, void* stream);

/*
 * Kernel 4, mixed form -- the attention of a mixed chunk + decode step in one launch: the varlen
 * attention the reference plans for mixing prefill chunks and decode tokens in one forward
 * (src/mini_infra/core/scheduler.py:310-311, src/mini_infra/core/types.py:108), over the same
 * rows the model's two paths would serve: chunk rows as mi_chunked_prefill_attention and decode
 * rows as mi_paged_decode_attention plus the K/V append of mi_reshape_and_cache's decode form
 * (reference qwen3.py:219-330, the append at qwen3.py:282-283).
 *
 * A flattened token batch of T = C + D rows, token-major ([T, H, 128] query, [T, H_kv, 128]
 * key / value with token and head strides; out [T, H * 128] with a token stride):
 *   tokens [0, C): P chunk rows with start_lens / chunk_lens / history_blocks as in
 *     mi_chunked_prefill_attention, each seen as a left-padded chunk of width L (L at least every
 *     chunk_lens[b]: the attention's tiling).  With chunk_first NULL, C = P L and row b is tokens
 *     [b L, b L + L) (padding included; padding rows get zero output).  With chunk_first (ragged
 *     rows, device [P]), C = chunk_tokens and row b's chunk_lens[b] real tokens are tokens
 *     chunk_first[b] .. chunk_first[b] + chunk_lens[b] - 1 (first clamped to [0, C - chunk_lens[b]]):
 *     no padding is stored or read, so C can be the sum of the lengths, and each token of [0, C)
 *     that no row covers (a padded step's tail) gets a zero row (a small launch before the
 *     attention's);
 *   tokens [C, T): D decode rows, one token each, context_lens[b] tokens including it: the
 *     first context_lens[b] - 1 are read from the pool through block_tables[b], the last is the
 *     row's own key / value, which the launch also appends to pool slot slot_mapping[b] (a slot
 *     outside the pool is skipped; context 0 marks a padding row: zero output, no append).
 * Chunk rows give the bits of mi_chunked_prefill_attention.  Decode rows are served by the same
 * chunk kernel (a 1-token chunk), within the same tolerance of the reference chain as kernel 3.
 * Either part may be empty (P = 0 or L = 0, D = 0).
 *
 * mi_mixed_paged_attention_exact -- the same with the reference numerics of
 * mi_chunked_prefill_attention_exact (decode rows as one-token chunks there too, their sums exact);
 * decode rows then give the bits of mi_paged_decode_attention_exact.
 */
int32_t mi_mixed_paged_attention(void* out, int64_t out_tok_stride, const void* query, int64_t query_tok_stride,
                                 int64_t query_head_stride, const void* key, int64_t key_tok_stride,
                                 int64_t key_head_stride, const void* value, int64_t value_tok_stride,
                                 int64_t value_head_stride, void* key_pool, void* value_pool, int64_t num_blocks,
                                 int32_t prefill_rows, int32_t prefill_width, int64_t chunk_tokens,
                                 const int64_t* chunk_first, const int64_t* history_blocks,
                                 int64_t history_stride, int32_t max_history_blocks, const int64_t* start_lens,
                                 const int64_t* chunk_lens, int64_t lens_stride, int32_t decode_rows,
                                 const int64_t* block_tables, int64_t block_table_stride, int32_t max_blocks,
                                 const int64_t* context_lens, int64_t context_lens_stride,
                                 const int64_t* slot_mapping, int64_t slot_stride, int32_t num_heads,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                                 void* stream);
int32_t mi_mixed_paged_attention_exact(void* out, int64_t out_tok_stride, const void* query,
                                       int64_t query_tok_stride, int64_t query_head_stride, const void* key,
                                       int64_t key_tok_stride, int64_t key_head_stride, const void* value,
                                       int64_t value_tok_stride, int64_t value_head_stride, void* key_pool,
                                       void* value_pool, int64_t num_blocks, int32_t prefill_rows,
                                       int32_t prefill_width, int64_t chunk_tokens, const int64_t* chunk_first,
                                       const int64_t* history_blocks, int64_t history_stride,
                                       int32_t max_history_blocks, const int64_t* start_lens,
                                       const int64_t* chunk_lens, int64_t lens_stride, int32_t decode_rows,
                                       const int64_t* block_tables, int64_t block_table_stride, int32_t max_blocks,
                                       const int64_t* context_lens, int64_t context_lens_stride,
                                       const int64_t* slot_mapping, int64_t slot_stride, int32_t num_heads,
                                       int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                                       void* stream);

/*
 * Fused layer ops: the elementwise chains around attention in a Qwen3 decoder layer, one
 * launch each, with the reference's bf16 rounding points.  All tensors are bf16, rows of
 * contiguous elements, 16-byte aligned.
 *
 * mi_rms_norm -- RMSNorm (src/mini_infra/model/qwen3.py:55-78), optionally after the residual
 * add of Qwen3DecoderLayer.forward (:368-400):
 *   h = residual ? bf16(x + residual) : x;  residual_out = h (when residual is given)
 *   out = bf16(weight * bf16(h * r)),  r = fp32(1 / sqrt(fp32(fp32(sum(h^2) / hidden) + eps)))
 * with the sum of squares exact and the square root and division in fp64 (the reference's fp32
 * mean, rsqrt and product, independent of the order of the sum).
 * x / residual / residual_out / out: [rows, hidden] contiguous; hidden a multiple of 8, <= 4096.
 */
int32_t mi_rms_norm(void* out, const void* x, const void* residual, void* residual_out, const void* weight,
                    int64_t rows, int32_t hidden, float eps, void* stream);

/*
 * mi_qk_norm_rope -- per-head q/k RMSNorm and RoPE of Qwen3Attention._project_qkv
 * (src/mini_infra/model/qwen3.py:182-217, 111-145):
 *   q_out[t, h] = rope(bf16(q_weight * bf16(norm(q[t, h]))), cos[t], sin[t])
 *   rope(x) = bf16(bf16(x * cos) + bf16(rotate_half(x) * sin)),  rotate_half(x) = cat(-x[64:], x[:64])
 * and the same for k with k_weight; v is copied unchanged.
 * Rows: with k_out / v_out ([T, Hkv, 128]) each token's k and v rows go there.
 * Slots: with slot_mapping they also go (or, without k_out / v_out, only go) straight to pool slot
 * slot_mapping[t * slot_stride] of key_pool / value_pool ([num_slots, Hkv, 128]) -- the
 * reshape-and-cache append of _apply_paged_kv_pool (:282-283) for a decode step, or
 * PagedKVCachePool.write_prefill (paged_kv_cache.py:74-95) for a prefill chunk whose block table
 * already covers it (paged_runner.py:49); out-of-range slots (-1 for left padding) are skipped.
 * q / k / v: token rows with element strides q_stride / k_stride / v_stride; cos / sin: [T, 128].
 * q_out: [T, Hq, 128].  head_dim must be 128.
 */
int32_t mi_qk_norm_rope(void* q_out, void* k_out, void* v_out, const void* q, int64_t q_stride, const void* k,
                        int64_t k_stride, const void* v, int64_t v_stride, const void* q_weight,
                        const void* k_weight, const void* cos, const void* sin, int64_t num_tokens,
                        int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float eps,
                        const int64_t* slot_mapping, int64_t slot_stride, void* key_pool, void* value_pool,
                        int64_t num_slots, void* stream);

/*
 * mi_silu_mul -- the SwiGLU product of Qwen3MLP.forward (src/mini_infra/model/qwen3.py:347-355):
 *   out = bf16(bf16(silu(gate)) * up),  silu(g) = g / (1 + exp(-g)) in fp32.
 * gate / up / out: [rows, cols] with row element strides; cols and strides multiples of 8.
 */
int32_t mi_silu_mul(void* out, int64_t out_stride, const void* gate, int64_t gate_stride, const void* up,
                    int64_t up_stride, int64_t rows, int32_t cols, void* stream);

/*
 * mi_argmax_rows -- greedy sampling, the torch.argmax of greedy_sample
 * (src/mini_infra/worker/sampler.py:9-23): out[r] = index of the largest of logits[r, 0:cols].
 * logits: bf16 rows with element stride row_stride >= cols; out: int64 [rows].
 * Ties go to the smallest index, -0 equals +0, a NaN is larger than every number (the first NaN
 * wins), as torch.argmax.  One workgroup per row; no workspace.
 */
int32_t mi_argmax_rows(int64_t* out, const void* logits, int64_t rows, int32_t cols, int64_t row_stride,
                       void* stream);

/*
 * KV block records -- the wire / swap format of whole physical blocks, for the "swap" preemption
 * mode the reference plans (src/mini_infra/core/types.py:110-114, core/scheduler.py:312-313:
 * a victim's physical KV blocks go to a CPU host swap pool over PCIe and come back on resume).
 * One record is one block of every layer, contiguous:
 *   record[layer][0 = K, 1 = V][block_size * H * D elements]   record_bytes = 2 * num_layers * block_bytes
 * where block_bytes is one layer's K (or V) block, as laid out in the pool of
 * src/mini_infra/worker/paged_kv_cache.py:23-52.  Records of one call are contiguous.
 *
 * mi_pack_blocks:   records[i] = block block_ids[i] of every layer (ids out of [0, num_blocks)
 *                   read the null block 0).
 * mi_unpack_blocks: block block_ids[i] of every layer = records[i] (out-of-range ids skipped;
 *                   ids must be unique).
 * key_pools / value_pools: num_layers device pointers, each num_blocks * block_bytes.
 * block_ids: device int64 [num_records].  Bit-exact copies; no workspace.
 */
int32_t mi_pack_blocks(void* records, const void* const* key_pools, const void* const* value_pools,
                       int64_t num_blocks, const int64_t* block_ids, int64_t num_records, int32_t num_layers,
                       int64_t block_bytes, void* stream);
int32_t mi_unpack_blocks(void* const* key_pools, void* const* value_pools, int64_t num_blocks,
                         const void* records, const int64_t* block_ids, int64_t num_records, int32_t num_layers,
                         int64_t block_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MI_PAGED_H */
