/*
 * C ABI of libmy_vllm_amd.so: gfx950 (MI355X) kernels for the ragged-batch
 * attention hot path of Nano-vLLM-v1 and its SiLU-and-mul op.
 *
 * Conventions shared by every entry point:
 *   - Buffers are raw device pointers; sizes and strides are int64 and count
 *     ELEMENTS (not bytes) unless the name says otherwise.
 *   - `dtype` is MVA_DTYPE_BF16 or MVA_DTYPE_F16 (storage type of activations
 *     and of the KV cache; all arithmetic is fp32).
 *   - `stream` is a hipStream_t (pass torch.cuda.current_stream().cuda_stream);
 *     launches are asynchronous and no entry point synchronizes the device.
 *   - Return 0 on success, a negative status otherwise; mva_last_error()
 *     returns the calling thread's last message.  Nothing throws across the ABI.
 *   - Load this library after the process's HIP runtime (torch's) is loaded,
 *     so both bind to the same runtime instance.
 */
#ifndef MY_VLLM_AMD_H_
#define MY_VLLM_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MVA_DTYPE_BF16 0
#define MVA_DTYPE_F16 1
#define MVA_DTYPE_F32 2 /* weights of mva_rms_norm / mva_fused_add_rms_norm only */

/* Message of the calling thread's most recent failed call ("" if none). */
const char* mva_last_error(void);

/* ABI revision of this header. */
int mva_abi_version(void);

/*
 * out[r, c] = silu(in[r, c]) * in[r, c + hidden] for r < rows, c < hidden.
 * `input` is a contiguous [rows, 2*hidden] buffer, `output` a contiguous
 * [rows, hidden] buffer; fp32 math, one rounding to `dtype`.
 * Replaces the reference's `nanovllm._C.forward` (csrc/silu_and_mul.cpp:24-29,
 * kernel csrc/silu_and_mul_kernel.cu:11-77), bound by
 * nanovllm/layers/cuda_ops.py:29-34; the Python side keeps its argument
 * checks and error messages (csrc/silu_and_mul.cpp:8-18).
 */
int mva_silu_and_mul(const void* input, void* output, int64_t rows, int64_t hidden, int dtype,
                     void* stream);

/*
 * slot_mapping KV-cache store.  For each token t < num_tokens whose slot
 * s = slot_mapping[t] satisfies 0 <= s < num_slots, copies row_elems elements
 * of key + t*key_row_stride to k_cache + s*row_elems and of
 * value + t*value_row_stride to v_cache + s*row_elems.  slot_mapping is int32,
 * or int64 when slot_is_int64 != 0.  row_elems = num_kv_heads * head_dim;
 * num_slots = num_pages * page_size.  Bit copy (no rounding).
 * Replaces `store_kvcache` (nanovllm/layers/attention.py:34-41, Triton kernel
 * :11-31) behind KVCacheStore (:44-101).
 */
int mva_kv_store(const void* key, int64_t key_row_stride, const void* value,
                 int64_t value_row_stride, void* k_cache, void* v_cache, int64_t num_slots,
                 const void* slot_mapping, int slot_is_int64, int64_t num_tokens, int64_t row_elems,
                 int dtype, void* stream);

/*
 * RMSNorm over rows of `hidden` elements:
 *   out[r] = T(T(x[r] * rsqrt(mean(x[r]^2) + eps)) * weight), fp32 statistics.
 * Row r is row i = r % rows_per_group of group g = r / rows_per_group, at
 * x + g*x_group_stride + i*x_row_stride (elements, unit inner stride; e.g.
 * the heads of a [tokens, heads, head_dim] view of a packed projection), and
 * likewise for out; out may equal x.  weight [hidden] has `weight_dtype`
 * MVA_DTYPE_F32 or the input dtype.
 * Replaces the reference's RMSNorm providers (nanovllm/layers/layernorm.py:
 * 31-40 native path, :65-72 rms_norm provider; FlashInfer rmsnorm,
 * nanovllm/layers/flashinfer_ops.py).
 */
int mva_rms_norm(const void* x, int64_t x_group_stride, int64_t x_row_stride, const void* weight, void* out,
                 int64_t out_group_stride, int64_t out_row_stride, int64_t rows, int64_t rows_per_group,
                 int64_t hidden, float eps, int dtype, int weight_dtype, void* stream);

/*
 * Fused residual add + RMSNorm:
 *   s = float(x) + float(residual); residual_out = T(s);
 *   out = T(T(s * rsqrt(mean(s^2) + eps)) * weight)  (statistics of the fp32 sum).
 * out may equal x and residual_out may equal residual (the in-place form of
 * the reference's forward_inplace).
 * Replaces the fused_add_rms_norm providers (nanovllm/layers/layernorm.py:
 * 42-52 native path, :74-88 forward / forward_inplace).
 */
int mva_fused_add_rms_norm(const void* x, int64_t x_row_stride, const void* residual,
                           int64_t residual_row_stride, const void* weight, void* out,
                           int64_t out_row_stride, void* residual_out, int64_t residual_out_row_stride,
                           int64_t rows, int64_t hidden, float eps, int dtype, int weight_dtype,
                           void* stream);

/*
 * Attention prologue in one launch, for num_tokens tokens:
 *   1. when q_norm_weight / k_norm_weight are given (both or neither): per-head
 *      RMSNorm of q and k over head_dim, T(T(x * rsqrt(mean(x^2) + eps)) * w);
 *   2. neox rotary embedding of q and k with cos_sin_cache [max_position,
 *      rotary_dim] fp32 (cos | sin) at positions [num_tokens] int64 (clamped to
 *      [0, max_position)), fp32 products rounded once to `dtype`;
 *   3. when k_cache is given: the slot_mapping store of the rotated k and of v
 *      (caches contiguous [pages, page_size, num_kv_heads, head_dim],
 *      num_slots = pages * page_size; slots outside [0, num_slots) skipped).
 * q / k rows: base + token*token_stride + head*head_stride (elements, unit
 * inner stride); outputs share the input strides and may alias the inputs.
 * Requires head_dim == rotary_dim == 128.
 * Replaces, as one launch, the reference's q_norm / k_norm RMSNorm, its
 * RotaryEmbedding provider (nanovllm/layers/rotary_embedding.py:18-110,
 * FlashInfer apply_rope_with_cos_sin_cache) and the KV store
 * (nanovllm/layers/attention.py:44-101), called in sequence at
 * nanovllm/models/qwen3.py:96-100 and attention.py:140-141.  With no norm
 * weights and no cache it is the RotaryEmbedding provider alone.
 */
int mva_qk_norm_rope_store(const void* q_in, void* q_out, int64_t q_token_stride, int64_t q_head_stride,
                           int num_q_heads, const void* k_in, void* k_out, int64_t k_token_stride,
                           int64_t k_head_stride, const void* v, int64_t v_token_stride, int64_t v_head_stride,
                           int num_kv_heads, const int64_t* positions, const float* cos_sin_cache,
                           int64_t max_position, int rotary_dim, const void* q_norm_weight,
                           const void* k_norm_weight, int weight_dtype, float eps, void* k_cache, void* v_cache,
                           int64_t num_slots, const void* slot_mapping, int slot_is_int64, int64_t num_tokens,
                           int head_dim, int dtype, void* stream);

/*
 * Bytes of device workspace mva_paged_decode / mva_paged_mixed need for
 * `num_part_slots` split-K partial slots (a scheduler area of piece-claim
 * counters, MIXED arrival counters and fused-store row flags, then fp32
 * partial outputs and log-sum-exps), or -1 for invalid arguments.  The
 * workspace must be zeroed once when first allocated; the kernels leave the
 * counters and flags zeroed again on return.  Launches that share a
 * workspace must not overlap.
 */
int64_t mva_decode_workspace_bytes(int64_t num_part_slots, int num_kv_heads, int group);

/* Byte offset, inside a decode workspace, of the int32 word that
 * mva_paged_decode_store sets when a new row's slot is not its sequence's
 * last position. */
#define MVA_DECODE_STORE_ERROR_OFFSET 4224

/*
 * Paged GQA decode (one query token per sequence) over an NHD page cache
 * k_cache / v_cache = [num_pages, page_size, num_kv_heads, head_dim] with
 * page_stride / token_stride element strides (head stride = head_dim).
 *   q:    query rows; q + row*q_token_stride + head*q_head_stride.
 *   block_tables [num_seqs, block_table_stride] int32 page ids; seq_lens
 *         [num_seqs] int32 context lengths (including the new token).
 *   items [num_items, 8] int32 pieces, each
 *         {seq, page_begin, page_end, chunk, n_chunks, part_base, q_row, kv_head}:
 *         pages [page_begin, page_end) of (sequence `seq`, KV head `kv_head`)
 *         (at most 128 pages), piece `chunk` of `n_chunks`; split-K partial
 *         slots part_base .. part_base + n_chunks - 1 (unused when
 *         n_chunks == 1); output row q_row.
 *   num_waves (1 .. num_items): wavefronts launched; wavefront w first runs
 *         piece w.  Its later pieces follow one of two schedules:
 *   wave_extra [num_waves + 1] int32, or NULL:
 *         piece lists: wavefront w then runs pieces wave_extra[w] ..
 *         wave_extra[w + 1] - 1 in order (num_waves <= wave_extra[w] <=
 *         wave_extra[w + 1] <= num_items); no workspace counter is touched.
 *         NULL: wavefront w runs piece num_waves + w and then claims later
 *         pieces from counters in the workspace, so pieces should be listed
 *         longest first.
 *   waves_per_group (1, 2, 4 or 8): wavefronts per workgroup; wavefronts
 *         g*waves_per_group .. (g+1)*waves_per_group - 1 share a CU.  Must be 1
 *         when wave_extra is NULL.
 *   merges [num_merges, 8] int32: one piece descriptor (chunk 0) of every
 *         (sequence, KV head) cut into n_chunks > 1 pieces; a second kernel on
 *         `stream` combines each one's partials into its output rows.
 *   num_part_slots: split-K partial slots the pieces use (part_base + chunk <
 *         num_part_slots); sizes the workspace.
 *   out:  out + row*out_token_stride + head*out_head_stride, `dtype`.
 * softmax over keys j < seq_len with scale `softmax_scale`; fp32 accumulate.
 * Requires head_dim 128, page_size 16, num_q_heads / num_kv_heads <= 16,
 * 16-byte aligned q/cache buffers and strides.
 * Replaces FlashInfer BatchDecodeWithPagedKVCacheWrapper.plan/run as used by
 * the reference's DECODE route (nanovllm/layers/attention_backend.py:826-840,
 * :995-997) and the decode half of MIXED_SPLIT (:874-889, :1020-1025).
 */
int mva_paged_decode(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                     const void* k_cache, const void* v_cache, int64_t num_pages,
                     int64_t page_stride, int64_t token_stride, const int32_t* block_tables,
                     int64_t block_table_stride, const int32_t* seq_lens, const int32_t* items,
                     int64_t num_items, int64_t num_waves, const int32_t* wave_extra,
                     int waves_per_group, const int32_t* merges,
                     int64_t num_merges, int64_t num_part_slots, void* out,
                     int64_t out_token_stride, int64_t out_head_stride, void* workspace,
                     int64_t workspace_bytes, int num_q_heads, int num_kv_heads, int head_dim,
                     int page_size, float softmax_scale, int dtype, void* stream);

/*
 * Host-side planners of mva_paged_decode's pieces (no device memory, no HIP
 * call; safe without a GPU).  Sequence first_seq + i has block_counts[i] > 0
 * pages and reads query row first_q_row + i.  Both write items [*, 8] as
 * mva_paged_decode takes them and, when `merges` is not NULL, the merge list
 * (the chunk-0 piece of every split segment, in item order), and set
 * out_counts[4] = {num_items, num_waves, num_part_slots, num_merges}.
 * Replace the host scheduling of FlashInfer's
 * BatchDecodeWithPagedKVCacheWrapper.plan, called per step by the
 * reference's build_plan (nanovllm/layers/attention_backend.py:826-840,
 * :877-889).
 *
 * Piece lists: the batch's pages, in batch order, cut into
 * G = min(num_groups, total pages) near-equal ranges (range g = pages
 * [g*T/G, (g+1)*T/G)); wavefront g*num_kv_heads + h streams KV head h of
 * range g, one piece per sequence the range touches, cut further to at most
 * max_piece_pages (1 .. 128).  wave_extra gets G*num_kv_heads + 1 entries
 * (the mva_paged_decode argument).  item_rows must be at least
 * mva_decode_plan_listed_rows(...), an upper bound on the rows written.
 */
int64_t mva_decode_plan_listed_rows(int64_t num_seqs, int64_t total_pages, int num_kv_heads, int num_groups,
                                    int max_piece_pages);
int mva_decode_plan_listed(const int64_t* block_counts, int64_t num_seqs, int64_t first_seq,
                           int64_t first_q_row, int num_kv_heads, int num_groups, int max_piece_pages,
                           int32_t* items, int64_t item_rows, int32_t* wave_extra, int64_t wave_extra_len,
                           int32_t* merges, int64_t merge_rows, int64_t* out_counts);

/*
 * Claims: every (sequence, KV head) segment of L pages cut into
 * ceil(L / P) near-equal pieces, P = clamp(ceil(total segment pages /
 * max(1, num_waves * max(1, pieces_per_wave))), min_piece_pages,
 * max_piece_pages); pieces longest first, then sequence-major with the KV
 * head fastest.  num_waves of the result = min(num_waves, num_items) (at
 * least 1).  item_rows must be at least mva_decode_plan_claims_rows(...).
 */
int64_t mva_decode_plan_claims_rows(int64_t num_seqs, int64_t total_pages, int num_kv_heads,
                                    int min_piece_pages);
int mva_decode_plan_claims(const int64_t* block_counts, int64_t num_seqs, int64_t first_seq,
                           int64_t first_q_row, int num_kv_heads, int64_t num_waves, double pieces_per_wave,
                           int min_piece_pages, int max_piece_pages, int32_t* items, int64_t item_rows,
                           int32_t* merges, int64_t merge_rows, int64_t* out_counts);

/*
 * mva_paged_decode with the slot_mapping KV store of the same step folded in
 * (piece lists only: wave_extra is required).  Before reading any page, the
 * wavefront whose piece holds the last page of a sequence writes the new
 * K and V rows of that piece's KV head, k_new / v_new
 * [num_new_tokens, num_kv_heads, 128] (row q_row of the piece, any 4-byte
 * aligned strides), to cache slot slot_mapping[q_row] (int32, or int64 when
 * slot_is_int64; -1 skips) when that slot is the sequence's last position
 * (last page, row (seq_len - 1) % 16), as the model runner builds it; then
 * the output and the caches equal mva_kv_store followed by
 * mva_paged_decode.  Every other row t < num_new_tokens with a slot >= 0 (a
 * slot elsewhere, which another wavefront may be reading, or a row no piece
 * names) is written by the merge kernel that always follows on the stream,
 * after the attention read the cache: the caches always equal
 * mva_kv_store's, and the launch sets the int32 word at byte
 * MVA_DECODE_STORE_ERROR_OFFSET of the workspace to 1 (only the caller
 * clears it).  num_new_tokens * num_kv_heads <= 65536.  Other arguments as
 * mva_paged_decode.
 * Replaces the KVCacheStore call (nanovllm/layers/attention.py:140-141)
 * together with the decode run that follows it (attention_backend.py:995-997).
 */
int mva_paged_decode_store(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                           const void* k_cache, const void* v_cache, int64_t num_pages,
                           int64_t page_stride, int64_t token_stride, const int32_t* block_tables,
                           int64_t block_table_stride, const int32_t* seq_lens, const int32_t* items,
                           int64_t num_items, int64_t num_waves, const int32_t* wave_extra,
                           int waves_per_group, const int32_t* merges, int64_t num_merges,
                           int64_t num_part_slots, void* out, int64_t out_token_stride,
                           int64_t out_head_stride, void* workspace, int64_t workspace_bytes,
                           const void* k_new, int64_t k_token_stride, int64_t k_head_stride,
                           const void* v_new, int64_t v_token_stride, int64_t v_head_stride,
                           const void* slot_mapping, int slot_is_int64, int64_t num_new_tokens,
                           int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                           float softmax_scale, int dtype, void* stream);

/*
 * Fixed-shape variant of mva_paged_decode for capture in a HIP graph: every
 * argument that changes from one decode step to the next lives in device
 * memory at a fixed address, so one captured launch serves every step whose
 * plan fits the capacities.
 *   counts [3] int32 (device): {num_items, num_waves, num_merges} of this
 *         step, each clamped to its capacity; wavefronts and merge
 *         wavefronts past them exit at once.
 *   items  [item_capacity, 8], wave_extra [wave_capacity + 1], merges
 *         [merge_capacity, 8]: the piece-list schedule of mva_paged_decode
 *         (wave_extra is required; no claims).
 *   wave_capacity (<= item_capacity) wavefronts and merge_capacity x
 *         (num_q_heads / num_kv_heads) merge wavefronts are launched.
 *   num_part_slots: split-K partial slots the largest fitting plan uses
 *         (sizes the workspace).
 * Other arguments as mva_paged_decode; block_tables, seq_lens, q, out and
 * the workspace must also stay at fixed addresses while a graph holds the
 * launch.  No counter in the workspace is used.
 * Serves the reference's full-decode CUDA-graph hooks
 * (nanovllm/layers/attention_backend.py:242-275, FlashInfer version
 * :1028-1225; capture and replay in nanovllm/engine/model_runner.py:631-742).
 */
int mva_paged_decode_graph(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                           const void* k_cache, const void* v_cache, int64_t num_pages,
                           int64_t page_stride, int64_t token_stride, const int32_t* block_tables,
                           int64_t block_table_stride, const int32_t* seq_lens, const int32_t* counts,
                           const int32_t* items, int64_t item_capacity, const int32_t* wave_extra,
                           int64_t wave_capacity, int waves_per_group, const int32_t* merges,
                           int64_t merge_capacity, int64_t num_part_slots, void* out,
                           int64_t out_token_stride, int64_t out_head_stride, void* workspace,
                           int64_t workspace_bytes, int num_q_heads, int num_kv_heads, int head_dim,
                           int page_size, float softmax_scale, int dtype, void* stream);

/* Bytes of the static device scratch mva_paged_decode_noalloc uses per GPU. */
#define MVA_DECODE_STATIC_SCRATCH_BYTES (64LL << 20)

/*
 * mva_paged_decode for callers that cannot allocate device memory: code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * No counterpart in the reference (its FlashInfer wrappers own workspaces the
 * caller allocated).  The decode workspace lives in a static device array of
 * MVA_DECODE_STATIC_SCRATCH_BYTES that each GPU holds until the process ends;
 * the call allocates and frees nothing.  Arguments as mva_paged_decode,
 * without workspace / workspace_bytes.
 *   - Plans whose workspace (mva_decode_workspace_bytes(num_part_slots,
 *     num_kv_heads, num_q_heads / num_kv_heads)) exceeds the scratch are
 *     rejected with an error before anything is launched.
 *   - The first call on a device looks up that device's scratch address and
 *     clears its scheduler counters with one small kernel on `stream`; make it
 *     outside graph capture.  The kernels leave the counters cleared again.
 *   - Every call on one GPU shares that GPU's scratch: calls that overlap on
 *     one GPU (other streams, other threads) race.  Calls in stream order,
 *     one after another, are safe.
 */
int mva_paged_decode_noalloc(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                             const void* k_cache, const void* v_cache, int64_t num_pages,
                             int64_t page_stride, int64_t token_stride, const int32_t* block_tables,
                             int64_t block_table_stride, const int32_t* seq_lens, const int32_t* items,
                             int64_t num_items, int64_t num_waves, const int32_t* wave_extra,
                             int waves_per_group, const int32_t* merges, int64_t num_merges,
                             int64_t num_part_slots, void* out, int64_t out_token_stride,
                             int64_t out_head_stride, int num_q_heads, int num_kv_heads, int head_dim,
                             int page_size, float softmax_scale, int dtype, void* stream);

/* Query tokens per prefill tile of mva_paged_mixed for a GQA ratio
 * (128 / ratio: 128 query rows), or -1 for invalid head counts.
 * mva_paged_prefill's tiles hold twice as many (256 query rows). */
int mva_prefill_tile_tokens(int num_q_heads, int num_kv_heads);

/* Bytes of the prefill workspace (the device-built tile list) for at most
 * max_tiles query tiles, or -1 for an invalid count. */
int64_t mva_prefill_workspace_bytes(int64_t max_tiles);

/* Byte offset, inside a prefill workspace, of the int32 word where
 * mva_paged_prefill writes how many of the batch's tiles exceeded max_tiles
 * (and were not run). */
#define MVA_PREFILL_DROPPED_TILES_OFFSET 4

/*
 * Ragged causal chunked prefill over prefix-cached pages (same cache and q/out
 * conventions as mva_paged_decode).  Sequence s < num_seqs has query rows
 * query_start_loc[s] .. query_start_loc[s+1] - 1 (q_s rows) and seq_lens[s]
 * keys including them; query i sees keys j <= seq_lens[s] - q_s + i.  The new
 * tokens' K/V are read from the cache (store them first).
 * The work list is built on the device from query_start_loc and seq_lens
 * (nothing is read back to the host): one query tile per
 * 2 * mva_prefill_tile_tokens() tokens x all query heads of a KV head (256
 * query rows), longest context first, written into `workspace`
 * (mva_prefill_workspace_bytes(max_tiles) bytes, 16-byte aligned).
 * max_tiles must bound the tile count, e.g. num_prefill_tokens / tile_tokens
 * + num_seqs with tile_tokens = 2 * mva_prefill_tile_tokens(); tiles beyond
 * it are not run (their output rows keep what `out` held), and the launch
 * writes their number to the int32 word at byte
 * MVA_PREFILL_DROPPED_TILES_OFFSET of the workspace (0 when max_tiles bounds
 * the batch).  A sequence with no queries, or more queries than keys, is
 * skipped.  A persistent grid of 512-thread workgroups, one per CU, then
 * streams the tiles.  Launches that share a workspace must not overlap.
 * Replaces FlashInfer BatchPrefillWithPagedKVCacheWrapper.plan/run on the
 * reference's PREFILL route (nanovllm/layers/attention_backend.py:810-825,
 * :992-994) and the prefill half of MIXED_SPLIT (:858-873, :1015-1019).
 */
int mva_paged_prefill(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                      const void* k_cache, const void* v_cache, int64_t num_pages,
                      int64_t page_stride, int64_t token_stride, const int32_t* block_tables,
                      int64_t block_table_stride, const int32_t* seq_lens,
                      const int32_t* query_start_loc, int64_t num_seqs, int64_t max_tiles,
                      void* workspace, int64_t workspace_bytes, void* out, int64_t out_token_stride,
                      int64_t out_head_stride, int num_q_heads, int num_kv_heads, int head_dim,
                      int page_size, float softmax_scale, int dtype, void* stream);

/*
 * mva_paged_prefill in two parts, for a step whose layers share one batch:
 * mva_paged_prefill_plan builds the tile list of the batch into `workspace`
 * once, and mva_paged_prefill_run then streams it for each layer's q, caches
 * and out (arguments as mva_paged_prefill).  A run needs the plan that
 * mva_paged_prefill_plan (or mva_paged_prefill) wrote into the same workspace
 * for the same block_tables, seq_lens, query_start_loc, num_seqs, max_tiles
 * and head counts, with none of them changed since; each run leaves the plan
 * ready for the next.  Both are ordered by `stream` and must not overlap
 * other launches on the workspace.  The dropped-tile word is written by the
 * plan.  Mirror the reference's once-per-step FlashInfer
 * BatchPrefillWithPagedKVCacheWrapper.plan (nanovllm/layers/attention_backend.py:810-825,
 * from build_plan :769-894) and its per-layer run (:992-994).
 */
int mva_paged_prefill_plan(const int32_t* block_tables, int64_t block_table_stride, int64_t num_pages,
                           const int32_t* seq_lens, const int32_t* query_start_loc, int64_t num_seqs,
                           int64_t max_tiles, void* workspace, int64_t workspace_bytes, int num_q_heads,
                           int num_kv_heads, void* stream);
int mva_paged_prefill_run(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                          const void* k_cache, const void* v_cache, int64_t num_pages,
                          int64_t page_stride, int64_t token_stride, const int32_t* block_tables,
                          int64_t block_table_stride, const int32_t* seq_lens,
                          const int32_t* query_start_loc, int64_t num_seqs, int64_t max_tiles,
                          void* workspace, int64_t workspace_bytes, void* out, int64_t out_token_stride,
                          int64_t out_head_stride, int num_q_heads, int num_kv_heads, int head_dim,
                          int page_size, float softmax_scale, int dtype, void* stream);

/*
 * MIXED batch in one launch: prefill tiles write the rows of the leading
 * num_prefill_seqs (<= 1024) sequences and decode pieces (as
 * mva_paged_decode, claim schedule) write the trailing decode rows of the
 * same `out` buffer.  The prefill tiles (mva_prefill_tile_tokens() tokens
 * x the query heads of a KV head: 128 query rows) are derived on the device
 * from query_start_loc and seq_lens, longest context first, and run by a
 * persistent pool of prefill workgroups; max_prefill_tiles bounds their
 * number (num_prefill_tokens / tile_tokens + num_prefill_seqs) and only
 * sizes the pool.  The workspace (mva_decode_workspace_bytes) also holds the
 * pool's claim counters and the split-K arrival counters, which the launch
 * leaves at zero.  Split decode segments are merged inside the launch: the
 * last piece of a segment to finish combines the partials, so no merge list
 * or merge kernel is involved.  At most 64 KV heads when prefill sequences
 * are present.
 * Replaces FlashInfer BatchAttention.plan/run on the reference's MIXED_UNIFIED
 * route (nanovllm/layers/attention_backend.py:841-857, :998-1009).
 */
int mva_paged_mixed(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                    const void* k_cache, const void* v_cache, int64_t num_pages,
                    int64_t page_stride, int64_t token_stride, const int32_t* block_tables,
                    int64_t block_table_stride, const int32_t* seq_lens,
                    const int32_t* query_start_loc, int64_t num_prefill_seqs, int64_t max_prefill_tiles,
                    const int32_t* decode_items, int64_t num_decode_items, int64_t num_decode_waves,
                    int64_t num_part_slots, void* out, int64_t out_token_stride, int64_t out_head_stride,
                    void* workspace, int64_t workspace_bytes, int num_q_heads, int num_kv_heads,
                    int head_dim, int page_size, float softmax_scale, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MY_VLLM_AMD_H_ */
