/*
 * nsd_attn.h -- C ABI of the MI355X (gfx950) verify/decode paged-attention
 * path of NebulaSD's swiftLLM backend.
 *
 * All tensors are caller-owned device buffers passed as raw pointers with
 * int64 sizes.  Every entry point is stream-ordered on the caller's
 * hipStream_t (passed as void*), never synchronises the host, never
 * allocates device memory, and returns an int status (NSD_OK == 0).  On a
 * nonzero status nsd_last_error() returns a thread-local message.
 *
 * Fixed layouts (identical to the reference, byte for byte):
 *   k_cache, v_cache : fp16 [num_blocks, num_layers, num_kv_heads, block_size, head_dim]
 *                      (swiftLLM/swiftllm/worker/model.py:152-166)
 *   block_table      : int32 [bt_rows, bt_stride] (row = seq_id)
 *                      (swiftLLM/swiftllm/worker/block_manager.py:112-117)
 *   q, o             : fp16 [n_rows, num_q_heads, head_dim], contiguous
 *   k, v (new rows)  : fp16 [n_rows, num_kv_heads, head_dim], contiguous
 * Supported: head_dim == 128, block_size == 16, num_q_heads % num_kv_heads == 0.
 *
 * `status` arguments are optional (may be NULL) device int32 words: a kernel
 * that meets an out-of-range block id, seq_id or position skips that access
 * and ORs a flag into *status (NSD_STATUS_*), so bad metadata never faults.
 */
#ifndef NSD_ATTN_H
#define NSD_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NSD_OK 0
#define NSD_ERR_INVALID 1      /* bad argument (null pointer, size, range) */
#define NSD_ERR_UNSUPPORTED 2  /* shape outside the supported set */
#define NSD_ERR_HIP 3          /* HIP runtime error */
#define NSD_ERR_WORKSPACE 4    /* workspace / plan buffer too small */

#define NSD_STATUS_BAD_BLOCK 1     /* block id outside [0, num_blocks) */
#define NSD_STATUS_BAD_SEQ 2       /* seq_id outside [0, bt_rows) or position outside the row */
#define NSD_STATUS_BAD_POSITION 4  /* RoPE position outside the cos/sin table */

#define NSD_COPY_D2H 0            /* device cache -> host plane (write-back / swap-out) */
#define NSD_COPY_H2D 1            /* host plane -> device cache (restore / swap-in) */
#define NSD_COPY_ENGINE_DMA 0     /* hipMemcpyAsync per run (system DMA engines) */
#define NSD_COPY_ENGINE_KERNEL 1  /* one gfx950 copy launch over every run */

#define NSD_PLAN_HEADER_WORDS 24

/* Library version (major*10000 + minor*100 + patch). */
int nsd_version(void);

/* Thread-local message of the last failing call on this thread. */
const char* nsd_last_error(void);

/*
 * QK-RMSNorm building block.  Replaces rmsnorm_inplace
 * (swiftLLM/swiftllm/worker/kernels/rmsnorm.py:26-37, kernel :5-24):
 * per row of `hidden` fp16 values, y = fp16(x * 1/sqrt(mean(x^2)+eps) * w),
 * computed in fp32, in place.
 */
int nsd_rmsnorm_inplace(void* x, const void* w, int64_t n_rows, int64_t hidden,
                        float eps, void* stream);

/*
 * Rotate-half RoPE, in place on q [n_tokens, Hq, d] and k [n_tokens, Hkv, d]
 * from per-token tables cos/sin [n_tokens, d/2] fp16.  Replaces
 * rotary_embedding_inplace (swiftLLM/swiftllm/worker/kernels/rotary_emb.py:44-58,
 * kernel :7-42).  Arithmetic in fp32, one rounding to fp16.
 */
int nsd_rotary_embedding_inplace(void* q, void* k, const void* cos_table,
                                 const void* sin_table, int64_t n_tokens,
                                 int num_q_heads, int num_kv_heads, int head_dim,
                                 void* stream);

/*
 * Decode/verify KV store.  Replaces the decoding half of store_kvcache
 * (swiftLLM/swiftllm/worker/kernels/kvcache_mgmt.py:81-122, kernel :50-79):
 * row r copies k[r], v[r] ([Hkv, d]) to slot (seq_lens[r]-1) % block_size of
 * block block_table[seq_ids[r], (seq_lens[r]-1) / block_size] at `layer`.
 * seq_ids / seq_lens are device int32 [n_rows].  Bit-exact copy.
 */
int nsd_store_kvcache(const void* k, const void* v, void* k_cache, void* v_cache,
                      const int32_t* block_table, int64_t bt_rows, int64_t bt_stride,
                      const int32_t* seq_ids, const int32_t* seq_lens, int64_t n_rows,
                      int64_t num_blocks, int num_layers, int layer, int num_kv_heads,
                      int head_dim, int block_size, int32_t* status, void* stream);

/*
 * Prefill KV store.  Replaces the prefill half of store_kvcache
 * (swiftLLM/swiftllm/worker/kernels/kvcache_mgmt.py:10-48): sequence s copies
 * its tokens k/v[start_locs[s] + i] to position i (0 <= i < prefill_lens[s])
 * of block_table[seq_ids[s]].  All index arrays are device int32 [n_seqs].
 */
int nsd_store_kvcache_prefill(const void* k, const void* v, void* k_cache, void* v_cache,
                              const int32_t* block_table, int64_t bt_rows, int64_t bt_stride,
                              const int32_t* seq_ids, const int32_t* start_locs,
                              const int32_t* prefill_lens, int64_t n_seqs,
                              int64_t max_prefill_len, int64_t num_blocks, int num_layers,
                              int layer, int num_kv_heads, int head_dim, int block_size,
                              int32_t* status, void* stream);

/*
 * Fused attention prologue of one decode/verify layer call, one launch.
 * Replaces the sequence rmsnorm_inplace(q) -> rmsnorm_inplace(k) ->
 * rotary_embedding_inplace -> store_kvcache of
 * swiftLLM/swiftllm/worker/layers/transformer_layer.py:114-145:
 *   q[r,h] = rope(fp16(rmsnorm(q[r,h]) * q_norm_w))    (in place)
 *   k[r,h] = rope(fp16(rmsnorm(k[r,h]) * k_norm_w))    (in place)
 *   k_cache/v_cache slot of (seq_ids[r], seq_lens[r]-1) <- k[r], v[r]
 * RoPE position = seq_lens[r]-1 (model.py:343-354), looked up in the full
 * cos/sin caches [n_positions, d/2] fp16 (model.py:242-252).
 * q_norm_w / k_norm_w may be NULL to skip the norm (models without QK-norm).
 */
int nsd_qk_norm_rope_store(void* q, void* k, const void* v, const void* q_norm_w,
                           const void* k_norm_w, float eps, const void* cos_cache,
                           const void* sin_cache, int64_t n_positions, void* k_cache,
                           void* v_cache, const int32_t* block_table, int64_t bt_rows,
                           int64_t bt_stride, const int32_t* seq_ids, const int32_t* seq_lens,
                           int64_t n_rows, int64_t num_blocks, int num_layers, int layer,
                           int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                           int32_t* status, void* stream);

/*
 * nsd_qk_norm_rope_store_strided: the same prologue for q/k/v rows that are
 * slices of one fused projection output [rows, (Hq + 2*Hkv) * d]: row i of
 * q, k and v starts q_row_stride, k_row_stride, v_row_stride elements after
 * row i-1 (even, and at least the row's heads x head_dim).  The normalised,
 * rotated q goes to q_out [rows, Hq, d] contiguous (what nsd_paged_attention
 * reads); k is rotated in place; K and V go to the cache as above.  One
 * q/k/v GEMM then replaces the reference's three (transformer_layer.py:107-109).
 */
int nsd_qk_norm_rope_store_strided(const void* q, int64_t q_row_stride, void* q_out, void* k,
                                   int64_t k_row_stride, const void* v, int64_t v_row_stride,
                                   const void* q_norm_w, const void* k_norm_w, float eps,
                                   const void* cos_cache, const void* sin_cache, int64_t n_positions,
                                   void* k_cache, void* v_cache, const int32_t* block_table,
                                   int64_t bt_rows, int64_t bt_stride, const int32_t* seq_ids,
                                   const int32_t* seq_lens, int64_t n_rows, int64_t num_blocks,
                                   int num_layers, int layer, int num_q_heads, int num_kv_heads,
                                   int head_dim, int block_size, int32_t* status, void* stream);

/*
 * Attention work plan (host side, no HIP calls).  The reference picks a
 * split size per forward (swiftLLM/swiftllm/worker/model.py:365-384) and
 * launches one program per (row, q-head, split) (kernels/paged_attn.py:182-211).
 * Here the plan is built once per forward from the host copies of the
 * rows' seq_ids / seq_lens (the lists model.forward already holds,
 * model.py:304-341) and reused by every layer:
 *   - consecutive rows with equal seq_id and seq_len increasing by one form
 *     a verify group (rows of speculative.py:75-89); each group is attended
 *     once per KV head with GQA-group x q_len query rows packed together;
 *     max_group_rows = 1 keeps every row its own group;
 *   - every (group, kv head) segment is cut into near-equal pieces of
 *     consecutive 16-token blocks (at most 256 each), n_workers pieces in
 *     all: each segment starts with the fewest pieces it needs and every
 *     further piece goes to the segment whose pieces are the longest (while
 *     pieces stay >= 4 blocks and <= 128 per segment), so no cut into as
 *     many pieces has a shorter longest piece;
 *   - one workgroup streams one piece; pieces are dealt longest first to
 *     the eight XCDs (workgroup i runs on XCD i % 8) with near-equal blocks
 *     and counts per XCD, each XCD's list longest first, except that with
 *     static_slots set, a list that puts two workgroups on some of the
 *     XCD's C = static_slots / 16 CUs (positions j and j + C of the list
 *     share a CU when the launch starts them together) pairs a long piece
 *     with a short one on each such CU, so the CUs' totals are near-equal;
 *   - a segment cut into several pieces gets partials (normalised O in
 *     fp16, log2-sum-exp in fp32), merged in slot order by a second launch
 *     of the same call.
 * nsd_attn_plan_bound gives the plan size in int32 words for plans of
 * n_workers pieces; when a plan needs more (segments longer than 256
 * blocks need several pieces each) and does not fit `plan_capacity`,
 * nsd_attn_plan_build returns NSD_ERR_WORKSPACE and sets *plan_words to the
 * size needed, so the caller can retry.
 * nsd_attn_plan_build validates (1 <= seq_len <= bt_stride*block_size,
 * 0 <= seq_id < bt_rows), writes the plan into `plan` (capacity
 * `plan_capacity` words), and returns its size and the workspace bytes
 * nsd_paged_attention needs.
 */
int64_t nsd_attn_plan_bound(int64_t n_rows, int num_kv_heads, int n_workers);
int nsd_attn_plan_build(const int32_t* seq_ids, const int32_t* seq_lens, int64_t n_rows,
                        int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                        int64_t bt_rows, int64_t bt_stride, int n_workers,
                        int max_group_rows, int32_t* plan, int64_t plan_capacity,
                        int64_t* plan_words, int64_t* workspace_bytes);
/*
 * nsd_attn_plan_build_claimed: nsd_attn_plan_build, with the workgroup
 * slots of the device given (static_slots, e.g. nsd_attn_num_workers):
 * when the plan has more pieces than slots, only the static_slots longest
 * are bound to workgroups (and XCDs) ahead of the launch; the rest are
 * claimed at run time, longest first, by the workgroups that start as
 * slots free up, so a faster XCD takes more of them.  static_slots = 0
 * binds every piece (nsd_attn_plan_build).  The workspace then holds a
 * claim counter that must be zero before the first call (every call leaves
 * it zero): allocate it zero-filled.
 */
int nsd_attn_plan_build_claimed(const int32_t* seq_ids, const int32_t* seq_lens, int64_t n_rows,
                                int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                int64_t bt_rows, int64_t bt_stride, int n_workers, int static_slots,
                                int max_group_rows, int32_t* plan, int64_t plan_capacity,
                                int64_t* plan_words, int64_t* workspace_bytes);

/*
 * Number of workers (workgroups) that fill the current device for a plan
 * whose groups hold at most `max_rows` query rows per KV head (occupancy x
 * compute units).  Needs a GPU.
 */
int nsd_attn_num_workers(int max_rows, int* n_workers);

/*
 * Paged verify/decode attention for one layer.  Replaces paged_attention
 * (swiftLLM/swiftllm/worker/kernels/paged_attn.py:152-222, kernels :9-149):
 * row r, q-head qh attends tokens [0, seq_len[r]) of block_table[seq_id[r]]
 * in kv head qh / (Hq/Hkv) with scores q.k * softmax_scale; o[r, qh] is the
 * softmax-weighted sum of V (fp16 out, fp32 math).  If lse != NULL it also
 * writes ln(sum exp(score)) as fp32 [n_rows, Hq].
 * plan_host / plan_dev: the same plan words on the host and on the device.
 * workspace: device buffer of at least the bytes reported by the plan (a
 * 256-byte claim counter, then the partials of the segments cut into
 * pieces), 16-byte aligned.  The counter must be zero before the first call
 * with a plan that has claimed pieces (nsd_attn_plan_build_claimed); every
 * call leaves it zero, so allocate the workspace zero-filled once.  Calls
 * that share a workspace must be ordered on one stream (never concurrent).
 * bt_rows / bt_stride: the block table's shape; the plan must have been
 * built for this row stride and at most this many rows.
 * Results are bit-reproducible: identical inputs give identical o and lse.
 */
int nsd_paged_attention(const void* q, void* o, float* lse, const void* k_cache,
                        const void* v_cache, int64_t num_blocks, int num_layers, int layer,
                        int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                        const int32_t* block_table, int64_t bt_rows, int64_t bt_stride,
                        const int32_t* plan_host, const int32_t* plan_dev,
                        void* workspace, int64_t workspace_bytes, float softmax_scale,
                        int32_t* status, void* stream);

/*
 * nsd_paged_attention_fused: the layer's prologue and its attention in one
 * launch.  Replaces the sequence nsd_qk_norm_rope_store (transformer_layer.py
 * :114-145: QK-RMSNorm, RoPE at position seq_len - 1, K/V into the cache
 * slot) then nsd_paged_attention, with identical results: o, lse and the
 * cache rows written are bit for bit those of the two calls (q itself is
 * not written back).  The rows' q, k and v are either fp16 rows (q, k, v
 * with row strides in elements; each 16-byte aligned, each stride a
 * multiple of 8) or, when partials != NULL, the fused q/k/v projection's
 * fp32 split partials [splits][rows][(Hq + 2 Hkv) * 128] (nsd_linear_partials), summed
 * in split order and rounded to fp16 first.  q_norm_w / k_norm_w: [128]
 * fp16 (both or neither), cos/sin: [n_positions, 64] fp16, all 16-byte
 * aligned.  The rows are the plan's (the plan carries each group's sequence
 * and positions).  Each workgroup builds its query rows itself, and the
 * workgroup that streams a cache block holding a new row writes that row
 * before it loads the block.  So the plan must keep every sequence's rows
 * in one verify group: a plan that splits a sequence over several groups
 * returns NSD_ERR_UNSUPPORTED (run the two calls instead), and positions
 * past the RoPE tables return NSD_ERR_INVALID, before any launch.  The
 * other arguments, the workspace and the status word are nsd_paged_attention's.
 */
int nsd_paged_attention_fused(const void* q, int64_t q_row_stride, const void* k, int64_t k_row_stride,
                              const void* v, int64_t v_row_stride, const float* partials, int splits,
                              const void* q_norm_w, const void* k_norm_w, float eps,
                              const void* cos_cache, const void* sin_cache, int64_t n_positions, void* o,
                              float* lse, void* k_cache, void* v_cache, int64_t num_blocks, int num_layers,
                              int layer, int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                              const int32_t* block_table, int64_t bt_rows, int64_t bt_stride,
                              const int32_t* plan_host, const int32_t* plan_dev, void* workspace,
                              int64_t workspace_bytes, float softmax_scale, int32_t* status, void* stream);

/*
 * nsd_paged_attention_noalloc: nsd_paged_attention without a workspace
 * argument, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  It
 * has no counterpart in the reference, whose wrapper allocates its partials
 * per call (swiftLLM/swiftllm/worker/kernels/paged_attn.py:170-180).
 * The partials live in a static device array of NSD_NOALLOC_SCRATCH_BYTES
 * per GPU (held until the process ends); a plan that needs more partial
 * bytes than it holds is rejected with NSD_ERR_WORKSPACE.  The call
 * allocates nothing.  Every call on one GPU shares the array: calls that
 * overlap on one GPU (two streams, two threads) race and must not overlap.
 * Issue them on one stream per GPU, or order the streams (an event between
 * one call's stream and the next call's) -- the library does not check.
 * Same arguments, results and errors as nsd_paged_attention.
 */
#define NSD_NOALLOC_SCRATCH_BYTES (16ll << 20)
int nsd_paged_attention_noalloc(const void* q, void* o, float* lse, const void* k_cache,
                                const void* v_cache, int64_t num_blocks, int num_layers, int layer,
                                int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                const int32_t* block_table, int64_t bt_rows,
                                int64_t bt_stride, const int32_t* plan_host,
                                const int32_t* plan_dev, float softmax_scale, int32_t* status,
                                void* stream);

/*
 * Prefill (prompt) attention, causal within each prompt of a packed batch.
 * Replaces flash_attn_varlen_func
 * (swiftLLM/swiftllm/worker/layers/transformer_layer.py:7-32, called at
 * :151-164 with cu_seqlens_q == cu_seqlens_k and causal=True) and the Triton
 * prefill_attention (swiftLLM/swiftllm/worker/kernels/prefill_attn.py:10-140):
 * prompt s holds tokens [cu_seqlens[s], cu_seqlens[s+1]) of q [T, Hq, d],
 * k and v [T, Hkv, d]; its position i, q-head qh attends positions 0..i in
 * kv head qh / (Hq/Hkv) with scores q.k * softmax_scale, and o [T, Hq, d]
 * gets the softmax-weighted sum of V (fp16 out, fp32 math).  If lse != NULL
 * it also writes ln(sum exp(score)) as fp32 [T, Hq].
 * cu_seqlens: device int32 [n_seqs + 1], non-decreasing; a prompt's end past
 * total_tokens is cut there (the reference's last prompt ends at the
 * forward's token count and is cut by slicing q[:num_prefill_tokens],
 * model.py:412-415).  max_seqlen bounds every prompt's length: a longer
 * prompt, a negative start or a decreasing pair sets NSD_STATUS_BAD_SEQ and
 * is not (fully) computed.  Hq/Hkv must divide 128.
 * seq_order (optional, device int32 [n_seqs]): the prompts longest first (a
 * permutation of 0..n_seqs-1; any order is correct, this one balances the
 * shader engines); NULL visits them in order.  An entry outside
 * [0, n_seqs) sets NSD_STATUS_BAD_SEQ.
 */
int nsd_prefill_attention(const void* q, const void* k, const void* v, void* o, float* lse,
                          const int32_t* cu_seqlens, const int32_t* seq_order, int n_seqs,
                          int max_seqlen,
                          int64_t total_tokens, int num_q_heads, int num_kv_heads, int head_dim,
                          float softmax_scale, int32_t* status, void* stream);

/*
 * Block-table metadata (the writes that produce the attention path's index
 * input).  block_table: device int32 [bt_rows, bt_stride]; num_alloc: device
 * int32 [bt_rows] (swiftLLM's num_seq_allocated_blocks); is_block_free:
 * device bool/uint8 [num_blocks].  Out-of-range rows, counts or block ids
 * are skipped and flagged in *status (NSD_STATUS_BAD_SEQ / _BAD_BLOCK).
 *
 * nsd_write_block_ranges: row rows[i] gets begins[i] + 0..counts[i]-1 in its
 * first counts[i] entries (and num_alloc[rows[i]] = counts[i] when num_alloc
 * is not NULL).  Replaces the bank metadata writer of
 * nebulasd/src/nebulasd/workers/dma_process.py:95-125 (host index/value
 * arrays, two H2D copies, index_copy_) and the per-request fill of
 * swiftLLM/swiftllm/worker/block_manager.py:685-691.  rows/begins/counts:
 * device int32 [n_ranges].
 */
int nsd_write_block_ranges(int32_t* block_table, int64_t bt_rows, int64_t bt_stride,
                           const int32_t* rows, const int32_t* begins, const int32_t* counts,
                           int64_t n_ranges, int32_t* num_alloc, int32_t* status, void* stream);

/*
 * set_block_table_and_num_seq_alloc_blocks
 * (swiftLLM/swiftllm/worker/kernels/block_mgmt.py:5-45): for batch entry i
 * with seq s, block_table[s][num_alloc[s] + j] = candidate_blocks[c_i + j]
 * for j < block_needed[i], where c_i is the sum of block_needed[0..i-1];
 * then num_alloc[s] += block_needed[i].  seq_ids must be distinct (as in the
 * reference, whose programs would race otherwise).
 */
int nsd_set_block_table(int32_t* num_alloc, int32_t* block_table, int64_t bt_rows,
                        int64_t bt_stride, const int32_t* candidate_blocks, int64_t n_candidates,
                        const int32_t* seq_ids, const int32_t* block_needed, int64_t batch,
                        int32_t* status, void* stream);

/*
 * unset_block_table_and_num_seq_alloc_blocks (block_mgmt.py:48-80): marks
 * block_table[s][0 .. num_alloc[s]) free in is_block_free and sets
 * num_alloc[s] = 0 for every s in seq_ids.
 */
int nsd_unset_block_table(int32_t* num_alloc, const int32_t* block_table, int64_t bt_rows,
                          int64_t bt_stride, const int32_t* seq_ids, int64_t batch,
                          uint8_t* is_block_free, int64_t num_blocks, int32_t* status,
                          void* stream);

/*
 * gather_allocated_blocks_and_unset (block_mgmt.py:83-127): as
 * nsd_unset_block_table, and the freed ids of seq_ids[0], seq_ids[1], ... are
 * written back to back into `gathered` (capacity entries; the reference
 * sizes it with the sum of num_alloc[seq_ids]).  batch <= 4096.
 */
int nsd_gather_allocated_blocks_and_unset(int32_t* num_alloc, const int32_t* block_table,
                                          int64_t bt_rows, int64_t bt_stride,
                                          const int32_t* seq_ids, int64_t batch,
                                          uint8_t* is_block_free, int64_t num_blocks,
                                          int32_t* gathered, int64_t gathered_capacity,
                                          int32_t* status, void* stream);

/*
 * HostKV block-range copies: byte images of KV-cache blocks between the
 * device caches k_cache/v_cache (gpu_blocks blocks of block_bytes each,
 * block-major) and two host planes host_k/host_v (host_blocks blocks each).
 *
 * nsd_copy_block_ranges: one copy plan of the HostKV DMA backend
 * (nebulasd/src/nebulasd/kv/cuda_transfer.py:78-108).  Region i moves
 * block_count[i] blocks starting at device block gpu_begin_block[i] and
 * host block host_begin_block[i] (the reference's
 * extent.offset_blocks + host_begin_block), K plane and V plane, in
 * `direction`.  Region arrays are HOST int64 [n_regions].  Every range is
 * checked before anything is enqueued ("copy exceeds GPU KV cache",
 * "copy exceeds HostKV plane", "negative copy range": NSD_ERR_INVALID).
 * Zero-count regions are skipped; regions that continue the previous one on
 * both sides merge into one run.  engine NSD_COPY_ENGINE_DMA keeps the
 * plan's order (a later region wins where destinations overlap);
 * NSD_COPY_ENGINE_KERNEL needs pinned host planes, 16-byte alignment and
 * disjoint destinations (NSD_ERR_INVALID / NSD_ERR_UNSUPPORTED otherwise).
 * Asynchronous on `stream`; the host planes must stay alive until it ends.
 */
int nsd_copy_block_ranges(void* k_cache, void* v_cache, int64_t gpu_blocks, void* host_k,
                          void* host_v, int64_t host_blocks, int64_t block_bytes,
                          const int64_t* gpu_begin_block, const int64_t* host_begin_block,
                          const int64_t* block_count, int64_t n_regions, int direction,
                          int engine, void* stream);

/*
 * nsd_swap_blocks: swiftLLM's swap_blocks (swiftLLM/csrc/src/block_swapping.cpp:22-85).
 * source_block_ids[i] is copied to target_block_ids[i] (HOST int64 [n]);
 * is_swap_in != 0 copies swap space -> device cache, else device cache ->
 * swap space; K and V both.  Runs of consecutive ids on both sides are one
 * copy, as in the reference.  Ids are range-checked (the reference does
 * not check them); engines as for nsd_copy_block_ranges.
 */
int nsd_swap_blocks(const int64_t* source_block_ids, const int64_t* target_block_ids, int64_t n,
                    int is_swap_in, void* k_cache, void* v_cache, int64_t gpu_blocks,
                    void* k_swap, void* v_swap, int64_t swap_blocks, int64_t block_bytes,
                    int engine, void* stream);

/*
 * The rest of the layer around the attention path (swiftLLM's element-wise
 * kernels between the GEMMs, and the post-layer argmax).  fp16 data, fp32
 * arithmetic, in place where the reference is in place.
 *
 * nsd_fused_add_rmsnorm_inplace: fused_add_rmsnorm_inplace
 * (swiftLLM/swiftllm/worker/kernels/rmsnorm.py:74-89, kernel :39-72): per row,
 * residual = x + residual (one fp16 rounding), then
 * x = fp16(residual * 1/sqrt(mean(residual^2) + eps) * weight) in fp32.
 * hidden a multiple of 8 and <= 8192; pointers 16-byte aligned.
 */
int nsd_fused_add_rmsnorm_inplace(void* x, void* residual, const void* weight, int64_t n_rows,
                                  int64_t hidden, float eps, void* stream);

/*
 * nsd_silu_and_mul_inplace: silu_and_mul_inplace
 * (swiftLLM/swiftllm/worker/kernels/silu_and_mul.py:25-34, kernel :5-23): x is
 * [n_tokens, 2 * inter_dim]; x[t, j] = x[t, j] * fp16(g / (1 + exp(-g))) with
 * g = x[t, inter_dim + j] in fp32, for j < inter_dim (the product rounded once
 * to fp16).  inter_dim a multiple of 8; x 16-byte aligned.
 */
int nsd_silu_and_mul_inplace(void* x, int64_t n_tokens, int64_t inter_dim, void* stream);

/*
 * nsd_up_gate_silu_and_mul: the layer's up/gate projection followed by
 * silu_and_mul (swiftLLM/swiftllm/worker/layers/transformer_layer.py:199-200:
 * `up_gate_proj = linear(o, up_gate_proj)`, then `silu_and_mul_inplace`)
 * in one pass over the weight, without the [n_rows, 2 * inter] product:
 * y[r][j] = fp16(up * fp16(g / (1 + exp(-g)))) with up = fp16(x[r] . W[j])
 * and g = fp16(x[r] . W[inter + j]) (fp32 sums), W = up_gate [2 * inter,
 * hidden] row-major (up rows, then gate rows), x [n_rows, hidden], y
 * [n_rows, inter], fp16.  hidden a multiple of 128, inter a multiple of 16,
 * pointers 16-byte aligned.  Rows are processed in passes of 128, each
 * reading W once: meant for decode and verify batches (a library GEMM is
 * faster at prefill sizes).
 */
int nsd_up_gate_silu_and_mul(const void* x, const void* up_gate, void* y, int64_t n_rows,
                             int64_t hidden, int64_t inter, void* stream);

/*
 * Split-k projection GEMM for decode/verify batches: the layer's q/k/v, O
 * and down projections (swiftLLM/swiftllm/worker/layers/transformer_layer.py:
 * 107-109, 187, 201, each `linear(x, W)` = F.linear, kernels/linear.py:3-12)
 * for n_rows <= 128.  partials [splits][n_rows][n_out] fp32 receives, per
 * split s, sum over k in split s's range of x[r][k] * W[j][k] (x [n_rows,
 * n_in], W [n_out, n_in] fp16 row-major); the projection is the sum of the
 * splits in split order rounded once to fp16, which nsd_sum_partials,
 * nsd_fused_add_rmsnorm_partials and nsd_qk_norm_rope_store_partials compute
 * where they read it.  nsd_linear_splits gives the split count (1..8) the
 * current device uses for a shape, to size `partials`.  n_out a multiple of
 * 16, n_in a multiple of 128, pointers 16-byte aligned.
 */
int nsd_linear_splits(int64_t n_rows, int64_t n_out, int64_t n_in, int* splits);
int nsd_linear_partials(const void* x, const void* w, float* partials, int64_t n_rows, int64_t n_out,
                        int64_t n_in, void* stream);

/*
 * nsd_sum_partials: y [n_rows, n_out] fp16 = fp16(sum over s < splits of
 * partials[s]) (split order): the projection nsd_linear_partials computed.
 */
int nsd_sum_partials(const float* partials, int splits, void* y, int64_t n_rows, int64_t n_out,
                     void* stream);

/*
 * nsd_fused_add_rmsnorm_partials: nsd_fused_add_rmsnorm_inplace whose x is a
 * projection given as split partials (the linear before fused_add_rmsnorm_inplace
 * in transformer_layer.py:187-192 and, across layers, :201 then :98-103):
 * residual += fp16(sum of the splits), out = the normalised residual.
 */
int nsd_fused_add_rmsnorm_partials(const float* partials, int splits, void* out, void* residual,
                                   const void* weight, int64_t n_rows, int64_t hidden, float eps,
                                   void* stream);

/*
 * nsd_qk_norm_rope_store_partials: nsd_qk_norm_rope_store_strided over the
 * fused q/k/v projection given as split partials [splits][n_rows][(Hq +
 * 2*Hkv) * d] (transformer_layer.py:107-145): q normalised and rotated into
 * q_out [n_rows, Hq, d], K and V written to the cache slots of the rows.
 */
int nsd_qk_norm_rope_store_partials(const float* partials, int splits, void* q_out, const void* q_norm_w,
                                    const void* k_norm_w, float eps, const void* cos_cache,
                                    const void* sin_cache, int64_t n_positions, void* k_cache,
                                    void* v_cache, const int32_t* block_table, int64_t bt_rows,
                                    int64_t bt_stride, const int32_t* seq_ids, const int32_t* seq_lens,
                                    int64_t n_rows, int64_t num_blocks, int num_layers, int layer,
                                    int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                    int32_t* status, void* stream);

/*
 * nsd_lm_head_argmax: the post-layer's logits and argmax
 * (swiftLLM/swiftllm/worker/layers/post_layer.py:70-71,
 * `argmax(linear(last_input, lm_head), dim=1)`) without the logits tensor:
 * tokens[r] = the first v maximising fp16(sum_h x[r][h] * lm_head[v][h])
 * (fp32 sums; a NaN logit counts as the maximum, -0 equals +0, as in
 * torch.argmax).  x [n_rows, hidden] and lm_head [vocab, hidden] fp16
 * row-major; hidden a multiple of 128.  keys: device uint64 [n_rows] that
 * must be zero on entry; the call leaves it zero.  tokens: device int64
 * [n_rows].  Calls that share `keys` must not overlap.  Rows are processed
 * in passes of 128 (each pass reads lm_head once).
 */
int nsd_lm_head_argmax(const void* x, const void* lm_head, int64_t n_rows, int64_t hidden,
                       int64_t vocab, uint64_t* keys, int64_t* tokens, void* stream);

/*
 * nsd_argmax_rows: torch.argmax(logits, dim=1) over fp16 logits
 * [n_rows, vocab] (first maximum; NaN counts as the maximum) into int64
 * tokens [n_rows] (post_layer.py:71 when the logits are materialised).
 */
int nsd_argmax_rows(const void* logits, int64_t n_rows, int64_t vocab, int64_t* tokens,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NSD_ATTN_H */
