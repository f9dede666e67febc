/*
 * pagedattn.h - C ABI of the MI355X (gfx950) paged-attention module.
 *
 * One shared library (libpagedattn.so) exports these entry points.  They
 * replace the FlashInfer calls that the serving engine's patched
 * LlamaAttention.forward makes (src/models/llama.py:39-249): batch planning,
 * RoPE, page append and paged prefill / decode attention.
 *
 * Conventions for every entry point:
 *   - Device pointers are plain `void*` / typed pointers to device memory
 *     (HBM of the current HIP device); "_host" pointers are host memory.
 *   - Strides are in elements, not bytes; the innermost (head_dim) axis must
 *     be contiguous.
 *   - `stream` is a hipStream_t passed as `void*` (NULL = default stream).
 *     Every kernel is launched on it; nothing synchronises the device.
 *   - The return value is 0 on success or one of the PAGEDATTN_ERR_* codes.
 *     A human-readable message for the last failure on the calling thread is
 *     available from pagedattn_last_error().  Invalid arguments are rejected
 *     on the host before any launch; device-side index checks skip (never
 *     fault on) out-of-range metadata and count it in `error_flag` where the
 *     call takes one.
 *   - kv_indices arguments come with num_indices, the number of valid
 *     entries; kernels never read past it (a page slot whose index would lie
 *     beyond it is treated as absent).
 *   - The library never allocates device memory.  Work lists and split-KV
 *     partials live in the caller's workspace buffer (128 MiB in the engine,
 *     src/models/llama.py:49-53).
 *
 * KV pool layout ("HND", src/engine/memory/allocator.py:25-36): one layer is
 * a contiguous [num_pages, 2, num_kv_heads, page_size, head_dim] array; K of
 * (page p, head h) is the page_size x head_dim block at element offset
 * ((p*2+0)*num_kv_heads+h)*page_size*head_dim, V at ((p*2+1)*...).
 * fp8 pools store OCP e4m3fn bytes in the same layout plus fp32 scales
 * [num_pages, 2, num_kv_heads]; the stored value is round(x / scale).
 */
#ifndef PAGEDATTN_H_
#define PAGEDATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types */
#define PAGEDATTN_F16 0
#define PAGEDATTN_BF16 1
#define PAGEDATTN_E4M3 2 /* OCP float8 e4m3fn; KV pool only */
#define PAGEDATTN_F32 3

/* status codes */
#define PAGEDATTN_OK 0
#define PAGEDATTN_ERR_INVALID 1     /* bad argument / metadata */
#define PAGEDATTN_ERR_UNSUPPORTED 2 /* shape or dtype not implemented */
#define PAGEDATTN_ERR_WORKSPACE 3   /* workspace too small for the plan */
#define PAGEDATTN_ERR_HIP 4         /* HIP runtime error (launch failure) */
#define PAGEDATTN_ERR_PLAN 5        /* run does not match its plan */

#define PAGEDATTN_ABI_VERSION 1

/* Opaque host-side plan: the work partition built by a *_plan call and
 * consumed by the matching *_run call.  One plan per wrapper object
 * (src/models/llama.py:55-67); it is not thread-safe. */
typedef struct pagedattn_plan pagedattn_plan;

int pagedattn_abi_version(void);
const char* pagedattn_last_error(void);

/* Number of compute units of the current device (0 if no device). */
int pagedattn_device_cu_count(void);

/* ---------------------------------------------------------------------------
 * flashinfer.get_batch_indices_positions(append_indptr, seq_lens, nnz)
 * (called from src/models/llama.py:70-83 build_batch_indices_positions).
 * For token j in [append_indptr[b], append_indptr[b+1]):
 *   batch_indices[j] = b
 *   positions[j]     = seq_lens[b] - (append_indptr[b+1]-append_indptr[b])
 *                      + (j - append_indptr[b])
 * append_indptr [batch_size+1], seq_lens [batch_size], outputs [nnz]; int32,
 * device.  Entries of the outputs not covered by append_indptr are left as
 * they are. */
int pagedattn_get_batch_indices_positions(const int32_t* append_indptr,
                                          const int32_t* seq_lens,
                                          int32_t batch_size, int32_t nnz,
                                          int32_t* batch_indices,
                                          int32_t* positions, void* stream);

/* ---------------------------------------------------------------------------
 * flashinfer.apply_rope_pos_ids_inplace(q, k, pos_ids, rotary_dim,
 *     interleave, rope_scale, rope_theta)  (src/models/llama.py:175-182).
 * q [nnz, num_qo_heads, head_dim], k [nnz, num_kv_heads, head_dim] (strided
 * views of the fused qkv projection), rotated in place in fp32:
 *   angle(i) = (pos / rope_scale) * rope_theta^(-2i/rotary_dim)
 *   non-interleaved (rotate-half) pairs (i, i + rotary_dim/2), i < rotary_dim/2;
 *   interleaved pairs (2i, 2i+1).
 * Dimensions >= rotary_dim are left unchanged. dtype: F16 or BF16. */
int pagedattn_apply_rope_pos_ids_inplace(
    void* q, void* k, const int32_t* pos_ids, int32_t nnz,
    int32_t num_qo_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t rotary_dim, int64_t q_stride_n, int64_t q_stride_h,
    int64_t k_stride_n, int64_t k_stride_h, int32_t interleave,
    float rope_scale, float rope_theta, int32_t dtype, void* stream);

/* ---------------------------------------------------------------------------
 * flashinfer.append_paged_kv_cache(append_key, append_value, batch_indices,
 *     positions, paged_kv_cache, kv_indices, kv_indptr, kv_last_page_len,
 *     kv_layout="HND")  (src/models/llama.py:188-210).
 * For token j: b = batch_indices[j], p = positions[j],
 *   page = kv_indices[kv_indptr[b] + p / page_size], slot = p % page_size,
 *   cache[page, 0, h, slot, :] = k[j, h, :];  cache[page, 1, h, slot, :] = v[j, h, :]
 * Bit-exact copy when cache_dtype == src_dtype.  cache_dtype E4M3 stores
 * round_to_nearest_even(clamp(x / scale, -448, 448)) with scale =
 * kv_scales[(page*2 + {0,1})*num_kv_heads + h] (kv_scales may be NULL
 * otherwise); a block whose scale is not positive and finite gets zero
 * codes.  kv_last_page_len is accepted for interface parity and, as in the
 * reference kernel, not used for addressing (may be NULL).
 * error_flag (device int32, may be NULL): error_flag[0] is incremented once
 * per token whose batch index, page slot or page id fall outside the
 * metadata (the token is skipped).  For an E4M3 cache error_flag holds two
 * int32: error_flag[1] is incremented once per 8-element piece of a written
 * row (elements [8i, 8i+8) of one K or V head row) in which some
 * |x / scale| exceeded 448 or whose scale was not positive and finite, so a
 * skipped token and a clamped value stay apart.  Both zero after a call
 * means every token landed unclamped. */
int pagedattn_append_paged_kv_cache(
    const void* append_key, const void* append_value, int64_t k_stride_n,
    int64_t k_stride_h, int64_t v_stride_n, int64_t v_stride_h,
    int32_t src_dtype, const int32_t* batch_indices, const int32_t* positions,
    int32_t nnz, void* paged_kv_cache, int32_t cache_dtype,
    const float* kv_scales, int32_t num_pages, const int32_t* kv_indices,
    int32_t num_indices, const int32_t* kv_indptr,
    const int32_t* kv_last_page_len, int32_t batch_size, int32_t num_kv_heads,
    int32_t head_dim, int32_t page_size, int32_t* error_flag, void* stream);

/* flashinfer.apply_rope_pos_ids_inplace(q, k, positions, interleave=False,
 * rope_scale, rope_theta) (src/models/llama.py:175-182) followed by
 * flashinfer.append_paged_kv_cache (:188-210), in one launch: q
 * [nnz, num_qo_heads, head_dim] and append_key are rotated in place over the
 * full head (non-interleaved halves) exactly as
 * pagedattn_apply_rope_pos_ids_inplace does, and the rotated K rows and the
 * V rows are written to their page slots as pagedattn_append_paged_kv_cache
 * does.  head_dim must be a multiple of 16.  Same metadata, error_flag and
 * e4m3 contract as pagedattn_append_paged_kv_cache. */
int pagedattn_rope_append_paged_kv_cache(
    void* q, int64_t q_stride_n, int64_t q_stride_h, int32_t num_qo_heads,
    void* append_key, const void* append_value, int64_t k_stride_n,
    int64_t k_stride_h, int64_t v_stride_n, int64_t v_stride_h,
    int32_t src_dtype, const int32_t* batch_indices, const int32_t* positions,
    int32_t nnz, float rope_scale, float rope_theta, void* paged_kv_cache,
    int32_t cache_dtype, const float* kv_scales, int32_t num_pages,
    const int32_t* kv_indices, int32_t num_indices, const int32_t* kv_indptr,
    int32_t batch_size, int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
    int32_t* error_flag, void* stream);

/* e4m3 append that maintains the page scales (no reference counterpart: the
 * engine's fp8 write path; the reference pool dtype is the model dtype,
 * src/engine/memory/allocator.py:34).  Same metadata, strides and error
 * contract as pagedattn_append_paged_kv_cache into an E4M3 cache.
 * A run = tokens of one sequence that land in one page, consecutive and in
 * position order in the token list (what get_batch_indices_positions
 * produces).  For each run and each (K|V, kv-head) block, with slot0 the
 * run's first slot and s = kv_scales[(page*2 + {0,1})*num_kv_heads + h]:
 *   s_old = slot0 > 0 ? s : 0
 *   s_new = max(s_old, smallest power of two p with 448 * p >= amax(run rows))
 *   if s_new > s_old: rows [0, slot0) are re-encoded as
 *       round(clamp(decode(row) * (s_old / s_new), +-448))
 *   run rows = round(clamp(x / s_new, +-448)), zero codes when s_new == 0
 *   s = s_new
 * (round = to nearest even e4m3fn).  kv_scales is read and written.  Two
 * runs that write one page in the same call race; the caller forks shared
 * pages first (pagedattn_fork_pages).  head_dim <= 256, multiple of 8. */
int pagedattn_append_paged_kv_cache_e4m3_amax(
    const void* append_key, const void* append_value, int64_t k_stride_n,
    int64_t k_stride_h, int64_t v_stride_n, int64_t v_stride_h, int32_t src_dtype,
    const int32_t* batch_indices, const int32_t* positions, int32_t nnz,
    void* paged_kv_cache, float* kv_scales, int32_t num_pages, const int32_t* kv_indices,
    int32_t num_indices, const int32_t* kv_indptr, int32_t batch_size,
    int32_t num_kv_heads, int32_t head_dim, int32_t page_size, int32_t* error_flag,
    void* stream);

/* Copy-on-write page fork over the whole pool (no FlashInfer counterpart; the
 * copy step of the reference's todo.md:17-19 "Copy-on-Write" item, for pages
 * shared through src/engine/memory/radix_cache.py:60-88).  kv_pool is the
 * engine's contiguous [num_layers, num_pages, 2, num_kv_heads, page_size,
 * head_dim] array of pool_dtype (F16, BF16 or E4M3; head_dim * element size a
 * multiple of 16 bytes).  For fork f and every layer l, rows
 * [0, valid_tokens[f]) (all page_size rows when valid_tokens is NULL) of
 * every (K|V, kv-head) block of page src_pages[f] are copied to page
 * dst_pages[f]; for E4M3 the kv_scales [num_layers, num_pages, 2,
 * num_kv_heads] entries are copied too (kv_scales may be NULL otherwise).
 * src/dst/valid are device int32 arrays of num_forks entries; a fork with a
 * page outside [0, num_pages) or a count outside [0, page_size] is skipped
 * and counted in *error_flag; src == dst is a no-op.  Destinations must be
 * distinct and must not be sources of the same call. */
int pagedattn_fork_pages(void* kv_pool, int32_t pool_dtype, int32_t num_layers,
                         int32_t num_pages, int32_t num_kv_heads, int32_t head_dim,
                         int32_t page_size, float* kv_scales, const int32_t* src_pages,
                         const int32_t* dst_pages, const int32_t* valid_tokens,
                         int32_t num_forks, int32_t* error_flag, void* stream);

/* Step metadata built on the device (replaces the Python list building and
 * upload of src/engine/runtime/step_executor.py:98-165 (prefill) and
 * :204-234 (decode), and the device-to-host sync of
 * build_batch_indices_positions, src/models/llama.py:70-83).
 * block_tables: [batch_size, table_stride] int32, the first max_pages
 * entries of row b are sequence b's pages; kv_lens[b]: tokens in the cache
 * once this step's tokens are appended; new_lens[b]: tokens this step adds
 * (NULL: a decode step, one token per sequence, token row b = sequence b).
 * Outputs (device, int32):
 *   kv_indptr [batch_size + 1], kv_indices [indices_capacity]: the first
 *     ceil(kv_lens[b] / 16) entries of every row (the decode step too; the
 *     reference passes the whole row, step_executor.py:209),
 *   kv_last_page_len [batch_size] = kv_lens % 16 or 16,
 *   qo_indptr [batch_size + 1] (may be NULL for decode): prefix sum of the
 *     new token counts,
 *   batch_indices / positions [tokens_capacity]: sequence and position of
 *     every new token (kv_lens[b] - n .. kv_lens[b] - 1).
 * One launch for batches up to 1024 sequences, two above, all with fixed
 * shapes (graph-capturable).  A row needing more than max_pages pages is
 * cut to them and outputs beyond a capacity are dropped; *error_flag is
 * incremented once per sequence whose row was cut and once per sequence
 * some of whose outputs were dropped, by both launch shapes. */
int pagedattn_build_paged_metadata(const int32_t* block_tables, int64_t table_stride,
                                   int32_t max_pages, const int32_t* kv_lens,
                                   const int32_t* new_lens, int32_t batch_size,
                                   int32_t* qo_indptr, int32_t* kv_indptr, int32_t* kv_indices,
                                   int32_t indices_capacity, int32_t* kv_last_page_len,
                                   int32_t* batch_indices, int32_t* positions,
                                   int32_t tokens_capacity, int32_t* error_flag, void* stream);

/* ---------------------------------------------------------------------------
 * Plans.  pagedattn_plan_create/destroy manage the host object.
 * BatchDecodeWithPagedKVCacheWrapper.begin_forward(kv_indptr, kv_indices,
 *     kv_last_page_len, Hq, Hkv, D, page_size, q_data_type)
 *     (src/models/llama.py:119-147).
 * The metadata arrays are host copies.  split_pages > 0 forces split-KV
 * chunks of that many pages (rounded up to a multiple of 8); 0 lets the
 * planner choose from the device's CU count; -1 disables splitting.
 * The work list and split partials are placed in `workspace` (device,
 * 256-byte aligned, workspace_bytes long) from byte 256 on, with one
 * hipMemcpyAsync on `stream`.  Bytes [0, 256) are the caller's, except
 * four int32 counters that runs increment and the library never clears:
 * byte 0, tokens the fused-append decode runs skipped; byte 4, e4m3 pieces
 * they clamped; byte 8, merge-slot waits of a shared-item decode run that
 * gave up (never in a consistent run: the item's output is then left
 * unwritten rather than merged wrongly); byte 12, q-tiles that device-planned
 * prefill runs dropped because they exceeded the plan's capacity (their
 * output rows are left unwritten). */
pagedattn_plan* pagedattn_plan_create(void);
void pagedattn_plan_destroy(pagedattn_plan* plan);

int pagedattn_decode_plan(pagedattn_plan* plan, const int32_t* kv_indptr_host,
                          const int32_t* kv_last_page_len_host,
                          int32_t batch_size, int32_t num_qo_heads,
                          int32_t num_kv_heads, int32_t head_dim,
                          int32_t page_size, int32_t split_pages,
                          void* workspace, size_t workspace_bytes,
                          void* stream);

/* Decode plan that reads no metadata on the host: the
 * BatchDecodeWithPagedKVCacheWrapper(use_cuda_graph=True) counterpart of
 * begin_forward (src/models/llama.py:133-147; the reference's todo.md:15
 * asks for CUDA-graph decode).  Only the batch size and head shape are
 * fixed here; every pagedattn_decode_run* with this plan partitions the
 * work on the device from the kv_indptr it is given (the balanced split of
 * pagedattn_decode_plan with split_pages = 0: the (sequence, head group,
 * page) stream cut into equal shares, one share per head group of waves),
 * then merges cut sequences in a second launch over all (sequence, kv head)
 * pairs.  When every CU would get 4 to 8 (sequence, KV head) items
 * (4 x CUs <= batch_size x num_kv_heads <= 8 x CUs) and batch_size <= 512,
 * the plan is a device shared-item one instead (PAGEDATTN_DECODE_SHARED=0
 * in the environment turns that off): one launch whose workgroups (one per
 * CU) rank the sequences by page count and take whole items, longest and
 * shortest paired, with no split partials and no merge.  The launches have
 * fixed shapes, no host synchronisation and no memsets, so a run can be
 * captured in a HIP graph and replayed while the metadata and pool change
 * in place.  The workspace holds the split partials only (2 x shares x
 * head-group waves slots; none for a shared-item plan). */
int pagedattn_decode_plan_device(pagedattn_plan* plan, int32_t batch_size,
                                 int32_t num_qo_heads, int32_t num_kv_heads,
                                 int32_t head_dim, int32_t page_size, void* workspace,
                                 size_t workspace_bytes);

/* The device half of BatchDecodeWithPagedKVCacheWrapper.begin_forward
 * (src/models/llama.py:119-147) for a device shared-item plan: one
 * one-workgroup launch on `stream` deals the (sequence, KV head) items of
 * the metadata now in kv_indptr / kv_last_page_len to the workgroups (the
 * same deal every run of the plan makes in its prologue otherwise) and
 * writes them, with their page ranges, into the workspace.  Until the next
 * pagedattn_decode_plan_device, runs of this plan read that table instead
 * of dealing: the metadata they are given must be the metadata of the last
 * update, as a FlashInfer run's must be its plan's.  So an engine step calls
 * it once after writing the step's metadata and then runs every layer; the
 * launch has a fixed shape and no host synchronisation, so it is captured
 * in a HIP graph with the runs.  Outputs are bit-identical to runs that deal
 * on their own.  For a device split plan (pagedattn_decode_plan_kind
 * PAGEDATTN_DECODE_DEVICE) there is nothing to deal ahead and the call
 * returns PAGEDATTN_OK without a launch.  The table takes CUs x 8 x 32
 * bytes after the 256-byte workspace header. */
int pagedattn_decode_plan_device_update(pagedattn_plan* plan, const int32_t* kv_indptr,
                                        const int32_t* kv_last_page_len, void* stream);

/* Which partition a decode plan holds (a diagnostic with no counterpart in
 * the reference, for tests and benchmarks): PAGEDATTN_DECODE_SPLIT (a work
 * list of head groups; sequences cut between groups are merged by a second
 * launch), PAGEDATTN_DECODE_SHARED (whole (sequence, KV head) items per
 * CU-sized workgroup whose waves share each item's pages; one launch),
 * PAGEDATTN_DECODE_DEVICE (partition made on the device at run time),
 * PAGEDATTN_DECODE_DEVICE_SHARED (shared-item partition dealt on the device
 * at run time, see pagedattn_decode_plan_device), or 0
 * for a plan that is not a decode plan.  pagedattn_decode_plan with
 * split_pages = 0 takes a shared plan when its busiest CU carries at most
 * PAGEDATTN_DECODE_SHARED_SLACK_KB (environment, default 96) KiB plus
 * PAGEDATTN_DECODE_SHARED_SLACK_PCT (default 4) percent of the mean more K/V
 * than the mean; PAGEDATTN_DECODE_SHARED=0 / =1 turns that off / takes one
 * whenever it fits.  A shared plan's waves take fixed page pairs, so repeated
 * runs give identical bits; PAGEDATTN_DECODE_DETERMINISTIC=0 (read at plan
 * time) lets them claim pairs in arrival order instead, which balances the
 * waves of a workgroup but lets the last bits of the output vary. */
#define PAGEDATTN_DECODE_SPLIT 1
#define PAGEDATTN_DECODE_SHARED 2
#define PAGEDATTN_DECODE_DEVICE 3
#define PAGEDATTN_DECODE_DEVICE_SHARED 4
int pagedattn_decode_plan_kind(const pagedattn_plan* plan);

/* BatchDecodeWithPagedKVCacheWrapper.forward(q, paged_kv_cache)
 * (src/models/llama.py:230-245).  q [batch, num_qo_heads, head_dim] strided;
 * out [batch, num_qo_heads, head_dim] contiguous, q dtype; lse (optional,
 * fp32 [batch, num_qo_heads], natural log of the softmax denominator of the
 * scaled scores) may be NULL.  kv_scales is required for E4M3 pools. */
int pagedattn_decode_run(const pagedattn_plan* plan, const void* q,
                         int64_t q_stride_n, int64_t q_stride_h,
                         int32_t q_dtype, const void* paged_kv_cache,
                         int32_t kv_dtype, const float* kv_scales,
                         int32_t num_pages, const int32_t* kv_indices,
                         int32_t num_indices, const int32_t* kv_indptr,
                         const int32_t* kv_last_page_len, void* out,
                         float* lse, float sm_scale, void* stream);

/* The decode step of the engine (src/models/llama.py:184-245 in decode mode,
 * metadata from src/engine/runtime/step_executor.py:220-225) in one launch:
 * flashinfer.append_paged_kv_cache(append_key, append_value,
 * batch_indices = arange(B), positions = kv_len - 1, ...) followed by
 * BatchDecodeWithPagedKVCacheWrapper.forward.  append_key / append_value
 * [B, num_kv_heads, head_dim] (q dtype, strided) are written into slot
 * kv_len_b - 1 of each sequence's last page (e4m3 pools: round(clamp(x /
 * scale, +-448)) with that page's scale) and take part in the attention.
 * Row b must be sequence b's new token: the caller's batch_indices of the
 * step must be arange(B) (src/engine/runtime/step_executor.py:220-222);
 * other token orders go through pagedattn_append_paged_kv_cache and
 * pagedattn_decode_run.  A sequence (with pages) whose new token falls
 * outside its pages or on an invalid page id is not appended and counted in
 * the int32 at byte 0 of the plan's workspace; e4m3 pieces clamped as in
 * pagedattn_append_paged_kv_cache are counted in the int32 at byte 4.
 * Same plan, pool and output contract as pagedattn_decode_run. */
int pagedattn_decode_run_append(
    const pagedattn_plan* plan, const void* q, int64_t q_stride_n,
    int64_t q_stride_h, int32_t q_dtype, const void* append_key,
    const void* append_value, int64_t k_stride_n, int64_t k_stride_h,
    int64_t v_stride_n, int64_t v_stride_h, void* paged_kv_cache,
    int32_t kv_dtype, const float* kv_scales, int32_t num_pages,
    const int32_t* kv_indices, int32_t num_indices, const int32_t* kv_indptr,
    const int32_t* kv_last_page_len, void* out, float* lse, float sm_scale,
    void* stream);

/* The whole attention of one decode step of the engine in one launch:
 * flashinfer.apply_rope_pos_ids_inplace(q, k, positions, interleave=False,
 * rope_scale, rope_theta) (src/models/llama.py:175-182), then
 * pagedattn_decode_run_append's append + attention.  q and append_key are
 * rotated in registers (they are read, not modified); the rotated new K row
 * is what lands in the pool.  positions [B] int32 (device; NULL means
 * kv_len_b - 1, the engine's decode positions) is each new token's position:
 * RoPE angle, and page positions/16, slot positions%16 of the append (a
 * position outside the sequence's pages is skipped).  Rotation math is the
 * one of pagedattn_apply_rope_pos_ids_inplace, so the output and the pool
 * equal (bit for bit) those of the three separate calls.  Same row order
 * requirement and error counter as pagedattn_decode_run_append. */
int pagedattn_decode_run_rope_append(
    const pagedattn_plan* plan, const void* q, int64_t q_stride_n,
    int64_t q_stride_h, int32_t q_dtype, const void* append_key,
    const void* append_value, int64_t k_stride_n, int64_t k_stride_h,
    int64_t v_stride_n, int64_t v_stride_h, const int32_t* positions,
    float rope_scale, float rope_theta, void* paged_kv_cache, int32_t kv_dtype,
    const float* kv_scales, int32_t num_pages, const int32_t* kv_indices,
    int32_t num_indices, const int32_t* kv_indptr,
    const int32_t* kv_last_page_len, void* out, float* lse, float sm_scale,
    void* stream);

/* BatchPrefillWithPagedKVCacheWrapper.begin_forward(qo_indptr, kv_indptr,
 *     kv_indices, kv_last_page_len, Hq, Hkv, D, page_size, q_data_type)
 *     (src/models/llama.py:86-116).  Host copies of the indptr arrays.
 * q-tiles of at most half a workgroup's rows are planned as pairs of KV
 * heads sharing one workgroup when num_kv_heads is even (same output bits);
 * PAGEDATTN_PREFILL_PAIR=0, read at plan time, plans every tile alone. */
int pagedattn_prefill_plan(pagedattn_plan* plan, const int32_t* qo_indptr_host,
                           const int32_t* kv_indptr_host,
                           const int32_t* kv_last_page_len_host,
                           int32_t batch_size, int32_t num_qo_heads,
                           int32_t num_kv_heads, int32_t head_dim,
                           int32_t page_size, void* workspace,
                           size_t workspace_bytes, void* stream);

/* Prefill plan that reads no metadata on the host, for a chunked-prefill
 * step captured in a HIP graph (the reference plans every step on the host,
 * src/models/llama.py:86-116; its todo.md:15 asks for CUDA graphs).  Only
 * the batch size, head shape and a bound on the query tokens of a run
 * (max_qo_tokens, the sum of the qo lengths) are fixed here.  Every
 * pagedattn_prefill_run with this plan first launches one workgroup that
 * cuts the q-tiles of the run's qo_indptr / kv_indptr / kv_last_page_len
 * exactly as pagedattn_prefill_plan does (same pairing, up to 1024 tiles
 * ordered longest first), into the workspace, then the attention over the
 * plan's fixed capacity of ceil(max_qo_tokens / q_tile) + batch_size tiles;
 * entries past the run's tiles return at once.  The outputs equal those of
 * a host plan bit for bit.  Tiles beyond the capacity (a run with more than
 * max_qo_tokens query tokens) are skipped and counted at byte 12 of the
 * workspace.  batch_size <= 4096. */
int pagedattn_prefill_plan_device(pagedattn_plan* plan, int32_t batch_size,
                                  int32_t num_qo_heads, int32_t num_kv_heads,
                                  int32_t head_dim, int32_t page_size, int64_t max_qo_tokens,
                                  void* workspace, size_t workspace_bytes);

/* The device half of BatchPrefillWithPagedKVCacheWrapper.begin_forward
 * (src/models/llama.py:86-116) for a device prefill plan: the one-workgroup
 * launch that cuts the q-tile list from the metadata now in qo_indptr /
 * kv_indptr / kv_last_page_len, on `stream`, once.  Until the next
 * pagedattn_prefill_plan_device, runs of this plan launch no list of their
 * own and read this one: their metadata must be the metadata of the last
 * update (as a FlashInfer run's must be its plan's), so an engine step calls
 * it once after writing the step's metadata and then runs every layer.
 * Fixed shape, no host synchronisation: captured in a HIP graph with the
 * runs.  Outputs are bit-identical to runs that cut their own list. */
int pagedattn_prefill_plan_device_update(pagedattn_plan* plan, const int32_t* qo_indptr,
                                         const int32_t* kv_indptr,
                                         const int32_t* kv_last_page_len, void* stream);

/* BatchPrefillWithPagedKVCacheWrapper.forward(q, paged_kv_cache, causal)
 * (src/models/llama.py:212-228).  Ragged q [nnz, num_qo_heads, head_dim];
 * with causal != 0, row i of sequence b sees kv token j iff
 * j <= kv_len_b - qo_len_b + i (bottom-right aligned). */
int pagedattn_prefill_run(const pagedattn_plan* plan, const void* q,
                          int64_t q_stride_n, int64_t q_stride_h,
                          int32_t q_dtype, const int32_t* qo_indptr,
                          const void* paged_kv_cache, int32_t kv_dtype,
                          const float* kv_scales, int32_t num_pages,
                          const int32_t* kv_indices, int32_t num_indices,
                          const int32_t* kv_indptr,
                          const int32_t* kv_last_page_len, void* out,
                          float* lse, int32_t causal, float sm_scale,
                          void* stream);

/* ---------------------------------------------------------------------------
 * No counterpart in the reference (its pool dtype equals the model dtype,
 * src/engine/memory/allocator.py:34).  Builds an fp8 pool from a bf16/fp16
 * pool: for every (page, K|V, kv-head) block, scale = amax / 448 (1.0 for an
 * all-zero block) and dst = e4m3fn(round(src / scale)).
 * src/dst [num_pages, 2, num_kv_heads, page_size, head_dim],
 * scales [num_pages, 2, num_kv_heads] fp32. */
int pagedattn_quantize_pages_e4m3(const void* src_cache, int32_t src_dtype,
                                  void* dst_cache, float* scales,
                                  int32_t num_pages, int32_t num_kv_heads,
                                  int32_t head_dim, int32_t page_size,
                                  void* stream);

/* ---------------------------------------------------------------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory: code under HIP graph capture, serving loops or harnesses that
 * forbid hipMalloc.  pagedattn_decode_run over the device-side partition of
 * pagedattn_decode_plan_device (the same kernels and partition, so the same
 * results bit for bit), with no plan object and no workspace: the split
 * partials live in a static device array of PAGEDATTN_NOALLOC_SCRATCH_BYTES
 * that every GPU the library runs on holds until the process ends.  The call
 * allocates nothing (its first call on a device looks up that device's copy
 * of the array with hipGetSymbolAddress).  The partials of a shape take
 * 2 x 4 x CUs slots of (Hq/Hkv) x (D + 1) fp32 values; a shape that does not
 * fit (none of the supported head shapes on a 256-CU MI355X) returns
 * PAGEDATTN_ERR_WORKSPACE.  Nothing in the array needs to start at zero,
 * but every call on a GPU shares it, so calls that overlap on one GPU
 * (different streams, or threads without ordering) race.  Arguments as for
 * pagedattn_decode_plan_device + pagedattn_decode_run. */
#define PAGEDATTN_NOALLOC_SCRATCH_BYTES (17u << 20)
int pagedattn_decode_run_noalloc(int32_t batch_size, int32_t num_qo_heads,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                 const void* q, int64_t q_stride_n, int64_t q_stride_h,
                                 int32_t q_dtype, const void* paged_kv_cache, int32_t kv_dtype,
                                 const float* kv_scales, int32_t num_pages,
                                 const int32_t* kv_indices, int32_t num_indices,
                                 const int32_t* kv_indptr, const int32_t* kv_last_page_len,
                                 void* out, float* lse, float sm_scale, void* stream);

/* No counterpart in the reference: a plain streaming copy of `bytes` bytes
 * (multiple of 16, 16-byte aligned pointers), used to calibrate HBM byte
 * counters against a kernel of known traffic. */
int pagedattn_copy_bytes(void* dst, const void* src, size_t bytes,
                         void* stream);

/* No counterpart in the reference: a plain streaming read of `bytes` bytes
 * (multiple of 16, 16-byte aligned), XOR-reduced into one dword per
 * workgroup in sink[0, min(sink_entries, 8 x CUs)); the read-only point of
 * the HBM byte-counter calibration. */
int pagedattn_read_bytes(const void* src, size_t bytes, uint32_t* sink,
                         int32_t sink_entries, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PAGEDATTN_H_ */
