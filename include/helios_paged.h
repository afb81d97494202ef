/*
 * helios_paged.h — C ABI of the MI355X paged-KV hot path.
 *
 * Three operations, matching the reference's paged KV cache
 * (src/helios/runtime/qwen3/paged_cache.py) and its dense-KV block copy
 * (src/helios/runtime/qwen3/cache.py):
 *   - KV append into a shared pool of pages           (hx_kv_append)
 *   - page-table-driven varlen GQA attention         (hx_varlen_attn*)
 *   - prefix block restore / page copy and gather    (hx_kv_copy_pages, hx_kv_gather)
 *
 * Conventions
 *   - Every pointer named *_pool, *_cache, q, k_new, v_new, out, lse, workspace,
 *     write_slots, pages, block_table, cu_seq_*, seqused_k is a DEVICE pointer
 *     unless the comment says "host".
 *   - Strides are in ELEMENTS, and the innermost (head_dim) dimension is contiguous.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *   - Calls are asynchronous and stream-ordered. The library never synchronises
 *     the device, never allocates device memory, and keeps no state between calls.
 *   - Return value: 0 on success; a negative HX_E* code for an argument error
 *     (the caller maps it to ValueError); a positive hipError_t for a launch error.
 *     Nothing throws or aborts across this ABI.
 *   - Device-side metadata (write slots, page ids, sequence lengths) is clamped or
 *     skipped when out of range, so no kernel reads or writes outside the buffers
 *     it was given; hx_varlen_attn_* also raise bits in the workspace error word.
 *
 * Pool layout (paged_cache.py:47-55): one K and one V tensor per layer, each
 *   [num_pages, page_size, n_kv_heads, head_dim], contiguous. Page id p addresses
 *   pool[p]; block tables are int32 [batch, width], padded with page 0.
 */
#ifndef HELIOS_PAGED_H
#define HELIOS_PAGED_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes --------------------------------------------------------- */
#define HX_OK 0
#define HX_E_INVALID_ARG (-1)   /* a size, stride, pointer or id is out of range   */
#define HX_E_UNSUPPORTED (-2)   /* head_dim / group size / dtype not built         */
#define HX_E_WORKSPACE (-3)     /* workspace missing, misaligned or too small      */
#define HX_E_OVERLAP (-4)       /* page copy source and destination sets overlap   */
#define HX_E_TOO_LARGE (-5)     /* beyond the no-allocation scratch (hx_varlen_attn_noalloc) */

/* ---- element types -------------------------------------------------------- */
#define HX_DTYPE_BF16 0
#define HX_DTYPE_FP16 1

/* ---- bits of the workspace error word (hx_varlen_attn_error_word) --------- */
#define HX_WERR_BAD_PAGE 1        /* a block-table entry outside [0, num_pages)     */
#define HX_WERR_CLAMPED_LEN 2     /* a sequence length above max_k / max_q / table  */
#define HX_WERR_BAD_CU_SEQ 4      /* cu_seq_q not monotone or beyond total_q        */
#define HX_WERR_GRID 8            /* more work items than the launch grid covered   */
#define HX_WERR_PLAN_MISMATCH 16  /* run called with a shape its plan was not built for */
#define HX_WERR_BAD_QUERY_ROW 32  /* a query row map entry outside [0, query_rows_total) */

/* Human-readable text for a status code (static storage). */
const char* hx_strerror(int code);

/* ABI version: bumped on any signature change. */
int hx_abi_version(void);

/*
 * KV append (replaces PagedBatchCache._write, paged_cache.py:335-345, i.e. two
 * index_copy_ calls on pool.view(-1, n_kv_heads, head_dim)):
 *   for t in [0, n_tokens): k_pool_rows[write_slots[t]] = k_new[t]
 *                           v_pool_rows[write_slots[t]] = v_new[t]
 * where a pool row is n_kv_heads * head_dim contiguous elements and pool_rows =
 * num_pages * page_size. k_new[t][h] starts at k_new + t*k_row_stride + h*k_head_stride.
 * Slots outside [0, pool_rows) are skipped. Duplicate slots: last writer is unspecified
 * (as for index_copy_). Bit-exact copy of elem_bytes-wide elements.
 */
int hx_kv_append(void* k_pool, void* v_pool, int64_t pool_rows,
                 const void* k_new, int64_t k_row_stride, int64_t k_head_stride,
                 const void* v_new, int64_t v_row_stride, int64_t v_head_stride,
                 const int64_t* write_slots, int64_t n_tokens,
                 int32_t n_kv_heads, int32_t head_dim, int32_t elem_bytes,
                 void* stream);

/*
 * Page copy across layers (the page-granular form of KVCache.snapshot_block /
 * restore_blocks, cache.py:109-147, which copy a block of tokens for every layer,
 * K and V, bit-exactly; and of PagedKVCache.restore_blocks, paged_cache.py:142-163,
 * when the restored pages must be private copies):
 *   for l < n_layers, i < n_pages:  k_pools[l][dst_pages[i]] = k_pools[l][src_pages[i]]
 *                                   v_pools[l][dst_pages[i]] = v_pools[l][src_pages[i]]
 * k_pools / v_pools are HOST arrays of n_layers device pointers (v_pools may be NULL
 * to copy K only); src_pages / dst_pages are HOST arrays of n_pages page ids.
 * page_bytes = page_size * n_kv_heads * head_dim * elem_bytes. Destination ids must
 * be distinct and disjoint from the sources (HX_E_OVERLAP otherwise).
 */
int hx_kv_copy_pages(void* const* k_pools, void* const* v_pools, int32_t n_layers,
                     const int32_t* src_pages, const int32_t* dst_pages, int32_t n_pages,
                     int32_t num_pool_pages, int64_t page_bytes, void* stream);

/*
 * Page gather paged -> dense (replaces _gather_cpu, paged_cache.py:405-414:
 * index_select over pages, flatten, keep the first `length` tokens, permute to
 * head-major):  out[h][j][:] = pool[pages[j / page_size]][j % page_size][h][:]
 * for j < length; out is [n_kv_heads, length, head_dim] contiguous. pages is a
 * DEVICE array of n_pages int32 ids; an id outside [0, num_pool_pages) yields zeros.
 */
int hx_kv_gather(const void* pool, int32_t num_pool_pages, int32_t page_size,
                 int32_t n_kv_heads, int32_t head_dim, int32_t elem_bytes,
                 const int32_t* pages, int32_t n_pages, int64_t length,
                 void* out, void* stream);

/*
 * Paged varlen GQA attention (replaces torch varlen_attn(q, k_cache, v_cache,
 * cu_seq_q, cu_seq_k, max_q, max_k, window_size=(-1, 0), enable_gqa=...,
 * seqused_k=..., block_table=..., num_splits=1) at paged_cache.py:316-329 and
 * :506-519). For sequence b with query rows cu_seq_q[b]..cu_seq_q[b+1] (n_b rows)
 * and L_b keys (seqused_k[b], or cu_seq_k[b+1]-cu_seq_k[b] when seqused_k is NULL),
 * row i sits at key position qpos = L_b - n_b + i (bottom-right aligned) and sees
 * keys j with  (window_left  < 0 or j >= qpos - window_left) and
 *              (window_right < 0 or j <= qpos + window_right) and j < L_b.
 * Query head h reads KV head h / (n_q_heads / n_kv_heads).
 *   O[row, h] = softmax_j(scale * q[row, h] . K[j, h/G]) @ V[j, h/G]
 * Keys live in pages when page_size > 0: key j of sequence b is row
 * block_table[b * block_table_stride + j / page_size] * page_size + j % page_size
 * of the pool viewed as [num_pages * page_size, n_kv_heads, head_dim]. When
 * page_size == 0 the keys are packed: key j of b is row cu_seq_k[b] + j of a
 * [total_k_rows, n_kv_heads, head_dim] tensor (block_table ignored).
 * A row with no visible key outputs zeros (lse = -inf).
 * head_dim: any multiple of 8 from 8 to 256; n_q_heads any multiple of n_kv_heads;
 * bf16 and fp16; softmax and accumulation in fp32.
 *
 * Work split at head_dim 128 with n_q_heads / n_kv_heads in {1, 2, 4, 8}: decode rows
 * (n_b == 1) run a split-K kernel, one workgroup per (256-key split, KV head) whose
 * query heads share each K/V read, and a deterministic combine; chunk rows (n_b > 1)
 * run a bf16/fp16 MFMA kernel. Every other shape runs one kernel for all rows: a
 * workgroup per (sequence, block of query rows, KV head, up to 16 of its query heads)
 * sharing each 64-key K/V tile through LDS, with fp32 scores and P.
 *
 * The workspace (size from hx_varlen_attn_workspace_bytes, 256-byte aligned) holds
 * the work plan and the split-K partials. hx_varlen_attn_plan writes the plan from
 * the metadata; hx_varlen_attn_run consumes it and may be called any number of
 * times (e.g. once per layer) while cu_seq_q / cu_seq_k / seqused_k and the scalar
 * shape arguments are unchanged. hx_varlen_attn = plan + run.
 *
 * decode_items_hint / prefill_items_hint size the launch grids. Pass -1 to use the
 * bound derived from (batch, max_q, max_k); a caller that knows the host-side
 * lengths passes the exact counts from hx_varlen_attn_count_items to avoid empty
 * workgroups. A hint below the real count sets HX_WERR_GRID (rows left unwritten).
 */
size_t hx_varlen_attn_workspace_bytes(int32_t batch, int32_t max_q, int32_t max_k,
                                      int32_t n_q_heads, int32_t n_kv_heads,
                                      int32_t head_dim);

/* Host-side item counts for known lengths (q_lens[b] = n_b, k_lens[b] = L_b, HOST
 * arrays); mirrors the device planner exactly. Returns 0 or HX_E_INVALID_ARG. */
int hx_varlen_attn_count_items(const int32_t* q_lens, const int32_t* k_lens, int32_t batch,
                               int32_t n_q_heads, int32_t n_kv_heads,
                               int32_t window_left, int32_t window_right,
                               int32_t* decode_items, int32_t* prefill_items,
                               int32_t* combine_seqs);

int hx_varlen_attn_plan(const int32_t* cu_seq_q, const int32_t* cu_seq_k,
                        const int32_t* seqused_k, int32_t batch, int32_t total_q,
                        int32_t max_q, int32_t max_k, int64_t total_k_rows,
                        int32_t page_size, int32_t block_table_stride,
                        int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                        int32_t window_left, int32_t window_right,
                        void* workspace, size_t workspace_bytes, void* stream);

int hx_varlen_attn_run(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                       const void* k_cache, const void* v_cache,
                       int64_t kv_row_stride, int64_t kv_head_stride,
                       int32_t num_pages, int32_t page_size,
                       const int32_t* block_table, int32_t block_table_stride,
                       int32_t batch, int32_t total_q, int32_t max_q, int32_t max_k,
                       int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                       float scale, int32_t window_left, int32_t window_right,
                       int32_t dtype,
                       void* out, int64_t o_row_stride, int64_t o_head_stride,
                       float* lse,
                       int32_t decode_items_hint, int32_t prefill_items_hint,
                       int32_t combine_seqs_hint,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * hx_varlen_attn_run with the packed query rows read through a row map: packed row t
 * reads query row query_rows[t] of q (query_rows: device int64 [total_q]; q holds
 * query_rows_total rows at q_row_stride). Outputs, lse and the plan stay indexed by
 * packed row. A map entry outside [0, query_rows_total) reads row 0 and sets
 * HX_WERR_BAD_QUERY_ROW. No reference counterpart: the shared-prefix cascade runs its
 * prefix levels over member rows that repeat the tick's decode rows, and reads them in
 * place instead of gathering them first.
 */
int hx_varlen_attn_run_rows(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                            const int64_t* query_rows, int64_t query_rows_total,
                            const void* k_cache, const void* v_cache,
                            int64_t kv_row_stride, int64_t kv_head_stride,
                            int32_t num_pages, int32_t page_size,
                            const int32_t* block_table, int32_t block_table_stride,
                            int32_t batch, int32_t total_q, int32_t max_q, int32_t max_k,
                            int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                            float scale, int32_t window_left, int32_t window_right,
                            int32_t dtype,
                            void* out, int64_t o_row_stride, int64_t o_head_stride,
                            float* lse,
                            int32_t decode_items_hint, int32_t prefill_items_hint,
                            int32_t combine_seqs_hint,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * hx_varlen_attn_run whose combine launch also does a shared-prefix cascade merge (the
 * work of hx_attn_merge after the run, without its launch). Member k is the decode row of
 * sequence member_seq[k] (member_of_seq[b]: sequence b's member index or -1, [batch]);
 * its parts are rows part_idx[part_start[k]] .. part_idx[part_start[k + 1] - 1] of
 * level_out ([level_rows, n_q_heads, 128], strides in elements) with natural-log
 * log-sum-exps level_lse[h * level_rows + row] (contiguous [n_q_heads, level_rows]). The
 * members' rows of out and lse get exactly what hx_varlen_attn_run followed by
 * hx_attn_merge over the same parts gives, bit for bit. Call it with the combine phase
 * (combine_seqs_hint != 0 or -1): the merge runs in this call's combine launch, which is
 * launched whenever n_members > 0. lse must be given; out and level_out need 16-byte
 * aligned rows (strides multiples of 8 elements); head_dim 128 with n_q_heads /
 * n_kv_heads in {1, 2, 4, 8} (HX_E_UNSUPPORTED otherwise). No reference counterpart.
 */
int hx_varlen_attn_run_merged(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                              const void* k_cache, const void* v_cache,
                              int64_t kv_row_stride, int64_t kv_head_stride,
                              int32_t num_pages, int32_t page_size,
                              const int32_t* block_table, int32_t block_table_stride,
                              int32_t batch, int32_t total_q, int32_t max_q, int32_t max_k,
                              int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                              float scale, int32_t window_left, int32_t window_right,
                              int32_t dtype,
                              void* out, int64_t o_row_stride, int64_t o_head_stride,
                              float* lse,
                              const void* level_out, int64_t level_row_stride, int64_t level_head_stride,
                              const float* level_lse, int64_t level_rows,
                              const int32_t* member_seq, const int32_t* member_of_seq, int32_t n_members,
                              const int32_t* part_start, const int32_t* part_idx, int32_t n_parts,
                              int32_t decode_items_hint, int32_t prefill_items_hint,
                              int32_t combine_seqs_hint,
                              void* workspace, size_t workspace_bytes, void* stream);

/*
 * hx_varlen_attn_run_merged that also finishes the level batch's own run: the level
 * plan (level_batch, level_max_q, level_max_k, same heads and head_dim, its workspace
 * level_workspace) writes level_out / level_lse ([level_rows] rows, lse [n_q_heads,
 * level_rows]). This call runs that plan's combine phase (level_combine_hint bounds its
 * records, as combine_seqs_hint does for a run) before the merge reads the level rows.
 * Its records run as extra workgroups after the decode workgroups of this call's decode
 * launch; without a decode launch in this call, or for level rows of more than 8192
 * keys, they get a combine launch of their own first.
 *
 * level_block_table == NULL: the level plan ran its decode and chunk phases earlier on
 * the same stream. Otherwise this call runs the level plan's chunk phase as well, in one
 * chunk launch with this call's own chunk items, ahead of the decode launch:
 * level_block_table / level_block_table_stride are the level batch's block table,
 * level_query_rows[level_query_rows_total] maps its packed rows to rows of q (as for
 * hx_varlen_attn_run_rows), level_prefill_hint bounds its chunk items, and
 * level_window_left / level_window_right are the window the level plan was built for
 * (both ignored when level_block_table is NULL). The level
 * plan must hold no decode rows (HX_WERR_GRID in its error word otherwise), and the call
 * appends nothing: its own chunk rows then run before its decode launch.
 *
 * level_out and level_lse end up with the bits of the level plan's own run, and out / lse
 * with the bits of hx_varlen_attn_run_merged. Same requirements as
 * hx_varlen_attn_run_merged; level_out rows need 8-byte alignment (16-byte for the merge,
 * as there). No reference counterpart: it saves the cascade one or two dependent launches
 * per layer.
 */
int hx_varlen_attn_run_cascade(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                               const void* k_cache, const void* v_cache,
                               int64_t kv_row_stride, int64_t kv_head_stride,
                               int32_t num_pages, int32_t page_size,
                               const int32_t* block_table, int32_t block_table_stride,
                               int32_t batch, int32_t total_q, int32_t max_q, int32_t max_k,
                               int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                               float scale, int32_t window_left, int32_t window_right,
                               int32_t dtype,
                               void* out, int64_t o_row_stride, int64_t o_head_stride,
                               float* lse,
                               void* level_out, int64_t level_row_stride, int64_t level_head_stride,
                               float* level_lse, int64_t level_rows,
                               int32_t level_batch, int32_t level_max_q, int32_t level_max_k,
                               int32_t level_combine_hint, void* level_workspace, size_t level_workspace_bytes,
                               const int32_t* level_block_table, int32_t level_block_table_stride,
                               const int64_t* level_query_rows, int64_t level_query_rows_total,
                               int32_t level_prefill_hint, int32_t level_window_left, int32_t level_window_right,
                               const int32_t* member_seq, const int32_t* member_of_seq, int32_t n_members,
                               const int32_t* part_start, const int32_t* part_idx, int32_t n_parts,
                               int32_t decode_items_hint, int32_t prefill_items_hint,
                               int32_t combine_seqs_hint,
                               void* workspace, size_t workspace_bytes, void* stream);

/*
 * KV append + attention in one call: the PagedBatchCache.attend sequence of the
 * reference (paged_cache.py:301-332 and :501-520: _write, i.e. index_copy_ of the new
 * rows into k_cache / v_cache at write_slots, then varlen_attn on the updated pool).
 * Row t of k_new / v_new ([total_q, n_kv_heads, head_dim], strides in elements) is
 * the new key / value of packed query row t. Decode rows are appended inside the
 * decode kernel (the workgroup owning the row's last split stores its head's slice
 * and uses it from registers), so a decode-only tick issues no separate append
 * launch. On a tick that may hold chunk rows (max_q >= 2), workgroups added to the
 * decode launch append every row, and the chunk kernel, launched after it, reads them;
 * when no decode launch runs, every row is appended first by the append kernel. The pool must hold the token of decode row b at block-table position
 * seqused_k[b] - 1, i.e. write_slots must agree with the block table, as the
 * reference's metadata does by construction. pool_rows = num_pages * page_size. The
 * pools must be contiguous rows: kv_row_stride == n_kv_heads * head_dim and
 * kv_head_stride == head_dim (HX_E_INVALID_ARG otherwise), since a write slot names a
 * whole pool row.
 */
int hx_varlen_attn_append_run(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                              void* k_cache, void* v_cache,
                              int64_t kv_row_stride, int64_t kv_head_stride,
                              int32_t num_pages, int32_t page_size,
                              const int32_t* block_table, int32_t block_table_stride,
                              int32_t batch, int32_t total_q, int32_t max_q, int32_t max_k,
                              int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                              float scale, int32_t window_left, int32_t window_right,
                              int32_t dtype,
                              void* out, int64_t o_row_stride, int64_t o_head_stride,
                              float* lse,
                              const void* k_new, int64_t k_new_row_stride, int64_t k_new_head_stride,
                              const void* v_new, int64_t v_new_row_stride, int64_t v_new_head_stride,
                              const int64_t* write_slots, int64_t pool_rows,
                              int32_t decode_items_hint, int32_t prefill_items_hint,
                              int32_t combine_seqs_hint,
                              void* workspace, size_t workspace_bytes, void* stream);

int hx_varlen_attn(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                   const void* k_cache, const void* v_cache,
                   int64_t kv_row_stride, int64_t kv_head_stride,
                   int32_t num_pages, int32_t page_size,
                   const int32_t* block_table, int32_t block_table_stride,
                   const int32_t* cu_seq_q, const int32_t* cu_seq_k,
                   const int32_t* seqused_k,
                   int32_t batch, int32_t total_q, int32_t max_q, int32_t max_k,
                   int64_t total_k_rows,
                   int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                   float scale, int32_t window_left, int32_t window_right,
                   int32_t dtype,
                   void* out, int64_t o_row_stride, int64_t o_head_stride,
                   float* lse,
                   void* workspace, size_t workspace_bytes, void* stream);

/* Byte offset of the int32 error word inside the workspace (OR of HX_WERR_* bits,
 * cleared by each hx_varlen_attn_plan). */
size_t hx_varlen_attn_error_word_offset(void);

/*
 * hx_varlen_attn without a workspace argument, for callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc. No counterpart in the reference (whose varlen_attn allocates through
 * torch). Same arguments and results as hx_varlen_attn; the plan and the split partials
 * live in a device array of HX_NOALLOC_SCRATCH_BYTES that the library holds on every
 * GPU it runs on until the process ends. The call allocates nothing: the array's device
 * address is looked up once per GPU, at that GPU's first call (make that first call
 * outside graph capture), with the stream's GPU current.
 *   - A shape whose workspace (hx_varlen_attn_workspace_bytes) exceeds the array
 *     returns HX_E_TOO_LARGE before any launch. Decode ticks of up to ~15000 256-key
 *     splits fit, and so do the mixed and long-context ticks of the Qwen3-4B
 *     workloads (about 71-100 MiB).
 *   - Every call on a GPU uses that GPU's one array: calls that overlap on one GPU
 *     (different streams, or host threads without stream order between them) race.
 *     Calls in order on one stream are safe; each call's plan rewrites what its run reads.
 *   - The error word is not readable through this entry point (use hx_varlen_attn with
 *     a workspace to diagnose metadata).
 */
#define HX_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)

int hx_varlen_attn_noalloc(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                           const void* k_cache, const void* v_cache,
                           int64_t kv_row_stride, int64_t kv_head_stride,
                           int32_t num_pages, int32_t page_size,
                           const int32_t* block_table, int32_t block_table_stride,
                           const int32_t* cu_seq_q, const int32_t* cu_seq_k,
                           const int32_t* seqused_k,
                           int32_t batch, int32_t total_q, int32_t max_q, int32_t max_k,
                           int64_t total_k_rows,
                           int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                           float scale, int32_t window_left, int32_t window_right,
                           int32_t dtype,
                           void* out, int64_t o_row_stride, int64_t o_head_stride,
                           float* lse, void* stream);

/*
 * Tick metadata on the device. Replaces the per-token list building of
 * PagedBatchCache.prepare (paged_cache.py:221-270) and PackedBatchCache.prepare_packed
 * (:418-494), and the host-to-device copies of `metadata` (:272-288).
 *
 * `seq` is a DEVICE int32 array of 3*batch values: lengths[b] (tokens cached before the
 * tick), counts[b] (tokens appended this tick) and logit_counts[b] (trailing rows of b
 * that produce logits). With E_b = lengths[b] + counts[b]:
 *   cu_seq_q  = [0, cumsum(counts)]          int32 [batch + 1]
 *   cu_seq_k  = [0, cumsum(E)]               int32 [batch + 1]
 *   seqused_k = E                            int32 [batch]
 * and for packed row t = cu_seq_q[b] + i, i < counts[b], pos = lengths[b] + i:
 *   positions[t]   = pos                                                       int64
 *   write_slots[t] = block_table[b * stride + pos / page_size] * page_size
 *                    + pos % page_size                                         int64
 *   logit_indices  = for b in order: cu_seq_q[b+1] - logit_counts[b] .. cu_seq_q[b+1] - 1
 * positions may be NULL, and logit_indices when n_logits == 0.
 *
 * total_q must be sum(counts) and n_logits must be sum(logit_counts). A row whose page
 * index reaches block_table_stride gets write slot -1, which hx_kv_append skips (rows
 * beyond sum(counts), if total_q is larger, get position -1 and slot -1). batch is at
 * most 4096.
 */
/*
 * Per-head RMSNorm + RoPE of the new queries and keys, fused with the KV append.
 * Replaces, for the paged path, q_norm / k_norm and apply_rope in
 * GroupedQueryAttention.forward (layers.py:146-160: RMSNorm over head_dim in fp32,
 * layers.py:30-40; x * cos + cat(-x2, x1) * sin in fp32, layers.py:54-72) followed by
 * _write (paged_cache.py:335-345). For packed row t and head h, with p = positions[t]
 * (clamped to [0, rope_rows)) and the reference's op order (no fused multiply-adds):
 *   n      = round((x * rsqrt(mean(x^2) + eps)) * weight)            (weight fp32 [128])
 *   out[i] = round(n[i] * cos[p][i] - n[i+64] * sin[p][i])             i < 64
 *   out[i] = round(n[i] * cos[p][i] + n[i-64] * sin[p][i])             i >= 64
 * Queries go to q_out [n_rows, n_q_heads, 128] (it may alias q). Keys go to pool row
 * write_slots[t] of k_pool, and v goes unchanged to the same row of v_pool. Rows whose
 * slot is outside [0, pool_rows) write no K/V. cos / sin are fp32 [rope_rows, 128]
 * tables (the model's rope_parameters buffers). head_dim must be 128; dtype is
 * HX_DTYPE_BF16 or HX_DTYPE_FP16 for q, k, v, q_out and the pools.
 */
int hx_qk_norm_rope_append(const void* q, int64_t q_row_stride, int64_t q_head_stride,
                           const void* k, int64_t k_row_stride, int64_t k_head_stride,
                           const void* v, int64_t v_row_stride, int64_t v_head_stride,
                           const float* q_norm_weight, const float* k_norm_weight,
                           const float* cos, const float* sin, int64_t rope_rows,
                           const int64_t* positions, int64_t n_rows,
                           int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                           float eps, int32_t dtype,
                           void* q_out, int64_t q_out_row_stride, int64_t q_out_head_stride,
                           void* k_pool, void* v_pool, int64_t pool_rows,
                           const int64_t* write_slots, void* stream);

/*
 * Merge of attention results over disjoint key sets of the same query rows (the
 * shared-prefix split of PagedBatchCache.attend; no counterpart in the reference, whose
 * varlen_attn reads every sequence's prefix pages itself). Entry j < n_rows merges its
 * parts into packed row r = rows[j] of (out, lse_out), in place: the parts are rows
 * part_idx[part_start[j]] .. part_idx[part_start[j + 1] - 1] of (o_a, lse_a), the range
 * clipped to [0, n_parts), or o_a row j alone when part_start and part_idx are NULL
 * (n_parts is then ignored). For head h, folding one part a
 * into the running result b (initially out[r][h], lse_out[h][r]) with m = max(lse_a, lse_b):
 *   o   = (o_a e^(lse_a - m) + o_b e^(lse_b - m)) / (e^(lse_a - m) + e^(lse_b - m))
 *   lse = m + log(e^(lse_a - m) + e^(lse_b - m))
 * in fp32, rounded to the element type once at the end. lse arrays are fp32
 * [n_heads, total] (the layout of hx_varlen_attn's lse): head h of row j is
 * lse_a[h * total_a + j], and o_a holds total_a rows. rows must not repeat within one
 * call; a part index outside [0, total_a) is skipped. Rows where every lse is -inf are
 * left unchanged. head_dim must be 128.
 */
int hx_attn_merge(void* out, int64_t out_row_stride, int64_t out_head_stride,
                  float* lse_out, int64_t total_out,
                  const void* o_a, int64_t a_row_stride, int64_t a_head_stride,
                  const float* lse_a, int64_t total_a,
                  const int64_t* rows, const int32_t* part_start, const int32_t* part_idx,
                  int64_t n_parts, int64_t n_rows, int32_t n_heads, int32_t head_dim,
                  int32_t dtype, void* stream);

int hx_tick_metadata(const int32_t* seq, int32_t batch, int32_t total_q, int32_t n_logits,
                     const int32_t* block_table, int32_t block_table_stride,
                     int32_t page_size,
                     int32_t* cu_seq_q, int32_t* cu_seq_k, int32_t* seqused_k,
                     int64_t* positions, int64_t* write_slots, int64_t* logit_indices,
                     void* stream);

/*
 * Final RMSNorm + lm_head + greedy argmax of the tick's logit rows. Replaces
 *   x.index_select(1, logit_indices); self.output(self.final_norm(x).to(dtype))
 * (model.py:108-110; RMSNorm over the hidden size in fp32, layers.py:29-39; the tied
 * embedding as a bias-free Linear) followed by heads.argmax(dim=-1) on the logits of
 * greedy rows (engine.py:470-473). For j < n_rows and row x = hidden_states[logit_indices[j]]:
 *   xn            = round((x * rsqrt(mean(x^2) + eps)) * norm_weight)      (fp32 weight)
 *   logit[v]      = round(sum_k xn[k] * embedding[v][k])                    (fp32 sum)
 *   token_ids[j]  = the smallest v with the largest logit[v]
 *   max_logits[j] = that logit (optional, may be NULL)
 *   logits        = [n_rows, vocab] rounded logits, row stride logits_row_stride
 *                   (optional: NULL writes none; the greedy path needs none)
 * An index outside [0, total_rows) gives token id -1 and max logit NaN. hidden must
 * be a multiple of 128; strides are in elements and multiples of 8; dtype is
 * HX_DTYPE_BF16 or HX_DTYPE_FP16 for hidden_states, embedding and logits. Up to 160
 * rows read the embedding once; more rows read it once per 160. The workspace is
 * hx_logits_workspace_bytes(n_rows, vocab, hidden) bytes, 256-byte aligned.
 */
size_t hx_logits_workspace_bytes(int64_t n_rows, int64_t vocab, int32_t hidden);

int hx_final_norm_logits_argmax(const void* hidden_states, int64_t hidden_row_stride,
                                int64_t total_rows, const int64_t* logit_indices,
                                int64_t n_rows, const float* norm_weight, float eps,
                                const void* embedding, int64_t embedding_row_stride,
                                int64_t vocab, int32_t hidden, int32_t dtype,
                                int64_t* token_ids, float* max_logits,
                                void* logits, int64_t logits_row_stride,
                                void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HELIOS_PAGED_H */
