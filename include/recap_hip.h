/* C ABI of librecap_hip.so: MI355X (gfx950) kernels of RECAP's corrected sparse-attention
 * operator.  Paths in the citations are relative to the lyraxtg/RECAP tree.
 *
 * Conventions
 *  - Every function returns 0 on success or a RECAP_E* code; recap_last_error() gives a
 *    thread-local message for the last failure.  Arguments are validated on the host
 *    before any launch; nothing is allocated and nothing synchronises the host.
 *  - Device pointers are raw; the caller owns every buffer.  `stream` is a hipStream_t
 *    (NULL = default stream); all work is enqueued on it.
 *  - A "bank" is one (batch, head) pair, bank = b * heads + h.  Q/K/V are native-order
 *    [batch, heads, tokens, dim] with element strides (stride_b, stride_h, stride_n) and a
 *    unit stride on dim; rows and strides must keep 16-byte alignment.
 *  - `rowmap[r]` (int32, [n_tokens]) is the native token of reordered row r: the Hilbert-
 *    ordered video tokens first, then the text tokens (recap/sparse/layout.py:44-61).
 *  - Block size is 128; dim is 64 or 128; dtype is RECAP_BF16 or RECAP_F16.
 *  - Derived sizes: nb = ceil(n_video/128) video blocks, tb = ceil(n_tokens/128) kernel
 *    blocks, R = floor(n_video/128)*128 refined rows.  With R = 0 (fewer than 128 video
 *    tokens) the buffers sized by R may be NULL: recap_coarse_tail and recap_drift_center
 *    do nothing, a capture writes stats = (0, 0) when stats is non-NULL, and the merge
 *    keeps the head.  Limits: tb <= 2048 for the attention entry points, nb <= 4096 for
 *    selection and the coarse tail (RECAP_EINVAL beyond).
 *  - Calls on distinct streams from distinct host threads may run concurrently when they
 *    use distinct buffers (work queues included); the library holds no mutable state on
 *    those paths.  The exceptions are recap_refresh_capture_noalloc (one static scratch
 *    array per GPU) and a pager, which one host thread drives.
 */
#ifndef RECAP_HIP_H
#define RECAP_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RECAP_ABI_VERSION 8

enum { RECAP_OK = 0, RECAP_EINVAL = 1, RECAP_EUNSUPPORTED = 2, RECAP_EHIP = 3 };
enum { RECAP_F16 = 1, RECAP_BF16 = 2 };
enum { RECAP_CLOSURE_ROT = 1, RECAP_CLOSURE_CVK = 2, RECAP_CLOSURE_SCATTER = 4 };

int recap_abi_version(void);
const char* recap_last_error(void);

/* Hilbert order of a (frames, height, width) video grid, host only: out[i] is the native
 * index t*H*W + y*W + x of reordered position i.
 * Replaces hilbert_permutation, recap/sparse/geometry.py:27-67. */
int recap_hilbert_permutation(int64_t frames, int64_t height, int64_t width, int64_t* out);

/* Stage 1 ------------------------------------------------------------------------------ */

/* fp32 means [banks, nb, dim] of the video tokens of x, gathered through rowmap.
 * Replaces pool_blocks, recap/sparse/pooling.py:10-34 (query pooling of
 * recap/sparse/attention.py:81). */
int recap_pool_blocks(const void* x, int dtype, int64_t batch, int64_t heads, int64_t dim,
                      int64_t stride_b, int64_t stride_h, int64_t stride_n,
                      const int32_t* rowmap, int64_t n_tokens, int64_t n_video,
                      float* means, void* stream);

/* One pass over K and V: packed K tiles and V^T tiles [banks, tb, 128*dim] for the
 * attention kernel, and the fp32 block means of K and V [banks, nb, dim].
 * Replaces Layout.reorder of K/V (recap/operator.py:497-498), the permute copies of
 * recap/kernels/block_sparse.py:112-114 and pool_blocks(K), pool_blocks(V)
 * (recap/sparse/attention.py:173-174). */
int recap_kv_pack(const void* k, const void* v, int dtype, int64_t batch, int64_t heads,
                  int64_t dim, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_n,
                  int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_n,
                  const int32_t* rowmap, int64_t n_tokens, int64_t n_video, void* k_tiles,
                  void* vt_tiles, float* k_means, float* v_means, void* stream);

/* Stage 1 in one call: pooled query means, fp32 block scores against k_means (from
 * recap_kv_pack), the top-keep selection with keep = max(1, round(density * nb)) (round half
 * to even) and the partial last block forced, then the kernel block mask.  partition
 * [banks, nb, nb] and kernel_mask [banks, tb, tb] (bool bytes); the intermediates live in
 * `workspace` (16-byte aligned, recap_pool_select_workspace_size bytes).  The kernel mask
 * replaces a CSR block list: the attention kernel compacts each mask row on chip.
 * Replaces SparseAttention.head_partition + block_proxy_mask + build_kernel_block_mask
 * (recap/sparse/attention.py:74-94, recap/sparse/router.py:10-23,
 * recap/kernels/block_sparse.py:52-75). */
int64_t recap_pool_select_workspace_size(int64_t banks, int64_t n_blocks, int64_t dim);
int recap_pool_select(const void* q, int dtype, int64_t batch, int64_t heads, int64_t dim,
                      int64_t stride_b, int64_t stride_h, int64_t stride_n,
                      const int32_t* rowmap, int64_t n_tokens, int64_t n_video,
                      const float* k_means, float scale, double density, void* workspace,
                      int64_t workspace_bytes, uint8_t* partition, uint8_t* kernel_mask,
                      void* stream);

/* fp32 block scores [banks, nb, nb] = fp32(scale) * (qbar . kbar), fixed summation order.
 * Replaces the matmul + mul_ of block_proxy_mask, recap/sparse/router.py:18-19. */
int recap_block_scores(const float* q_means, const float* k_means, int64_t banks,
                       int64_t n_blocks, int64_t dim, float scale, float* scores, void* stream);

/* Boolean partition [banks, nb, nb] (uint8 0/1): top-`keep` per row, ties to the lower
 * index; force_last also selects the trailing partial block as row and column.
 * Replaces topk + scatter of recap/sparse/router.py:20-22 and _match_kernel_granularity,
 * recap/sparse/attention.py:84-94. */
int recap_topk_blocks(const float* scores, int64_t banks, int64_t n_blocks, int64_t keep,
                      int force_last, uint8_t* partition, void* stream);

/* Kernel-grid mask [banks, tb, tb] with text/partial rows and columns dense.
 * Replaces build_kernel_block_mask, recap/kernels/block_sparse.py:52-75. */
int recap_kernel_block_mask(const uint8_t* partition, int64_t banks, int64_t n_tokens,
                            int64_t n_video, uint8_t* kernel_mask, void* stream);

/* work[0] = |new & old|, work[1] = |new| over `count` bytes; work holds 514 uint64.
 * Replaces the overlap sums of recap/operator.py:423-428 (the caller reads the two counts
 * to decide the rerank, as the reference does). */
int recap_mask_overlap(const uint8_t* new_mask, const uint8_t* old_mask, int64_t count,
                       uint64_t* work, void* stream);

/* Stage 3 ------------------------------------------------------------------------------ */

/* Number of partial groups of recap_closure_stats for `group` blocks per workgroup. */
int64_t recap_closure_groups(int64_t n_video, int64_t group);

/* Closure statistics from the packed tiles.  flags: ROT (needs u_hi_t/u_lo_t, writes
 * variance [banks, nb, dim]), CVK (writes cvk_partial [banks, groups, dim, dim]),
 * SCATTER (writes scatter_partial); allowed sets: ROT, CVK|SCATTER, ROT|CVK.
 * Replaces rotated_leaf_moments_triton and pooled_cross_centered_triton_fp32,
 * recap/kernels/closure_stats.py:96-290, and pooled_within_block_scatter,
 * recap/sparse/closure.py:42-72. */
int recap_closure_stats(const void* k_tiles, const void* vt_tiles, const float* k_means,
                        int dtype, const void* u_hi_t, const void* u_lo_t, int64_t banks,
                        int64_t dim, int64_t n_tokens, int64_t n_video, int64_t group,
                        int flags, float* variance, float* cvk_partial, float* scatter_partial,
                        void* stream);

/* out[b, e] = sum_g partial[b, g, e] / divisor, fixed order over g.
 * Replaces the final divisions of recap/kernels/closure_stats.py:290 and
 * recap/sparse/closure.py:72. */
int recap_partial_reduce(const float* partial, int64_t banks, int64_t groups, int64_t elems,
                         float divisor, float* out, void* stream);

/* Eigenvalues (ascending, [batch, n]) and orthonormal eigenvectors (columns, [batch, n, n])
 * of the symmetrised 0.5 (a + a^T) of `batch` row-major fp32 n x n matrices, n <= 128:
 * the contract of torch.linalg.eigh.  Two-sided parallel Jacobi in one workgroup per matrix;
 * eigenvectors are unique up to sign (and to a rotation within a repeated eigenvalue).
 * Replaces the torch.linalg.eigh call of closure_basis, recap/sparse/closure.py:75-81. */
int recap_symmetric_eigen(const float* a, int64_t batch, int64_t n, float* eigenvalues,
                          float* eigenvectors, void* stream);

/* Query-type tables of the coarse tail: w = fold_rank(variance, rank), kbar, vbar, each
 * [banks, ceil(nb/32)*32, width] elements, row j holding key block j (rows past nb zero),
 * width = dim for kbar and vbar and recap_coarse_w_width() for w.  The coarse tail gathers
 * the rows of the blocks it visits from these tables.  w is either the full fold_rank row
 * (columns in swap23 order) or, when the fold leaves few distinct values (bf16,
 * 1 <= rank <= 13), the 16 features [w_0 .. w_{rank-1}, rho, rho, rho, 0 ...] with rho the
 * mean of the folded columns.
 * Replaces fold_rank (recap/sparse/closure.py:96-104) and the casts of
 * recap/kernels/coarse_tail.py:238-241. */
int recap_coarse_tables(const float* variance, const float* k_means, const float* v_means,
                        int dtype, int64_t banks, int64_t n_blocks, int64_t dim, int64_t rank,
                        void* w, void* kbar, void* vbar, void* stream);

/* Columns of the w table for (dtype, dim, rank): 16 in the folded form, else dim; -1 for
 * invalid arguments.  Host only.  Sizes the w buffer of recap_coarse_tables (no
 * counterpart in the reference, whose w keeps dim columns). */
int64_t recap_coarse_w_width(int dtype, int64_t dim, int64_t rank);

/* Basis tables [banks, dim, dim]: U^T split hi/lo (closure statistics), U^T and C_vk in
 * the query type (coarse tail).  Any output may be NULL; cvk may be NULL if cvk_t is.
 * Replaces basis.to(dtype) / operator.to(dtype) of recap/sparse/closure.py:84-93 and the
 * basis split of recap/kernels/closure_stats.py:133-135. */
int recap_basis_tables(const float* basis, const float* cvk, int dtype, int64_t banks,
                       int64_t dim, void* u_hi_t, void* u_lo_t, void* u_t, void* cvk_t,
                       void* stream);

/* Corrected coarse tail for the R refined rows: go [banks, R, dim] (query type),
 * gl [banks, R] fp32; with glref [banks, R] also drift_partial [banks, R/128].  kbar, vbar
 * and w are the tables written by recap_coarse_tables with the same dtype, dim and
 * rank (the closure rank of fold_rank, which selects the w layout).
 * Replaces coarse_tail_attention + _coarse_tail_kernel (recap/kernels/coarse_tail.py:
 * 35-312), build_coarse_tail_plan (recap/sparse/planner.py:11-38), rotated_query_square
 * and value_drift (recap/sparse/closure.py:84-93) and coarse_tail_apply
 * (recap/sparse/attention.py:204-231). */
int recap_coarse_tail(const void* q, int dtype, int64_t batch, int64_t heads, int64_t dim,
                      int64_t stride_b, int64_t stride_h, int64_t stride_n,
                      const int32_t* rowmap, const uint8_t* partition, const void* kbar,
                      const void* vbar, const void* w, const void* u_t, const void* cvk_t,
                      int64_t n_tokens, int64_t n_video, float scale, float theta,
                      int64_t rank, const float* glref, void* go, float* gl,
                      float* drift_partial, void* stream);

/* center[b] = sum(drift_partial[b, :]) / R.
 * Replaces _drift_center, recap/operator.py:148-150. */
int recap_drift_center(const float* drift_partial, int64_t banks, int64_t n_video,
                       float* center, void* stream);

/* Stage 2 ------------------------------------------------------------------------------ */

/* Head branch at a refresh: exact attention over the kernel mask, reordered order:
 * head_out [banks, n_tokens, dim] in `dtype` (the external kernel returns its output in
 * the input type), head_lse [banks, n_tokens] fp32 (natural log).
 * Replaces block_sparse_exact, recap/kernels/block_sparse.py:78-139. */
int recap_block_sparse_attn(const void* q, int dtype, int64_t batch, int64_t heads,
                            int64_t dim, int64_t stride_b, int64_t stride_h, int64_t stride_n,
                            const void* k_tiles, const void* vt_tiles, const int32_t* rowmap,
                            const uint8_t* kernel_mask, int64_t n_tokens, float scale,
                            void* head_out, float* head_lse, void* stream);

/* A refresh's two attention results in one pass over the keys: the dense output and LSE
 * as recap_dense_attn, and the head branch of `kernel_mask` as recap_block_sparse_attn
 * (head_out [banks, n_tokens, dim] in `dtype` and head_lse [banks, n_tokens], reordered
 * rows; bit-identical to recap_block_sparse_attn's).  Each query block walks its kept key
 * blocks first and stores the head branch from the running softmax state when they are
 * done, then walks the rest.
 * Replaces the two attention calls of a refresh: aten._scaled_dot_product_flash_attention,
 * recap/operator.py:254-256, and block_sparse_exact, recap/operator.py:345-346 with
 * recap/kernels/block_sparse.py:78-139. */
int recap_dense_head_attn(const void* q, int dtype, int64_t batch, int64_t heads, int64_t dim,
                          int64_t stride_b, int64_t stride_h, int64_t stride_n,
                          const void* k_tiles, const void* vt_tiles, const int32_t* rowmap,
                          const uint8_t* kernel_mask, int64_t n_tokens, float scale, void* out,
                          int64_t out_stride_b, int64_t out_stride_h, int64_t out_stride_n,
                          float* lse, void* head_out, float* head_lse, uint32_t* work_queue,
                          void* stream);

/* Dense attention with LSE, native order: out [batch, heads, n_tokens, dim] with the
 * given strides, lse [banks, n_tokens].
 * Replaces aten._scaled_dot_product_flash_attention at recap/operator.py:254-256. */
int recap_dense_attn(const void* q, int dtype, int64_t batch, int64_t heads, int64_t dim,
                     int64_t stride_b, int64_t stride_h, int64_t stride_n, const void* k_tiles,
                     const void* vt_tiles, const int32_t* rowmap, int64_t n_tokens, float scale,
                     void* out, int64_t out_stride_b, int64_t out_stride_h,
                     int64_t out_stride_n, float* lse, void* stream);

/* The corrected sparse output in one pass: head attention with the merge of the coarse
 * tail (go, gl), the refinement (det fp16 [banks, R, dim], dl [banks, R]) and the drift
 * weight exp(-|gl - glref - center|) fused into the epilogue, stored in native order.
 * alpha_override >= 0 replaces the drift weight (test knob; pass a negative value for
 * the reference behaviour).
 * Replaces block_sparse_exact + sparse_merge + Layout.restore, recap/operator.py:500-527
 * and recap/kernels/detail_cache.py:188-301, 402-456. */
int recap_sparse_merge_attn(const void* q, int dtype, int64_t batch, int64_t heads,
                            int64_t dim, int64_t stride_b, int64_t stride_h, int64_t stride_n,
                            const void* k_tiles, const void* vt_tiles, const int32_t* rowmap,
                            const uint8_t* kernel_mask, int64_t n_tokens, int64_t n_video,
                            float scale, const void* go, const float* gl, const void* det,
                            const float* dl, const float* glref, const float* center,
                            float alpha_override, void* out, int64_t out_stride_b,
                            int64_t out_stride_h, int64_t out_stride_n, uint32_t* work_queue,
                            void* stream);

/* Words of the optional `work_queue` of recap_dense_head_attn and recap_sparse_merge_attn
 * (16-byte aligned device memory, contents ignored: the call zeroes it on `stream` before the
 * launch).  With it, workgroups claim their query blocks from per-XCD queues and XCDs that
 * finish early take the others' last blocks; NULL keeps the static assignment.  Outputs are
 * identical either way.  Calls that may overlap need separate queues.  No counterpart in
 * the reference (the external kernel schedules itself). */
int64_t recap_attn_queue_words(void);

/* Stage 4 ------------------------------------------------------------------------------ */

/* Number of (err2, ref2) partial pairs recap_refresh_capture writes. */
int64_t recap_capture_partials(int64_t banks, int64_t dim, int64_t n_video);

/* Refinement capture in place into det (fp16 [banks, R, dim]) and dl ([banks, R]) from the
 * dense output (native order, query type), the head branch (query type, as written by
 * recap_block_sparse_attn or recap_dense_head_attn) and the coarse tail.  With
 * glref and center non-NULL the previous refinement is scored first: stat_partial
 * receives the partial pairs and stats[2] = (sum err^2, sum ref^2).
 * Replaces refresh_detail + _refresh_detail_kernel, recap/kernels/detail_cache.py:25-186,
 * 304-379. */
int recap_refresh_capture(const void* dense_out, int dtype, int64_t batch, int64_t heads,
                          int64_t dim, int64_t out_stride_b, int64_t out_stride_h,
                          int64_t out_stride_n, const float* dense_lse, const void* head_out,
                          const float* head_lse, const void* go, const float* gl,
                          const int32_t* rowmap, int64_t n_tokens, int64_t n_video, void* det,
                          float* dl, const float* glref, const float* center,
                          float* stat_partial, float* stats, void* stream);

/* recap_refresh_capture without a caller workspace: the validation's partial pairs go to
 * a static device array of RECAP_CAPTURE_NOALLOC_MAX_PAIRS pairs (4 MiB) that each GPU holds
 * from the first call on it until the process ends; the call allocates nothing.  Same
 * arguments and results as recap_refresh_capture minus stat_partial; a validation needing
 * more pairs than recap_capture_partials() allows fails with RECAP_EINVAL.  Every pair the
 * final sum reads is written by the same call first, so nothing needs clearing; calls that
 * overlap on one GPU (concurrent streams) race on the array and must be serialised.
 * No counterpart in the reference: for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops that forbid hipMalloc). */
#define RECAP_CAPTURE_NOALLOC_MAX_PAIRS (1 << 19)
int recap_refresh_capture_noalloc(const void* dense_out, int dtype, int64_t batch,
                                  int64_t heads, int64_t dim, int64_t out_stride_b,
                                  int64_t out_stride_h, int64_t out_stride_n,
                                  const float* dense_lse, const void* head_out,
                                  const float* head_lse, const void* go, const float* gl,
                                  const int32_t* rowmap, int64_t n_tokens, int64_t n_video,
                                  void* det, float* dl, const float* glref,
                                  const float* center, float* stats, void* stream);

/* Host-bank pager -------------------------------------------------------------------- */

/* Refinement banks of n_keys (stream, layer) keys held in pinned host memory
 * (hipHostMalloc, allocated on a key's first write-back or by recap_pager_reserve) and staged
 * through n_slots device slots.  A bank is n_fields byte ranges of the given sizes (the
 * operator pages value fp16 [banks, R, dim], log_mass fp32 [banks, R], partition
 * [B, H, nb, nb], kernel mask [banks, tb, tb] and the drift reference fp32 [banks, R]); a
 * slot's device fields are owned by the caller and bound once (a field of zero bytes may
 * be bound as NULL).  The pager owns a prefetch
 * and a write-back stream (non-blocking, default priority) and the events that fence every
 * reuse of a slot and of a key's host copy.  RECAP_PAGER_TIMING times every copy batch
 * (recap_pager_copy_time).  One pager is driven by one host thread; destroying it waits
 * for its transfers.
 * Replaces HostBankOperator's slots, pinned banks, streams and events,
 * recap/host_banks.py:45-56, 60-103, 200-262. */
typedef struct recap_pager recap_pager;
#define RECAP_PAGER_TIMING 1
int recap_pager_create(int64_t n_keys, int32_t n_slots, const int64_t* field_bytes,
                       int32_t n_fields, int32_t flags, recap_pager** out);
int recap_pager_destroy(recap_pager* pager);
int recap_pager_bind(recap_pager* pager, int32_t slot, void* const* device_fields);
/* Allocate the pinned host banks of keys 0 .. n_keys-1 now.
 * Replaces HostBankOperator.preallocate_host, recap/host_banks.py:85-97. */
int recap_pager_reserve(recap_pager* pager, int64_t n_keys);
/* Make key's bank the contents of slot for the work queued next on `stream` (the compute
 * stream): waits for a prefetch of that key into that slot, else copies it on `stream` after
 * the slot's pending write-back.  The key must hold a bank.
 * Replaces _stage_in, recap/host_banks.py:200-207. */
int recap_pager_stage_in(recap_pager* pager, int64_t key, int32_t slot, void* stream);
/* Copy key's bank into slot on the prefetch stream once the compute stream has released the
 * slot and its last write-back is done; a key with no bank is skipped.
 * Replaces _maybe_prefetch, recap/host_banks.py:209-225. */
int recap_pager_prefetch(recap_pager* pager, int64_t key, int32_t slot);
/* Copy slot's contents into key's host bank on the write-back stream after the work queued
 * so far on `stream`; the key then holds a bank.
 * Replaces _stage_out and _split_out, recap/host_banks.py:132-146, 227-242. */
int recap_pager_stage_out(recap_pager* pager, int64_t key, int32_t slot, void* stream);
/* Order `stream` after every transfer in flight on the slot (its last write-back, a prefetch
 * into it), for a call that writes the slot without loading it (a first refresh).  Replaces
 * the wait for a pending write-back from the slot, recap/host_banks.py:169-173. */
int recap_pager_acquire(recap_pager* pager, int32_t slot, void* stream);
/* The work queued so far on `stream` is the slot's last use before it may be refilled.
 * Replaces the slot_free event, recap/host_banks.py:194-196. */
int recap_pager_release(recap_pager* pager, int32_t slot, void* stream);
/* Wait for every transfer in flight.  Replaces finish, recap/host_banks.py:246-258. */
int recap_pager_finish(recap_pager* pager);
/* 1 if key holds a bank, 0 if not, -1 for bad arguments.  Host only. */
int recap_pager_stored(const recap_pager* pager, int64_t key);
/* Pinned host bytes allocated (-1 for a NULL pager).
 * Replaces peak_bank_bytes, recap/host_banks.py:270-276. */
int64_t recap_pager_host_bytes(const recap_pager* pager);
/* counts[4]: stage-ins served by a prefetch, stage-ins copied on the compute stream,
 * prefetches issued, stage-outs.  Host only; no counterpart in the reference. */
int recap_pager_counts(const recap_pager* pager, int64_t* counts);
/* Total milliseconds of the timed copy batches and their number (RECAP_PAGER_TIMING);
 * waits for them.  No counterpart in the reference (its copies are untimed). */
int recap_pager_copy_time(recap_pager* pager, double* total_ms, int64_t* copies);
/* New field sizes for every key, after a change of the bank geometry (a per-prompt text
 * length changes the kernel mask's [banks, tb, tb]).  Waits for the transfers in flight;
 * every key then holds no bank (the next refresh writes one back), host fields that the
 * new sizes outgrow are freed and reallocated on the next write-back, and every slot must
 * be bound again.  Replaces the reallocation of the split state and of the host banks on a
 * shape change, recap/host_banks.py:58-64, 116-146, 164-167. */
int recap_pager_resize(recap_pager* pager, const int64_t* field_bytes, int32_t n_fields);

/* Asynchronous copy of a refinement bank between pinned host memory and the device on
 * `stream` (hipMemcpyAsync, direction inferred).
 * Replaces the non_blocking copy_ of recap/host_banks.py:99-103. */
int recap_bank_copy_async(void* dst, const void* src, int64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RECAP_HIP_H */
