/*
 * pagedkv.h — C ABI of the MI355X (gfx950) paged-KV library.
 *
 * Plain pointers, sizes and a HIP stream handle (hipStream_t passed as void*;
 * NULL means the null stream). Every device pointer is an ordinary device
 * allocation (or pinned host memory where stated). No torch types cross this
 * boundary. Every call is asynchronous on `stream` unless stated otherwise;
 * the kernels never read or write out of bounds: an out-of-range page id or
 * slot is skipped and reported through `status_word` (a device int32 whose
 * bits are OR-ed in; see PKV_STATUS_*), which the caller reads at a declared
 * check point.
 *
 * Return value: PKV_OK, or an error code with a message in pkv_last_error()
 * (thread-local, valid until the next call on the same thread).
 *
 * Pool layout (the reference's, serving/backends/paged_torch.py:127-137):
 * one allocation of `n_layers * 2` planes, plane (layer, kv) at
 * base + (layer * 2 + kv) * plane_bytes, each plane a contiguous
 * [num_blocks, page_size, n_kv_heads, head_dim] array. A per-layer K (or V)
 * pool is exactly one plane, so a caller that only has per-layer tensors
 * passes that plane's address to the per-layer entry points.
 */
#ifndef PAGEDKV_H
#define PAGEDKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types of the pool, q, k, v and out */
#define PKV_DTYPE_F16 0
#define PKV_DTYPE_BF16 1
#define PKV_DTYPE_F32 2

/* return codes */
#define PKV_OK 0
#define PKV_ERR_INVALID 1     /* argument or metadata error (Python: ValueError) */
#define PKV_ERR_RANGE 2       /* block id out of range (Python: IndexError) */
#define PKV_ERR_HIP 3         /* HIP runtime error */
#define PKV_ERR_CAPACITY 4    /* caller-provided buffer too small */

/* bits OR-ed into *status_word by the kernels */
#define PKV_STATUS_BAD_SLOT 1   /* slot_mapping entry outside [0, num_slots) */
#define PKV_STATUS_BAD_PAGE 2   /* kv_indices entry outside [0, num_blocks) */
#define PKV_STATUS_BAD_BLOCK 4  /* copy/gather/scatter id outside [0, num_blocks) */

/* Version of this ABI; bumped on any signature change. */
int pkv_abi_version(void);

/* Message for the last non-zero return on this thread ("" if none). */
const char* pkv_last_error(void);

/*
 * KV append — replaces PagedTorchBackend.append_kv
 * (serving/backends/paged_torch.py:209-276) and FlashInfer's
 * append_paged_kv_cache call (serving/backends/flashinfer_backend.py:502-512):
 * for t < n_tokens, row slot_mapping[t] of the flat [num_slots, n_kv_heads,
 * head_dim] view of k_pool / v_pool receives row t of k / v. k and v are
 * contiguous [n_tokens, n_kv_heads, head_dim] in the pool dtype.
 * Idempotent. Slots outside [0, num_slots) are skipped and flagged.
 */
int pkv_append_kv(void* k_pool, void* v_pool, int64_t num_slots,
                  const void* k, const void* v, const int32_t* slot_mapping,
                  int64_t n_tokens, int32_t n_kv_heads, int32_t head_dim,
                  int32_t dtype, int32_t* status_word, void* stream);

/*
 * Decode plan (host function, synchronous, no device access) — the
 * counterpart of the reference fast path's plan step
 * (serving/backends/flashinfer_backend.py:566-676), computed once per batch
 * and reused by every layer. Checks that every sequence has
 * ceil(kv_len / page_size) pages and that kv_last_page_len agrees
 * (PKV_ERR_INVALID, message naming kv_last_page_len, as
 * serving/backends/paged_torch.py:379-392 does).
 *
 * Each sequence of np pages is cut into pieces of part_pages pages, the
 * remainder last, a remainder shorter than both 4 pages and half a piece
 * joining the piece before it (a function of its own length only: at most
 * ceil(np / part_pages) pieces of at most part_pages + 3 pages); the pieces
 * are
 * dealt longest first to the least-loaded of at most
 * max_workgroups / (n_kv_heads / heads-per-workgroup) bins. The plan is
 * bins blocks of *plan_stride_out ints: {n_items, n_pages, 0, 0}, n_pages
 * page words (kv_indices entries, with the page's live row count - 1 in bits
 * 27..30 and an out-of-range flag in bit 31), and n_items items {seq,
 * n_pages, first token, kv_len, partial slot (-1: a whole sequence), pieces
 * of the sequence, its first slot, flags (bit 0: the piece holds the
 * sequence's last page)} at the end of the block, item i at 8 (i + 1) ints
 * before the next block -- pieces of cut sequences before their last, whole
 * sequences, then the last pieces; then 64 zero ints. *plan_stride_out is at
 * least 68.
 * *plan_needed (if not NULL) receives the ints required; a plan larger than
 * plan_capacity returns PKV_ERR_CAPACITY and writes nothing else.
 * *n_work_out is the grid size (workgroups), *n_slots_out the partial slots
 * (workspace size). num_blocks must not exceed 2^27.
 */
int pkv_plan_decode(const int32_t* kv_indptr, const int32_t* kv_indices,
                    const int32_t* kv_lens, const int32_t* kv_last_page_len,
                    int32_t n_seqs, int32_t page_size, int64_t num_blocks,
                    int32_t n_kv_heads, int32_t part_pages, int32_t max_workgroups,
                    int32_t* plan, int64_t plan_capacity, int64_t* plan_needed,
                    int32_t* n_work_out, int32_t* n_slots_out, int32_t* plan_stride_out);

/*
 * Workgroups a decode plan should be dealt into on the current device: the
 * device's compute units times the fast decode kernel's resident workgroups
 * per compute unit for this geometry, capped at per_cu. 0 if the geometry has
 * no fast kernel (or no device is current). No reference counterpart: it is
 * the grid-size half of the plan step FlashInfer's plan performs internally
 * (serving/backends/flashinfer_backend.py:658-670).
 */
int pkv_decode_workgroups(int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                          int32_t dtype, int32_t per_cu);

/*
 * Bytes of workspace pkv_attend_decode needs: arrival counters for
 * n_seqs * n_kv_heads (zero before the first launch that uses the workspace;
 * every launch leaves them zero) then n_slots partial results. 0 when
 * n_slots is 0 (no sequence is cut; no workspace is read).
 */
int64_t pkv_decode_workspace_bytes(int32_t n_seqs, int32_t n_slots, int32_t n_heads,
                                   int32_t n_kv_heads, int32_t head_dim);

/*
 * 1 if pkv_attend_decode runs its fast kernel for this geometry (and so
 * accepts a fused append), 0 if it falls back to the generic kernel.
 */
int pkv_decode_fast_path(int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                         int32_t page_size, int32_t dtype, int32_t part_pages);

/*
 * Paged decode attention — replaces PagedTorchBackend.attend
 * (serving/backends/paged_torch.py:280-485) and FlashInfer's decode wrapper
 * run (serving/backends/flashinfer_backend.py:556-562, planned at :658-670)
 * for batches where every sequence contributes exactly one query token
 * (token i belongs to sequence i). q, out: [n_seqs, n_heads, head_dim];
 * query head h reads KV head h / (n_heads / n_kv_heads); no mask (the
 * single query is the last position). `plan` is the device copy of
 * pkv_plan_decode's output, with its n_work, n_slots and plan_stride. Cut
 * sequences merge inside the launch through `workspace` (256-byte aligned,
 * pkv_decode_workspace_bytes long); launches that share a workspace must not
 * overlap in time (same stream is fine).
 *
 * Fused append: if k_new / v_new ([n_seqs, n_kv_heads, head_dim]) and
 * slot_mapping ([n_seqs]) are given, the launch also performs pkv_append_kv
 * of those rows, with the same result as the two calls in sequence (fast
 * path only). Pass NULL for all three otherwise.
 *
 * Geometries outside the fast kernel (head_dim not 64/128, more than 16
 * query heads per KV head, page_size != 16, fp32) run the generic kernel,
 * which reads kv_indptr / kv_indices / kv_lens instead of the plan.
 */
int pkv_attend_decode(const void* q, void* out,
                      void* k_pool, void* v_pool, int64_t num_blocks,
                      const int32_t* kv_indptr, const int32_t* kv_indices,
                      const int32_t* kv_lens, int32_t n_seqs,
                      int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                      int32_t page_size, float scale, int32_t dtype,
                      const int32_t* plan, int32_t n_work, int32_t n_slots,
                      int32_t plan_stride,
                      const void* k_new, const void* v_new, const int32_t* slot_mapping,
                      void* workspace, int64_t workspace_bytes,
                      int32_t* status_word, void* stream);

/*
 * No-allocation decode — no counterpart in the reference. For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): the same launch as
 * pkv_attend_decode, same arguments without the workspace. The split-K
 * workspace is a file-scope device array of PKV_DECODE_SCRATCH_BYTES on each
 * GPU the library runs on (held until the process ends); a plan whose
 * pkv_decode_workspace_bytes exceeds it is rejected with PKV_ERR_CAPACITY.
 * Allocates nothing: no hipMalloc, hipFree or allocating library call. The
 * arrival counters are cleared by a fill kernel on `stream` before each launch.
 * Every call on one GPU shares that GPU's array, so calls that overlap in
 * time on one GPU (different streams, or threads) race; calls in order on one
 * stream do not.
 */
#define PKV_DECODE_SCRATCH_BYTES (64LL * 1024 * 1024)

int pkv_attend_decode_noalloc(const void* q, void* out,
                              void* k_pool, void* v_pool, int64_t num_blocks,
                              const int32_t* kv_indptr, const int32_t* kv_indices,
                              const int32_t* kv_lens, int32_t n_seqs,
                              int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                              int32_t page_size, float scale, int32_t dtype,
                              const int32_t* plan, int32_t n_work, int32_t n_slots,
                              int32_t plan_stride,
                              const void* k_new, const void* v_new, const int32_t* slot_mapping,
                              int32_t* status_word, void* stream);

/*
 * Prefill plan (host function) — tiles each sequence's query rows for
 * pkv_attend_prefill. Output `plan` = n_tiles items {seq, q_start, q_len,
 * 0}, ordered by descending work.
 */
int pkv_plan_prefill(const int32_t* cu_query_lens, const int32_t* kv_indptr,
                     const int32_t* kv_lens, const int32_t* kv_last_page_len,
                     int32_t n_seqs, int32_t page_size, int32_t q_tile,
                     int32_t* plan, int64_t plan_capacity, int32_t* n_tiles_out);

/*
 * Query tile (tokens per plan tile) for which pkv_attend_prefill runs its
 * matrix-core kernel on this geometry: 128 / (n_heads / n_kv_heads), so a
 * tile is 128 query rows of one KV head. 0 if the geometry has no such
 * kernel (any q_tile then runs the generic kernel). Counterpart of the
 * tile choice inside FlashInfer's prefill plan
 * (serving/backends/flashinfer_backend.py:635-649).
 */
int pkv_prefill_q_tile(int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                       int32_t page_size, int32_t dtype);

/*
 * Paged attention for arbitrary per-sequence query lengths (chunked prefill,
 * mixed prefill+decode) — replaces PagedTorchBackend.attend
 * (serving/backends/paged_torch.py:280-485) and FlashInfer's prefill wrapper
 * run (serving/backends/flashinfer_backend.py:556-562, planned with
 * causal=True at :635-649). Query j of sequence i (q_len_i queries,
 * kv_len_i keys) attends keys [0, kv_len_i - q_len_i + j] (bottom-right
 * causal). q, out: [n_tokens, n_heads, head_dim]. `batch_indices` maps each
 * token to its sequence. `plan` is the device copy of pkv_plan_prefill's
 * output (q_tile must match the one given to the plan). The matrix-core
 * kernel runs when q_tile == pkv_prefill_q_tile(...) != 0; otherwise the
 * generic kernel runs (it reads cu_query_lens / batch_indices, not the plan).
 */
int pkv_attend_prefill(const void* q, void* out,
                       const void* k_pool, const void* v_pool, int64_t num_blocks,
                       const int32_t* cu_query_lens, const int32_t* kv_indptr,
                       const int32_t* kv_indices, const int32_t* kv_lens,
                       const int32_t* batch_indices,
                       int32_t n_seqs, int32_t n_tokens,
                       int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                       int32_t page_size, float scale, int32_t dtype,
                       const int32_t* plan, int32_t n_tiles, int32_t q_tile,
                       int32_t* status_word, void* stream);

/*
 * Batched block copy over every layer, K and V — replaces
 * PagedTorchBackend.copy_block (serving/backends/paged_torch.py:181-207),
 * called once per pair by RadixCache.ensure_writable
 * (serving/cache/radix.py:672-674). For each pair p, block dst[p] of every
 * plane becomes a copy of block src[p]. All sources are read before any
 * destination is written only if no dst appears among the srcs; the caller
 * guarantees that (and that dsts are distinct). Ids outside
 * [0, num_blocks) are skipped and flagged.
 */
int pkv_copy_blocks(void* pool_base, int32_t n_layers, int64_t plane_bytes,
                    int64_t block_bytes, int64_t num_blocks,
                    const int32_t* src, const int32_t* dst, int32_t n_pairs,
                    int32_t* status_word, void* stream);

/*
 * Metadata upload — replaces the host-to-device tensor builds of
 * build_batch_meta (serving/engine_iface/batch.py:246-318; one pinned buffer
 * per step here): `bytes` bytes of the pinned host buffer `host` (allocated
 * pinned, hence mapped for the device) are copied to device memory `dst` by
 * a kernel on `stream` that reads the buffer through its device mapping, so
 * the copy is ordered on the launch stream like the kernels that read it,
 * with no copy-engine hand-off. `host` must stay unchanged until the copy
 * has run (the caller records an event after it). PKV_ERR_INVALID if `host`
 * is not pinned memory mapped for the device.
 */
int pkv_upload_pinned(void* dst, const void* host, int64_t bytes, void* stream);

/*
 * Swap-out gather — the device half of KVSwapSpace._to_host
 * (serving/scheduler/preemption.py:490-509): staging[kv][layer][i] = block
 * ids[i] of plane (layer, kv), i.e. staging is [2][n_layers][n_ids][block]
 * (K half first), the reference's SwapHandle.k / .v layout
 * (serving/scheduler/preemption.py:303-332). `staging` may be device memory
 * or pinned host memory mapped for the device.
 */
int pkv_gather_blocks(const void* pool_base, int32_t n_layers, int64_t plane_bytes,
                      int64_t block_bytes, int64_t num_blocks,
                      const int32_t* ids, int32_t n_ids, void* staging,
                      int32_t* status_word, void* stream);

/*
 * Swap-in scatter — the device half of KVSwapSpace._from_host
 * (serving/scheduler/preemption.py:511-523): the inverse of
 * pkv_gather_blocks; block ids[i] of plane (layer, kv) receives
 * staging[kv][layer][i]. ids must be distinct.
 */
int pkv_scatter_blocks(void* pool_base, int32_t n_layers, int64_t plane_bytes,
                       int64_t block_bytes, int64_t num_blocks,
                       const int32_t* ids, int32_t n_ids, const void* staging,
                       int32_t* status_word, void* stream);

/*
 * Greedy sampling — the scheduler's torch.argmax(logits, dim=-1)
 * (serving/scheduler/scheduler.py:752-757) on the device: out_ids[r] = the
 * index of the largest of the `vocab` logits of row r (row r starts at
 * element r * row_stride), with torch's order: a NaN beats every number
 * and between equal values the smaller index wins. logits are f16, bf16 or
 * f32 (dtype); out_ids is a device int64 array of n_rows entries. n_rows = 0
 * does nothing.
 */
int pkv_argmax_rows(const void* logits, int64_t n_rows, int64_t vocab, int64_t row_stride,
                    int32_t dtype, int64_t* out_ids, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PAGEDKV_H */
