/*
 * cacheblend_hip.h -- C ABI of the MI355X (gfx950) CacheBlend KV data-movement
 * and selection kernels.
 *
 * Plain pointers and sizes only. Every pointer named *_dev is device memory;
 * every entry point is stream-ordered on `stream` (a hipStream_t, NULL = the
 * legacy default stream), never synchronises, never allocates, and returns
 * CBK_OK or a negative CBK_ERR_* code (cbk_last_error() holds a message for
 * the calling thread). Strides are in BYTES unless named *_elems.
 *
 * Each entry point cites the reference (zoudinghong2000/PIC-KVCache) function
 * it replaces. The reference is a Python/torch package; its "FFI" for this
 * path is the Python signature, which the ctypes binding in
 * pic-kvcache_amd/cacheblend_vllm/_native.py maps onto these symbols.
 */
#ifndef CACHEBLEND_HIP_H_
#define CACHEBLEND_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* cbk_stream_t; /* hipStream_t */

enum {
  CBK_OK = 0,
  CBK_ERR_INVALID = -1,     /* bad argument: shape, stride, alignment, range */
  CBK_ERR_UNSUPPORTED = -2, /* valid request this library does not implement */
  CBK_ERR_LAUNCH = -3,      /* HIP launch/runtime failure */
  CBK_ERR_WORKSPACE = -4    /* workspace too small */
};

enum { CBK_DTYPE_F32 = 0, CBK_DTYPE_BF16 = 1, CBK_DTYPE_F16 = 2 };

/* ABI version, bumped on any signature change. */
int cbk_abi_version(void);
/* Static string for a CBK_* code. */
const char* cbk_error_string(int code);
/* Message of the last failed call on this thread ("" if none). */
const char* cbk_last_error(void);

/*
 * One paged KV layer, any of vLLM's three layouts (reference
 * cacheblend_vllm/kv_layout.py:12-20, 110-118):
 *   merged_first [2, NB, bs, H, D]  k_base = &kv[0,0,0], v_base = &kv[1,0,0]
 *   merged_block [NB, 2, bs, H, D]  k_base = &kv[0,0,0], v_base = &kv[0,1,0]
 *   separate     K,V [NB, bs, H, D] k_base = K, v_base = V
 * A token's [H, D] row must be contiguous (row_bytes bytes).
 */
typedef struct cbk_kv_desc {
  void* k_base;
  void* v_base;
  int64_t num_blocks;
  int64_t block_size;   /* tokens per block */
  int64_t block_stride; /* bytes between blocks */
  int64_t token_stride; /* bytes between tokens of one block */
  int64_t row_bytes;    /* bytes of one token's [H, D] row */
} cbk_kv_desc;

/*
 * Paged gather: out_{k,v}[t] = {K,V}[slot_t / bs][slot_t % bs].
 * Replaces gather_paged_kv(kv_layer, slot_mapping, block_size, out)
 * (cacheblend_vllm/kv_layout.py:90-122) and the native paged-cache load it
 * dispatches to (kv_layout.py:27-87). slots_dev: int64 [num_tokens].
 * A slot outside [0, num_blocks*block_size) writes a zero row and adds one
 * to *bad_slots_dev when that pointer is non-NULL.
 */
int cbk_paged_gather(const cbk_kv_desc* kv, const int64_t* slots_dev, int64_t num_tokens,
                     void* out_k_dev, void* out_v_dev, int64_t out_token_stride,
                     int32_t* bad_slots_dev, cbk_stream_t stream);

/*
 * Paged scatter: {K,V}[slot_t / bs][slot_t % bs] = in_{k,v}[t].
 * With kv->v_base and in_v_dev both NULL only the K plane moves (also for
 * cbk_paged_gather with out_v_dev NULL); a block_size of 1 turns the
 * descriptor into a plain row table, e.g. the row write-back
 * flat_old_k[absolute_indices] = k (cacheblend_vllm/ascend.py:552, 592-593).
 * Replaces scatter_paged_kv(contiguous, kv_layer, slot_mapping, block_size)
 * (cacheblend_vllm/kv_layout.py:125-161) and reshape_and_cache
 * (kv_layout.py:137-146). Out-of-range slots are skipped and counted.
 */
int cbk_paged_scatter(const void* in_k_dev, const void* in_v_dev, int64_t in_token_stride,
                      const cbk_kv_desc* kv, const int64_t* slots_dev, int64_t num_tokens,
                      int32_t* bad_slots_dev, cbk_stream_t stream);

/*
 * Multi-layer gather in one launch per 64 layers: for layer l,
 * out + l*out_layer_stride + c*out_plane_stride + t*out_token_stride
 * receives plane c of kv[l] at slot t. All layers share the geometry of
 * kv[0] (only k_base/v_base differ). This is the whole-prompt store path of
 * CacheBlendConnectorV1.save_kv_layer/_enqueue_store_batch
 * (cacheblend_vllm/connector.py:281-447) batched over layers.
 */
int cbk_paged_gather_layers(const cbk_kv_desc* kv, int32_t num_layers, const int64_t* slots_dev,
                            int64_t num_tokens, void* out_dev, int64_t out_layer_stride,
                            int64_t out_plane_stride, int64_t out_token_stride,
                            int32_t* bad_slots_dev, cbk_stream_t stream);

/* Inverse of cbk_paged_gather_layers (batched scatter_paged_kv). */
int cbk_paged_scatter_layers(const void* in_dev, int64_t in_layer_stride, int64_t in_plane_stride,
                             int64_t in_token_stride, const cbk_kv_desc* kv, int32_t num_layers,
                             const int64_t* slots_dev, int64_t num_tokens, int32_t* bad_slots_dev,
                             cbk_stream_t stream);

/*
 * Gather straight into host chunks (the fused store path): token t of the
 * batch is written to chunk c = t / chunk_tokens, row r = t % chunk_tokens,
 * i.e. to chunk_k[c] + r * chunk_token_stride (K plane) and chunk_v[c] + ...
 * (V plane). chunk_k / chunk_v are HOST arrays of ceil(num_tokens /
 * chunk_tokens) device-addressable destinations (pinned host memory from
 * cbk_slab_alloc or hipHostMalloc, 16-byte aligned). A grid of at most
 * max_workgroups workgroups (<= 0: 64) strides over the batch: the copy is
 * host-link bound and leaves the other CUs free.
 * Replaces _enqueue_store_batch's gather + pinned D2H pair and the
 * per-layer pinned batch (cacheblend_vllm/connector.py:401-429).
 */
int cbk_paged_gather_chunks(const cbk_kv_desc* kv, const int64_t* slots_dev, int64_t num_tokens,
                            int64_t chunk_tokens, void* const* chunk_k, void* const* chunk_v,
                            int64_t chunk_token_stride, int32_t max_workgroups,
                            int32_t* bad_slots_dev, cbk_stream_t stream);

/*
 * The inverse: scatter chunk rows into the pages. Token t of the batch is
 * read from chunk c = t / chunk_tokens, row r = t % chunk_tokens (chunk_k[c]
 * + r * chunk_token_stride, chunk_v[c] + ...; HOST arrays of device-
 * addressable sources, e.g. pinned slab slots read over the host link) and
 * written to slot slots_dev[t]; tokens with an out-of-range slot are skipped
 * and counted in bad_slots_dev when non-NULL. Grid and alignment as for
 * cbk_paged_gather_chunks.
 * Replaces the reload of stored chunks: the H2D copy of the host chunk
 * (cacheblend_vllm/ascend.py:224-278) followed by scatter_paged_kv
 * (cacheblend_vllm/kv_layout.py:125-161), with no device staging.
 */
int cbk_paged_scatter_chunks(const void* const* chunk_k, const void* const* chunk_v, int64_t chunk_tokens,
                             int64_t chunk_token_stride, const cbk_kv_desc* kv, const int64_t* slots_dev,
                             int64_t num_tokens, int32_t max_workgroups, int32_t* bad_slots_dev,
                             cbk_stream_t stream);

/*
 * Pinned host chunk slab: fixed-size, 256-byte aligned slots carved from
 * pinned, coherent host arenas (hipHostMalloc) of chunks_per_arena slots,
 * recycled through a free list; max_bytes 0 = unbounded. Thread-safe.
 * Replaces the per-layer torch pinned allocation of the reference store path
 * (cacheblend_vllm/connector.py:421-426); slots hold the store's
 * [2, chunk, H, D] chunk format (connector.py:449-466).
 */
int cbk_slab_create(size_t chunk_bytes, size_t chunks_per_arena, size_t max_bytes, void** out_handle);
int cbk_slab_alloc(void* handle, void** out_chunk);
/* n slots into out_chunks[0..n): consecutive in one arena when a run of n
 * free slots exists or a new arena can hold it (n <= chunks_per_arena), so
 * one DMA copy can fill them; otherwise the lowest free slots. All or none. */
int cbk_slab_alloc_run(void* handle, int64_t n, void** out_chunks);
int cbk_slab_free(void* handle, void* chunk);
int cbk_slab_stats(void* handle, size_t* arenas, size_t* free_chunks, size_t* live_chunks);
int cbk_slab_destroy(void* handle);

/*
 * *accessible = 1 when [ptr, ptr + bytes) lies in page-locked host memory
 * that kernels can read and write at the host address (slab slots, torch
 * pinned tensors), else 0. Pageable memory is not an error. Gates the
 * host-chunk entry points (cbk_paged_gather_chunks, cbk_blend_assemble_chunks).
 */
int cbk_host_accessible(const void* ptr, size_t bytes, int* accessible);

/*
 * Up to n non-blocking side streams (*found of them) that run concurrently
 * with `serving` and with each other, measured: HIP maps streams onto a few
 * hardware queues (GPU_MAX_HW_QUEUES) round-robin in creation order, and
 * streams sharing a queue execute in order. Each of up to max_candidates new
 * streams is kept when a spin of spin_ms on it overlaps spins on `serving`
 * and on every stream kept so far. Synchronizes `serving` first. The Load,
 * copy and Store side streams of the layerwise pipelines (the reference
 * creates them with torch.npu.Stream(), cacheblend_vllm/connector.py:198-199,
 * ascend.py:212). Release with cbk_stream_destroy.
 */
int cbk_side_streams(cbk_stream_t serving, int32_t n, int32_t max_candidates, float spin_ms,
                     cbk_stream_t* out_streams, int32_t* found);
int cbk_stream_destroy(cbk_stream_t stream);

/*
 * n asynchronous copies dst[i] <- src[i] of bytes[i] bytes on `stream`
 * (direction from the addresses); the tables are host arrays and the runs
 * must not overlap. The DMA path of the layerwise loads and stores: one
 * call per layer for the pinned runs that the reference copies with one
 * non_blocking torch copy each (cacheblend_vllm/ascend.py:358-370,
 * connector.py:425-429). Consecutive runs are folded into as few DMA
 * commands as their addresses allow: runs adjacent in dst and in src into
 * one hipMemcpyAsync, runs of one size at constant dst and src pitches
 * into one hipMemcpy2DAsync. A folded command whose runs lie in different
 * allocations (addresses that only happen to line up) is rejected by the
 * runtime before anything is enqueued; its runs are then issued one by one.
 */
int cbk_memcpy_runs(const uint64_t* dst, const uint64_t* src, const uint64_t* bytes, int64_t n,
                    cbk_stream_t stream);

/*
 * The number of DMA commands cbk_memcpy_runs issues for these runs (no GPU
 * call). The loader compares bytes per command against its threshold to
 * choose DMA or in-place host reads (the reference always copies,
 * cacheblend_vllm/ascend.py:358-370).
 */
int cbk_memcpy_runs_commands(const uint64_t* dst, const uint64_t* src, const uint64_t* bytes, int64_t n,
                             int64_t* commands);

/*
 * K-deviation scores: scores[i] = sum_j (f32(fresh[i, j]) - f32(cached[r_i, j]))^2
 * over `width` elements, r_i = cached_rows_dev ? cached_rows_dev[i] : cached_row0 + i.
 * A row index outside [0, cached_num_rows) yields a NaN score (never read).
 * Replaces the inline score of Qwen3BlendExecutor._compute_layer
 * (cacheblend_vllm/ascend.py:534-538). Row strides are in elements.
 */
int cbk_kdev_scores(const void* fresh_dev, int64_t fresh_row_stride_elems, const void* cached_dev,
                    int64_t cached_row_stride_elems, int64_t cached_num_rows,
                    const int64_t* cached_rows_dev, int64_t cached_row0, int64_t n, int64_t width,
                    int32_t dtype, float* scores_dev, cbk_stream_t stream);

/* Workspace bytes cbk_select / cbk_kdev_select need for n tokens. */
size_t cbk_select_workspace_bytes(int64_t n);

/*
 * Budgeted selection: sorted int64 indices of
 *   base | top_k(scores.masked_fill(base, -inf)),
 *   base = gap | forced | dilate(gap, radius),
 *   k = budget(n, #gap, #base, ratio)   (int(cached * ratio), >= 1, <= available)
 * with ties at the k-th score going to the lower index. Writes the indices to
 * out_idx_dev[0 .. count) (capacity n) and count to *out_count_dev.
 * forced_dev may be NULL; radius 0 disables dilation.
 * Replaces Qwen3BlendExecutor._select (cacheblend_vllm/ascend.py:757-796) at
 * TP1, composed with the overflow dilation of _sparse_q_scores
 * (ascend.py:662-671) when radius > 0. Masks are uint8 (0/1).
 *
 * A count of -1 means the one-launch select gave up and wrote no index: it
 * runs every 4096-token tile in its own workgroup with grid barriers between
 * phases, launched only when the occupancy query says all the workgroups fit
 * on the device at once; workgroups of kernels on other streams can still
 * hold the CUs, and a barrier that waits about 2^22 polls for the missing
 * workgroups marks the launch failed (every workgroup then writes -1 and
 * exits). The count is device memory, so only a caller that reads it can
 * react: run cbk_select_ex with CBK_SELECT_MULTI_LAUNCH on the same scores
 * (the Python select() and kdev_select() do this). Callers that cannot read
 * it in between (graph capture) pass CBK_SELECT_MULTI_LAUNCH up front.
 */
int cbk_select(const float* scores_dev, const uint8_t* gap_dev, const uint8_t* forced_dev,
               int64_t n, int64_t radius, double ratio, int64_t* out_idx_dev,
               int64_t* out_count_dev, void* workspace_dev, size_t workspace_bytes,
               cbk_stream_t stream);

/* cbk_select_ex / cbk_kdev_select_ex flags. */
/* The five-launch select (one launch per radix phase, no grid barrier, no
 * co-residency assumption; about 25 us slower at 64K tokens): never -1. */
#define CBK_SELECT_MULTI_LAUNCH 1u
/* Tests only: the one-launch select's first barrier expects one arrival more
 * than the grid makes and polls 0 times, so every workgroup gives up at once
 * and exits normally; the count is -1. */
#define CBK_SELECT_TEST_GIVE_UP 2u

/* cbk_select with CBK_SELECT_* flags (cbk_select is flags 0). */
int cbk_select_ex(const float* scores_dev, const uint8_t* gap_dev, const uint8_t* forced_dev,
                  int64_t n, int64_t radius, double ratio, int64_t* out_idx_dev,
                  int64_t* out_count_dev, void* workspace_dev, size_t workspace_bytes,
                  uint32_t flags, cbk_stream_t stream);

/*
 * K-deviation selection in one call: cbk_kdev_scores (scores_dev receives
 * the scores) followed by cbk_select on them, with no host round trip. The
 * count follows cbk_select's contract (-1: run cbk_select_ex with
 * CBK_SELECT_MULTI_LAUNCH on scores_dev).
 */
int cbk_kdev_select(const void* fresh_dev, int64_t fresh_row_stride_elems, const void* cached_dev,
                    int64_t cached_row_stride_elems, int64_t cached_num_rows,
                    const int64_t* cached_rows_dev,
                    int64_t cached_row0, int64_t n, int64_t width, int32_t dtype,
                    const uint8_t* gap_dev, const uint8_t* forced_dev, int64_t radius,
                    double ratio, float* scores_dev, int64_t* out_idx_dev,
                    int64_t* out_count_dev, void* workspace_dev, size_t workspace_bytes,
                    cbk_stream_t stream);

/* cbk_kdev_select with CBK_SELECT_* flags (cbk_kdev_select is flags 0). */
int cbk_kdev_select_ex(const void* fresh_dev, int64_t fresh_row_stride_elems, const void* cached_dev,
                       int64_t cached_row_stride_elems, int64_t cached_num_rows,
                       const int64_t* cached_rows_dev, int64_t cached_row0, int64_t n, int64_t width,
                       int32_t dtype, const uint8_t* gap_dev, const uint8_t* forced_dev,
                       int64_t radius, double ratio, float* scores_dev, int64_t* out_idx_dev,
                       int64_t* out_count_dev, void* workspace_dev, size_t workspace_bytes,
                       uint32_t flags, cbk_stream_t stream);

/* Largest n cbk_kdev_select_noalloc accepts. */
#define CBK_NOALLOC_SELECT_MAX_TOKENS 1048576

/*
 * cbk_kdev_select without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). No counterpart in the reference. The workspace is
 * a static device array sized for CBK_NOALLOC_SELECT_MAX_TOKENS tokens
 * (5.11 MiB per GPU, held until the process ends); larger n is rejected
 * with CBK_ERR_INVALID. The caller passes every input and output. Calls
 * that overlap on one GPU (concurrent streams) race on the shared array;
 * calls in sequence do not (each clears the counters it needs). The count
 * follows cbk_select's contract: -1 (the one-launch select could not hold
 * the device) wrote no index; scores_dev is complete, so a caller that can
 * allocate selects again with cbk_select_ex(CBK_SELECT_MULTI_LAUNCH), and
 * one that cannot repeats the call once the device is less busy.
 */
int cbk_kdev_select_noalloc(const void* fresh_dev, int64_t fresh_row_stride_elems,
                            const void* cached_dev, int64_t cached_row_stride_elems,
                            int64_t cached_num_rows, const int64_t* cached_rows_dev,
                            int64_t cached_row0, int64_t n, int64_t width, int32_t dtype,
                            const uint8_t* gap_dev, const uint8_t* forced_dev, int64_t radius,
                            double ratio, float* scores_dev, int64_t* out_idx_dev,
                            int64_t* out_count_dev, cbk_stream_t stream);

/*
 * Blend-buffer assembly for one layer: out_{k,v}[p] for p in [0, num_tokens)
 * from src_map_dev[p] (int32):
 *   >= 0  hit staging row r = src_map[p]: hit_{k,v} + r * hit_token_stride;
 *         with `relocate`, the K row is RoPE-relocated from position
 *         old_pos_dev[r] to new_pos_dev[p] (new_pos_dev NULL: p) with the
 *         [rows, head_dim] cos|sin table cos_sin_dev (key dtype; neox or
 *         interleaved pairs), each op rounded to the key dtype
 *   -1    zero row (gap)
 *   -2    page row at slot slots_dev[p] of `kv` (APC prefix)
 * out_v_dev NULL processes the K plane only (standalone relocation).
 * Replaces PagedBlendLoader.prefetch's prefix gather, _zero_gaps and
 * _load_segments_fused placement (cacheblend_vllm/ascend.py:230-253,
 * 280-287, 313-370) fused with relocate_key (ascend.py:52-103).
 * Rows whose source is out of range are zeroed and counted in *bad_dev.
 */
int cbk_blend_assemble(const cbk_kv_desc* kv, const int64_t* slots_dev, const int32_t* src_map_dev,
                       int64_t num_tokens, const void* hit_k_dev, const void* hit_v_dev,
                       int64_t hit_token_stride, int64_t hit_rows, const int32_t* old_pos_dev,
                       const int32_t* new_pos_dev, const void* cos_sin_dev,
                       int64_t cos_sin_row_stride_elems, int64_t cos_sin_rows, int64_t heads,
                       int64_t head_dim, int32_t relocate, int32_t neox, int32_t dtype,
                       void* out_k_dev, void* out_v_dev, int64_t out_token_stride,
                       int32_t* bad_dev, cbk_stream_t stream);

/*
 * cbk_blend_assemble with the hit rows read directly from host chunks (the
 * fused H2D path): hit row h = src_map[p] lives in chunk c = h /
 * chunk_tokens at row h % chunk_tokens; hit_chunks_dev is a DEVICE array
 * [chunks][2] of device-addressable K / V plane addresses (pinned host
 * memory, 16-byte aligned). At most max_workgroups workgroups (<= 0:
 * enough for every row) stride over the rows. Replaces the per-segment
 * H2D copies of _load_segments_fused (cacheblend_vllm/ascend.py:333-342)
 * together with everything cbk_blend_assemble replaces.
 */
int cbk_blend_assemble_chunks(const cbk_kv_desc* kv, const int64_t* slots_dev,
                              const int32_t* src_map_dev, int64_t num_tokens,
                              const uint64_t* hit_chunks_dev, int64_t chunk_tokens,
                              int64_t chunk_token_stride, int64_t hit_rows,
                              const int32_t* old_pos_dev, const void* cos_sin_dev,
                              int64_t cos_sin_row_stride_elems, int64_t cos_sin_rows, int64_t heads,
                              int64_t head_dim, int32_t relocate, int32_t neox, int32_t dtype,
                              void* out_k_dev, void* out_v_dev, int64_t out_token_stride,
                              int32_t* bad_dev, int32_t max_workgroups, cbk_stream_t stream);

/*
 * Side-forward attention of the selected queries:
 *   out[i, h] = sum_{k <= pos_i} softmax_k( r(r(q[i, h] . key[k, h/G]) * scale) ) value[k, h/G]
 * q [nq, hq, head_dim], key/value [nk, hkv, head_dim], out [nq, hq, head_dim]
 * (row strides in elements), pos [nq] int64 in [0, nk), G = hq / hkv, r
 * rounding to the input dtype (none for float32). Replaces
 * Qwen3BlendExecutor._attention (cacheblend_vllm/ascend.py:798-846:
 * npu_fused_infer_attention_score or the einsum path) with the causal mask
 * q_pos < k_pos evaluated in the kernel. bf16/f16: head_dim 64 or 128,
 * 16-byte aligned pointers and row strides, K/V row strides < 2^24
 * elements; float32: head_dim <= 128.
 */
int cbk_blend_attention(const void* q_dev, int64_t q_row_stride_elems, const int64_t* q_pos_dev, int64_t nq,
                        const void* k_dev, int64_t k_row_stride_elems, const void* v_dev,
                        int64_t v_row_stride_elems, int64_t nk, int64_t hq, int64_t hkv, int64_t head_dim,
                        float scale, int32_t dtype, void* out_dev, int64_t out_row_stride_elems,
                        cbk_stream_t stream);

/* Workspace bytes cbk_sparse_q_scores needs: row statistics, a record per
 * 16-query tile, per-KV-head partial column sums and a dense copy of the
 * query rows (sized for head_dim 128): about nq * hq * 264 + nk * hkv * 4
 * bytes. */
size_t cbk_sparse_q_workspace_bytes(int64_t nq, int64_t nk, int64_t hq, int64_t hkv);

/*
 * Sparse-Q attention mass per key:
 *   full[k] = sum_{h < hq} sum_{i < nq, pos_i >= k}
 *             softmax_k( r(q[row_i, h, :] . key[k, h / (hq/hkv), :]) * scale )
 * with row_i = q_index_dev ? q_index_dev[i] : i, pos_i = positions_dev[row_i],
 * the softmax over all nk keys with keys k > pos_i masked, and r rounding to
 * bf16 (round_logits 1), f16 (2) or not at all (0). q is [*, hq, head_dim]
 * (row stride q_row_stride_elems), key is [nk, hkv, head_dim]. Writes
 * out_scores_dev[i] = full[out_index_dev[i]] (i < n_out; out_index NULL:
 * identity) and, when non-NULL, full_scores_dev[0 .. nk).
 * bf16/f16 run on MFMA (head_dim 64 or 128, up to 16 query heads per KV
 * head, nq <= 2^26, K row stride < 2^24 elements); f32 runs exact float32
 * dots. Deterministic (no float atomics).
 * Replaces Qwen3BlendExecutor._sparse_q_scores' score loop and its
 * index_select (cacheblend_vllm/ascend.py:683-701).
 */
int cbk_sparse_q_scores(const void* q_dev, int64_t q_row_stride_elems, const int64_t* q_index_dev,
                        int64_t nq, const int64_t* positions_dev, const void* k_dev,
                        int64_t k_row_stride_elems, int64_t nk, int64_t hq, int64_t hkv,
                        int64_t head_dim, float scale, int32_t dtype, int32_t round_logits,
                        const int64_t* out_index_dev, int64_t n_out, float* out_scores_dev,
                        float* full_scores_dev, void* workspace_dev, size_t workspace_bytes,
                        cbk_stream_t stream);

/* Largest dilation radius cbk_select / cbk_kdev_select accept. */
#define CBK_MAX_DILATION_RADIUS 4096

/*
 * forced_dev[i] = any(gap_dev[max(0, i - radius) .. min(n, i + radius + 1)))
 * Replaces the prefix-sum window of _sparse_q_scores
 * (cacheblend_vllm/ascend.py:662-671).
 */
int cbk_dilate(const uint8_t* gap_dev, int64_t n, int64_t radius, uint8_t* forced_dev,
               cbk_stream_t stream);

/* ------------------------------------------------ token-range matcher
 * Host code (no GPU calls): the scheduler-side lookup that finds stored
 * chunks at any offset of a prompt. Tokens are int64; a chunk's hash is
 * H(t_0..t_{w-1}) = sum_j (t_j + 1) * 1000003^(w-1-j) mod 2^64.
 */

/*
 * out[i] = H(tokens[i .. i + window)) for i in [0, n - window]; writes
 * nothing when n < window. O(n) rolling update.
 * Replaces rolling_hash_values (cacheblend_vllm/hashing.py:42-53).
 */
int cbk_rolling_hashes(const int64_t* tokens, int64_t n, int64_t window, uint64_t* out);

/* Creates an empty matcher of chunk_size-token records
 * (TokenRangeMatcher.__init__, cacheblend_vllm/matcher.py:25-32). */
int cbk_matcher_create(int64_t chunk_size, void** out_handle);
int cbk_matcher_destroy(void* handle);

/*
 * Registers chunk_size tokens under (scope, hash) with the caller's record
 * key; a key registered before is replaced (its old record is removed and
 * the new one appended after the others of its (scope, hash)). The hash is
 * taken as given, unchecked against the tokens.
 * Replaces TokenRangeMatcher.register (cacheblend_vllm/matcher.py:53-63).
 */
int cbk_matcher_register(void* handle, uint64_t scope, uint64_t key, uint64_t hash,
                         const int64_t* tokens);

/* Removes a key's record; unknown keys are ignored
 * (TokenRangeMatcher.unregister, cacheblend_vllm/matcher.py:65-78). */
int cbk_matcher_unregister(void* handle, uint64_t key);

/* Number of registered records (TokenRangeMatcher.__len__, matcher.py:131-133). */
int64_t cbk_matcher_size(void* handle);

/*
 * Leftmost-greedy, non-overlapping exact matches of registered chunks in
 * tokens[start .. n) for one scope: scanning window starts in increasing
 * order, a start at or after the end of the last match whose window hash is
 * registered and whose tokens equal a record's (the first such record in
 * registration order) is a match. Writes out_starts[i] (absolute start) and
 * out_keys[i] for i < *out_count; more than `capacity` matches is an error
 * (n / chunk_size + 1 is always enough).
 * Replaces TokenRangeMatcher.match (cacheblend_vllm/matcher.py:80-125).
 */
int cbk_matcher_match(void* handle, uint64_t scope, const int64_t* tokens, int64_t n,
                      int64_t start, int64_t* out_starts, uint64_t* out_keys, int64_t capacity,
                      int64_t* out_count);

#ifdef __cplusplus
}
#endif

#endif /* CACHEBLEND_HIP_H_ */
