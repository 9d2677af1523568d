/*
 * daric_cache_ops.h -- C ABI of the MI355X (gfx950) KV-reuse hot path.
 *
 * This library replaces the reference's pybind11 module `daric.cache_ops`
 * (reference: csrc/cache_ops/bindings.cpp:7-31, stub daric/cache_ops.pyi:1-53)
 * and the Triton re-rotation kernel (daric/adaption/adapter.py:30-88), and adds
 * the entry points the reference lacks (fused scatter+re-rotate, fp8
 * dequant->rotate->requant, recompute selection and merge).
 *
 * Conventions
 *  - Every function returns DARIC_OK (0) or a non-zero status; the message of
 *    the last failure on the calling thread is returned by daric_last_error().
 *  - Tensors cross the boundary as `daric_tensor` views: a data pointer plus
 *    sizes/strides in elements, the element size and the device ordinal.
 *    No torch type appears in any signature.
 *  - `stream` is a raw hipStream_t cast to uint64_t. 0 means the HIP null
 *    stream; the Python layer resolves the reference's "0 = current torch
 *    stream" rule (reference csrc/cache_ops/copier.cpp:27-30) before calling.
 *  - All device work is asynchronous on `stream`. Nothing here synchronises,
 *    except where a function says so.
 *  - Host-side validation happens before any device work, so a failing call
 *    leaves device memory untouched.
 *  - A call whose job descriptors fit in 2816 bytes passes them in the kernel
 *    arguments and enqueues only kernels, so it may be recorded by a HIP
 *    stream capture. A larger call stages them in a per-device ring of pinned
 *    slots and returns DARIC_ERR_INVALID while `stream` is capturing, except
 *    daric_copier_scatter_pages_rerotate_noalloc, which stages them in a
 *    static device array and may be captured.
 */
#ifndef DARIC_CACHE_OPS_H
#define DARIC_CACHE_OPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DARIC_ABI_VERSION 5

/* Status codes. */
#define DARIC_OK 0
#define DARIC_ERR_INVALID 1   /* argument validation failed (reference: TORCH_CHECK) */
#define DARIC_ERR_RUNTIME 2   /* std::runtime_error in the reference (e.g. byte_size mismatch) */
#define DARIC_ERR_HIP 3       /* a HIP runtime call failed */
#define DARIC_ERR_NOMEM 4     /* host allocation failed */
#define DARIC_ERR_VALUE 5     /* a cache layout the rotation does not accept (reference: ValueError,
                                 daric/adaption/adapter.py:20-27, 336-368) */

/* Element type codes carried by daric_tensor.dtype. */
#define DARIC_DTYPE_UINT8 0
#define DARIC_DTYPE_INT32 1
#define DARIC_DTYPE_INT64 2
#define DARIC_DTYPE_FLOAT16 3
#define DARIC_DTYPE_BFLOAT16 4
#define DARIC_DTYPE_FLOAT32 5
#define DARIC_DTYPE_FP8_E4M3FN 6 /* OCP e4m3 (finite, NaN = 0x7F/0xFF); a uint8 cache is read as this */
#define DARIC_DTYPE_OTHER 15

#define DARIC_MAX_DIMS 8

/* A strided tensor view. `data` is the address of element [0,...,0];
 * `device` is the HIP device ordinal, or -1 for host memory. */
typedef struct daric_tensor {
    void* data;
    int32_t ndim;
    int32_t elem_size;
    int32_t device;
    int32_t dtype;
    int64_t sizes[DARIC_MAX_DIMS];
    int64_t strides[DARIC_MAX_DIMS];
} daric_tensor;

/* Rotary parameters for every re-rotation entry point.
 *  inv_freq   : device fp32 array of rotary_dim/2 inverse frequencies; the
 *               angle of pair i for a shift of d positions is the fp32 product
 *               (float)d * inv_freq[i].
 *  rotary_dim : number of rotated dims at the start of each K head row (even).
 *  is_neox    : 1 pairs (i, i + rotary_dim/2); 0 pairs (2i, 2i+1) (GPT-J).
 * Same meaning as vLLM RotaryEmbedding.rotary_dim / is_neox_style consumed at
 * reference daric/adaption/adapter.py:176-194, 270-295, 378-396. */
typedef struct daric_rope {
    const float* inv_freq;
    int32_t rotary_dim;
    int32_t is_neox;
} daric_rope;

/* ---------------------------------------------------------------------- */
/* Library                                                                 */
/* ---------------------------------------------------------------------- */

int daric_abi_version(void);
const char* daric_last_error(void);

/* Kernel timing: when enabled, every kernel this library launches carries a
 * start/stop HIP event pair in its dispatch (hipExtLaunchKernel), so the pair
 * brackets the kernel's execution on its launch stream. daric_timing_read
 * synchronises those events and returns the summed kernel time (ms) and the
 * number of launches since the last read (or enable), then resets them.
 * This has no counterpart in the reference; it exists for measurement. */
int daric_timing_enable(int enable);
int daric_timing_read(double* total_ms, int64_t* launches);

/* Host-side counters since the library was loaded, for tests and monitoring
 * (any pointer may be NULL): descriptor_uploads counts descriptor sets handed
 * to the per-device descriptor ring (each copies into a pinned slot),
 * ring_allocations the pinned/device buffer pairs the ring has allocated, and
 * scratch_waits the cross-stream waits the allocation-free entry point has
 * enqueued to order its calls on a GPU's scratch array. No counterpart in
 * the reference. */
int daric_debug_counters(int64_t* descriptor_uploads, int64_t* ring_allocations,
                         int64_t* scratch_waits);

/* ---------------------------------------------------------------------- */
/* CacheCopier: reference csrc/cache_ops/cache_ops.h:91-125, copier.cpp   */
/* ---------------------------------------------------------------------- */

typedef struct daric_copier daric_copier;

/* CacheCopier.__init__ (reference bindings.cpp:10-11). */
int daric_copier_create(daric_copier** out);
int daric_copier_destroy(daric_copier* copier);

/* CacheCopier.register_layer (reference copier.cpp:7-11): the tensor must be
 * on a device; a second registration of `name` replaces the first. */
int daric_copier_register_layer(daric_copier* copier, const char* name,
                                const daric_tensor* tensor, int is_page_first);

/* CacheCopier.register_store (reference copier.cpp:13-25): 1-D contiguous
 * uint8 device buffer. Offsets of gather/scatter jobs are relative to it. */
int daric_copier_register_store(daric_copier* copier, const daric_tensor* buffer);

/* Per-layer fp32 K scales for an fp8 (e4m3) layer: `k_scale` is a device
 * array of at least H positive floats (one per KV head), checked when a fused
 * job uses the layer. They do not change the result: the rotation is linear,
 * so a per-head scale cancels and the stored codes are rotated directly, as
 * the reference rotates the raw fp8 values (adapter.py:370-373).
 * No counterpart in the reference (it has no scaled fp8 path). */
int daric_copier_register_k_scale(daric_copier* copier, const char* name,
                                  const daric_tensor* k_scale);

/* CacheCopier.gather_pages (reference copier.cpp:41-76, kernels.cu:52-84,
 * 127-217): for job i, copy the selected pages of layer `layer_names[i]` into
 * the store at offsets[i], laid out [prefix][n_sel][page span bytes]. Pages
 * whose block id is 0 are skipped and their store bytes left untouched.
 * `indices_flat` is a 1-D contiguous int32 device tensor; job i uses
 * indices_flat[indices_offsets[i] : indices_offsets[i+1]]. The n_* arguments
 * are the lengths of the arrays that follow the reference's Python lists
 * (offsets, byte_sizes, indices_offsets); mismatches are reported in the
 * reference's order (helpers.cu:156-158). */
int daric_copier_gather_pages(daric_copier* copier, const char* const* layer_names,
                              int64_t n_jobs, const int64_t* offsets, int64_t n_offsets,
                              const int64_t* byte_sizes, int64_t n_byte_sizes,
                              const daric_tensor* indices_flat,
                              const int64_t* indices_offsets,
                              int64_t n_indices_offsets, uint64_t stream);

/* CacheCopier.scatter_pages (reference copier.cpp:78-111, kernels.cu:86-123,
 * 219-292): inverse of gather_pages, block id 0 skipped. */
int daric_copier_scatter_pages(daric_copier* copier, const char* const* layer_names,
                               int64_t n_jobs, const int64_t* offsets, int64_t n_offsets,
                               const int64_t* byte_sizes, int64_t n_byte_sizes,
                               const daric_tensor* indices_flat,
                               const int64_t* indices_offsets,
                               int64_t n_indices_offsets, uint64_t stream);

/* Fused load path: scatter_pages plus the re-rotation the reference applies
 * afterwards in the worker (adapter.py:196-295), in one pass over the bytes.
 * Job i rotates the K rows of its first num_tokens[i] tokens (token j is slot
 * j % PS of page j / PS of the job) by deltas[i] positions; V rows, rotary
 * tails and tokens >= num_tokens[i] are copied unchanged. For an fp8 layer
 * the e4m3 codes are decoded, rotated in fp32 and re-encoded (saturating
 * round-to-nearest-even); a per-head scale would cancel, see
 * daric_copier_register_k_scale. The one-pass kernel needs 16-byte aligned
 * pages, strides and store offsets, K head rows dense in the page span and
 * rotated halves that are 16-byte multiples; for any other layout accepted
 * by the copy and rotation checks, the call scatters with the copy kernel and
 * then rotates the moved tokens in place (pages with id 0 skipped by both),
 * to the same results up to the rotation's rounding. (A page listed by two
 * jobs of one call is written twice, a race on either path; on the two-pass
 * path it is also rotated once per listing.)
 * New entry point; no counterpart in the reference (which scatters in the
 * store process and rotates later in the worker process). */
int daric_copier_scatter_pages_rerotate(daric_copier* copier,
                                        const char* const* layer_names, int64_t n_jobs,
                                        const int64_t* offsets, int64_t n_offsets,
                                        const int64_t* byte_sizes, int64_t n_byte_sizes,
                                        const daric_tensor* indices_flat,
                                        const int64_t* indices_offsets,
                                        int64_t n_indices_offsets,
                                        const int64_t* deltas, const int64_t* num_tokens,
                                        const daric_rope* rope, uint64_t stream);

/* Allocation-free variant of daric_copier_scatter_pages_rerotate: the same
 * arguments, checks, kernels and results. No counterpart in the reference;
 * it is for callers that cannot allocate: code under HIP stream capture,
 * serving loops with a fixed memory budget, harnesses that forbid hipMalloc.
 * Where daric_copier_scatter_pages_rerotate stages a job list too large for
 * the kernel arguments in its descriptor ring (pinned host and device memory
 * that it allocates on first use), this entry point stages it in a static
 * device array of 262144 bytes per GPU (3276 jobs of 80 bytes), carried there
 * by kernels whose arguments hold the bytes. It calls no hipMalloc, hipFree
 * or hipHostMalloc and enqueues only kernels (plus, for staged job lists,
 * one event record, and a stream wait when the stream changes; the event is
 * created once per GPU, with the array's address, at the first staging call).
 * A call whose jobs need more than the array holds, or whose layout needs the
 * scatter-then-rotate form, returns DARIC_ERR_INVALID before any device work.
 * Every call on one GPU uses that GPU's array, which keeps the last call's
 * descriptors. Eager calls are ordered on it by the library: a call on
 * another stream than the previous staging call waits for that call's
 * kernels before it overwrites the array, and calls from different host
 * threads enqueue one at a time. Calls recorded under stream capture add no
 * such ordering: a graph replay that overlaps another call on the same GPU
 * races on the array, and the caller must order those. */
int daric_copier_scatter_pages_rerotate_noalloc(daric_copier* copier,
                                                const char* const* layer_names, int64_t n_jobs,
                                                const int64_t* offsets, int64_t n_offsets,
                                                const int64_t* byte_sizes, int64_t n_byte_sizes,
                                                const daric_tensor* indices_flat,
                                                const int64_t* indices_offsets,
                                                int64_t n_indices_offsets,
                                                const int64_t* deltas, const int64_t* num_tokens,
                                                const daric_rope* rope, uint64_t stream);

/* Token-major gather: like gather_pages, but job i's store range holds the
 * selected pages' rows token by token, [n_kv][n_sel * PS][H][D] (K rows, then
 * V rows; n_kv = 1 for a 3-D MLA cache), whatever the cache layout: NHD
 * [2, NB, PS, H, D], HND (the same with H and PS swapped in memory),
 * page-first [NB, 2, PS, H, D], packed [NB, H, PS, 2D] or MLA [NB, PS, hidden].
 * byte_sizes[i] must equal n_kv * n_sel * PS * H * D * element size. Pages
 * whose id is 0 or outside [1, num_blocks) are skipped and their rows of the
 * store left untouched. Same argument checks, in the same order, as
 * gather_pages. No counterpart in the reference, whose staging is the
 * physical page span (kernels.cu:20-44): token-major for NHD pages only. */
int daric_copier_gather_tokens(daric_copier* copier, const char* const* layer_names,
                               int64_t n_jobs, const int64_t* offsets, int64_t n_offsets,
                               const int64_t* byte_sizes, int64_t n_byte_sizes,
                               const daric_tensor* indices_flat,
                               const int64_t* indices_offsets,
                               int64_t n_indices_offsets, uint64_t stream);

/* Token-major scatter: inverse of daric_copier_gather_tokens; skipped pages
 * are not written. No counterpart in the reference. */
int daric_copier_scatter_tokens(daric_copier* copier, const char* const* layer_names,
                                int64_t n_jobs, const int64_t* offsets, int64_t n_offsets,
                                const int64_t* byte_sizes, int64_t n_byte_sizes,
                                const daric_tensor* indices_flat,
                                const int64_t* indices_offsets,
                                int64_t n_indices_offsets, uint64_t stream);

/* batched_memcpy_d2h / batched_memcpy_h2d (reference helpers.cu:187-248):
 * one hipMemcpyAsync per region on `stream`. */
int daric_batched_memcpy_d2h(const daric_tensor* staging, const daric_tensor* shm,
                             const int64_t* stg_offsets, const int64_t* shm_offsets,
                             const int64_t* sizes, int64_t n, uint64_t stream);
int daric_batched_memcpy_h2d(const daric_tensor* shm, const daric_tensor* staging,
                             const int64_t* shm_offsets, const int64_t* stg_offsets,
                             const int64_t* sizes, int64_t n, uint64_t stream);

/* ---------------------------------------------------------------------- */
/* In-place re-rotation: replaces _fused_rerotate_kernel and               */
/* Adapter._launch_triton_rerotate (reference adapter.py:30-88, 297-396).  */
/* ---------------------------------------------------------------------- */

/* A run of consecutive tokens that move by the same number of positions.
 * Token j of the run (0 <= j < n_tokens) is position p = tok_start + j of the
 * block list block_table[bt_offset ...]; its slot is
 * block_table[bt_offset + p / PS] * PS + p % PS (reference adapter.py:164-170,
 * 258-264). */
typedef struct daric_rope_segment {
    int64_t bt_offset;
    int64_t tok_start;
    int64_t n_tokens;
    int64_t delta;
} daric_rope_segment;

/* Rotate, in place, the K rows of every listed token in every layer of
 * `layers` (all with the same shape, strides and dtype; page_first as in
 * reference adapter.py:311-368). `k_scales` is NULL or an [n_layers, H] fp32
 * device tensor of positive per-head scales for fp8 layers; it is checked but
 * does not change the result: the rotation is linear, so the stored codes are
 * rotated directly (rot(q * s) / s = rot(q)), as the reference's kernel
 * rotates the raw fp8 values (adapter.py:30-88). `block_table` is a 1-D
 * contiguous int32 device tensor. Every slot must be listed at most once
 * across the segments: workgroups rotate their tokens concurrently, so a
 * repeated slot gets an unspecified result (one program per token races the
 * same way in the reference). */
int daric_rerotate_pages(const daric_tensor* layers, int64_t n_layers, int page_first,
                         const daric_tensor* block_table,
                         const daric_rope_segment* segments, int64_t n_segments,
                         const daric_rope* rope, const daric_tensor* k_scales,
                         uint64_t stream);

/* ---------------------------------------------------------------------- */
/* Recompute selection (no reference kernel; the reference's budget is     */
/* the positional DARICPolicy, daric/adaption/policy.py:45-103).           */
/* ---------------------------------------------------------------------- */

/* A chunk of consecutive tokens of one request: token j (0 <= j < n_tokens)
 * is token p = tok_start + j of the block list that begins at
 * block_table[bt_offset], so it lives at slot
 * block_table[bt_offset + p / PS] * PS + p % PS of the paged cache, and at
 * row row_offset + j of the contiguous recomputed tensors. `k` is the number
 * of tokens to select in it. tok_start lets a chunk begin inside a page, as
 * the groups of a request do (group i of the reference's group_ptr starts at
 * token group_ptr[i] - group_ptr[0] of the request's blocks,
 * daric/adaption/adapter.py:127-171). */
typedef struct daric_chunk {
    int64_t bt_offset;
    int64_t row_offset;
    int64_t n_tokens;
    int64_t k;
    int64_t tok_start;
} daric_chunk;

/* keys[l, row_offset + j] = sum over (h, d) of (k_new[l, row, h, d] - K_cache)^2
 * in fp32, in the fixed order documented in daric_amd/csrc/select_kernels.hip.
 * layers: n_layers paged caches (same geometry); k_new: [n_layers, T, H, D]
 * contiguous, bf16 or fp16; keys: [n_layers, T] fp32 contiguous. For an fp8
 * (e4m3) cache, k_scales is NULL (scale 1) or an [n_layers, H] fp32 device
 * tensor: cached K is dequantised as float32(code value * scale[l, h]). A
 * token whose block id lies outside [0, num_blocks) is not read and gets
 * key 0. Rows of keys outside every chunk are not written. */
int daric_kv_deviation(const daric_tensor* layers, int64_t n_layers, int page_first,
                       const daric_tensor* block_table, const daric_tensor* k_new,
                       const daric_chunk* chunks, int64_t n_chunks,
                       const daric_tensor* k_scales, daric_tensor* keys, uint64_t stream);

/* For every (layer, chunk) select the chunk's k tokens with the largest keys
 * (ties: lower token index first) and write their chunk-local token indices
 * in ascending order to out_idx[l, c, 0:k]; slots k..kmax-1 are set to -1.
 * keys: [n_layers, T] fp32; out_idx: [n_layers, n_chunks, kmax] int32.
 * Chunks of any length: keys of chunks up to 8192 tokens are staged in LDS,
 * longer chunks are read from global memory in each radix pass. */
int daric_topk_per_chunk(const daric_tensor* keys, const daric_chunk* chunks,
                         int64_t n_chunks, daric_tensor* out_idx, uint64_t stream);

/* Write the selected rows of k_new / v_new ([n_layers, T, H, D]) into the K
 * and V rows of their slots in the paged caches: the counterpart of the write
 * vLLM's reshape_and_cache makes for the reference's recompute sub-requests
 * (daric/integration/vllm/worker.py:336-345, utils.py:406-427). sel_idx is
 * the output of daric_topk_per_chunk (entries < 0 are ignored); slots in
 * block 0 are skipped like the reference's copy kernels skip block 0.
 * Rows in the cache's element type are copied as bytes (k_scales and v_scales
 * NULL). bfloat16 / float16 rows for an fp8 (e4m3) cache are quantised:
 * code = saturating round-to-nearest-even e4m3 of float32(x) / scale, the
 * division correctly rounded, with scale = k_scales[l, h] for K rows and
 * v_scales[l, h] for V rows (contiguous [n_layers, H] fp32 device tensors of
 * positive, finite values). */
int daric_merge_rows(const daric_tensor* layers, int64_t n_layers, int page_first,
                     const daric_tensor* block_table, const daric_tensor* k_new,
                     const daric_tensor* v_new, const daric_chunk* chunks,
                     int64_t n_chunks, const daric_tensor* sel_idx,
                     const daric_tensor* k_scales, const daric_tensor* v_scales,
                     uint64_t stream);

/* The whole recompute selection in one call: daric_kv_deviation (unless
 * flags has DARIC_SELECT_KEYS_READY: keys already hold the keys), then
 * daric_topk_per_chunk into sel_idx, then daric_merge_rows of the selected
 * rows, with the same arguments, checks and results (keys, sel_idx and the
 * merged cache bytes equal those of the three calls). For an fp8 (e4m3)
 * cache, k_scales are the cache's per-(layer, head) K scales (they
 * dequantise the cached K for the keys and quantise the merged K rows) and
 * v_scales the V scales; k_new and v_new are bfloat16 or float16 rows. Other
 * caches take rows of their own type and NULL scales.
 * Where every chunk has at most 8192 tokens, its keys and kmax row slots fit
 * in 48 KiB of LDS, the merge kernel takes the rows, and kmax selected K and
 * V rows make at most 12 rounds of 2048 16-byte units (e.g. 77 of 512 rows
 * of 8 x 128 bf16, not 205 of 2048): the keys come from the deviation
 * kernel, then one workgroup per (layer, chunk) runs the chunk's top-k on
 * its keys in LDS and merges the selected rows, with no index round trip
 * through memory (one workgroup walking more rounds measured slower than the
 * merge kernel's spread). DARIC_SELECT_ONE_PASS computes the keys
 * in that workgroup too (one launch; it measured 4-7% slower on MI355X at
 * the Llama-3-8B and -70B selection workloads, and is kept for measurement;
 * it lifts the 12-round limit). Other calls run the three kernels in turn.
 * New entry point; no counterpart in the reference. */
#define DARIC_SELECT_KEYS_READY 1
#define DARIC_SELECT_ONE_PASS 2
int daric_select_merge(const daric_tensor* layers, int64_t n_layers, int page_first,
                       const daric_tensor* block_table, const daric_tensor* k_new,
                       const daric_tensor* v_new, const daric_chunk* chunks, int64_t n_chunks,
                       const daric_tensor* k_scales, const daric_tensor* v_scales,
                       daric_tensor* keys, daric_tensor* sel_idx, int flags, uint64_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DARIC_CACHE_OPS_H */
