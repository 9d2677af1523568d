// Launchers of the gfx950 kernels (defined in the .hip files).
#pragma once

#include <algorithm>
#include <mutex>

#include <hip/hip_runtime_api.h>

#include <cstdint>

#include "jobs.h"

namespace daric {

// Fast 32-bit division by a run-time constant d (n, d < 2^31):
// q = (umulhi(n, m) + n) >> s with s = ceil(log2 d), m = floor(2^32 (2^s - d) / d) + 1.
struct FastDiv {
    uint32_t d = 1, m = 1, s = 0;
    FastDiv() = default;
    explicit FastDiv(uint32_t div) : d(div) {
        s = 0;
        while ((1ull << s) < div) ++s;
        m = static_cast<uint32_t>(((1ull << 32) * ((1ull << s) - div)) / div + 1);
    }
#ifdef __HIPCC__
    __host__ __device__
#endif
    inline uint32_t div(uint32_t n) const {
        // (n * m) >> 32 lowers to v_mul_hi_u32 on the device.
        const uint32_t hi = static_cast<uint32_t>((static_cast<uint64_t>(n) * m) >> 32);
        return (hi + n) >> s;
    }
};

struct RowGeomDiv {
    RowGeom g;
    FastDiv ipr, tok_div, ps;
};

// Layer-minor block order for kernels over (layer, work item) pairs: block b
// of a launch takes layer l0 + b % nl and work item w0 + b / nl. Workgroups
// are dispatched to the 8 XCDs in turn, so with nl a multiple of 8 each XCD
// works on a fixed eighth of the layers, and its address translations and L2
// see an eighth of the layers' memory. On MI355X that made the row merge 8-12%
// faster, the fused top-k + merge 5-7% and the in-place re-rotation 4-10%
// than work-item-major grids (in same-process A/Bs at configs 2, 3 and 5);
// the deviation kernel, which streams each layer's rows in order, ran 4-5%
// slower that way and keeps its tile-major grid.
struct LayerMinor {
    int32_t l0 = 0;     // first layer of the launch
    int32_t nl = 1;     // layers of the launch
    int64_t w0 = 0;     // first work item of the launch
    // (layer, work item) of block b of the launch
#ifdef __HIPCC__
    __host__ __device__
#endif
    inline void at_block(uint32_t b, int& l, int64_t& w) const {
        const uint32_t n = static_cast<uint32_t>(nl);
        l = l0 + static_cast<int>(b % n);
        w = w0 + static_cast<int64_t>(b / n);
    }
#ifdef __HIPCC__
    __device__ inline void at(int& l, int64_t& w) const { at_block(blockIdx.x, l, w); }
#endif
};

// Largest grid.x of a 256-lane launch (grid.x * 256 lanes < 2^32).
constexpr int64_t kMaxGridBlocks = (1ll << 24) - 1;

// Calls launch(LayerMinor, blocks) for launches that together cover
// n_layers x n_items, each of at most kMaxGridBlocks blocks.
template <class F>
void for_layer_minor(int n_layers, int64_t n_items, F&& launch) {
    if (n_layers <= 0 || n_items <= 0) return;
    const int64_t nl = std::min<int64_t>(n_layers, kMaxGridBlocks);
    const int64_t per = std::max<int64_t>(1, kMaxGridBlocks / nl);
    for (int64_t l0 = 0; l0 < n_layers; l0 += nl) {
        LayerMinor lm;
        lm.l0 = static_cast<int32_t>(l0);
        lm.nl = static_cast<int32_t>(std::min<int64_t>(nl, n_layers - l0));
        for (int64_t w0 = 0; w0 < n_items; w0 += per) {
            lm.w0 = w0;
            const int64_t ni = std::min<int64_t>(per, n_items - w0);
            launch(lm, static_cast<unsigned>(lm.nl * ni));
        }
    }
}

// XCD-aware unit order for grids whose consecutive units write consecutive
// bytes (the gathers: staging is the contiguous side). Workgroups are
// dispatched to the 8 XCDs round-robin, so with a grid row length divisible
// by 8, unit u runs on XCD u % 8 and neighbouring parts of the staging side
// would be written from different XCDs. map() permutes [0, full) so that XCD
// x's i-th unit becomes unit (i / run * 8 + x) * run + i % run: each XCD
// writes runs of `run` consecutive units. Runs of ~256 KiB measured fastest
// on MI355X (gathers 1-3% faster than the plain order); runs of 32-64 KiB
// were slower than the plain order. Units past `full` keep their place.
struct XcdRuns {
    static constexpr int kXcds = 8;
    static constexpr int64_t kRunBytes = 256 * 1024;
    int32_t log2_run = 0;   // 0: identity
    int32_t full = 0;
    XcdRuns() = default;
    XcdRuns(int64_t grid_x, int64_t unit_bytes) {
        if (grid_x % kXcds != 0 || unit_bytes <= 0) return;
        while (log2_run < 10 && (unit_bytes << (log2_run + 1)) <= kRunBytes) ++log2_run;
        const int64_t group = static_cast<int64_t>(kXcds) << log2_run;
        full = static_cast<int32_t>(grid_x / group * group);
    }
#ifdef __HIPCC__
    __host__ __device__
#endif
    inline int map(int u) const {
        if (log2_run == 0 || u >= full) return u;
        const int i = u >> 3, x = u & 7;
        return ((((i >> log2_run) << 3) + x) << log2_run) + (i & ((1 << log2_run) - 1));
    }
};

// One token-major copy job: the pages idx[0 .. n_sel) of one layer to or from
// staging laid out as [n_kv][n_sel * PS][H][row_bytes] (K rows, then V rows).
// A workgroup moves one part: part_tokens consecutive tokens (all heads) of
// one page and one of K or V. Byte units.
struct alignas(16) TokenJob {
    uint8_t* layer;          // K element [0, ..., 0] of the layer
    uint8_t* stage;          // first byte of the job's staging range
    const int32_t* idx;      // page ids; ids outside [1, num_blocks) are skipped
    int64_t sb, ss, sh;      // page, token and head strides
    int64_t v_off;           // V plane relative to K (n_kv == 2)
    int32_t n_sel;
    int32_t num_blocks;
    int32_t PS;
    int32_t H;
    int32_t row_bytes;       // D * element size
    int32_t n_kv;            // 2, or 1 for a cache without V (MLA)
    int32_t part_tokens;
    int32_t parts_per_page;  // ceil(PS / part_tokens)
    FastDiv d_upr;           // row_bytes / access width
    FastDiv d_h;             // H
};
static_assert(sizeof(TokenJob) == 112, "TokenJob layout");

// Token-major gather (staging <- cache) or scatter; lds selects the
// LDS-staged transpose for head-major pages ([H, PS, D] dense); vw is 16 or 1.
// part_bytes: the largest part's staging bytes (sets the XCD run length).
void launch_token_copy(const DescArg& d, int n_jobs, int max_parts, int64_t part_bytes, int vw,
                       bool lds, bool gather, hipStream_t stream);

// Plain page copies of the n_jobs CopyJobs in `d`. vw is the access width in
// bytes (16, 4 or 1); max_span
// is the largest page span (bytes) of the jobs.
void launch_copy_pages(const DescArg& d, int n_jobs, int max_tiles, int64_t max_span, int vw,
                       bool gather, hipStream_t stream);

// Fused scatter + K re-rotation of the n_jobs CopyJobs in `d`; kind is an
// ElemKind. All jobs share `geom`.
void launch_scatter_rotate(const DescArg& d, int n_jobs, int max_tiles,
                           const RowGeomDiv& geom, int kind, bool neox, const float* inv_freq,
                           hipStream_t stream);

// In-place K re-rotation over segments of tokens. `d` holds the n_segs
// RopeSegs, then (at byte layer_off) the n_layers K base pointers. `path`:
// kRotElem (per-element access), kRotVec (16-byte items, tiles of
// g.tile_tokens tokens) or kRotLane (one tile per page of dense K rows, see
// rerotate_lane_kernel). fp8 codes are rotated as stored (a per-head scale
// cancels in a linear rotation).
enum RotPath { kRotElem = 0, kRotVec = 1, kRotLane = 2 };
void launch_rerotate_inplace(const DescArg& d, int layer_off, int n_layers, const InplaceGeom& g,
                             int n_segs, int n_tiles, const int32_t* block_table,
                             const float* inv_freq, int kind, bool neox, int path, hipStream_t stream);

// Selection kernels. deviation_tile_tokens: tokens per deviation workgroup
// (the tiling launch_deviation expects in SelChunk::tile_begin).
int deviation_tile_tokens(int cache_kind);
// Selection launchers: `d` holds the n_chunks SelChunks, then (deviation and
// merge, at byte layer_off) the n_layers layer base pointers.
void launch_deviation(const DescArg& d, int layer_off, int n_layers, const KVGeom& g, int cache_kind,
                      const int32_t* block_table, const uint8_t* k_new, int new_kind,
                      int64_t T, int n_chunks, int n_tiles,
                      const float* k_scales, float* keys, hipStream_t stream);
void launch_topk(const float* keys, int n_layers, int64_t T, const DescArg& d,
                 int n_chunks, int max_tokens, int32_t* out_idx, int kmax, hipStream_t stream);
// merge: quant_from is -1 (rows are copied as bytes) or the ElemKind of
// bf16 / fp16 rows quantised into an e4m3 cache with the [n_layers, H] fp32
// k_scales / v_scales. merge_fits_rows: whether the row kernel takes the
// geometry (required for quantising); merge_max_row_bytes: the most bytes of
// recomputed K+V values per token it takes.
bool merge_fits_rows(const KVGeom& g, int elem_size, bool quant);
int64_t merge_max_row_bytes();
void launch_merge(const DescArg& d, int layer_off, int n_layers, const KVGeom& g, int elem_size,
                  const int32_t* block_table, const uint8_t* k_new, const uint8_t* v_new,
                  int64_t T, int n_chunks, const int32_t* sel_idx, int kmax, int quant_from,
                  const float* k_scales, const float* v_scales, hipStream_t stream);
// Fused selection, one workgroup per (layer, chunk): top-k on the chunk's
// keys held in LDS and the merge of its selected rows, with (with_keys) or
// without (keys already hold them) the chunk's deviation keys computed first
// in the same workgroup. select_merge_fits: whether it takes the geometry and
// chunk sizes, and (unless one_pass) whether a chunk's selected rows are few
// enough for one workgroup to merge faster than the merge kernel (else the
// three launches above do the same work).
bool select_merge_fits(const KVGeom& g, int elem_size, bool quant, int64_t max_tokens, int64_t kmax,
                       bool one_pass);
void launch_select_merge(const DescArg& d, int layer_off, int n_layers, const KVGeom& g, int cache_kind,
                         int elem_size, const int32_t* block_table, const uint8_t* k_new, int new_kind,
                         const uint8_t* v_new, int64_t T, int n_chunks, int max_tokens, bool with_keys,
                         float* keys, int32_t* sel_idx, int kmax, bool quant, const float* k_scales,
                         const float* v_scales, hipStream_t stream);

// Copies n16 16-byte units from host-pinned `src` to device `dst` on `stream`
// (descriptor upload; both 16-byte aligned).
void launch_upload(const void* src, void* dst, size_t n16, hipStream_t stream);

// Allocation-free descriptor staging (noalloc.hip). Each GPU holds a static
// device array of kNoAllocScratchBytes; noalloc_scratch returns its address on
// `device` (looked up once per device). stash_descriptors enqueues kernels on
// `stream` that write `bytes` (a multiple of 16) from host memory `src` to
// `dst` in that array, carrying them in their kernel arguments.
constexpr size_t kNoAllocScratchBytes = 256 * 1024;
uint8_t* noalloc_scratch(int device);
void stash_descriptors(const void* src, size_t bytes, uint8_t* dst, hipStream_t stream);

// One call's use of a GPU's scratch array. The constructor takes the device's
// call lock and, when the previous eager call used another stream, makes
// `stream` wait for that call's last kernel; finish() is called after the
// call's last launch that reads the array and records the device's event on
// `stream`. Under stream capture neither the wait nor the record is made.
struct ScratchState;
class ScratchUse {
public:
    ScratchUse(int device, hipStream_t stream);
    // A call that stops before finish() (an error after some of its kernels
    // were enqueued) still records the event, so that later calls order
    // after whatever it enqueued.
    ~ScratchUse();
    ScratchUse(const ScratchUse&) = delete;
    ScratchUse& operator=(const ScratchUse&) = delete;
    uint8_t* ptr() const;
    void finish();

private:
    ScratchState* state_;
    hipStream_t stream_;
    std::unique_lock<std::mutex> lock_;
    bool capture_ = false;
    bool finished_ = false;
};
// Cross-stream waits ScratchUse has enqueued since the library was loaded.
int64_t scratch_stream_waits();

// Launch-configuration error check after a <<<>>> launch.
void check_launch(const char* what);

}  // namespace daric
