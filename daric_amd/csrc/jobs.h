// Device-side descriptors shared by the host launchers and the kernels.
#pragma once

#include <cstdint>

namespace daric {

// Hand-over of a call's descriptors (jobs, segments, chunks, layer pointer
// tables) to its kernels. Descriptors of up to kInlineDescBytes travel inline
// in the kernel arguments (`ptr` null): no descriptor copy, no ring slot and
// no completion event, ~4 us per call on MI355X against ~9 us through the
// ring; such a launch also carries its descriptors by value, as a captured
// graph node needs. Larger sets go through the descriptor ring and `ptr`
// points at them (device memory, or the pinned host slot itself).
constexpr int kInlineDescBytes = 2816;
struct alignas(16) DescArg {
    const uint8_t* ptr;
    uint64_t reserved;
    alignas(16) uint8_t inl[kInlineDescBytes];
#ifdef __HIPCC__
    __host__ __device__
#endif
    const uint8_t* base() const { return ptr != nullptr ? ptr : inl; }
};

#ifdef __HIPCC__
// Descriptors are read-only and uniform across a workgroup: kernels address
// them in the constant address space, so they load through the scalar unit
// into SGPRs (a generic pointer would put them in VGPRs).
template <typename T>
using DescPtr = const __attribute__((address_space(4))) T*;
template <typename T>
__device__ __forceinline__ DescPtr<T> desc_at(const DescArg& d, int byte_off) {
    return (DescPtr<T>)(d.base() + byte_off);
}
// Copies one descriptor out of the constant address space, word by word.
template <typename T>
__device__ __forceinline__ T desc_load(DescPtr<T> p) {
    static_assert(sizeof(T) % 4 == 0, "descriptors are whole 32-bit words");
    T v;
    uint32_t* dst = reinterpret_cast<uint32_t*>(&v);
    const __attribute__((address_space(4))) uint32_t* src =
        reinterpret_cast<const __attribute__((address_space(4))) uint32_t*>(p);
#pragma unroll
    for (unsigned i = 0; i < sizeof(T) / 4; ++i) dst[i] = src[i];
    return v;
}
#endif

// One page-copy job: one (layer, chunk) pair, the counterpart of the
// reference's PageCopyJobDesc (csrc/cache_ops/cache_ops.h:24-36). Byte units.
// Tile t of the job (t < prefix * n_sel) is prefix index p = t / n_sel and
// selected page s = t % n_sel; its staging bytes are
// stage[(p * n_sel + s) * span, +span) and its cache bytes are
// layer[p * prefix_stride + idx[s] * page_stride, +span).
struct alignas(16) CopyJob {
    uint8_t* layer;
    uint8_t* stage;
    const int32_t* idx;
    int64_t prefix_stride;
    int64_t page_stride;
    int64_t span;
    int32_t n_sel;
    int32_t prefix;
    int32_t num_pages;        // page ids outside [1, num_pages) are skipped
    int32_t n_tokens;         // fused rotate: tokens of the job to rotate
    float delta;              // fused rotate: fp32(new_pos - old_pos)
    int32_t pad0;
};
static_assert(sizeof(CopyJob) == 80, "CopyJob layout");

// Row structure of a page span for the fused scatter + rotate kernel. The
// span is n_rows rows of W elements (rows dense, W contiguous). Rows
// [0, krows) of prefix index 0 hold K head rows: row r is token
// (r / tok_div) % PS and head h = tok_div == 1 ? (r / PS) % H : r % H.
// Elements [0, R) of a K row are rotated; everything else is copied.
struct RowGeom {
    int32_t W;         // row width in elements
    int32_t n_rows;    // rows per page span
    int32_t krows;     // K rows (prefix index 0 only)
    int32_t tok_div;   // 1 (head-major rows) or H (token-major rows)
    int32_t PS;        // tokens per page
    int32_t H;         // heads
    int32_t R;         // rotary dim
    int32_t ipr;       // work items per row
    int32_t n_rot;     // rotated items per row
    int32_t pad0;
};

// In-place rotation geometry (elements): K element (b, s, h, d) of a layer is
// at base + b*sb + s*ss + h*sh + d, d < R (reference adapter.py:312-364).
struct InplaceGeom {
    int64_t sb;
    int64_t ss;
    int64_t sh;
    int32_t PS;
    int32_t H;
    int32_t R;
    int32_t num_blocks;
    int32_t n_rot;     // rotated items per head row (lane path: rotated units per pair half)
    int32_t tile_tokens;
    int32_t upr;       // lane path: 16-byte units per K row (a power of two dividing 64)
    int32_t tok_div;   // lane path: rows per token step (H: token-major rows, 1: head-major)
    int32_t log2_parts;  // lane path: parts per page tile
    int32_t min_block;   // block ids below it are skipped: 0, or 1 to skip the null block too
};

struct RopeSeg {
    int64_t bt_offset;
    int32_t tok_start;
    int32_t n_tokens;
    float delta;
    int32_t tile_begin;   // first tile of this segment
    int32_t pad0;
    int32_t pad1;
};

// Paged K/V row geometry for the selection kernels (elements, D contiguous).
struct KVGeom {
    int64_t sb, ss, sh;     // block, slot, head strides
    int64_t v_off;          // element offset of V row relative to K row (-1: no V)
    int32_t PS, H, D, num_blocks;
};

struct SelChunk {
    int64_t bt_offset;
    int64_t row_offset;
    int32_t n_tokens;
    int32_t k;
    int32_t tile_begin;
    int32_t tok0;          // position of token 0 in the page at bt_offset (0 <= tok0 < PS)
};

}  // namespace daric
