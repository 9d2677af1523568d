// Launchers of the gfx950 kernels (defined in the .hip files).
#pragma once

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
void launch_token_copy(const DescArg& d, int n_jobs, int max_parts, int vw, bool lds,
                       bool gather, hipStream_t stream);

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
// RopeSegs, then (at byte layer_off) the n_layers K base pointers; `vec`
// selects 16-byte (true) or per-element (false) access. fp8 codes are
// rotated as stored (a per-head scale cancels in a linear rotation).
void launch_rerotate_inplace(const DescArg& d, int layer_off, int n_layers, const InplaceGeom& g,
                             int n_segs, int n_tiles, const int32_t* block_table,
                             const float* inv_freq, int kind, bool neox, bool vec, hipStream_t stream);

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
void launch_merge(const DescArg& d, int layer_off, int n_layers, const KVGeom& g, int elem_size,
                  const int32_t* block_table, const uint8_t* k_new, const uint8_t* v_new,
                  int64_t T, int n_chunks, const int32_t* sel_idx, int kmax, hipStream_t stream);

// Copies n16 16-byte units from host-pinned `src` to device `dst` on `stream`
// (descriptor upload; both 16-byte aligned).
void launch_upload(const void* src, void* dst, size_t n16, hipStream_t stream);

// Launch-configuration error check after a <<<>>> launch.
void check_launch(const char* what);

}  // namespace daric
