// Token-major copies between a paged KV cache and staging (gfx950).
//
// The reference stages the physical page span (csrc/cache_ops/kernels.cu:
// 20-44), which is token-major only for vLLM's [.., PS, H, D] pages. These
// kernels produce (gather) or consume (scatter) [n_kv][tokens][H][D] for any
// cache layout -- NHD, HND ([.., H, PS, D]), page-first, packed [NB, H, PS, 2D]
// and MLA -- so a caller gets the canonical [L, 2, T, H, D] rows whatever the
// layout.
//
// A workgroup moves one part: part_tokens tokens x all heads of one page's K
// or V plane. Two kernels:
//
//  * token_rows_kernel: unit i of the part is taken in token-major order, so
//    the staging side is one contiguous run and the cache side is row-sized
//    runs (row = D * element bytes). Used for token-major pages (where both
//    sides are contiguous), for rows below 128 bytes and for unaligned
//    layouts (1-byte accesses).
//  * token_lds_kernel: for head-major pages with rows of >= 128 bytes. The
//    cache side is read (gather) or written (scatter) in its own order --
//    per head one contiguous run of part_tokens rows -- and the part is
//    transposed through 8 KiB of LDS, so both HBM streams are contiguous runs
//    of >= 1 KiB.
//
// Measured on MI355X at the Llama-3-8B shape in HND layout (32 layers x 8192
// tokens, D = 128 bf16, 2 GiB moved per call), same-process comparisons:
//  - gather: LDS kernel 6.2-6.3 TB/s against 5.4-5.5 TB/s for the row kernel
//    (at D = 64, 6.1 against 5.7 TB/s; at D = 32 and 16 the row kernel was
//    faster, so the host picks it there); 8 KiB parts beat whole 32 KiB
//    pages (5.9 TB/s), 16 KiB parts were no faster; part-major order within
//    a job beat a job-minor order (5.3 TB/s);
//  - scatter: job-minor order 6.4-6.6 TB/s against 5.5-5.9 TB/s part-major.
// The physical-span gather_pages of the same pages ran 6.2-6.4 TB/s, so the
// transpose costs about 1%.
//
// Pages whose id is 0 or outside [1, num_blocks) are skipped: their staging
// rows are left untouched (gather) and nothing is written to the cache
// (scatter), as for gather_pages / scatter_pages.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "elem.h"
#include "kernels.h"
#include "launch.h"

namespace daric {

namespace {

constexpr int kThreads = 256;
constexpr int kRowUnroll = 8;
constexpr int kLdsUnits = 512;   // 16-byte units of LDS per workgroup (8 KiB)
constexpr int kMaxY = 65535;
constexpr int64_t kMaxBlocksX = (1ll << 24) - 1;
constexpr bool kTokenJobMinor = true;    // scatter direction: job-minor block order

template <typename T>
__device__ __forceinline__ T ld_nt(const T* p) { return __builtin_nontemporal_load(p); }
template <typename T>
__device__ __forceinline__ void st_nt(T* p, T v) { __builtin_nontemporal_store(v, p); }

template <int VW> struct Unit;
template <> struct Unit<16> { using T = u32x4; };
template <> struct Unit<1> { using T = uint8_t; };

// Resolves workgroup (part q of the job) to its cache and staging bases and
// token count; false when the part is past the job's end or its page is
// skipped.
__device__ __forceinline__ bool resolve_part(const TokenJob& j, int q, uint8_t*& cache,
                                             uint8_t*& stage, int& n_tok) {
    const int per_kv = j.n_sel * j.parts_per_page;
    if (q >= j.n_kv * per_kv) return false;
    const int kv = q / per_kv;
    const int r = q - kv * per_kv;
    const int s = r / j.parts_per_page;
    const int pp = r - s * j.parts_per_page;
    const int blk = j.idx[s];
    if (blk <= 0 || blk >= j.num_blocks) return false;
    const int tok0 = pp * j.part_tokens;
    n_tok = min(j.part_tokens, j.PS - tok0);
    const int64_t T = static_cast<int64_t>(j.n_sel) * j.PS;
    cache = j.layer + blk * j.sb + (kv ? j.v_off : 0) + tok0 * j.ss;
    stage = j.stage + ((kv * T + static_cast<int64_t>(s) * j.PS + tok0) * j.H) * j.row_bytes;
    return true;
}

// Workgroup -> (job, part): part-major within a job (grid.y = job), or
// job-minor (consecutive workgroups take the same part of consecutive jobs).
template <bool JOB_MINOR>
__device__ __forceinline__ void block_part(FastDiv njobs, int& job, int& q) {
    if (JOB_MINOR) {
        const uint32_t x = blockIdx.x;
        const uint32_t p = njobs.div(x);
        q = static_cast<int>(p);
        job = static_cast<int>(x - p * njobs.d);
    } else {
        job = static_cast<int>(blockIdx.y);
        q = static_cast<int>(blockIdx.x);
    }
}

template <int VW, bool GATHER, bool JOB_MINOR>
__global__ __launch_bounds__(kThreads) void token_rows_kernel(DescArg d, int job0, FastDiv njobs, XcdRuns xr) {
    using T = typename Unit<VW>::T;
    int jb, q;
    block_part<JOB_MINOR>(njobs, jb, q);
    if (!JOB_MINOR) q = xr.map(q);
    const TokenJob j = desc_load(desc_at<TokenJob>(d, 0) + job0 + jb);
    uint8_t *cache, *stage;
    int n_tok;
    if (!resolve_part(j, q, cache, stage, n_tok)) return;
    const int upr = static_cast<int>(j.d_upr.d);
    const int units = n_tok * j.H * upr;
    T* __restrict__ st = reinterpret_cast<T*>(stage);
    for (int base = 0; base < units; base += kThreads * kRowUnroll) {
        T v[kRowUnroll];
        T* cp[kRowUnroll];
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) {
            const int i = base + u * kThreads + static_cast<int>(threadIdx.x);
            cp[u] = nullptr;
            if (i >= units) continue;
            const uint32_t row = j.d_upr.div(static_cast<uint32_t>(i));   // token-major: tok * H + h
            const int k = i - static_cast<int>(row) * upr;
            const uint32_t tok = j.d_h.div(row);
            const int h = static_cast<int>(row - tok * static_cast<uint32_t>(j.H));
            cp[u] = reinterpret_cast<T*>(cache + tok * j.ss + h * j.sh) + k;
            v[u] = GATHER ? ld_nt(cp[u]) : ld_nt(st + i);
        }
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) {
            const int i = base + u * kThreads + static_cast<int>(threadIdx.x);
            if (cp[u] == nullptr) continue;
            if (GATHER) st_nt(st + i, v[u]);
            else st_nt(cp[u], v[u]);
        }
    }
}

// Head-major pages: the cache side of a part is H runs of n_tok rows, each
// run contiguous (token stride == row bytes, head stride == PS * row bytes).
template <bool GATHER, bool JOB_MINOR>
__global__ __launch_bounds__(kThreads) void token_lds_kernel(DescArg d, int job0, FastDiv njobs, XcdRuns xr) {
    __shared__ u32x4 sm[kLdsUnits];
    int jb, q;
    block_part<JOB_MINOR>(njobs, jb, q);
    if (!JOB_MINOR) q = xr.map(q);
    const TokenJob j = desc_load(desc_at<TokenJob>(d, 0) + job0 + jb);
    uint8_t *cache, *stage;
    int n_tok;
    if (!resolve_part(j, q, cache, stage, n_tok)) return;
    const int upr = static_cast<int>(j.d_upr.d);
    const int run = n_tok * upr;                 // units per head run
    const int units = j.H * run;                 // <= kLdsUnits (host-checked)
    constexpr int kPer = kLdsUnits / kThreads;
    u32x4* __restrict__ st = reinterpret_cast<u32x4*>(stage);
    u32x4 v[kPer];
    if (GATHER) {
        // cache order (h, tok, k) -> LDS at token-major position
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int i = u * kThreads + static_cast<int>(threadIdx.x);
            if (i < units) {
                const int h = i / run;
                const int rem = i - h * run;
                v[u] = ld_nt(reinterpret_cast<const u32x4*>(cache + h * j.sh) + rem);
            }
        }
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int i = u * kThreads + static_cast<int>(threadIdx.x);
            if (i < units) {
                const int h = i / run;
                const int rem = i - h * run;
                const int tok = rem / upr;
                const int k = rem - tok * upr;
                sm[(tok * j.H + h) * upr + k] = v[u];
            }
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int i = u * kThreads + static_cast<int>(threadIdx.x);
            if (i < units) st_nt(st + i, sm[i]);
        }
    } else {
        // staging in token-major order -> LDS at cache position -> cache runs
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int i = u * kThreads + static_cast<int>(threadIdx.x);
            if (i < units) v[u] = ld_nt(st + i);
        }
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int i = u * kThreads + static_cast<int>(threadIdx.x);
            if (i < units) {
                const int row = i / upr;
                const int k = i - row * upr;
                const int tok = row / j.H;
                const int h = row - tok * j.H;
                sm[h * run + tok * upr + k] = v[u];
            }
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int i = u * kThreads + static_cast<int>(threadIdx.x);
            if (i < units) {
                const int h = i / run;
                const int rem = i - h * run;
                st_nt(reinterpret_cast<u32x4*>(cache + h * j.sh) + rem, sm[i]);
            }
        }
    }
}

}  // namespace

void launch_token_copy(const DescArg& d, int n_jobs, int max_parts, int64_t part_bytes, int vw,
                       bool lds, bool gather, hipStream_t stream) {
#define DARIC_TOK(JM, FD, XR)                                                                            \
    do {                                                                                               \
        if (lds) {                                                                                     \
            if (gather) DARIC_LAUNCH((token_lds_kernel<true, JM>), grid, kThreads, 0, stream, d, j0, FD, XR);  \
            else DARIC_LAUNCH((token_lds_kernel<false, JM>), grid, kThreads, 0, stream, d, j0, FD, XR);        \
        } else if (vw == 16) {                                                                         \
            if (gather) DARIC_LAUNCH((token_rows_kernel<16, true, JM>), grid, kThreads, 0, stream, d, j0, FD, XR); \
            else DARIC_LAUNCH((token_rows_kernel<16, false, JM>), grid, kThreads, 0, stream, d, j0, FD, XR);   \
        } else {                                                                                       \
            if (gather) DARIC_LAUNCH((token_rows_kernel<1, true, JM>), grid, kThreads, 0, stream, d, j0, FD, XR); \
            else DARIC_LAUNCH((token_rows_kernel<1, false, JM>), grid, kThreads, 0, stream, d, j0, FD, XR);    \
        }                                                                                              \
        check_launch(gather ? "gather_tokens" : "scatter_tokens");                                    \
    } while (0)
    if (kTokenJobMinor && !gather) {
        // job-minor: slices of jobs so that the grid fits grid.x
        const int slice = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(n_jobs, kMaxBlocksX / max_parts)));
        for (int j0 = 0; j0 < n_jobs; j0 += slice) {
            const int nj = std::min(slice, n_jobs - j0);
            const FastDiv fd(static_cast<uint32_t>(nj));
            const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(max_parts) * nj));
            DARIC_TOK(true, fd, XcdRuns());
        }
        return;
    }
    const XcdRuns xr(max_parts, part_bytes);
    for (int j0 = 0; j0 < n_jobs; j0 += kMaxY) {
        const int nj = std::min(kMaxY, n_jobs - j0);
        const dim3 grid(static_cast<unsigned>(max_parts), static_cast<unsigned>(nj));
        const FastDiv fd(1);
        DARIC_TOK(false, fd, xr);
    }
#undef DARIC_TOK
}

}  // namespace daric
