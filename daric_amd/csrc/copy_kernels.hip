// Paged-KV gather / scatter and the fused scatter + K re-rotation (gfx950).
//
// Work decomposition: blockIdx.y is the job (one (layer, chunk) pair),
// blockIdx.x a tile = one page span of one prefix index (K or V half of a
// page for vLLM's [2, blocks, PS, H, D] layout: 32 KiB at Llama-3-8B shape).
// A 256-lane workgroup streams the span with 16-byte accesses, 8 in flight
// per lane (32 KiB per round), loads before stores. Cache-side stores and
// staging-side loads are marked nontemporal: every byte is touched once.
// Pages whose block id is 0 (vLLM's null block) are skipped, as the
// reference's kernels skip them (csrc/cache_ops/kernels.cu:26,39,69,79,104,117);
// ids outside [0, num_pages) are skipped as well instead of faulting.
#include <hip/hip_runtime.h>

#include "elem.h"
#include "jobs.h"
#include "kernels.h"

namespace daric {

constexpr int kThreads = 256;
constexpr int kUnroll = 8;
constexpr int kRotUnroll = 4;
constexpr int kMaxHalfRot = 256;  // rotary_dim / 2 limit of the LDS cos/sin table

template <int VW> struct VecOf;
template <> struct VecOf<16> { using T = u32x4; };
template <> struct VecOf<4> { using T = uint32_t; };
template <> struct VecOf<1> { using T = uint8_t; };

template <typename T>
__device__ __forceinline__ T ld_nt(const T* p) { return __builtin_nontemporal_load(p); }
template <typename T>
__device__ __forceinline__ void st_nt(T* p, T v) { __builtin_nontemporal_store(v, p); }

// Copies `span` bytes (a multiple of VW, < 2^31) from src to dst.
template <int VW>
__device__ __forceinline__ void copy_span(const uint8_t* __restrict__ src,
                                          uint8_t* __restrict__ dst, int64_t span) {
    using T = typename VecOf<VW>::T;
    const T* s = reinterpret_cast<const T*>(src);
    T* d = reinterpret_cast<T*>(dst);
    const int n = static_cast<int>(span / VW);
    for (int base = 0; base < n; base += kThreads * kUnroll) {
        T v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int i = base + u * kThreads + static_cast<int>(threadIdx.x);
            if (i < n) v[u] = ld_nt(s + i);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int i = base + u * kThreads + static_cast<int>(threadIdx.x);
            if (i < n) st_nt(d + i, v[u]);
        }
    }
}

// Resolves tile blockIdx.x of job blockIdx.y. Returns false when the tile is
// beyond the job or its page is skipped.
__device__ __forceinline__ bool resolve_tile(const CopyJob& j, int t, int& p, int& s,
                                             uint8_t*& cache, uint8_t*& stage) {
    const int n_sel = j.n_sel;
    if (t >= j.prefix * n_sel) return false;
    p = t / n_sel;
    s = t - p * n_sel;
    const int page = j.idx[s];
    if (page <= 0 || page >= j.num_pages) return false;
    cache = j.layer + p * j.prefix_stride + static_cast<int64_t>(page) * j.page_stride;
    stage = j.stage + static_cast<int64_t>(t) * j.span;
    return true;
}

template <int VW, bool GATHER>
__global__ __launch_bounds__(kThreads) void copy_pages_kernel(const CopyJob* __restrict__ jobs) {
    const CopyJob& j = jobs[blockIdx.y];
    int p, s;
    uint8_t *cache, *stage;
    if (!resolve_tile(j, static_cast<int>(blockIdx.x), p, s, cache, stage)) return;
    if (GATHER)
        copy_span<VW>(cache, stage, j.span);
    else
        copy_span<VW>(stage, cache, j.span);
}

// Fused scatter + rotation. A work item of a K row is either a rotated item
// (NeoX: the two 16-byte units holding pairs (i, i + R/2) for i in
// [k*VE, k*VE + VE); GPT-J: one unit holding VE/2 adjacent pairs) or a
// pass-through unit of the row's unrotated tail. Rows that are not rotated
// (V rows, tokens past the job's n_tokens) are copied bit-exactly.
template <int KIND, bool NEOX>
__global__ __launch_bounds__(kThreads) void scatter_rotate_kernel(
    const CopyJob* __restrict__ jobs, RowGeomDiv gd, const float* __restrict__ inv_freq) {
    using E = Elem<KIND>;
    constexpr int VE = E::VE;
    __shared__ float s_cos[kMaxHalfRot];
    __shared__ float s_sin[kMaxHalfRot];

    const CopyJob& j = jobs[blockIdx.y];
    int p, s;
    uint8_t *cache, *stage;
    if (!resolve_tile(j, static_cast<int>(blockIdx.x), p, s, cache, stage)) return;

    const RowGeom& g = gd.g;
    const int n_valid = min(max(j.n_tokens - s * g.PS, 0), g.PS);
    if (p != 0 || n_valid == 0 || j.delta == 0.0f || g.krows == 0) {
        copy_span<16>(stage, cache, j.span);
        return;
    }

    const int half = g.R / 2;
    for (int i = threadIdx.x; i < half; i += kThreads) {
        float sn, cs;
        sincosf(j.delta * inv_freq[i], &sn, &cs);
        s_cos[i] = cs;
        s_sin[i] = sn;
    }
    __syncthreads();

    const u32x4* __restrict__ src = reinterpret_cast<const u32x4*>(stage);
    u32x4* __restrict__ dst = reinterpret_cast<u32x4*>(cache);
    const int upr = g.W / VE;                      // 16-byte units per row
    const int partner = NEOX ? half / VE : 0;      // unit distance of pair halves
    const int pass0 = NEOX ? 2 * g.n_rot : g.n_rot;  // first pass-through unit
    const int items = g.n_rows * g.ipr;
    const float* __restrict__ ksc = j.k_scale;

    for (int base = 0; base < items; base += kThreads * kRotUnroll) {
        u32x4 a[kRotUnroll], b[kRotUnroll];
        int ua[kRotUnroll], kk[kRotUnroll], rr[kRotUnroll];
        bool rot[kRotUnroll], pair[kRotUnroll], ok[kRotUnroll];
#pragma unroll
        for (int u = 0; u < kRotUnroll; ++u) {
            const int it = base + u * kThreads + static_cast<int>(threadIdx.x);
            ok[u] = it < items;
            const int r = static_cast<int>(gd.ipr.div(static_cast<uint32_t>(it)));
            const int k = it - r * g.ipr;
            const int row0 = r * upr;
            rr[u] = r;
            kk[u] = k;
            if (k < g.n_rot) {
                ua[u] = row0 + k;
                pair[u] = NEOX;
                const uint32_t q = gd.tok_div.div(static_cast<uint32_t>(r));
                const int token = static_cast<int>(q - gd.ps.div(q) * g.PS);
                rot[u] = (r < g.krows) && (token < n_valid);
            } else {
                ua[u] = row0 + pass0 + (k - g.n_rot);
                pair[u] = false;
                rot[u] = false;
            }
            if (ok[u]) {
                a[u] = ld_nt(src + ua[u]);
                if (pair[u]) b[u] = ld_nt(src + ua[u] + partner);
            }
        }
#pragma unroll
        for (int u = 0; u < kRotUnroll; ++u) {
            if (!ok[u]) continue;
            if (!rot[u]) {
                st_nt(dst + ua[u], a[u]);
                if (pair[u]) st_nt(dst + ua[u] + partner, b[u]);
                continue;
            }
            float scale = 1.0f;
            if (KIND == kE4M3 && ksc != nullptr) {
                const uint32_t r = static_cast<uint32_t>(rr[u]);
                const int h = g.tok_div == 1
                    ? static_cast<int>(gd.ps.div(r) - gd.h.div(gd.ps.div(r)) * g.H)
                    : static_cast<int>(r - gd.h.div(r) * g.H);
                scale = ksc[h];
            }
            const float inv = 1.0f / scale;
            float x[VE];
            E::unpack(a[u], x, scale);
            if (NEOX) {
                float y[VE];
                E::unpack(b[u], y, scale);
                const int i0 = kk[u] * VE;
#pragma unroll
                for (int e = 0; e < VE; ++e) {
                    const float c = s_cos[i0 + e], sn = s_sin[i0 + e];
                    const float x1 = x[e], x2 = y[e];
                    x[e] = x1 * c - x2 * sn;
                    y[e] = x2 * c + x1 * sn;
                }
                st_nt(dst + ua[u], E::pack(x, inv));
                st_nt(dst + ua[u] + partner, E::pack(y, inv));
            } else {
                const int i0 = kk[u] * (VE / 2);
#pragma unroll
                for (int m = 0; m < VE / 2; ++m) {
                    const float c = s_cos[i0 + m], sn = s_sin[i0 + m];
                    const float x1 = x[2 * m], x2 = x[2 * m + 1];
                    x[2 * m] = x1 * c - x2 * sn;
                    x[2 * m + 1] = x2 * c + x1 * sn;
                }
                st_nt(dst + ua[u], E::pack(x, inv));
            }
        }
    }
}

void launch_copy_pages(const CopyJob* d_jobs, int n_jobs, int max_tiles, int vw, bool gather,
                       hipStream_t stream) {
    constexpr int kMaxY = 65535;
    for (int j0 = 0; j0 < n_jobs; j0 += kMaxY) {
        const int nj = n_jobs - j0 < kMaxY ? n_jobs - j0 : kMaxY;
        const dim3 grid(static_cast<unsigned>(max_tiles), static_cast<unsigned>(nj));
        const CopyJob* jp = d_jobs + j0;
        if (vw == 16) {
            if (gather) copy_pages_kernel<16, true><<<grid, kThreads, 0, stream>>>(jp);
            else copy_pages_kernel<16, false><<<grid, kThreads, 0, stream>>>(jp);
        } else if (vw == 4) {
            if (gather) copy_pages_kernel<4, true><<<grid, kThreads, 0, stream>>>(jp);
            else copy_pages_kernel<4, false><<<grid, kThreads, 0, stream>>>(jp);
        } else {
            if (gather) copy_pages_kernel<1, true><<<grid, kThreads, 0, stream>>>(jp);
            else copy_pages_kernel<1, false><<<grid, kThreads, 0, stream>>>(jp);
        }
        check_launch(gather ? "gather_pages" : "scatter_pages");
    }
}

void launch_scatter_rotate(const CopyJob* d_jobs, int n_jobs, int max_tiles,
                           const RowGeomDiv& geom, int kind, bool neox, const float* inv_freq,
                           hipStream_t stream) {
    constexpr int kMaxY = 65535;
    for (int j0 = 0; j0 < n_jobs; j0 += kMaxY) {
        const int nj = n_jobs - j0 < kMaxY ? n_jobs - j0 : kMaxY;
        const dim3 grid(static_cast<unsigned>(max_tiles), static_cast<unsigned>(nj));
        const CopyJob* jp = d_jobs + j0;
#define DARIC_SR(K, N) scatter_rotate_kernel<K, N><<<grid, kThreads, 0, stream>>>(jp, geom, inv_freq)
        if (kind == kBF16) { if (neox) DARIC_SR(kBF16, true); else DARIC_SR(kBF16, false); }
        else if (kind == kF16) { if (neox) DARIC_SR(kF16, true); else DARIC_SR(kF16, false); }
        else { if (neox) DARIC_SR(kE4M3, true); else DARIC_SR(kE4M3, false); }
#undef DARIC_SR
        check_launch("scatter_pages_rerotate");
    }
}

}  // namespace daric
