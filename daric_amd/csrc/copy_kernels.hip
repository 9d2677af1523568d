// Paged-KV gather / scatter and the fused scatter + K re-rotation (gfx950).
//
// Work decomposition: a job is one (layer, chunk) pair; a tile is one page
// span of one prefix index (the K or V half of a page for vLLM's
// [2, blocks, PS, H, D] layout: 32 KiB at Llama-3-8B shape). A 256-lane
// workgroup streams a tile, or a part of one, with 16-byte accesses, 8 in
// flight per lane, loads before stores. Staging-side loads and cache-side
// stores are nontemporal: every byte is touched once.
//
// Block order (measured on MI355X at the Llama-3-8B shape): both directions
// cut each tile into parts of ~8 KiB. The scatter direction runs job-minor --
// consecutive workgroups take the same part of consecutive jobs -- which
// sustained ~6.3 TB/s against ~6.0 TB/s for a tile-major order (256 jobs of
// 64 pages) and 5.9 against 5.3-5.4 TB/s (32 jobs of 4096 pages); the gather
// direction runs tile-major within a job, which sustained ~6.3 TB/s (256 x 64)
// and 5.8-6.0 TB/s (32 x 4096), against 5.5-5.6 TB/s for whole-tile
// workgroups and job-minor orders. The fused scatter + rotation runs job-minor
// on whole tiles.
//
// Pages whose block id is 0 (vLLM's null block) are skipped, as the
// reference's kernels skip them (csrc/cache_ops/kernels.cu:26,39,69,79,104,117);
// ids outside [0, num_pages) are skipped as well instead of faulting.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "elem.h"
#include "jobs.h"
#include "kernels.h"
#include "launch.h"

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

// Copies n_units units of VW bytes from src to dst (n_units < 2^31).
template <int VW>
__device__ __forceinline__ void copy_units(const uint8_t* __restrict__ src,
                                           uint8_t* __restrict__ dst, int n_units) {
    using T = typename VecOf<VW>::T;
    const T* s = reinterpret_cast<const T*>(src);
    T* d = reinterpret_cast<T*>(dst);
    for (int base = 0; base < n_units; base += kThreads * kUnroll) {
        T v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int i = base + u * kThreads + static_cast<int>(threadIdx.x);
            if (i < n_units) v[u] = ld_nt(s + i);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int i = base + u * kThreads + static_cast<int>(threadIdx.x);
            if (i < n_units) st_nt(d + i, v[u]);
        }
    }
}

template <int VW>
__device__ __forceinline__ void copy_span(const uint8_t* __restrict__ src,
                                          uint8_t* __restrict__ dst, int64_t span) {
    copy_units<VW>(src, dst, static_cast<int>(span / VW));
}

// Resolves tile t of job j. Returns false when the tile is beyond the job or
// its page is skipped.
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

// Block -> (job, unit) mapping. Job-minor: block b takes job b % n_jobs and
// unit b / n_jobs; tile-major: job blockIdx.y, unit blockIdx.x. A unit is part
// (unit & (parts - 1)) of tile (unit >> log2 parts).
template <bool JOB_MINOR>
__device__ __forceinline__ void block_unit(const FastDiv& njobs, int& job, int& unit) {
    if (JOB_MINOR) {
        const uint32_t b = blockIdx.x;
        const uint32_t q = njobs.div(b);
        job = static_cast<int>(b - q * njobs.d);
        unit = static_cast<int>(q);
    } else {
        job = static_cast<int>(blockIdx.y);
        unit = static_cast<int>(blockIdx.x);
    }
}

template <int VW, bool GATHER, bool JOB_MINOR>
__global__ __launch_bounds__(kThreads) void copy_pages_kernel(DescArg d, int job0, FastDiv njobs,
                                                              int log2_parts, XcdRuns xr) {
    int jb, unit;
    block_unit<JOB_MINOR>(njobs, jb, unit);
    if (!JOB_MINOR) unit = xr.map(unit);
    const CopyJob j = desc_load(desc_at<CopyJob>(d, 0) + job0 + jb);
    int p, s;
    uint8_t *cache, *stage;
    if (!resolve_tile(j, unit >> log2_parts, p, s, cache, stage)) return;
    const int n_units = static_cast<int>(j.span / VW);
    const int parts = 1 << log2_parts;
    const int per = (n_units + parts - 1) >> log2_parts;
    const int u0 = (unit & (parts - 1)) * per;
    const int cnt = min(per, n_units - u0);
    if (cnt <= 0) return;
    const int64_t b0 = static_cast<int64_t>(u0) * VW;
    if (GATHER)
        copy_units<VW>(cache + b0, stage + b0, cnt);
    else
        copy_units<VW>(stage + b0, cache + b0, cnt);
}

// Fused scatter + rotation, job-minor block order. A work item of a K row is
// either a rotated item (NeoX: the two 16-byte units holding pairs
// (i, i + R/2) for i in [k*VE, k*VE + VE); GPT-J: one unit holding VE/2
// adjacent pairs) or a pass-through unit of the row's unrotated tail. Rows
// that are not rotated (V rows, tokens past the job's n_tokens) are copied
// bit-exactly. The first round's loads are issued before the workgroup
// computes the tile's cos/sin values into LDS, so the sincos latency overlaps
// the memory latency. fp8 codes are rotated as stored: a per-head scale
// cancels in a linear rotation.
template <int KIND, bool NEOX>
__global__ __launch_bounds__(kThreads) void scatter_rotate_kernel(
    DescArg d, int job0, FastDiv njobs, RowGeomDiv gd, const float* __restrict__ inv_freq) {
    using E = Elem<KIND>;
    constexpr int VE = E::VE;
    __shared__ float s_cos[kMaxHalfRot];
    __shared__ float s_sin[kMaxHalfRot];

    int jb, unit;
    block_unit<true>(njobs, jb, unit);
    const CopyJob j = desc_load(desc_at<CopyJob>(d, 0) + job0 + jb);
    int p, s;
    uint8_t *cache, *stage;
    if (!resolve_tile(j, unit, p, s, cache, stage)) return;

    const RowGeom& g = gd.g;
    const int n_valid = min(max(j.n_tokens - s * g.PS, 0), g.PS);
    if (p != 0 || n_valid == 0 || j.delta == 0.0f || g.krows == 0) {
        copy_span<16>(stage, cache, j.span);
        return;
    }

    const int half = g.R / 2;
    const u32x4* __restrict__ src = reinterpret_cast<const u32x4*>(stage);
    u32x4* __restrict__ dst = reinterpret_cast<u32x4*>(cache);
    const int upr = g.W / VE;                      // 16-byte units per row
    const int partner = NEOX ? half / VE : 0;      // unit distance of pair halves
    const int pass0 = NEOX ? 2 * g.n_rot : g.n_rot;  // first pass-through unit
    const int items = g.n_rows * g.ipr;

    for (int base = 0; base < items; base += kThreads * kRotUnroll) {
        u32x4 a[kRotUnroll], b[kRotUnroll];
        int ua[kRotUnroll], kk[kRotUnroll];
        bool rot[kRotUnroll], pair[kRotUnroll], ok[kRotUnroll];
#pragma unroll
        for (int u = 0; u < kRotUnroll; ++u) {
            const int it = base + u * kThreads + static_cast<int>(threadIdx.x);
            ok[u] = it < items;
            const int r = static_cast<int>(gd.ipr.div(static_cast<uint32_t>(it)));
            const int k = it - r * g.ipr;
            const int row0 = r * upr;
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
        if (base == 0) {
            for (int i = threadIdx.x; i < half; i += kThreads) {
                float sn, cs;
                sincosf(j.delta * inv_freq[i], &sn, &cs);
                s_cos[i] = cs;
                s_sin[i] = sn;
            }
            __syncthreads();
        }
#pragma unroll
        for (int u = 0; u < kRotUnroll; ++u) {
            if (!ok[u]) continue;
            if (!rot[u]) {
                st_nt(dst + ua[u], a[u]);
                if (pair[u]) st_nt(dst + ua[u] + partner, b[u]);
                continue;
            }
            float x[VE];
            E::unpack(a[u], x, 1.0f);
            if (NEOX) {
                float y[VE];
                E::unpack(b[u], y, 1.0f);
                const int i0 = kk[u] * VE;
#pragma unroll
                for (int e = 0; e < VE; ++e) {
                    const float c = s_cos[i0 + e], sn = s_sin[i0 + e];
                    const float x1 = x[e], x2 = y[e];
                    x[e] = x1 * c - x2 * sn;
                    y[e] = x2 * c + x1 * sn;
                }
                st_nt(dst + ua[u], E::pack(x, 1.0f));
                st_nt(dst + ua[u] + partner, E::pack(y, 1.0f));
            } else {
                const int i0 = kk[u] * (VE / 2);
#pragma unroll
                for (int m = 0; m < VE / 2; ++m) {
                    const float c = s_cos[i0 + m], sn = s_sin[i0 + m];
                    const float x1 = x[2 * m], x2 = x[2 * m + 1];
                    x[2 * m] = x1 * c - x2 * sn;
                    x[2 * m + 1] = x2 * c + x1 * sn;
                }
                st_nt(dst + ua[u], E::pack(x, 1.0f));
            }
        }
    }
}

// Lane-exchange variant of the fused kernel, used when the 16-byte units of a
// row (upr = W / VE) divide the 64-lane wavefront. Lanes keep the plain
// copy's access pattern -- unit i of the tile is lane i % 256 of round
// i / 256, fully coalesced -- so a lane's position k = i % upr inside its row
// is fixed, and so are its rotary pair indices: its cos/sin values are read
// from LDS into registers once per tile. NeoX pair halves (units k and
// k +- n_rot of the same row, always in the same wavefront) are exchanged with
// ds_bpermute. GPT-J pairs are adjacent elements of one unit and need no
// exchange. Values are converted, rotated and repacked one 32-bit word at a
// time. Rows that are not rotated are stored as loaded.
//
// fp8 (e4m3) with per-head scales: dequantise -> rotate -> requantise is
// sat_rtne(rot(q * s) / s) with one scale s for both members of a pair (they
// lie in the same head row), and a rotation is linear, so that equals
// sat_rtne(rot(q)) up to float32 rounding (relative 2^-24, far below the
// e4m3 quantum). The kernel therefore rotates the code values directly and
// saturates on requantisation; the registered scales are needed only where
// cached values meet other data (kv_deviation).
// Units in flight per lane in the lane kernel.
constexpr int kRotLaneUnroll = 4;

template <int KIND, bool NEOX>
__global__ __launch_bounds__(kThreads) void scatter_rotate_lane_kernel(
    DescArg d, int job0, FastDiv njobs, RowGeomDiv gd, const float* __restrict__ inv_freq, int log2_parts) {
    using E = Elem<KIND>;
    constexpr int VE = E::VE;
    constexpr int EPW = E::EPW;
    // A lane's cos/sin values (one per pair it touches) stay in registers for
    // 16-bit types. For e4m3 a 16-byte unit spans 16 pairs, and 32 registers
    // of them held the kernel at 114 VGPRs (4 waves/SIMD); it reads them from
    // LDS instead, interleaved (cos, sin) so one float4 serves two pairs: 66
    // VGPRs, 7 waves/SIMD, 1.6% faster at config 5 in a same-process A/B. For
    // bf16 the register form measured 1% faster. Both give identical bits.
    constexpr bool CSL = KIND == kE4M3;
    constexpr int NC = CSL ? 1 : (NEOX ? VE : VE / 2);  // cos/sin values per lane
    constexpr int UNR = kRotLaneUnroll;
    __shared__ float s_cos[kMaxHalfRot];
    __shared__ float s_sin[kMaxHalfRot];
    __shared__ float4 s_cs[kMaxHalfRot / 2];   // CSL: (cos, sin) of pairs 2i and 2i+1

    int jb, unit;
    block_unit<true>(njobs, jb, unit);
    const CopyJob j = desc_load(desc_at<CopyJob>(d, 0) + job0 + jb);
    int p, s;
    uint8_t *cache, *stage;
    if (!resolve_tile(j, unit >> log2_parts, p, s, cache, stage)) return;
    const int n_units = static_cast<int>(j.span / 16);
    const int per = n_units >> log2_parts;
    const int u0 = (unit & ((1 << log2_parts) - 1)) * per;
    const int u1 = u0 + per;

    const RowGeom& g = gd.g;
    const int n_valid = min(max(j.n_tokens - s * g.PS, 0), g.PS);
    if (p != 0 || n_valid == 0 || j.delta == 0.0f || g.krows == 0) {
        copy_units<16>(stage + static_cast<int64_t>(u0) * 16, cache + static_cast<int64_t>(u0) * 16, per);
        return;
    }

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63;
    const int upr = g.W / VE;                       // a power of two <= 64
    const int log2_upr = __builtin_ctz(static_cast<unsigned>(upr));
    const int k = tid & (upr - 1);
    const int nr = g.n_rot;
    const bool rot_lane = NEOX ? k < 2 * nr : k < nr;
    const bool first = k < nr;
    const int src_lane = (NEOX && rot_lane) ? (first ? lane + nr : lane - nr) : lane;
    const int pi0 = NEOX ? (first ? k : k - nr) * VE : k * (VE / 2);
    const int half = g.R / 2;
    const u32x4* __restrict__ src = reinterpret_cast<const u32x4*>(stage);
    u32x4* __restrict__ dst = reinterpret_cast<u32x4*>(cache);

    float cs[NC], ss[NC];
    for (int base = u0; base < u1; base += kThreads * UNR) {
        u32x4 v[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int i = base + u * kThreads + tid;
            v[u] = u32x4{0u, 0u, 0u, 0u};
            if (i < u1) v[u] = ld_nt(src + i);
        }
        if (base == u0) {
            // 16-bit types: lane k takes pairs kk*NC .. kk*NC + NC-1 into
            // registers. The table is stored transposed, pair i at
            // (i % NC) * (half / NC) + i / NC, so the lanes of a wavefront
            // read consecutive words for each e (the row-major, stride-NC
            // reads took 5.5 M bank-conflict cycles per launch at config 2).
            // e4m3 (CSL): the (cos, sin) entries are transposed the same way
            // -- NeoX float4 j (pairs 2j, 2j+1 of a unit) of unit kk at
            // j * (half / VE) + kk, GPT-J float2 pair pi at pi * (half /
            // (VE / 2)) + kk -- so each LDS read instruction takes consecutive
            // entries across the lanes (interleaved in pair order, they took
            // 30% of the kernel's LDS cycles in bank conflicts at config 5).
            const int cols = half / NC;
            for (int i = tid; i < half; i += kThreads) {
                float sn, c;
                sincosf(j.delta * inv_freq[i], &sn, &c);
                if (CSL) {
                    float* q;
                    if (NEOX) {
                        const int f = i >> 1;
                        q = reinterpret_cast<float*>(s_cs + (f % (VE / 2)) * (half / VE) + f / (VE / 2)) + 2 * (i & 1);
                    } else {
                        q = reinterpret_cast<float*>(s_cs) + 2 * ((i % (VE / 2)) * (half / (VE / 2)) + i / (VE / 2));
                    }
                    q[0] = c;
                    q[1] = sn;
                } else {
                    const int at = (i % NC) * cols + i / NC;
                    s_cos[at] = c;
                    s_sin[at] = sn;
                }
            }
            __syncthreads();
            if (!CSL) {
                const int kk = pi0 / NC;
#pragma unroll
                for (int e = 0; e < NC; ++e) {
                    const int at = rot_lane ? e * cols + kk : 0;
                    cs[e] = s_cos[at];
                    ss[e] = (NEOX && first) ? -s_sin[at] : s_sin[at];
                }
            }
        }
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int i = base + u * kThreads + tid;
            u32x4 pv = v[u];
            if (NEOX) {
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    pv[w] = static_cast<uint32_t>(__shfl(static_cast<int>(v[u][w]), src_lane, 64));
            }
            if (i >= u1) continue;
            const uint32_t r = static_cast<uint32_t>(i >> log2_upr);
            const uint32_t q = gd.tok_div.div(r);
            const int token = static_cast<int>(q - gd.ps.div(q) * g.PS);
            const bool rot = rot_lane && static_cast<int>(r) < g.krows && token < n_valid;
            if (!rot) {
                st_nt(dst + i, v[u]);
                continue;
            }
            u32x4 out;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                float x[EPW];
                E::unpack_word(v[u][w], x);
                if (NEOX) {
                    float y[EPW];
                    E::unpack_word(pv[w], y);
                    if (CSL) {
                        // pairs pi0 + w*EPW .. +EPW-1: EPW/2 float4 reads
                        const int kk = pi0 / VE;
#pragma unroll
                        for (int h2 = 0; h2 < EPW / 2; ++h2) {
                            const float4 t = s_cs[(w * (EPW / 2) + h2) * (half / VE) + kk];
                            const float s0 = first ? -t.y : t.y, s1 = first ? -t.w : t.w;
                            x[2 * h2] = x[2 * h2] * t.x + y[2 * h2] * s0;
                            x[2 * h2 + 1] = x[2 * h2 + 1] * t.z + y[2 * h2 + 1] * s1;
                        }
                    } else {
#pragma unroll
                        for (int e = 0; e < EPW; ++e)
                            x[e] = x[e] * cs[w * EPW + e] + y[e] * ss[w * EPW + e];
                    }
                } else {
#pragma unroll
                    for (int m = 0; m < EPW / 2; ++m) {
                        const int pi = w * (EPW / 2) + m;
                        float c, sn;
                        if (CSL) {
                            const float* csq = reinterpret_cast<const float*>(s_cs) +
                                               2 * (pi * (half / (VE / 2)) + pi0 / (VE / 2));
                            c = csq[0];
                            sn = csq[1];
                        } else {
                            c = cs[pi];
                            sn = ss[pi];
                        }
                        const float x1 = x[2 * m], x2 = x[2 * m + 1];
                        x[2 * m] = x1 * c - x2 * sn;
                        x[2 * m + 1] = x2 * c + x1 * sn;
                    }
                }
                out[w] = E::pack_word(x);
            }
            st_nt(dst + i, out);
        }
    }
}

// Descriptor upload: one 16-byte unit per lane, read from host memory.
__global__ __launch_bounds__(kThreads) void upload_kernel(const u32x4* __restrict__ src,
                                                         u32x4* __restrict__ dst, uint32_t n16) {
    const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < n16) dst[i] = src[i];
}

// Largest grid.x: grid.x * 256 lanes must stay below 2^32.
constexpr int64_t kMaxBlocksX = (1ll << 24) - 1;
constexpr int kMaxY = 65535;

void launch_copy_pages(const DescArg& d, int n_jobs, int max_tiles, int64_t max_span, int vw,
                       bool gather, hipStream_t stream) {
    // tiles cut into parts of about 8 KiB
    int log2_parts = 0;
    while (log2_parts < 3 && (max_span >> (log2_parts + 1)) >= 8192 &&
           (static_cast<int64_t>(max_tiles) << (log2_parts + 1)) <= kMaxBlocksX)
        ++log2_parts;
    if (!gather) {
        // job-minor: slices of jobs so that the grid fits grid.x
        const int64_t units = static_cast<int64_t>(max_tiles) << log2_parts;
        const int slice = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(n_jobs, kMaxBlocksX / units)));
        for (int j0 = 0; j0 < n_jobs; j0 += slice) {
            const int nj = std::min(slice, n_jobs - j0);
            const FastDiv fd(static_cast<uint32_t>(nj));
            const dim3 grid(static_cast<unsigned>(units * nj));
            if (vw == 16) DARIC_LAUNCH((copy_pages_kernel<16, false, true>), grid, kThreads, 0, stream, d, j0, fd, log2_parts, XcdRuns());
            else if (vw == 4) DARIC_LAUNCH((copy_pages_kernel<4, false, true>), grid, kThreads, 0, stream, d, j0, fd, log2_parts, XcdRuns());
            else DARIC_LAUNCH((copy_pages_kernel<1, false, true>), grid, kThreads, 0, stream, d, j0, fd, log2_parts, XcdRuns());
            check_launch("scatter_pages");
        }
        return;
    }
    // gather: tile-major within a job
    const FastDiv fd(1);
    const int64_t gx = static_cast<int64_t>(max_tiles) << log2_parts;
    const XcdRuns xr(gx, max_span >> log2_parts);
    for (int j0 = 0; j0 < n_jobs; j0 += kMaxY) {
        const int nj = std::min(kMaxY, n_jobs - j0);
        const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(nj));
        if (vw == 16) DARIC_LAUNCH((copy_pages_kernel<16, true, false>), grid, kThreads, 0, stream, d, j0, fd, log2_parts, xr);
        else if (vw == 4) DARIC_LAUNCH((copy_pages_kernel<4, true, false>), grid, kThreads, 0, stream, d, j0, fd, log2_parts, xr);
        else DARIC_LAUNCH((copy_pages_kernel<1, true, false>), grid, kThreads, 0, stream, d, j0, fd, log2_parts, xr);
        check_launch("gather_pages");
    }
}

void launch_upload(const void* src, void* dst, size_t n16, hipStream_t stream) {
    if (n16 == 0) return;
    const dim3 grid(static_cast<unsigned>((n16 + kThreads - 1) / kThreads));
    upload_kernel<<<grid, kThreads, 0, stream>>>(static_cast<const u32x4*>(src), static_cast<u32x4*>(dst),
                                                 static_cast<uint32_t>(n16));
    check_launch("descriptor upload");
}

void launch_scatter_rotate(const DescArg& d, int n_jobs, int max_tiles,
                           const RowGeomDiv& geom, int kind, bool neox, const float* inv_freq,
                           hipStream_t stream) {
    // the lane-exchange kernel needs whole rows inside a wavefront
    const int ve = kind == kE4M3 ? 16 : 8;
    const int upr = geom.g.W / ve;
    const bool lane = upr > 0 && 64 % upr == 0;
    // Lane kernel: pages cut into parts of at least 16 KiB, whole rows each.
    // Two 16 KiB halves of the 32 KiB bf16 pages measured ~1% faster than
    // whole pages at config 2, kernel and whole call alike (347.2 against
    // 350.2 us per kernel, 347.5 against 350.7 us per call; bit-identical
    // output); 8 KiB parts were 4% slower.
    int lp = 0;
    if (lane) {
        const int64_t units = static_cast<int64_t>(geom.g.n_rows) * upr;   // 16-byte units per page
        while ((units >> (lp + 1)) * 16 >= 16384 && units % (2ll << lp) == 0 && (units >> (lp + 1)) % upr == 0)
            ++lp;
    }
    const int64_t units_per_job = static_cast<int64_t>(max_tiles) << lp;
    const int slice = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(n_jobs, kMaxBlocksX / units_per_job)));
    for (int j0 = 0; j0 < n_jobs; j0 += slice) {
        const int nj = std::min(slice, n_jobs - j0);
        const FastDiv fd(static_cast<uint32_t>(nj));
        const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(max_tiles) * nj));
        if (lane) {
            const dim3 grid2(static_cast<unsigned>(units_per_job * nj));
#define DARIC_SR(K, N) DARIC_LAUNCH((scatter_rotate_lane_kernel<K, N>), grid2, kThreads, 0, stream, d, j0, fd, geom, inv_freq, lp)
            if (kind == kBF16) { if (neox) DARIC_SR(kBF16, true); else DARIC_SR(kBF16, false); }
            else if (kind == kF16) { if (neox) DARIC_SR(kF16, true); else DARIC_SR(kF16, false); }
            else { if (neox) DARIC_SR(kE4M3, true); else DARIC_SR(kE4M3, false); }
#undef DARIC_SR
        } else {
#define DARIC_SR(K, N) DARIC_LAUNCH((scatter_rotate_kernel<K, N>), grid, kThreads, 0, stream, d, j0, fd, geom, inv_freq)
            if (kind == kBF16) { if (neox) DARIC_SR(kBF16, true); else DARIC_SR(kBF16, false); }
            else if (kind == kF16) { if (neox) DARIC_SR(kF16, true); else DARIC_SR(kF16, false); }
            else { if (neox) DARIC_SR(kE4M3, true); else DARIC_SR(kE4M3, false); }
#undef DARIC_SR
        }
        check_launch("scatter_pages_rerotate");
    }
}

}  // namespace daric
