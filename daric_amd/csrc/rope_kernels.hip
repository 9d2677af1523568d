// In-place re-rotation of cached K rows (gfx950): the counterpart of the
// reference's Triton _fused_rerotate_kernel (daric/adaption/adapter.py:30-88).
//
// The reference launches one program per (token, head) with a per-token
// cos/sin table read from HBM. Here a workgroup takes a tile of tokens of one
// segment (a run of tokens that all move by the same delta), computes the
// segment's rotary_dim/2 cos/sin values once in fp32 into LDS, and streams
// the tile's K head rows with 16-byte accesses. A tile is the segment's
// tokens in one page when the page's K rows are dense (rerotate_lane_kernel),
// else a run of about 1024 16-byte items (rerotate_vec_kernel), or of pairs
// with per-element accesses when the layout is not 16-byte aligned
// (rerotate_elem_kernel). Only the rotated [0, R) part of each head row is
// read and written; V and the rotary tail are never touched.
#include <hip/hip_runtime.h>

#include "elem.h"
#include "jobs.h"
#include "kernels.h"
#include "launch.h"

namespace daric {

namespace {

constexpr int kThreads = 256;
constexpr int kVecUnroll = 2;
constexpr int kMaxHalfRot = 256;

__device__ __forceinline__ int find_segment(DescPtr<RopeSeg> segs, int n, int tile) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (segs[mid].tile_begin <= tile) lo = mid; else hi = mid - 1;
    }
    return lo;
}

__device__ __forceinline__ void fill_cos_sin(float* s_cos, float* s_sin, int half, float delta,
                                             const float* __restrict__ inv_freq) {
    for (int i = threadIdx.x; i < half; i += kThreads) {
        float sn, cs;
        sincosf(delta * inv_freq[i], &sn, &cs);
        s_cos[i] = cs;
        s_sin[i] = sn;
    }
    __syncthreads();
}

// One item = one 16-byte unit of a head row's rotated part (NeoX: a unit of
// the first half and its partner rotary_dim/2 elements on). Each thread
// issues its first kVecUnroll items' loads before the cos/sin table is
// filled, so the loads are in flight while sincosf runs.
//
// fp8 codes are rotated as they are stored: the rotation is linear, so a
// positive per-head scale s gives rot(q * s) / s = rot(q) and cancels.
template <int KIND, bool NEOX>
__global__ __launch_bounds__(kThreads) void rerotate_vec_kernel(
    DescArg d, int layer_off, int layer0, InplaceGeom g, int n_segs,
    const int32_t* __restrict__ bt, const float* __restrict__ inv_freq,
    FastDiv d_tok, FastDiv d_rot, FastDiv d_ps) {
    using E = Elem<KIND>;
    constexpr int VE = E::VE;
    constexpr int ES = KIND == kE4M3 ? 1 : 2;
    __shared__ float s_cos[kMaxHalfRot];
    __shared__ float s_sin[kMaxHalfRot];

    const DescPtr<RopeSeg> segs = desc_at<RopeSeg>(d, 0);
    const DescPtr<uint8_t*> layers = desc_at<uint8_t*>(d, layer_off) + layer0;
    const int tile = static_cast<int>(blockIdx.x);
    const RopeSeg sg = desc_load(segs + find_segment(segs, n_segs, tile));
    const int tok0 = (tile - sg.tile_begin) * g.tile_tokens;
    const int n_tok = min(g.tile_tokens, sg.n_tokens - tok0);
    if (n_tok <= 0 || sg.delta == 0.0f) return;
    const int half = g.R / 2;

    uint8_t* __restrict__ base = layers[blockIdx.y];
    const int per_tok = g.H * g.n_rot;
    const int items = n_tok * per_tok;
    const int partner = NEOX ? half * ES / 16 : 0;      // in 16-byte units
    const uint32_t pos0 = static_cast<uint32_t>(sg.tok_start + tok0);

    for (int b0 = 0; b0 < items; b0 += kThreads * kVecUnroll) {
        u32x4 a[kVecUnroll], bb[kVecUnroll];
        u32x4* p[kVecUnroll];
        int kk[kVecUnroll];
#pragma unroll
        for (int u = 0; u < kVecUnroll; ++u) {
            const int it = b0 + u * kThreads + static_cast<int>(threadIdx.x);
            p[u] = nullptr;
            kk[u] = 0;
            if (it >= items) continue;
            const uint32_t t = d_tok.div(static_cast<uint32_t>(it));
            const uint32_t rem = static_cast<uint32_t>(it) - t * static_cast<uint32_t>(per_tok);
            const uint32_t h = d_rot.div(rem);
            const uint32_t pos = pos0 + t;
            const uint32_t q = d_ps.div(pos);
            const int blk = bt[sg.bt_offset + q];
            if (blk < g.min_block || blk >= g.num_blocks) continue;
            kk[u] = static_cast<int>(rem - h * static_cast<uint32_t>(g.n_rot));
            p[u] = reinterpret_cast<u32x4*>(
                       base + (static_cast<int64_t>(blk) * g.sb +
                               static_cast<int64_t>(pos - q * static_cast<uint32_t>(g.PS)) * g.ss +
                               static_cast<int64_t>(h) * g.sh) * ES) + kk[u];
            a[u] = *p[u];
            if (NEOX) bb[u] = p[u][partner];
        }
        if (b0 == 0) fill_cos_sin(s_cos, s_sin, half, sg.delta, inv_freq);
#pragma unroll
        for (int u = 0; u < kVecUnroll; ++u) {
            if (!p[u]) continue;
            float x[VE];
            E::unpack(a[u], x, 1.0f);
            if (NEOX) {
                float y[VE];
                E::unpack(bb[u], y, 1.0f);
                const int i0 = kk[u] * VE;
#pragma unroll
                for (int e = 0; e < VE; ++e) {
                    const float c = s_cos[i0 + e], sn = s_sin[i0 + e];
                    const float x1 = x[e], x2 = y[e];
                    x[e] = x1 * c - x2 * sn;
                    y[e] = x2 * c + x1 * sn;
                }
                *p[u] = E::pack(x, 1.0f);
                p[u][partner] = E::pack(y, 1.0f);
            } else {
                const int i0 = kk[u] * (VE / 2);
#pragma unroll
                for (int m = 0; m < VE / 2; ++m) {
                    const float c = s_cos[i0 + m], sn = s_sin[i0 + m];
                    const float x1 = x[2 * m], x2 = x[2 * m + 1];
                    x[2 * m] = x1 * c - x2 * sn;
                    x[2 * m + 1] = x2 * c + x1 * sn;
                }
                *p[u] = E::pack(x, 1.0f);
            }
        }
    }
}

// Page-tile variant for K rows that are dense in the page (token-major
// [PS, H, W] or head-major [H, PS, W] rows, W a 16-byte multiple). A
// workgroup takes the segment's tokens in one page of one layer; the
// segment's tiles are its pages (the first and last may be partial). Unit
// i of the page's K rows goes to lane i % 256, as in a plain copy, so every
// lane keeps one position k = i % upr within its rows: its cos/sin values
// stay in registers for the whole page, and the NeoX partner unit (k +/- nr)
// of the same row sits in the same wavefront, fetched with a lane exchange.
// Only units of the rotated part and of the segment's tokens are read and
// written. A page of 32 KiB or more is split into parts of at least 16 KiB
// (whole rows), one workgroup each: 0.9% faster than whole pages at config 2.
// Loads are nontemporal and stores plain: in place, nontemporal
// stores of the lines just read ran 12% slower on MI355X. On the config-2
// in-place call (32 layers x 7168 tokens) this kernel ran 3-4% faster than
// the item kernel; 2, 4 or 8 units in flight per lane measured the same.
template <typename T>
__device__ __forceinline__ T ld_nt(const T* p) { return __builtin_nontemporal_load(p); }

constexpr int kLaneUnroll = 2;
// e4m3: 4 units in flight per lane, so a workgroup holds a whole 16 KiB K page
// of the Llama-3-70B shape in one round.
constexpr int kLaneUnrollFp8 = 4;

// CSL (e4m3): a lane reads its cos/sin values from LDS at each use instead of
// holding them in registers. A 16-byte e4m3 unit spans 16 pairs: held in
// registers they took the kernel to 96 VGPRs (5 waves/SIMD); read from LDS as
// (cos, sin) float4s of two pairs, as the fused kernel does, it takes 50. With
// kLaneUnrollFp8 it ran the config-5 in-place call (15 chunks x 2048 tokens x
// 80 layers) in 1018 against 1033 us, at the rate of the same kernel with the
// rotation taken out (1015 us, a pure read-modify-write of the same pages), in
// a same-process A/B on MI355X. Both forms give identical bits.
template <int KIND, bool NEOX, bool CSL, int UNR>
__global__ __launch_bounds__(kThreads) void rerotate_lane_kernel(
    DescArg d, int layer_off, LayerMinor lm, InplaceGeom g, int n_segs,
    const int32_t* __restrict__ bt, const float* __restrict__ inv_freq, FastDiv d_tok, FastDiv d_ps,
    int log2_parts) {
    using E = Elem<KIND>;
    constexpr int VE = E::VE;
    constexpr int EPW = E::EPW;
    constexpr int ES = KIND == kE4M3 ? 1 : 2;
    constexpr int NC = CSL ? 1 : (NEOX ? VE : VE / 2);   // cos/sin values per lane in registers
    __shared__ float s_cos[kMaxHalfRot];
    __shared__ float s_sin[kMaxHalfRot];
    __shared__ float4 s_cs[kMaxHalfRot / 2];   // CSL: (cos, sin) of two pairs per entry

    const DescPtr<RopeSeg> segs = desc_at<RopeSeg>(d, 0);
    const DescPtr<uint8_t*> layers = desc_at<uint8_t*>(d, layer_off);
    int lyr;
    int64_t item;
    lm.at(lyr, item);
    const int tile = static_cast<int>(item);
    const RopeSeg sg = desc_load(segs + find_segment(segs, n_segs, tile));
    if (sg.delta == 0.0f) return;
    const int page = sg.tok_start / g.PS + ((tile - sg.tile_begin) >> log2_parts);
    const int part = (tile - sg.tile_begin) & ((1 << log2_parts) - 1);
    const int page_tok0 = page * g.PS;
    const int lo = max(sg.tok_start - page_tok0, 0);
    const int hi = min(sg.tok_start + sg.n_tokens - page_tok0, g.PS);
    if (hi <= lo) return;
    const int blk = bt[sg.bt_offset + page];
    if (blk < g.min_block || blk >= g.num_blocks) return;
    u32x4* __restrict__ pg = reinterpret_cast<u32x4*>(layers[lyr] + static_cast<int64_t>(blk) * g.sb * ES);

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63;
    const int log2_upr = __builtin_ctz(static_cast<unsigned>(g.upr));
    const int k = tid & (g.upr - 1);
    const int nr = g.n_rot;
    const bool rot_lane = NEOX ? k < 2 * nr : k < nr;
    const bool first = k < nr;
    const int src_lane = (NEOX && rot_lane) ? (first ? lane + nr : lane - nr) : lane;
    const int pi0 = NEOX ? (first ? k : k - nr) * VE : k * (VE / 2);
    const int n_units = g.PS * g.H * g.upr;
    const int per = n_units >> log2_parts;
    const int u0 = part * per, u1 = u0 + per;
    const int half = g.R / 2;

    float cs[NC], ss[NC];
    for (int base = u0; base < u1; base += kThreads * UNR) {
        u32x4 v[UNR];
        bool act[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int i = base + u * kThreads + tid;
            const uint32_t r = static_cast<uint32_t>(i >> log2_upr);
            const uint32_t q = d_tok.div(r);
            const int token = static_cast<int>(q - d_ps.div(q) * static_cast<uint32_t>(g.PS));
            act[u] = rot_lane && i < u1 && token >= lo && token < hi;
            v[u] = u32x4{0u, 0u, 0u, 0u};
            if (act[u]) v[u] = ld_nt(pg + i);
        }
        if (base == u0) {
            // Lane k needs pairs kk*NC .. kk*NC + NC-1. The table is stored
            // transposed, pair i at (i % NC) * (half / NC) + i / NC, so that
            // the lanes of a wavefront read consecutive words for each e
            // (row-major, the stride-NC reads took 2-way bank conflicts:
            // 30% of the kernel's LDS cycles at config 2).
            // CSL: the (cos, sin) entries are transposed the same way -- NeoX
            // float4 j (pairs 2j, 2j+1 of a unit) of unit kk at
            // j * (half / VE) + kk, GPT-J float2 pair pi at
            // pi * (half / (VE / 2)) + kk -- so each LDS read takes
            // consecutive entries across the lanes.
            const int cols = half / NC;
            for (int i = tid; i < half; i += kThreads) {
                float sn, c;
                sincosf(sg.delta * inv_freq[i], &sn, &c);
                if constexpr (CSL) {
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
            if constexpr (!CSL) {
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
            u32x4 pv = v[u];
            if (NEOX) {
#pragma unroll
                for (int w = 0; w < 4; ++w)
                    pv[w] = static_cast<uint32_t>(__shfl(static_cast<int>(v[u][w]), src_lane, 64));
            }
            if (!act[u]) continue;
            u32x4 out;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                float x[EPW];
                E::unpack_word(v[u][w], x);
                if (NEOX) {
                    float y[EPW];
                    E::unpack_word(pv[w], y);
                    if constexpr (CSL) {
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
                        if constexpr (CSL) {
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
            pg[base + u * kThreads + tid] = out;
        }
    }
}

// Per-element variant for layouts whose rows or pair halves are not 16-byte
// aligned. One item = one rotation pair; fp8 codes are rotated as stored, as
// in the vector kernel.
template <int KIND>
__device__ __forceinline__ float load_elem(const uint8_t* p) {
    if (KIND == kBF16) return bf16_to_f32(*reinterpret_cast<const uint16_t*>(p));
    if (KIND == kF16) return f16_to_f32(*reinterpret_cast<const uint16_t*>(p));
    return e4m3_to_f32(*p);
}
template <int KIND>
__device__ __forceinline__ void store_elem(uint8_t* p, float v) {
    if (KIND == kBF16) *reinterpret_cast<uint16_t*>(p) = static_cast<uint16_t>(f32_to_bf16(v));
    else if (KIND == kF16) *reinterpret_cast<uint16_t*>(p) = static_cast<uint16_t>(f32_to_f16(v));
    else *p = static_cast<uint8_t>(f32_to_e4m3(v));
}

template <int KIND, bool NEOX>
__global__ __launch_bounds__(kThreads) void rerotate_elem_kernel(
    DescArg d, int layer_off, int layer0, InplaceGeom g, int n_segs,
    const int32_t* __restrict__ bt, const float* __restrict__ inv_freq) {
    constexpr int ES = KIND == kE4M3 ? 1 : 2;
    __shared__ float s_cos[kMaxHalfRot];
    __shared__ float s_sin[kMaxHalfRot];
    const DescPtr<RopeSeg> segs = desc_at<RopeSeg>(d, 0);
    const DescPtr<uint8_t*> layers = desc_at<uint8_t*>(d, layer_off) + layer0;
    const int tile = static_cast<int>(blockIdx.x);
    const RopeSeg sg = desc_load(segs + find_segment(segs, n_segs, tile));
    const int tok0 = (tile - sg.tile_begin) * g.tile_tokens;
    const int n_tok = min(g.tile_tokens, sg.n_tokens - tok0);
    if (n_tok <= 0 || sg.delta == 0.0f) return;
    const int half = g.R / 2;
    fill_cos_sin(s_cos, s_sin, half, sg.delta, inv_freq);
    uint8_t* __restrict__ base = layers[blockIdx.y];
    const int per_tok = g.H * half;
    const int items = n_tok * per_tok;
    for (int it = threadIdx.x; it < items; it += kThreads) {
        const int t = it / per_tok;
        const int rem = it - t * per_tok;
        const int h = rem / half;
        const int i = rem - h * half;
        const int pos = sg.tok_start + tok0 + t;
        const int blk = bt[sg.bt_offset + pos / g.PS];
        if (blk < g.min_block || blk >= g.num_blocks) continue;
        const int64_t row = static_cast<int64_t>(blk) * g.sb +
                            static_cast<int64_t>(pos % g.PS) * g.ss + static_cast<int64_t>(h) * g.sh;
        const int64_t e1 = NEOX ? row + i : row + 2 * i;
        const int64_t e2 = NEOX ? row + i + half : row + 2 * i + 1;
        const float x1 = load_elem<KIND>(base + e1 * ES);
        const float x2 = load_elem<KIND>(base + e2 * ES);
        const float c = s_cos[i], sn = s_sin[i];
        store_elem<KIND>(base + e1 * ES, x1 * c - x2 * sn);
        store_elem<KIND>(base + e2 * ES, x2 * c + x1 * sn);
    }
}

}  // namespace

void launch_rerotate_inplace(const DescArg& d, int layer_off, int n_layers, const InplaceGeom& g,
                             int n_segs, int n_tiles, const int32_t* block_table,
                             const float* inv_freq, int kind, bool neox, int path, hipStream_t stream) {
    constexpr int kMaxY = 65535;
    const FastDiv d_tok(static_cast<uint32_t>(g.H * g.n_rot)), d_rot(static_cast<uint32_t>(g.n_rot)),
        d_ps(static_cast<uint32_t>(g.PS)), d_ltok(static_cast<uint32_t>(g.tok_div > 0 ? g.tok_div : 1));
    if (path == kRotLane) {
        // one workgroup per (layer, page part), layer-minor
        for_layer_minor(n_layers, n_tiles, [&](const LayerMinor& lm, unsigned blocks) {
#define DARIC_RL(K, N) DARIC_LAUNCH((rerotate_lane_kernel<K, N, K == kE4M3, K == kE4M3 ? kLaneUnrollFp8 : kLaneUnroll>), blocks, kThreads, 0, stream, d, layer_off, lm, g, n_segs, block_table, inv_freq, d_ltok, d_ps, g.log2_parts)
            if (kind == kBF16) { if (neox) DARIC_RL(kBF16, true); else DARIC_RL(kBF16, false); }
            else if (kind == kF16) { if (neox) DARIC_RL(kF16, true); else DARIC_RL(kF16, false); }
            else { if (neox) DARIC_RL(kE4M3, true); else DARIC_RL(kE4M3, false); }
#undef DARIC_RL
            check_launch("rerotate_pages");
        });
        return;
    }
    for (int l0 = 0; l0 < n_layers; l0 += kMaxY) {
        const int nl = n_layers - l0 < kMaxY ? n_layers - l0 : kMaxY;
        const dim3 grid(static_cast<unsigned>(n_tiles), static_cast<unsigned>(nl));
#define DARIC_RV(K, N) DARIC_LAUNCH((rerotate_vec_kernel<K, N>), grid, kThreads, 0, stream, d, layer_off, l0, g, n_segs, block_table, inv_freq, d_tok, d_rot, d_ps)
#define DARIC_RE(K, N) DARIC_LAUNCH((rerotate_elem_kernel<K, N>), grid, kThreads, 0, stream, d, layer_off, l0, g, n_segs, block_table, inv_freq)
        if (path == kRotVec) {
            if (kind == kBF16) { if (neox) DARIC_RV(kBF16, true); else DARIC_RV(kBF16, false); }
            else if (kind == kF16) { if (neox) DARIC_RV(kF16, true); else DARIC_RV(kF16, false); }
            else { if (neox) DARIC_RV(kE4M3, true); else DARIC_RV(kE4M3, false); }
        } else {
            if (kind == kBF16) { if (neox) DARIC_RE(kBF16, true); else DARIC_RE(kBF16, false); }
            else if (kind == kF16) { if (neox) DARIC_RE(kF16, true); else DARIC_RE(kF16, false); }
            else { if (neox) DARIC_RE(kE4M3, true); else DARIC_RE(kE4M3, false); }
        }
#undef DARIC_RV
#undef DARIC_RE
        check_launch("rerotate_pages");
    }
}

}  // namespace daric
