// Recompute selection kernels (gfx950): per-token K deviation, per-chunk
// top-k by LDS radix select, and the merge of recomputed rows.
//
// Deviation order (the keys are bit-exact against the CPU oracle, which sums
// in exactly this order): a wavefront owns one token; the token's H*D
// elements, in (h, d) order, are cut into vectors of 8 elements; vector v is
// loaded by lane v % 64 in round v / 64; each lane accumulates
// acc = acc + diff * diff element by element (float32, no contraction),
// rounds ascending; the 64 lane sums are then combined by a butterfly over
// xor offsets 32, 16, 8, 4, 2, 1. Any NaN key is stored as 0x7FC00000.
//
// Top-k ranks keys by the IEEE total order of their float32 bits (NaN above
// +inf), ties to the lower token index, and writes the selected chunk-local
// indices in ascending order.
#include <hip/hip_runtime.h>

#include "common.h"
#include "elem.h"
#include "jobs.h"
#include "kernels.h"
#include "launch.h"

namespace daric {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
// Tokens per wavefront in the deviation kernel: 8 for 16-bit caches (16 loads
// of 16 bytes in flight per lane; 3-4% faster than 4 at config 3), 4 for fp8
// caches, where the 8-token form measured slower (config 5).
template <int CK> constexpr int dev_tok_per_wave() { return CK == kE4M3 ? 4 : 8; }
constexpr int kMergeTok = 8;                       // selected tokens per merge workgroup
constexpr int kMaxGridYZ = 65535;                  // grid.y / grid.z limit; larger counts are sliced
constexpr int kTopkLdsTokens = 8192;               // top-k keys staged in LDS up to this chunk length

__device__ __forceinline__ int find_chunk(DescPtr<SelChunk> ch, int n, int tile) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (ch[mid].tile_begin <= tile) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// 8 elements: 16 bytes for 2-byte types, 8 bytes for fp8. Loaded raw (so a
// lane keeps few registers per load in flight) and converted when summed.
template <int KIND> struct Raw8 { u32x4 w; };
template <> struct Raw8<kE4M3> { u32x2 w; };

template <int KIND>
__device__ __forceinline__ Raw8<KIND> load_raw8(const uint8_t* p) {
    Raw8<KIND> r;
    if constexpr (KIND == kE4M3)
        r.w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    else
        r.w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return r;
}

template <int KIND>
__device__ __forceinline__ void unpack8(const Raw8<KIND>& r, float* x, float scale) {
    if constexpr (KIND == kE4M3) {
#ifdef DARIC_FP8_SOFTWARE
#pragma unroll
        for (int b = 0; b < 4; ++b) { x[b] = e4m3_to_f32((r.w[0] >> (8 * b)) & 0xffu); x[4 + b] = e4m3_to_f32((r.w[1] >> (8 * b)) & 0xffu); }
#else
        e4m3x4_to_f32_hw(r.w[0], x);
        e4m3x4_to_f32_hw(r.w[1], x + 4);
#endif
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = x[i] * scale;
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (KIND == kBF16) {
                x[2 * q] = u2f(r.w[q] << 16);
                x[2 * q + 1] = u2f(r.w[q] & 0xffff0000u);
            } else {
                const uint32_t word = r.w[q];
                x[2 * q] = f16_to_f32(word & 0xffffu);
                x[2 * q + 1] = f16_to_f32(word >> 16);
            }
        }
    }
}

// Keys of tokens j0 .. j0 + TPW - 1 of chunk c in layer l, summed by one
// wavefront in the fixed order above; the butterfly leaves every key in every
// lane. A token past the chunk's end, or whose block id lies outside
// [0, num_blocks), is not read and gets key 0; a NaN key is 0x7FC00000.
template <int CK, int NK, int TPW>
__device__ __forceinline__ void wave_keys(const SelChunk& c, int j0, int lane, const KVGeom& g,
                                          const uint8_t* __restrict__ base, const int32_t* __restrict__ bt,
                                          const uint8_t* __restrict__ k_new, int64_t T, int l,
                                          const float* __restrict__ ksc, float* key) {
#pragma clang fp contract(off)
    constexpr int CES = CK == kE4M3 ? 1 : 2;
    const int N = g.H * g.D;
    const int n_vec = N >> 3;
    const int rounds = (n_vec + 63) >> 6;

    int64_t cache_row[TPW];
    const uint8_t* new_row[TPW];
    bool valid[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        const int j = j0 + i;
        const int p = c.tok0 + j;                  // position in the chunk's block list
        int blk = -1;
        if (j < c.n_tokens) blk = bt[c.bt_offset + p / g.PS];
        valid[i] = j < c.n_tokens && blk >= 0 && blk < g.num_blocks;
        cache_row[i] = static_cast<int64_t>(blk) * g.sb + static_cast<int64_t>(p % g.PS) * g.ss;
        new_row[i] = k_new + ((static_cast<int64_t>(l) * T + c.row_offset + j) * N) * 2;
    }

    float acc[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) acc[i] = 0.0f;

    for (int r = 0; r < rounds; ++r) {
        const int v = r * 64 + lane;
        if (v >= n_vec) break;
        const int e0 = v << 3;
        const int h = e0 / g.D;
        const int d0 = e0 - h * g.D;
        const float scale = (CK == kE4M3 && ksc) ? ksc[h] : 1.0f;
        Raw8<NK> ra[TPW];
        Raw8<CK> rb[TPW];
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
            if (!valid[i]) continue;
            ra[i] = load_raw8<NK>(new_row[i] + static_cast<int64_t>(e0) * 2);
            rb[i] = load_raw8<CK>(base + (cache_row[i] + static_cast<int64_t>(h) * g.sh + d0) * CES);
        }
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
            if (!valid[i]) continue;
            float a[8], b[8];
            unpack8<NK>(ra[i], a, 1.0f);
            unpack8<CK>(rb[i], b, scale);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float df = a[e] - b[e];
                const float sq = df * df;
                acc[i] = acc[i] + sq;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        float s = acc[i];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) s = s + __shfl_xor(s, off, 64);
        float k = valid[i] ? s : 0.0f;
        if (k != k) k = u2f(0x7fc00000u);
        key[i] = k;
    }
}

template <int CK, int NK>
__global__ __launch_bounds__(kThreads) void deviation_kernel(
    DescArg d, int layer_off, KVGeom g, const int32_t* __restrict__ bt,
    const uint8_t* __restrict__ k_new, int64_t T, int n_chunks,
    const float* __restrict__ k_scales, float* __restrict__ keys, int l0) {
    const DescPtr<SelChunk> chunks = desc_at<SelChunk>(d, 0);
    const DescPtr<uint8_t*> layers = desc_at<uint8_t*>(d, layer_off);
    const int l = static_cast<int>(blockIdx.y) + l0;
    const int tile = static_cast<int>(blockIdx.x);
    const SelChunk c = desc_load(chunks + find_chunk(chunks, n_chunks, tile));
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    constexpr int kTokPerWave = dev_tok_per_wave<CK>();
    constexpr int kTileTokens = kWaves * kTokPerWave;
    const int j0 = (tile - c.tile_begin) * kTileTokens + wave * kTokPerWave;
    const float* ksc = k_scales ? k_scales + static_cast<int64_t>(l) * g.H : nullptr;
    float key[kTokPerWave];
    wave_keys<CK, NK, kTokPerWave>(c, j0, lane, g, layers[l], bt, k_new, T, l, ksc, key);
#pragma unroll
    for (int i = 0; i < kTokPerWave; ++i) {
        const int j = j0 + i;
        if (lane == 0 && j < c.n_tokens) keys[static_cast<int64_t>(l) * T + c.row_offset + j] = key[i];
    }
}

__device__ __forceinline__ uint32_t order_key(float f) {
    uint32_t b = f2u(f);
    if ((b & 0x7fffffffu) > 0x7f800000u) b = 0x7fc00000u;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Exclusive prefix count of `flag` over the workgroup; *total gets the sum.
__device__ __forceinline__ int block_excl_count(bool flag, int* s_wave, int* total) {
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const unsigned long long m = __ballot(flag);
    const int below = __popcll(m & ((1ull << lane) - 1ull));
    if (lane == 0) s_wave[wave] = __popcll(m);
    __syncthreads();
    int before = 0, sum = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const int cnt = s_wave[w];
        before += w < wave ? cnt : 0;
        sum += cnt;
    }
    __syncthreads();
    *total = sum;
    return before + below;
}

// LDS_KEYS: the chunk's order keys are staged in LDS (chunks of at most
// kTopkLdsTokens tokens); otherwise every pass reads them from global memory,
// where a chunk's keys (4 bytes per token) stay in L2 across the five passes.
// Per-chunk top-k by the workgroup (kThreads lanes): the k largest of the n
// order keys key_at(0 .. n-1), ties to the lower index, written in ascending
// index order to orow[0 .. k-1] (when not null) and, when s_sel is not null,
// to the LDS array s_sel (visible to the other lanes after the caller's next
// barrier). Four
// 8-bit radix passes over LDS histograms find the k-th largest key.
template <typename KeyAt>
__device__ __forceinline__ void chunk_topk(KeyAt key_at, int n, int k, int32_t* __restrict__ orow,
                                           int32_t* s_sel, uint32_t* hist, uint32_t* s_digit,
                                           uint32_t* s_above, int* s_wave) {
    const int tid = static_cast<int>(threadIdx.x);
    uint32_t prefix = 0, mask = 0, krem = static_cast<uint32_t>(k);
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        hist[tid] = 0;
        __syncthreads();
        // Lanes of a wavefront whose keys share a digit are found with eight
        // ballots, and one of them adds the group's count: one LDS atomic per
        // distinct digit instead of up to 64 colliding ones (the leading
        // digits of one chunk's keys are nearly all equal).
        for (int b = 0; b < n; b += kThreads) {
            const int i = b + tid;
            const uint32_t key = i < n ? key_at(i) : 0u;
            const bool act = i < n && (key & mask) == prefix;
            const uint32_t dig = (key >> shift) & 255u;
            unsigned long long same = __ballot(act);
#pragma unroll
            for (int bit = 0; bit < 8; ++bit) {
                const unsigned long long ones = __ballot((dig >> bit) & 1u);
                same &= ((dig >> bit) & 1u) ? ones : ~ones;
            }
            if (act && (tid & 63) == __ffsll(static_cast<long long>(same)) - 1)
                atomicAdd(&hist[dig], static_cast<uint32_t>(__popcll(same)));
        }
        __syncthreads();
        // suffix sums over digits (from 255 down): thread t holds digit 255 - t
        const uint32_t cnt = hist[255 - tid];
        uint32_t incl = cnt;
        const int lane = tid & 63;
        const int wave = tid >> 6;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t o = __shfl_up(incl, off, 64);
            if (lane >= off) incl += o;
        }
        if (lane == 63) s_wave[wave] = static_cast<int>(incl);
        __syncthreads();
        uint32_t before = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) before += w < wave ? static_cast<uint32_t>(s_wave[w]) : 0u;
        incl += before;
        const uint32_t excl = incl - cnt;  // keys with a larger digit
        if (excl < krem && incl >= krem) {
            *s_digit = static_cast<uint32_t>(255 - tid);
            *s_above = excl;
        }
        __syncthreads();
        prefix |= *s_digit << shift;
        mask |= 255u << shift;
        krem -= *s_above;
        __syncthreads();
    }
    // prefix is the k-th largest key; take every larger key and the first
    // krem keys equal to it, in index order.
    int running = 0, eq_seen = 0;
    for (int b = 0; b < n; b += kThreads) {
        const int i = b + tid;
        const uint32_t key = i < n ? key_at(i) : 0u;
        const bool gt = i < n && key > prefix;
        const bool eq = i < n && key == prefix;
        int eq_total, sel_total;
        const int eq_rank = eq_seen + block_excl_count(eq, s_wave, &eq_total);
        const bool sel = gt || (eq && eq_rank < static_cast<int>(krem));
        const int pos = running + block_excl_count(sel, s_wave, &sel_total);
        if (sel && pos < k) {
            if (orow != nullptr) orow[pos] = i;
            if (s_sel != nullptr) s_sel[pos] = i;
        }
        running += sel_total;
        eq_seen += eq_total;
    }
}

// LDS_KEYS: the chunk's order keys are staged in LDS (chunks of at most
// kTopkLdsTokens tokens); otherwise every pass reads them from global memory,
// where a chunk's keys (4 bytes per token) stay in L2 across the five passes.
template <bool LDS_KEYS>
__global__ __launch_bounds__(kThreads) void topk_kernel(const float* __restrict__ keys, int64_t T,
                                                        DescArg d, int n_chunks,
                                                        int32_t* __restrict__ out, int kmax, int l0) {
    const DescPtr<SelChunk> chunks = desc_at<SelChunk>(d, 0);
    extern __shared__ uint32_t s_keys[];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_digit, s_above;
    __shared__ int s_wave[kWaves];

    const int l = static_cast<int>(blockIdx.y) + l0;
    const int ci = static_cast<int>(blockIdx.x);
    const SelChunk c = desc_load(chunks + ci);
    const int n = c.n_tokens;
    const int k = min(max(c.k, 0), n);
    int32_t* __restrict__ orow = out + (static_cast<int64_t>(l) * n_chunks + ci) * kmax;
    const int tid = static_cast<int>(threadIdx.x);

    for (int i = k + tid; i < kmax; i += kThreads) orow[i] = -1;
    if (k == 0) return;
    const float* krow = keys + static_cast<int64_t>(l) * T + c.row_offset;
    if (LDS_KEYS)
        for (int i = tid; i < n; i += kThreads) s_keys[i] = order_key(krow[i]);
    const auto key_at = [&](int i) -> uint32_t { return LDS_KEYS ? s_keys[i] : order_key(krow[i]); };
    chunk_topk(key_at, n, k, orow, nullptr, hist, &s_digit, &s_above, s_wave);
}

template <int VW>
__global__ __launch_bounds__(kThreads) void merge_kernel(
    DescArg d, int layer_off, KVGeom g, int es, const int32_t* __restrict__ bt,
    const uint8_t* __restrict__ k_new, const uint8_t* __restrict__ v_new, int64_t T,
    int n_chunks, const int32_t* __restrict__ sel, int kmax, int c0, int l0) {
    const DescPtr<SelChunk> chunks = desc_at<SelChunk>(d, 0);
    const DescPtr<uint8_t*> layers = desc_at<uint8_t*>(d, layer_off);
    using V = typename std::conditional<VW == 16, u32x4, uint8_t>::type;
    const int l = static_cast<int>(blockIdx.z) + l0;
    const int ci = static_cast<int>(blockIdx.y) + c0;
    const SelChunk c = desc_load(chunks + ci);
    const int q0 = static_cast<int>(blockIdx.x) * kMergeTok;
    const int32_t* srow = sel + (static_cast<int64_t>(l) * n_chunks + ci) * kmax;
    uint8_t* __restrict__ base = layers[l];
    const int upr = g.D * es / VW;               // units per head row
    const int per_tok = 2 * g.H * upr;           // K and V rows
    const int items = kMergeTok * per_tok;
    const int64_t rowbytes = static_cast<int64_t>(g.H) * g.D * es;
    for (int it = threadIdx.x; it < items; it += kThreads) {
        const int t = it / per_tok;
        int rem = it - t * per_tok;
        const int kv = rem / (g.H * upr);
        rem -= kv * g.H * upr;
        const int h = rem / upr;
        const int u = rem - h * upr;
        const int q = q0 + t;
        if (q >= kmax || q >= c.k) continue;
        const int j = srow[q];
        if (j < 0 || j >= c.n_tokens) continue;
        if (kv == 1 && g.v_off < 0) continue;
        const int p = c.tok0 + j;
        const int blk = bt[c.bt_offset + p / g.PS];
        if (blk <= 0 || blk >= g.num_blocks) continue;
        const int64_t dst_el = static_cast<int64_t>(blk) * g.sb + static_cast<int64_t>(p % g.PS) * g.ss +
                               static_cast<int64_t>(h) * g.sh + (kv ? g.v_off : 0);
        const uint8_t* src = (kv ? v_new : k_new) +
                             (static_cast<int64_t>(l) * T + c.row_offset + j) * rowbytes +
                             static_cast<int64_t>(h) * g.D * es;
        *reinterpret_cast<V*>(base + dst_el * es + static_cast<int64_t>(u) * VW) =
            *reinterpret_cast<const V*>(src + static_cast<int64_t>(u) * VW);
    }
}

// Row merge for 16-byte-aligned rows. A workgroup writes `tpb` consecutive
// selected slots of one (layer, chunk): its first lanes resolve each slot's
// recomputed row and cache row (selection index, block table) into LDS; then
// its lanes walk the 16-byte source units of those K and V rows, up to
// kMergeUnits per lane, with every load issued before the first store. A lane
// holds only its loaded values and recomputes the addresses from LDS at store
// time (holding 16 destination pointers per lane took 112 VGPRs, capping the
// kernel at 4 waves per SIMD).
// MODE 0 copies bytes (rows and cache share their element type). MODE kBF16 /
// kF16 + 1 quantises bf16 / fp16 rows into an e4m3 cache as vLLM's fp8 cache
// write does: code = saturating RTNE of float32(x) / scale[l, h], the
// division correctly rounded (quant_quotient: one reciprocal per 16-byte unit
// and two FMAs per element instead of a division per element).
constexpr int kMergeUnits = 8;
// 256 lanes x 8 units in flight, nontemporal loads (and stores of copied
// rows): 2% faster for the copy and 4-5% for the quantising merge than plain
// accesses, in alternating processes. A same-process sweep at config 3 put 128
// or 512 lanes, 1 to 16 units, a precomputed slot table, two groups per
// workgroup and one-wavefront-per-token forms within +-2% of this. The
// layer-minor block order (LayerMinor) then took the config-3 merge from
// 704-749 to 622-689 us in same-process A/Bs, about the rate of a page
// scatter of the same bytes onto the same cache layers.
constexpr int kMergeThreads = 256;
constexpr int kMergeMaxTok = 64;
constexpr int kMergeCopy = 0;
constexpr int kMergeFromBF16 = kBF16 + 1;
constexpr int kMergeFromF16 = kF16 + 1;

// Where selected token j of chunk c in layer l is merged: *src, the byte
// offset of its recomputed rows (-1: skip the token: an index outside the
// chunk, or a block id of 0 or outside the cache), and *dst, the byte offset
// of its K row in the layer.
__device__ __forceinline__ void merge_slot(int j, const SelChunk& c, int l, const KVGeom& g, int64_t T,
                                           int64_t row_bytes, int ces, const int32_t* __restrict__ bt,
                                           int64_t* src, int64_t* dst) {
    *src = -1;
    *dst = 0;
    if (j < 0 || j >= c.n_tokens) return;
    const int p = c.tok0 + j;
    const int blk = bt[c.bt_offset + p / g.PS];
    if (blk <= 0 || blk >= g.num_blocks) return;
    *src = (static_cast<int64_t>(l) * T + c.row_offset + j) * row_bytes;
    *dst = (static_cast<int64_t>(blk) * g.sb + static_cast<int64_t>(p % g.PS) * g.ss) * ces;
}

// Copies (or quantises) the K and V rows of n_tok tokens whose slots
// s_src / s_dst (LDS) hold, walking their 16-byte source units in rounds of
// kMergeThreads x kMergeUnits: every load of a round is issued before its
// first store. Shared by merge_rows_kernel (one round per workgroup) and the
// fused selection kernel (all of a chunk's selected tokens).
template <int MODE, bool DENSE>
__device__ __forceinline__ void merge_units(
    int n_tok, const int64_t* s_src, const int64_t* s_dst, int l, uint8_t* __restrict__ base, const KVGeom& g,
    int ces, const uint8_t* __restrict__ k_new, const uint8_t* __restrict__ v_new, int units,
    FastDiv d_tok_units, FastDiv d_upr, const float* __restrict__ k_scales, const float* __restrict__ v_scales) {
    const int tid = static_cast<int>(threadIdx.x);
    const int tok_units = static_cast<int>(d_tok_units.d);   // units per token: K row, then V row
    const int total = n_tok * tok_units;
    const int upr = static_cast<int>(d_upr.d);
    for (int f0 = 0; f0 < total; f0 += kMergeThreads * kMergeUnits) {
        // Every slot loads (lanes past the end reload the last unit, skipped
        // rows read the first unit of k_new) so that the values stay plain
        // registers; only the stores are conditional.
        u32x4 v[kMergeUnits];
#pragma unroll
        for (int s = 0; s < kMergeUnits; ++s) {
            const int f = min(f0 + tid + s * kMergeThreads, total - 1);
            const int t = static_cast<int>(d_tok_units.div(static_cast<uint32_t>(f)));
            const int r = f - t * tok_units;
            const int kv = r >= units ? 1 : 0;
            const int64_t src = s_src[t];
            const uint8_t* p = src >= 0 ? (kv ? v_new : k_new) + src + static_cast<int64_t>(r - kv * units) * 16 : k_new;
            v[s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
        }
        // An opaque copy of the thread index: the compiler would otherwise keep
        // every slot's decoded address alive across the loads (240 VGPRs).
        int tid_s = f0 + tid;
        asm volatile("" : "+v"(tid_s));
#pragma unroll
        for (int s = 0; s < kMergeUnits; ++s) {
            const int f = tid_s + s * kMergeThreads;
            if (f >= total) continue;
            const int t = static_cast<int>(d_tok_units.div(static_cast<uint32_t>(f)));
            const int r = f - t * tok_units;
            const int kv = r >= units ? 1 : 0;
            if (s_src[t] < 0) continue;
            const int u = r - kv * units;
            // DENSE: the head rows of a token are contiguous (sh == D), so unit u
            // of the token row lands at u * (cache bytes per unit)
            const int h = DENSE && MODE == kMergeCopy ? 0 : static_cast<int>(d_upr.div(static_cast<uint32_t>(u)));
            const int un = DENSE ? u : u - h * upr;
            uint8_t* dst = base + s_dst[t] + (static_cast<int64_t>(DENSE ? 0 : h) * g.sh + (kv ? g.v_off : 0)) * ces;
            if constexpr (MODE == kMergeCopy) {
                __builtin_nontemporal_store(v[s], reinterpret_cast<u32x4*>(dst + static_cast<int64_t>(un) * 16));
            } else {
                const QuantDiv qd = quant_div((kv ? v_scales : k_scales)[l * g.H + h]);
                float x[8];
#pragma unroll
                for (int w = 0; w < 4; ++w) Elem<MODE - 1>::unpack_word(v[s][w], x + 2 * w);
                if (qd.fast) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) x[i] = quant_quotient_fast(qd, x[i]);
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) x[i] = x[i] / qd.s;
                }
                u32x2 o;
                o[0] = f32x4_to_e4m3_hw(x);
                o[1] = f32x4_to_e4m3_hw(x + 4);
                *reinterpret_cast<u32x2*>(dst + static_cast<int64_t>(un) * 8) = o;
            }
        }
    }
}

template <int MODE, bool DENSE>
__global__ __launch_bounds__(kMergeThreads) void merge_rows_kernel(
    DescArg d, int layer_off, KVGeom g, int ces, const int32_t* __restrict__ bt,
    const uint8_t* __restrict__ k_new, const uint8_t* __restrict__ v_new, int64_t T,
    int n_chunks, const int32_t* __restrict__ sel, int kmax, int tpb, int units,
    FastDiv d_tok_units, FastDiv d_upr, const float* __restrict__ k_scales,
    const float* __restrict__ v_scales, LayerMinor lm, int64_t nbx) {
    __shared__ int64_t s_src[kMergeMaxTok];   // byte offset of the token's recomputed rows (-1: skip)
    __shared__ int64_t s_dst[kMergeMaxTok];   // byte offset of the token's K row in the layer
    const DescPtr<SelChunk> chunks = desc_at<SelChunk>(d, 0);
    const DescPtr<uint8_t*> layers = desc_at<uint8_t*>(d, layer_off);
    // work item = (chunk, row batch), the batches of a chunk consecutive
    int l;
    int64_t item;
    lm.at(l, item);
    const int ci = static_cast<int>(item / nbx);
    const int bx = static_cast<int>(item - static_cast<int64_t>(ci) * nbx);
    const SelChunk c = desc_load(chunks + ci);
    const int tid = static_cast<int>(threadIdx.x);
    const int ses = MODE == kMergeCopy ? ces : 2;                    // source element size
    const int64_t row_bytes = static_cast<int64_t>(g.H) * g.D * ses;
    if (tid < tpb) {
        const int q = bx * tpb + tid;
        const int j = q < min(kmax, c.k) ? sel[(static_cast<int64_t>(l) * n_chunks + ci) * kmax + q] : -1;
        merge_slot(j, c, l, g, T, row_bytes, ces, bt, &s_src[tid], &s_dst[tid]);
    }
    __syncthreads();
    merge_units<MODE, DENSE>(tpb, s_src, s_dst, l, layers[l], g, ces, k_new, v_new, units, d_tok_units, d_upr,
                             k_scales, v_scales);
}

// The whole selection of one (layer, chunk) in one workgroup: the chunk's
// deviation keys (wave_keys, the fixed order of deviation_kernel; WITH_KEYS
// false: read from `keys` instead), its top-k on the keys held in LDS
// (chunk_topk), then the slots of all its selected tokens (merge_slot) and
// the merge of their rows (merge_units). Keys and indices are written out as
// kv_deviation and topk_per_chunk write them. Dynamic LDS (select_merge_lds):
// n_max order keys, kmax selected indices, kmax source and kmax destination
// offsets.
template <int CK, int NK, int MODE, bool DENSE, bool WITH_KEYS>
__global__ __launch_bounds__(kThreads) void select_merge_kernel(
    DescArg d, int layer_off, KVGeom g, int ces, const int32_t* __restrict__ bt,
    const uint8_t* __restrict__ k_new, const uint8_t* __restrict__ v_new, int64_t T, int n_chunks,
    const float* __restrict__ dev_scales, float* __restrict__ keys, int32_t* __restrict__ sel, int kmax,
    int n_max, int units, FastDiv d_tok_units, FastDiv d_upr, const float* __restrict__ k_scales,
    const float* __restrict__ v_scales, LayerMinor lm) {
    extern __shared__ __align__(16) uint32_t s_dyn[];   // keys, indices, then 8-byte offsets
    __shared__ uint32_t hist[256];
    __shared__ uint32_t s_digit, s_above;
    __shared__ int s_wave[kWaves];
    uint32_t* s_keys = s_dyn;
    int32_t* s_sel = reinterpret_cast<int32_t*>(s_dyn + n_max);
    int64_t* s_src = reinterpret_cast<int64_t*>(s_dyn + ((n_max + kmax + 1) & ~1));
    int64_t* s_dst = s_src + kmax;
    const DescPtr<SelChunk> chunks = desc_at<SelChunk>(d, 0);
    const DescPtr<uint8_t*> layers = desc_at<uint8_t*>(d, layer_off);
    int l;
    int64_t item;
    lm.at(l, item);
    const int ci = static_cast<int>(item);
    const SelChunk c = desc_load(chunks + ci);
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n = c.n_tokens;
    const int k = min(max(c.k, 0), n);
    uint8_t* __restrict__ base = layers[l];
    float* krow = keys + static_cast<int64_t>(l) * T + c.row_offset;
    if constexpr (WITH_KEYS) {
        constexpr int TPW = dev_tok_per_wave<CK>();
        const float* ksc = dev_scales ? dev_scales + static_cast<int64_t>(l) * g.H : nullptr;
        for (int j0 = wave * TPW; j0 < n; j0 += kWaves * TPW) {
            float key[TPW];
            wave_keys<CK, NK, TPW>(c, j0, lane, g, base, bt, k_new, T, l, ksc, key);
#pragma unroll
            for (int i = 0; i < TPW; ++i) {
                const int j = j0 + i;
                if (lane == i && j < n) {
                    krow[j] = key[i];
                    s_keys[j] = order_key(key[i]);
                }
            }
        }
    } else {
        for (int i = tid; i < n; i += kThreads) s_keys[i] = order_key(krow[i]);
    }
    int32_t* __restrict__ orow = sel + (static_cast<int64_t>(l) * n_chunks + ci) * kmax;
    for (int i = k + tid; i < kmax; i += kThreads) orow[i] = -1;
    if (k == 0) return;
    __syncthreads();
    chunk_topk([&](int i) -> uint32_t { return s_keys[i]; }, n, k, orow, s_sel, hist, &s_digit, &s_above,
               s_wave);
    __syncthreads();
    const int ses = MODE == kMergeCopy ? ces : 2;
    const int64_t row_bytes = static_cast<int64_t>(g.H) * g.D * ses;
    for (int q = tid; q < k; q += kThreads) merge_slot(s_sel[q], c, l, g, T, row_bytes, ces, bt, &s_src[q], &s_dst[q]);
    __syncthreads();
    merge_units<MODE, DENSE>(k, s_src, s_dst, l, base, g, ces, k_new, v_new, units, d_tok_units, d_upr,
                             k_scales, v_scales);
}

}  // namespace

int deviation_tile_tokens(int cache_kind) {
    return kWaves * (cache_kind == kE4M3 ? dev_tok_per_wave<kE4M3>() : dev_tok_per_wave<kBF16>());
}

void launch_deviation(const DescArg& d, int layer_off, int n_layers, const KVGeom& g, int cache_kind,
                      const int32_t* block_table, const uint8_t* k_new, int new_kind,
                      int64_t T, int n_chunks, int n_tiles,
                      const float* k_scales, float* keys, hipStream_t stream) {
    for (int l0 = 0; l0 < n_layers; l0 += kMaxGridYZ) {
        const dim3 grid(static_cast<unsigned>(n_tiles), static_cast<unsigned>(std::min(kMaxGridYZ, n_layers - l0)));
#define DARIC_DV(C, N) DARIC_LAUNCH((deviation_kernel<C, N>), grid, kThreads, 0, stream, d, layer_off, g, block_table, k_new, T, n_chunks, k_scales, keys, l0)
        if (new_kind == kBF16) {
            if (cache_kind == kBF16) DARIC_DV(kBF16, kBF16);
            else if (cache_kind == kF16) DARIC_DV(kF16, kBF16);
            else DARIC_DV(kE4M3, kBF16);
        } else {
            if (cache_kind == kBF16) DARIC_DV(kBF16, kF16);
            else if (cache_kind == kF16) DARIC_DV(kF16, kF16);
            else DARIC_DV(kE4M3, kF16);
        }
#undef DARIC_DV
        check_launch("kv_deviation");
    }
}

void launch_topk(const float* keys, int n_layers, int64_t T, const DescArg& d,
                 int n_chunks, int max_tokens, int32_t* out_idx, int kmax, hipStream_t stream) {
    const bool lds = max_tokens <= kTopkLdsTokens;
    const size_t lds_bytes = lds ? static_cast<size_t>(max_tokens) * sizeof(uint32_t) : 0;
    for (int l0 = 0; l0 < n_layers; l0 += kMaxGridYZ) {
        const dim3 grid(static_cast<unsigned>(n_chunks), static_cast<unsigned>(std::min(kMaxGridYZ, n_layers - l0)));
        if (lds)
            DARIC_LAUNCH((topk_kernel<true>), grid, kThreads, lds_bytes, stream, keys, T, d, n_chunks, out_idx, kmax, l0);
        else
            DARIC_LAUNCH((topk_kernel<false>), grid, kThreads, 0, stream, keys, T, d, n_chunks, out_idx, kmax, l0);
        check_launch("topk_per_chunk");
    }
}

bool merge_fits_rows(const KVGeom& g, int elem_size, bool quant) {
    const int ses = quant ? 2 : elem_size;
    if ((g.D * ses) % 16 != 0) return false;
    const int64_t dst_unit = quant ? 8 : 16;     // cache bytes per 16-byte source unit
    if ((g.sb * elem_size) % dst_unit || (g.ss * elem_size) % dst_unit || (g.sh * elem_size) % dst_unit ||
        (g.v_off >= 0 && (g.v_off * elem_size) % dst_unit))
        return false;
    const int64_t tok_units = static_cast<int64_t>(g.v_off >= 0 ? 2 : 1) * g.H * (g.D * ses / 16);
    return tok_units <= static_cast<int64_t>(kMergeThreads) * kMergeUnits;
}

int64_t merge_max_row_bytes() { return static_cast<int64_t>(kMergeThreads) * kMergeUnits * 16; }

void launch_merge(const DescArg& d, int layer_off, int n_layers, const KVGeom& g, int elem_size,
                  const int32_t* block_table, const uint8_t* k_new, const uint8_t* v_new,
                  int64_t T, int n_chunks, const int32_t* sel_idx, int kmax, int quant_from,
                  const float* k_scales, const float* v_scales, hipStream_t stream) {
    const bool quant = quant_from >= 0;
    if (merge_fits_rows(g, elem_size, quant)) {
        // one workgroup per (layer, chunk, batch of tpb selected rows), layer-minor
        const int ses = quant ? 2 : elem_size;
        const int upr = g.D * ses / 16;                              // source units per head row
        const int units = g.H * upr;                                 // per K (or V) token row
        const int tok_units = (g.v_off >= 0 ? 2 : 1) * units;
        const int tpb = std::min(kMergeMaxTok, std::max(1, kMergeThreads * kMergeUnits / tok_units));
        const int64_t nbx = (static_cast<int64_t>(kmax) + tpb - 1) / tpb;
        const FastDiv dtu(static_cast<uint32_t>(tok_units)), dupr(static_cast<uint32_t>(upr));
        const bool dense = g.sh == g.D;
        for_layer_minor(n_layers, nbx * n_chunks, [&](const LayerMinor& lm, unsigned blocks) {
#define DARIC_MR(M, DN) DARIC_LAUNCH((merge_rows_kernel<M, DN>), blocks, kMergeThreads, 0, stream, d, layer_off, g, \
                                     elem_size, block_table, k_new, v_new, T, n_chunks, sel_idx, kmax, tpb, units, \
                                     dtu, dupr, k_scales, v_scales, lm, nbx)
            if (!quant) { if (dense) DARIC_MR(kMergeCopy, true); else DARIC_MR(kMergeCopy, false); }
            else if (quant_from == kBF16) { if (dense) DARIC_MR(kMergeFromBF16, true); else DARIC_MR(kMergeFromBF16, false); }
            else { if (dense) DARIC_MR(kMergeFromF16, true); else DARIC_MR(kMergeFromF16, false); }
#undef DARIC_MR
            check_launch("merge_rows");
        });
        return;
    }
    // grid.y (chunks) and grid.z (layers) are cut into slices of at most 65535
    for (int l0 = 0; l0 < n_layers; l0 += kMaxGridYZ) {
        const int nl = std::min(kMaxGridYZ, n_layers - l0);
        for (int c0 = 0; c0 < n_chunks; c0 += kMaxGridYZ) {
            const int nc = std::min(kMaxGridYZ, n_chunks - c0);
            const dim3 grid(static_cast<unsigned>((kmax + kMergeTok - 1) / kMergeTok), static_cast<unsigned>(nc),
                            static_cast<unsigned>(nl));
            const bool vec = (g.D * elem_size) % 16 == 0 && (g.sb * elem_size) % 16 == 0 &&
                             (g.ss * elem_size) % 16 == 0 && (g.sh * elem_size) % 16 == 0 &&
                             (g.v_off < 0 || (g.v_off * elem_size) % 16 == 0);
            if (vec)
                DARIC_LAUNCH((merge_kernel<16>), grid, kThreads, 0, stream, d, layer_off, g, elem_size, block_table,
                             k_new, v_new, T, n_chunks, sel_idx, kmax, c0, l0);
            else
                DARIC_LAUNCH((merge_kernel<1>), grid, kThreads, 0, stream, d, layer_off, g, elem_size, block_table,
                             k_new, v_new, T, n_chunks, sel_idx, kmax, c0, l0);
            check_launch("merge_rows");
        }
    }
}

// Dynamic LDS of the fused kernel: keys and indices (4 bytes each), then the
// source and destination offsets of the selected tokens (8 bytes each).
size_t select_merge_lds(int64_t max_tokens, int64_t kmax) {
    const int64_t n = std::max<int64_t>(max_tokens, 1), k = std::max<int64_t>(kmax, 1);
    return static_cast<size_t>(((n + k + 1) & ~int64_t(1)) * 4 + 2 * k * 8);
}

constexpr size_t kSelectMergeMaxLds = 48 * 1024;
// A fused workgroup merges its chunk's selected rows alone, in rounds of
// kMergeThreads x kMergeUnits 16-byte units. Up to this many rounds per chunk
// the fused top-k + merge beat topk_kernel + merge_rows_kernel on MI355X
// (config 3: 77 rows of 4 KiB, 10 rounds, 0.635 ms against 0.039 + 0.611 ms,
// both layer-minor); beyond it the merge kernel's spread over (chunk, row
// batch) wins (config 5: 205 quantised rows, 26 rounds, 0.39 ms against
// 0.36 ms).
constexpr int64_t kFusedMaxRounds = 12;

bool select_merge_fits(const KVGeom& g, int elem_size, bool quant, int64_t max_tokens, int64_t kmax,
                       bool one_pass) {
    if (!merge_fits_rows(g, elem_size, quant) || max_tokens > kTopkLdsTokens ||
        select_merge_lds(max_tokens, kmax) > kSelectMergeMaxLds)
        return false;
    const int ses = quant ? 2 : elem_size;
    const int64_t tok_units = static_cast<int64_t>(g.v_off >= 0 ? 2 : 1) * g.H * (g.D * ses / 16);
    const int64_t rounds = (kmax * tok_units + kMergeThreads * kMergeUnits - 1) / (kMergeThreads * kMergeUnits);
    return one_pass || rounds <= kFusedMaxRounds;
}

void launch_select_merge(const DescArg& d, int layer_off, int n_layers, const KVGeom& g, int cache_kind,
                         int elem_size, const int32_t* block_table, const uint8_t* k_new, int new_kind,
                         const uint8_t* v_new, int64_t T, int n_chunks, int max_tokens, bool with_keys,
                         float* keys, int32_t* sel_idx, int kmax, bool quant, const float* k_scales,
                         const float* v_scales, hipStream_t stream) {
    static_assert(kThreads == kMergeThreads, "the fused kernel's merge batches use every lane");
    const int ses = quant ? 2 : elem_size;
    const int upr = g.D * ses / 16;
    const int units = g.H * upr;
    const int tok_units = (g.v_off >= 0 ? 2 : 1) * units;
    const FastDiv dtu(static_cast<uint32_t>(tok_units)), dupr(static_cast<uint32_t>(upr));
    const bool dense = g.sh == g.D;
    const int n_max = std::max(max_tokens, 1);
    const size_t lds = select_merge_lds(max_tokens, kmax);
    // deviation scales: per-head K scales of an fp8 cache (the quantising
    // merge's K scales are the same ones)
    const float* dev_scales = cache_kind == kE4M3 ? k_scales : nullptr;
    // one workgroup per (layer, chunk), layer-minor
    for_layer_minor(n_layers, n_chunks, [&](const LayerMinor& lm, unsigned blocks) {
#define DARIC_SM(C, N, M, DN, WK) DARIC_LAUNCH((select_merge_kernel<C, N, M, DN, WK>), blocks, kThreads, lds, stream, \
                                           d, layer_off, g, elem_size, block_table, k_new, v_new, T, n_chunks, \
                                           dev_scales, keys, sel_idx, kmax, n_max, units, dtu, dupr, \
                                           k_scales, v_scales, lm)
#define DARIC_SM_K(C, N, M, DN) do { if (with_keys) DARIC_SM(C, N, M, DN, true); else DARIC_SM(C, N, M, DN, false); } while (0)
#define DARIC_SM_D(C, N, M) do { if (dense) DARIC_SM_K(C, N, M, true); else DARIC_SM_K(C, N, M, false); } while (0)
        if (cache_kind == kBF16) {
            if (new_kind == kBF16) DARIC_SM_D(kBF16, kBF16, kMergeCopy);
            else DARIC_SM_D(kBF16, kF16, kMergeCopy);
        } else if (cache_kind == kF16) {
            if (new_kind == kBF16) DARIC_SM_D(kF16, kBF16, kMergeCopy);
            else DARIC_SM_D(kF16, kF16, kMergeCopy);
        } else if (quant) {
            if (new_kind == kBF16) DARIC_SM_D(kE4M3, kBF16, kMergeFromBF16);
            else DARIC_SM_D(kE4M3, kF16, kMergeFromF16);
        } else {
            throw Error(DARIC_ERR_INVALID, "select_merge on an fp8 cache merges bf16/fp16 rows with scales");
        }
#undef DARIC_SM_D
#undef DARIC_SM_K
#undef DARIC_SM
        check_launch("select_merge");
    });
}

}  // namespace daric
