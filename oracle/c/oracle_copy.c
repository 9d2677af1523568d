/* CPU restatement, in C, of the page copies and the fused scatter + K
 * re-rotation -- TEST INFRASTRUCTURE ONLY (a second oracle beside the numpy
 * one, and the multithreaded CPU baseline of bench.py).
 *
 * Follows reference csrc/cache_ops/kernels.cu:20-44 (gather) and :98-122
 * (scatter): for prefix index p, selected page s and byte b < span,
 *   gather : store[off + (p*n_sel + s)*span + b] = layer[p*prefix_stride + idx[s]*page_stride + b]
 *   scatter: layer[p*prefix_stride + idx[s]*page_stride + b] = store[off + (p*n_sel + s)*span + b]
 * with pages whose id is 0 (vLLM's null block) -- or outside [0, num_pages),
 * which this build skips instead of touching out-of-bounds memory -- left alone.
 *
 * The rotation follows reference daric/adaption/adapter.py:30-88 (NeoX pairs
 * (i, i + R/2), GPT-J pairs (2i, 2i + 1); out1 = x1 c - x2 s, out2 = x2 c + x1 s)
 * with the angle float32(delta) * inv_freq[i] rounded to float32 and the
 * arithmetic in double, results rounded to float32 and then to the cache
 * type, exactly as oracle/rope.py does it. fp8 values are code value * k_scale[h]
 * and go back as (value / k_scale[h]) saturated to +-448 with
 * round-to-nearest-even.
 *
 * Jobs run in order, one after another; the pages (copies) or tokens
 * (rotation) of one job are spread over threads when they are distinct, so a
 * page or slot listed twice gets the same sequential result as the numpy
 * oracle. Layout checks and the job plan are the Python side's
 * (oracle/copy.py); this file trusts what it is given.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { OC_BF16 = 0, OC_F16 = 1, OC_E4M3 = 2 };

typedef struct oc_layer {
    uint8_t* data;          /* byte address of element [0, ..., 0] */
    int64_t prefix;         /* page-copy shape, bytes (oracle/layout.py page_copy_shape) */
    int64_t num_pages;
    int64_t page_stride;
    int64_t prefix_stride;
    int64_t suffix;
    uint8_t* k_base;        /* byte address of the first K element of block 0, slot 0, head 0 */
    int64_t sb, ss, sh;     /* K view strides in elements: block, slot, head */
    int32_t page_size;      /* tokens per block */
    int32_t heads;
    int32_t kind;           /* OC_BF16, OC_F16 or OC_E4M3 */
    int32_t pad;
    const double* k_scale;  /* NULL (scale 1) or [heads], fp8 only */
} oc_layer;

/* ------------------------------------------------------------ conversions */

static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static double bf16_value(uint16_t h) { return (double)bits_f32((uint32_t)h << 16); }

static uint16_t bf16_code(float f) {
    uint32_t u = f32_bits(f);
    if (isnan(f)) return (uint16_t)(((u >> 16) & 0x8000u) | 0x7fc0u);
    /* round to nearest even on the 16 dropped bits */
    uint32_t lsb = (u >> 16) & 1u;
    return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

static double f16_value(uint16_t h) {
    int sign = h >> 15, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    double v;
    if (e == 0) v = ldexp((double)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexp((double)(m | 0x400), e - 25);
    return sign ? -v : v;
}

/* float -> IEEE binary16, round to nearest even, overflow to infinity. */
static uint16_t f16_code(float f) {
    uint16_t sign = (uint16_t)((f32_bits(f) >> 16) & 0x8000u);
    if (isnan(f)) return (uint16_t)(sign | 0x7e00u);
    double a = fabs((double)f);
    if (a >= 65520.0) return (uint16_t)(sign | 0x7c00u);  /* rounds past 65504 */
    if (a < ldexp(1.0, -14)) {                            /* subnormal: multiples of 2^-24 */
        double q = nearbyint(ldexp(a, 24));               /* default mode: ties to even */
        return (uint16_t)(sign | (uint16_t)q);            /* q == 1024 is the smallest normal */
    }
    int e;
    double fr = frexp(a, &e);                 /* a = fr * 2^e, fr in [0.5, 1) */
    double q = nearbyint(ldexp(fr, 11));      /* 11 significant bits, in [1024, 2048] */
    if (q == 2048.0) { q = 1024.0; ++e; }
    if (e - 1 + 15 >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | (uint16_t)((e - 1 + 15) << 10) | (uint16_t)((int)q - 1024));
}

static double e4m3_value(uint8_t c) {
    int sign = c >> 7, e = (c >> 3) & 0xf, m = c & 7;
    double v;
    if (e == 15 && m == 7) return NAN;
    if (e == 0) v = ldexp((double)m, -9);
    else v = ldexp((double)(8 | m), e - 10);
    return sign ? -v : v;
}

/* float -> OCP e4m3fn, clamped to +-448, round to nearest even. */
static uint8_t e4m3_code(float f) {
    uint8_t sign = (uint8_t)((f32_bits(f) >> 24) & 0x80u);
    if (isnan(f)) return (uint8_t)(sign | 0x7fu);
    double a = fabs((double)f);
    if (a > 448.0) a = 448.0;
    if (a < ldexp(1.0, -6)) {                 /* subnormal: multiples of 2^-9 */
        double q = nearbyint(ldexp(a, 9));
        return (uint8_t)(sign | (uint8_t)q);  /* q == 8 is the smallest normal */
    }
    int e;
    double fr = frexp(a, &e);
    double q = nearbyint(ldexp(fr, 4));       /* 4 significant bits, in [8, 16] */
    if (q == 16.0) { q = 8.0; ++e; }
    int be = e - 1 + 7;
    if (be > 15 || (be == 15 && q > 14.0)) { be = 15; q = 14.0; }  /* 448 */
    return (uint8_t)(sign | (uint8_t)(be << 3) | (uint8_t)((int)q - 8));
}

static double load_value(const uint8_t* p, int kind) {
    if (kind == OC_E4M3) return e4m3_value(*p);
    uint16_t h;
    memcpy(&h, p, 2);
    return kind == OC_BF16 ? bf16_value(h) : f16_value(h);
}

static void store_value(uint8_t* p, int kind, double v) {
    float f = (float)v;
    if (kind == OC_E4M3) { *p = e4m3_code(f); return; }
    uint16_t h = kind == OC_BF16 ? bf16_code(f) : f16_code(f);
    memcpy(p, &h, 2);
}

/* Conversion hooks for the tests: values -> codes (dir 0) or codes -> values
 * (dir 1) over n elements of `kind`. */
void oc_convert(int kind, int dir, int64_t n, const void* in, void* out) {
    const int es = kind == OC_E4M3 ? 1 : 2;
    for (int64_t i = 0; i < n; ++i) {
        if (dir == 0) store_value((uint8_t*)out + i * es, kind, ((const float*)in)[i]);
        else ((double*)out)[i] = load_value((const uint8_t*)in + i * es, kind);
    }
}

/* ------------------------------------------------------------ page copies */

static int cmp_i32(const void* a, const void* b) {
    int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
    return (x > y) - (x < y);
}

/* 1 when every in-range page id of sel appears once. */
static int distinct_pages(const int32_t* sel, int64_t n, int64_t num_pages) {
    int32_t* tmp = (int32_t*)malloc((size_t)(n > 0 ? n : 1) * sizeof(int32_t));
    int64_t k = 0;
    for (int64_t i = 0; i < n; ++i)
        if (sel[i] > 0 && sel[i] < num_pages) tmp[k++] = sel[i];
    qsort(tmp, (size_t)k, sizeof(int32_t), cmp_i32);
    int ok = 1;
    for (int64_t i = 1; i < k && ok; ++i) ok = tmp[i] != tmp[i - 1];
    free(tmp);
    return ok;
}

static void copy_job(const oc_layer* L, uint8_t* store, int64_t off, const int32_t* sel,
                     int64_t n_sel, int gather, int threads) {
    const int64_t n = L->prefix * n_sel;
    const int par = threads > 1 && (gather || distinct_pages(sel, n_sel, L->num_pages));
#pragma omp parallel for schedule(static) num_threads(threads) if (par)
    for (int64_t it = 0; it < n; ++it) {
        const int64_t p = it / n_sel, s = it % n_sel;
        const int64_t page = sel[s];
        if (page <= 0 || page >= L->num_pages) continue;
        uint8_t* cache = L->data + p * L->prefix_stride + page * L->page_stride;
        uint8_t* stage = store + off + (p * n_sel + s) * L->suffix;
        if (gather) memcpy(stage, cache, (size_t)L->suffix);
        else memcpy(cache, stage, (size_t)L->suffix);
    }
}

/* Gather (gather = 1) or scatter (0) of n_jobs jobs: job i copies the pages
 * idx[ioff[i] .. ioff[i+1]) of layers[job_layer[i]] to or from the store at
 * byte offset offsets[i]. */
void oc_copy_pages(const oc_layer* layers, const int32_t* job_layer, const int64_t* offsets,
                   const int32_t* idx, const int64_t* ioff, int64_t n_jobs, uint8_t* store,
                   int gather, int threads) {
    for (int64_t i = 0; i < n_jobs; ++i)
        copy_job(&layers[job_layer[i]], store, offsets[i], idx + ioff[i], ioff[i + 1] - ioff[i],
                 gather, threads);
}

/* --------------------------------------------------------------- rotation */

static inline uint16_t ld16(const uint8_t* p) { uint16_t h; memcpy(&h, p, 2); return h; }
static inline void st16(uint8_t* p, uint16_t h) { memcpy(p, &h, 2); }

static double f16_table[65536];
static double e4m3_table[256];

static void init_tables(void) {
    static int done = 0;
#pragma omp critical(oc_tables)
    if (!done) {
        for (int i = 0; i < 65536; ++i) f16_table[i] = f16_value((uint16_t)i);
        for (int i = 0; i < 256; ++i) e4m3_table[i] = e4m3_value((uint8_t)i);
        done = 1;
    }
}

/* One head row: pairs (e1, e2) = (i, i + half) for NeoX or (2i, 2i + 1). The
 * kind is fixed per loop so each loop keeps only its own conversions. */
static void rotate_row(uint8_t* row, int kind, double scale, const double* c, const double* s,
                       int half, int is_neox) {
    const int st = is_neox ? 1 : 2;          /* element step between pairs */
    const int d2 = is_neox ? half : 1;       /* element distance inside a pair */
    if (kind == OC_BF16) {
        for (int i = 0; i < half; ++i) {
            uint8_t* p1 = row + (int64_t)i * st * 2;
            uint8_t* p2 = p1 + (int64_t)d2 * 2;
            const double x1 = bf16_value(ld16(p1)), x2 = bf16_value(ld16(p2));
            st16(p1, bf16_code((float)(x1 * c[i] - x2 * s[i])));
            st16(p2, bf16_code((float)(x2 * c[i] + x1 * s[i])));
        }
    } else if (kind == OC_F16) {
        for (int i = 0; i < half; ++i) {
            uint8_t* p1 = row + (int64_t)i * st * 2;
            uint8_t* p2 = p1 + (int64_t)d2 * 2;
            const double x1 = f16_table[ld16(p1)], x2 = f16_table[ld16(p2)];
            st16(p1, f16_code((float)(x1 * c[i] - x2 * s[i])));
            st16(p2, f16_code((float)(x2 * c[i] + x1 * s[i])));
        }
    } else {
        for (int i = 0; i < half; ++i) {
            uint8_t* p1 = row + (int64_t)i * st;
            uint8_t* p2 = p1 + d2;
            const double x1 = e4m3_table[*p1] * scale, x2 = e4m3_table[*p2] * scale;
            *p1 = e4m3_code((float)((x1 * c[i] - x2 * s[i]) / scale));
            *p2 = e4m3_code((float)((x2 * c[i] + x1 * s[i]) / scale));
        }
    }
}

static void rotate_token(const oc_layer* L, int64_t page, int64_t slot, const double* c,
                         const double* s, int rotary_dim, int is_neox) {
    const int es = L->kind == OC_E4M3 ? 1 : 2;
    for (int h = 0; h < L->heads; ++h) {
        uint8_t* row = L->k_base + (page * L->sb + slot * L->ss + (int64_t)h * L->sh) * es;
        const double scale = (L->kind == OC_E4M3 && L->k_scale) ? L->k_scale[h] : 1.0;
        rotate_row(row, L->kind, scale, c, s, rotary_dim / 2, is_neox);
    }
}

/* scatter (as oc_copy_pages), then the K rows of the first ntok[i] tokens of
 * job i -- token j at slot j % PS of page sel[j / PS], null and out-of-range
 * pages excluded -- rotated by deltas[i] positions (oracle/copy.py
 * OracleCopier.scatter_pages_rerotate). inv_freq has rotary_dim / 2 entries. */
void oc_scatter_rerotate(const oc_layer* layers, const int32_t* job_layer,
                         const int64_t* offsets, const int32_t* idx, const int64_t* ioff,
                         const int64_t* deltas, const int64_t* ntok, int64_t n_jobs,
                         uint8_t* store, const float* inv_freq, int rotary_dim, int is_neox,
                         int threads) {
    init_tables();
    oc_copy_pages(layers, job_layer, offsets, idx, ioff, n_jobs, store, 0, threads);
    const int half = rotary_dim / 2;
    double* c = (double*)malloc((size_t)(half > 0 ? half : 1) * sizeof(double));
    double* s = (double*)malloc((size_t)(half > 0 ? half : 1) * sizeof(double));
    for (int64_t i = 0; i < n_jobs; ++i) {
        const oc_layer* L = &layers[job_layer[i]];
        const int32_t* sel = idx + ioff[i];
        const int64_t n_sel = ioff[i + 1] - ioff[i];
        const int64_t ps = L->page_size;
        int64_t nt = ntok[i] < n_sel * ps ? ntok[i] : n_sel * ps;
        if (deltas[i] == 0 || nt <= 0) continue;
        for (int k = 0; k < half; ++k) {
            const float a = (float)deltas[i] * inv_freq[k];   /* rounded to float32 */
            c[k] = cos((double)a);
            s[k] = sin((double)a);
        }
        const int par = threads > 1 && distinct_pages(sel, n_sel, L->num_pages);
#pragma omp parallel for schedule(static) num_threads(threads) if (par)
        for (int64_t j = 0; j < nt; ++j) {
            const int64_t page = sel[j / ps];
            if (page <= 0 || page >= L->num_pages) continue;
            rotate_token(L, page, j % ps, c, s, rotary_dim, is_neox);
        }
    }
    free(c);
    free(s);
}
