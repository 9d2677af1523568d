// Element types of a KV cache and their conversions to/from fp32.
//
// All conversions round to nearest even. The fp8 format is OCP e4m3fn
// (bias 7, no infinities, S.1111.111 = NaN, max finite 448); fp32 -> e4m3
// saturates to +-448 instead of producing NaN. The scalar functions compile
// for host and device so host tests can check them exhaustively.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace daric {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__host__ __device__ inline float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
__host__ __device__ inline uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }

// ---- bf16 ----------------------------------------------------------------
__host__ __device__ inline float bf16_to_f32(uint32_t h) { return u2f(h << 16); }

__host__ __device__ inline uint32_t f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u | ((u >> 16) & 0x8000u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// ---- fp16 ----------------------------------------------------------------
__host__ __device__ inline float f16_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
__host__ __device__ inline uint32_t f32_to_f16(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// ---- fp8 e4m3fn ------------------------------------------------------------
__host__ __device__ inline float e4m3_to_f32(uint32_t c) {
    const uint32_t s = (c & 0x80u) << 24;
    const uint32_t em = c & 0x7fu;
    if (em == 0x7fu) return u2f(s | 0x7fc00000u);
    const uint32_t e = em >> 3, m = em & 7u;
    if (e == 0) return u2f(s | f2u((float)m * 0.001953125f));  // m * 2^-9
    return u2f(s | ((e + 120u) << 23) | (m << 20));
}

__host__ __device__ inline uint32_t f32_to_e4m3(float f) {
    const uint32_t u = f2u(f);
    const uint32_t s = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return s | 0x7fu;       // NaN
    if (a >= 0x43e80000u) return s | 0x7eu;      // |f| >= 464 (and inf): saturate
    if (a < 0x3c800000u) {                       // |f| < 2^-6: multiples of 2^-9
        const float q = __builtin_rintf(u2f(a) * 512.0f);
        return s | (uint32_t)q;                  // q == 8 is the smallest normal
    }
    const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
    uint32_t code = (((r >> 23) - 120u) << 3) | ((r >> 20) & 7u);
    if (code > 0x7eu) code = 0x7eu;
    return s | code;
}

// gfx950 conversion instructions (v_cvt_pk_f32_fp8 / v_cvt_pk_fp8_f32, OCP
// e4m3 on this target). The encoder clamps to +-448 first, so the result is
// the saturating RTNE code for every finite input and infinity; NaN inputs
// get the NaN code of their sign (gfx950's conversion: NaN -> 0xff, +inf ->
// 0x7f, -inf -> 0xff). The host pass (never executed) falls back to the
// scalar functions.
__device__ inline void e4m3x4_to_f32_hw(uint32_t w, float* out) {
#ifdef __HIP_DEVICE_COMPILE__
    auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
    auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    out[0] = lo[0]; out[1] = lo[1]; out[2] = hi[0]; out[3] = hi[1];
#else
    for (int b = 0; b < 4; ++b) out[b] = e4m3_to_f32((w >> (8 * b)) & 0xffu);
#endif
}
__device__ inline uint32_t f32x4_to_e4m3_hw(const float* v) {
#ifdef __HIP_DEVICE_COMPILE__
    // The clamp would turn a NaN into a finite value, and the conversion gives
    // every NaN the code 0xff; an infinity of the NaN's sign converts to the
    // NaN code of that sign (0x7f or 0xff), as f32_to_e4m3 encodes NaN.
    float c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        c[i] = v[i] != v[i] ? __builtin_copysignf(__builtin_huge_valf(), v[i])
                            : __builtin_amdgcn_fmed3f(v[i], -448.0f, 448.0f);
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(c[0], c[1], 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c[2], c[3], w, true);
    return static_cast<uint32_t>(w);
#else
    return f32_to_e4m3(v[0]) | (f32_to_e4m3(v[1]) << 8) | (f32_to_e4m3(v[2]) << 16) |
           (f32_to_e4m3(v[3]) << 24);
#endif
}

// ---- x / scale for quantising writes ---------------------------------------
// A cache write quantises x as e4m3(x / scale), the quotient correctly rounded
// to fp32. For scales in [2^-60, 2^60] one correctly rounded reciprocal per
// scale replaces the per-element division: q0 = x * r, the remainder
// x - q0 * scale exactly by one FMA, and one correction q0 + rem * r by a
// second (Markstein's correction step). That gives the correctly rounded
// quotient wherever the code depends on it, and a quotient that saturates the
// same way where it does not (checked for every bf16 and fp16 x against a set
// of scales by the CPU tests). Other scales, NaN among them, divide.
struct QuantDiv {
    float s, r;
    bool fast;
};
__host__ __device__ inline QuantDiv quant_div(float s) {
    QuantDiv d;
    d.s = s;
    d.r = 1.0f / s;
    d.fast = s >= 0x1p-60f && s <= 0x1p60f;
    return d;
}
// The quotient for a scale with d.fast set.
__host__ __device__ inline float quant_quotient_fast(const QuantDiv& d, float x) {
    const float q0 = x * d.r;
    // the negated remainder q0 * scale - x, so that x = -0 ends as
    // -0 + -0 = -0 (with x - q0 * scale it would end as +0)
    const float nrem = __builtin_fmaf(q0, d.s, -x);
    const float q1 = __builtin_fmaf(-nrem, d.r, q0);
    return __builtin_isfinite(q0) ? q1 : q0;   // x infinite or NaN, or the quotient overflowed
}
__host__ __device__ inline float quant_quotient(const QuantDiv& d, float x) {
    return d.fast ? quant_quotient_fast(d, x) : x / d.s;
}

// ---- 16-byte vector <-> fp32 lanes ----------------------------------------
// Kind codes used as template parameters.
enum ElemKind : int { kBF16 = 0, kF16 = 1, kE4M3 = 2 };

template <int KIND> struct Elem;

// Per-32-bit-word forms (EPW elements per word) let a kernel convert, compute
// and repack one word at a time, which keeps few values live in registers.
template <> struct Elem<kBF16> {
    static constexpr int VE = 8;  // elements per 16 bytes
    static constexpr int EPW = 2;
    __device__ static inline void unpack_word(uint32_t w, float* x) {
        x[0] = u2f(w << 16);
        x[1] = u2f(w & 0xffff0000u);
    }
    __device__ static inline uint32_t pack_word(const float* x) {
#ifdef __HIP_DEVICE_COMPILE__
        const f32x2 p = {x[0], x[1]};
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(p, bf16x2));
#else
        return f32_to_bf16(x[0]) | (f32_to_bf16(x[1]) << 16);
#endif
    }
    __device__ static inline void unpack(const u32x4& v, float* x, float) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            x[2 * w] = u2f(v[w] << 16);
            x[2 * w + 1] = u2f(v[w] & 0xffff0000u);
        }
    }
    // gfx950's v_cvt_pk_bf16_f32 rounds to nearest even like f32_to_bf16
    // (checked over every float32 bit pattern on MI355X; NaNs stay NaNs but
    // may keep payload bits that f32_to_bf16 replaces).
    __device__ static inline u32x4 pack(const float* x, float) {
        u32x4 v;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
#ifdef __HIP_DEVICE_COMPILE__
            const f32x2 p = {x[2 * w], x[2 * w + 1]};
            v[w] = __builtin_bit_cast(uint32_t, __builtin_convertvector(p, bf16x2));
#else
            v[w] = f32_to_bf16(x[2 * w]) | (f32_to_bf16(x[2 * w + 1]) << 16);
#endif
        }
        return v;
    }
};

template <> struct Elem<kF16> {
    static constexpr int VE = 8;
    static constexpr int EPW = 2;
    __device__ static inline void unpack_word(uint32_t w, float* x) {
        x[0] = f16_to_f32(w & 0xffffu);
        x[1] = f16_to_f32(w >> 16);
    }
    __device__ static inline uint32_t pack_word(const float* x) {
        return f32_to_f16(x[0]) | (f32_to_f16(x[1]) << 16);
    }
    __device__ static inline void unpack(const u32x4& v, float* x, float) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t word = v[w];
            x[2 * w] = f16_to_f32(word & 0xffffu);
            x[2 * w + 1] = f16_to_f32(word >> 16);
        }
    }
    __device__ static inline u32x4 pack(const float* x, float) {
        u32x4 v;
#pragma unroll
        for (int w = 0; w < 4; ++w) v[w] = f32_to_f16(x[2 * w]) | (f32_to_f16(x[2 * w + 1]) << 16);
        return v;
    }
};

// fp8 values are dequantised as code_value * scale and requantised as
// sat_rtne(value * (1 / scale)).
template <> struct Elem<kE4M3> {
    static constexpr int VE = 16;
    static constexpr int EPW = 4;
    __device__ static inline void unpack_word(uint32_t w, float* x) {
#ifdef DARIC_FP8_SOFTWARE
#pragma unroll
        for (int b = 0; b < 4; ++b) x[b] = e4m3_to_f32((w >> (8 * b)) & 0xffu);
#else
        e4m3x4_to_f32_hw(w, x);
#endif
    }
    __device__ static inline uint32_t pack_word(const float* x) {
#ifdef DARIC_FP8_SOFTWARE
        return f32_to_e4m3(x[0]) | (f32_to_e4m3(x[1]) << 8) | (f32_to_e4m3(x[2]) << 16) |
               (f32_to_e4m3(x[3]) << 24);
#else
        return f32x4_to_e4m3_hw(x);
#endif
    }
    __device__ static inline void unpack(const u32x4& v, float* x, float scale) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
#ifdef DARIC_FP8_SOFTWARE
#pragma unroll
            for (int b = 0; b < 4; ++b) x[4 * w + b] = e4m3_to_f32((v[w] >> (8 * b)) & 0xffu);
#else
            e4m3x4_to_f32_hw(v[w], x + 4 * w);
#endif
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] *= scale;
    }
    __device__ static inline u32x4 pack(const float* x, float inv_scale) {
        float y[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) y[i] = x[i] * inv_scale;
        u32x4 v;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
#ifdef DARIC_FP8_SOFTWARE
            v[w] = f32_to_e4m3(y[4 * w]) | (f32_to_e4m3(y[4 * w + 1]) << 8) |
                   (f32_to_e4m3(y[4 * w + 2]) << 16) | (f32_to_e4m3(y[4 * w + 3]) << 24);
#else
            v[w] = f32x4_to_e4m3_hw(y + 4 * w);
#endif
        }
        return v;
    }
};

}  // namespace daric
