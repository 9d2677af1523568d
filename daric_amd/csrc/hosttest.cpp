// Host-only hooks for the CPU test suite: the scalar element conversions and
// the fast divider that the kernels use, compiled for the host from the same
// headers. Not part of the product ABI (include/daric_cache_ops.h).
#include <cstdint>

#include "elem.h"
#include "kernels.h"

extern "C" {

uint32_t daric_hosttest_f32_to_bf16(float f) { return daric::f32_to_bf16(f); }
uint32_t daric_hosttest_f32_to_f16(float f) { return daric::f32_to_f16(f); }
uint32_t daric_hosttest_f32_to_e4m3(float f) { return daric::f32_to_e4m3(f); }
float daric_hosttest_e4m3_to_f32(uint32_t c) { return daric::e4m3_to_f32(c); }

// Encodes n floats into out (uint8 codes).
void daric_hosttest_encode_e4m3(const float* in, uint8_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = static_cast<uint8_t>(daric::f32_to_e4m3(in[i]));
}
void daric_hosttest_encode_bf16(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = static_cast<uint16_t>(daric::f32_to_bf16(in[i]));
}

// out[i * n_x + j] = the quantising writes' quotient of x[j] by scales[i].
void daric_hosttest_quant_quotients(const float* x, int64_t n_x, const float* scales, int64_t n_s,
                                    float* out) {
    for (int64_t i = 0; i < n_s; ++i) {
        const daric::QuantDiv d = daric::quant_div(scales[i]);
        for (int64_t j = 0; j < n_x; ++j) out[i * n_x + j] = daric::quant_quotient(d, x[j]);
    }
}

// Returns the number of n in [n0, n1) for which FastDiv(d).div(n) != n / d.
int64_t daric_hosttest_fastdiv_errors(uint32_t d, uint32_t n0, uint32_t n1) {
    const daric::FastDiv f(d);
    int64_t bad = 0;
    for (uint64_t n = n0; n < n1; ++n)
        if (f.div(static_cast<uint32_t>(n)) != static_cast<uint32_t>(n) / d) ++bad;
    return bad;
}

}
