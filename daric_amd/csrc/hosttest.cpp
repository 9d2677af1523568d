// Host-only hooks for the CPU test suite: the scalar element conversions and
// the fast divider that the kernels use, compiled for the host from the same
// headers. Not part of the product ABI (include/daric_cache_ops.h).
#include <cstdint>
#include <vector>

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


// Walks the launches for_layer_minor makes for n_layers x n_items and
// decodes every block with LayerMinor::at_block. Returns the number of
// launches when every (layer, item) pair is covered exactly once and no
// launch exceeds kMaxGridBlocks, else -1 (a pair missed, repeated or out of
// range) or -2 (an oversized launch).
int64_t daric_hosttest_layer_minor(int n_layers, int64_t n_items) {
    std::vector<uint8_t> seen(static_cast<size_t>(n_layers) * static_cast<size_t>(n_items), 0);
    int64_t launches = 0;
    bool bad = false, big = false;
    daric::for_layer_minor(n_layers, n_items, [&](const daric::LayerMinor& lm, unsigned blocks) {
        ++launches;
        if (static_cast<int64_t>(blocks) > daric::kMaxGridBlocks || blocks == 0) big = true;
        for (uint32_t b = 0; b < blocks; ++b) {
            int l;
            int64_t w;
            lm.at_block(b, l, w);
            if (l < 0 || l >= n_layers || w < 0 || w >= n_items) { bad = true; continue; }
            uint8_t& s = seen[static_cast<size_t>(l) * static_cast<size_t>(n_items) + static_cast<size_t>(w)];
            if (s) bad = true;
            s = 1;
        }
    });
    for (uint8_t s : seen)
        if (!s) bad = true;
    if (big) return -2;
    return bad ? -1 : launches;
}

}
