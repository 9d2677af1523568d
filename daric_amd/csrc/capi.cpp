// C ABI of the KV-reuse hot path: CacheCopier, batched copies, re-rotation,
// recompute selection. Host-side validation follows the reference's checks
// (csrc/cache_ops/helpers.cu:15-174, copier.cpp:7-111, kernels.cu:127-330)
// in the same order and with the same messages; no device work is enqueued
// before every check has passed.
#include <optional>
#include <algorithm>
#include <limits>
#include <map>
#include <string>
#include <string_view>
#include <tuple>
#include <unordered_map>

#include "common.h"
#include "elem.h"
#include "kernels.h"

using namespace daric;

namespace {

constexpr int64_t kInt64Max = std::numeric_limits<int64_t>::max();
constexpr int64_t kIntMax = std::numeric_limits<int>::max();
constexpr int64_t kMaxTiles = (1ll << 24) - 1;  // grid.x * 256 lanes must stay < 2^32

int64_t checked_multiply(int64_t lhs, int64_t rhs, const char* context) {
    DARIC_CHECK(lhs >= 0 && rhs >= 0, context, " must be non-negative");
    DARIC_CHECK(lhs == 0 || rhs <= kInt64Max / lhs, context, " exceeds int64 range");
    return lhs * rhs;
}

// helpers.cu:22-64
int64_t dense_span_elements(const daric_tensor& t, int first_dim) {
    struct Dim { int dim; int64_t size, stride; };
    std::vector<Dim> dims;
    for (int d = first_dim; d < t.ndim; ++d) {
        const int64_t size = t.sizes[d], stride = t.strides[d];
        DARIC_CHECK(size > 0, "KV cache copy dimensions must be non-empty", " | shape=", sizes_str(t),
                    " | stride=", strides_str(t), " | failed_dim=", d);
        if (size == 1) continue;
        DARIC_CHECK(stride > 0, "KV cache non-singleton dimensions must have positive strides",
                    " | shape=", sizes_str(t), " | stride=", strides_str(t), " | failed_dim=", d,
                    " | actual_stride=", stride);
        dims.push_back({d, size, stride});
    }
    std::sort(dims.begin(), dims.end(), [](const Dim& a, const Dim& b) { return a.stride < b.stride; });
    int64_t expected = 1;
    for (const auto& dm : dims) {
        DARIC_CHECK(dm.stride == expected, "KV cache copy dimensions must form a dense physical span",
                    " | shape=", sizes_str(t), " | stride=", strides_str(t), " | failed_dim=", dm.dim,
                    " | expected_stride=", expected, " | actual_stride=", dm.stride,
                    " | relation=", dm.stride > expected ? "hole" : "overlap");
        expected = checked_multiply(expected, dm.size, "KV cache dense span");
    }
    return expected;
}

// helpers.cu:66-90
void validate_outer_regions(const daric_tensor& t, int64_t prefix_size, int64_t num_pages,
                            int64_t prefix_stride, int64_t page_stride, int64_t suffix) {
    std::vector<std::pair<int64_t, int64_t>> axes;
    if (prefix_size > 1) axes.emplace_back(prefix_stride, prefix_size);
    if (num_pages > 1) axes.emplace_back(page_stride, num_pages);
    std::sort(axes.begin(), axes.end());
    int64_t occupied = suffix;
    for (const auto& [stride, size] : axes) {
        DARIC_CHECK(stride >= occupied, "KV cache prefix/page regions overlap", " | shape=",
                    sizes_str(t), " | stride=", strides_str(t), " | region_size=", suffix,
                    " | required_stride=", occupied, " | actual_stride=", stride);
        const int64_t extent = checked_multiply(size - 1, stride, "KV cache outer span");
        DARIC_CHECK(extent <= kInt64Max - occupied, "KV cache outer span exceeds int64 range");
        occupied += extent;
    }
}

struct PageShape {
    int64_t num_pages, prefix_size, page_stride, suffix, prefix_stride;
};

// helpers.cu:94-148
PageShape page_copy_shape(const daric_tensor& t, bool page_first) {
    DARIC_CHECK(t.device >= 0, "KV cache tensor must be on CUDA");
    DARIC_CHECK(t.ndim >= 1, "KV cache tensor must have at least one dimension");
    const int64_t e = t.elem_size;
    PageShape s{};
    if (page_first) {
        DARIC_CHECK(t.sizes[0] > 0, "page dimension must be non-zero");
        DARIC_CHECK(t.sizes[0] <= kIntMax, "number of pages exceeds int range: ", t.sizes[0]);
        s.num_pages = t.sizes[0];
        s.prefix_size = 1;
        s.prefix_stride = 0;
        s.page_stride = checked_multiply(t.strides[0], e, "KV cache page stride");
        s.suffix = checked_multiply(dense_span_elements(t, 1), e, "KV cache page span");
        if (s.num_pages > 1)
            DARIC_CHECK(s.page_stride >= s.suffix, "KV cache pages overlap", " | shape=", sizes_str(t),
                        " | stride=", strides_str(t), " | page_stride=", s.page_stride,
                        " | page_span=", s.suffix);
    } else {
        DARIC_CHECK(t.ndim >= 2, "non-page-first KV cache tensor must have at least two dimensions");
        DARIC_CHECK(t.sizes[0] > 0, "prefix dimension must be non-zero");
        DARIC_CHECK(t.sizes[1] > 0, "page dimension must be non-zero");
        DARIC_CHECK(t.sizes[0] <= kIntMax, "prefix size exceeds int range: ", t.sizes[0]);
        DARIC_CHECK(t.sizes[1] <= kIntMax, "number of pages exceeds int range: ", t.sizes[1]);
        s.prefix_size = t.sizes[0];
        s.num_pages = t.sizes[1];
        s.prefix_stride = checked_multiply(t.strides[0], e, "KV cache prefix stride");
        s.page_stride = checked_multiply(t.strides[1], e, "KV cache page stride");
        s.suffix = checked_multiply(dense_span_elements(t, 2), e, "KV cache suffix span");
        validate_outer_regions(t, s.prefix_size, s.num_pages, s.prefix_stride, s.page_stride, s.suffix);
    }
    DARIC_CHECK(s.page_stride > 0, "page_stride must be positive");
    return s;
}

// helpers.cu:150-174
void validate_common_job_inputs(int64_t n_jobs, const int64_t* offsets, int64_t n_offsets,
                                const int64_t* byte_sizes, int64_t n_byte_sizes,
                                const int64_t* indices_offsets, int64_t n_indices_offsets,
                                const daric_tensor* indices) {
    DARIC_CHECK(n_offsets == n_jobs && offsets != nullptr, "offsets length mismatch");
    DARIC_CHECK(n_byte_sizes == n_jobs && byte_sizes != nullptr, "byte_sizes length mismatch");
    DARIC_CHECK(n_indices_offsets == n_jobs + 1 && indices_offsets != nullptr,
                "indices_offsets size must be num_jobs + 1");
    check_tensor_struct(indices, "indices_flat");
    DARIC_CHECK(indices->device >= 0, "indices_flat must be on CUDA");
    DARIC_CHECK(indices->ndim == 1, "indices_flat must be 1D");
    DARIC_CHECK(indices->dtype == DARIC_DTYPE_INT32, "indices_flat must be int32");
    DARIC_CHECK(is_contiguous(*indices), "indices_flat must be contiguous");
    DARIC_CHECK(indices_offsets[0] >= 0, "indices_offsets[0] must be non-negative");
    DARIC_CHECK(indices_offsets[n_jobs] <= numel(*indices),
                "indices_offsets.back() exceeds indices_flat.numel()");
    for (int64_t i = 0; i < n_jobs; ++i) {
        DARIC_CHECK(offsets[i] >= 0, "negative store offset at job ", i);
        DARIC_CHECK(byte_sizes[i] >= 0, "negative byte size at job ", i);
        DARIC_CHECK(indices_offsets[i] >= 0, "negative indices offset at job ", i);
        DARIC_CHECK(indices_offsets[i] <= indices_offsets[i + 1],
                    "indices_offsets must be non-decreasing at job ", i);
    }
}

int elem_kind(const daric_tensor& t) {
    switch (t.dtype) {
        case DARIC_DTYPE_BFLOAT16: return kBF16;
        case DARIC_DTYPE_FLOAT16: return kF16;
        case DARIC_DTYPE_UINT8:
        case DARIC_DTYPE_FP8_E4M3FN: return kE4M3;
        default: return -1;
    }
}

const char* quant_name(int kind) { return kind == kBF16 ? "bfloat16" : "float16"; }

// Rotary layout resolution of reference adapter.py:311-368.
struct RopeLayout {
    int64_t PS, H, D, sb, ss, sh, num_blocks, row_width;
};

RopeLayout rope_layout(const daric_tensor& t, bool page_first, int rotary_dim) {
    RopeLayout r{};
    if (t.ndim == 5) {
        r.PS = t.sizes[2]; r.H = t.sizes[3]; r.D = t.sizes[4];
        if (page_first) { r.sb = t.strides[0]; r.num_blocks = t.sizes[0]; }
        else { r.sb = t.strides[1]; r.num_blocks = t.sizes[1]; }
        r.ss = t.strides[2]; r.sh = t.strides[3];
        r.row_width = r.D;
        DARIC_CHECK(t.strides[4] == 1 || r.D == 1, "KV cache head_dim stride must equal 1 for rerotate");
    } else if (t.ndim == 4) {
        const char* constraint = nullptr;
        if (!page_first) constraint = "page_first must be true";
        else if (t.sizes[3] <= 0 || t.sizes[3] % 2 != 0) constraint = "packed content dimension must be positive and even";
        else if (t.strides[3] != 1) constraint = "packed content feature stride must equal 1";
        const int64_t hd = t.sizes[3] / 2;
        if (!constraint && (rotary_dim <= 0 || rotary_dim % 2 != 0 || rotary_dim > hd))
            constraint = "rotary_dim must be positive, even, and no greater than the packed K head dimension";
        if (constraint)
            throw Error(DARIC_ERR_VALUE,
                        cat("Invalid 4D KV cache for rerotate: shape=", sizes_str(t), ", stride=",
                            strides_str(t), ", rotary_dim=", rotary_dim, ", constraint=", constraint));
        r.PS = t.sizes[2]; r.H = t.sizes[1]; r.D = hd;
        r.sb = t.strides[0]; r.ss = t.strides[2]; r.sh = t.strides[1];
        r.num_blocks = t.sizes[0];
        r.row_width = 2 * hd;
    } else if (t.ndim == 3) {
        r.PS = t.sizes[1]; r.H = 1; r.D = t.sizes[2];
        r.sb = t.strides[0]; r.ss = t.strides[1]; r.sh = 0;
        r.num_blocks = t.sizes[0];
        r.row_width = r.D;
        DARIC_CHECK(t.strides[2] == 1 || r.D == 1, "KV cache hidden stride must equal 1 for rerotate");
    } else {
        throw Error(DARIC_ERR_VALUE, cat("Unsupported KV cache rank for rerotate: ", t.ndim));
    }
    DARIC_CHECK(rotary_dim > 0 && rotary_dim % 2 == 0 && rotary_dim <= r.D,
                "rotary_dim must be positive, even and no greater than head_dim (", r.D,
                "), got ", rotary_dim);
    DARIC_CHECK(r.num_blocks <= kIntMax && r.PS <= kIntMax && r.H <= kIntMax,
                "KV cache dimensions exceed int range");
    return r;
}

void check_rope(const daric_rope* rope) {
    DARIC_CHECK(rope != nullptr, "rope parameters must not be null");
    DARIC_CHECK(rope->inv_freq != nullptr, "inv_freq must not be null");
    DARIC_CHECK(rope->rotary_dim > 0 && rope->rotary_dim % 2 == 0 && rope->rotary_dim / 2 <= 256,
                "rotary_dim must be positive, even and at most 512, got ", rope->rotary_dim);
}

bool aligned(const void* p, int64_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

hipStream_t as_stream(uint64_t s) { return reinterpret_cast<hipStream_t>(static_cast<uintptr_t>(s)); }

}  // namespace

// ====================================================================== copier
struct daric_copier {
    struct Layer {
        daric_tensor t;
        bool page_first;
        const float* k_scale = nullptr;
        int64_t k_scale_numel = 0;
        // Page-copy shape of the tensor, computed once at registration. A
        // layout the copy path rejects keeps its error here; it is raised when
        // a job uses the layer, as the reference raises it at call time.
        PageShape shape{};
        int shape_status = DARIC_OK;
        std::string shape_msg;
        // Rotary row geometry for the last (rotary_dim, is_neox) the fused
        // path asked for (geom_rot == 0: not computed yet).
        int geom_rot = 0;
        int geom_neox = -1;
        int geom_status = DARIC_OK;
        std::string geom_msg;   // rope_layout error, or why row_geometry refused
        bool geom_ok = false;
        RopeLayout lay{};
        RowGeom geom{};
    };
    std::unordered_map<std::string, Layer> layers;
    // Lookup index keyed by views of the map's own key strings (the map's
    // nodes are stable), so resolving a const char* allocates nothing.
    std::unordered_map<std::string_view, Layer*> by_name;
    daric_tensor store{};
    bool has_store = false;
    std::mutex mu;  // registration vs. lookups from concurrent calls
};

namespace {

struct ResolvedJobs {
    std::vector<CopyJob> jobs;
    std::vector<daric_copier::Layer*> layers;
    int64_t max_tiles = 0;
    int64_t max_elements = 0;
    int64_t max_span = 0;
    int vw = 16;
    int device = -1;
};

// Shared front half of every page-list copy: the reference's check order
// (copier.cpp:46-66). Returns the jobs' layers (empty for an empty job list).
std::vector<daric_copier::Layer*> resolve_front(daric_copier* c, const char* const* names,
                                               int64_t n_jobs, const int64_t* offsets,
                                               int64_t n_offsets, const int64_t* byte_sizes,
                                               int64_t n_byte_sizes, const daric_tensor* indices,
                                               const int64_t* indices_offsets,
                                               int64_t n_indices_offsets, bool gather) {
    std::vector<daric_copier::Layer*> layers;
    DARIC_CHECK(c->has_store, "store buffer not registered; call register_store() first");
    if (n_jobs == 0) return layers;
    DARIC_CHECK(n_jobs > 0 && names != nullptr, "layer_names must not be empty");
    DARIC_CHECK(n_jobs <= kIntMax, "too many jobs in one call: ", n_jobs);
    validate_common_job_inputs(n_jobs, offsets, n_offsets, byte_sizes, n_byte_sizes, indices_offsets,
                               n_indices_offsets, indices);
    const int64_t store_size = numel(c->store);
    for (int64_t i = 0; i < n_jobs; ++i) {
        DARIC_CHECK(offsets[i] >= 0, "negative store offset at job ", i);
        DARIC_CHECK(byte_sizes[i] >= 0, "negative store byte size at job ", i);
        DARIC_CHECK(offsets[i] <= store_size, "store offset out of range at job ", i);
        DARIC_CHECK(byte_sizes[i] <= store_size - offsets[i], "store range out of bounds at job ", i);
    }
    layers.reserve(n_jobs);
    for (int64_t i = 0; i < n_jobs; ++i) {
        DARIC_CHECK(names[i] != nullptr, "layer not registered: (null)");
        auto it = c->by_name.find(std::string_view(names[i]));
        DARIC_CHECK(it != c->by_name.end(), "layer not registered: ", names[i]);
        layers.push_back(it->second);
    }
    const int device = layers[0]->t.device;
    DARIC_CHECK(indices->device == device, "indices_flat must be on the same device as kvcache");
    for (int64_t i = 0; i < n_jobs; ++i) {
        DARIC_CHECK(layers[i]->t.device >= 0, gather ? "all source layers must be CUDA tensors; job "
                                                     : "all destination layers must be CUDA tensors; job ", i);
        DARIC_CHECK(layers[i]->t.device == device,
                    gather ? "all source layers must be on the same device; job "
                           : "all destination layers must be on the same device; job ", i);
    }
    return layers;
}

// gather/scatter_pages: the front half, then the launcher's per-job shape and
// byte-size checks (kernels.cu:135-161).
ResolvedJobs resolve_jobs(daric_copier* c, const char* const* names, int64_t n_jobs,
                          const int64_t* offsets, int64_t n_offsets, const int64_t* byte_sizes,
                          int64_t n_byte_sizes, const daric_tensor* indices,
                          const int64_t* indices_offsets, int64_t n_indices_offsets, bool gather) {
    ResolvedJobs r;
    r.layers = resolve_front(c, names, n_jobs, offsets, n_offsets, byte_sizes, n_byte_sizes, indices,
                             indices_offsets, n_indices_offsets, gather);
    if (r.layers.empty()) return r;
    r.device = r.layers[0]->t.device;
    uint8_t* store = static_cast<uint8_t*>(c->store.data);
    const int32_t* idx = static_cast<const int32_t*>(indices->data);
    r.jobs.resize(n_jobs);
    bool a16 = aligned(store, 16), a4 = aligned(store, 4);
    for (int64_t i = 0; i < n_jobs; ++i) {
        const daric_tensor& t = r.layers[i]->t;
        if (r.layers[i]->shape_status != DARIC_OK)
            throw Error(r.layers[i]->shape_status, r.layers[i]->shape_msg);
        const PageShape& s = r.layers[i]->shape;
        const int64_t n_sel = indices_offsets[i + 1] - indices_offsets[i];
        const int64_t num = s.prefix_size * n_sel * s.suffix;
        if (byte_sizes[i] != num)
            throw Error(DARIC_ERR_RUNTIME,
                        cat("byte_size mismatch at job ", i, " | C++ expected bytes: ", num,
                            " | Python passed bytes: ", byte_sizes[i], " | Tensor shape: ",
                            sizes_str(t), " | Tensor strides: ", strides_str(t)));
        DARIC_CHECK(n_sel <= kIntMax, "too many selected pages at job ", i);
        DARIC_CHECK(s.suffix <= kIntMax, "page span exceeds int range at job ", i);
        CopyJob& j = r.jobs[i];
        j.layer = static_cast<uint8_t*>(t.data);
        j.stage = store + offsets[i];
        j.idx = idx + indices_offsets[i];
        j.prefix_stride = s.prefix_stride;
        j.page_stride = s.page_stride;
        j.span = s.suffix;
        j.n_sel = static_cast<int32_t>(n_sel);
        j.prefix = static_cast<int32_t>(s.prefix_size);
        j.num_pages = static_cast<int32_t>(s.num_pages);
        j.n_tokens = 0;
        j.delta = 0.0f;
        r.max_tiles = std::max(r.max_tiles, s.prefix_size * n_sel);
        r.max_elements = std::max(r.max_elements, num);
        r.max_span = std::max(r.max_span, s.suffix);
        const auto al = [&](int64_t a) {
            return s.suffix % a == 0 && s.page_stride % a == 0 && s.prefix_stride % a == 0 &&
                   offsets[i] % a == 0 && aligned(t.data, a);
        };
        a16 = a16 && al(16);
        a4 = a4 && al(4);
    }
    DARIC_CHECK(r.max_tiles <= kMaxTiles, "too many pages in one job: ", r.max_tiles);
    r.vw = a16 ? 16 : (a4 ? 4 : 1);
    return r;
}

// Token-major view of a KV layer for gather/scatter_tokens, in elements.
struct TokenLayout {
    int64_t PS, H, D, sb, ss, sh, v_off, num_blocks;
    int n_kv;
};

TokenLayout token_layout(const daric_tensor& t, bool page_first) {
    TokenLayout r{};
    if (t.ndim == 5) {
        // [2, NB, PS, H, D] or page-first [NB, 2, PS, H, D], any strides
        r.PS = t.sizes[2]; r.H = t.sizes[3]; r.D = t.sizes[4];
        const int kv_dim = page_first ? 1 : 0;
        DARIC_CHECK(t.sizes[kv_dim] == 2, "token-major copies need a K/V dimension of size 2, got shape=",
                    sizes_str(t));
        r.v_off = t.strides[kv_dim];
        r.sb = t.strides[page_first ? 0 : 1];
        r.num_blocks = t.sizes[page_first ? 0 : 1];
        r.ss = t.strides[2]; r.sh = t.strides[3];
        r.n_kv = 2;
        DARIC_CHECK(t.strides[4] == 1 || r.D == 1, "KV cache head_dim stride must equal 1 for token-major copies");
    } else if (t.ndim == 4) {
        // packed [NB, H, PS, 2D]: K in [0, D), V in [D, 2D) of every row
        DARIC_CHECK(page_first, "a 4-D (packed) KV cache must be page_first");
        DARIC_CHECK(t.sizes[3] > 0 && t.sizes[3] % 2 == 0 && t.strides[3] == 1,
                    "packed KV rows must have an even, contiguous last dimension, got shape=", sizes_str(t),
                    ", stride=", strides_str(t));
        r.PS = t.sizes[2]; r.H = t.sizes[1]; r.D = t.sizes[3] / 2;
        r.sb = t.strides[0]; r.ss = t.strides[2]; r.sh = t.strides[1];
        r.v_off = r.D;
        r.num_blocks = t.sizes[0];
        r.n_kv = 2;
    } else if (t.ndim == 3) {
        // MLA [NB, PS, hidden]: one latent row per token, no V
        r.PS = t.sizes[1]; r.H = 1; r.D = t.sizes[2];
        r.sb = t.strides[0]; r.ss = t.strides[1]; r.sh = 0; r.v_off = 0;
        r.num_blocks = t.sizes[0];
        r.n_kv = 1;
        DARIC_CHECK(t.strides[2] == 1 || r.D == 1, "KV cache hidden stride must equal 1 for token-major copies");
    } else {
        throw Error(DARIC_ERR_INVALID, cat("Unsupported KV cache rank for token-major copies: ", t.ndim));
    }
    DARIC_CHECK(r.PS > 0 && r.H > 0 && r.D > 0, "token-major copies need non-empty pages, got shape=",
                sizes_str(t));
    DARIC_CHECK(r.num_blocks <= kIntMax && r.PS <= kIntMax && r.H <= kIntMax && r.D * t.elem_size <= kIntMax,
                "KV cache dimensions exceed int range");
    return r;
}

int copy_tokens(daric_copier* c, const char* const* names, int64_t n_jobs, const int64_t* offsets,
                int64_t n_offsets, const int64_t* byte_sizes, int64_t n_byte_sizes,
                const daric_tensor* indices, const int64_t* indices_offsets,
                int64_t n_indices_offsets, uint64_t stream, bool gather) {
    return guarded([&] {
        DARIC_CHECK(c != nullptr, "copier must not be null");
        std::lock_guard<std::mutex> lk(c->mu);
        const auto layers = resolve_front(c, names, n_jobs, offsets, n_offsets, byte_sizes, n_byte_sizes,
                                          indices, indices_offsets, n_indices_offsets, gather);
        if (layers.empty()) return;
        const int device = layers[0]->t.device;
        uint8_t* store = static_cast<uint8_t*>(c->store.data);
        const int32_t* idx = static_cast<const int32_t*>(indices->data);
        std::vector<TokenJob> jobs(n_jobs);
        std::vector<int64_t> units_per_row(n_jobs);
        bool vec = true, lds = true;
        for (int64_t i = 0; i < n_jobs; ++i) {
            const daric_tensor& t = layers[i]->t;
            if (layers[i]->shape_status != DARIC_OK) throw Error(layers[i]->shape_status, layers[i]->shape_msg);
            const TokenLayout L = token_layout(t, layers[i]->page_first);
            const int64_t e = t.elem_size;
            const int64_t n_sel = indices_offsets[i + 1] - indices_offsets[i];
            const int64_t row = checked_multiply(checked_multiply(L.PS * L.H, L.D, "token-major rows"), e,
                                                 "token-major rows");
            const int64_t num = checked_multiply(checked_multiply(L.n_kv, n_sel, "token-major rows"), row,
                                                 "token-major rows");
            if (byte_sizes[i] != num)
                throw Error(DARIC_ERR_RUNTIME,
                            cat("byte_size mismatch at job ", i, " | C++ expected bytes: ", num,
                                " | Python passed bytes: ", byte_sizes[i], " | Tensor shape: ",
                                sizes_str(t), " | Tensor strides: ", strides_str(t)));
            DARIC_CHECK(n_sel <= kIntMax, "too many selected pages at job ", i);
            TokenJob& j = jobs[i];
            j.layer = static_cast<uint8_t*>(t.data);
            j.stage = store + offsets[i];
            j.idx = idx + indices_offsets[i];
            j.sb = L.sb * e; j.ss = L.ss * e; j.sh = L.sh * e; j.v_off = L.v_off * e;
            j.n_sel = static_cast<int32_t>(n_sel);
            j.num_blocks = static_cast<int32_t>(L.num_blocks);
            j.PS = static_cast<int32_t>(L.PS);
            j.H = static_cast<int32_t>(L.H);
            j.row_bytes = static_cast<int32_t>(L.D * e);
            j.n_kv = L.n_kv;
            const bool a16 = j.row_bytes % 16 == 0 && j.sb % 16 == 0 && j.ss % 16 == 0 && j.sh % 16 == 0 &&
                             j.v_off % 16 == 0 && aligned(t.data, 16) && aligned(j.stage, 16);
            vec = vec && a16;
            // head-major dense pages with rows of >= 128 bytes take the LDS transpose
            lds = lds && a16 && j.H > 1 && j.ss == j.row_bytes && j.sh == static_cast<int64_t>(j.PS) * j.row_bytes &&
                  j.row_bytes >= 128 && static_cast<int64_t>(j.H) * (j.row_bytes / 16) <= 512;
        }
        const int vw = vec ? 16 : 1;
        int64_t max_parts = 0, part_bytes = 0;
        for (TokenJob& j : jobs) {
            const int64_t row_units = j.row_bytes / vw;
            const int64_t head_units = static_cast<int64_t>(j.H) * row_units;
            int64_t pt;
            if (lds) pt = std::max<int64_t>(1, 512 / head_units);                 // 8 KiB of LDS
            else pt = std::max<int64_t>(1, (vw == 16 ? 16384 : 4096) / (static_cast<int64_t>(j.H) * j.row_bytes));
            pt = std::min<int64_t>(pt, j.PS);
            j.part_tokens = static_cast<int32_t>(pt);
            j.parts_per_page = static_cast<int32_t>((j.PS + pt - 1) / pt);
            j.d_upr = FastDiv(static_cast<uint32_t>(row_units));
            j.d_h = FastDiv(static_cast<uint32_t>(j.H));
            DARIC_CHECK(pt * head_units <= kIntMax, "page part exceeds int range");
            max_parts = std::max<int64_t>(max_parts, static_cast<int64_t>(j.n_kv) * j.n_sel * j.parts_per_page);
            part_bytes = std::max<int64_t>(part_bytes, pt * j.H * j.row_bytes);
        }
        if (max_parts == 0) return;
        DARIC_CHECK(max_parts <= kMaxTiles, "too many pages in one job: ", max_parts);
        DeviceGuard guard(device);
        const hipStream_t st = as_stream(stream);
        DescHandOver ho(device, jobs.data(), jobs.size() * sizeof(TokenJob), st);
        launch_token_copy(ho.arg(), static_cast<int>(jobs.size()), static_cast<int>(max_parts), part_bytes,
                          vw, lds, gather, st);
    });
}

int copy_pages(daric_copier* c, const char* const* names, int64_t n_jobs, const int64_t* offsets,
               int64_t n_offsets, const int64_t* byte_sizes, int64_t n_byte_sizes,
               const daric_tensor* indices, const int64_t* indices_offsets,
               int64_t n_indices_offsets, uint64_t stream, bool gather) {
    return guarded([&] {
        DARIC_CHECK(c != nullptr, "copier must not be null");
        std::lock_guard<std::mutex> lk(c->mu);
        ResolvedJobs r = resolve_jobs(c, names, n_jobs, offsets, n_offsets, byte_sizes, n_byte_sizes,
                                      indices, indices_offsets, n_indices_offsets, gather);
        if (r.jobs.empty() || r.max_elements == 0) return;
        DeviceGuard guard(r.device);
        const hipStream_t st = as_stream(stream);
        DescHandOver ho(r.device, r.jobs.data(), r.jobs.size() * sizeof(CopyJob), st);
        launch_copy_pages(ho.arg(), static_cast<int>(r.jobs.size()), static_cast<int>(r.max_tiles),
                          r.max_span, r.vw, gather, st);
    });
}

// Row model of a page span for the fused kernel; returns false when the
// layout does not have dense K head rows (the fused path then refuses).
bool row_geometry(const daric_tensor& t, bool page_first, const RopeLayout& L, int rotary_dim,
                  bool neox, int64_t span_bytes, RowGeom* out, std::string* why) {
    const int64_t e = t.elem_size;
    const int64_t W = L.row_width;
    const int kind = elem_kind(t);
    const int64_t VE = kind == kE4M3 ? 16 : 8;
    int64_t tok_div;
    if (L.H == 1 || L.PS == 1) {
        tok_div = L.H == 1 ? 1 : L.H;
        if (L.H == 1 && L.PS > 1 && L.ss != W) { *why = "token rows are not dense"; return false; }
        if (L.PS == 1 && L.H > 1 && L.sh != W) { *why = "head rows are not dense"; return false; }
    } else if (L.ss == L.H * W && L.sh == W) {
        tok_div = L.H;  // [.., PS, H, D]
    } else if (L.sh == L.PS * W && L.ss == W) {
        tok_div = 1;    // [.., H, PS, D]
    } else {
        *why = "K head rows are not dense in the page span";
        return false;
    }
    const int64_t krows = L.PS * L.H;
    int64_t n_rows = krows;
    if (t.ndim == 5 && page_first) {
        if (t.strides[1] != krows * W) { *why = "the V half does not follow the K half in a page"; return false; }
        n_rows = 2 * krows;
    }
    if (n_rows * W * e != span_bytes) { *why = "page span is not the K/V head rows"; return false; }
    if ((W * e) % 16 != 0) { *why = "row bytes are not a multiple of 16"; return false; }
    const int64_t rot_units_elems = neox ? rotary_dim / 2 : rotary_dim;
    if (rot_units_elems % VE != 0) { *why = "rotary pairs are not 16-byte aligned"; return false; }
    RowGeom g{};
    g.W = static_cast<int32_t>(W);
    g.n_rows = static_cast<int32_t>(n_rows);
    g.krows = static_cast<int32_t>(krows);
    g.tok_div = static_cast<int32_t>(tok_div);
    g.PS = static_cast<int32_t>(L.PS);
    g.H = static_cast<int32_t>(L.H);
    g.R = rotary_dim;
    g.n_rot = static_cast<int32_t>(rot_units_elems / VE);
    g.ipr = static_cast<int32_t>(g.n_rot + (W - rotary_dim) / VE);
    *out = g;
    return true;
}

}  // namespace

extern "C" {

int daric_copier_create(daric_copier** out) {
    return guarded([&] {
        DARIC_CHECK(out != nullptr, "out must not be null");
        *out = new daric_copier();
    });
}

int daric_copier_destroy(daric_copier* copier) {
    return guarded([&] { delete copier; });
}

int daric_copier_register_layer(daric_copier* c, const char* name, const daric_tensor* tensor,
                                int is_page_first) {
    return guarded([&] {
        DARIC_CHECK(c != nullptr && name != nullptr, "copier and name must not be null");
        check_tensor_struct(tensor, "kvcache tensor");
        DARIC_CHECK(tensor->device >= 0, "kvcache tensor must be on GPU: ", name);
        std::lock_guard<std::mutex> lk(c->mu);
        daric_copier::Layer L;
        L.t = *tensor;
        L.page_first = is_page_first != 0;
        try {
            L.shape = page_copy_shape(L.t, L.page_first);
        } catch (const Error& e) {
            L.shape_status = e.status;
            L.shape_msg = e.what();
        }
        auto it = c->layers.find(name);
        if (it != c->layers.end()) {
            L.k_scale = it->second.k_scale;
            L.k_scale_numel = it->second.k_scale_numel;
        }
        auto res = c->layers.insert_or_assign(name, std::move(L));
        c->by_name[std::string_view(res.first->first)] = &res.first->second;
    });
}

int daric_copier_register_store(daric_copier* c, const daric_tensor* buffer) {
    return guarded([&] {
        DARIC_CHECK(c != nullptr, "copier must not be null");
        check_tensor_struct(buffer, "store buffer");
        DARIC_CHECK(buffer->device >= 0, "staging buffer must be on CUDA");
        DARIC_CHECK(buffer->ndim == 1, "store buffer must be 1D");
        DARIC_CHECK(buffer->dtype == DARIC_DTYPE_UINT8, "store buffer must be uint8");
        DARIC_CHECK(is_contiguous(*buffer), "store buffer must be contiguous");
        std::lock_guard<std::mutex> lk(c->mu);
        c->store = *buffer;
        c->has_store = true;
    });
}

int daric_copier_register_k_scale(daric_copier* c, const char* name, const daric_tensor* k_scale) {
    return guarded([&] {
        DARIC_CHECK(c != nullptr && name != nullptr, "copier and name must not be null");
        std::lock_guard<std::mutex> lk(c->mu);
        auto it = c->layers.find(name);
        DARIC_CHECK(it != c->layers.end(), "layer not registered: ", name);
        if (k_scale == nullptr || k_scale->data == nullptr) {
            it->second.k_scale = nullptr;
            it->second.k_scale_numel = 0;
            return;
        }
        DARIC_CHECK(k_scale->device == it->second.t.device, "k_scale must be on the layer's device");
        DARIC_CHECK(k_scale->dtype == DARIC_DTYPE_FLOAT32 && is_contiguous(*k_scale),
                    "k_scale must be a contiguous float32 tensor");
        it->second.k_scale = static_cast<const float*>(k_scale->data);
        it->second.k_scale_numel = numel(*k_scale);
    });
}

int daric_copier_gather_pages(daric_copier* c, const char* const* names, int64_t n_jobs,
                              const int64_t* offsets, int64_t n_offsets, const int64_t* byte_sizes,
                              int64_t n_byte_sizes, const daric_tensor* indices,
                              const int64_t* indices_offsets, int64_t n_indices_offsets,
                              uint64_t stream) {
    return copy_pages(c, names, n_jobs, offsets, n_offsets, byte_sizes, n_byte_sizes, indices,
                      indices_offsets, n_indices_offsets, stream, true);
}

int daric_copier_scatter_pages(daric_copier* c, const char* const* names, int64_t n_jobs,
                              const int64_t* offsets, int64_t n_offsets, const int64_t* byte_sizes,
                              int64_t n_byte_sizes, const daric_tensor* indices,
                              const int64_t* indices_offsets, int64_t n_indices_offsets,
                              uint64_t stream) {
    return copy_pages(c, names, n_jobs, offsets, n_offsets, byte_sizes, n_byte_sizes, indices,
                      indices_offsets, n_indices_offsets, stream, false);
}

int daric_copier_gather_tokens(daric_copier* c, const char* const* names, int64_t n_jobs,
                               const int64_t* offsets, int64_t n_offsets, const int64_t* byte_sizes,
                               int64_t n_byte_sizes, const daric_tensor* indices,
                               const int64_t* indices_offsets, int64_t n_indices_offsets,
                               uint64_t stream) {
    return copy_tokens(c, names, n_jobs, offsets, n_offsets, byte_sizes, n_byte_sizes, indices,
                       indices_offsets, n_indices_offsets, stream, true);
}

int daric_copier_scatter_tokens(daric_copier* c, const char* const* names, int64_t n_jobs,
                                const int64_t* offsets, int64_t n_offsets, const int64_t* byte_sizes,
                                int64_t n_byte_sizes, const daric_tensor* indices,
                                const int64_t* indices_offsets, int64_t n_indices_offsets,
                                uint64_t stream) {
    return copy_tokens(c, names, n_jobs, offsets, n_offsets, byte_sizes, n_byte_sizes, indices,
                       indices_offsets, n_indices_offsets, stream, false);
}

}  // extern "C"

namespace {

// ---- in-place re-rotation planning (shared with daric_rerotate_pages)

// All layers of one call must share shape, strides, dtype and device.
void check_same_layers(const daric_tensor* layers, int64_t n) {
    const daric_tensor& a = layers[0];
    for (int64_t i = 1; i < n; ++i) {
        const daric_tensor& b = layers[i];
        bool same = a.ndim == b.ndim && a.dtype == b.dtype && a.elem_size == b.elem_size &&
                    a.device == b.device;
        for (int d = 0; same && d < a.ndim; ++d)
            same = a.sizes[d] == b.sizes[d] && a.strides[d] == b.strides[d];
        DARIC_CHECK(same, "all layers of one call must share shape, strides, dtype and device; layer ", i,
                    " differs");
    }
}

void check_block_table(const daric_tensor* bt, int device) {
    check_tensor_struct(bt, "block_table");
    DARIC_CHECK(bt->device == device, "block_table must be on the layers' device");
    DARIC_CHECK(bt->ndim == 1 && bt->dtype == DARIC_DTYPE_INT32 && is_contiguous(*bt),
                "block_table must be a 1-D contiguous int32 tensor");
}

std::vector<uint8_t*> layer_ptrs(const daric_tensor* layers, int64_t n) {
    std::vector<uint8_t*> v(n);
    for (int64_t i = 0; i < n; ++i) v[i] = static_cast<uint8_t*>(layers[i].data);
    return v;
}

// A validated in-place rotation: the geometry, kernel path and descriptor
// bytes (segments, then the layer pointer table) of one call.
struct InplacePlan {
    InplaceGeom g{};
    std::vector<uint8_t> blob;
    int seg_bytes = 0, n_layers = 0, n_segs = 0, path = kRotElem, kind = 0, device = -1;
    int64_t tiles = 0;
    bool neox = false;
    const int32_t* block_table = nullptr;
    const float* inv_freq = nullptr;
};

// Every check of daric_rerotate_pages, and the plan of its launch; no device
// work. Segments with no tokens or no shift are dropped (n_segs may be 0).
// min_block: block ids below it are skipped (1 also skips the null block).
InplacePlan plan_inplace(const daric_tensor* layers, int64_t n_layers, int page_first,
                     const daric_tensor* block_table, const daric_rope_segment* segments,
                     int64_t n_segments, const daric_rope* rope, const daric_tensor* k_scales,
                     int min_block) {
    InplacePlan plan;
    DARIC_CHECK(n_layers > 0 && layers != nullptr, "layers must not be empty");
    DARIC_CHECK(n_segments > 0 && segments != nullptr, "segments must not be null");
    check_rope(rope);
    for (int64_t i = 0; i < n_layers; ++i) check_tensor_struct(&layers[i], "kv layer");
    check_same_layers(layers, n_layers);
    const daric_tensor& t = layers[0];
    DARIC_CHECK(t.device >= 0, "KV cache tensor must be on CUDA");
    const int kind = elem_kind(t);
    DARIC_CHECK(kind >= 0, "unsupported KV cache dtype for rerotate");
    const RopeLayout L = rope_layout(t, page_first != 0, rope->rotary_dim);
    check_block_table(block_table, t.device);
    const int64_t bt_n = numel(*block_table);
    if (k_scales != nullptr && k_scales->data != nullptr) {
        DARIC_CHECK(k_scales->device == t.device && k_scales->dtype == DARIC_DTYPE_FLOAT32 &&
                    is_contiguous(*k_scales) && numel(*k_scales) == n_layers * L.H,
                    "k_scales must be a contiguous float32 [n_layers, H] tensor on the layers' device");
    }
    const bool neox = rope->is_neox != 0;
    const int64_t e = t.elem_size;
    const int64_t VE = kind == kE4M3 ? 16 : 8;
    const int64_t half = rope->rotary_dim / 2;
    bool vec = (L.sb * e) % 16 == 0 && (L.ss * e) % 16 == 0 && (L.sh * e) % 16 == 0 &&
               (neox ? half % VE == 0 : rope->rotary_dim % VE == 0);
    for (int64_t i = 0; i < n_layers && vec; ++i) vec = aligned(layers[i].data, 16);

    InplaceGeom& g = plan.g;
    g.min_block = min_block;
    g.sb = L.sb; g.ss = L.ss; g.sh = L.sh;
    g.PS = static_cast<int32_t>(L.PS);
    g.H = static_cast<int32_t>(L.H);
    g.R = rope->rotary_dim;
    g.num_blocks = static_cast<int32_t>(L.num_blocks);
    g.n_rot = static_cast<int32_t>(vec ? (neox ? half / VE : rope->rotary_dim / VE) : half);
    const int64_t per_tok = L.H * g.n_rot;
    // about 1024 items (vector path) or 2048 pairs (element path) per tile
    const int64_t tile_items = vec ? 1024 : 2048;
    g.tile_tokens = static_cast<int32_t>(std::max<int64_t>(1, tile_items / std::max<int64_t>(per_tok, 1)));
    // Page tiles (rerotate_lane_kernel) when a page's K rows are dense
    // rows of a power-of-two number (<= 64) of 16-byte units.
    int path = vec ? kRotVec : kRotElem;
    if (vec) {
        const int64_t W = L.row_width;
        const int64_t upr = W * e / 16;
        int64_t tok_div = 0;
        if (L.H == 1 && L.ss == W) tok_div = 1;
        else if (L.H > 1 && L.ss == L.H * W && L.sh == W) tok_div = L.H;     // [PS, H, W] rows
        else if (L.H > 1 && L.sh == L.PS * W && L.ss == W) tok_div = 1;      // [H, PS, W] rows
        if (tok_div > 0 && (W * e) % 16 == 0 && upr > 0 && upr <= 64 && (upr & (upr - 1)) == 0 &&
            L.PS * L.H * upr <= kIntMax) {
            path = kRotLane;
            g.upr = static_cast<int32_t>(upr);
            g.tok_div = static_cast<int32_t>(tok_div);
            // page tiles in parts of at least 16 KiB (whole rows each): two
            // halves of a 32 KiB bf16 K page measured ~1% faster at config 2
            const int64_t units = L.PS * L.H * upr;
            int lp = 0;
            while ((units >> (lp + 1)) * 16 >= 16384 && units % (2ll << lp) == 0 &&
                   (units >> (lp + 1)) % upr == 0)
                ++lp;
            g.log2_parts = lp;
        }
    }

    std::vector<RopeSeg> segs;
    int64_t tiles = 0;
    for (int64_t i = 0; i < n_segments; ++i) {
        const daric_rope_segment& s = segments[i];
        DARIC_CHECK(s.n_tokens >= 0 && s.tok_start >= 0 && s.bt_offset >= 0,
                    "negative segment field at segment ", i);
        DARIC_CHECK(s.delta > -(1ll << 24) && s.delta < (1ll << 24), "delta out of range at segment ", i);
        if (s.n_tokens == 0 || s.delta == 0) continue;
        DARIC_CHECK(s.tok_start + s.n_tokens <= kIntMax, "segment too long at segment ", i);
        const int64_t last_block = (s.tok_start + s.n_tokens - 1) / L.PS;
        DARIC_CHECK(s.bt_offset + last_block < bt_n, "segment ", i,
                    " reads past the end of block_table");
        RopeSeg rs{};
        rs.bt_offset = s.bt_offset;
        rs.tok_start = static_cast<int32_t>(s.tok_start);
        rs.n_tokens = static_cast<int32_t>(s.n_tokens);
        rs.delta = static_cast<float>(s.delta);
        rs.tile_begin = static_cast<int32_t>(tiles);
        if (path == kRotLane)
            tiles += (last_block - s.tok_start / L.PS + 1) << g.log2_parts;   // the pages the segment touches
        else
            tiles += (s.n_tokens + g.tile_tokens - 1) / g.tile_tokens;
        segs.push_back(rs);
    }
    DARIC_CHECK(tiles <= kMaxTiles, "too many tokens in one rerotate call");
    if (segs.empty()) return plan;
    const size_t seg_bytes = segs.size() * sizeof(RopeSeg);
    plan.blob.resize(seg_bytes + n_layers * sizeof(uint8_t*));
    std::memcpy(plan.blob.data(), segs.data(), seg_bytes);
    const auto ptrs = layer_ptrs(layers, n_layers);
    std::memcpy(plan.blob.data() + seg_bytes, ptrs.data(), n_layers * sizeof(uint8_t*));
    plan.seg_bytes = static_cast<int>(seg_bytes);
    plan.n_layers = static_cast<int>(n_layers);
    plan.n_segs = static_cast<int>(segs.size());
    plan.path = path;
    plan.kind = kind;
    plan.device = t.device;
    plan.tiles = tiles;
    plan.neox = neox;
    plan.block_table = static_cast<const int32_t*>(block_table->data);
    plan.inv_freq = rope->inv_freq;
    return plan;
}

void launch_inplace(const InplacePlan& p, hipStream_t st) {
    DescHandOver ho(p.device, p.blob.data(), p.blob.size(), st);
    launch_rerotate_inplace(ho.arg(), p.seg_bytes, p.n_layers, p.g, p.n_segs, static_cast<int>(p.tiles),
                            p.block_table, p.inv_freq, p.kind, p.neox, p.path, st);
}


// scatter_pages_rerotate for layouts the fused kernel does not take: the
// jobs are scattered by the copy kernel, then each layer's moved tokens are
// rotated in place (one in-place call per layer, over the job's page ids).
// Pages with id 0 are skipped by both, as the fused kernel skips them. Every
// rotation is planned, and so validated, before the scatter is enqueued.
void scatter_then_rotate(const ResolvedJobs& r, const daric_tensor* indices, const int64_t* indices_offsets,
                         const int64_t* deltas, const int64_t* num_tokens, const daric_rope* rope,
                         uint64_t stream) {
    std::vector<daric_copier::Layer*> order;
    std::unordered_map<daric_copier::Layer*, std::vector<daric_rope_segment>> segs;
    for (size_t i = 0; i < r.jobs.size(); ++i) {
        daric_copier::Layer* L = r.layers[i];
        const int64_t page_tokens = static_cast<int64_t>(r.jobs[i].n_sel) * L->lay.PS;
        const int64_t n = std::min(num_tokens[i], page_tokens);
        if (deltas[i] == 0 || n <= 0) continue;
        auto it = segs.find(L);
        if (it == segs.end()) {
            order.push_back(L);
            it = segs.emplace(L, std::vector<daric_rope_segment>{}).first;
        }
        it->second.push_back(daric_rope_segment{indices_offsets[i], 0, n, deltas[i]});
    }
    std::vector<InplacePlan> plans;
    for (daric_copier::Layer* L : order) {
        const auto& sv = segs[L];
        InplacePlan p = plan_inplace(&L->t, 1, L->page_first ? 1 : 0, indices, sv.data(),
                                     static_cast<int64_t>(sv.size()), rope, nullptr, 1);
        if (p.n_segs > 0) plans.push_back(std::move(p));
    }
    DeviceGuard guard(r.device);
    const hipStream_t st = as_stream(stream);
    {
        DescHandOver ho(r.device, r.jobs.data(), r.jobs.size() * sizeof(CopyJob), st);
        launch_copy_pages(ho.arg(), static_cast<int>(r.jobs.size()), static_cast<int>(r.max_tiles), r.max_span,
                          r.vw, false, st);
    }
    for (const InplacePlan& p : plans) launch_inplace(p, st);
}

// scatter_pages_rerotate and its allocation-free variant: the same checks
// and kernels; they differ only in how the job descriptors reach the kernels
// when they do not fit in the kernel arguments (the ring, or the static
// scratch array).
int scatter_rerotate(daric_copier* c, const char* const* names, int64_t n_jobs, const int64_t* offsets,
                     int64_t n_offsets, const int64_t* byte_sizes, int64_t n_byte_sizes,
                     const daric_tensor* indices, const int64_t* indices_offsets, int64_t n_indices_offsets,
                     const int64_t* deltas, const int64_t* num_tokens, const daric_rope* rope,
                     uint64_t stream, bool noalloc) {
    return guarded([&] {
        DARIC_CHECK(c != nullptr, "copier must not be null");
        std::lock_guard<std::mutex> lk(c->mu);
        ResolvedJobs r = resolve_jobs(c, names, n_jobs, offsets, n_offsets, byte_sizes, n_byte_sizes,
                                      indices, indices_offsets, n_indices_offsets, false);
        if (r.jobs.empty() || r.max_elements == 0) return;
        check_rope(rope);
        DARIC_CHECK(deltas != nullptr && num_tokens != nullptr, "deltas and num_tokens must not be null");
        // The fused kernel needs 16-byte aligned pages and dense K head rows
        // whose rotated halves are 16-byte multiples; otherwise the call
        // scatters with the copy kernel and then rotates in place.
        bool fused = r.vw == 16;
        // Group jobs by row geometry and element type; one launch per group
        // (normally one: every layer of a model shares its geometry).
        struct Group {
            int kind;
            RowGeom g;
            std::vector<CopyJob> jobs;
            int64_t max_tiles = 0;
        };
        std::vector<Group> groups;
        for (int64_t i = 0; i < n_jobs; ++i) {
            daric_copier::Layer* L = r.layers[i];
            const int kind = elem_kind(L->t);
            DARIC_CHECK(kind >= 0, "unsupported KV cache dtype for rerotate at job ", i);
            DARIC_CHECK(deltas[i] > -(1ll << 24) && deltas[i] < (1ll << 24),
                        "delta out of range at job ", i, ": ", deltas[i]);
            DARIC_CHECK(num_tokens[i] >= 0, "negative num_tokens at job ", i);
            const int neox = rope->is_neox != 0 ? 1 : 0;
            if (L->geom_rot != rope->rotary_dim || L->geom_neox != neox) {
                L->geom_rot = rope->rotary_dim;
                L->geom_neox = neox;
                L->geom_status = DARIC_OK;
                L->geom_msg.clear();
                L->geom_ok = false;
                try {
                    L->lay = rope_layout(L->t, L->page_first, rope->rotary_dim);
                    L->geom_ok = row_geometry(L->t, L->page_first, L->lay, rope->rotary_dim, neox != 0,
                                              L->shape.suffix, &L->geom, &L->geom_msg);
                } catch (const Error& e) {
                    L->geom_status = e.status;
                    L->geom_msg = e.what();
                }
            }
            if (L->geom_status != DARIC_OK) throw Error(L->geom_status, L->geom_msg);
            DARIC_CHECK(L->k_scale == nullptr || L->k_scale_numel >= L->lay.H,
                        "k_scale of job ", i, " has ", L->k_scale_numel, " entries, the layer has ",
                        L->lay.H, " heads");
            fused = fused && L->geom_ok;
            CopyJob& j = r.jobs[i];
            j.delta = static_cast<float>(deltas[i]);
            j.n_tokens = static_cast<int32_t>(std::min<int64_t>(num_tokens[i], kIntMax));
            Group* grp = nullptr;
            for (auto& gr : groups)
                if (gr.kind == kind && std::memcmp(&gr.g, &L->geom, sizeof(RowGeom)) == 0) { grp = &gr; break; }
            if (grp == nullptr) {
                groups.push_back(Group{kind, L->geom, {}, 0});
                grp = &groups.back();
                grp->jobs.reserve(n_jobs);
            }
            grp->jobs.push_back(j);
            grp->max_tiles = std::max<int64_t>(grp->max_tiles, int64_t(j.prefix) * j.n_sel);
        }
        if (!fused) {
            DARIC_CHECK(!noalloc, "scatter_pages_rerotate_noalloc needs a layout the fused kernel takes "
                                  "(16-byte aligned pages, dense K head rows, 16-byte rotated halves)");
            scatter_then_rotate(r, indices, indices_offsets, deltas, num_tokens, rope, stream);
            return;
        }
        // Allocation-free variant: job sets that do not travel inline are
        // staged in the static scratch array, one region per launch group.
        size_t staged = 0;
        if (noalloc) {
            for (const Group& gr : groups) {
                const size_t b = gr.jobs.size() * sizeof(CopyJob);
                if (gr.max_tiles > 0 && b > static_cast<size_t>(kInlineDescBytes)) staged += (b + 255) / 256 * 256;
            }
            DARIC_CHECK(staged <= kNoAllocScratchBytes, "scatter_pages_rerotate_noalloc: the jobs' descriptors need ",
                        staged, " bytes of scratch, more than the ", kNoAllocScratchBytes, " bytes (",
                        kNoAllocScratchBytes / sizeof(CopyJob), " jobs) it holds; split the call");
        }
        DeviceGuard guard(r.device);
        const hipStream_t st = as_stream(stream);
        // staged descriptors: this call's turn on the GPU's scratch array
        std::optional<ScratchUse> use;
        if (staged > 0) use.emplace(r.device, st);
        uint8_t* scratch = use ? use->ptr() : nullptr;
        size_t scratch_off = 0;
        for (const Group& gr : groups) {
            if (gr.max_tiles == 0) continue;
            RowGeomDiv gd;
            gd.g = gr.g;
            gd.ipr = FastDiv(gd.g.ipr);
            gd.tok_div = FastDiv(gd.g.tok_div);
            gd.ps = FastDiv(gd.g.PS);
            const size_t bytes = gr.jobs.size() * sizeof(CopyJob);
            if (noalloc) {
                DescArg arg;
                arg.ptr = nullptr;
                arg.reserved = 0;
                if (bytes <= static_cast<size_t>(kInlineDescBytes)) {
                    std::memcpy(arg.inl, gr.jobs.data(), bytes);
                } else {
                    stash_descriptors(gr.jobs.data(), bytes, scratch + scratch_off, st);
                    arg.ptr = scratch + scratch_off;
                    scratch_off += (bytes + 255) / 256 * 256;
                }
                launch_scatter_rotate(arg, static_cast<int>(gr.jobs.size()), static_cast<int>(gr.max_tiles),
                                      gd, gr.kind, rope->is_neox != 0, rope->inv_freq, st);
                continue;
            }
            // Job sets too large to travel inline are read by the fused
            // kernels straight from the pinned slot (one 80-byte read per
            // workgroup of at least 16 KiB): no upload kernel and no
            // dependency gap before them, ~4 us less per call on MI355X. The
            // copy kernels keep the upload: their 8 KiB workgroups are more,
            // and reading over the host link cost the gather ~5 us.
            DescHandOver ho(r.device, gr.jobs.data(), bytes, st, true);
            launch_scatter_rotate(ho.arg(), static_cast<int>(gr.jobs.size()), static_cast<int>(gr.max_tiles),
                                  gd, gr.kind, rope->is_neox != 0, rope->inv_freq, st);
        }
        if (use) use->finish();
    });
}

}  // namespace

extern "C" {

int daric_copier_scatter_pages_rerotate(daric_copier* c, const char* const* names, int64_t n_jobs,
                                        const int64_t* offsets, int64_t n_offsets,
                                        const int64_t* byte_sizes, int64_t n_byte_sizes,
                                        const daric_tensor* indices,
                                        const int64_t* indices_offsets, int64_t n_indices_offsets,
                                        const int64_t* deltas, const int64_t* num_tokens,
                                        const daric_rope* rope, uint64_t stream) {
    return scatter_rerotate(c, names, n_jobs, offsets, n_offsets, byte_sizes, n_byte_sizes, indices,
                            indices_offsets, n_indices_offsets, deltas, num_tokens, rope, stream, false);
}

int daric_copier_scatter_pages_rerotate_noalloc(daric_copier* c, const char* const* names, int64_t n_jobs,
                                                const int64_t* offsets, int64_t n_offsets,
                                                const int64_t* byte_sizes, int64_t n_byte_sizes,
                                                const daric_tensor* indices,
                                                const int64_t* indices_offsets, int64_t n_indices_offsets,
                                                const int64_t* deltas, const int64_t* num_tokens,
                                                const daric_rope* rope, uint64_t stream) {
    return scatter_rerotate(c, names, n_jobs, offsets, n_offsets, byte_sizes, n_byte_sizes, indices,
                            indices_offsets, n_indices_offsets, deltas, num_tokens, rope, stream, true);
}

// ------------------------------------------------------------ batched memcpy
static int batched_memcpy(const daric_tensor* dev_t, const daric_tensor* host_t,
                          const int64_t* dev_offsets, const int64_t* host_offsets,
                          const int64_t* sizes, int64_t n, uint64_t stream, bool d2h) {
    return guarded([&] {
        if (n == 0) return;
        DARIC_CHECK(n > 0 && dev_offsets && host_offsets && sizes, "offset/size arrays must not be null");
        check_tensor_struct(dev_t, "staging");
        check_tensor_struct(host_t, "shm");
        DARIC_CHECK(dev_t->device >= 0, "staging must be a device tensor");
        DARIC_CHECK(host_t->device < 0, "shm must be a host tensor");
        const int64_t dev_bytes = numel(*dev_t) * dev_t->elem_size;
        const int64_t host_bytes = numel(*host_t) * host_t->elem_size;
        for (int64_t i = 0; i < n; ++i) {
            DARIC_CHECK(dev_offsets[i] >= 0 && host_offsets[i] >= 0 && sizes[i] >= 0,
                        "negative offset or size at region ", i);
            DARIC_CHECK(dev_offsets[i] <= dev_bytes && sizes[i] <= dev_bytes - dev_offsets[i],
                        "staging range out of bounds at region ", i);
            DARIC_CHECK(host_offsets[i] <= host_bytes && sizes[i] <= host_bytes - host_offsets[i],
                        "shm range out of bounds at region ", i);
        }
        DeviceGuard guard(dev_t->device);
        const hipStream_t st = as_stream(stream);
        uint8_t* dv = static_cast<uint8_t*>(dev_t->data);
        uint8_t* hv = static_cast<uint8_t*>(host_t->data);
        for (int64_t i = 0; i < n; ++i) {
            if (sizes[i] == 0) continue;
            if (d2h)
                DARIC_HIP_CHECK(hipMemcpyAsync(hv + host_offsets[i], dv + dev_offsets[i],
                                               static_cast<size_t>(sizes[i]), hipMemcpyDeviceToHost, st));
            else
                DARIC_HIP_CHECK(hipMemcpyAsync(dv + dev_offsets[i], hv + host_offsets[i],
                                               static_cast<size_t>(sizes[i]), hipMemcpyHostToDevice, st));
        }
    });
}

int daric_batched_memcpy_d2h(const daric_tensor* staging, const daric_tensor* shm,
                             const int64_t* stg_offsets, const int64_t* shm_offsets,
                             const int64_t* sizes, int64_t n, uint64_t stream) {
    return batched_memcpy(staging, shm, stg_offsets, shm_offsets, sizes, n, stream, true);
}

int daric_batched_memcpy_h2d(const daric_tensor* shm, const daric_tensor* staging,
                             const int64_t* shm_offsets, const int64_t* stg_offsets,
                             const int64_t* sizes, int64_t n, uint64_t stream) {
    return batched_memcpy(staging, shm, stg_offsets, shm_offsets, sizes, n, stream, false);
}

}  // extern "C"

// ====================================================== in-place re-rotation
extern "C" int daric_rerotate_pages(const daric_tensor* layers, int64_t n_layers, int page_first,
                                    const daric_tensor* block_table,
                                    const daric_rope_segment* segments, int64_t n_segments,
                                    const daric_rope* rope, const daric_tensor* k_scales,
                                    uint64_t stream) {
    return guarded([&] {
        if (n_layers == 0 || n_segments == 0) return;
        const InplacePlan p = plan_inplace(layers, n_layers, page_first, block_table, segments, n_segments, rope,
                                           k_scales, 0);
        if (p.n_segs == 0) return;
        DeviceGuard guard(p.device);
        launch_inplace(p, as_stream(stream));
    });
}

// ====================================================== recompute selection
namespace {

KVGeom kv_geom(const daric_tensor& t, bool page_first) {
    const RopeLayout L = rope_layout(t, page_first, 2);
    KVGeom g{};
    g.sb = L.sb; g.ss = L.ss; g.sh = L.sh;
    g.PS = static_cast<int32_t>(L.PS);
    g.H = static_cast<int32_t>(L.H);
    g.D = static_cast<int32_t>(L.D);
    g.num_blocks = static_cast<int32_t>(L.num_blocks);
    if (t.ndim == 5) g.v_off = page_first ? t.strides[1] : t.strides[0];
    else if (t.ndim == 4) g.v_off = L.D;
    else g.v_off = -1;
    return g;
}

struct Chunks {
    std::vector<SelChunk> v;
    int64_t tiles = 0;
    int64_t max_tokens = 0;
    int64_t max_k = 0;
};

Chunks build_chunks(const daric_chunk* chunks, int64_t n, int64_t PS, int64_t bt_n, int64_t T,
                    int tile_tokens) {
    DARIC_CHECK(n > 0 && chunks != nullptr, "chunks must not be empty");
    Chunks c;
    c.v.reserve(n);
    for (int64_t i = 0; i < n; ++i) {
        const daric_chunk& s = chunks[i];
        DARIC_CHECK(s.n_tokens >= 0 && s.row_offset >= 0 && s.bt_offset >= 0 && s.k >= 0 &&
                    s.tok_start >= 0, "negative chunk field at chunk ", i);
        DARIC_CHECK(s.n_tokens <= kIntMax && s.k <= kIntMax, "chunk too long at chunk ", i);
        DARIC_CHECK(s.tok_start <= kIntMax && s.bt_offset <= kInt64Max - kIntMax, "chunk ", i,
                    " starts too far into its block list");
        DARIC_CHECK(s.row_offset + s.n_tokens <= T, "chunk ", i, " rows exceed the recomputed tensor");
        // the chunk's first page, and its first token's place in that page
        const int64_t bt_first = s.bt_offset + s.tok_start / PS;
        if (s.n_tokens > 0)
            DARIC_CHECK(bt_first + (s.tok_start % PS + s.n_tokens - 1) / PS < bt_n, "chunk ", i,
                        " reads past the end of block_table");
        SelChunk sc{};
        sc.bt_offset = bt_first;
        sc.tok0 = static_cast<int32_t>(s.tok_start % PS);
        sc.row_offset = s.row_offset;
        sc.n_tokens = static_cast<int32_t>(s.n_tokens);
        sc.k = static_cast<int32_t>(s.k);
        sc.tile_begin = static_cast<int32_t>(c.tiles);
        c.tiles += (s.n_tokens + tile_tokens - 1) / tile_tokens;
        c.max_tokens = std::max(c.max_tokens, s.n_tokens);
        c.max_k = std::max(c.max_k, std::min(s.k, s.n_tokens));
        c.v.push_back(sc);
    }
    return c;
}

void check_rows_tensor(const daric_tensor* x, const daric_tensor& layer, int64_t n_layers,
                       int64_t H, int64_t D, const char* what, int64_t* T) {
    check_tensor_struct(x, what);
    DARIC_CHECK(x->device == layer.device, what, " must be on the layers' device");
    DARIC_CHECK(x->ndim == 4 && x->sizes[0] == n_layers && x->sizes[2] == H && x->sizes[3] == D &&
                is_contiguous(*x), what, " must be a contiguous [n_layers, T, H, D] tensor");
    DARIC_CHECK(aligned(x->data, 16), what, " must be 16-byte aligned");
    *T = x->sizes[1];
}

}  // namespace

extern "C" {

int daric_kv_deviation(const daric_tensor* layers, int64_t n_layers, int page_first,
                       const daric_tensor* block_table, const daric_tensor* k_new,
                       const daric_chunk* chunks, int64_t n_chunks, const daric_tensor* k_scales,
                       daric_tensor* keys, uint64_t stream) {
    return guarded([&] {
        DARIC_CHECK(n_layers > 0 && layers != nullptr, "layers must not be empty");
        for (int64_t i = 0; i < n_layers; ++i) check_tensor_struct(&layers[i], "kv layer");
        check_same_layers(layers, n_layers);
        const daric_tensor& t = layers[0];
        DARIC_CHECK(t.device >= 0, "KV cache tensor must be on CUDA");
        const int ck = elem_kind(t);
        DARIC_CHECK(ck >= 0, "unsupported KV cache dtype for kv_deviation");
        const KVGeom g = kv_geom(t, page_first != 0);
        check_block_table(block_table, t.device);
        int64_t T = 0;
        check_rows_tensor(k_new, t, n_layers, g.H, g.D, "k_new", &T);
        const int nk = k_new->dtype == DARIC_DTYPE_BFLOAT16 ? kBF16 : (k_new->dtype == DARIC_DTYPE_FLOAT16 ? kF16 : -1);
        DARIC_CHECK(nk >= 0, "k_new must be bfloat16 or float16");
        check_tensor_struct(keys, "keys");
        DARIC_CHECK(keys->device == t.device && keys->dtype == DARIC_DTYPE_FLOAT32 && keys->ndim == 2 &&
                    keys->sizes[0] == n_layers && keys->sizes[1] == T && is_contiguous(*keys),
                    "keys must be a contiguous float32 [n_layers, T] tensor");
        const bool has_scales = k_scales != nullptr && k_scales->data != nullptr;
        if (has_scales) {
            DARIC_CHECK(ck == kE4M3, "k_scales apply to fp8 (e4m3) caches only");
            DARIC_CHECK(k_scales->device == t.device && k_scales->dtype == DARIC_DTYPE_FLOAT32 &&
                        is_contiguous(*k_scales) && numel(*k_scales) == n_layers * g.H,
                        "k_scales must be a contiguous float32 [n_layers, H] tensor on the layers' device");
        }
        const int64_t ces = t.elem_size;
        const int64_t need = ck == kE4M3 ? 8 : 16;
        DARIC_CHECK(g.D % 8 == 0 && (g.sb * ces) % need == 0 && (g.ss * ces) % need == 0 &&
                    (g.sh * ces) % need == 0 && aligned(t.data, need),
                    "kv_deviation needs head_dim % 8 == 0 and aligned K rows");
        for (int64_t i = 1; i < n_layers; ++i) DARIC_CHECK(aligned(layers[i].data, need), "misaligned layer ", i);
        Chunks c = build_chunks(chunks, n_chunks, g.PS, numel(*block_table), T, deviation_tile_tokens(ck));
        if (c.tiles == 0) return;
        DARIC_CHECK(c.tiles <= kMaxTiles, "too many tokens in one kv_deviation call");
        DeviceGuard guard(t.device);
        const hipStream_t st = as_stream(stream);
        const size_t cb = c.v.size() * sizeof(SelChunk);
        std::vector<uint8_t> blob(cb + n_layers * sizeof(uint8_t*));
        std::memcpy(blob.data(), c.v.data(), cb);
        const auto ptrs = layer_ptrs(layers, n_layers);
        std::memcpy(blob.data() + cb, ptrs.data(), n_layers * sizeof(uint8_t*));
        DescHandOver ho(t.device, blob.data(), blob.size(), st);
        launch_deviation(ho.arg(), static_cast<int>(cb), static_cast<int>(n_layers), g, ck,
                         static_cast<const int32_t*>(block_table->data),
                         static_cast<const uint8_t*>(k_new->data), nk, T, static_cast<int>(c.v.size()),
                         static_cast<int>(c.tiles),
                         has_scales ? static_cast<const float*>(k_scales->data) : nullptr,
                         static_cast<float*>(keys->data), st);
    });
}

int daric_topk_per_chunk(const daric_tensor* keys, const daric_chunk* chunks, int64_t n_chunks,
                         daric_tensor* out_idx, uint64_t stream) {
    return guarded([&] {
        check_tensor_struct(keys, "keys");
        DARIC_CHECK(keys->device >= 0 && keys->dtype == DARIC_DTYPE_FLOAT32 && keys->ndim == 2 &&
                    is_contiguous(*keys), "keys must be a contiguous float32 [n_layers, T] device tensor");
        const int64_t L = keys->sizes[0], T = keys->sizes[1];
        check_tensor_struct(out_idx, "out_idx");
        DARIC_CHECK(out_idx->device == keys->device && out_idx->dtype == DARIC_DTYPE_INT32 &&
                    out_idx->ndim == 3 && out_idx->sizes[0] == L && out_idx->sizes[1] == n_chunks &&
                    is_contiguous(*out_idx), "out_idx must be a contiguous int32 [n_layers, n_chunks, kmax] tensor");
        const int64_t kmax = out_idx->sizes[2];
        Chunks c = build_chunks(chunks, n_chunks, 1, kInt64Max, T, 1);
        DARIC_CHECK(c.max_k <= kmax, "out_idx kmax (", kmax, ") is smaller than a chunk's k (", c.max_k, ")");
        DARIC_CHECK(n_chunks <= kMaxTiles, "too many chunks in one topk_per_chunk call: ", n_chunks);
        if (L == 0 || kmax == 0) return;
        DeviceGuard guard(keys->device);
        const hipStream_t st = as_stream(stream);
        DescHandOver ho(keys->device, c.v.data(), c.v.size() * sizeof(SelChunk), st);
        launch_topk(static_cast<const float*>(keys->data), static_cast<int>(L), T, ho.arg(),
                    static_cast<int>(n_chunks),
                    static_cast<int>(std::max<int64_t>(c.max_tokens, 1)),
                    static_cast<int32_t*>(out_idx->data), static_cast<int>(kmax), st);
    });
}

int daric_merge_rows(const daric_tensor* layers, int64_t n_layers, int page_first,
                     const daric_tensor* block_table, const daric_tensor* k_new,
                     const daric_tensor* v_new, const daric_chunk* chunks, int64_t n_chunks,
                     const daric_tensor* sel_idx, const daric_tensor* k_scales,
                     const daric_tensor* v_scales, uint64_t stream) {
    return guarded([&] {
        DARIC_CHECK(n_layers > 0 && layers != nullptr, "layers must not be empty");
        for (int64_t i = 0; i < n_layers; ++i) check_tensor_struct(&layers[i], "kv layer");
        check_same_layers(layers, n_layers);
        const daric_tensor& t = layers[0];
        DARIC_CHECK(t.device >= 0, "KV cache tensor must be on CUDA");
        const KVGeom g = kv_geom(t, page_first != 0);
        check_block_table(block_table, t.device);
        int64_t T = 0, Tv = 0;
        check_rows_tensor(k_new, t, n_layers, g.H, g.D, "k_new", &T);
        // Rows in the cache's element type are copied as bytes; bf16 / fp16
        // rows for an fp8 (e4m3) cache are quantised with per-(layer, head)
        // scales, as vLLM's fp8 cache write quantises them.
        const int ck = elem_kind(t);
        const int nk = elem_kind(*k_new);
        const bool same_type = k_new->elem_size == t.elem_size &&
                               (k_new->dtype == t.dtype || (ck == kE4M3 && nk == kE4M3));
        const bool quant = ck == kE4M3 && (nk == kBF16 || nk == kF16);
        DARIC_CHECK(same_type || quant,
                    "k_new must have the cache's element type, or be bfloat16/float16 rows for an fp8 "
                    "(e4m3) cache");
        if (g.v_off >= 0) {
            check_rows_tensor(v_new, t, n_layers, g.H, g.D, "v_new", &Tv);
            DARIC_CHECK(Tv == T && v_new->dtype == k_new->dtype && v_new->elem_size == k_new->elem_size,
                        "v_new must match k_new");
        }
        const auto check_scales = [&](const daric_tensor* sc, const char* what) {
            DARIC_CHECK(sc != nullptr && sc->data != nullptr, "merging ", quant_name(nk),
                        " rows into an fp8 cache needs ", what);
            check_tensor_struct(sc, what);
            DARIC_CHECK(sc->device == t.device && sc->dtype == DARIC_DTYPE_FLOAT32 && is_contiguous(*sc) &&
                        numel(*sc) == n_layers * g.H,
                        what, " must be a contiguous float32 [n_layers, H] tensor on the layers' device");
        };
        if (quant) {
            check_scales(k_scales, "k_scales");
            if (g.v_off >= 0) check_scales(v_scales, "v_scales");
            DARIC_CHECK(merge_fits_rows(g, t.elem_size, true),
                        "quantising merge_rows needs head_dim % 8 == 0, 8-byte aligned cache rows and K+V "
                        "rows of at most ", merge_max_row_bytes() / 1024, " KiB of recomputed values per token");
            for (int64_t i = 0; i < n_layers; ++i)
                DARIC_CHECK(aligned(layers[i].data, 8), "misaligned layer ", i);
        } else {
            DARIC_CHECK((k_scales == nullptr || k_scales->data == nullptr) &&
                        (v_scales == nullptr || v_scales->data == nullptr),
                        "k_scales / v_scales apply only when bf16/fp16 rows are merged into an fp8 cache");
        }
        check_tensor_struct(sel_idx, "sel_idx");
        DARIC_CHECK(sel_idx->device == t.device && sel_idx->dtype == DARIC_DTYPE_INT32 &&
                    sel_idx->ndim == 3 && sel_idx->sizes[0] == n_layers &&
                    sel_idx->sizes[1] == n_chunks && is_contiguous(*sel_idx),
                    "sel_idx must be a contiguous int32 [n_layers, n_chunks, kmax] tensor");
        const int64_t kmax = sel_idx->sizes[2];
        Chunks c = build_chunks(chunks, n_chunks, g.PS, numel(*block_table), T, 1);
        // Nothing is selected (no rows, no chunk with k > 0 and tokens, or no
        // index slots): no launch, so empty k_new / v_new (whose data pointer
        // may be null) are never read.
        if (kmax == 0 || T == 0 || c.max_k == 0) return;
        DeviceGuard guard(t.device);
        const hipStream_t st = as_stream(stream);
        const size_t cb = c.v.size() * sizeof(SelChunk);
        std::vector<uint8_t> blob(cb + n_layers * sizeof(uint8_t*));
        std::memcpy(blob.data(), c.v.data(), cb);
        const auto ptrs = layer_ptrs(layers, n_layers);
        std::memcpy(blob.data() + cb, ptrs.data(), n_layers * sizeof(uint8_t*));
        DescHandOver ho(t.device, blob.data(), blob.size(), st);
        launch_merge(ho.arg(), static_cast<int>(cb), static_cast<int>(n_layers), g, t.elem_size,
                     static_cast<const int32_t*>(block_table->data),
                     static_cast<const uint8_t*>(k_new->data),
                     g.v_off >= 0 ? static_cast<const uint8_t*>(v_new->data) : nullptr, T,
                     static_cast<int>(n_chunks), static_cast<const int32_t*>(sel_idx->data),
                     static_cast<int>(kmax), quant ? nk : -1,
                     quant ? static_cast<const float*>(k_scales->data) : nullptr,
                     quant && g.v_off >= 0 ? static_cast<const float*>(v_scales->data) : nullptr, st);
    });
}

int daric_select_merge(const daric_tensor* layers, int64_t n_layers, int page_first,
                       const daric_tensor* block_table, const daric_tensor* k_new, const daric_tensor* v_new,
                       const daric_chunk* chunks, int64_t n_chunks, const daric_tensor* k_scales,
                       const daric_tensor* v_scales, daric_tensor* keys, daric_tensor* sel_idx,
                       int flags, uint64_t stream) {
    return guarded([&] {
        DARIC_CHECK(n_layers > 0 && layers != nullptr, "layers must not be empty");
        for (int64_t i = 0; i < n_layers; ++i) check_tensor_struct(&layers[i], "kv layer");
        check_same_layers(layers, n_layers);
        const daric_tensor& t = layers[0];
        DARIC_CHECK(t.device >= 0, "KV cache tensor must be on CUDA");
        const int ck = elem_kind(t);
        DARIC_CHECK(ck >= 0, "unsupported KV cache dtype for select_merge");
        const KVGeom g = kv_geom(t, page_first != 0);
        check_block_table(block_table, t.device);
        int64_t T = 0, Tv = 0;
        check_rows_tensor(k_new, t, n_layers, g.H, g.D, "k_new", &T);
        const int nk = k_new->dtype == DARIC_DTYPE_BFLOAT16 ? kBF16 : (k_new->dtype == DARIC_DTYPE_FLOAT16 ? kF16 : -1);
        DARIC_CHECK(nk >= 0, "k_new must be bfloat16 or float16");
        DARIC_CHECK((flags & ~(DARIC_SELECT_KEYS_READY | DARIC_SELECT_ONE_PASS)) == 0, "unknown select_merge flags ",
                    flags);
        const bool keys_ready = (flags & DARIC_SELECT_KEYS_READY) != 0;
        const bool one_pass = !keys_ready && (flags & DARIC_SELECT_ONE_PASS) != 0;
        const bool quant = ck == kE4M3;
        DARIC_CHECK(quant || k_new->dtype == t.dtype,
                    "k_new must have the cache's element type, or be bfloat16/float16 rows for an fp8 "
                    "(e4m3) cache");
        if (g.v_off >= 0) {
            check_rows_tensor(v_new, t, n_layers, g.H, g.D, "v_new", &Tv);
            DARIC_CHECK(Tv == T && v_new->dtype == k_new->dtype && v_new->elem_size == k_new->elem_size,
                        "v_new must match k_new");
        }
        const auto check_scales = [&](const daric_tensor* sc, const char* what) {
            DARIC_CHECK(sc != nullptr && sc->data != nullptr, "selecting and merging ", quant_name(nk),
                        " rows on an fp8 cache needs ", what);
            check_tensor_struct(sc, what);
            DARIC_CHECK(sc->device == t.device && sc->dtype == DARIC_DTYPE_FLOAT32 && is_contiguous(*sc) &&
                        numel(*sc) == n_layers * g.H,
                        what, " must be a contiguous float32 [n_layers, H] tensor on the layers' device");
        };
        if (quant) {
            check_scales(k_scales, "k_scales");
            if (g.v_off >= 0) check_scales(v_scales, "v_scales");
            DARIC_CHECK(merge_fits_rows(g, t.elem_size, true),
                        "quantising merge needs head_dim % 8 == 0, 8-byte aligned cache rows and K+V "
                        "rows of at most ", merge_max_row_bytes() / 1024, " KiB of recomputed values per token");
        } else {
            DARIC_CHECK((k_scales == nullptr || k_scales->data == nullptr) &&
                        (v_scales == nullptr || v_scales->data == nullptr),
                        "k_scales / v_scales apply only to an fp8 cache");
        }
        const int64_t ces = t.elem_size;
        const int64_t need = quant ? 8 : 16;
        DARIC_CHECK(g.D % 8 == 0 && (g.sb * ces) % need == 0 && (g.ss * ces) % need == 0 &&
                    (g.sh * ces) % need == 0 && (g.v_off < 0 || (g.v_off * ces) % need == 0),
                    "select_merge needs head_dim % 8 == 0 and aligned K/V rows");
        for (int64_t i = 0; i < n_layers; ++i) DARIC_CHECK(aligned(layers[i].data, need), "misaligned layer ", i);
        check_tensor_struct(keys, "keys");
        DARIC_CHECK(keys->device == t.device && keys->dtype == DARIC_DTYPE_FLOAT32 && keys->ndim == 2 &&
                    keys->sizes[0] == n_layers && keys->sizes[1] == T && is_contiguous(*keys),
                    "keys must be a contiguous float32 [n_layers, T] tensor");
        check_tensor_struct(sel_idx, "sel_idx");
        DARIC_CHECK(sel_idx->device == t.device && sel_idx->dtype == DARIC_DTYPE_INT32 &&
                    sel_idx->ndim == 3 && sel_idx->sizes[0] == n_layers &&
                    sel_idx->sizes[1] == n_chunks && is_contiguous(*sel_idx),
                    "sel_idx must be a contiguous int32 [n_layers, n_chunks, kmax] tensor");
        const int64_t kmax = sel_idx->sizes[2];
        Chunks c = build_chunks(chunks, n_chunks, g.PS, numel(*block_table), T, deviation_tile_tokens(ck));
        DARIC_CHECK(c.max_k <= kmax, "sel_idx kmax (", kmax, ") is smaller than a chunk's k (", c.max_k, ")");
        DARIC_CHECK(c.tiles <= kMaxTiles && n_chunks <= kMaxTiles, "too many tokens in one select_merge call");
        if (c.tiles == 0 && kmax == 0) return;   // no tokens to read, no index rows to fill
        DeviceGuard guard(t.device);
        const hipStream_t st = as_stream(stream);
        const size_t cb = c.v.size() * sizeof(SelChunk);
        std::vector<uint8_t> blob(cb + n_layers * sizeof(uint8_t*));
        std::memcpy(blob.data(), c.v.data(), cb);
        const auto ptrs = layer_ptrs(layers, n_layers);
        std::memcpy(blob.data() + cb, ptrs.data(), n_layers * sizeof(uint8_t*));
        DescHandOver ho(t.device, blob.data(), blob.size(), st);
        const float* ksc = quant ? static_cast<const float*>(k_scales->data) : nullptr;
        const float* vsc = quant && g.v_off >= 0 ? static_cast<const float*>(v_scales->data) : nullptr;
        float* kd = static_cast<float*>(keys->data);
        int32_t* sd = static_cast<int32_t*>(sel_idx->data);
        const auto* kn = static_cast<const uint8_t*>(k_new->data);
        const auto* vn = g.v_off >= 0 ? static_cast<const uint8_t*>(v_new->data) : nullptr;
        const auto* btp = static_cast<const int32_t*>(block_table->data);
        if (kmax > 0 && select_merge_fits(g, t.elem_size, quant, c.max_tokens, kmax, one_pass)) {
            // the keys by the deviation kernel (unless given, or one_pass), then
            // one workgroup per (layer, chunk) for its top-k and merge
            if (!keys_ready && !one_pass && c.tiles > 0)
                launch_deviation(ho.arg(), static_cast<int>(cb), static_cast<int>(n_layers), g, ck, btp, kn, nk, T,
                                 static_cast<int>(n_chunks), static_cast<int>(c.tiles), quant ? ksc : nullptr, kd,
                                 st);
            launch_select_merge(ho.arg(), static_cast<int>(cb), static_cast<int>(n_layers), g, ck, t.elem_size, btp,
                                kn, nk, vn, T, static_cast<int>(n_chunks), static_cast<int>(c.max_tokens), one_pass,
                                kd, sd, static_cast<int>(kmax), quant, ksc, vsc, st);
            return;
        }
        // the same work as three launches (chunks longer than the fused
        // kernel's LDS holds, or rows it does not take)
        if (!keys_ready && c.tiles > 0)
            launch_deviation(ho.arg(), static_cast<int>(cb), static_cast<int>(n_layers), g, ck, btp, kn, nk, T,
                             static_cast<int>(n_chunks), static_cast<int>(c.tiles), quant ? ksc : nullptr, kd, st);
        if (kmax == 0) return;
        launch_topk(kd, static_cast<int>(n_layers), T, ho.arg(), static_cast<int>(n_chunks),
                    static_cast<int>(std::max<int64_t>(c.max_tokens, 1)), sd, static_cast<int>(kmax), st);
        if (c.max_k == 0) return;
        launch_merge(ho.arg(), static_cast<int>(cb), static_cast<int>(n_layers), g, t.elem_size, btp, kn, vn, T,
                     static_cast<int>(n_chunks), sd, static_cast<int>(kmax), quant ? nk : -1, ksc, vsc, st);
    });
}

}  // extern "C"
