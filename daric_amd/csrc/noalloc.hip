// Descriptor staging that allocates nothing: a file-scope device array per
// GPU holds the descriptors of daric_copier_scatter_pages_rerotate_noalloc,
// and small kernels carry the descriptor bytes into it by value in their
// kernel arguments. No hipMalloc, hipHostMalloc or copy-engine transfer is
// involved, so callers that may not allocate (stream capture, serving loops
// with a fixed memory budget) can use it. Every call on one GPU shares that
// GPU's array: calls that overlap on one GPU (different streams, or graphs
// replayed concurrently) race on it.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>

#include "common.h"
#include "kernels.h"

namespace daric {

namespace {

// Each GPU holds its own copy of this array from the library's load until
// the process ends. Host code must not use the name as an address: the
// device address comes from hipGetSymbolAddress, per device.
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

using u32x4 = __attribute__((ext_vector_type(4))) uint32_t;

// Lane i writes 16-byte unit i of the blob (vector stores) to dst.
__global__ __launch_bounds__(256) void stash_kernel(DescArg blob, u32x4* __restrict__ dst, uint32_t n16) {
    const uint32_t i = threadIdx.x;
    if (i < n16) dst[i] = desc_load(desc_at<u32x4>(blob, static_cast<int>(i * 16)));
}

static_assert(kInlineDescBytes % 16 == 0 && kInlineDescBytes / 16 <= 256, "one stash workgroup per blob");

}  // namespace

uint8_t* noalloc_scratch(int device) {
    static std::mutex mu;
    static std::map<int, uint8_t*> ptrs;
    std::lock_guard<std::mutex> lk(mu);
    auto it = ptrs.find(device);
    if (it != ptrs.end()) return it->second;
    DeviceGuard guard(device);   // the symbol's address on `device`
    void* p = nullptr;
    DARIC_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    DARIC_CHECK(p != nullptr && reinterpret_cast<uintptr_t>(p) % 256 == 0,
                "scratch array has no usable device address on device ", device);
    ptrs[device] = static_cast<uint8_t*>(p);
    return static_cast<uint8_t*>(p);
}

void stash_descriptors(const void* src, size_t bytes, uint8_t* dst, hipStream_t stream) {
    for (size_t off = 0; off < bytes; off += kInlineDescBytes) {
        const size_t n = std::min<size_t>(kInlineDescBytes, bytes - off);
        DescArg blob;
        blob.ptr = nullptr;
        blob.reserved = 0;
        std::memset(blob.inl, 0, sizeof(blob.inl));
        std::memcpy(blob.inl, static_cast<const uint8_t*>(src) + off, n);
        const uint32_t n16 = static_cast<uint32_t>((n + 15) / 16);
        hipLaunchKernelGGL(stash_kernel, dim3(1), dim3(256), 0, stream, blob,
                           reinterpret_cast<u32x4*>(dst + off), n16);
        check_launch("descriptor stash");
    }
}

}  // namespace daric
