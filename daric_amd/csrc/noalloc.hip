// Descriptor staging that allocates nothing: a file-scope device array per
// GPU holds the descriptors of daric_copier_scatter_pages_rerotate_noalloc,
// and small kernels carry the descriptor bytes into it by value in their
// kernel arguments. No hipMalloc, hipHostMalloc or copy-engine transfer is
// involved, so callers that may not allocate (stream capture, serving loops
// with a fixed memory budget) can use it. Every call on one GPU shares that
// GPU's array. Eager calls are ordered on it: a call's stash kernels wait
// (hipStreamWaitEvent) for an event recorded after the previous call's last
// kernel when the two calls use different streams, and calls of different
// host threads enqueue one at a time. Calls recorded into a graph take no
// part in that ordering: replays of such a graph that overlap another call
// on the same GPU race on the array.
#include <hip/hip_runtime.h>

#include <atomic>
#include <map>
#include <memory>
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

// Per-GPU state of the scratch array, set up once per device with that
// device current: the array's device address, and the event that completes
// with the last kernel of the last eager call that read the array.
struct ScratchState {
    uint8_t* ptr = nullptr;
    hipEvent_t done = nullptr;
    hipStream_t last = nullptr;   // stream `done` was recorded on
    bool recorded = false;
    std::mutex call_mu;           // held by one call from its first stash to its record
};

namespace {

std::atomic<int64_t> g_scratch_waits{0};

ScratchState& scratch_state(int device) {
    static std::mutex mu;
    static std::map<int, std::unique_ptr<ScratchState>> states;
    std::lock_guard<std::mutex> lk(mu);
    auto& s = states[device];
    if (s) return *s;
    std::unique_ptr<ScratchState> fresh(new ScratchState());
    DeviceGuard guard(device);   // the symbol's address, and the event, on `device`
    void* p = nullptr;
    DARIC_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    DARIC_CHECK(p != nullptr && reinterpret_cast<uintptr_t>(p) % 256 == 0,
                "scratch array has no usable device address on device ", device);
    fresh->ptr = static_cast<uint8_t*>(p);
    DARIC_HIP_CHECK(hipEventCreateWithFlags(&fresh->done, hipEventDisableTiming));
    s = std::move(fresh);
    return *s;
}

// Whether work enqueued on `stream` is being recorded into a graph (an
// unanswerable query counts as capturing: no event work is added then).
bool capturing(hipStream_t stream) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess) {
        (void)hipGetLastError();
        return true;
    }
    return cs != hipStreamCaptureStatusNone;
}

}  // namespace

uint8_t* noalloc_scratch(int device) { return scratch_state(device).ptr; }

ScratchUse::ScratchUse(int device, hipStream_t stream)
    : state_(&scratch_state(device)), stream_(stream), lock_(state_->call_mu) {
    capture_ = capturing(stream);
    if (!capture_ && state_->recorded && state_->last != stream) {
        DARIC_HIP_CHECK(hipStreamWaitEvent(stream, state_->done, 0));
        g_scratch_waits.fetch_add(1, std::memory_order_relaxed);
    }
}

uint8_t* ScratchUse::ptr() const { return state_->ptr; }

void ScratchUse::finish() {
    finished_ = true;
    if (capture_) return;
    DARIC_HIP_CHECK(hipEventRecord(state_->done, stream_));
    state_->last = stream_;
    state_->recorded = true;
}

ScratchUse::~ScratchUse() {
    if (finished_ || capture_) return;
    if (hipEventRecord(state_->done, stream_) == hipSuccess) {
        state_->last = stream_;
        state_->recorded = true;
    } else {
        (void)hipGetLastError();
    }
}

int64_t scratch_stream_waits() { return g_scratch_waits.load(std::memory_order_relaxed); }

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
