// Host runtime support: error state, tensor helpers, descriptor ring, timing.
#include <atomic>
#include <map>
#include <memory>

#include "common.h"
#include "kernels.h"
#include "launch.h"

namespace daric {

namespace {
thread_local std::string g_last_error;
std::atomic<bool> g_timing{false};
std::mutex g_timing_mu;
struct TimedLaunch {
    hipEvent_t start, stop;
};
std::vector<TimedLaunch> g_timed;
}  // namespace

void set_last_error(const std::string& msg) { g_last_error = msg; }
const char* last_error() { return g_last_error.c_str(); }

std::string fmt_dims(const int64_t* v, int n) {
    std::ostringstream ss;
    ss << "[";
    for (int i = 0; i < n; ++i) ss << (i ? ", " : "") << v[i];
    ss << "]";
    return ss.str();
}

bool is_contiguous(const daric_tensor& t) {
    // as torch: a tensor without elements is contiguous whatever its strides
    for (int d = 0; d < t.ndim; ++d)
        if (t.sizes[d] == 0) return true;
    int64_t expected = 1;
    for (int d = t.ndim - 1; d >= 0; --d) {
        if (t.sizes[d] == 1) continue;
        if (t.strides[d] != expected) return false;
        expected *= t.sizes[d];
    }
    return true;
}

int64_t numel(const daric_tensor& t) {
    int64_t n = 1;
    for (int d = 0; d < t.ndim; ++d) n *= t.sizes[d];
    return n;
}

void check_tensor_struct(const daric_tensor* t, const char* what) {
    DARIC_CHECK(t != nullptr, what, " must not be null");
    DARIC_CHECK(t->ndim >= 0 && t->ndim <= DARIC_MAX_DIMS, what, " has an invalid rank: ", t->ndim);
    DARIC_CHECK(t->elem_size > 0, what, " has an invalid element size");
}

void check_launch(const char* what) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        throw Error(DARIC_ERR_HIP, cat("HIP error launching ", what, " - ", hipGetErrorString(err),
                                       " (error code ", static_cast<int>(err), ")"));
}

DeviceGuard::DeviceGuard(int device) {
    DARIC_HIP_CHECK(hipGetDevice(&prev_));
    if (prev_ != device) DARIC_HIP_CHECK(hipSetDevice(device));
}
DeviceGuard::~DeviceGuard() {
    int cur = -1;
    if (hipGetDevice(&cur) == hipSuccess && cur != prev_ && prev_ >= 0) (void)hipSetDevice(prev_);
}

int device_cu_count(int device) {
    int n = 0;
    DARIC_HIP_CHECK(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device));
    return n;
}

// ---------------------------------------------------------------- DescRing
DescRing& DescRing::for_device(int device) {
    static std::mutex mu;
    static std::map<int, std::unique_ptr<DescRing>> rings;
    std::lock_guard<std::mutex> lk(mu);
    auto& r = rings[device];
    if (!r) r.reset(new DescRing());
    return *r;
}

namespace {
std::atomic<int64_t> g_ring_uploads{0};
std::atomic<int64_t> g_ring_allocations{0};
}  // namespace

void* DescRing::upload(const void* src, size_t bytes, hipStream_t stream, int* slot_out, bool direct) {
    g_ring_uploads.fetch_add(1, std::memory_order_relaxed);
    // A slot between upload() and release() belongs to a call that is still
    // enqueueing kernels on it; skip such slots (wait if all are taken). The
    // lock covers only the choice of the slot: waiting for its previous
    // kernels and filling it happen outside, so that other threads can take
    // slots meanwhile.
    int idx = -1;
    {
        std::unique_lock<std::mutex> lk(mu_);
        for (;;) {
            for (int k = 0; k < kSlots; ++k) {
                const int c = (next_ + k) % kSlots;
                if (!slots_[c].in_use) { idx = c; break; }
            }
            if (idx >= 0) break;
            lk.unlock();
            std::this_thread::yield();
            lk.lock();
        }
        // All slots get kInitialCap bytes at the ring's first use: growing a
        // slot later frees device memory (hipFree waits for the device), which
        // would stall a call in the middle of a pipelined stream of calls.
        // 1 MiB holds the descriptors of ~13000 copy jobs.
        if (!initialised_) {
            for (Slot& t : slots_) {
                if (t.ev == nullptr) DARIC_HIP_CHECK(hipEventCreateWithFlags(&t.ev, hipEventDisableTiming));
                if (t.cap == 0) {
                    g_ring_allocations.fetch_add(1, std::memory_order_relaxed);
                    DARIC_HIP_CHECK(hipHostMalloc(&t.host, kInitialCap, hipHostMallocCoherent));
                    DARIC_HIP_CHECK(hipMalloc(&t.dev, kInitialCap));
                    t.cap = kInitialCap;
                }
            }
            initialised_ = true;
        }
        next_ = (idx + 1) % kSlots;
        slots_[idx].in_use = true;
    }
    Slot& s = slots_[idx];
    *slot_out = idx;
    try {
        if (s.pending) {
            DARIC_HIP_CHECK(hipEventSynchronize(s.ev));
            s.pending = false;
        }
        if (bytes > s.cap) {
            size_t cap = s.cap * 2;
            while (cap < bytes) cap *= 2;
            if (s.host) DARIC_HIP_CHECK(hipHostFree(s.host));
            if (s.dev) DARIC_HIP_CHECK(hipFree(s.dev));
            s.host = nullptr;
            s.dev = nullptr;
            s.cap = 0;
            // Coherent (fine-grained) pinned memory: the upload kernel reads it
            // over the bus, so no stale GPU-cached copy of an earlier use of the
            // slot can be seen.
            g_ring_allocations.fetch_add(1, std::memory_order_relaxed);
            DARIC_HIP_CHECK(hipHostMalloc(&s.host, cap, hipHostMallocCoherent));
            DARIC_HIP_CHECK(hipMalloc(&s.dev, cap));
            s.cap = cap;
        }
        std::memcpy(s.host, src, bytes);
        // Direct: the kernels read the coherent pinned slot themselves; the
        // event recorded at release() keeps the slot until they are done.
        if (direct) return s.host;
        // Otherwise a kernel on `stream` copies the slot to the device.
        // Unlike hipMemcpyAsync (a copy-engine transfer the compute queue
        // must then wait for, ~17 us per call in a back-to-back pipeline on
        // MI355X) it stays on the compute queue (~3 us). Slots are 16-byte
        // multiples of at least 1 MiB, so the rounded copy stays in bounds.
        launch_upload(s.host, s.dev, (bytes + 15) / 16, stream);
    } catch (...) {
        std::lock_guard<std::mutex> lk(mu_);
        s.in_use = false;
        throw;
    }
    return s.dev;
}

void DescRing::release(int slot, hipStream_t stream, bool bound) {
    if (slot < 0) return;
    std::lock_guard<std::mutex> lk(mu_);
    Slot& s = slots_[slot];
    // The event marks the end of every kernel that reads the slot: the last
    // one carried it (kernels of one stream finish in order), or it is
    // recorded here; if it cannot be, wait for the stream so reuse stays safe.
    if (bound) s.pending = true;
    else if (hipEventRecord(s.ev, stream) == hipSuccess) s.pending = true;
    else (void)hipStreamSynchronize(stream);
    s.in_use = false;
}

namespace {
thread_local hipEvent_t t_completion = nullptr;
thread_local hipEvent_t t_completion_bound = nullptr;
}  // namespace

void set_completion_event(hipEvent_t ev) {
    t_completion = ev;
    t_completion_bound = nullptr;
}
hipEvent_t completion_event() { return t_completion; }
void note_completion_bound(hipEvent_t ev) { t_completion_bound = ev; }
hipEvent_t completion_bound() { return t_completion_bound; }

// ---------------------------------------------------------------- timing
void timing_events(hipEvent_t* start, hipEvent_t* stop) {
    *start = *stop = nullptr;
    if (!g_timing.load(std::memory_order_relaxed)) return;
    hipEvent_t a = nullptr, b = nullptr;
    if (hipEventCreate(&a) != hipSuccess) return;
    if (hipEventCreate(&b) != hipSuccess) {
        (void)hipEventDestroy(a);
        return;
    }
    *start = a;
    *stop = b;
}

void timing_record(hipEvent_t start, hipEvent_t stop) {
    if (start == nullptr || stop == nullptr) return;
    std::lock_guard<std::mutex> lk(g_timing_mu);
    g_timed.push_back({start, stop});
}

}  // namespace daric

using namespace daric;

extern "C" {

int daric_abi_version(void) { return DARIC_ABI_VERSION; }

const char* daric_last_error(void) { return daric::last_error(); }

int daric_timing_enable(int enable) {
    return guarded([&] { g_timing.store(enable != 0); });
}

int daric_debug_counters(int64_t* descriptor_uploads, int64_t* ring_allocations, int64_t* scratch_waits) {
    return guarded([&] {
        if (descriptor_uploads) *descriptor_uploads = g_ring_uploads.load(std::memory_order_relaxed);
        if (ring_allocations) *ring_allocations = g_ring_allocations.load(std::memory_order_relaxed);
        if (scratch_waits) *scratch_waits = scratch_stream_waits();
    });
}

int daric_timing_read(double* total_ms, int64_t* launches) {
    return guarded([&] {
        std::vector<TimedLaunch> v;
        {
            std::lock_guard<std::mutex> lk(g_timing_mu);
            v.swap(g_timed);
        }
        double sum = 0.0;
        for (auto& t : v) {
            DARIC_HIP_CHECK(hipEventSynchronize(t.stop));
            float ms = 0.0f;
            DARIC_HIP_CHECK(hipEventElapsedTime(&ms, t.start, t.stop));
            sum += ms;
            (void)hipEventDestroy(t.start);
            (void)hipEventDestroy(t.stop);
        }
        if (total_ms) *total_ms = sum;
        if (launches) *launches = static_cast<int64_t>(v.size());
    });
}

}  // extern "C"
