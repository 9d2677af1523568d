// Host-side support shared by the C-ABI implementation: error state, HIP
// error checks, tensor helpers and the per-device descriptor ring.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstring>
#include <mutex>
#include <optional>
#include <sstream>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "../../include/daric_cache_ops.h"
#include "jobs.h"
#include "launch.h"

namespace daric {

// Errors raised by host code carry the status the C ABI returns.
struct Error : std::runtime_error {
    int status;
    Error(int st, const std::string& msg) : std::runtime_error(msg), status(st) {}
};

void set_last_error(const std::string& msg);
const char* last_error();

template <typename... Args>
std::string cat(Args&&... args) {
    std::ostringstream ss;
    (ss << ... << args);
    return ss.str();
}

// TORCH_CHECK counterpart: invalid argument.
#define DARIC_CHECK(cond, ...)                                                 \
    do {                                                                       \
        if (!(cond)) throw ::daric::Error(DARIC_ERR_INVALID, ::daric::cat(__VA_ARGS__)); \
    } while (0)

// Reference CUDA_CHECK message format (csrc/cache_ops/cache_ops.h:12-22).
#define DARIC_HIP_CHECK(call)                                                  \
    do {                                                                       \
        hipError_t err_ = (call);                                              \
        if (err_ != hipSuccess) {                                              \
            throw ::daric::Error(DARIC_ERR_HIP,                                \
                ::daric::cat("HIP error at ", __FILE__, ":", __LINE__, " - ",  \
                             hipGetErrorString(err_), " (error code ",         \
                             static_cast<int>(err_), ")"));                    \
        }                                                                      \
    } while (0)

// Runs `fn`, converting exceptions into a status code + thread-local message.
template <typename F>
int guarded(F&& fn) {
    try {
        fn();
        return DARIC_OK;
    } catch (const Error& e) {
        set_last_error(e.what());
        return e.status;
    } catch (const std::bad_alloc&) {
        set_last_error("host allocation failed");
        return DARIC_ERR_NOMEM;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return DARIC_ERR_RUNTIME;
    }
}

std::string fmt_dims(const int64_t* v, int n);
inline std::string sizes_str(const daric_tensor& t) { return fmt_dims(t.sizes, t.ndim); }
inline std::string strides_str(const daric_tensor& t) { return fmt_dims(t.strides, t.ndim); }

bool is_contiguous(const daric_tensor& t);
int64_t numel(const daric_tensor& t);
void check_tensor_struct(const daric_tensor* t, const char* what);

// Upload area for per-call job descriptors. Each device owns a ring of slots;
// a slot pairs a pinned host buffer with a device buffer and an event recorded
// after the launches that read it. A slot is reused only after its event has
// completed, so concurrent calls on different streams never share live
// descriptor memory.
class DescRing {
public:
    struct Slot {
        void* host = nullptr;
        void* dev = nullptr;
        size_t cap = 0;
        hipEvent_t ev = nullptr;
        bool pending = false;  // ev marks the last kernels that read the slot
        bool in_use = false;   // between upload() and release()
    };
    static DescRing& for_device(int device);
    // Copies `bytes` from `src` into a slot, enqueues the H2D copy on `stream`
    // and returns the device address. With `direct`, no copy is enqueued and
    // the slot's pinned host address is returned: the kernels then read the
    // descriptors over the host link. The caller must call release() with
    // the returned slot index after enqueueing every kernel that reads it.
    void* upload(const void* src, size_t bytes, hipStream_t stream, int* slot_out, bool direct = false);
    // The slot's reuse guard. If the caller's last kernel launch carried it
    // (`bound`), it completes with that kernel; else release() records it on
    // `stream`.
    hipEvent_t slot_event(int slot) const { return slots_[slot].ev; }
    void release(int slot, hipStream_t stream, bool bound = false);

private:
    DescRing() = default;
    static constexpr int kSlots = 16;
    static constexpr size_t kInitialCap = 1 << 20;
    bool initialised_ = false;
    int next_ = 0;
    Slot slots_[kSlots];
    std::mutex mu_;
};

// RAII helper: uploads a descriptor array (or, with `direct`, hands out its
// pinned host copy) and releases its slot at scope exit.
// While it lives, the slot's event is the calling thread's completion event
// (see DARIC_LAUNCH), so the call's kernels carry it.
void set_completion_event(hipEvent_t ev);
hipEvent_t completion_bound();

class DescUpload {
public:
    DescUpload(int device, const void* src, size_t bytes, hipStream_t stream, bool direct = false)
        : ring_(DescRing::for_device(device)), stream_(stream) {
        ptr_ = ring_.upload(src, bytes, stream, &slot_, direct);
        ev_ = ring_.slot_event(slot_);
        prev_ = completion_event();
        set_completion_event(ev_);
    }
    ~DescUpload() {
        // bound: the last launch since the constructor carried this slot's event
        const bool bound = completion_bound() == ev_;
        set_completion_event(prev_);
        ring_.release(slot_, stream_, bound);
    }
    void* get() const { return ptr_; }

private:
    DescRing& ring_;
    hipStream_t stream_;
    int slot_ = -1;
    void* ptr_ = nullptr;
    hipEvent_t ev_ = nullptr;
    hipEvent_t prev_ = nullptr;
};

// Hands a call's descriptor bytes to its kernels: inline in the kernel
// arguments when they fit (DescArg), else through the ring (an upload, or with
// `direct` the pinned slot itself), released at scope exit.
class DescHandOver {
public:
    DescHandOver(int device, const void* src, size_t bytes, hipStream_t stream, bool direct = false) {
        arg_.ptr = nullptr;
        arg_.reserved = 0;
        if (bytes <= static_cast<size_t>(kInlineDescBytes)) {
            if (bytes) std::memcpy(arg_.inl, src, bytes);
        } else {
            // The ring's slots are rewritten by later calls, so a graph node
            // pointing at one would replay stale descriptors: refuse capture.
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
                throw Error(DARIC_ERR_INVALID,
                            cat("this call's descriptors (", bytes, " bytes) exceed the ", kInlineDescBytes,
                                " bytes that travel in kernel arguments; it cannot be captured in a graph"));
            up_.emplace(device, src, bytes, stream, direct);
            arg_.ptr = static_cast<const uint8_t*>(up_->get());
        }
    }
    const DescArg& arg() const { return arg_; }

private:
    DescArg arg_;
    std::optional<DescUpload> up_;
};

// Sets the current device for the scope and restores the previous one.
class DeviceGuard {
public:
    explicit DeviceGuard(int device);
    ~DeviceGuard();

private:
    int prev_ = -1;
};

int device_cu_count(int device);

}  // namespace daric
