// Kernel launch wrapper shared by the .hip files. When kernel timing is
// enabled (daric_timing_enable) a launch goes through hipExtLaunchKernelGGL,
// so that the dispatch packet itself records start/stop timestamps: the
// measured interval is the kernel's execution, the same interval rocprofv3
// reports, without the gap an event recorded before and after the launch on
// the stream would add. Otherwise it is a plain launch, which is also what a
// stream capture records into a graph.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

namespace daric {

// Create a start/stop event pair when timing is enabled (else both null).
void timing_events(hipEvent_t* start, hipEvent_t* stop);
// Hand a pair filled by a launch to daric_timing_read (no-op for nulls).
void timing_record(hipEvent_t start, hipEvent_t stop);

// Completion event of the calling thread's current descriptor slot (null when
// the call's descriptors travel inline). A launch binds it to its own
// dispatch, so it completes with the kernel and no separate event packet
// follows the kernel on the stream (that packet cost ~5 us between
// back-to-back calls on MI355X). note_completion_bound() records which event
// the last launch carried.
hipEvent_t completion_event();
void note_completion_bound(hipEvent_t ev);

}  // namespace daric

#define DARIC_LAUNCH(kern, grid, block, shmem, stream, ...)                                   \
    do {                                                                                      \
        hipEvent_t daric_ev0_ = nullptr, daric_ev1_ = nullptr;                               \
        ::daric::timing_events(&daric_ev0_, &daric_ev1_);                                     \
        hipEvent_t daric_done_ = ::daric::completion_event();                                 \
        if (daric_ev0_ != nullptr) {                                                          \
            hipExtLaunchKernelGGL(kern, dim3(grid), dim3(block), static_cast<std::uint32_t>(shmem), \
                                  stream, daric_ev0_, daric_ev1_, 0, __VA_ARGS__);            \
            ::daric::timing_record(daric_ev0_, daric_ev1_);                                   \
        } else if (daric_done_ != nullptr) {                                                  \
            hipExtLaunchKernelGGL(kern, dim3(grid), dim3(block), static_cast<std::uint32_t>(shmem), \
                                  stream, nullptr, daric_done_, 0, __VA_ARGS__);              \
            ::daric::note_completion_bound(daric_done_);                                      \
        } else {                                                                              \
            /* plain launch: the form graph capture records */                               \
            hipLaunchKernelGGL(kern, dim3(grid), dim3(block), static_cast<std::uint32_t>(shmem), \
                               stream, __VA_ARGS__);                                          \
        }                                                                                     \
    } while (0)
