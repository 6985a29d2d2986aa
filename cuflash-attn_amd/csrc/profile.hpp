#pragma once

// Opt-in per-kernel timing with HIP events (measurement hook for benchmarks).
//
// When enabled through cuflash_profile_enable(1), every kernel launch of the library is made with
// hipExtLaunchKernelGGL and a start / stop event pair, which HIP fills with the dispatch's own
// begin and end timestamps (the interval a kernel trace reports, with no queue gap before the
// kernel counted). The pairs come from a pool created once, so the launch path creates nothing.
// cuflash_profile_report() waits for the recorded events and returns, per kernel label, the
// launch count and the summed kernel time. Disabled (the default), profile_kernel() is a single
// relaxed atomic load and launch_kernel() launches without events.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

namespace cuflash {
namespace detail {

bool profiling_on();

struct ProfileEvents {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};

// Records a launch under `label` and returns the event pair its launch_kernel() fills; both
// events are null when profiling is off (or no pair could be created).
ProfileEvents profile_begin(const char* label);

template <typename T>
const char* dtype_tag();

// profile_begin with the label "<kernel>_<dtype>_d<head_dim>".
template <typename T, int D>
ProfileEvents profile_kernel(const char* kernel) {
    if (!profiling_on()) return ProfileEvents{};
    char label[96];
    std::snprintf(label, sizeof(label), "%s_%s_d%d", kernel, dtype_tag<T>(), D);
    return profile_begin(label);
}

// Launches `kernel` on `stream`; with the event pair of a profiled launch, the events record
// the kernel's own start and end.
template <typename... Args, typename F>
void launch_kernel(const ProfileEvents& ev, F kernel, const dim3& grid, const dim3& block,
                   uint32_t lds_bytes, hipStream_t stream, Args... args) {
    hipExtLaunchKernelGGL(kernel, grid, block, lds_bytes, stream, ev.start, ev.stop, 0u, args...);
}

}  // namespace detail
}  // namespace cuflash
