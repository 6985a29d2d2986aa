#pragma once

// Opt-in per-kernel timing with HIP events (measurement hook for benchmarks).
//
// When enabled through cuflash_profile_enable(1), every kernel launch of the library is
// bracketed by two hipEventRecord calls on the launch stream; cuflash_profile_report() waits
// for the recorded events and returns, per kernel label, the launch count and the summed
// event-to-event time. Disabled (the default), profile_begin() is a single relaxed atomic load.

#include <hip/hip_runtime.h>

#include <cstdio>

namespace cuflash {
namespace detail {

bool profiling_on();

// Returns a token for profile_end(), or -1 when profiling is off.
int profile_begin(const char* label, hipStream_t stream);
void profile_end(int token, hipStream_t stream);

template <typename T>
const char* dtype_tag();

// profile_begin with the label "<kernel>_<dtype>_d<head_dim>".
template <typename T, int D>
int profile_kernel(const char* kernel, hipStream_t stream) {
    if (!profiling_on()) return -1;
    char label[96];
    std::snprintf(label, sizeof(label), "%s_%s_d%d", kernel, dtype_tag<T>(), D);
    return profile_begin(label, stream);
}

}  // namespace detail
}  // namespace cuflash
