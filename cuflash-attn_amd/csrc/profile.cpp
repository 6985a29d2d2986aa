// Opt-in per-kernel HIP-event timing (see profile.hpp).

#include "profile.hpp"

#include <atomic>
#include <cstdio>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "cuflash/flash_attention.h"

namespace cuflash {
namespace detail {

namespace {

struct Record {
    std::string label;
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};

std::atomic<int> g_enabled{0};
std::mutex g_mu;
std::vector<Record> g_records;

}  // namespace

template <>
const char* dtype_tag<float>() {
    return "f32";
}
template <>
const char* dtype_tag<__half>() {
    return "f16";
}
template <>
const char* dtype_tag<__hip_bfloat16>() {
    return "bf16";
}

bool profiling_on() { return g_enabled.load(std::memory_order_relaxed) != 0; }

int profile_begin(const char* label, hipStream_t stream) {
    if (!g_enabled.load(std::memory_order_relaxed)) return -1;
    Record r;
    r.label = label;
    if (hipEventCreate(&r.start) != hipSuccess) return -1;
    if (hipEventCreate(&r.stop) != hipSuccess) {
        (void)hipEventDestroy(r.start);
        return -1;
    }
    (void)hipEventRecord(r.start, stream);
    std::lock_guard<std::mutex> lock(g_mu);
    g_records.push_back(r);
    return static_cast<int>(g_records.size()) - 1;
}

void profile_end(int token, hipStream_t stream) {
    if (token < 0) return;
    std::lock_guard<std::mutex> lock(g_mu);
    if (token < static_cast<int>(g_records.size()))
        (void)hipEventRecord(g_records[token].stop, stream);
}

}  // namespace detail
}  // namespace cuflash

extern "C" {

void cuflash_profile_enable(int enabled) {
    cuflash::detail::g_enabled.store(enabled ? 1 : 0, std::memory_order_relaxed);
}

int cuflash_profile_report(char* buf, int buflen) {
    using namespace cuflash::detail;
    std::vector<Record> recs;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        recs.swap(g_records);
    }
    std::map<std::string, std::pair<long, double>> agg;
    for (Record& r : recs) {
        float ms = 0.0f;
        if (hipEventSynchronize(r.stop) == hipSuccess &&
            hipEventElapsedTime(&ms, r.start, r.stop) == hipSuccess) {
            auto& a = agg[r.label];
            a.first += 1;
            a.second += ms;
        }
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    std::string out;
    char line[256];
    for (const auto& kv : agg) {
        std::snprintf(line, sizeof(line), "%s\t%ld\t%.6f\n", kv.first.c_str(), kv.second.first,
                      kv.second.second);
        out += line;
    }
    if (buf && buflen > 0) {
        const int n = static_cast<int>(out.size()) < buflen - 1 ? static_cast<int>(out.size())
                                                                 : buflen - 1;
        out.copy(buf, static_cast<size_t>(n));
        buf[n] = '\0';
    }
    return static_cast<int>(out.size()) + 1;
}

}  // extern "C"
