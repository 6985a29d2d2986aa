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
    ProfileEvents ev;
};

std::atomic<int> g_enabled{0};
std::mutex g_mu;
std::vector<Record> g_records;
std::vector<ProfileEvents> g_free;  // created event pairs not in use

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

ProfileEvents profile_begin(const char* label) {
    if (!g_enabled.load(std::memory_order_relaxed)) return ProfileEvents{};
    Record r;
    r.label = label;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_free.empty()) {
        r.ev = g_free.back();
        g_free.pop_back();
    } else {
        if (hipEventCreate(&r.ev.start) != hipSuccess) return ProfileEvents{};
        if (hipEventCreate(&r.ev.stop) != hipSuccess) {
            (void)hipEventDestroy(r.ev.start);
            return ProfileEvents{};
        }
    }
    g_records.push_back(r);
    return r.ev;
}

// Pre-creates event pairs so that a timed region's launches find them in the pool.
void profile_reserve(int pairs) {
    std::lock_guard<std::mutex> lock(g_mu);
    while (static_cast<int>(g_free.size()) < pairs) {
        ProfileEvents ev;
        if (hipEventCreate(&ev.start) != hipSuccess) return;
        if (hipEventCreate(&ev.stop) != hipSuccess) {
            (void)hipEventDestroy(ev.start);
            return;
        }
        g_free.push_back(ev);
    }
}

}  // namespace detail
}  // namespace cuflash

extern "C" {

void cuflash_profile_enable(int enabled) {
    if (enabled) cuflash::detail::profile_reserve(256);
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
        if (hipEventSynchronize(r.ev.stop) == hipSuccess &&
            hipEventElapsedTime(&ms, r.ev.start, r.ev.stop) == hipSuccess) {
            auto& a = agg[r.label];
            a.first += 1;
            a.second += ms;
        }
    }
    {
        std::lock_guard<std::mutex> lock(g_mu);
        for (Record& r : recs) g_free.push_back(r.ev);
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
