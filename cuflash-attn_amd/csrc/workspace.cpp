// Library-owned stream-ordered memory pools for the launchers' workspaces (one per device).
//
// hipMallocAsync from a pool whose release threshold is 0 (the default) hands freed memory back
// at every synchronization, so each call's workspace needs fresh driver work. A private pool per
// device whose release threshold is kKeepBytes keeps the few MiB the launchers usually use (the
// backward's row statistics, the decode partials) cached, gives larger workspaces (grouped-query
// dK/dV shares) back at synchronization, and leaves the application's pools alone.

#include <cstdint>
#include <mutex>

#include "launch.hpp"

namespace cuflash {
namespace detail {

namespace {
constexpr int kMaxDevices = 64;
constexpr uint64_t kKeepBytes = 256ull << 20;  // pool memory kept across synchronizations
std::mutex g_pool_mutex;
hipMemPool_t g_pools[kMaxDevices] = {};
bool g_tried[kMaxDevices] = {};
}  // namespace

hipMemPool_t workspace_pool() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_pool_mutex);
    if (!g_tried[dev]) {
        g_tried[dev] = true;
        hipMemPoolProps props = {};
        props.allocType = hipMemAllocationTypePinned;
        props.handleTypes = hipMemHandleTypeNone;
        props.location.type = hipMemLocationTypeDevice;
        props.location.id = dev;
        hipMemPool_t pool = nullptr;
        if (hipMemPoolCreate(&pool, &props) == hipSuccess) {
            uint64_t keep = kKeepBytes;
            if (hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep) == hipSuccess) {
                g_pools[dev] = pool;
            } else {
                (void)hipGetLastError();  // clear only the error of this call
                (void)hipMemPoolDestroy(pool);
            }
        } else {
            (void)hipGetLastError();
        }
    }
    return g_pools[dev];
}

int compute_units() {
    static int cached[kMaxDevices] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return 256;
    }
    std::lock_guard<std::mutex> lock(g_pool_mutex);
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0) {
            (void)hipGetLastError();
            n = 256;
        }
        cached[dev] = n;
    }
    return cached[dev];
}

}  // namespace detail
}  // namespace cuflash
