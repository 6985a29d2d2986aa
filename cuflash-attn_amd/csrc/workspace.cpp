// Library-owned stream-ordered memory pools for the launchers' workspaces (one per device).
//
// hipMallocAsync from a pool whose release threshold is 0 (the default) hands freed memory back
// at every synchronization, so each call's workspace needs fresh driver work. A private pool per
// device whose release threshold is kKeepBytes keeps the few MiB the launchers usually use (the
// backward's row statistics, the decode partials) cached, gives larger workspaces (grouped-query
// dK/dV shares) back at synchronization, and leaves the application's pools alone.
// stream_cached_buffer keeps one buffer per (device, stream) from that pool for the small
// per-call workspaces (see launch.hpp).

#include <algorithm>
#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <utility>
#include <vector>

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

struct StreamCacheEntry {
    std::mutex use;  // held by the call that is enqueuing work with the buffer
    void* ptr = nullptr;
    size_t bytes = 0;
    bool released = false;  // freed by release_stream_buffers (set under `use`)
};

namespace {
std::mutex g_cache_mutex;
// Shared ownership: a call that has looked an entry up keeps it alive while it waits for the
// entry's lock, also when release_stream_buffers takes the entry out of the map meanwhile.
std::map<std::pair<int, hipStream_t>, std::shared_ptr<StreamCacheEntry>> g_cache;
size_t g_cache_bytes[kMaxDevices] = {};  // bytes of the cached buffers per device
}  // namespace

bool stream_capturing(hipStream_t stream) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &status) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return status != hipStreamCaptureStatusNone;
}

bool stream_cached_buffer(hipStream_t stream, size_t bytes, void** out,
                          std::unique_lock<std::mutex>* lock, FlashAttentionError* err) {
    if (stream == hipStreamPerThread || stream_capturing(stream)) return false;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return false;
    }
    std::shared_ptr<StreamCacheEntry> e;
    {
        std::lock_guard<std::mutex> guard(g_cache_mutex);
        auto it = g_cache.find({dev, stream});
        if (it == g_cache.end()) {
            // No entry for a stream whose first buffer would not fit under the device total
            // (an entry that could never hold a buffer would only grow the map).
            const size_t first = (bytes + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1);
            if (g_cache_bytes[dev] + first > kStreamCacheTotalBytes) return false;
            it = g_cache.emplace(std::make_pair(dev, stream), std::make_shared<StreamCacheEntry>())
                     .first;
        }
        e = it->second;
    }
    std::unique_lock<std::mutex> use(e->use);
    if (e->released) return false;  // released after the lookup: this call takes a workspace
    if (e->bytes < bytes) {
        // Grow to at least twice the old size (in whole MiB, at most kStreamCacheBytes).
        size_t want = std::max(bytes, std::min(2 * e->bytes, kStreamCacheBytes));
        want = std::min(kStreamCacheBytes, (want + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1));
        {
            // The device's cached total stays within kStreamCacheTotalBytes: past it this call
            // takes a per-call workspace and the stream keeps its current buffer.
            std::lock_guard<std::mutex> guard(g_cache_mutex);
            if (g_cache_bytes[dev] - e->bytes + want > kStreamCacheTotalBytes) return false;
            g_cache_bytes[dev] += want - e->bytes;
        }
        void* p = nullptr;
        hipMemPool_t pool = workspace_pool();
        const hipError_t r = pool ? hipMallocFromPoolAsync(&p, want, pool, stream)
                                  : hipMallocAsync(&p, want, stream);
        if (r != hipSuccess) {
            (void)hipGetLastError();
            {
                std::lock_guard<std::mutex> guard(g_cache_mutex);
                g_cache_bytes[dev] -= want - e->bytes;
            }
            *err = r == hipErrorOutOfMemory ? FlashAttentionError::OUT_OF_MEMORY
                                            : FlashAttentionError::CUDA_ERROR;
            *out = nullptr;
            return true;
        }
        if (e->ptr) (void)hipFreeAsync(e->ptr, stream);  // after every earlier use on the stream
        e->ptr = p;
        e->bytes = want;
    }
    *out = e->ptr;
    *err = FlashAttentionError::SUCCESS;
    *lock = std::move(use);
    return true;
}

FlashAttentionError release_stream_buffers() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return FlashAttentionError::CUDA_ERROR;
    }
    // The entries are locked first, so that no call can enqueue work with their buffers, then
    // the device is drained (whether or not the streams still exist), then the buffers go back
    // to the pool. An entry held by a call on another host thread is kept.
    std::lock_guard<std::mutex> guard(g_cache_mutex);
    FlashAttentionError status = FlashAttentionError::SUCCESS;
    // `keep` is declared first so that it is destroyed last: the entries outlive their locks.
    std::vector<std::shared_ptr<StreamCacheEntry>> keep;
    std::vector<std::unique_lock<std::mutex>> held;
    for (auto& kv : g_cache) {
        if (kv.first.first != dev) continue;
        std::unique_lock<std::mutex> use(kv.second->use, std::try_to_lock);
        if (use.owns_lock()) {
            keep.push_back(kv.second);
            held.push_back(std::move(use));
        } else {
            status = FlashAttentionError::CUDA_ERROR;
        }
    }
    if (held.empty()) return status;
    if (hipDeviceSynchronize() != hipSuccess) {
        (void)hipGetLastError();
        return FlashAttentionError::CUDA_ERROR;  // nothing freed
    }
    for (auto it = g_cache.begin(); it != g_cache.end();) {
        StreamCacheEntry* e = it->second.get();
        const bool mine = std::find(keep.begin(), keep.end(), it->second) != keep.end();
        if (!mine) {
            ++it;
            continue;
        }
        // Stream-ordered free on the null stream: nothing is pending on the device any more.
        if (e->ptr && hipFreeAsync(e->ptr, nullptr) != hipSuccess) {
            (void)hipGetLastError();
            status = FlashAttentionError::CUDA_ERROR;
        }
        g_cache_bytes[dev] -= e->bytes;
        e->ptr = nullptr;
        e->bytes = 0;
        e->released = true;
        it = g_cache.erase(it);  // callers that looked it up keep it alive and see `released`
    }
    return status;  // `held` unlocks the entries
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

extern "C" {

int cuflash_release_workspaces(void) {
    return static_cast<int>(cuflash::detail::release_stream_buffers());
}

}  // extern "C"
