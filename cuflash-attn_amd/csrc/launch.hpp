#pragma once

// Internal launcher interface between the validating API layer (api.cpp) and the gfx950
// kernels (forward.hip, backward.hip, decode.hip). Arguments have already been validated when a
// launcher runs; launchers only check the HIP runtime.

#include <mutex>

#include "cuflash/flash_attention.h"

namespace cuflash {
namespace detail {

// Counterpart of the reference's launch_flash_attention_forward_typed<T>
// (src/forward/flash_attention_forward_typed.cu:212-302).
template <typename T>
FlashAttentionError launch_forward(const T* Q, const T* K, const T* V, T* O, float* L,
                                   int batch_size, int num_heads, int seq_len, int head_dim,
                                   float scale, bool causal, hipStream_t stream);

// Counterpart of the reference's launch_flash_attention_backward_typed<T>
// (src/backward/flash_attention_backward_typed.cu:440-579).
template <typename T>
FlashAttentionError launch_backward(const T* Q, const T* K, const T* V, const T* O,
                                    const float* L, const T* dO, T* dQ, T* dK, T* dV,
                                    int batch_size, int num_heads, int seq_len, int head_dim,
                                    float scale, bool causal, hipStream_t stream);

// Forward and backward with separate query / key lengths, num_kv_heads key/value heads shared by
// num_heads / num_kv_heads query heads each, and head_dim in {32, 64, 96, 128, 256}
// (no reference counterpart). Q, O, dO, dQ are [B, num_heads, q_len, D], K, V, dK, dV are
// [B, num_kv_heads, kv_len, D]; a causal mask is aligned to the end of the key sequence
// (query i sees keys j <= i + kv_len - q_len) and needs q_len <= kv_len.
template <typename T>
FlashAttentionError launch_forward_ext(const T* Q, const T* K, const T* V, T* O, float* L,
                                       int batch_size, int num_heads, int num_kv_heads,
                                       int q_len, int kv_len, int head_dim, float scale,
                                       bool causal, hipStream_t stream);
template <typename T>
FlashAttentionError launch_backward_ext(const T* Q, const T* K, const T* V, const T* O,
                                        const float* L, const T* dO, T* dQ, T* dK, T* dV,
                                        int batch_size, int num_heads, int num_kv_heads,
                                        int q_len, int kv_len, int head_dim, float scale,
                                        bool causal, hipStream_t stream);

// Split-KV decode (no reference counterpart).
template <typename T>
FlashAttentionError launch_decode(const T* Q, const T* K, const T* V, T* O, float* L,
                                  int batch_size, int num_heads, int kv_len, int head_dim,
                                  float scale, int num_splits, hipStream_t stream);

// Decode with num_kv_heads key/value heads shared by num_heads / num_kv_heads query heads each
// (K, V [B, num_kv_heads, kv_len, D]).
template <typename T>
FlashAttentionError launch_decode_gqa(const T* Q, const T* K, const T* V, T* O, float* L,
                                      int batch_size, int num_heads, int num_kv_heads,
                                      int kv_len, int head_dim, float scale, int num_splits,
                                      hipStream_t stream);

// Decode over a paged cache K_cache, V_cache [num_pages, page_size, num_kv_heads, D] with
// block_table [B, max_pages_per_seq] and seq_lens [B].
template <typename T>
FlashAttentionError launch_decode_paged(const T* Q, const T* K_cache, const T* V_cache, T* O,
                                        float* L, const int* block_table, const int* seq_lens,
                                        int batch_size, int num_heads, int num_kv_heads,
                                        int page_size, int max_pages_per_seq, int head_dim,
                                        float scale, int num_splits, hipStream_t stream);

// Decode (as launch_decode) with the split partials in a fixed device array of
// kDecodeScratchBytes per GPU instead of an allocated workspace: no allocation of any kind.
// A call whose partials, B * H * splits * (head_dim + 2) * 4 bytes, exceed the array returns
// OUT_OF_MEMORY before any launch. Calls that overlap in time on one GPU share the array and
// race. Instantiated for __half.
constexpr size_t kDecodeScratchBytes = size_t(32) << 20;
template <typename T>
FlashAttentionError launch_decode_noalloc(const T* Q, const T* K, const T* V, T* O, float* L,
                                          int batch_size, int num_heads, int kv_len,
                                          int head_dim, float scale, int num_splits,
                                          hipStream_t stream);

// Maps a HIP status after a launch or allocation to the library's error code.
inline FlashAttentionError from_hip(hipError_t e) {
    if (e == hipSuccess) return FlashAttentionError::SUCCESS;
    if (e == hipErrorOutOfMemory) return FlashAttentionError::OUT_OF_MEMORY;
    return FlashAttentionError::CUDA_ERROR;
}

// Compute units of the current device (cached per device; 256 on MI355X when the query fails).
int compute_units();

// The library's own stream-ordered memory pool on the current device (created on first use and
// kept until the process ends; up to 256 MiB of freed blocks stay in the pool across
// synchronizations, so later allocations of the same size need no driver call). Using a private
// pool leaves the application's default pool and its settings untouched. nullptr when it cannot
// be created (the workspaces then come from the device's current pool).
hipMemPool_t workspace_pool();

// A device buffer kept per (device, stream) for the launchers' small workspaces: the first
// call on a stream allocates it stream-ordered from workspace_pool(), later calls reuse it, and a
// call that needs more replaces it (the old one is freed stream-ordered, after every earlier use
// on the stream). Reusing it saves each call the stream-ordered allocation and free, which leave
// the GPU idle for about 6 us between the call's last kernel and the next work on the stream.
// The returned lock holds the entry until the caller's kernels are enqueued, so that two host
// threads on one stream cannot free a buffer the other is about to use; calls on different
// streams never share one. Up to kStreamCacheBytes per (device, stream) stay allocated until the
// process ends. hipStreamPerThread names a different stream in every host thread, so it is not
// cached (stream_cached_buffer returns false), nor is a stream that is being captured into a
// graph: every replay of the graph would use the buffer, after later calls had replaced it.
// The buffers of all streams of one device total at most kStreamCacheTotalBytes: a call whose
// stream would need a new or larger cached buffer beyond that gets a per-call workspace instead
// (stream_cached_buffer returns false), so an application that creates a stream per request does
// not grow device memory without bound. Nothing is evicted (a cached stream handle may already
// be destroyed, so its buffer cannot be freed stream-ordered); cuflash_release_workspaces()
// frees them all.
constexpr size_t kStreamCacheBytes = size_t(64) << 20;
constexpr size_t kStreamCacheTotalBytes = size_t(256) << 20;
struct StreamCacheEntry;
bool stream_cached_buffer(hipStream_t stream, size_t bytes, void** out,
                          std::unique_lock<std::mutex>* lock, FlashAttentionError* err);

// cuflash_release_workspaces: takes the cached buffers of the current device's streams away
// from later calls, waits for the device, then frees them. CUDA_ERROR if the device wait fails
// (nothing is freed) or a buffer is in use by a call on another host thread (that buffer is
// kept). A call that looked its stream's buffer up before the release takes a per-call
// workspace instead.
FlashAttentionError release_stream_buffers();

// Whether `stream` is being captured into a graph (false if that cannot be determined).
bool stream_capturing(hipStream_t stream);

// Stream-ordered device workspace, the counterpart of the reference's AsyncFloatBuffer
// (src/backward/flash_attention_backward_typed.cu:374-394). Either the stream's cached buffer
// (`cached`, for workspaces of at most kStreamCacheBytes; at most one cached workspace per call)
// or a per-call hipMallocFromPoolAsync / hipFreeAsync on the caller's stream (hipMallocAsync from
// the device's current pool on a stream that is being captured, which the graph records as an
// allocation and a free of its own). Either way the host never synchronizes and concurrent calls
// on different streams never share memory.
class StreamWorkspace {
public:
    explicit StreamWorkspace(hipStream_t stream, bool cached = false)
        : stream_(stream), cached_(cached) {}
    StreamWorkspace(const StreamWorkspace&) = delete;
    StreamWorkspace& operator=(const StreamWorkspace&) = delete;
    ~StreamWorkspace() {
        if (ptr_ && owned_) (void)hipFreeAsync(ptr_, stream_);
    }
    FlashAttentionError alloc(size_t bytes) {
        if (cached_ && bytes <= kStreamCacheBytes) {
            FlashAttentionError err = FlashAttentionError::SUCCESS;
            if (stream_cached_buffer(stream_, bytes, &ptr_, &lock_, &err)) {
                owned_ = false;
                return err;
            }
        }
        hipMemPool_t pool = stream_capturing(stream_) ? nullptr : workspace_pool();
        hipError_t e = pool ? hipMallocFromPoolAsync(&ptr_, bytes, pool, stream_)
                            : hipMallocAsync(&ptr_, bytes, stream_);
        if (e != hipSuccess) {
            ptr_ = nullptr;
            (void)hipGetLastError();
            return e == hipErrorOutOfMemory ? FlashAttentionError::OUT_OF_MEMORY
                                            : FlashAttentionError::CUDA_ERROR;
        }
        owned_ = true;
        return FlashAttentionError::SUCCESS;
    }
    void* get() const { return ptr_; }

private:
    hipStream_t stream_;
    bool cached_;
    bool owned_ = false;
    void* ptr_ = nullptr;
    std::unique_lock<std::mutex> lock_;  // held while the cached buffer is in use by this call
};

}  // namespace detail
}  // namespace cuflash
