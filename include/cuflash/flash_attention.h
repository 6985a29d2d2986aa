#pragma once

// Public API of libcuflash_attn for AMD Instinct MI355X (gfx950).
//
// Drop-in for the reference's include/cuflash/flash_attention.h:
//   - same namespace, enum, enum values and order (SUCCESS=0 ... UNSUPPORTED_DTYPE=7),
//     reference flash_attention.h:12-21;
//   - same C++ overload set (float / half / bfloat16; L is always float*),
//     reference flash_attention.h:30-71;
//   - same C ABI names and argument order, reference flash_attention.h:81-118.
// CUDA types map to their HIP equivalents: half -> __half (hip_fp16.h),
// __nv_bfloat16 -> __hip_bfloat16 (hip_bf16.h), cudaStream_t -> hipStream_t. The C ABI is
// binary-identical for ctypes callers (every tensor is an opaque device pointer and the stream
// is an opaque pointer); the C++ overloads are source-compatible.
//
// Layout: every tensor is a contiguous row-major [batch_size, num_heads, seq_len, head_dim]
// device buffer; L is [batch_size, num_heads, seq_len] float. All work is enqueued on `stream`
// and nothing synchronizes the host; kernel execution errors surface at the caller's next
// synchronizing call, as in the reference.
//
// Additive entry points (no counterpart in the reference, which lists split-KV decoding as a
// roadmap item, ROADMAP.md:24-25): flash_attention_decode / cuflash_attention_decode_*.

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "cuflash/export.h"

namespace cuflash {

// Error codes. Values and order are part of the ABI (reference flash_attention.h:12-21).
enum class FlashAttentionError {
    SUCCESS = 0,
    INVALID_DIMENSION,     // a dimension is <= 0, or scale is NaN/Inf/negative
    DIMENSION_MISMATCH,    // declared for compatibility; never returned
    NULL_POINTER,          // an input or output pointer is null
    CUDA_ERROR,            // the HIP runtime reported an error (launch or allocation)
    OUT_OF_MEMORY,         // the backward/decode workspace could not be allocated
    UNSUPPORTED_HEAD_DIM,  // head_dim is not 32, 64 or 128
    UNSUPPORTED_DTYPE      // declared for compatibility; never returned
};

// Fixed English message per error code (reference src/api/flash_attention_api.cu:21-42).
CUFLASH_EXPORT const char* get_error_string(FlashAttentionError error);

// ---- Forward: O = softmax(scale * Q K^T [+ causal mask]) V,  L = logsumexp of each row ----
// Reference: include/cuflash/flash_attention.h:30-34 (float), :48-52 (half), :60-65 (bf16).
CUFLASH_EXPORT FlashAttentionError flash_attention_forward(const float* Q, const float* K,
                                                           const float* V, float* O, float* L,
                                                           int batch_size, int num_heads,
                                                           int seq_len, int head_dim, float scale,
                                                           bool causal, hipStream_t stream = 0);

CUFLASH_EXPORT FlashAttentionError flash_attention_forward(const __half* Q, const __half* K,
                                                           const __half* V, __half* O, float* L,
                                                           int batch_size, int num_heads,
                                                           int seq_len, int head_dim, float scale,
                                                           bool causal, hipStream_t stream = 0);

CUFLASH_EXPORT FlashAttentionError flash_attention_forward(
    const __hip_bfloat16* Q, const __hip_bfloat16* K, const __hip_bfloat16* V, __hip_bfloat16* O,
    float* L, int batch_size, int num_heads, int seq_len, int head_dim, float scale, bool causal,
    hipStream_t stream = 0);

// ---- Backward: dQ, dK, dV from Q, K, V, O, L (fp32 logsumexp) and dO ----
// dQ/dK/dV are overwritten. Reference: include/cuflash/flash_attention.h:37-40, :54-57, :67-71.
CUFLASH_EXPORT FlashAttentionError flash_attention_backward(
    const float* Q, const float* K, const float* V, const float* O, const float* L, const float* dO,
    float* dQ, float* dK, float* dV, int batch_size, int num_heads, int seq_len, int head_dim,
    float scale, bool causal, hipStream_t stream = 0);

CUFLASH_EXPORT FlashAttentionError flash_attention_backward(
    const __half* Q, const __half* K, const __half* V, const __half* O, const float* L,
    const __half* dO, __half* dQ, __half* dK, __half* dV, int batch_size, int num_heads,
    int seq_len, int head_dim, float scale, bool causal, hipStream_t stream = 0);

CUFLASH_EXPORT FlashAttentionError flash_attention_backward(
    const __hip_bfloat16* Q, const __hip_bfloat16* K, const __hip_bfloat16* V,
    const __hip_bfloat16* O, const float* L, const __hip_bfloat16* dO, __hip_bfloat16* dQ,
    __hip_bfloat16* dK, __hip_bfloat16* dV, int batch_size, int num_heads, int seq_len,
    int head_dim, float scale, bool causal, hipStream_t stream = 0);

// ---- Split-KV decode (additive; no reference counterpart, see ROADMAP.md:24-25) ----
// One query row per (batch, head) attends to kv_len keys, non-causal:
//   Q, O: [batch_size, num_heads, 1, head_dim]; K, V: [batch_size, num_heads, kv_len, head_dim];
//   L: [batch_size, num_heads] float logsumexp.
// The keys are cut into num_splits chunks; each chunk yields an unnormalized partial (O_s, m_s,
// l_s) in a stream-ordered workspace and a second kernel merges them with the online-softmax
// rule. num_splits == 0 picks a split count from the device's CU count; larger values than
// ceil(kv_len / 16) or 1024 are reduced to that. num_splits < 0 is INVALID_DIMENSION.
CUFLASH_EXPORT FlashAttentionError flash_attention_decode(const float* Q, const float* K,
                                                          const float* V, float* O, float* L,
                                                          int batch_size, int num_heads,
                                                          int kv_len, int head_dim, float scale,
                                                          int num_splits, hipStream_t stream = 0);

CUFLASH_EXPORT FlashAttentionError flash_attention_decode(const __half* Q, const __half* K,
                                                          const __half* V, __half* O, float* L,
                                                          int batch_size, int num_heads,
                                                          int kv_len, int head_dim, float scale,
                                                          int num_splits, hipStream_t stream = 0);

CUFLASH_EXPORT FlashAttentionError flash_attention_decode(
    const __hip_bfloat16* Q, const __hip_bfloat16* K, const __hip_bfloat16* V, __hip_bfloat16* O,
    float* L, int batch_size, int num_heads, int kv_len, int head_dim, float scale,
    int num_splits, hipStream_t stream = 0);

// ---- Grouped-query and paged decode (additive; extensions of the decode above) ----
// Grouped-query / multi-query attention: K, V have num_kv_heads heads, [batch_size,
// num_kv_heads, kv_len, head_dim], and query head h attends with key/value head
// h / (num_heads / num_kv_heads). num_heads must be a multiple of num_kv_heads
// (DIMENSION_MISMATCH otherwise). num_kv_heads == num_heads is flash_attention_decode.
CUFLASH_EXPORT FlashAttentionError flash_attention_decode_gqa(
    const float* Q, const float* K, const float* V, float* O, float* L, int batch_size, int num_heads,
    int num_kv_heads, int kv_len, int head_dim, float scale, int num_splits,
    hipStream_t stream = 0);
CUFLASH_EXPORT FlashAttentionError flash_attention_decode_gqa(
    const __half* Q, const __half* K, const __half* V, __half* O, float* L, int batch_size, int num_heads,
    int num_kv_heads, int kv_len, int head_dim, float scale, int num_splits,
    hipStream_t stream = 0);
CUFLASH_EXPORT FlashAttentionError flash_attention_decode_gqa(
    const __hip_bfloat16* Q, const __hip_bfloat16* K, const __hip_bfloat16* V, __hip_bfloat16* O, float* L, int batch_size, int num_heads,
    int num_kv_heads, int kv_len, int head_dim, float scale, int num_splits,
    hipStream_t stream = 0);

// Paged KV cache: K_cache, V_cache [num_pages, page_size, num_kv_heads, head_dim];
// block_table [batch_size, max_pages_per_seq] (int32) gives the page of keys
// [p * page_size, (p + 1) * page_size) of each sequence; seq_lens [batch_size] (int32) its
// length, clamped to [0, page_size * max_pages_per_seq]. Grouped-query heads as above. A
// sequence of length 0 gives O = 0 and L = -inf. All of Q, K_cache, V_cache, O, L,
// block_table and seq_lens are device pointers.
CUFLASH_EXPORT FlashAttentionError flash_attention_decode_paged(
    const float* Q, const float* K_cache, const float* V_cache, float* O, float* L,
    const int* block_table, const int* seq_lens, int batch_size, int num_heads, int num_kv_heads,
    int page_size, int max_pages_per_seq, int head_dim, float scale, int num_splits,
    hipStream_t stream = 0);
CUFLASH_EXPORT FlashAttentionError flash_attention_decode_paged(
    const __half* Q, const __half* K_cache, const __half* V_cache, __half* O, float* L,
    const int* block_table, const int* seq_lens, int batch_size, int num_heads, int num_kv_heads,
    int page_size, int max_pages_per_seq, int head_dim, float scale, int num_splits,
    hipStream_t stream = 0);
CUFLASH_EXPORT FlashAttentionError flash_attention_decode_paged(
    const __hip_bfloat16* Q, const __hip_bfloat16* K_cache, const __hip_bfloat16* V_cache, __hip_bfloat16* O, float* L,
    const int* block_table, const int* seq_lens, int batch_size, int num_heads, int num_kv_heads,
    int page_size, int max_pages_per_seq, int head_dim, float scale, int num_splits,
    hipStream_t stream = 0);

// ---- Extended forward / backward (additive; no reference counterpart) ----
// The forward and backward above with
//  * separate query and key/value lengths: Q, O, dO, dQ are [batch_size, num_heads, q_len,
//    head_dim], K, V, dK, dV are [batch_size, num_kv_heads, kv_len, head_dim], L is
//    [batch_size, num_heads, q_len] (prefill against a KV cache, cross-attention);
//  * grouped-query / multi-query heads: query head h reads key/value head
//    h / (num_heads / num_kv_heads); dK and dV of a key/value head are the sums over its query
//    heads. num_heads must be a multiple of num_kv_heads (DIMENSION_MISMATCH otherwise);
//  * head_dim in {32, 64, 96, 128, 256} (the functions above keep the reference's 32 / 64 / 128
//    and report UNSUPPORTED_HEAD_DIM for the others; so do these, with the same message).
// A causal mask is aligned to the end of the key sequence: query i sees keys
// j <= i + kv_len - q_len, so it needs q_len <= kv_len (DIMENSION_MISMATCH otherwise);
// q_len == kv_len is the usual mask. With num_kv_heads == num_heads, q_len == kv_len and a
// head_dim of 32 / 64 / 128 the results equal flash_attention_forward / _backward.
CUFLASH_EXPORT FlashAttentionError flash_attention_forward_ext(
    const float* Q, const float* K, const float* V, float* O, float* L, int batch_size,
    int num_heads, int num_kv_heads, int q_len, int kv_len, int head_dim, float scale,
    bool causal = false, hipStream_t stream = 0);
CUFLASH_EXPORT FlashAttentionError flash_attention_forward_ext(
    const __half* Q, const __half* K, const __half* V, __half* O, float* L, int batch_size,
    int num_heads, int num_kv_heads, int q_len, int kv_len, int head_dim, float scale,
    bool causal = false, hipStream_t stream = 0);
CUFLASH_EXPORT FlashAttentionError flash_attention_forward_ext(
    const __hip_bfloat16* Q, const __hip_bfloat16* K, const __hip_bfloat16* V,
    __hip_bfloat16* O, float* L, int batch_size, int num_heads, int num_kv_heads, int q_len,
    int kv_len, int head_dim, float scale, bool causal = false, hipStream_t stream = 0);
CUFLASH_EXPORT FlashAttentionError flash_attention_backward_ext(
    const float* Q, const float* K, const float* V, const float* O, const float* L,
    const float* dO, float* dQ, float* dK, float* dV, int batch_size, int num_heads,
    int num_kv_heads, int q_len, int kv_len, int head_dim, float scale, bool causal = false,
    hipStream_t stream = 0);
CUFLASH_EXPORT FlashAttentionError flash_attention_backward_ext(
    const __half* Q, const __half* K, const __half* V, const __half* O, const float* L,
    const __half* dO, __half* dQ, __half* dK, __half* dV, int batch_size, int num_heads,
    int num_kv_heads, int q_len, int kv_len, int head_dim, float scale, bool causal = false,
    hipStream_t stream = 0);
CUFLASH_EXPORT FlashAttentionError flash_attention_backward_ext(
    const __hip_bfloat16* Q, const __hip_bfloat16* K, const __hip_bfloat16* V,
    const __hip_bfloat16* O, const float* L, const __hip_bfloat16* dO, __hip_bfloat16* dQ,
    __hip_bfloat16* dK, __hip_bfloat16* dV, int batch_size, int num_heads, int num_kv_heads,
    int q_len, int kv_len, int head_dim, float scale, bool causal = false,
    hipStream_t stream = 0);

}  // namespace cuflash

#ifdef __cplusplus
extern "C" {
#endif

// Stable C ABI. Return values are the integer value of cuflash::FlashAttentionError.
// Each declaration replaces the reference symbol of the same name
// (include/cuflash/flash_attention.h:81-118; defined at src/api/flash_attention_api.cu:188-240).

// Replaces reference flash_attention.h:83-86.
CUFLASH_EXPORT int cuflash_attention_forward_f32(const float* Q, const float* K, const float* V,
                                                 float* O, float* L, int batch_size, int num_heads,
                                                 int seq_len, int head_dim, float scale,
                                                 bool causal, hipStream_t stream);

// Replaces reference flash_attention.h:88-92.
CUFLASH_EXPORT int cuflash_attention_backward_f32(const float* Q, const float* K, const float* V,
                                                  const float* O, const float* L, const float* dO,
                                                  float* dQ, float* dK, float* dV, int batch_size,
                                                  int num_heads, int seq_len, int head_dim,
                                                  float scale, bool causal, hipStream_t stream);

// Replaces reference flash_attention.h:94-97.
CUFLASH_EXPORT int cuflash_attention_forward_f16(const __half* Q, const __half* K, const __half* V,
                                                 __half* O, float* L, int batch_size,
                                                 int num_heads, int seq_len, int head_dim,
                                                 float scale, bool causal, hipStream_t stream);

// Replaces reference flash_attention.h:99-103.
CUFLASH_EXPORT int cuflash_attention_backward_f16(const __half* Q, const __half* K,
                                                  const __half* V, const __half* O, const float* L,
                                                  const __half* dO, __half* dQ, __half* dK,
                                                  __half* dV, int batch_size, int num_heads,
                                                  int seq_len, int head_dim, float scale,
                                                  bool causal, hipStream_t stream);

// Replaces reference flash_attention.h:105-109.
CUFLASH_EXPORT int cuflash_attention_forward_bf16(const __hip_bfloat16* Q,
                                                  const __hip_bfloat16* K,
                                                  const __hip_bfloat16* V, __hip_bfloat16* O,
                                                  float* L, int batch_size, int num_heads,
                                                  int seq_len, int head_dim, float scale,
                                                  bool causal, hipStream_t stream);

// Replaces reference flash_attention.h:111-116.
CUFLASH_EXPORT int cuflash_attention_backward_bf16(
    const __hip_bfloat16* Q, const __hip_bfloat16* K, const __hip_bfloat16* V,
    const __hip_bfloat16* O, const float* L, const __hip_bfloat16* dO, __hip_bfloat16* dQ,
    __hip_bfloat16* dK, __hip_bfloat16* dV, int batch_size, int num_heads, int seq_len,
    int head_dim, float scale, bool causal, hipStream_t stream);

// Replaces reference flash_attention.h:119 (cuflash_error_string).
CUFLASH_EXPORT const char* cuflash_error_string(int error_code);

// Additive split-KV decode ABI (no reference counterpart; ROADMAP.md:24-25 lists it as planned).
CUFLASH_EXPORT int cuflash_attention_decode_f32(const float* Q, const float* K, const float* V,
                                                float* O, float* L, int batch_size, int num_heads,
                                                int kv_len, int head_dim, float scale,
                                                int num_splits, hipStream_t stream);

CUFLASH_EXPORT int cuflash_attention_decode_f16(const __half* Q, const __half* K, const __half* V,
                                                __half* O, float* L, int batch_size,
                                                int num_heads, int kv_len, int head_dim,
                                                float scale, int num_splits, hipStream_t stream);

CUFLASH_EXPORT int cuflash_attention_decode_bf16(const __hip_bfloat16* Q, const __hip_bfloat16* K,
                                                 const __hip_bfloat16* V, __hip_bfloat16* O,
                                                 float* L, int batch_size, int num_heads,
                                                 int kv_len, int head_dim, float scale,
                                                 int num_splits, hipStream_t stream);

// Decode that allocates nothing. No counterpart in the reference: it is for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc). Same arguments, validation and results as cuflash_attention_decode_f16,
// bitwise; the split partials, batch_size * num_heads * splits * (head_dim + 2) * 4 bytes, go to
// a fixed 32 MiB device array that the library holds on every GPU it runs on until the process
// ends, instead of a stream-ordered workspace. A call whose partials exceed 32 MiB returns
// OUT_OF_MEMORY (5) before any device work (pass num_splits explicitly to bound them; config 4,
// 16 x 32 heads at 64 splits, needs 16.3 MiB). Calls on one GPU share the array: calls that
// overlap in time on one GPU (two streams, two host threads) race; calls ordered on one stream
// do not.
CUFLASH_EXPORT int cuflash_attention_decode_noalloc_f16(const __half* Q, const __half* K,
                                                        const __half* V, __half* O, float* L,
                                                        int batch_size, int num_heads, int kv_len,
                                                        int head_dim, float scale, int num_splits,
                                                        hipStream_t stream);

// Grouped-query and paged decode ABI (additive; same arguments as the C++ functions above).
CUFLASH_EXPORT int cuflash_attention_decode_gqa_f32(
    const float* Q, const float* K, const float* V, float* O, float* L, int batch_size, int num_heads,
    int num_kv_heads, int kv_len, int head_dim, float scale, int num_splits, hipStream_t stream);
CUFLASH_EXPORT int cuflash_attention_decode_paged_f32(
    const float* Q, const float* K_cache, const float* V_cache, float* O, float* L,
    const int* block_table, const int* seq_lens, int batch_size, int num_heads, int num_kv_heads,
    int page_size, int max_pages_per_seq, int head_dim, float scale, int num_splits,
    hipStream_t stream);
CUFLASH_EXPORT int cuflash_attention_decode_gqa_f16(
    const __half* Q, const __half* K, const __half* V, __half* O, float* L, int batch_size, int num_heads,
    int num_kv_heads, int kv_len, int head_dim, float scale, int num_splits, hipStream_t stream);
CUFLASH_EXPORT int cuflash_attention_decode_paged_f16(
    const __half* Q, const __half* K_cache, const __half* V_cache, __half* O, float* L,
    const int* block_table, const int* seq_lens, int batch_size, int num_heads, int num_kv_heads,
    int page_size, int max_pages_per_seq, int head_dim, float scale, int num_splits,
    hipStream_t stream);
CUFLASH_EXPORT int cuflash_attention_decode_gqa_bf16(
    const __hip_bfloat16* Q, const __hip_bfloat16* K, const __hip_bfloat16* V, __hip_bfloat16* O, float* L, int batch_size, int num_heads,
    int num_kv_heads, int kv_len, int head_dim, float scale, int num_splits, hipStream_t stream);
CUFLASH_EXPORT int cuflash_attention_decode_paged_bf16(
    const __hip_bfloat16* Q, const __hip_bfloat16* K_cache, const __hip_bfloat16* V_cache, __hip_bfloat16* O, float* L,
    const int* block_table, const int* seq_lens, int batch_size, int num_heads, int num_kv_heads,
    int page_size, int max_pages_per_seq, int head_dim, float scale, int num_splits,
    hipStream_t stream);

// Extended forward / backward ABI (additive; same arguments as the C++ functions above).
CUFLASH_EXPORT int cuflash_attention_forward_ext_f32(
    const float* Q, const float* K, const float* V, float* O, float* L, int batch_size,
    int num_heads, int num_kv_heads, int q_len, int kv_len, int head_dim, float scale,
    bool causal, hipStream_t stream);
CUFLASH_EXPORT int cuflash_attention_backward_ext_f32(
    const float* Q, const float* K, const float* V, const float* O, const float* L,
    const float* dO, float* dQ, float* dK, float* dV, int batch_size, int num_heads,
    int num_kv_heads, int q_len, int kv_len, int head_dim, float scale, bool causal,
    hipStream_t stream);
CUFLASH_EXPORT int cuflash_attention_forward_ext_f16(
    const __half* Q, const __half* K, const __half* V, __half* O, float* L, int batch_size,
    int num_heads, int num_kv_heads, int q_len, int kv_len, int head_dim, float scale,
    bool causal, hipStream_t stream);
CUFLASH_EXPORT int cuflash_attention_backward_ext_f16(
    const __half* Q, const __half* K, const __half* V, const __half* O, const float* L,
    const __half* dO, __half* dQ, __half* dK, __half* dV, int batch_size, int num_heads,
    int num_kv_heads, int q_len, int kv_len, int head_dim, float scale, bool causal,
    hipStream_t stream);
CUFLASH_EXPORT int cuflash_attention_forward_ext_bf16(
    const __hip_bfloat16* Q, const __hip_bfloat16* K, const __hip_bfloat16* V,
    __hip_bfloat16* O, float* L, int batch_size, int num_heads, int num_kv_heads, int q_len,
    int kv_len, int head_dim, float scale, bool causal, hipStream_t stream);
CUFLASH_EXPORT int cuflash_attention_backward_ext_bf16(
    const __hip_bfloat16* Q, const __hip_bfloat16* K, const __hip_bfloat16* V,
    const __hip_bfloat16* O, const float* L, const __hip_bfloat16* dO, __hip_bfloat16* dQ,
    __hip_bfloat16* dK, __hip_bfloat16* dV, int batch_size, int num_heads, int num_kv_heads,
    int q_len, int kv_len, int head_dim, float scale, bool causal, hipStream_t stream);

// Library version string (CUFLASH_VERSION); additive.
CUFLASH_EXPORT const char* cuflash_version(void);

// Measurement hooks (additive; no reference counterpart). While enabled, each kernel launch is
// bracketed by hipEventRecord on its stream. cuflash_profile_report waits for the recorded
// events, writes one "label<TAB>launches<TAB>total_ms" line per kernel label into buf (at most
// buflen bytes, NUL-terminated), clears the records and returns the size the full report needs.
CUFLASH_EXPORT void cuflash_profile_enable(int enabled);
CUFLASH_EXPORT int cuflash_profile_report(char* buf, int buflen);

// Releases the small per-stream workspaces the library caches on the current device (no
// reference counterpart; the reference allocates and frees per call). Calls on a stream reuse
// one device buffer of up to 64 MiB, kept from call to call; the buffers of all streams of a
// device total at most 256 MiB, past which further streams get per-call workspaces. This call
// synchronizes the device and frees them all; later calls allocate afresh. Call it before
// destroying streams that the library has used if new streams may get the same handle values
// while earlier work could still be in flight, and when the memory is wanted back. Returns 0,
// or 4 (CUDA_ERROR) if the device wait fails or a buffer is in use by a concurrent call on
// another host thread (that buffer is kept).
CUFLASH_EXPORT int cuflash_release_workspaces(void);

#ifdef __cplusplus
}
#endif
