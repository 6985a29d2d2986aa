// Validating API layer and C ABI of libcuflash_attn.
//
// Mirrors the reference's src/api/flash_attention_api.cu: the same validation order
// (null pointers -> dimensions -> head_dim -> scale; backward checks its gradient pointers
// first), the same error codes, and the same fixed message strings, so callers that compare
// codes or strings (reference tests/unit/test_error_handling.cu:21-253,
// tests/integration/test_api_smoke.cpp:11-41) see identical behaviour. No HIP call is made
// before validation succeeds, so every validation error is reported without touching a GPU.

#include <cmath>

#include "cuflash/flash_attention.h"
#include "cuflash/version.h"
#include "launch.hpp"

namespace cuflash {

// Reference: src/api/flash_attention_api.cu:21-42. The strings are part of the interface
// (compared verbatim by the reference's ErrorStrings test), so they are kept unchanged.
const char* get_error_string(FlashAttentionError error) {
    switch (error) {
        case FlashAttentionError::SUCCESS:
            return "Success";
        case FlashAttentionError::INVALID_DIMENSION:
            return "Invalid dimension: dimensions must be positive";
        case FlashAttentionError::DIMENSION_MISMATCH:
            return "Dimension mismatch: Q, K, V tensors have incompatible shapes";
        case FlashAttentionError::NULL_POINTER:
            return "Null pointer: input or output pointer is null";
        case FlashAttentionError::CUDA_ERROR:
            return "CUDA error occurred";
        case FlashAttentionError::OUT_OF_MEMORY:
            return "Out of memory: insufficient GPU memory";
        case FlashAttentionError::UNSUPPORTED_HEAD_DIM:
            return "Unsupported head_dim: must be 32, 64, or 128";
        case FlashAttentionError::UNSUPPORTED_DTYPE:
            return "Unsupported data type";
        default:
            return "Unknown error";
    }
}

namespace {

bool supported_head_dim(int head_dim) {
    return head_dim == 32 || head_dim == 64 || head_dim == 128;
}

// Reference: validate_common_params, src/api/flash_attention_api.cu:45-66.
FlashAttentionError check_common(const void* Q, const void* K, const void* V, const void* O,
                                 const void* L, int batch_size, int num_heads, int seq_len,
                                 int head_dim, float scale) {
    if (!Q || !K || !V || !O || !L) return FlashAttentionError::NULL_POINTER;
    if (batch_size <= 0 || num_heads <= 0 || seq_len <= 0 || head_dim <= 0)
        return FlashAttentionError::INVALID_DIMENSION;
    if (!supported_head_dim(head_dim)) return FlashAttentionError::UNSUPPORTED_HEAD_DIM;
    if (!std::isfinite(scale) || scale < 0.0f) return FlashAttentionError::INVALID_DIMENSION;
    return FlashAttentionError::SUCCESS;
}

// Reference: validate_params_backward, src/api/flash_attention_api.cu:69-79.
FlashAttentionError check_backward(const void* Q, const void* K, const void* V, const void* O,
                                   const void* L, const void* dO, const void* dQ, const void* dK,
                                   const void* dV, int batch_size, int num_heads, int seq_len,
                                   int head_dim, float scale) {
    if (!dO || !dQ || !dK || !dV) return FlashAttentionError::NULL_POINTER;
    return check_common(Q, K, V, O, L, batch_size, num_heads, seq_len, head_dim, scale);
}

// Decode uses the forward checks with kv_len in place of seq_len, plus num_splits >= 0.
FlashAttentionError check_decode(const void* Q, const void* K, const void* V, const void* O,
                                 const void* L, int batch_size, int num_heads, int kv_len,
                                 int head_dim, float scale, int num_splits) {
    FlashAttentionError err =
        check_common(Q, K, V, O, L, batch_size, num_heads, kv_len, head_dim, scale);
    if (err != FlashAttentionError::SUCCESS) return err;
    if (num_splits < 0) return FlashAttentionError::INVALID_DIMENSION;
    return FlashAttentionError::SUCCESS;
}

// Grouped-query decode: the decode checks with the key/value head count, then the grouping
// (num_heads a multiple of num_kv_heads, else DIMENSION_MISMATCH).
FlashAttentionError check_decode_gqa(const void* Q, const void* K, const void* V, const void* O,
                                     const void* L, int batch_size, int num_heads,
                                     int num_kv_heads, int kv_len, int head_dim, float scale,
                                     int num_splits) {
    FlashAttentionError err =
        check_decode(Q, K, V, O, L, batch_size, num_heads, kv_len, head_dim, scale, num_splits);
    if (err != FlashAttentionError::SUCCESS) return err;
    if (num_kv_heads <= 0) return FlashAttentionError::INVALID_DIMENSION;
    if (num_heads % num_kv_heads != 0) return FlashAttentionError::DIMENSION_MISMATCH;
    return FlashAttentionError::SUCCESS;
}

// Paged decode: every pointer (also block_table and seq_lens) non-null, then page_size and
// max_pages_per_seq positive; the capacity page_size * max_pages_per_seq then stands in for
// kv_len in the grouped-query checks.
FlashAttentionError check_decode_paged(const void* Q, const void* K, const void* V,
                                       const void* O, const void* L, const int* block_table,
                                       const int* seq_lens, int batch_size, int num_heads,
                                       int num_kv_heads, int page_size, int max_pages_per_seq,
                                       int head_dim, float scale, int num_splits) {
    if (!Q || !K || !V || !O || !L || !block_table || !seq_lens)
        return FlashAttentionError::NULL_POINTER;
    if (page_size <= 0 || max_pages_per_seq <= 0) return FlashAttentionError::INVALID_DIMENSION;
    const long long cap = static_cast<long long>(page_size) * max_pages_per_seq;
    if (cap > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
    return check_decode_gqa(Q, K, V, O, L, batch_size, num_heads, num_kv_heads,
                            static_cast<int>(cap), head_dim, scale, num_splits);
}

// Extended forward / backward: the forward checks in the same order with num_kv_heads, q_len and
// kv_len as dimensions and head_dim in {32, 64, 96, 128, 256}; then num_heads must be a
// multiple of num_kv_heads, and a causal mask needs q_len <= kv_len (the queries are the last
// q_len positions of the key sequence), else DIMENSION_MISMATCH.
bool supported_head_dim_ext(int head_dim) {
    return supported_head_dim(head_dim) || head_dim == 96 || head_dim == 256;
}

FlashAttentionError check_ext(const void* Q, const void* K, const void* V, const void* O,
                              const void* L, int batch_size, int num_heads, int num_kv_heads,
                              int q_len, int kv_len, int head_dim, float scale, bool causal) {
    if (!Q || !K || !V || !O || !L) return FlashAttentionError::NULL_POINTER;
    if (batch_size <= 0 || num_heads <= 0 || num_kv_heads <= 0 || q_len <= 0 || kv_len <= 0 ||
        head_dim <= 0)
        return FlashAttentionError::INVALID_DIMENSION;
    if (!supported_head_dim_ext(head_dim)) return FlashAttentionError::UNSUPPORTED_HEAD_DIM;
    if (!std::isfinite(scale) || scale < 0.0f) return FlashAttentionError::INVALID_DIMENSION;
    if (num_heads % num_kv_heads != 0) return FlashAttentionError::DIMENSION_MISMATCH;
    if (causal && q_len > kv_len) return FlashAttentionError::DIMENSION_MISMATCH;
    return FlashAttentionError::SUCCESS;
}

template <typename T>
FlashAttentionError forward_ext_impl(const T* Q, const T* K, const T* V, T* O, float* L, int b,
                                     int h, int hkv, int nq, int nk, int d, float scale,
                                     bool causal, hipStream_t stream) {
    FlashAttentionError err = check_ext(Q, K, V, O, L, b, h, hkv, nq, nk, d, scale, causal);
    if (err != FlashAttentionError::SUCCESS) return err;
    return detail::launch_forward_ext<T>(Q, K, V, O, L, b, h, hkv, nq, nk, d, scale, causal,
                                         stream);
}

template <typename T>
FlashAttentionError backward_ext_impl(const T* Q, const T* K, const T* V, const T* O,
                                      const float* L, const T* dO, T* dQ, T* dK, T* dV, int b,
                                      int h, int hkv, int nq, int nk, int d, float scale,
                                      bool causal, hipStream_t stream) {
    if (!dO || !dQ || !dK || !dV) return FlashAttentionError::NULL_POINTER;
    FlashAttentionError err = check_ext(Q, K, V, O, L, b, h, hkv, nq, nk, d, scale, causal);
    if (err != FlashAttentionError::SUCCESS) return err;
    return detail::launch_backward_ext<T>(Q, K, V, O, L, dO, dQ, dK, dV, b, h, hkv, nq, nk, d,
                                          scale, causal, stream);
}

template <typename T>
FlashAttentionError forward_impl(const T* Q, const T* K, const T* V, T* O, float* L, int b,
                                 int h, int n, int d, float scale, bool causal,
                                 hipStream_t stream) {
    FlashAttentionError err = check_common(Q, K, V, O, L, b, h, n, d, scale);
    if (err != FlashAttentionError::SUCCESS) return err;
    return detail::launch_forward<T>(Q, K, V, O, L, b, h, n, d, scale, causal, stream);
}

template <typename T>
FlashAttentionError backward_impl(const T* Q, const T* K, const T* V, const T* O,
                                  const float* L, const T* dO, T* dQ, T* dK, T* dV, int b, int h,
                                  int n, int d, float scale, bool causal, hipStream_t stream) {
    FlashAttentionError err = check_backward(Q, K, V, O, L, dO, dQ, dK, dV, b, h, n, d, scale);
    if (err != FlashAttentionError::SUCCESS) return err;
    return detail::launch_backward<T>(Q, K, V, O, L, dO, dQ, dK, dV, b, h, n, d, scale, causal,
                                      stream);
}

template <typename T>
FlashAttentionError decode_impl(const T* Q, const T* K, const T* V, T* O, float* L, int b, int h,
                                int kv_len, int d, float scale, int num_splits,
                                hipStream_t stream) {
    FlashAttentionError err = check_decode(Q, K, V, O, L, b, h, kv_len, d, scale, num_splits);
    if (err != FlashAttentionError::SUCCESS) return err;
    return detail::launch_decode<T>(Q, K, V, O, L, b, h, kv_len, d, scale, num_splits, stream);
}

template <typename T>
FlashAttentionError decode_gqa_impl(const T* Q, const T* K, const T* V, T* O, float* L, int b,
                                    int h, int hkv, int kv_len, int d, float scale,
                                    int num_splits, hipStream_t stream) {
    FlashAttentionError err =
        check_decode_gqa(Q, K, V, O, L, b, h, hkv, kv_len, d, scale, num_splits);
    if (err != FlashAttentionError::SUCCESS) return err;
    return detail::launch_decode_gqa<T>(Q, K, V, O, L, b, h, hkv, kv_len, d, scale, num_splits,
                                        stream);
}

template <typename T>
FlashAttentionError decode_paged_impl(const T* Q, const T* Kc, const T* Vc, T* O, float* L,
                                      const int* table, const int* lens, int b, int h, int hkv,
                                      int page_size, int max_pages, int d, float scale,
                                      int num_splits, hipStream_t stream) {
    FlashAttentionError err = check_decode_paged(Q, Kc, Vc, O, L, table, lens, b, h, hkv,
                                                 page_size, max_pages, d, scale, num_splits);
    if (err != FlashAttentionError::SUCCESS) return err;
    return detail::launch_decode_paged<T>(Q, Kc, Vc, O, L, table, lens, b, h, hkv, page_size,
                                          max_pages, d, scale, num_splits, stream);
}

}  // namespace

// ===== C++ API (reference src/api/flash_attention_api.cu:84-180) =====

FlashAttentionError flash_attention_forward(const float* Q, const float* K, const float* V,
                                            float* O, float* L, int batch_size, int num_heads,
                                            int seq_len, int head_dim, float scale, bool causal,
                                            hipStream_t stream) {
    return forward_impl(Q, K, V, O, L, batch_size, num_heads, seq_len, head_dim, scale, causal,
                        stream);
}

FlashAttentionError flash_attention_forward(const __half* Q, const __half* K, const __half* V,
                                            __half* O, float* L, int batch_size, int num_heads,
                                            int seq_len, int head_dim, float scale, bool causal,
                                            hipStream_t stream) {
    return forward_impl(Q, K, V, O, L, batch_size, num_heads, seq_len, head_dim, scale, causal,
                        stream);
}

FlashAttentionError flash_attention_forward(const __hip_bfloat16* Q, const __hip_bfloat16* K,
                                            const __hip_bfloat16* V, __hip_bfloat16* O, float* L,
                                            int batch_size, int num_heads, int seq_len,
                                            int head_dim, float scale, bool causal,
                                            hipStream_t stream) {
    return forward_impl(Q, K, V, O, L, batch_size, num_heads, seq_len, head_dim, scale, causal,
                        stream);
}

FlashAttentionError flash_attention_backward(const float* Q, const float* K, const float* V,
                                             const float* O, const float* L, const float* dO,
                                             float* dQ, float* dK, float* dV, int batch_size,
                                             int num_heads, int seq_len, int head_dim, float scale,
                                             bool causal, hipStream_t stream) {
    return backward_impl(Q, K, V, O, L, dO, dQ, dK, dV, batch_size, num_heads, seq_len, head_dim,
                         scale, causal, stream);
}

FlashAttentionError flash_attention_backward(const __half* Q, const __half* K, const __half* V,
                                             const __half* O, const float* L, const __half* dO,
                                             __half* dQ, __half* dK, __half* dV, int batch_size,
                                             int num_heads, int seq_len, int head_dim, float scale,
                                             bool causal, hipStream_t stream) {
    return backward_impl(Q, K, V, O, L, dO, dQ, dK, dV, batch_size, num_heads, seq_len, head_dim,
                         scale, causal, stream);
}

FlashAttentionError flash_attention_backward(const __hip_bfloat16* Q, const __hip_bfloat16* K,
                                             const __hip_bfloat16* V, const __hip_bfloat16* O,
                                             const float* L, const __hip_bfloat16* dO,
                                             __hip_bfloat16* dQ, __hip_bfloat16* dK,
                                             __hip_bfloat16* dV, int batch_size, int num_heads,
                                             int seq_len, int head_dim, float scale, bool causal,
                                             hipStream_t stream) {
    return backward_impl(Q, K, V, O, L, dO, dQ, dK, dV, batch_size, num_heads, seq_len, head_dim,
                         scale, causal, stream);
}

FlashAttentionError flash_attention_decode(const float* Q, const float* K, const float* V,
                                           float* O, float* L, int batch_size, int num_heads,
                                           int kv_len, int head_dim, float scale, int num_splits,
                                           hipStream_t stream) {
    return decode_impl(Q, K, V, O, L, batch_size, num_heads, kv_len, head_dim, scale, num_splits,
                       stream);
}

FlashAttentionError flash_attention_decode(const __half* Q, const __half* K, const __half* V,
                                           __half* O, float* L, int batch_size, int num_heads,
                                           int kv_len, int head_dim, float scale, int num_splits,
                                           hipStream_t stream) {
    return decode_impl(Q, K, V, O, L, batch_size, num_heads, kv_len, head_dim, scale, num_splits,
                       stream);
}

FlashAttentionError flash_attention_decode(const __hip_bfloat16* Q, const __hip_bfloat16* K,
                                           const __hip_bfloat16* V, __hip_bfloat16* O, float* L,
                                           int batch_size, int num_heads, int kv_len, int head_dim,
                                           float scale, int num_splits, hipStream_t stream) {
    return decode_impl(Q, K, V, O, L, batch_size, num_heads, kv_len, head_dim, scale, num_splits,
                       stream);
}

FlashAttentionError flash_attention_decode_gqa(const float* Q, const float* K, const float* V,
                                               float* O, float* L, int batch_size, int num_heads,
                                               int num_kv_heads, int kv_len, int head_dim,
                                               float scale, int num_splits, hipStream_t stream) {
    return decode_gqa_impl(Q, K, V, O, L, batch_size, num_heads, num_kv_heads, kv_len, head_dim,
                           scale, num_splits, stream);
}

FlashAttentionError flash_attention_decode_paged(const float* Q, const float* K_cache,
                                                 const float* V_cache, float* O, float* L,
                                                 const int* block_table, const int* seq_lens,
                                                 int batch_size, int num_heads, int num_kv_heads,
                                                 int page_size, int max_pages_per_seq,
                                                 int head_dim, float scale, int num_splits,
                                                 hipStream_t stream) {
    return decode_paged_impl(Q, K_cache, V_cache, O, L, block_table, seq_lens, batch_size,
                             num_heads, num_kv_heads, page_size, max_pages_per_seq, head_dim,
                             scale, num_splits, stream);
}

FlashAttentionError flash_attention_decode_gqa(const __half* Q, const __half* K, const __half* V,
                                               __half* O, float* L, int batch_size, int num_heads,
                                               int num_kv_heads, int kv_len, int head_dim,
                                               float scale, int num_splits, hipStream_t stream) {
    return decode_gqa_impl(Q, K, V, O, L, batch_size, num_heads, num_kv_heads, kv_len, head_dim,
                           scale, num_splits, stream);
}

FlashAttentionError flash_attention_decode_paged(const __half* Q, const __half* K_cache,
                                                 const __half* V_cache, __half* O, float* L,
                                                 const int* block_table, const int* seq_lens,
                                                 int batch_size, int num_heads, int num_kv_heads,
                                                 int page_size, int max_pages_per_seq,
                                                 int head_dim, float scale, int num_splits,
                                                 hipStream_t stream) {
    return decode_paged_impl(Q, K_cache, V_cache, O, L, block_table, seq_lens, batch_size,
                             num_heads, num_kv_heads, page_size, max_pages_per_seq, head_dim,
                             scale, num_splits, stream);
}

FlashAttentionError flash_attention_decode_gqa(const __hip_bfloat16* Q, const __hip_bfloat16* K, const __hip_bfloat16* V,
                                               __hip_bfloat16* O, float* L, int batch_size, int num_heads,
                                               int num_kv_heads, int kv_len, int head_dim,
                                               float scale, int num_splits, hipStream_t stream) {
    return decode_gqa_impl(Q, K, V, O, L, batch_size, num_heads, num_kv_heads, kv_len, head_dim,
                           scale, num_splits, stream);
}

FlashAttentionError flash_attention_decode_paged(const __hip_bfloat16* Q, const __hip_bfloat16* K_cache,
                                                 const __hip_bfloat16* V_cache, __hip_bfloat16* O, float* L,
                                                 const int* block_table, const int* seq_lens,
                                                 int batch_size, int num_heads, int num_kv_heads,
                                                 int page_size, int max_pages_per_seq,
                                                 int head_dim, float scale, int num_splits,
                                                 hipStream_t stream) {
    return decode_paged_impl(Q, K_cache, V_cache, O, L, block_table, seq_lens, batch_size,
                             num_heads, num_kv_heads, page_size, max_pages_per_seq, head_dim,
                             scale, num_splits, stream);
}

// ===== Extended forward / backward (no reference counterpart) =====

#define CUFLASH_EXT_OVERLOADS(T)                                                                 \
    FlashAttentionError flash_attention_forward_ext(                                            \
        const T* Q, const T* K, const T* V, T* O, float* L, int batch_size, int num_heads,       \
        int num_kv_heads, int q_len, int kv_len, int head_dim, float scale, bool causal,         \
        hipStream_t stream) {                                                                    \
        return forward_ext_impl(Q, K, V, O, L, batch_size, num_heads, num_kv_heads, q_len,       \
                                kv_len, head_dim, scale, causal, stream);                        \
    }                                                                                            \
    FlashAttentionError flash_attention_backward_ext(                                           \
        const T* Q, const T* K, const T* V, const T* O, const float* L, const T* dO, T* dQ,      \
        T* dK, T* dV, int batch_size, int num_heads, int num_kv_heads, int q_len, int kv_len,    \
        int head_dim, float scale, bool causal, hipStream_t stream) {                            \
        return backward_ext_impl(Q, K, V, O, L, dO, dQ, dK, dV, batch_size, num_heads,           \
                                 num_kv_heads, q_len, kv_len, head_dim, scale, causal, stream);  \
    }
CUFLASH_EXT_OVERLOADS(float)
CUFLASH_EXT_OVERLOADS(__half)
CUFLASH_EXT_OVERLOADS(__hip_bfloat16)
#undef CUFLASH_EXT_OVERLOADS

}  // namespace cuflash

// ===== C ABI (reference src/api/flash_attention_api.cu:186-242) =====

extern "C" {

int cuflash_attention_forward_f32(const float* Q, const float* K, const float* V, float* O,
                                  float* L, int batch_size, int num_heads, int seq_len,
                                  int head_dim, float scale, bool causal, hipStream_t stream) {
    return static_cast<int>(cuflash::flash_attention_forward(
        Q, K, V, O, L, batch_size, num_heads, seq_len, head_dim, scale, causal, stream));
}

int cuflash_attention_backward_f32(const float* Q, const float* K, const float* V, const float* O,
                                   const float* L, const float* dO, float* dQ, float* dK, float* dV,
                                   int batch_size, int num_heads, int seq_len, int head_dim,
                                   float scale, bool causal, hipStream_t stream) {
    return static_cast<int>(cuflash::flash_attention_backward(Q, K, V, O, L, dO, dQ, dK, dV,
                                                              batch_size, num_heads, seq_len,
                                                              head_dim, scale, causal, stream));
}

int cuflash_attention_forward_f16(const __half* Q, const __half* K, const __half* V, __half* O,
                                  float* L, int batch_size, int num_heads, int seq_len,
                                  int head_dim, float scale, bool causal, hipStream_t stream) {
    return static_cast<int>(cuflash::flash_attention_forward(
        Q, K, V, O, L, batch_size, num_heads, seq_len, head_dim, scale, causal, stream));
}

int cuflash_attention_backward_f16(const __half* Q, const __half* K, const __half* V,
                                   const __half* O, const float* L, const __half* dO, __half* dQ,
                                   __half* dK, __half* dV, int batch_size, int num_heads,
                                   int seq_len, int head_dim, float scale, bool causal,
                                   hipStream_t stream) {
    return static_cast<int>(cuflash::flash_attention_backward(Q, K, V, O, L, dO, dQ, dK, dV,
                                                              batch_size, num_heads, seq_len,
                                                              head_dim, scale, causal, stream));
}

int cuflash_attention_forward_bf16(const __hip_bfloat16* Q, const __hip_bfloat16* K,
                                   const __hip_bfloat16* V, __hip_bfloat16* O, float* L,
                                   int batch_size, int num_heads, int seq_len, int head_dim,
                                   float scale, bool causal, hipStream_t stream) {
    return static_cast<int>(cuflash::flash_attention_forward(
        Q, K, V, O, L, batch_size, num_heads, seq_len, head_dim, scale, causal, stream));
}

int cuflash_attention_backward_bf16(const __hip_bfloat16* Q, const __hip_bfloat16* K,
                                    const __hip_bfloat16* V, const __hip_bfloat16* O,
                                    const float* L, const __hip_bfloat16* dO, __hip_bfloat16* dQ,
                                    __hip_bfloat16* dK, __hip_bfloat16* dV, int batch_size,
                                    int num_heads, int seq_len, int head_dim, float scale,
                                    bool causal, hipStream_t stream) {
    return static_cast<int>(cuflash::flash_attention_backward(Q, K, V, O, L, dO, dQ, dK, dV,
                                                              batch_size, num_heads, seq_len,
                                                              head_dim, scale, causal, stream));
}

const char* cuflash_error_string(int error_code) {
    return cuflash::get_error_string(static_cast<cuflash::FlashAttentionError>(error_code));
}

int cuflash_attention_decode_f32(const float* Q, const float* K, const float* V, float* O,
                                 float* L, int batch_size, int num_heads, int kv_len, int head_dim,
                                 float scale, int num_splits, hipStream_t stream) {
    return static_cast<int>(cuflash::flash_attention_decode(
        Q, K, V, O, L, batch_size, num_heads, kv_len, head_dim, scale, num_splits, stream));
}

int cuflash_attention_decode_f16(const __half* Q, const __half* K, const __half* V, __half* O,
                                 float* L, int batch_size, int num_heads, int kv_len, int head_dim,
                                 float scale, int num_splits, hipStream_t stream) {
    return static_cast<int>(cuflash::flash_attention_decode(
        Q, K, V, O, L, batch_size, num_heads, kv_len, head_dim, scale, num_splits, stream));
}

int cuflash_attention_decode_noalloc_f16(const __half* Q, const __half* K, const __half* V,
                                         __half* O, float* L, int batch_size, int num_heads,
                                         int kv_len, int head_dim, float scale, int num_splits,
                                         hipStream_t stream) {
    cuflash::FlashAttentionError err = cuflash::check_decode(Q, K, V, O, L, batch_size, num_heads,
                                                             kv_len, head_dim, scale, num_splits);
    if (err == cuflash::FlashAttentionError::SUCCESS)
        err = cuflash::detail::launch_decode_noalloc<__half>(Q, K, V, O, L, batch_size, num_heads,
                                                             kv_len, head_dim, scale, num_splits,
                                                             stream);
    return static_cast<int>(err);
}

int cuflash_attention_decode_bf16(const __hip_bfloat16* Q, const __hip_bfloat16* K,
                                  const __hip_bfloat16* V, __hip_bfloat16* O, float* L,
                                  int batch_size, int num_heads, int kv_len, int head_dim,
                                  float scale, int num_splits, hipStream_t stream) {
    return static_cast<int>(cuflash::flash_attention_decode(
        Q, K, V, O, L, batch_size, num_heads, kv_len, head_dim, scale, num_splits, stream));
}

int cuflash_attention_decode_gqa_f32(const float* Q, const float* K, const float* V, float* O,
                                     float* L, int batch_size, int num_heads, int num_kv_heads,
                                     int kv_len, int head_dim, float scale, int num_splits,
                                     hipStream_t stream) {
    return static_cast<int>(cuflash::flash_attention_decode_gqa(Q, K, V, O, L, batch_size,
                                                                num_heads, num_kv_heads, kv_len,
                                                                head_dim, scale, num_splits,
                                                                stream));
}

int cuflash_attention_decode_paged_f32(const float* Q, const float* K_cache, const float* V_cache,
                                       float* O, float* L, const int* block_table,
                                       const int* seq_lens, int batch_size, int num_heads,
                                       int num_kv_heads, int page_size, int max_pages_per_seq,
                                       int head_dim, float scale, int num_splits,
                                       hipStream_t stream) {
    return static_cast<int>(cuflash::flash_attention_decode_paged(
        Q, K_cache, V_cache, O, L, block_table, seq_lens, batch_size, num_heads, num_kv_heads,
        page_size, max_pages_per_seq, head_dim, scale, num_splits, stream));
}

int cuflash_attention_decode_gqa_f16(const __half* Q, const __half* K, const __half* V, __half* O,
                                     float* L, int batch_size, int num_heads, int num_kv_heads,
                                     int kv_len, int head_dim, float scale, int num_splits,
                                     hipStream_t stream) {
    return static_cast<int>(cuflash::flash_attention_decode_gqa(Q, K, V, O, L, batch_size,
                                                                num_heads, num_kv_heads, kv_len,
                                                                head_dim, scale, num_splits,
                                                                stream));
}

int cuflash_attention_decode_paged_f16(const __half* Q, const __half* K_cache, const __half* V_cache,
                                       __half* O, float* L, const int* block_table,
                                       const int* seq_lens, int batch_size, int num_heads,
                                       int num_kv_heads, int page_size, int max_pages_per_seq,
                                       int head_dim, float scale, int num_splits,
                                       hipStream_t stream) {
    return static_cast<int>(cuflash::flash_attention_decode_paged(
        Q, K_cache, V_cache, O, L, block_table, seq_lens, batch_size, num_heads, num_kv_heads,
        page_size, max_pages_per_seq, head_dim, scale, num_splits, stream));
}

int cuflash_attention_decode_gqa_bf16(const __hip_bfloat16* Q, const __hip_bfloat16* K, const __hip_bfloat16* V, __hip_bfloat16* O,
                                     float* L, int batch_size, int num_heads, int num_kv_heads,
                                     int kv_len, int head_dim, float scale, int num_splits,
                                     hipStream_t stream) {
    return static_cast<int>(cuflash::flash_attention_decode_gqa(Q, K, V, O, L, batch_size,
                                                                num_heads, num_kv_heads, kv_len,
                                                                head_dim, scale, num_splits,
                                                                stream));
}

int cuflash_attention_decode_paged_bf16(const __hip_bfloat16* Q, const __hip_bfloat16* K_cache, const __hip_bfloat16* V_cache,
                                       __hip_bfloat16* O, float* L, const int* block_table,
                                       const int* seq_lens, int batch_size, int num_heads,
                                       int num_kv_heads, int page_size, int max_pages_per_seq,
                                       int head_dim, float scale, int num_splits,
                                       hipStream_t stream) {
    return static_cast<int>(cuflash::flash_attention_decode_paged(
        Q, K_cache, V_cache, O, L, block_table, seq_lens, batch_size, num_heads, num_kv_heads,
        page_size, max_pages_per_seq, head_dim, scale, num_splits, stream));
}

#define CUFLASH_EXT_C_ABI(SFX, T)                                                                \
    int cuflash_attention_forward_ext_##SFX(const T* Q, const T* K, const T* V, T* O, float* L,  \
                                            int batch_size, int num_heads, int num_kv_heads,     \
                                            int q_len, int kv_len, int head_dim, float scale,    \
                                            bool causal, hipStream_t stream) {                   \
        return static_cast<int>(cuflash::flash_attention_forward_ext(                            \
            Q, K, V, O, L, batch_size, num_heads, num_kv_heads, q_len, kv_len, head_dim, scale,  \
            causal, stream));                                                                    \
    }                                                                                            \
    int cuflash_attention_backward_ext_##SFX(                                                    \
        const T* Q, const T* K, const T* V, const T* O, const float* L, const T* dO, T* dQ,      \
        T* dK, T* dV, int batch_size, int num_heads, int num_kv_heads, int q_len, int kv_len,    \
        int head_dim, float scale, bool causal, hipStream_t stream) {                            \
        return static_cast<int>(cuflash::flash_attention_backward_ext(                           \
            Q, K, V, O, L, dO, dQ, dK, dV, batch_size, num_heads, num_kv_heads, q_len, kv_len,   \
            head_dim, scale, causal, stream));                                                   \
    }
CUFLASH_EXT_C_ABI(f32, float)
CUFLASH_EXT_C_ABI(f16, __half)
CUFLASH_EXT_C_ABI(bf16, __hip_bfloat16)
#undef CUFLASH_EXT_C_ABI

const char* cuflash_version(void) { return CUFLASH_VERSION; }

}  // extern "C"
