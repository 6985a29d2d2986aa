#pragma once

// Public tile-level matrix products of libcuflash_attn (namespace cuflash::kernels).
// Same declarations as the reference's include/cuflash/kernels/matmul.cuh:8-71, with the HIP
// stream type. Each call runs one workgroup on the caller's stream over small fp32 matrices in
// device memory; the library computes them on gfx950's fp32 matrix cores
// (v_mfma_f32_32x32x2f32, one wave per 32 x 32 block of C).
//
// Instantiated for (M, N, K) in {(64,64,32), (32,32,32), (64,64,64), (32,32,128), (64,64,128),
// (32,64,32), (32,64,64), (64,32,64)}, the set the reference library exports
// (src/kernels/matmul.cu:236-319). Null A, B or C returns NULL_POINTER; a launch failure returns
// CUDA_ERROR.

#include <hip/hip_runtime.h>

#include "cuflash/export.h"
#include "cuflash/flash_attention.h"  // FlashAttentionError

namespace cuflash {
namespace kernels {

/// C = scale * A B^T, A [M, K] and B [N, K] row-major, C [M, N] (reference matmul.cuh:35-36).
template <int M, int N, int K>
CUFLASH_EXPORT FlashAttentionError matmul_ABt(const float* A, const float* B, float* C,
                                              float scale, hipStream_t stream = 0);

/// C = scale * A B, A [M, K] and B [K, N] (reference matmul.cuh:45-46).
template <int M, int N, int K>
CUFLASH_EXPORT FlashAttentionError matmul_AB(const float* A, const float* B, float* C,
                                             float scale, hipStream_t stream = 0);

/// C += scale * A B, A [M, K] and B [K, N] (reference matmul.cuh:55-56).
template <int M, int N, int K>
CUFLASH_EXPORT FlashAttentionError matmul_AB_acc(const float* A, const float* B, float* C,
                                                 float scale, hipStream_t stream = 0);

/// C = scale * A^T B, A [K, M] and B [K, N] (reference matmul.cuh:65-66).
template <int M, int N, int K>
CUFLASH_EXPORT FlashAttentionError matmul_AtB(const float* A, const float* B, float* C,
                                              float scale, hipStream_t stream = 0);

}  // namespace kernels
}  // namespace cuflash
