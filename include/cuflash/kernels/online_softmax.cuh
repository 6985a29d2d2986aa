#pragma once

// Public online-softmax primitives of libcuflash_attn (namespace cuflash::kernels).
// Same declarations as the reference's include/cuflash/kernels/online_softmax.cuh:8-112, with
// the HIP stream type. The state of a row is (m, l): the running maximum and the running sum
// of exp(x - m). Null pointers return NULL_POINTER, a dimension <= 0 returns
// INVALID_DIMENSION, a launch failure returns CUDA_ERROR.

#include <hip/hip_runtime.h>

#include "cuflash/export.h"
#include "cuflash/flash_attention.h"  // FlashAttentionError

namespace cuflash {
namespace kernels {

/// state_m[r] = -inf, state_l[r] = 0 for r < rows (reference online_softmax.cuh:37-38).
CUFLASH_EXPORT FlashAttentionError online_softmax_init(float* state_m, float* state_l, int rows,
                                                       hipStream_t stream = 0);

/// Merges a block's (block_max, block_sum = sum of exp(x - block_max)) into each row's state:
/// m' = max(m, block_max), l' = l exp(m - m') + block_sum exp(block_max - m')
/// (reference online_softmax.cuh:50-54).
CUFLASH_EXPORT FlashAttentionError online_softmax_update(const float* block_max,
                                                         const float* block_sum, float* state_m,
                                                         float* state_l, int rows,
                                                         hipStream_t stream = 0);

/// logsumexp[r] = m + log(l), normalizer[r] = 1 / l (reference online_softmax.cuh:65-68).
CUFLASH_EXPORT FlashAttentionError online_softmax_finalize(const float* state_m,
                                                           const float* state_l,
                                                           float* logsumexp, float* normalizer,
                                                           int rows, hipStream_t stream = 0);

/// Row-wise softmax of input [rows, cols] into output, with logsumexp [rows]; the row is
/// streamed in blocks of block_size columns through the online state
/// (reference online_softmax.cuh:84-86).
CUFLASH_EXPORT FlashAttentionError online_softmax_forward(const float* input, float* output,
                                                          float* logsumexp, int rows, int cols,
                                                          int block_size, hipStream_t stream = 0);

/// Maximum of val over the calling wavefront (64 lanes on gfx950); every lane gets the result.
/// All lanes of the wavefront must call it (reference online_softmax.cuh:94-100, 32 lanes).
__device__ __forceinline__ float warp_reduce_max(float val) {
#pragma unroll
    for (int offset = 32; offset > 0; offset /= 2) val = fmaxf(val, __shfl_xor(val, offset, 64));
    return val;
}

/// Sum of val over the calling wavefront (64 lanes); every lane gets the result
/// (reference online_softmax.cuh:102-109).
__device__ __forceinline__ float warp_reduce_sum(float val) {
#pragma unroll
    for (int offset = 32; offset > 0; offset /= 2) val += __shfl_xor(val, offset, 64);
    return val;
}

}  // namespace kernels
}  // namespace cuflash
