#pragma once

// Public tile copy primitives of libcuflash_attn (namespace cuflash::kernels).
// Same declarations as the reference's include/cuflash/kernels/tile_io.cuh:8-93, with the HIP
// stream and half types. A tile is the window [row_start, row_start + BLOCK_ROWS) x
// [col_start, col_start + BLOCK_COLS) of a row-major [max_rows, max_cols] tensor with the given
// row stride (elements); the buffer side is a dense [BLOCK_ROWS, BLOCK_COLS] fp32 array in
// device memory. Elements of the window outside the tensor read as 0 on load and are not
// written on store. fp16 is converted to fp32 exactly on load and rounded to nearest even on
// store.
//
// Instantiated for (BLOCK_ROWS, BLOCK_COLS) in {(64,64), (64,32), (32,32), (32,64), (32,128),
// (64,128)}; load_store_tile_roundtrip for (64,64) (reference src/kernels/tile_io.cu:229-287).
// Null pointers return NULL_POINTER; max_rows, max_cols or the stride <= 0, or a start outside
// the tensor, return INVALID_DIMENSION (reference primitive_api_utils.cuh:30-43).

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "cuflash/export.h"
#include "cuflash/flash_attention.h"  // FlashAttentionError

namespace cuflash {
namespace kernels {

/// dst = the fp32 tile of src (reference tile_io.cuh:43-46).
template <int BLOCK_ROWS, int BLOCK_COLS>
CUFLASH_EXPORT FlashAttentionError load_tile(const float* src, float* dst, int row_start,
                                             int col_start, int max_rows, int max_cols,
                                             int src_stride, hipStream_t stream = 0);

/// dst = the fp16 tile of src converted to fp32 (reference tile_io.cuh:50-53).
template <int BLOCK_ROWS, int BLOCK_COLS>
CUFLASH_EXPORT FlashAttentionError load_tile(const __half* src, float* dst, int row_start,
                                             int col_start, int max_rows, int max_cols,
                                             int src_stride, hipStream_t stream = 0);

/// Writes the fp32 tile buffer src into the window of dst (reference tile_io.cuh:70-73).
template <int BLOCK_ROWS, int BLOCK_COLS>
CUFLASH_EXPORT FlashAttentionError store_tile(const float* src, float* dst, int row_start,
                                              int col_start, int max_rows, int max_cols,
                                              int dst_stride, hipStream_t stream = 0);

/// Writes the fp32 tile buffer src into the window of the fp16 tensor dst
/// (reference tile_io.cuh:77-80).
template <int BLOCK_ROWS, int BLOCK_COLS>
CUFLASH_EXPORT FlashAttentionError store_tile(const float* src, __half* dst, int row_start,
                                              int col_start, int max_rows, int max_cols,
                                              int dst_stride, hipStream_t stream = 0);

/// Loads the window of src and stores it into the same window of dst (both with `stride`):
/// the in-tensor part of the window is copied (reference tile_io.cuh:88-91).
template <int BLOCK_ROWS, int BLOCK_COLS>
CUFLASH_EXPORT FlashAttentionError load_store_tile_roundtrip(const float* src, float* dst,
                                                             int row_start, int col_start,
                                                             int max_rows, int max_cols,
                                                             int stride, hipStream_t stream = 0);

}  // namespace kernels
}  // namespace cuflash
