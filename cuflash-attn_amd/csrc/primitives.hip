// Public primitive layer cuflash::kernels::* (matmul, online softmax, tile I/O).
//
// The reference library exports these single-block primitives from src/kernels/matmul.cu,
// online_softmax.cu and tile_io.cu (declarations in include/cuflash/kernels/*.cuh), pinned by
// its tests/unit/test_{matmul,online_softmax,tile_io}.cu. They are small test and building-
// block operations, not part of the flash kernels; this file restates their contracts for
// gfx950:
//   * matmul_*: one workgroup, one wave per 32 x 32 block of C, products on the fp32 matrix
//     cores (v_mfma_f32_32x32x2f32, two k per instruction, fp32 accumulation) with the operands
//     read straight from global memory (the tiles are at most 64 x 128 floats);
//   * online_softmax_*: elementwise state kernels with the reference's update rule
//     (impl/online_softmax.cuh:28-39), and a row softmax with one wave per row whose block
//     statistics merge through that rule;
//   * load_tile / store_tile: one workgroup copying the window with zero fill on load and
//     skipped writes on store (impl/tile_io.cuh:30-495), fp16 <-> fp32 with RNE on store.
// Validation order and error codes follow src/kernels/primitive_api_utils.cuh:12-58.

#include "cuflash/kernels/matmul.cuh"
#include "cuflash/kernels/online_softmax.cuh"
#include "cuflash/kernels/tile_io.cuh"

#include <initializer_list>

#include "common.hpp"

namespace cuflash {
namespace kernels {
namespace {

FlashAttentionError check_non_null(std::initializer_list<const void*> ptrs) {
    for (const void* p : ptrs)
        if (p == nullptr) return FlashAttentionError::NULL_POINTER;
    return FlashAttentionError::SUCCESS;
}

FlashAttentionError check_positive(std::initializer_list<int> dims) {
    for (int d : dims)
        if (d <= 0) return FlashAttentionError::INVALID_DIMENSION;
    return FlashAttentionError::SUCCESS;
}

// The window must start inside a tensor with positive extents and stride
// (reference primitive_api_utils.cuh:30-43).
FlashAttentionError check_window(int row_start, int col_start, int max_rows, int max_cols,
                                 int stride) {
    const FlashAttentionError e = check_positive({max_rows, max_cols, stride});
    if (e != FlashAttentionError::SUCCESS) return e;
    if (row_start < 0 || col_start < 0 || row_start >= max_rows || col_start >= max_cols)
        return FlashAttentionError::INVALID_DIMENSION;
    return FlashAttentionError::SUCCESS;
}

// Any launch error maps to CUDA_ERROR, as in the reference (primitive_api_utils.cuh:52-55).
FlashAttentionError launch_status() {
    return hipGetLastError() == hipSuccess ? FlashAttentionError::SUCCESS
                                           : FlashAttentionError::CUDA_ERROR;
}

}  // namespace

// ------------------------------------------------------------------------------------------
// Matrix products
// ------------------------------------------------------------------------------------------
namespace dev {

// How the operands of C[m][n] = scale * sum_k a(m, k) b(k, n) are stored.
enum MmMode { kABt = 0, kAB = 1, kAtB = 2 };

// Wave w computes the 32 x 32 block (w / (N / 32), w % (N / 32)) of C. In each MFMA lane l
// supplies a(m0 + l % 32, k0 + l / 32) and b(k0 + l / 32, n0 + l % 32) and receives rows
// 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32 of the block in accumulator register r.
template <int M, int N, int K, int MODE, bool ACC>
__global__ void __launch_bounds__(256)
    tile_matmul_kernel(const float* __restrict__ A, const float* __restrict__ B,
                       float* __restrict__ C, float scale) {
    static_assert(M % 32 == 0 && N % 32 == 0 && K % 2 == 0, "tile shape");
    constexpr int TN = N / 32;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int m0 = (wave / TN) * 32;
    const int n0 = (wave % TN) * 32;
    const int i = lane & 31;
    const int h = lane >> 5;

    cuflash::dev::f32x16 acc = {};
#pragma unroll 8
    for (int k0 = 0; k0 < K; k0 += 2) {
        const int k = k0 + h;
        const float a = (MODE == kAtB) ? A[k * M + m0 + i] : A[(m0 + i) * K + k];
        const float b = (MODE == kABt) ? B[(n0 + i) * K + k] : B[k * N + n0 + i];
        acc = cuflash::dev::mma_f32(a, b, acc);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = m0 + 8 * (r >> 2) + 4 * h + (r & 3);
        float* c = C + row * N + n0 + i;
        const float v = acc[r] * scale;
        *c = ACC ? *c + v : v;
    }
}

template <int M, int N, int K, int MODE, bool ACC>
FlashAttentionError run_matmul(const float* A, const float* B, float* C, float scale,
                               hipStream_t stream) {
    const FlashAttentionError e = check_non_null({A, B, C});
    if (e != FlashAttentionError::SUCCESS) return e;
    hipLaunchKernelGGL((tile_matmul_kernel<M, N, K, MODE, ACC>), dim3(1),
                       dim3(64 * (M / 32) * (N / 32)), 0, stream, A, B, C, scale);
    return launch_status();
}

}  // namespace dev

template <int M, int N, int K>
FlashAttentionError matmul_ABt(const float* A, const float* B, float* C, float scale,
                               hipStream_t stream) {
    return dev::run_matmul<M, N, K, dev::kABt, false>(A, B, C, scale, stream);
}

template <int M, int N, int K>
FlashAttentionError matmul_AB(const float* A, const float* B, float* C, float scale,
                              hipStream_t stream) {
    return dev::run_matmul<M, N, K, dev::kAB, false>(A, B, C, scale, stream);
}

template <int M, int N, int K>
FlashAttentionError matmul_AB_acc(const float* A, const float* B, float* C, float scale,
                                  hipStream_t stream) {
    return dev::run_matmul<M, N, K, dev::kAB, true>(A, B, C, scale, stream);
}

template <int M, int N, int K>
FlashAttentionError matmul_AtB(const float* A, const float* B, float* C, float scale,
                               hipStream_t stream) {
    return dev::run_matmul<M, N, K, dev::kAtB, false>(A, B, C, scale, stream);
}

#define CUFLASH_MATMUL_SHAPE(M, N, K)                                                            \
    template CUFLASH_EXPORT FlashAttentionError matmul_ABt<M, N, K>(const float*, const float*,  \
                                                                    float*, float, hipStream_t); \
    template CUFLASH_EXPORT FlashAttentionError matmul_AB<M, N, K>(const float*, const float*,   \
                                                                   float*, float, hipStream_t);  \
    template CUFLASH_EXPORT FlashAttentionError matmul_AB_acc<M, N, K>(                          \
        const float*, const float*, float*, float, hipStream_t);                                 \
    template CUFLASH_EXPORT FlashAttentionError matmul_AtB<M, N, K>(const float*, const float*,  \
                                                                    float*, float, hipStream_t);
// The shapes the reference exports (src/kernels/matmul.cu:236-319).
CUFLASH_MATMUL_SHAPE(64, 64, 32)
CUFLASH_MATMUL_SHAPE(32, 32, 32)
CUFLASH_MATMUL_SHAPE(64, 64, 64)
CUFLASH_MATMUL_SHAPE(32, 32, 128)
CUFLASH_MATMUL_SHAPE(64, 64, 128)
CUFLASH_MATMUL_SHAPE(32, 64, 32)
CUFLASH_MATMUL_SHAPE(32, 64, 64)
CUFLASH_MATMUL_SHAPE(64, 32, 64)
#undef CUFLASH_MATMUL_SHAPE

// ------------------------------------------------------------------------------------------
// Online softmax
// ------------------------------------------------------------------------------------------
namespace dev {

// The reference's merge of a block (bm, bs) into (m, l) (impl/online_softmax.cuh:28-33),
// written the same way so that degenerate inputs behave the same.
__device__ __forceinline__ void softmax_merge(float& m, float& l, float bm, float bs) {
    const float m_max = fmaxf(m, bm);
    l = l * expf(m - m_max) + bs * expf(bm - m_max);
    m = m_max;
}

__global__ void softmax_init_kernel(float* __restrict__ m, float* __restrict__ l, int rows) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r < rows) {
        m[r] = -INFINITY;
        l[r] = 0.0f;
    }
}

__global__ void softmax_update_kernel(const float* __restrict__ bmax, const float* __restrict__ bsum,
                                      float* __restrict__ m, float* __restrict__ l, int rows) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r < rows) {
        float mr = m[r], lr = l[r];
        softmax_merge(mr, lr, bmax[r], bsum[r]);
        m[r] = mr;
        l[r] = lr;
    }
}

__global__ void softmax_finalize_kernel(const float* __restrict__ m, const float* __restrict__ l,
                                        float* __restrict__ lse, float* __restrict__ norm,
                                        int rows) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r < rows) {
        lse[r] = m[r] + logf(l[r]);
        norm[r] = 1.0f / l[r];
    }
}

// One wave per row, four rows per workgroup. Pass 1 streams the row in blocks of BLOCK
// columns, each block's (max, sum of exp(x - max)) merged into the row state; pass 2 writes
// exp(x - block max) * exp(block max - m) / l per block, the reference's output formula
// (online_softmax.cu:137-152).
template <int BLOCK>
__global__ void __launch_bounds__(256)
    softmax_rows_kernel(const float* __restrict__ in, float* __restrict__ out,
                        float* __restrict__ lse, int rows, int cols) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;  // wave-uniform
    const int lane = threadIdx.x & 63;
    const float* x = in + static_cast<size_t>(row) * cols;
    float* y = out + static_cast<size_t>(row) * cols;

    auto block_max = [&](int start, int end) {
        float v = -INFINITY;
        for (int c = start + lane; c < end; c += 64) v = fmaxf(v, x[c]);
        return warp_reduce_max(v);
    };
    float m = -INFINITY, l = 0.0f;
    for (int start = 0; start < cols; start += BLOCK) {
        const int end = min(start + BLOCK, cols);
        const float bm = block_max(start, end);
        float s = 0.0f;
        for (int c = start + lane; c < end; c += 64) s += expf(x[c] - bm);
        softmax_merge(m, l, bm, warp_reduce_sum(s));
    }
    const float l_inv = 1.0f / l;
    for (int start = 0; start < cols; start += BLOCK) {
        const int end = min(start + BLOCK, cols);
        const float bm = block_max(start, end);
        const float rescale = expf(bm - m);
        for (int c = start + lane; c < end; c += 64) y[c] = expf(x[c] - bm) * rescale * l_inv;
    }
    if (lane == 0) lse[row] = m + logf(l);
}

}  // namespace dev

FlashAttentionError online_softmax_init(float* state_m, float* state_l, int rows,
                                        hipStream_t stream) {
    FlashAttentionError e = check_non_null({state_m, state_l});
    if (e != FlashAttentionError::SUCCESS) return e;
    e = check_positive({rows});
    if (e != FlashAttentionError::SUCCESS) return e;
    hipLaunchKernelGGL(dev::softmax_init_kernel, dim3((rows + 255) / 256), dim3(256), 0, stream,
                       state_m, state_l, rows);
    return launch_status();
}

FlashAttentionError online_softmax_update(const float* block_max, const float* block_sum,
                                          float* state_m, float* state_l, int rows,
                                          hipStream_t stream) {
    FlashAttentionError e = check_non_null({block_max, block_sum, state_m, state_l});
    if (e != FlashAttentionError::SUCCESS) return e;
    e = check_positive({rows});
    if (e != FlashAttentionError::SUCCESS) return e;
    hipLaunchKernelGGL(dev::softmax_update_kernel, dim3((rows + 255) / 256), dim3(256), 0,
                       stream, block_max, block_sum, state_m, state_l, rows);
    return launch_status();
}

FlashAttentionError online_softmax_finalize(const float* state_m, const float* state_l,
                                            float* logsumexp, float* normalizer, int rows,
                                            hipStream_t stream) {
    FlashAttentionError e = check_non_null({state_m, state_l, logsumexp, normalizer});
    if (e != FlashAttentionError::SUCCESS) return e;
    e = check_positive({rows});
    if (e != FlashAttentionError::SUCCESS) return e;
    hipLaunchKernelGGL(dev::softmax_finalize_kernel, dim3((rows + 255) / 256), dim3(256), 0,
                       stream, state_m, state_l, logsumexp, normalizer, rows);
    return launch_status();
}

FlashAttentionError online_softmax_forward(const float* input, float* output, float* logsumexp,
                                           int rows, int cols, int block_size,
                                           hipStream_t stream) {
    FlashAttentionError e = check_non_null({input, output, logsumexp});
    if (e != FlashAttentionError::SUCCESS) return e;
    e = check_positive({rows, cols, block_size});
    if (e != FlashAttentionError::SUCCESS) return e;
    // The block size selects 32, 64 or 128 columns per block (online_softmax.cu:222-232).
    const dim3 grid((rows + 3) / 4);
    if (block_size <= 32)
        hipLaunchKernelGGL(dev::softmax_rows_kernel<32>, grid, dim3(256), 0, stream, input,
                           output, logsumexp, rows, cols);
    else if (block_size <= 64)
        hipLaunchKernelGGL(dev::softmax_rows_kernel<64>, grid, dim3(256), 0, stream, input,
                           output, logsumexp, rows, cols);
    else
        hipLaunchKernelGGL(dev::softmax_rows_kernel<128>, grid, dim3(256), 0, stream, input,
                           output, logsumexp, rows, cols);
    return launch_status();
}

// ------------------------------------------------------------------------------------------
// Tile I/O
// ------------------------------------------------------------------------------------------
namespace dev {

__device__ __forceinline__ float to_float(float v) { return v; }
__device__ __forceinline__ float to_float(__half v) { return __half2float(v); }
__device__ __forceinline__ void from_float(float v, float* dst) { *dst = v; }
__device__ __forceinline__ void from_float(float v, __half* dst) { *dst = __float2half_rn(v); }

// Tensor window -> dense fp32 tile, zero outside the tensor.
template <int BR, int BC, typename S>
__global__ void __launch_bounds__(256)
    tile_load_kernel(const S* __restrict__ src, float* __restrict__ dst, int row_start,
                     int col_start, int max_rows, int max_cols, int stride) {
    for (int e = threadIdx.x; e < BR * BC; e += blockDim.x) {
        const int gr = row_start + e / BC;
        const int gc = col_start + e % BC;
        dst[e] = (gr < max_rows && gc < max_cols)
                     ? to_float(src[static_cast<size_t>(gr) * stride + gc])
                     : 0.0f;
    }
}

// Dense fp32 tile -> tensor window, elements outside the tensor skipped.
template <int BR, int BC, typename D>
__global__ void __launch_bounds__(256)
    tile_store_kernel(const float* __restrict__ src, D* __restrict__ dst, int row_start,
                      int col_start, int max_rows, int max_cols, int stride) {
    for (int e = threadIdx.x; e < BR * BC; e += blockDim.x) {
        const int gr = row_start + e / BC;
        const int gc = col_start + e % BC;
        if (gr < max_rows && gc < max_cols)
            from_float(src[e], dst + static_cast<size_t>(gr) * stride + gc);
    }
}

// Load into LDS, then store back to the same window of dst.
template <int BR, int BC>
__global__ void __launch_bounds__(256)
    tile_roundtrip_kernel(const float* __restrict__ src, float* __restrict__ dst, int row_start,
                          int col_start, int max_rows, int max_cols, int stride) {
    __shared__ float tile[BR * BC];
    for (int e = threadIdx.x; e < BR * BC; e += blockDim.x) {
        const int gr = row_start + e / BC;
        const int gc = col_start + e % BC;
        tile[e] = (gr < max_rows && gc < max_cols) ? src[static_cast<size_t>(gr) * stride + gc]
                                                   : 0.0f;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < BR * BC; e += blockDim.x) {
        const int gr = row_start + e / BC;
        const int gc = col_start + e % BC;
        if (gr < max_rows && gc < max_cols) dst[static_cast<size_t>(gr) * stride + gc] = tile[e];
    }
}

}  // namespace dev

template <int BR, int BC>
FlashAttentionError load_tile(const float* src, float* dst, int row_start, int col_start,
                              int max_rows, int max_cols, int src_stride, hipStream_t stream) {
    FlashAttentionError e = check_non_null({src, dst});
    if (e != FlashAttentionError::SUCCESS) return e;
    e = check_window(row_start, col_start, max_rows, max_cols, src_stride);
    if (e != FlashAttentionError::SUCCESS) return e;
    hipLaunchKernelGGL((dev::tile_load_kernel<BR, BC, float>), dim3(1), dim3(256), 0, stream,
                       src, dst, row_start, col_start, max_rows, max_cols, src_stride);
    return launch_status();
}

template <int BR, int BC>
FlashAttentionError load_tile(const __half* src, float* dst, int row_start, int col_start,
                              int max_rows, int max_cols, int src_stride, hipStream_t stream) {
    FlashAttentionError e = check_non_null({src, dst});
    if (e != FlashAttentionError::SUCCESS) return e;
    e = check_window(row_start, col_start, max_rows, max_cols, src_stride);
    if (e != FlashAttentionError::SUCCESS) return e;
    hipLaunchKernelGGL((dev::tile_load_kernel<BR, BC, __half>), dim3(1), dim3(256), 0, stream,
                       src, dst, row_start, col_start, max_rows, max_cols, src_stride);
    return launch_status();
}

template <int BR, int BC>
FlashAttentionError store_tile(const float* src, float* dst, int row_start, int col_start,
                               int max_rows, int max_cols, int dst_stride, hipStream_t stream) {
    FlashAttentionError e = check_non_null({src, dst});
    if (e != FlashAttentionError::SUCCESS) return e;
    e = check_window(row_start, col_start, max_rows, max_cols, dst_stride);
    if (e != FlashAttentionError::SUCCESS) return e;
    hipLaunchKernelGGL((dev::tile_store_kernel<BR, BC, float>), dim3(1), dim3(256), 0, stream,
                       src, dst, row_start, col_start, max_rows, max_cols, dst_stride);
    return launch_status();
}

template <int BR, int BC>
FlashAttentionError store_tile(const float* src, __half* dst, int row_start, int col_start,
                               int max_rows, int max_cols, int dst_stride, hipStream_t stream) {
    FlashAttentionError e = check_non_null({src, dst});
    if (e != FlashAttentionError::SUCCESS) return e;
    e = check_window(row_start, col_start, max_rows, max_cols, dst_stride);
    if (e != FlashAttentionError::SUCCESS) return e;
    hipLaunchKernelGGL((dev::tile_store_kernel<BR, BC, __half>), dim3(1), dim3(256), 0, stream,
                       src, dst, row_start, col_start, max_rows, max_cols, dst_stride);
    return launch_status();
}

template <int BR, int BC>
FlashAttentionError load_store_tile_roundtrip(const float* src, float* dst, int row_start,
                                              int col_start, int max_rows, int max_cols,
                                              int stride, hipStream_t stream) {
    FlashAttentionError e = check_non_null({src, dst});
    if (e != FlashAttentionError::SUCCESS) return e;
    e = check_window(row_start, col_start, max_rows, max_cols, stride);
    if (e != FlashAttentionError::SUCCESS) return e;
    hipLaunchKernelGGL((dev::tile_roundtrip_kernel<BR, BC>), dim3(1), dim3(256), 0, stream, src,
                       dst, row_start, col_start, max_rows, max_cols, stride);
    return launch_status();
}

#define CUFLASH_TILE_SHAPE(BR, BC)                                                              \
    template CUFLASH_EXPORT FlashAttentionError load_tile<BR, BC>(                             \
        const float*, float*, int, int, int, int, int, hipStream_t);                           \
    template CUFLASH_EXPORT FlashAttentionError load_tile<BR, BC>(                             \
        const __half*, float*, int, int, int, int, int, hipStream_t);                          \
    template CUFLASH_EXPORT FlashAttentionError store_tile<BR, BC>(                            \
        const float*, float*, int, int, int, int, int, hipStream_t);                           \
    template CUFLASH_EXPORT FlashAttentionError store_tile<BR, BC>(                            \
        const float*, __half*, int, int, int, int, int, hipStream_t);
// The shapes the reference exports (src/kernels/tile_io.cu:229-287).
CUFLASH_TILE_SHAPE(64, 64)
CUFLASH_TILE_SHAPE(64, 32)
CUFLASH_TILE_SHAPE(32, 32)
CUFLASH_TILE_SHAPE(32, 64)
CUFLASH_TILE_SHAPE(32, 128)
CUFLASH_TILE_SHAPE(64, 128)
#undef CUFLASH_TILE_SHAPE
template CUFLASH_EXPORT FlashAttentionError load_store_tile_roundtrip<64, 64>(
    const float*, float*, int, int, int, int, int, hipStream_t);

}  // namespace kernels
}  // namespace cuflash
