#pragma once

// LDS tile layouts of the LDS-DMA kernels: the forward kernels' layouts, used by the backward's
// work items and by the matrix-core decode.

#include "common.hpp"

namespace cuflash {
namespace dev {

// LDS layout of a 16-bit tile with D-element rows, as in the forward kernels: rows in groups
// filled by 1 KB load instructions (lane i writes the 16-byte slot i of its kilobyte).
//   D = 128 (fwd16_d128_kernel): 4-row groups of 1088 bytes, chunk c of row r at 16 (4 c + r).
//   D = 64 (fwd16_d64_kernel): 8-row groups of 1152 bytes, chunk c of row r at
//            16 (8 c + (r ^ 4 ((c >> 1) & 1))).
//   D = 256 (fwd16_d256_kernel): 4-row groups of 2112 bytes, two 1 KB column halves laid out
//            as the D = 128 groups.
// Both serve conflict-free row reads (A operands of 32 rows x 16 k) and transpose reads
// (A operands whose k runs down 16 rows) with per-lane offsets and immediates.
template <int D>
struct TileGroups;
template <>
struct TileGroups<128> {
    static constexpr int kRows = 4;        // rows per group
    static constexpr int kBytes = 1088;    // bytes per group
    static constexpr int kHalves = 1;      // 1 KB load instructions per group
    static constexpr int kTrRows16 = 4 * kBytes;  // transpose reads: 16 rows further
    static constexpr int kTrHigh = 2 * kBytes;    // second read of a transpose operand (+8 rows)
    static constexpr int k_off(int ks) { return ks * 128; }     // row reads: k-step ks
    static constexpr int dtile_off(int dt) { return dt * 256; }  // transpose reads: 32 columns
    __device__ static int ld_row(int lane) { return lane & 3; }
    __device__ static int ld_col(int lane) { return (lane >> 2) * 8; }
    // Row reads, k-step ks: this lane's 16 bytes (row lane % 32, chunk 2 ks + lane / 32) sit at
    // row_base(lane, ks & 1) + k_off(ks).
    __device__ static int row_base(int lane, int) {
        return ((lane & 31) >> 2) * kBytes + (lane >> 5) * 64 + (lane & 3) * 16;
    }
    // Transpose reads (see tr_frag_at): lane provides the 8-byte chunk of row 4 (lane / 32) +
    // (lane % 16) / 4, columns 16 ((lane / 16) % 2) + 4 (lane % 4).
    __device__ static int tr_off(int lane) {
        const int kq = lane & 15;
        return (lane >> 5) * kBytes + (2 * ((lane >> 4) & 1) + ((kq & 3) >> 1)) * 64 +
               (kq >> 2) * 16 + (kq & 1) * 8;
    }
};
template <>
struct TileGroups<256> : TileGroups<128> {
    static constexpr int kBytes = 2 * 1024 + 64;
    static constexpr int kHalves = 2;
    static constexpr int kTrRows16 = 4 * kBytes;
    static constexpr int kTrHigh = 2 * kBytes;
    static constexpr int k_off(int ks) { return (ks >> 3) * 1024 + (ks & 7) * 128; }
    static constexpr int dtile_off(int dt) { return (dt >> 2) * 1024 + (dt & 3) * 256; }
    __device__ static int row_base(int lane, int) {
        return ((lane & 31) >> 2) * kBytes + (lane >> 5) * 64 + (lane & 3) * 16;
    }
    __device__ static int tr_off(int lane) {
        const int kq = lane & 15;
        return (lane >> 5) * kBytes + (2 * ((lane >> 4) & 1) + ((kq & 3) >> 1)) * 64 +
               (kq >> 2) * 16 + (kq & 1) * 8;
    }
};
template <>
struct TileGroups<64> {
    static constexpr int kRows = 8;
    static constexpr int kBytes = 1152;
    static constexpr int kHalves = 1;
    static constexpr int kTrRows16 = 2 * kBytes;
    static constexpr int kTrHigh = kBytes;
    static constexpr int k_off(int ks) { return ks * 256; }
    static constexpr int dtile_off(int dt) { return dt * 512; }
    __device__ static int ld_row(int lane) { return (lane & 7) ^ (4 * ((lane >> 4) & 1)); }
    __device__ static int ld_col(int lane) { return (lane >> 3) * 8; }
    __device__ static int row_base(int lane, int odd) {
        return ((lane & 31) >> 3) * kBytes + (lane >> 5) * 128 + ((lane & 7) ^ (4 * odd)) * 16;
    }
    __device__ static int tr_off(int lane) {
        const int kq = lane & 15;
        const int gl = (lane >> 4) & 1;
        return (2 * gl + ((kq & 3) >> 1)) * 128 + ((lane >> 5) ^ gl) * 64 + (kq >> 2) * 16 +
               (kq & 1) * 8;
    }
};
// head_dim 32: the head_dim-64 layout with each 64-byte row in the first half of its 128-byte
// slot (operand reads touch chunks 0-3 only); lanes 32-63 of a load read the row's four
// chunks again into the unused slots 4-7.
template <>
struct TileGroups<32> : TileGroups<64> {
    __device__ static int ld_col(int lane) { return ((lane >> 3) & 3) * 8; }
};
// head_dim 96: the head_dim-128 layout with each 192-byte row in the first 12 chunks of its
// 256-byte slot (operand reads touch chunks 0-11 only); lanes 48-63 of a load read chunks 0-3
// again into the unused slots 12-15.
template <>
struct TileGroups<96> : TileGroups<128> {
    __device__ static int ld_col(int lane) { return ((lane >> 2) % 12) * 8; }
};

}  // namespace dev
}  // namespace cuflash
