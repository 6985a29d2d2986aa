#pragma once

// Device-side building blocks shared by the gfx950 kernels: element traits for the three
// storage types, CDNA4 MFMA wrappers, 16-byte vector I/O, wave reductions and the workgroup
// scheduling helpers.
//
// MFMA register layouts used throughout (wave64, verified on gfx950):
//   v_mfma_f32_32x32x16_{bf16,f16}:  A (32x16): lane l holds A[l%32][8*(l/32) + 0..7]
//                                    B (16x32): lane l holds B[8*(l/32) + 0..7][l%32]
//                                    C (32x32): lane l holds C[8*(r/4) + 4*(l/32) + r%4][l%32],
//                                               r = 0..15
//   v_mfma_f32_32x32x2f32:           A: lane l holds A[l%32][l/32]; B: B[l/32][l%32]; C as above.
// Because the sum over k is order-free, a kernel may assign any logical k index to each
// (lane-half, slot) pair as long as the A and B operands agree; the kernels use this to feed
// an accumulator tile (C layout) straight back as the B operand of the next product.

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cuflash {
namespace dev {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kFltMin = 1.17549435e-38f;  // smallest normal float

// ---------------------------------------------------------------------------------------------
// Element traits. 16-bit types are moved around as raw uint16_t bit patterns; conversions use
// the hardware round-to-nearest-even converts (v_cvt_pk_bf16_f32, v_cvt_f16_f32), matching the
// reference's __float2bfloat16_rn / __float2half (src/kernels/impl/type_adapter.cuh:18-32).
// ---------------------------------------------------------------------------------------------
template <typename T>
struct Elem;

template <>
struct Elem<__hip_bfloat16> {
    using frag = bf16x8;
    static __device__ __forceinline__ float to_f(uint16_t v) {
        return __uint_as_float(static_cast<uint32_t>(v) << 16);
    }
    // Two floats -> two RNE bf16 packed in one dword (low half = a).
    static __device__ __forceinline__ uint32_t pack2(float a, float b) {
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        bf16x2 r;
        r[0] = static_cast<__bf16>(a);
        r[1] = static_cast<__bf16>(b);
        return __builtin_bit_cast(uint32_t, r);
    }
    static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    // acc + a.lo b.lo + a.hi b.hi of two packed pairs, in fp32 (v_dot2_f32_bf16).
    static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                               __builtin_bit_cast(bf16x2, b), acc, false);
    }
};

template <>
struct Elem<__half> {
    using frag = f16x8;
    static __device__ __forceinline__ float to_f(uint16_t v) {
        return static_cast<float>(__builtin_bit_cast(_Float16, v));
    }
    // Two floats -> two RNE halves packed in one dword (low half = a): one v_cvt_pk_f16_f32.
    static __device__ __forceinline__ uint32_t pack2(float a, float b) {
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        f32x2 v;
        v[0] = a;
        v[1] = b;
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
    }
    static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    // acc + a.lo b.lo + a.hi b.hi of two packed pairs, in fp32 (v_dot2_f32_f16).
    static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b),
                                      acc, false);
    }
};

// 16 bytes of 16-bit elements reinterpreted as an MFMA operand.
template <typename T>
__device__ __forceinline__ typename Elem<T>::frag as_frag(u32x4 v) {
    return __builtin_bit_cast(typename Elem<T>::frag, v);
}

// Eight floats -> eight 16-bit elements packed as an MFMA operand.
template <typename T>
__device__ __forceinline__ typename Elem<T>::frag pack_frag(float a0, float a1, float a2, float a3,
                                                            float a4, float a5, float a6,
                                                            float a7) {
    u32x4 v;
    v[0] = Elem<T>::pack2(a0, a1);
    v[1] = Elem<T>::pack2(a2, a3);
    v[2] = Elem<T>::pack2(a4, a5);
    v[3] = Elem<T>::pack2(a6, a7);
    return as_frag<T>(v);
}

__device__ __forceinline__ f32x16 mma_f32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------------------------
// Global / LDS vector access
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ u32x4 ld16(const void* p) {
    return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
// Non-temporal 16-byte store (global_store_dwordx4 ... nt): for outputs written once.
__device__ __forceinline__ void st16_nt(void* p, u32x4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}
__device__ __forceinline__ void st8(void* p, u32x2 v) { *reinterpret_cast<u32x2*>(p) = v; }

// ---------------------------------------------------------------------------------------------
// Row-tile store through LDS. A wave holds 32 rows of a [rows, D] 16-bit output as accumulator
// tiles (lane l: row r0 + l % 32, columns 32 dt + 8 (r / 4) + 4 (l / 32) + r % 4 of acc[dt][r]).
// Stored straight from that layout, each 8-byte store instruction writes 16-byte pieces of 32
// rows 2 D bytes apart. store_rows_staged instead writes the rows (times mul, RNE) to the wave's
// LDS area stg (32 rows of 2 D + 16 bytes; the padding spreads the 32 rows over the banks) and
// stores 1 KB of whole contiguous rows per instruction, non-temporally. Rows at or past nrows
// are not stored. LDS accesses of one wave are performed in order, so the caller only has to
// make sure no other wave still uses stg.
// ---------------------------------------------------------------------------------------------
template <int D>
constexpr int staged_rows_bytes() {
    return 32 * (2 * D + 16);
}
template <typename T, int D>
__device__ __forceinline__ void store_rows_staged(const f32x16 (&acc)[D / 32], float mul,
                                                  unsigned char* stg, uint16_t* base, int r0,
                                                  int nrows) {
    constexpr int P = 2 * D + 16;  // staging row pitch (bytes)
    constexpr int LPR = D / 8;     // 16-byte chunks per row
    static_assert(D % 32 == 0, "whole 32-column accumulator tiles");
    const int lane = threadIdx.x & 63;
    const int l32 = lane & 31;
    const int g2 = lane >> 5;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            u32x2 w;
            w[0] = Elem<T>::pack2(acc[dt][4 * a + 0] * mul, acc[dt][4 * a + 1] * mul);
            w[1] = Elem<T>::pack2(acc[dt][4 * a + 2] * mul, acc[dt][4 * a + 3] * mul);
            st8(stg + l32 * P + (32 * dt + 8 * a + 4 * g2) * 2, w);
        }
    }
    // 16-byte chunk 64 i + lane of the 32 rows (LPR per row, 32 LPR = 64 (D / 16) in all).
#pragma unroll
    for (int i = 0; i < D / 16; ++i) {
        const int r = (64 * i + lane) / LPR;
        const int cc = (64 * i + lane) % LPR;
        const u32x4 v = ld16(stg + r * P + cc * 16);
        if (r0 + r < nrows) st16_nt(base + static_cast<size_t>(r0 + r) * D + cc * 8, v);
    }
}

// ---------------------------------------------------------------------------------------------
// LDS transpose read (gfx950 ds_read_b64_tr_b16).
// Within each 16-lane group, result lane i, slot j (j = 0..3) is element i%4 of the 8-byte chunk
// addressed by lane 4*j + i/4 of the same group (verified on gfx950). `read_tr_frag` uses it to
// build a 32x32x16 operand whose k index runs down the ROWS of a row-major LDS matrix M
// (pitch in elements): lane l receives M[k0 + kslot(l/32, t)][n0 + l%32] for t = 0..7, where
// kslot(h, t) = 8*(t/4) + 4*h + t%4. This is the k assignment of an accumulator tile reused as
// an operand (C-layout rows of one lane: 8*(r/4) + 4*(l/32) + r%4), so products such as P*V,
// dS*K, P^T*dO and dS^T*Q read V, K, dO and Q in their natural row-major layout.
// ---------------------------------------------------------------------------------------------
typedef short i16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i16x4 lds_read_tr16(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4*)(const_cast<uint16_t*>(p)));
}

// Per-lane element offset of the transpose read for k0 = n0 = 0 (add k0 * pitch + n0).
__device__ __forceinline__ int tr_lane_offset(int pitch) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4;   // 16-lane group
    const int kq = lane & 15;  // lane inside the group
    const int row = 4 * (lane >> 5) + (kq >> 2);
    const int col = 16 * (g & 1) + 4 * (kq & 3);
    return row * pitch + col;
}

template <typename T>
__device__ __forceinline__ typename Elem<T>::frag read_tr_frag(const uint16_t* lds_lane,
                                                               int pitch) {
    const i16x4 lo = lds_read_tr16(lds_lane);
    const i16x4 hi = lds_read_tr16(lds_lane + 8 * pitch);
    u32x4 v;
    v[0] = __builtin_bit_cast(u32x2, lo)[0];
    v[1] = __builtin_bit_cast(u32x2, lo)[1];
    v[2] = __builtin_bit_cast(u32x2, hi)[0];
    v[3] = __builtin_bit_cast(u32x2, hi)[1];
    return as_frag<T>(v);
}

// ---------------------------------------------------------------------------------------------
// MFMA policy: one interface over v_mfma_f32_32x32x16_{bf16,f16} (k = 16 per instruction) and
// v_mfma_f32_32x32x2f32 (k = 2), so a kernel is written once for all three element types.
//   row_operand(p): operand whose k index runs along a row of a row-major matrix; p points at
//                   element k0 of this lane's row. Lane half h supplies k = k0 + kslot_row(h, .).
//   acc_operand(c, j): step j of a 32-row accumulator tile reused as an operand (k = tile rows).
//   col_operand(tile, j, pitch): operand whose k index runs down the rows of a row-major LDS
//                   tile (32 rows); `tile` already includes this lane's column offset and, for
//                   16-bit types, the transpose-read lane offset (tr_lane_offset).
//   kSteps = 32 / KW MFMAs contract one 32-row tile.
// ---------------------------------------------------------------------------------------------
template <typename T>
struct Mma {
    using elem = uint16_t;
    using frag = typename Elem<T>::frag;
    static constexpr int KW = 16;
    static constexpr int kSteps = 2;
    static __device__ __forceinline__ frag zero() { return as_frag<T>(u32x4{0u, 0u, 0u, 0u}); }
    static __device__ __forceinline__ frag row_operand(const elem* p) {
        return as_frag<T>(ld16(p + 8 * ((threadIdx.x & 63) >> 5)));
    }
    static __device__ __forceinline__ frag acc_operand(const f32x16& c, int j) {
        return pack_frag<T>(c[8 * j + 0], c[8 * j + 1], c[8 * j + 2], c[8 * j + 3], c[8 * j + 4],
                            c[8 * j + 5], c[8 * j + 6], c[8 * j + 7]);
    }
    // `tile` = tile base + tr_lane_offset(pitch) + column offset.
    static __device__ __forceinline__ frag col_operand(const elem* tile, int j, int pitch) {
        return read_tr_frag<T>(tile + 16 * j * pitch, pitch);
    }
    static __device__ __forceinline__ int col_lane_offset(int pitch) {
        return tr_lane_offset(pitch);
    }
    static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
        return Elem<T>::mma(a, b, c);
    }
};

template <>
struct Mma<float> {
    using elem = float;
    using frag = float;
    static constexpr int KW = 2;
    static constexpr int kSteps = 16;
    static __device__ __forceinline__ frag zero() { return 0.0f; }
    static __device__ __forceinline__ frag row_operand(const elem* p) {
        return p[(threadIdx.x & 63) >> 5];
    }
    static __device__ __forceinline__ frag acc_operand(const f32x16& c, int j) { return c[j]; }
    // `tile` = tile base + col_lane_offset(pitch) + column offset; step j reads tile row
    // 8*(j/4) + 4*h + j%4 (h = lane half), the accumulator row held in register j.
    static __device__ __forceinline__ frag col_operand(const elem* tile, int j, int pitch) {
        return tile[(8 * (j >> 2) + (j & 3)) * pitch];
    }
    static __device__ __forceinline__ int col_lane_offset(int pitch) {
        const int lane = threadIdx.x & 63;
        return 4 * (lane >> 5) * pitch + (lane & 31);
    }
    static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
        return mma_f32(a, b, c);
    }
};

// Transpose-read operand from two explicit LDS byte addresses (the rows k0 + kslot(h, 0..3) and
// k0 + 8 + kslot(h, 0..3) of the same layout as read_tr_frag).
template <typename T>
__device__ __forceinline__ typename Elem<T>::frag tr_frag_at(const unsigned char* p0,
                                                             const unsigned char* p1) {
    const i16x4 lo = lds_read_tr16(reinterpret_cast<const uint16_t*>(p0));
    const i16x4 hi = lds_read_tr16(reinterpret_cast<const uint16_t*>(p1));
    u32x4 v;
    v[0] = __builtin_bit_cast(u32x2, lo)[0];
    v[1] = __builtin_bit_cast(u32x2, lo)[1];
    v[2] = __builtin_bit_cast(u32x2, hi)[0];
    v[3] = __builtin_bit_cast(u32x2, hi)[1];
    return as_frag<T>(v);
}

// ---------------------------------------------------------------------------------------------
// Global -> LDS direct loads (gfx950 global_load_lds_dwordx4): lane i of the wave writes the 16
// bytes at its own global address to lds_base + 16 * i (verified on gfx950). lds_base must be
// wave-uniform; the load is tracked by vmcnt like any other global load.
// ---------------------------------------------------------------------------------------------
// The loads are issued from inline assembly. The compiler then does not know that they write
// LDS and adds no waits for them, so the kernel must order every LDS access itself
// (s_waitcnt vmcnt(0) and a barrier before the data is read, and before a buffer is reused).
// This lets a kernel rotate buffers with run-time offsets, where the compiler would otherwise
// wait for every outstanding load before each LDS read. The LDS base goes in as an M0 operand
// (constraint "{m0}"), so the compiler writes M0 itself and knows that the register is taken.
// The compiler cannot see the memory instruction inside the statement, so it inserts none of
// the wait states that instruction needs. An SALU write of M0 needs one before an LDS DMA that
// uses it, which the `s_nop 0` inside the statement provides whatever the compiler placed in
// between. A VALU write of an SGPR (v_readfirstlane, v_readlane) needs five before a memory
// instruction reads that SGPR, as M0 or as the scalar base address, or the load can use the
// register's previous value: the bases and LDS addresses given to these helpers are scalar
// (SALU) values, and tests/test_code_hazards.py checks every LDS-DMA load of the built library
// for a VALU write of its SGPRs within five wait states. A base that comes from a lane
// (v_readlane) needs the five-wait-state form (decode.hip's lds_dma16_nt_s: 1-3% slower in the
// head_dim-128 and 256 forward and backward kernels).
__device__ __forceinline__ unsigned lds_address(const void* p) {
    return static_cast<unsigned>(reinterpret_cast<uintptr_t>(
        (const __attribute__((address_space(3))) unsigned char*)(p)));
}
__device__ __forceinline__ void lds_dma16_async(const void* src, unsigned char* lds_base) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds_address(lds_base)))
                 : "memory");
}
// The same load with a wave-uniform base address in SGPRs and a 32-bit per-lane byte offset:
// the address of lane i is sbase + voff(i), so a kernel that streams tiles keeps voff fixed and
// only advances sbase (scalar adds) from tile to tile.
__device__ __forceinline__ void lds_dma16_async_s(const void* sbase, unsigned voff,
                                                  unsigned char* lds_base) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(sbase),
                   "{m0}"(__builtin_amdgcn_readfirstlane(lds_address(lds_base)))
                 : "memory");
}
__device__ __forceinline__ void lds_dma4_async(const void* src, unsigned char* lds_base) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off"
                 :
                 : "v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds_address(lds_base)))
                 : "memory");
}

// ---------------------------------------------------------------------------------------------
// Wave reductions
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float xor_shuffle(float v, int mask) {
    return __shfl_xor(v, mask, 64);
}

// max / sum of v over the lane pair (l, l ^ 32), with gfx950's v_permlane32_swap (VALU, no LDS).
__device__ __forceinline__ float pair_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// ---------------------------------------------------------------------------------------------
// Workgroup scheduling.
// Workgroups are dispatched round-robin over the 8 XCDs of an MI355X (workgroup i -> XCD i % 8),
// and each XCD has its own L2. `xcd_remap` renumbers dispatch slots so that consecutive logical
// ids land on the same XCD: the blocks of one (batch, head) share K/V in one L2.
// ---------------------------------------------------------------------------------------------
constexpr int kNumXcd = 8;

__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
    if (nblocks % kNumXcd != 0) return bid;
    const int per_xcd = nblocks / kNumXcd;
    return (bid % kNumXcd) * per_xcd + bid / kNumXcd;
}

// Workgroup id -> (head, rank) for grids of BH heads x nranks blocks whose blocks of one head
// share K/V. When BH is a multiple of 8 every XCD gets BH / 8 whole heads (their K/V stay in its
// L2) and, inside an XCD, blocks are dispatched rank-major (rank 0 of each of its heads, then
// rank 1, ...); otherwise ranks are dispatched round-robin over all heads. Kernels map rank 0 to
// their longest block, so long blocks start first in either case.
__device__ __forceinline__ void head_rank_order(int bid, int BH, int& bh, int& rank) {
    if (BH % kNumXcd == 0) {
        const int hpx = BH / kNumXcd;
        const int k = bid / kNumXcd;
        rank = k / hpx;
        bh = (bid % kNumXcd) * hpx + k % hpx;
    } else {
        rank = bid / BH;
        bh = bid % BH;
    }
}

// Work item / workgroup id -> (head, rank) for `heads` * `per_head` items whose items of one head
// share K/V (forward, dq) or Q/dO (dkdv). Rank-major (head_rank_order: rank 0 of every head of an
// XCD first, the longest item under a causal mask) unless `head_major`: then, with the heads
// split over the XCDs as in head_rank_order, an XCD takes all ranks of one head before the next
// head, so the items of a head that run at the same time read the same rows and share them in
// the XCD's L2 and the Infinity Cache, at the price of starting a head's longest items late.
__device__ __forceinline__ void item_order(int bid, int heads, int per_head, bool head_major,
                                           int& h, int& r) {
    if (head_major && heads % kNumXcd == 0) {
        const int hpx = heads / kNumXcd;
        const int k = bid / kNumXcd;
        h = (bid % kNumXcd) * hpx + k / per_head;
        r = k % per_head;
    } else {
        head_rank_order(bid, heads, h, r);
    }
}

}  // namespace dev
}  // namespace cuflash
