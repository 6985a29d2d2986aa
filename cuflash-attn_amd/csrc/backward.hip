// FlashAttention backward for gfx950 (MI355X).
//
// Same flow as the reference launcher (src/backward/flash_attention_backward_typed.cu:440-579):
//   1. delta_kernel:  D_i = sum_d dO_id * O_id in fp32 (reference compute_D_kernel, :13-34),
//                     into a stream-ordered workspace (reference AsyncFloatBuffer, :374-394);
//   2. dq_kernel:     Q-stationary. Per key block: S = scale*Q K^T, P = exp(S - L),
//                     dP = dO V^T, dS = P (dP - D), dQ += scale * dS K
//                     (reference flash_attention_backward_dq_kernel, :37-143);
//   3. dkdv_kernel:   KV-stationary. Per query block: P as above, dV += P^T dO,
//                     dS = P (dP - D), dK += scale * dS^T Q
//                     (reference flash_attention_backward_dkdv_kernel, :146-288).
// Masked (causal / out-of-range) entries contribute 0, as in the reference (:108-110, :214-220).
//
// Every product runs on MFMA (32x32x16 for fp16/bf16, 32x32x2 for fp32) through the Mma<T>
// policy. Scores are formed transposed where that makes the consumer's operand come straight
// out of the accumulator registers:
//   dq_kernel   S^T = K Q^T, dP^T = V dO^T (lane = query),  dQ^T += K^T dS^T (K via transpose reads)
//   dkdv_kernel S = Q K^T, dP = dO V^T (lane = key),       dV^T += dO^T P, dK^T += Q^T dS
// so each lane owns one query row of dQ, or one key row of dK/dV, for the whole kernel. For
// fp16/bf16 P and dS are rounded to the input type before their products (fp32 accumulate).
// For fp16/bf16 (every head_dim) the same steps run as delta_ld_kernel, then
// dq_lds_tiles and dkdv_lds_tiles items in one launch (bwd_fused_kernel, section 4). Every path is
// deterministic: no atomics, and each output element is written by exactly one lane.
//
// Shapes: Q, O, dO, dQ are [BH, Nq, D], K, V, dK, dV are [BH / group, Nk, D] (query head bh
// reads key/value head bh / group), L and D are [BH, Nq]. With a causal mask query i sees the
// keys j <= i + coff, coff = Nk - Nq >= 0. The key-stationary kernels accumulate dK and dV of a
// key/value head over all `group` query heads that read it, in registers, before one store.

#include "common.hpp"
#include "launch.hpp"
#include "profile.hpp"
#include "tile_groups.hpp"

#include <algorithm>
#include <type_traits>

namespace cuflash {
namespace dev {

// LDS pitches (elements). Row-operand tiles: rows 16 bytes apart modulo 256 bytes. Column
// (transpose-read) tiles: rows 64 bytes apart modulo 128 bytes. fp32 tiles keep 16-byte rows.
template <typename T, int D>
struct BwdPitch {
    static constexpr int RP = D + 8;
    static constexpr int CP = ((2 * D) % 128 == 64) ? D : D + 32;
};
template <int D>
struct BwdPitch<float, D> {
    static constexpr int RP = D + 4;
    static constexpr int CP = D + 8;
};

// Copies a ROWS x D row-major tile of global memory into registers (16-byte chunks, rows past
// `valid_rows` read as zero) and later into one or two LDS tiles.
template <typename E, int ROWS, int D, int THREADS>
struct TileCopy {
    static constexpr int VEC = 16 / static_cast<int>(sizeof(E));
    static constexpr int CPR = D / VEC;
    static constexpr int CHUNKS = ROWS * CPR;
    static constexpr int PER_THREAD = (CHUNKS + THREADS - 1) / THREADS;
    u32x4 reg[PER_THREAD];

    __device__ __forceinline__ void fetch(const E* src, int valid_rows, int tid) {
#pragma unroll
        for (int i = 0; i < PER_THREAD; ++i) {
            const int id = i * THREADS + tid;
            const int row = id / CPR;
            const int col = (id % CPR) * VEC;
            reg[i] = u32x4{0u, 0u, 0u, 0u};
            if (id < CHUNKS && row < valid_rows) reg[i] = ld16(src + static_cast<size_t>(row) * D + col);
        }
    }
    __device__ __forceinline__ void stage(E* dst, int pitch, int tid) const {
#pragma unroll
        for (int i = 0; i < PER_THREAD; ++i) {
            const int id = i * THREADS + tid;
            if (id < CHUNKS) st16(dst + (id / CPR) * pitch + (id % CPR) * VEC, reg[i]);
        }
    }
};

// ------------------------------------------------------------------------------------------
// 1. D = rowsum(dO * O)
// ------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float dot16(u32x4 a, u32x4 b);

template <>
__device__ __forceinline__ float dot16<float>(u32x4 a, u32x4 b) {
    const f32x4 x = __builtin_bit_cast(f32x4, a);
    const f32x4 y = __builtin_bit_cast(f32x4, b);
    return x[0] * y[0] + x[1] * y[1] + x[2] * y[2] + x[3] * y[3];
}

template <typename T>
__device__ __forceinline__ float dot16(u32x4 a, u32x4 b) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        s += Elem<T>::to_f(static_cast<uint16_t>(a[i])) * Elem<T>::to_f(static_cast<uint16_t>(b[i]));
        s += Elem<T>::to_f(static_cast<uint16_t>(a[i] >> 16)) *
             Elem<T>::to_f(static_cast<uint16_t>(b[i] >> 16));
    }
    return s;
}

// Lanes per row of delta_kernel: the 16-byte chunks of a row, rounded up to a power of two so
// that the xor-butterfly sum stays inside the row's lanes (head_dim 96: 12 chunks -> 16 lanes).
template <int CHUNKS>
constexpr int delta_lanes() {
    int l = 1;
    while (l < CHUNKS) l *= 2;
    return l;
}

template <typename T, int D>
__global__ void __launch_bounds__(256)
    delta_kernel(const typename Mma<T>::elem* __restrict__ dO,
                 const typename Mma<T>::elem* __restrict__ O, float* __restrict__ Dst,
                 long long rows) {
    using E = typename Mma<T>::elem;
    constexpr int VEC = 16 / static_cast<int>(sizeof(E));
    constexpr int CHUNKS = D / VEC;                 // 16-byte chunks per row
    constexpr int LPR = delta_lanes<CHUNKS>();      // lanes per row
    static_assert(LPR <= 64, "a row's lanes must fit in one wave");
    const long long t = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    const long long row = t / LPR;
    const int part = static_cast<int>(t % LPR);
    float s = 0.0f;
    if (row < rows && part < CHUNKS) {
        const size_t off = static_cast<size_t>(row) * D + part * VEC;
        s = dot16<T>(ld16(dO + off), ld16(O + off));
    }
#pragma unroll
    for (int w = LPR / 2; w > 0; w >>= 1) s += xor_shuffle(s, w);
    if (row < rows && part == 0) Dst[row] = s;
}

// ------------------------------------------------------------------------------------------
// 2. dQ (query-stationary)
// ------------------------------------------------------------------------------------------
template <typename T, int D>
struct DqCfg {
    static constexpr int kThreads = 256;
    static constexpr int BM = 128;  // query rows per workgroup (32 per wave)
    static constexpr int BN = 32;   // keys per block
    static constexpr int RP = BwdPitch<T, D>::RP;
    static constexpr int CP = BwdPitch<T, D>::CP;
};

// fp32 operands at D = 128 need more than the 256 registers a 2-wave budget allows.
template <typename T, int D>
constexpr int dq_min_waves() {
    return ((std::is_same<T, float>::value && D >= 128) || D >= 256) ? 1 : 2;
}

// Query block `bid` of `nblocks` (= BH * nqb); dq_kernel runs one per workgroup.
template <typename T, int D>
__device__ __forceinline__ void dq_body(const typename Mma<T>::elem* __restrict__ Q,
                                        const typename Mma<T>::elem* __restrict__ K,
                                        const typename Mma<T>::elem* __restrict__ V,
                                        const float* __restrict__ L,
                                        const typename Mma<T>::elem* __restrict__ dO,
                                        const float* __restrict__ Dl,
                                        typename Mma<T>::elem* __restrict__ dQ, int Nq, int Nk,
                                        int coff, int group, int nqb, float c, float scale,
                                        int causal, int bid, int nblocks) {
    using M = Mma<T>;
    using E = typename M::elem;
    using frag = typename M::frag;
    using Cfg = DqCfg<T, D>;
    __shared__ __attribute__((aligned(16))) E Ks[Cfg::BN * Cfg::RP];
    __shared__ __attribute__((aligned(16))) E Kc[Cfg::BN * Cfg::CP];
    __shared__ __attribute__((aligned(16))) E Vs[Cfg::BN * Cfg::RP];

    const int lid = xcd_remap(bid, nblocks);
    const int bh = lid / nqb;
    const int qb = causal ? nqb - 1 - lid % nqb : lid % nqb;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int l32 = lane & 31;
    const int g2 = lane >> 5;

    const size_t head = static_cast<size_t>(bh) * Nq * D;             // Q, dO, dQ
    const size_t kv_head = static_cast<size_t>(bh / group) * Nk * D;  // K, V
    const int q0 = qb * Cfg::BM + wave * 32;
    const int q = q0 + l32;
    const bool q_ok = q < Nq;

    frag qf[D / M::KW];
    frag of[D / M::KW];
#pragma unroll
    for (int ks = 0; ks < D / M::KW; ++ks) {
        qf[ks] = M::zero();
        of[ks] = M::zero();
        if (q_ok) {
            qf[ks] = M::row_operand(Q + head + static_cast<size_t>(q) * D + M::KW * ks);
            of[ks] = M::row_operand(dO + head + static_cast<size_t>(q) * D + M::KW * ks);
        }
    }
    // Rows past Nq get L = +inf so that P = exp(S - L) is exactly 0 there.
    const float l2 = q_ok ? L[static_cast<size_t>(bh) * Nq + q] * kLog2e : INFINITY;
    const float dq_row = q_ok ? Dl[static_cast<size_t>(bh) * Nq + q] : 0.0f;

    f32x16 acc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) acc[dt] = f32x16{};

    const int kv_end = causal ? min(Nk, (qb + 1) * Cfg::BM + coff) : Nk;
    const int nkb = (kv_end + Cfg::BN - 1) / Cfg::BN;
    TileCopy<E, Cfg::BN, D, Cfg::kThreads> kcp, vcp;
    const int col_off = M::col_lane_offset(Cfg::CP);

    if (nkb > 0) {
        kcp.fetch(K + kv_head, Nk, tid);
        vcp.fetch(V + kv_head, Nk, tid);
    }
    for (int kb = 0; kb < nkb; ++kb) {
        const int key0 = kb * Cfg::BN;
        __syncthreads();
        kcp.stage(Ks, Cfg::RP, tid);
        kcp.stage(Kc, Cfg::CP, tid);
        vcp.stage(Vs, Cfg::RP, tid);
        __syncthreads();
        if (kb + 1 < nkb) {
            const size_t off = kv_head + static_cast<size_t>(key0 + Cfg::BN) * D;
            kcp.fetch(K + off, Nk - key0 - Cfg::BN, tid);
            vcp.fetch(V + off, Nk - key0 - Cfg::BN, tid);
        }
        if (causal && key0 > q0 + 31 + coff) continue;

        f32x16 s = f32x16{};
        f32x16 dp = f32x16{};
#pragma unroll
        for (int ks = 0; ks < D / M::KW; ++ks) {
            s = M::mma(M::row_operand(&Ks[l32 * Cfg::RP + M::KW * ks]), qf[ks], s);
            dp = M::mma(M::row_operand(&Vs[l32 * Cfg::RP + M::KW * ks]), of[ks], dp);
        }
        const bool masked = (key0 + Cfg::BN > Nk) || (causal && key0 + Cfg::BN - 1 > q0 + coff);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float p = fast_exp2(fmaf(s[r], c, -l2));
            if (masked) {
                const int key = key0 + 8 * (r >> 2) + 4 * g2 + (r & 3);
                if (key >= Nk || (causal && key > q + coff)) p = 0.0f;
            }
            s[r] = p * (dp[r] - dq_row);
        }
#pragma unroll
        for (int j = 0; j < M::kSteps; ++j) {
            const frag b = M::acc_operand(s, j);
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt)
                acc[dt] = M::mma(M::col_operand(&Kc[32 * dt + col_off], j, Cfg::CP), b, acc[dt]);
        }
    }

    if (q_ok) {
        E* row = dQ + head + static_cast<size_t>(q) * D;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const int d = 32 * dt + 8 * a + 4 * g2;
                if constexpr (std::is_same<T, float>::value) {
                    f32x4 w;
#pragma unroll
                    for (int u = 0; u < 4; ++u) w[u] = acc[dt][4 * a + u] * scale;
                    st16(row + d, __builtin_bit_cast(u32x4, w));
                } else {
                    u32x2 w;
                    w[0] = Elem<T>::pack2(acc[dt][4 * a + 0] * scale, acc[dt][4 * a + 1] * scale);
                    w[1] = Elem<T>::pack2(acc[dt][4 * a + 2] * scale, acc[dt][4 * a + 3] * scale);
                    st8(row + d, w);
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------------------
// 3. dK, dV (key/value-stationary)
// ------------------------------------------------------------------------------------------
template <typename T, int D>
struct DkvCfg {
    static constexpr int kThreads = 256;
    static constexpr int BN = 128;  // keys per workgroup (32 per wave)
    static constexpr int BM = 32;   // query rows per block
    static constexpr int RP = BwdPitch<T, D>::RP;
    static constexpr int CP = BwdPitch<T, D>::CP;
};

// Key block `bid` of `nblocks` (= BHkv * nkb); dkdv_kernel runs one per workgroup.
template <typename T, int D>
__device__ __forceinline__ void dkdv_body(const typename Mma<T>::elem* __restrict__ Q,
                                          const typename Mma<T>::elem* __restrict__ K,
                                          const typename Mma<T>::elem* __restrict__ V,
                                          const float* __restrict__ L,
                                          const typename Mma<T>::elem* __restrict__ dO,
                                          const float* __restrict__ Dl,
                                          typename Mma<T>::elem* __restrict__ dK,
                                          typename Mma<T>::elem* __restrict__ dV, int Nq, int Nk,
                                          int coff, int group, int nkb, float c, float scale,
                                          int causal, int bid, int nblocks) {
    using M = Mma<T>;
    using E = typename M::elem;
    using frag = typename M::frag;
    using Cfg = DkvCfg<T, D>;
    __shared__ __attribute__((aligned(16))) E Qs[Cfg::BM * Cfg::RP];
    __shared__ __attribute__((aligned(16))) E Qc[Cfg::BM * Cfg::CP];
    __shared__ __attribute__((aligned(16))) E Os[Cfg::BM * Cfg::RP];
    __shared__ __attribute__((aligned(16))) E Oc[Cfg::BM * Cfg::CP];
    __shared__ __attribute__((aligned(16))) float Ls[Cfg::BM];
    __shared__ __attribute__((aligned(16))) float Ds[Cfg::BM];

    const int lid = xcd_remap(bid, nblocks);
    const int bkv = lid / nkb;  // key/value head
    const int kb = lid % nkb;   // ascending: with a causal mask the first blocks carry the most work
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int l32 = lane & 31;
    const int g2 = lane >> 5;

    const size_t kv_head = static_cast<size_t>(bkv) * Nk * D;  // K, V, dK, dV
    const int k0 = kb * Cfg::BN + wave * 32;  // first key of this wave
    const int key = k0 + l32;                 // key row owned by this lane
    const bool key_ok = key < Nk;

    frag kf[D / M::KW];
    frag vf[D / M::KW];
#pragma unroll
    for (int ks = 0; ks < D / M::KW; ++ks) {
        kf[ks] = M::zero();
        vf[ks] = M::zero();
        if (key_ok) {
            kf[ks] = M::row_operand(K + kv_head + static_cast<size_t>(key) * D + M::KW * ks);
            vf[ks] = M::row_operand(V + kv_head + static_cast<size_t>(key) * D + M::KW * ks);
        }
    }

    f32x16 dk[D / 32];
    f32x16 dv[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        dk[dt] = f32x16{};
        dv[dt] = f32x16{};
    }

    // Query blocks [qb_begin, nqb) of each of the `group` query heads of this key/value head, as
    // one sequence of n_it iterations (it -> head bkv * group + it / span, block
    // qb_begin + it % span). With a causal mask the blocks before the first query that sees
    // key kb * BN are skipped.
    const int nqb = (Nq + Cfg::BM - 1) / Cfg::BM;
    const int qb_begin = causal ? max(0, kb * Cfg::BN - coff) / Cfg::BM : 0;
    const int span = nqb - qb_begin;
    const int n_it = span > 0 ? group * span : 0;
    TileCopy<E, Cfg::BM, D, Cfg::kThreads> qcp, ocp;
    float lreg = 0.0f;
    auto fetch = [&](int it) {
        const int bh = bkv * group + it / span;
        const int r0 = (qb_begin + it % span) * Cfg::BM;
        const size_t q_head = static_cast<size_t>(bh) * Nq * D;
        qcp.fetch(Q + q_head + static_cast<size_t>(r0) * D, Nq - r0, tid);
        ocp.fetch(dO + q_head + static_cast<size_t>(r0) * D, Nq - r0, tid);
        if (tid < 2 * Cfg::BM) {
            const int r = r0 + (tid % Cfg::BM);
            const size_t row = static_cast<size_t>(bh) * Nq + r;
            if (tid < Cfg::BM)
                lreg = r < Nq ? L[row] * kLog2e : INFINITY;  // rows past Nq: P = 0
            else
                lreg = r < Nq ? Dl[row] : 0.0f;
        }
    };
    const int col_off = M::col_lane_offset(Cfg::CP);

    if (n_it > 0) fetch(0);
    for (int it = 0; it < n_it; ++it) {
        const int q0 = (qb_begin + it % span) * Cfg::BM;
        __syncthreads();
        qcp.stage(Qs, Cfg::RP, tid);
        qcp.stage(Qc, Cfg::CP, tid);
        ocp.stage(Os, Cfg::RP, tid);
        ocp.stage(Oc, Cfg::CP, tid);
        if (tid < Cfg::BM)
            Ls[tid] = lreg;
        else if (tid < 2 * Cfg::BM)
            Ds[tid - Cfg::BM] = lreg;
        __syncthreads();
        if (it + 1 < n_it) fetch(it + 1);
        // Waves whose keys all follow every query of the block still run (P = 0 there): a
        // branch around the MFMAs would make the compiler copy the dK/dV accumulators between
        // AGPRs and VGPRs on every iteration.

        // S = Q K^T and dP = dO V^T: rows = queries, column = this lane's key.
        f32x16 s = f32x16{};
        f32x16 dp = f32x16{};
#pragma unroll
        for (int ks = 0; ks < D / M::KW; ++ks) {
            s = M::mma(M::row_operand(&Qs[l32 * Cfg::RP + M::KW * ks]), kf[ks], s);
            dp = M::mma(M::row_operand(&Os[l32 * Cfg::RP + M::KW * ks]), vf[ks], dp);
        }
        const bool masked = causal && (k0 + 31 > q0 + coff);
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            const f32x4 lv = *reinterpret_cast<const f32x4*>(&Ls[8 * a + 4 * g2]);
            const f32x4 dv4 = *reinterpret_cast<const f32x4*>(&Ds[8 * a + 4 * g2]);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int r = 4 * a + u;
                float p = fast_exp2(fmaf(s[r], c, -lv[u]));
                if (masked && key > q0 + 8 * a + 4 * g2 + u + coff) p = 0.0f;
                s[r] = p;
                dp[r] = p * (dp[r] - dv4[u]);
            }
        }
        // dV^T += dO^T P and dK^T += Q^T dS: k = the block's query rows.
#pragma unroll
        for (int j = 0; j < M::kSteps; ++j) {
            const frag bp = M::acc_operand(s, j);
            const frag bs = M::acc_operand(dp, j);
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
                dv[dt] = M::mma(M::col_operand(&Oc[32 * dt + col_off], j, Cfg::CP), bp, dv[dt]);
                dk[dt] = M::mma(M::col_operand(&Qc[32 * dt + col_off], j, Cfg::CP), bs, dk[dt]);
            }
        }
    }

    if (key_ok) {
        E* krow = dK + kv_head + static_cast<size_t>(key) * D;
        E* vrow = dV + kv_head + static_cast<size_t>(key) * D;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const int d = 32 * dt + 8 * a + 4 * g2;
                if constexpr (std::is_same<T, float>::value) {
                    f32x4 wk, wv;
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        wk[u] = dk[dt][4 * a + u] * scale;
                        wv[u] = dv[dt][4 * a + u];
                    }
                    st16(krow + d, __builtin_bit_cast(u32x4, wk));
                    st16(vrow + d, __builtin_bit_cast(u32x4, wv));
                } else {
                    u32x2 wk, wv;
                    wk[0] = Elem<T>::pack2(dk[dt][4 * a + 0] * scale, dk[dt][4 * a + 1] * scale);
                    wk[1] = Elem<T>::pack2(dk[dt][4 * a + 2] * scale, dk[dt][4 * a + 3] * scale);
                    wv[0] = Elem<T>::pack2(dv[dt][4 * a + 0], dv[dt][4 * a + 1]);
                    wv[1] = Elem<T>::pack2(dv[dt][4 * a + 2], dv[dt][4 * a + 3]);
                    st8(krow + d, wk);
                    st8(vrow + d, wv);
                }
            }
        }
    }
}

template <typename T, int D>
__global__ void __launch_bounds__(256, (dq_min_waves<T, D>()))
    dq_kernel(const typename Mma<T>::elem* __restrict__ Q,
              const typename Mma<T>::elem* __restrict__ K,
              const typename Mma<T>::elem* __restrict__ V, const float* __restrict__ L,
              const typename Mma<T>::elem* __restrict__ dO, const float* __restrict__ Dl,
              typename Mma<T>::elem* __restrict__ dQ, int Nq, int Nk, int coff, int group,
              int nqb, float c, float scale, int causal) {
    dq_body<T, D>(Q, K, V, L, dO, Dl, dQ, Nq, Nk, coff, group, nqb, c, scale, causal,
                  blockIdx.x, gridDim.x);
}

template <typename T, int D>
__global__ void __launch_bounds__(256, 1)
    dkdv_kernel(const typename Mma<T>::elem* __restrict__ Q,
                const typename Mma<T>::elem* __restrict__ K,
                const typename Mma<T>::elem* __restrict__ V, const float* __restrict__ L,
                const typename Mma<T>::elem* __restrict__ dO, const float* __restrict__ Dl,
                typename Mma<T>::elem* __restrict__ dK, typename Mma<T>::elem* __restrict__ dV,
                int Nq, int Nk, int coff, int group, int nkb, float c, float scale, int causal) {
    dkdv_body<T, D>(Q, K, V, L, dO, Dl, dK, dV, Nq, Nk, coff, group, nkb, c, scale, causal,
                    blockIdx.x, gridDim.x);
}

// Both passes in one launch, for launches too small to fill the GPU one after the other: the
// first n_dkdv workgroups run dkdv_body (the longer items first), the others dq_body. The two
// bodies' LDS arrays add up; the register budget is dkdv's.
template <typename T, int D>
__global__ void __launch_bounds__(256, 1)
    dq_dkdv_kernel(const typename Mma<T>::elem* __restrict__ Q,
                   const typename Mma<T>::elem* __restrict__ K,
                   const typename Mma<T>::elem* __restrict__ V, const float* __restrict__ L,
                   const typename Mma<T>::elem* __restrict__ dO, const float* __restrict__ Dl,
                   typename Mma<T>::elem* __restrict__ dQ, typename Mma<T>::elem* __restrict__ dK,
                   typename Mma<T>::elem* __restrict__ dV, int Nq, int Nk, int coff, int group,
                   int nqb, int nkb, int n_dkdv, float c, float scale, int causal) {
    if (static_cast<int>(blockIdx.x) < n_dkdv)
        dkdv_body<T, D>(Q, K, V, L, dO, Dl, dK, dV, Nq, Nk, coff, group, nkb, c, scale, causal,
                        blockIdx.x, n_dkdv);
    else
        dq_body<T, D>(Q, K, V, L, dO, Dl, dQ, Nq, Nk, coff, group, nqb, c, scale, causal,
                      blockIdx.x - n_dkdv, gridDim.x - n_dkdv);
}

// ------------------------------------------------------------------------------------------
// 4. Backward for head_dim 64, 128 and 256 (fp16 / bf16)
// ------------------------------------------------------------------------------------------
// Row statistics for bwd_fused_kernel: LD[bh * Npad + r] = (L * log2(e), D) for r < N and
// (+inf, 0) for the padding rows N <= r < Npad (Npad = N rounded up to 32), so that P = 0 there
// without any masking. At head_dim 64 (neg_d_rows) each 32 rows are stored instead as the 32
// values L * log2(e), then the 32 values -D (same 256 bytes): the dkdv items then start their
// dP MFMA chain from -D read straight into the accumulator, so dS = P (dP - D) takes one
// multiply per score instead of a subtract and a multiply (head_dim 64, where the vector work
// sets the time: backward 3-5% faster; at 128 the same form measured 1.5% slower non-causal and
// at 32 mixed, so they keep the interleaved pairs). N is the query length. Block 0 also clears
// the kNumXcd work-queue counters of the bwd_fused_kernel launch that follows on the stream.
template <int D>
constexpr bool neg_d_rows() {
    return D == 64;
}
template <typename T, int D>
__global__ void __launch_bounds__(256)
    delta_ld_kernel(const uint16_t* __restrict__ dO, const uint16_t* __restrict__ O,
                    const float* __restrict__ L, float2* __restrict__ LD, int N, int Npad,
                    long long rows_pad, int* __restrict__ queues) {
    if (blockIdx.x == 0 && threadIdx.x < kNumXcd) queues[threadIdx.x] = 0;
    constexpr int CHUNKS = D / 8;                // 16-byte chunks per row
    constexpr int LPR = delta_lanes<CHUNKS>();   // lanes per row (a power of two)
    const long long t = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    const long long prow = t / LPR;  // padded row index
    const int part = static_cast<int>(t % LPR);
    const long long bh = prow / Npad;
    const int r = static_cast<int>(prow % Npad);
    const bool real = prow < rows_pad && r < N;
    float s = 0.0f;
    if (real && part < CHUNKS) {
        const size_t off = static_cast<size_t>(bh * N + r) * D + part * 8;
        s = dot16<T>(ld16(dO + off), ld16(O + off));
    }
#pragma unroll
    for (int w = LPR / 2; w > 0; w >>= 1) s += xor_shuffle(s, w);
    if (prow < rows_pad && part == 0) {
        const float lv = real ? L[bh * N + r] * kLog2e : INFINITY;
        if constexpr (neg_d_rows<D>()) {
            float* blk = reinterpret_cast<float*>(LD) + (prow >> 5) * 64 + (prow & 31);
            blk[0] = lv;
            blk[32] = real ? -s : 0.0f;
        } else {
            LD[prow] = make_float2(lv, real ? s : 0.0f);
        }
    }
}

// ------------------------------------------------------------------------------------------
// dkdv_lds_tiles and dq_lds_tiles restate dkdv_kernel and dq_kernel (same products, same
// rounding of P and dS to T) with a gfx950 data path: tiles go global -> LDS by direct loads
// (global_load_lds_dwordx4, issued from inline assembly so that buffers can rotate at run time)
// into the padded row-group layout of the forward kernels (TileGroups below), whose single copy
// of a tile serves both the row reads of S = Q K^T / dP = dO V^T and the transpose reads of
// dV^T += dO^T P /
// dK^T += Q^T dS / dQ^T += K^T dS^T without bank conflicts; blocks are double-buffered with one
// barrier per block; (L log2 e, D) rows come padded from delta_ld_kernel; and the register
// budget allows two workgroups per CU at head_dim 64 and 128, so the two waves of each SIMD hide
// each other's latencies (one at head_dim 256).
// TileGroups<D> (tile_groups.hpp) gives these layouts per head_dim.
// Item orders (item_order, common.hpp), measured bitwise equal: dq items head-major 0.3-3%
// faster at every shape (config 3 447.6 -> 443.3 us, config 5 -2.9%); dkdv items head-major
// 2.2-3.5% faster at config 5 but up to 11% slower at config 3 causal, where a head's longest
// items then start too late to finish with the rest.

// Key-stationary part of work item `bid` of heads * nkb (kb = 0 has the most work; the order
// of the ids is item_order's, bit 0 of `order`); smem
// holds at least dkdv_lds<D>() bytes. Without kShares an item is (key/value head, key block) and runs
// over all `group` query heads of its key/value head (heads = BHkv), storing dK, dV. With
// kShares an item is (query head, key block) (heads = BH): it runs over that query head only
// and stores its fp32 share of dK (scaled) and dV at part[bh] and part[BH + bh] ([BH, Nk, D]
// each), which dkdv_reduce_kernel sums over each group.
// Whether the items address the tile loads of whole tiles as a scalar base plus a fixed
// per-lane offset (no per-load VALU address arithmetic). Measured at config 3's shape: head_dim
// 128 causal 1.5% faster, 96 5%; head_dim 256 and the head_dim-64 layout (also used at 32)
// 0.5-2% slower, so those keep the per-lane addresses.
template <int D>
constexpr bool bwd_scalar_tile_base() {
    return D == 128 || D == 96;
}
// Whether the items store their output rows through LDS (store_rows_staged: whole contiguous
// rows per store instruction). Not at head_dim 128, where the staging code makes the kernel
// spill at its 256-register budget and measured no faster.
template <int D>
constexpr bool bwd_staged_store() {
    return D != 128;
}
template <int D>
constexpr int dkdv_lds() {  // two sets of Q tile, dO tile and 32 (L, D) rows
    return 2 * (2 * (32 / TileGroups<D>::kRows) * TileGroups<D>::kBytes + 32 * 8);
}
template <typename T, int D, bool kShares>
__device__ __forceinline__ void dkdv_lds_tiles(const uint16_t* __restrict__ Q,
                                          const uint16_t* __restrict__ K,
                                          const uint16_t* __restrict__ V,
                                          const float2* __restrict__ LD,
                                          const uint16_t* __restrict__ dO,
                                          uint16_t* __restrict__ dK, uint16_t* __restrict__ dV,
                                          int Nq, int Nk, int coff, int group, int Npad,
                                          int heads, float c, float scale, int causal, int bid,
                                          unsigned char* smem, float* __restrict__ part,
                                          int nkb_items, int order) {
    using G = TileGroups<D>;
    constexpr int BN = 128;  // keys per workgroup (32 per wave)
    constexpr int BM = 32;   // query rows per block
    constexpr int GRP = G::kBytes;
    constexpr int QT = (BM / G::kRows) * GRP;
    constexpr int SET = 2 * QT + BM * 8;  // Q tile, dO tile, 32 x (L, D)
    constexpr int kLoadsPerWave = BM / G::kRows * G::kHalves / 4;  // per 32-row tile
    constexpr int NDT = D / 32;                                   // 32-column tiles of dK, dV
    static_assert(2 * SET == dkdv_lds<D>(), "LDS size");
    using frag = typename Elem<T>::frag;

    int hi, kb;  // item head, key block
    item_order(__builtin_amdgcn_readfirstlane(bid), heads, nkb_items, order & 1, hi, kb);
    const int bkv = kShares ? hi / group : hi;    // key/value head
    const int bq0 = kShares ? hi : hi * group;    // first query head of the item
    const int qheads = kShares ? 1 : group;       // query heads of the item
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l32 = lane & 31;
    const int g2 = lane >> 5;

    const size_t kv_head = static_cast<size_t>(bkv) * Nk * D;  // K, V, dK, dV
    const int kwg = kb * BN;
    const int k0 = kwg + wave * 32;
    const int key = k0 + l32;
    const bool key_ok = key < Nk;

    frag kf[D / 16];
    frag vf[D / 16];
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
        u32x4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
        if (key_ok) {
            kv = ld16(K + kv_head + static_cast<size_t>(key) * D + 16 * ks + 8 * g2);
            vv = ld16(V + kv_head + static_cast<size_t>(key) * D + 16 * ks + 8 * g2);
        }
        kf[ks] = as_frag<T>(kv);
        vf[ks] = as_frag<T>(vv);
    }

    // Query blocks [qb_begin, nqb) of each query head of the item, as one sequence of n_it
    // iterations (it -> head bq0 + it / span, block qb_begin + it % span); with a causal mask
    // the blocks before the first query that sees key kwg are skipped. qb_begin < nqb because
    // that query is below Nq.
    const int nqb = Npad / BM;
    const int qb_begin = causal ? max(0, kwg - coff) / BM : 0;
    const int span = nqb - qb_begin;
    const int n_it = qheads * span;

    const int ld_row = G::ld_row(lane);
    const int ld_col = G::ld_col(lane);
    // Byte offset of this lane's 16 bytes in a load of group `wave` (rows from the tile's
    // first row): the loads of whole tiles add only scalar offsets to it.
    const unsigned ld_voff = static_cast<unsigned>(((G::kRows * wave + ld_row) * D + ld_col) * 2);
    auto load_block = [&](int it, int b) {
        const int bh = bq0 + it / span;
        const int r0 = (qb_begin + it % span) * BM;
        const size_t q_head = static_cast<size_t>(bh) * Nq * D;
        const uint16_t* Qh = Q + q_head;
        const uint16_t* Oh = dO + q_head;
        const float* LDh = reinterpret_cast<const float*>(LD + static_cast<size_t>(bh) * Npad);
        unsigned char* set = smem + b * SET;
        if (bwd_scalar_tile_base<D>() && r0 + BM <= Nq) {
            // Whole tile inside Q / dO: a scalar base per load, the fixed per-lane offset ld_voff.
#pragma unroll
            for (int i = 0; i < kLoadsPerWave; ++i) {
                const int grp = wave + 4 * (i / G::kHalves);
                const int half = i % G::kHalves;
                const size_t sofs =
                    static_cast<size_t>(r0 + 4 * G::kRows * (i / G::kHalves)) * D + 128 * half;
                const int dst = grp * GRP + half * 1024;
                lds_dma16_async_s(Qh + sofs, ld_voff, set + dst);
                lds_dma16_async_s(Oh + sofs, ld_voff, set + QT + dst);
            }
        } else {
#pragma unroll
            for (int i = 0; i < kLoadsPerWave; ++i) {
                const int grp = wave + 4 * (i / G::kHalves);
                const int half = i % G::kHalves;
                const int row = min(r0 + G::kRows * grp + ld_row, Nq - 1);
                const size_t src = static_cast<size_t>(row) * D + 128 * half + ld_col;
                const int dst = grp * GRP + half * 1024;
                lds_dma16_async(Qh + src, set + dst);
                lds_dma16_async(Oh + src, set + QT + dst);
            }
        }
        if (wave == 3) lds_dma4_async(LDh + 2 * r0 + lane, set + 2 * QT);
    };
    const int row_base[2] = {G::row_base(lane, 0), G::row_base(lane, 1)};
    const int tr_off = G::tr_off(lane);

    f32x16 dk[D / 32];
    f32x16 dv[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        dk[dt] = f32x16{};
        dv[dt] = f32x16{};
    }
    const float cs = fmaxf(c, kFltMin);

    load_block(0, 0);
    int b = 0;
    for (int it = 0; it < n_it; ++it, b ^= 1) {
        const int q0 = (qb_begin + it % span) * BM;
        __builtin_amdgcn_s_waitcnt(0);  // block it is in LDS
        __syncthreads();                // ... for every wave; block it - 1 is no longer read
        const unsigned char* qt = smem + b * SET;
        const unsigned char* ot = qt + QT;
        const float2* ldv = reinterpret_cast<const float2*>(qt + 2 * QT);
        const float* ldf = reinterpret_cast<const float*>(ldv);  // neg_d_rows: 32 L, then 32 -D

        // S = Q K^T and dP = dO V^T: rows = queries, lane = key. Operand i (i even: Q, odd: dO;
        // k-step i / 2) is read kAhead MFMAs before its product; the scheduling fences keep the
        // compiler from undoing that order.
        f32x16 s = f32x16{};
        f32x16 dp = f32x16{};
        if constexpr (neg_d_rows<D>()) {
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const f32x4 nd = *reinterpret_cast<const f32x4*>(&ldf[32 + 8 * a + 4 * g2]);
                dp[4 * a + 0] = nd[0];
                dp[4 * a + 1] = nd[1];
                dp[4 * a + 2] = nd[2];
                dp[4 * a + 3] = nd[3];
            }
        }
        {
            constexpr int kAhead = 3;
            constexpr int kMma = 2 * (D / 16);
            static_assert(kAhead <= kMma, "operands read ahead within the chain");
            frag fa[kMma];
            auto operand = [&](int k) {
                const int ks = k >> 1;
                return as_frag<T>(ld16((k & 1 ? ot : qt) + row_base[ks & 1] + G::k_off(ks)));
            };
#pragma unroll
            for (int i = 0; i < kMma; ++i) {
                if (i == 0) {
#pragma unroll
                    for (int k = 0; k < kAhead; ++k) fa[k] = operand(k);
                }
                if (i + kAhead < kMma) fa[i + kAhead] = operand(i + kAhead);
                if (i & 1)
                    dp = Elem<T>::mma(fa[i], vf[i >> 1], dp);
                else
                    s = Elem<T>::mma(fa[i], kf[i >> 1], s);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if ((causal && k0 + 31 > q0 + coff) || k0 + 31 >= Nk) {
            const int lim = !key_ok ? 1 << 30 : (causal ? key - coff - q0 - 4 * g2 : -1);
#pragma unroll
            for (int r = 0; r < 16; ++r)
                s[r] = (8 * (r >> 2) + (r & 3) < lim) ? -INFINITY : s[r];
        }
        // Next block's tile loads. Issued here, after the S / dP MFMAs: a load waits at issue
        // while the CU's vector memory path drains the other waves' loads, and here that wait
        // overlaps the MFMAs in flight; before them it delays the MFMAs, after the P / dS
        // arithmetic it delays the dV / dK MFMAs (both measured slower).
        if (it + 1 < n_it) load_block(it + 1, b ^ 1);
        frag bp[2], bs[2];
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            if constexpr (neg_d_rows<D>()) {
                const f32x4 lv = *reinterpret_cast<const f32x4*>(&ldf[8 * a + 4 * g2]);
#pragma unroll
                for (int k2 = 0; k2 < 4; ++k2) {
                    const int r = 4 * a + k2;
                    const float p = fast_exp2(fmaf(s[r], cs, -lv[k2]));
                    s[r] = p;
                    dp[r] = p * dp[r];  // the dP chain started from -D
                }
            } else {
                const f32x4 x = *reinterpret_cast<const f32x4*>(&ldv[8 * a + 4 * g2]);
                const f32x4 y = *reinterpret_cast<const f32x4*>(&ldv[8 * a + 4 * g2 + 2]);
                const float lv[4] = {x[0], x[2], y[0], y[2]};
                const float dd[4] = {x[1], x[3], y[1], y[3]};
#pragma unroll
                for (int k2 = 0; k2 < 4; ++k2) {
                    const int r = 4 * a + k2;
                    const float p = fast_exp2(fmaf(s[r], cs, -lv[k2]));
                    s[r] = p;
                    dp[r] = p * (dp[r] - dd[k2]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            bp[j] = pack_frag<T>(s[8 * j + 0], s[8 * j + 1], s[8 * j + 2], s[8 * j + 3],
                                 s[8 * j + 4], s[8 * j + 5], s[8 * j + 6], s[8 * j + 7]);
            bs[j] = pack_frag<T>(dp[8 * j + 0], dp[8 * j + 1], dp[8 * j + 2], dp[8 * j + 3],
                                 dp[8 * j + 4], dp[8 * j + 5], dp[8 * j + 6], dp[8 * j + 7]);
        }
        // dV^T += dO^T P and dK^T += Q^T dS (k = the block's 32 query rows). Operand i
        // (j = i / 8, dt = (i / 2) % 4; even: dO^T, odd: Q^T) is read kAhead MFMAs ahead.
        {
            constexpr int kAhead = 3;
            constexpr int kMma = 4 * NDT;  // (dV, dK) x 2 query halves x NDT column tiles
            static_assert(kAhead <= kMma, "operands read ahead within the chain");
            frag fa[kMma];
            auto operand = [&](int i) {
                const unsigned char* a = (i & 1 ? qt : ot) + tr_off +
                                         (i / (2 * NDT)) * G::kTrRows16 +
                                         G::dtile_off((i >> 1) % NDT);
                return tr_frag_at<T>(a, a + G::kTrHigh);
            };
#pragma unroll
            for (int i = 0; i < kMma; ++i) {
                if (i == 0) {
#pragma unroll
                    for (int k = 0; k < kAhead; ++k) fa[k] = operand(k);
                }
                if (i + kAhead < kMma) fa[i + kAhead] = operand(i + kAhead);
                const int j = i / (2 * NDT);
                const int dt = (i >> 1) % NDT;
                if (i & 1)
                    dk[dt] = Elem<T>::mma(fa[i], bs[j], dk[dt]);
                else
                    dv[dt] = Elem<T>::mma(fa[i], bp[j], dv[dt]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    if (kShares && key_ok) {
        float* krow = part + (static_cast<size_t>(hi) * Nk + key) * D;
        float* vrow = part + (static_cast<size_t>(heads + hi) * Nk + key) * D;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const int d = 32 * dt + 8 * a + 4 * g2;
                f32x4 wk, wv;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    wk[u] = dk[dt][4 * a + u] * scale;
                    wv[u] = dv[dt][4 * a + u];
                }
                st16(krow + d, __builtin_bit_cast(u32x4, wk));
                st16(vrow + d, __builtin_bit_cast(u32x4, wv));
            }
        }
    } else if constexpr (!kShares && bwd_staged_store<D>()) {
        // dK and dV rows through LDS (the tile sets, free once every wave is past its last
        // block), one after the other in the wave's area.
        static_assert(4 * staged_rows_bytes<D>() <= dkdv_lds<D>(), "staging area");
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        unsigned char* stg = smem + wave * staged_rows_bytes<D>();
        store_rows_staged<T, D>(dk, scale, stg, dK + kv_head, k0, Nk);
        store_rows_staged<T, D>(dv, 1.0f, stg, dV + kv_head, k0, Nk);
    } else if (!kShares && key_ok) {
        uint16_t* krow = dK + kv_head + static_cast<size_t>(key) * D;
        uint16_t* vrow = dV + kv_head + static_cast<size_t>(key) * D;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const int d = 32 * dt + 8 * a + 4 * g2;
                u32x2 wk, wv;
                wk[0] = Elem<T>::pack2(dk[dt][4 * a + 0] * scale, dk[dt][4 * a + 1] * scale);
                wk[1] = Elem<T>::pack2(dk[dt][4 * a + 2] * scale, dk[dt][4 * a + 3] * scale);
                wv[0] = Elem<T>::pack2(dv[dt][4 * a + 0], dv[dt][4 * a + 1]);
                wv[1] = Elem<T>::pack2(dv[dt][4 * a + 2], dv[dt][4 * a + 3]);
                st8(krow + d, wk);
                st8(vrow + d, wv);
            }
        }
    }
}

// Query-stationary part of work item `bid` of BH * nqb (rank 0 has the most work with a causal
// mask; the order of the ids is item_order's, bit 1 of `order`); smem holds at least
// dq_lds<D>() bytes.
template <int D>
constexpr int dq_lds() {  // two sets of K tile and V tile
    return 2 * 2 * (32 / TileGroups<D>::kRows) * TileGroups<D>::kBytes;
}
template <typename T, int D>
__device__ __forceinline__ void dq_lds_tiles(const uint16_t* __restrict__ Q,
                                        const uint16_t* __restrict__ K,
                                        const uint16_t* __restrict__ V,
                                        const float2* __restrict__ LD,
                                        const uint16_t* __restrict__ dO,
                                        uint16_t* __restrict__ dQ, int Nq, int Nk, int coff,
                                        int group, int Npad, int nqb, int BH, float c,
                                        float scale, int causal, int bid, unsigned char* smem,
                                        int order) {
    using G = TileGroups<D>;
    constexpr int BM = 128;  // query rows per workgroup (32 per wave)
    constexpr int BN = 32;   // keys per block
    constexpr int GRP = G::kBytes;
    constexpr int KT = (BN / G::kRows) * GRP;
    constexpr int SET = 2 * KT;  // K tile, V tile
    constexpr int kLoadsPerWave = BN / G::kRows * G::kHalves / 4;
    constexpr int NDT = D / 32;  // 32-column tiles of dQ
    static_assert(2 * SET == dq_lds<D>(), "LDS size");
    using frag = typename Elem<T>::frag;

    int bh, rank;
    item_order(__builtin_amdgcn_readfirstlane(bid), BH, nqb, (order >> 1) & 1, bh, rank);
    const int qb = causal ? nqb - 1 - rank : rank;  // causal: longest query blocks first
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l32 = lane & 31;
    const int g2 = lane >> 5;

    const size_t head = static_cast<size_t>(bh) * Nq * D;             // Q, dO, dQ
    const size_t kv_head = static_cast<size_t>(bh / group) * Nk * D;  // K, V
    const uint16_t* Kh = K + kv_head;
    const uint16_t* Vh = V + kv_head;
    const int q0 = qb * BM + wave * 32;  // first query row of this wave
    const int q = q0 + l32;              // query row owned by this lane
    const bool q_ok = q < Nq;

    // Q^T and dO^T as B operands of S^T = K Q^T and dP^T = V dO^T (k = d).
    frag qf[D / 16];
    frag of[D / 16];
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
        u32x4 qv = {0u, 0u, 0u, 0u}, ov = {0u, 0u, 0u, 0u};
        if (q_ok) {
            qv = ld16(Q + head + static_cast<size_t>(q) * D + 16 * ks + 8 * g2);
            ov = ld16(dO + head + static_cast<size_t>(q) * D + 16 * ks + 8 * g2);
        }
        qf[ks] = as_frag<T>(qv);
        of[ks] = as_frag<T>(ov);
    }
    // (L log2 e, D) of this lane's query (stored as -D in the neg_d_rows layout); padding rows
    // give P = 0.
    float2 ldq = make_float2(INFINITY, 0.0f);
    if (q < Npad) {
        if constexpr (neg_d_rows<D>()) {
            const float* blk = reinterpret_cast<const float*>(LD) +
                               (static_cast<size_t>(bh) * Npad + (q & ~31)) * 2 + (q & 31);
            ldq = make_float2(blk[0], -blk[32]);
        } else {
            ldq = LD[static_cast<size_t>(bh) * Npad + q];
        }
    }

    const int ld_row = G::ld_row(lane);
    const int ld_col = G::ld_col(lane);
    const unsigned ld_voff = static_cast<unsigned>(((G::kRows * wave + ld_row) * D + ld_col) * 2);
    auto load_block = [&](int kb, int b) {
        const int r0 = kb * BN;
        unsigned char* set = smem + b * SET;
        if (bwd_scalar_tile_base<D>() && r0 + BN <= Nk) {
            // Whole tile inside K / V: a scalar base per load, the fixed per-lane offset ld_voff.
#pragma unroll
            for (int i = 0; i < kLoadsPerWave; ++i) {
                const int grp = wave + 4 * (i / G::kHalves);
                const int half = i % G::kHalves;
                const size_t sofs =
                    static_cast<size_t>(r0 + 4 * G::kRows * (i / G::kHalves)) * D + 128 * half;
                const int dst = grp * GRP + half * 1024;
                lds_dma16_async_s(Kh + sofs, ld_voff, set + dst);
                lds_dma16_async_s(Vh + sofs, ld_voff, set + KT + dst);
            }
        } else {
#pragma unroll
            for (int i = 0; i < kLoadsPerWave; ++i) {
                const int grp = wave + 4 * (i / G::kHalves);
                const int half = i % G::kHalves;
                const int row = min(r0 + G::kRows * grp + ld_row, Nk - 1);
                const size_t src = static_cast<size_t>(row) * D + 128 * half + ld_col;
                const int dst = grp * GRP + half * 1024;
                lds_dma16_async(Kh + src, set + dst);
                lds_dma16_async(Vh + src, set + KT + dst);
            }
        }
    };
    const int row_base[2] = {G::row_base(lane, 0), G::row_base(lane, 1)};
    const int tr_off = G::tr_off(lane);

    f32x16 acc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) acc[dt] = f32x16{};
    const float cs = fmaxf(c, kFltMin);
    const int kv_end = causal ? min(Nk, (qb + 1) * BM + coff) : Nk;
    const int nkb = (kv_end + BN - 1) / BN;

    load_block(0, 0);
    int b = 0;
    for (int kb = 0; kb < nkb; ++kb, b ^= 1) {
        const int key0 = kb * BN;
        __builtin_amdgcn_s_waitcnt(0);  // block kb is in LDS
        __syncthreads();                // ... for every wave; block kb - 1 is no longer read
        if (kb + 1 < nkb) load_block(kb + 1, b ^ 1);
        const unsigned char* kt = smem + b * SET;
        const unsigned char* vt = kt + KT;

        // S^T = K Q^T and dP^T = V dO^T: rows = keys, lane = query. Operand i (even: K, odd:
        // V; k-step i / 2) is read kAhead MFMAs before its product.
        f32x16 s = f32x16{};
        f32x16 dp = f32x16{};
        if constexpr (neg_d_rows<D>()) {
#pragma unroll
            for (int r = 0; r < 16; ++r) dp[r] = -ldq.y;
        }
        {
            constexpr int kAhead = 3;
            constexpr int kMma = 2 * (D / 16);
            static_assert(kAhead <= kMma, "operands read ahead within the chain");
            frag fa[kMma];
            auto operand = [&](int k) {
                const int ks = k >> 1;
                return as_frag<T>(ld16((k & 1 ? vt : kt) + row_base[ks & 1] + G::k_off(ks)));
            };
#pragma unroll
            for (int i = 0; i < kMma; ++i) {
                if (i == 0) {
#pragma unroll
                    for (int k = 0; k < kAhead; ++k) fa[k] = operand(k);
                }
                if (i + kAhead < kMma) fa[i + kAhead] = operand(i + kAhead);
                if (i & 1)
                    dp = Elem<T>::mma(fa[i], of[i >> 1], dp);
                else
                    s = Elem<T>::mma(fa[i], qf[i >> 1], s);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (key0 + BN > Nk || (causal && key0 + BN - 1 > q0 + coff)) {
            const int lim = min(Nk, causal ? q + 1 + coff : Nk) - key0 - 4 * g2;
#pragma unroll
            for (int r = 0; r < 16; ++r)
                s[r] = (8 * (r >> 2) + (r & 3) < lim) ? s[r] : -INFINITY;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float p = fast_exp2(fmaf(s[r], cs, -ldq.x));
            if constexpr (neg_d_rows<D>())
                s[r] = p * dp[r];  // dS^T (the dP chain started from -D)
            else
                s[r] = p * (dp[r] - ldq.y);  // dS^T
        }
        // dQ^T += K^T dS^T (k = the block's 32 keys; K^T by transpose reads). Operand i
        // (j = i / 4, dt = i % 4) is read kAhead MFMAs ahead.
        {
            frag bsf[2];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bsf[j] = pack_frag<T>(s[8 * j + 0], s[8 * j + 1], s[8 * j + 2], s[8 * j + 3],
                                      s[8 * j + 4], s[8 * j + 5], s[8 * j + 6], s[8 * j + 7]);
            constexpr int kMma = 2 * NDT;  // 2 key halves x NDT column tiles
            constexpr int kAhead = kMma < 3 ? kMma : 3;  // 2 MFMAs at head_dim 32
            frag fa[kMma];
            auto operand = [&](int i) {
                const unsigned char* a =
                    kt + tr_off + (i / NDT) * G::kTrRows16 + G::dtile_off(i % NDT);
                return tr_frag_at<T>(a, a + G::kTrHigh);
            };
#pragma unroll
            for (int i = 0; i < kMma; ++i) {
                if (i == 0) {
#pragma unroll
                    for (int k = 0; k < kAhead; ++k) fa[k] = operand(k);
                }
                if (i + kAhead < kMma) fa[i + kAhead] = operand(i + kAhead);
                acc[i % NDT] = Elem<T>::mma(fa[i], bsf[i / NDT], acc[i % NDT]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    if constexpr (bwd_staged_store<D>()) {
        // dQ rows through LDS (the tile sets, free once every wave is past its last block).
        static_assert(4 * staged_rows_bytes<D>() <= dq_lds<D>(), "staging area");
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        store_rows_staged<T, D>(acc, scale, smem + wave * staged_rows_bytes<D>(), dQ + head, q0,
                                Nq);
    } else if (q_ok) {
        uint16_t* row = dQ + head + static_cast<size_t>(q) * D;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                u32x2 w;
                w[0] = Elem<T>::pack2(acc[dt][4 * a + 0] * scale, acc[dt][4 * a + 1] * scale);
                w[1] = Elem<T>::pack2(acc[dt][4 * a + 2] * scale, acc[dt][4 * a + 3] * scale);
                st8(row + 32 * dt + 8 * a + 4 * g2, w);
            }
        }
    }
}

// One launch for both passes (they are independent once delta_ld_kernel has run), as a pool
// of resident workgroups that take work items from kNumXcd queues. Queue x belongs to XCD x:
// even XCDs take the dkdv items (128 keys each, BHkv * nkb of them), odd XCDs the dq items
// (128 query rows each, BH * nqb), each XCD the ids congruent to x / 2 modulo 4, in increasing
// order: every XCD keeps its own heads (their tiles stay in its L2), in the item order `order`
// selects (bit 0: dkdv items head-major, bit 1: dq items head-major; item_order). A workgroup
// whose own queue is empty takes from the next XCD's queue, then from the others, and exits
// when every queue is empty. At head_dim 128 the dq items need about 80% of the dkdv items'
// time (config 3: 84.5 against 105 µs of block loop per item in an instrumented build), so
// without the hand-over the dq XCDs would idle for the last fifth of the launch.
// Counters are cleared by delta_ld_kernel; every workgroup ends after at most one failed pass
// over the queues, so the launch always drains.
__device__ __forceinline__ int xcc_id() {
    return static_cast<int>(__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20)) &
           (kNumXcd - 1);  // HW_REG_XCC_ID[3:0]
}

// Resident workgroups per CU: two, except at head_dim 256, whose dK/dV accumulators and K/V
// operands need the registers of a whole SIMD lane, and at head_dim 32, whose items fit 128
// registers, so four share a CU (causal B=2 H=16 N=4096: 217.5 -> 206.8 us; config 2's shape at
// head_dim 32: 219.7 -> 196.4 us). Three at head_dim 64 would need 168 registers; the compiler
// then spills and the launch is no faster.
template <int D>
constexpr int bwd_fused_wgs_per_cu() {
    return D >= 256 ? 1 : D == 32 ? 4 : 2;
}

template <typename T, int D, bool kShares>
__global__ void __launch_bounds__(256, (bwd_fused_wgs_per_cu<D>()))
    bwd_fused_kernel(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                    const uint16_t* __restrict__ V, const float2* __restrict__ LD,
                    const uint16_t* __restrict__ dO, uint16_t* __restrict__ dQ,
                    uint16_t* __restrict__ dK, uint16_t* __restrict__ dV, int Nq, int Nk,
                    int coff, int group, int Npad, int nqb, int nkb, int BH, float c,
                    float scale, int causal, int* __restrict__ queues, float* __restrict__ part,
                    int order) {
    constexpr int kLds = dkdv_lds<D>() > dq_lds<D>() ? dkdv_lds<D>() : dq_lds<D>();
    __shared__ __attribute__((aligned(1024))) unsigned char smem[kLds];
    __shared__ int item;
    const int dkdv_heads = kShares ? BH : BH / group;  // see dkdv_lds_tiles
    const int n_dq = BH * nqb;
    const int n_dkdv = dkdv_heads * nkb;
    const int home = xcc_id();
    for (;;) {
        if (threadIdx.x == 0) {
            int got = -1;
            for (int t = 0; t < kNumXcd && got < 0; ++t) {
                const int qx = (home + t) & (kNumXcd - 1);
                const int j = qx >> 1;
                const int n = (qx & 1) ? n_dq : n_dkdv;
                const int len = n > j ? (n - j + 3) / 4 : 0;  // ids j, j + 4, ... below n
                if (__hip_atomic_load(&queues[qx], __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) >= len)
                    continue;  // empty: no read-modify-write on a drained counter
                const int k = atomicAdd(&queues[qx], 1);
                if (k < len) got = ((qx & 1) << 30) | (4 * k + j);
            }
            item = got;
        }
        __syncthreads();
        const int it = item;
        __syncthreads();  // every wave has read `item` before thread 0 writes the next one
        if (it < 0) break;
        const int id = it & ((1 << 30) - 1);
        if (it >> 30)
            dq_lds_tiles<T, D>(Q, K, V, LD, dO, dQ, Nq, Nk, coff, group, Npad, nqb, BH, c, scale,
                          causal, id, smem, order);
        else
            dkdv_lds_tiles<T, D, kShares>(Q, K, V, LD, dO, dK, dV, Nq, Nk, coff, group, Npad,
                                     dkdv_heads, c, scale, causal, id, smem, part, nkb, order);
        __syncthreads();  // the next item reuses the LDS tiles
    }
}

// dK, dV of each key/value head from the fp32 shares of its `group` query heads (the
// part != nullptr mode of dkdv_lds_tiles): part holds dK shares [BH, Nk, D], then dV shares. Eight
// elements per thread; sums in fp32 in head order, one rounding to T.
template <typename T>
__global__ void __launch_bounds__(256)
    dkdv_reduce_kernel(const float* __restrict__ part, uint16_t* __restrict__ dK,
                       uint16_t* __restrict__ dV, long long kv_elems, long long head_elems,
                       int group) {
    const long long e = (static_cast<long long>(blockIdx.x) * 256 + threadIdx.x) * 8;
    if (e >= kv_elems) return;
    const long long bkv = e / head_elems;
    const long long off = e - bkv * head_elems;
    const long long q_elems = kv_elems * group;  // BH * Nk * D
#pragma unroll
    for (int which = 0; which < 2; ++which) {
        const float* src = part + which * q_elems + (bkv * group) * head_elems + off;
        f32x4 a = __builtin_bit_cast(f32x4, ld16(src));
        f32x4 b = __builtin_bit_cast(f32x4, ld16(src + 4));
        for (int g = 1; g < group; ++g) {
            a += __builtin_bit_cast(f32x4, ld16(src + g * head_elems));
            b += __builtin_bit_cast(f32x4, ld16(src + g * head_elems + 4));
        }
        u32x4 w;
        w[0] = Elem<T>::pack2(a[0], a[1]);
        w[1] = Elem<T>::pack2(a[2], a[3]);
        w[2] = Elem<T>::pack2(b[0], b[1]);
        w[3] = Elem<T>::pack2(b[2], b[3]);
        st16((which ? dV : dK) + e, w);
    }
}

}  // namespace dev

namespace detail {

namespace {

// Query/key extents of one launch (see the shape note at the top of this file).
struct BwdShape {
    int BH;     // query heads over the batch
    int Nq;     // query rows per head
    int Nk;     // key rows per key/value head
    int group;  // query heads per key/value head
};

// Generic path (fp32, and head_dim 32 / 64 / 96 / 256): delta, dq_kernel, dkdv_kernel.
template <typename T, int D>
FlashAttentionError run_backward_two_pass(const T* Q, const T* K, const T* V, const T* O,
                                          const float* L, const T* dO, T* dQ, T* dK, T* dV,
                                          const BwdShape& sh, float scale, bool causal,
                                          hipStream_t stream) {
    using E = typename dev::Mma<T>::elem;
    const E* q = reinterpret_cast<const E*>(Q);
    const E* k = reinterpret_cast<const E*>(K);
    const E* v = reinterpret_cast<const E*>(V);
    const E* o = reinterpret_cast<const E*>(O);
    const E* go = reinterpret_cast<const E*>(dO);
    const int coff = sh.Nk - sh.Nq;
    const int BHkv = sh.BH / sh.group;

    const long long rows = static_cast<long long>(sh.BH) * sh.Nq;
    StreamWorkspace ws(stream, true);
    FlashAttentionError err = ws.alloc(static_cast<size_t>(rows) * sizeof(float));
    if (err != FlashAttentionError::SUCCESS) return err;
    float* delta = static_cast<float*>(ws.get());

    constexpr int LPR = dev::delta_lanes<D * static_cast<int>(sizeof(E)) / 16>();
    const long long dthreads = rows * LPR;
    const long long dblocks = (dthreads + 255) / 256;
    if (dblocks > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
    ProfileEvents tok = profile_kernel<T, D>("backward_delta");
    launch_kernel(tok, (dev::delta_kernel<T, D>), dim3(static_cast<unsigned>(dblocks)), dim3(256),
                       0, stream, go, o, delta, rows);
    err = from_hip(hipGetLastError());
    if (err != FlashAttentionError::SUCCESS) return err;

    const float c = scale * dev::kLog2e;
    using QCfg = dev::DqCfg<T, D>;
    using KCfg = dev::DkvCfg<T, D>;
    const int nqb = (sh.Nq + QCfg::BM - 1) / QCfg::BM;
    const int nkb = (sh.Nk + KCfg::BN - 1) / KCfg::BN;
    const long long qblocks = static_cast<long long>(nqb) * sh.BH;
    const long long kblocks = static_cast<long long>(nkb) * BHkv;
    if (qblocks + kblocks > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
    // Both grids together fit in one round of workgroups: one launch, so that the dq and dkdv
    // items run side by side instead of each half-filling the GPU in turn (up to head_dim 128:
    // the two bodies' LDS arrays add up).
    if constexpr (D <= 128) {
        if (qblocks + kblocks <= compute_units()) {
            tok = profile_kernel<T, D>("backward_dq_dkdv");
            launch_kernel(tok, (dev::dq_dkdv_kernel<T, D>),
                               dim3(static_cast<unsigned>(qblocks + kblocks)), dim3(256), 0,
                               stream, q, k, v, L, go, delta, reinterpret_cast<E*>(dQ),
                               reinterpret_cast<E*>(dK), reinterpret_cast<E*>(dV), sh.Nq, sh.Nk,
                               coff, sh.group, nqb, nkb, static_cast<int>(kblocks), c, scale,
                               causal ? 1 : 0);
            return from_hip(hipGetLastError());
        }
    }
    tok = profile_kernel<T, D>("backward_dq");
    launch_kernel(tok, (dev::dq_kernel<T, D>), dim3(static_cast<unsigned>(qblocks)),
                       dim3(QCfg::kThreads), 0, stream, q, k, v, L, go, delta,
                       reinterpret_cast<E*>(dQ), sh.Nq, sh.Nk, coff, sh.group, nqb, c, scale,
                       causal ? 1 : 0);
    err = from_hip(hipGetLastError());
    if (err != FlashAttentionError::SUCCESS) return err;
    tok = profile_kernel<T, D>("backward_dkdv");
    launch_kernel(tok, (dev::dkdv_kernel<T, D>), dim3(static_cast<unsigned>(kblocks)),
                       dim3(KCfg::kThreads), 0, stream, q, k, v, L, go, delta,
                       reinterpret_cast<E*>(dK), reinterpret_cast<E*>(dV), sh.Nq, sh.Nk, coff,
                       sh.group, nkb, c, scale, causal ? 1 : 0);
    err = from_hip(hipGetLastError());
    return err;
}

// Path for fp16 / bf16 at head_dim 128 and 64: delta_ld_kernel, then bwd_fused_kernel (dq and
// dkdv in one launch).
template <typename T, int D>
FlashAttentionError run_backward_fused(const T* Q, const T* K, const T* V, const T* O,
                                               const float* L, const T* dO, T* dQ, T* dK, T* dV,
                                               const BwdShape& sh, float scale, bool causal,
                                               hipStream_t stream) {
    const int Npad = (sh.Nq + 31) / 32 * 32;
    const long long rows_pad = static_cast<long long>(sh.BH) * Npad;
    StreamWorkspace ws(stream, true);
    // (L log2 e, D) rows, then the kNumXcd work-queue counters of bwd_fused_kernel
    const size_t ld_bytes = static_cast<size_t>(rows_pad) * sizeof(float2);
    FlashAttentionError err = ws.alloc(ld_bytes + dev::kNumXcd * sizeof(int));
    if (err != FlashAttentionError::SUCCESS) return err;
    float2* ld = static_cast<float2*>(ws.get());
    int* queues = reinterpret_cast<int*>(static_cast<unsigned char*>(ws.get()) + ld_bytes);

    const long long dblocks = (rows_pad * dev::delta_lanes<D / 8>() + 255) / 256;
    const int nqb = (sh.Nq + 127) / 128;
    const int nkb = (sh.Nk + 127) / 128;
    // Grouped heads: one dkdv item per (query head, key block) with fp32 shares of dK, dV that a
    // second kernel sums, when the shares fit in kMaxShareBytes; an item per (key/value head,
    // key block) would run `group` times longer and leave the launch's tail to a few of them.
    constexpr long long kMaxShareBytes = 2LL << 30;
    const long long share_bytes = 2LL * sh.BH * sh.Nk * D * static_cast<long long>(sizeof(float));
    const bool shares = sh.group > 1 && share_bytes <= kMaxShareBytes;
    const long long qblocks = static_cast<long long>(nqb) * sh.BH;
    const long long kblocks = static_cast<long long>(nkb) * (shares ? sh.BH : sh.BH / sh.group);
    if (dblocks > 0x7fffffffLL || qblocks + kblocks > 0x7fffffffLL)
        return FlashAttentionError::INVALID_DIMENSION;
    const float c = scale * dev::kLog2e;
    const uint16_t* q = reinterpret_cast<const uint16_t*>(Q);
    const uint16_t* k = reinterpret_cast<const uint16_t*>(K);
    const uint16_t* v = reinterpret_cast<const uint16_t*>(V);
    const uint16_t* go = reinterpret_cast<const uint16_t*>(dO);

    ProfileEvents tok = profile_kernel<T, D>("backward_delta");
    launch_kernel(tok, (dev::delta_ld_kernel<T, D>), dim3(static_cast<unsigned>(dblocks)), dim3(256),
                       0, stream, go, reinterpret_cast<const uint16_t*>(O), L, ld, sh.Nq, Npad,
                       rows_pad, queues);
    err = from_hip(hipGetLastError());
    if (err != FlashAttentionError::SUCCESS) return err;

    StreamWorkspace share_ws(stream);
    float* part = nullptr;
    if (shares) {
        err = share_ws.alloc(static_cast<size_t>(share_bytes));
        if (err != FlashAttentionError::SUCCESS) return err;
        part = static_cast<float*>(share_ws.get());
    }

    // The resident workgroups (one or two per CU) take the qblocks + kblocks work items.
    const long long pool = std::min<long long>(
        qblocks + kblocks, static_cast<long long>(dev::bwd_fused_wgs_per_cu<D>()) * compute_units());
    // dq items head-major always; dkdv items head-major without a causal mask (all of one
    // length: 0.2-0.8% faster at the non-causal shapes measured) or once there are at least
    // eight per resident workgroup (config 5: 4096 items for 512 workgroups), where the tail
    // that a head's late longest items leave is short against the launch.
    const int order = 2 | ((!causal || kblocks >= 8 * pool) ? 1 : 0);
    tok = profile_kernel<T, D>("backward_dq_dkdv");
    auto kernel = shares ? dev::bwd_fused_kernel<T, D, true> : dev::bwd_fused_kernel<T, D, false>;
    launch_kernel(tok, kernel, dim3(static_cast<unsigned>(pool)), dim3(256), 0, stream, q, k, v,
                       ld, go, reinterpret_cast<uint16_t*>(dQ), reinterpret_cast<uint16_t*>(dK),
                       reinterpret_cast<uint16_t*>(dV), sh.Nq, sh.Nk, sh.Nk - sh.Nq, sh.group,
                       Npad, nqb, nkb, sh.BH, c, scale, causal ? 1 : 0, queues, part, order);
    err = from_hip(hipGetLastError());
    if (err != FlashAttentionError::SUCCESS || !shares) return err;

    const long long kv_elems = static_cast<long long>(sh.BH / sh.group) * sh.Nk * D;
    const long long rblocks = (kv_elems / 8 + 255) / 256;
    tok = profile_kernel<T, D>("backward_dkdv_reduce");
    launch_kernel(tok, (dev::dkdv_reduce_kernel<T>), dim3(static_cast<unsigned>(rblocks)),
                       dim3(256), 0, stream, part, reinterpret_cast<uint16_t*>(dK),
                       reinterpret_cast<uint16_t*>(dV), kv_elems,
                       static_cast<long long>(sh.Nk) * D, sh.group);
    return from_hip(hipGetLastError());
}

template <typename T, int D>
FlashAttentionError run_backward_d(const T* Q, const T* K, const T* V, const T* O,
                                   const float* L, const T* dO, T* dQ, T* dK, T* dV,
                                   const BwdShape& sh, float scale, bool causal,
                                   hipStream_t stream) {
    if constexpr (!std::is_same<T, float>::value &&
                  (D == 128 || D == 64 || D == 256 || D == 32 || D == 96))
        return run_backward_fused<T, D>(Q, K, V, O, L, dO, dQ, dK, dV, sh, scale, causal,
                                                stream);
    else
        return run_backward_two_pass<T, D>(Q, K, V, O, L, dO, dQ, dK, dV, sh, scale, causal,
                                           stream);
}

// head_dim dispatch; `extended` admits the head dims beyond the reference's 32 / 64 / 128.
template <typename T>
FlashAttentionError run_backward(const T* Q, const T* K, const T* V, const T* O, const float* L,
                                 const T* dO, T* dQ, T* dK, T* dV, const BwdShape& sh,
                                 int head_dim, bool extended, float scale, bool causal,
                                 hipStream_t stream) {
    switch (head_dim) {
        case 32:
            return run_backward_d<T, 32>(Q, K, V, O, L, dO, dQ, dK, dV, sh, scale, causal,
                                         stream);
        case 64:
            return run_backward_d<T, 64>(Q, K, V, O, L, dO, dQ, dK, dV, sh, scale, causal,
                                         stream);
        case 128:
            return run_backward_d<T, 128>(Q, K, V, O, L, dO, dQ, dK, dV, sh, scale, causal,
                                          stream);
        case 96:
            if (extended)
                return run_backward_d<T, 96>(Q, K, V, O, L, dO, dQ, dK, dV, sh, scale, causal,
                                             stream);
            break;
        case 256:
            if (extended)
                return run_backward_d<T, 256>(Q, K, V, O, L, dO, dQ, dK, dV, sh, scale, causal,
                                              stream);
            break;
    }
    return FlashAttentionError::UNSUPPORTED_HEAD_DIM;
}

}  // namespace

template <typename T>
FlashAttentionError launch_backward(const T* Q, const T* K, const T* V, const T* O,
                                    const float* L, const T* dO, T* dQ, T* dK, T* dV,
                                    int batch_size, int num_heads, int seq_len, int head_dim,
                                    float scale, bool causal, hipStream_t stream) {
    const long long bh = static_cast<long long>(batch_size) * num_heads;
    if (bh > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
    const BwdShape sh{static_cast<int>(bh), seq_len, seq_len, 1};
    return run_backward<T>(Q, K, V, O, L, dO, dQ, dK, dV, sh, head_dim, false, scale, causal,
                           stream);
}

template <typename T>
FlashAttentionError launch_backward_ext(const T* Q, const T* K, const T* V, const T* O,
                                        const float* L, const T* dO, T* dQ, T* dK, T* dV,
                                        int batch_size, int num_heads, int num_kv_heads,
                                        int q_len, int kv_len, int head_dim, float scale,
                                        bool causal, hipStream_t stream) {
    const long long bh = static_cast<long long>(batch_size) * num_heads;
    if (bh > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
    const BwdShape sh{static_cast<int>(bh), q_len, kv_len, num_heads / num_kv_heads};
    return run_backward<T>(Q, K, V, O, L, dO, dQ, dK, dV, sh, head_dim, true, scale, causal,
                           stream);
}

#define CUFLASH_BACKWARD_TYPE(T)                                                              \
    template FlashAttentionError launch_backward<T>(const T*, const T*, const T*, const T*,   \
                                                    const float*, const T*, T*, T*, T*, int,  \
                                                    int, int, int, float, bool, hipStream_t); \
    template FlashAttentionError launch_backward_ext<T>(                                      \
        const T*, const T*, const T*, const T*, const float*, const T*, T*, T*, T*, int, int,  \
        int, int, int, int, float, bool, hipStream_t);
CUFLASH_BACKWARD_TYPE(float)
CUFLASH_BACKWARD_TYPE(__half)
CUFLASH_BACKWARD_TYPE(__hip_bfloat16)
#undef CUFLASH_BACKWARD_TYPE

}  // namespace detail
}  // namespace cuflash
