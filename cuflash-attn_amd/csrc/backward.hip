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

#include "common.hpp"
#include "launch.hpp"
#include "profile.hpp"

#include <cstdlib>

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

// When dq_acc is non-null the kernel also clears the fp32 dQ accumulator of the fused backward
// (the same rows, VEC floats per lane), which saves a separate fill pass over it.
template <typename T, int D>
__global__ void __launch_bounds__(256)
    delta_kernel(const typename Mma<T>::elem* __restrict__ dO,
                 const typename Mma<T>::elem* __restrict__ O, float* __restrict__ Dst,
                 float* __restrict__ dq_acc, long long rows) {
    using E = typename Mma<T>::elem;
    constexpr int VEC = 16 / static_cast<int>(sizeof(E));
    constexpr int LPR = D / VEC;  // lanes per row
    const long long t = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    const long long row = t / LPR;
    const int part = static_cast<int>(t % LPR);
    float s = 0.0f;
    if (row < rows) {
        const size_t off = static_cast<size_t>(row) * D + part * VEC;
        s = dot16<T>(ld16(dO + off), ld16(O + off));
        if (dq_acc) {
#pragma unroll
            for (int i = 0; i < VEC; i += 4) st16(dq_acc + off + i, u32x4{0u, 0u, 0u, 0u});
        }
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
    return (std::is_same<T, float>::value && D == 128) ? 1 : 2;
}

template <typename T, int D>
__global__ void __launch_bounds__(256, (dq_min_waves<T, D>()))
    dq_kernel(const typename Mma<T>::elem* __restrict__ Q,
              const typename Mma<T>::elem* __restrict__ K,
              const typename Mma<T>::elem* __restrict__ V, const float* __restrict__ L,
              const typename Mma<T>::elem* __restrict__ dO, const float* __restrict__ Dl,
              typename Mma<T>::elem* __restrict__ dQ, int N, int nqb, float c, float scale,
              int causal) {
    using M = Mma<T>;
    using E = typename M::elem;
    using frag = typename M::frag;
    using Cfg = DqCfg<T, D>;
    __shared__ __attribute__((aligned(16))) E Ks[Cfg::BN * Cfg::RP];
    __shared__ __attribute__((aligned(16))) E Kc[Cfg::BN * Cfg::CP];
    __shared__ __attribute__((aligned(16))) E Vs[Cfg::BN * Cfg::RP];

    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = lid / nqb;
    const int qb = causal ? nqb - 1 - lid % nqb : lid % nqb;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int l32 = lane & 31;
    const int g2 = lane >> 5;

    const size_t head = static_cast<size_t>(bh) * N * D;
    const int q0 = qb * Cfg::BM + wave * 32;
    const int q = q0 + l32;
    const bool q_ok = q < N;

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
    // Rows past N get L = +inf so that P = exp(S - L) is exactly 0 there.
    const float l2 = q_ok ? L[static_cast<size_t>(bh) * N + q] * kLog2e : INFINITY;
    const float dq_row = q_ok ? Dl[static_cast<size_t>(bh) * N + q] : 0.0f;

    f32x16 acc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) acc[dt] = f32x16{};

    const int kv_end = causal ? min(N, (qb + 1) * Cfg::BM) : N;
    const int nkb = (kv_end + Cfg::BN - 1) / Cfg::BN;
    TileCopy<E, Cfg::BN, D, Cfg::kThreads> kcp, vcp;
    const int col_off = M::col_lane_offset(Cfg::CP);

    if (nkb > 0) {
        kcp.fetch(K + head, N, tid);
        vcp.fetch(V + head, N, tid);
    }
    for (int kb = 0; kb < nkb; ++kb) {
        const int key0 = kb * Cfg::BN;
        __syncthreads();
        kcp.stage(Ks, Cfg::RP, tid);
        kcp.stage(Kc, Cfg::CP, tid);
        vcp.stage(Vs, Cfg::RP, tid);
        __syncthreads();
        if (kb + 1 < nkb) {
            kcp.fetch(K + head + static_cast<size_t>(key0 + Cfg::BN) * D, N - key0 - Cfg::BN, tid);
            vcp.fetch(V + head + static_cast<size_t>(key0 + Cfg::BN) * D, N - key0 - Cfg::BN, tid);
        }
        if (causal && key0 > q0 + 31) continue;

        f32x16 s = f32x16{};
        f32x16 dp = f32x16{};
#pragma unroll
        for (int ks = 0; ks < D / M::KW; ++ks) {
            s = M::mma(M::row_operand(&Ks[l32 * Cfg::RP + M::KW * ks]), qf[ks], s);
            dp = M::mma(M::row_operand(&Vs[l32 * Cfg::RP + M::KW * ks]), of[ks], dp);
        }
        const bool masked = (key0 + Cfg::BN > N) || (causal && key0 + Cfg::BN - 1 > q0);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float p = fast_exp2(fmaf(s[r], c, -l2));
            if (masked) {
                const int key = key0 + 8 * (r >> 2) + 4 * g2 + (r & 3);
                if (key >= N || (causal && key > q)) p = 0.0f;
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

template <typename T, int D>
__global__ void __launch_bounds__(256, 1)
    dkdv_kernel(const typename Mma<T>::elem* __restrict__ Q,
                const typename Mma<T>::elem* __restrict__ K,
                const typename Mma<T>::elem* __restrict__ V, const float* __restrict__ L,
                const typename Mma<T>::elem* __restrict__ dO, const float* __restrict__ Dl,
                typename Mma<T>::elem* __restrict__ dK, typename Mma<T>::elem* __restrict__ dV,
                int N, int nkb, float c, float scale, int causal) {
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

    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = lid / nkb;
    const int kb = lid % nkb;  // ascending: with a causal mask the first blocks carry the most work
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int l32 = lane & 31;
    const int g2 = lane >> 5;

    const size_t head = static_cast<size_t>(bh) * N * D;
    const float* Lh = L + static_cast<size_t>(bh) * N;
    const float* Dh = Dl + static_cast<size_t>(bh) * N;
    const int k0 = kb * Cfg::BN + wave * 32;  // first key of this wave
    const int key = k0 + l32;                 // key row owned by this lane
    const bool key_ok = key < N;

    frag kf[D / M::KW];
    frag vf[D / M::KW];
#pragma unroll
    for (int ks = 0; ks < D / M::KW; ++ks) {
        kf[ks] = M::zero();
        vf[ks] = M::zero();
        if (key_ok) {
            kf[ks] = M::row_operand(K + head + static_cast<size_t>(key) * D + M::KW * ks);
            vf[ks] = M::row_operand(V + head + static_cast<size_t>(key) * D + M::KW * ks);
        }
    }

    f32x16 dk[D / 32];
    f32x16 dv[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        dk[dt] = f32x16{};
        dv[dt] = f32x16{};
    }

    const int nqb = (N + Cfg::BM - 1) / Cfg::BM;
    const int qb_begin = causal ? (kb * Cfg::BN) / Cfg::BM : 0;
    TileCopy<E, Cfg::BM, D, Cfg::kThreads> qcp, ocp;
    float lreg = 0.0f;
    auto fetch = [&](int qb) {
        const int r0 = qb * Cfg::BM;
        qcp.fetch(Q + head + static_cast<size_t>(r0) * D, N - r0, tid);
        ocp.fetch(dO + head + static_cast<size_t>(r0) * D, N - r0, tid);
        if (tid < 2 * Cfg::BM) {
            const int r = r0 + (tid % Cfg::BM);
            if (tid < Cfg::BM)
                lreg = r < N ? Lh[r] * kLog2e : INFINITY;  // rows past N: P = 0
            else
                lreg = r < N ? Dh[r] : 0.0f;
        }
    };
    const int col_off = M::col_lane_offset(Cfg::CP);

    if (qb_begin < nqb) fetch(qb_begin);
    for (int qb = qb_begin; qb < nqb; ++qb) {
        const int q0 = qb * Cfg::BM;
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
        if (qb + 1 < nqb) fetch(qb + 1);
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
        const bool masked = causal && (k0 + 31 > q0);
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            const f32x4 lv = *reinterpret_cast<const f32x4*>(&Ls[8 * a + 4 * g2]);
            const f32x4 dv4 = *reinterpret_cast<const f32x4*>(&Ds[8 * a + 4 * g2]);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int r = 4 * a + u;
                float p = fast_exp2(fmaf(s[r], c, -lv[u]));
                if (masked && key > q0 + 8 * a + 4 * g2 + u) p = 0.0f;
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
        E* krow = dK + head + static_cast<size_t>(key) * D;
        E* vrow = dV + head + static_cast<size_t>(key) * D;
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

// ------------------------------------------------------------------------------------------
// 4. Fused dK, dV, dQ (fp16 / bf16): one pass, five products per tile
// ------------------------------------------------------------------------------------------
// KV-stationary like dkdv_kernel (each wave owns 32 keys, the workgroup 128), but every query
// block also yields its dQ contribution: the waves write dS^T (rounded to T) to LDS, and after
// one barrier wave w forms the 32x32 tile dQ[q0:q0+32, 32*(w % NDT) : +32] over the workgroup's
// keys (A = dS via transpose reads of dS^T, B = K via transpose reads of the LDS copy of K) and
// adds it to an fp32 accumulator in HBM with global_atomic_add_f32. No score is computed twice
// (S, dP, dV, dK, dQ), against seven products for dq_kernel + dkdv_kernel.
// The query blocks are double-buffered in LDS (Q and dO in a row-read layout and a
// transpose-read layout, L and D), and so is dS^T, so one barrier per block suffices:
//   compute block i from buffer b; write dS^T[b]; stage block i+1 into buffer b^1 (fetched into
//   registers one block earlier); fetch block i+2; barrier; dQ of block i from dS^T[b].
// The atomics of block i are issued during block i+1, after its first products, so their wait
// on the dQ products overlaps with other work.
template <int D>
struct FusedCfg {
    static constexpr int kThreads = 256;
    static constexpr int BN = 128;  // keys per workgroup (32 per wave)
    static constexpr int BM = 32;   // query rows per block
    static constexpr int RP = D + 8;                              // row-read pitch (Q, dO)
    static constexpr int CP = ((2 * D) % 128 == 64) ? D : D + 32;  // transpose-read pitch
    static constexpr int SP = 32;   // dS^T pitch: 4 rows of 64 bytes cover the 64 banks
    static constexpr int NDT = D / 32;      // 32-column tiles of dQ
    static constexpr int KSPLIT = 4 / NDT;  // waves per dQ tile, each over BN / KSPLIT keys
    static constexpr int KSTEPS = BN / KSPLIT / 16;  // 16-key MFMA steps per wave for dQ
};

template <typename T, int D>
__global__ void __launch_bounds__(256, 1)
    bwd_fused_kernel(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                     const uint16_t* __restrict__ V, const float* __restrict__ L,
                     const uint16_t* __restrict__ dO, const float* __restrict__ Dl,
                     float* __restrict__ dq_acc, uint16_t* __restrict__ dK,
                     uint16_t* __restrict__ dV, int N, int nkb, float c, float scale,
                     int causal) {
    using frag = typename Elem<T>::frag;
    using Cfg = FusedCfg<D>;
    constexpr int BM = Cfg::BM;
    constexpr int RP = Cfg::RP;
    constexpr int CP = Cfg::CP;
    constexpr int SP = Cfg::SP;
    __shared__ __attribute__((aligned(16))) uint16_t Qs[2][BM * RP];
    __shared__ __attribute__((aligned(16))) uint16_t Qc[2][BM * CP];
    __shared__ __attribute__((aligned(16))) uint16_t Os[2][BM * RP];
    __shared__ __attribute__((aligned(16))) uint16_t Oc[2][BM * CP];
    __shared__ __attribute__((aligned(16))) uint16_t St[2][Cfg::BN * SP];
    __shared__ __attribute__((aligned(16))) uint16_t Kc[Cfg::BN * CP];
    __shared__ __attribute__((aligned(16))) float Ls[2][BM];
    __shared__ __attribute__((aligned(16))) float Ds[2][BM];

    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = lid / nkb;
    const int kb = lid % nkb;  // ascending: with a causal mask the first blocks carry the most work
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int l32 = lane & 31;
    const int g2 = lane >> 5;

    const size_t head = static_cast<size_t>(bh) * N * D;
    const float* Lh = L + static_cast<size_t>(bh) * N;
    const float* Dh = Dl + static_cast<size_t>(bh) * N;
    const int kwg = kb * Cfg::BN;             // first key of the workgroup
    const int k0 = kwg + wave * 32;           // first key of this wave
    const int key = k0 + l32;                 // key row owned by this lane
    const bool key_ok = key < N;

    // K and V of this lane's key as B operands (k = d), and K of the whole workgroup in LDS.
    frag kf[D / 16];
    frag vf[D / 16];
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
        u32x4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
        if (key_ok) {
            kv = ld16(K + head + static_cast<size_t>(key) * D + 16 * ks + 8 * g2);
            vv = ld16(V + head + static_cast<size_t>(key) * D + 16 * ks + 8 * g2);
        }
        kf[ks] = as_frag<T>(kv);
        vf[ks] = as_frag<T>(vv);
    }
    {
        TileCopy<uint16_t, Cfg::BN, D, Cfg::kThreads> kcp;
        kcp.fetch(K + head + static_cast<size_t>(kwg) * D, N - kwg, tid);
        kcp.stage(Kc, CP, tid);
    }

    f32x16 dk[D / 32];
    f32x16 dv[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
        dk[dt] = f32x16{};
        dv[dt] = f32x16{};
    }

    const int nqb = (N + BM - 1) / BM;
    const int qb_begin = causal ? kwg / BM : 0;
    TileCopy<uint16_t, BM, D, Cfg::kThreads> qcp, ocp;
    float lreg = 0.0f;
    auto fetch = [&](int qb) {
        const int r0 = qb * BM;
        qcp.fetch(Q + head + static_cast<size_t>(r0) * D, N - r0, tid);
        ocp.fetch(dO + head + static_cast<size_t>(r0) * D, N - r0, tid);
        if (tid < 2 * BM) {
            const int r = r0 + (tid % BM);
            if (tid < BM)
                lreg = r < N ? Lh[r] * kLog2e : INFINITY;  // rows past N: P = 0
            else
                lreg = r < N ? Dh[r] : 0.0f;
        }
    };
    auto stage = [&](int b) {
        qcp.stage(Qs[b], RP, tid);
        qcp.stage(Qc[b], CP, tid);
        ocp.stage(Os[b], RP, tid);
        ocp.stage(Oc[b], CP, tid);
        if (tid < BM)
            Ls[b][tid] = lreg;
        else if (tid < 2 * BM)
            Ds[b][tid - BM] = lreg;
    };

    const int tr_c = tr_lane_offset(CP);
    const int tr_s = tr_lane_offset(SP);
    const int dtile = wave % Cfg::NDT;           // dQ column tile of this wave
    const int jbeg = (wave / Cfg::NDT) * Cfg::KSTEPS;  // first 16-key step of its key range
    float* dq_head = dq_acc + head;

    f32x16 dq_prev = f32x16{};
    int q0_prev = -1;
    auto flush_dq = [&]() {
        if (q0_prev < 0) return;
        float* base = dq_head + 32 * dtile + l32;
        if (q0_prev + BM <= N) {  // wave-uniform: every row of the block exists
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int q = q0_prev + 8 * (r >> 2) + 4 * g2 + (r & 3);
                unsafeAtomicAdd(base + static_cast<size_t>(q) * D, dq_prev[r]);
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int q = q0_prev + 8 * (r >> 2) + 4 * g2 + (r & 3);
                if (q < N) unsafeAtomicAdd(base + static_cast<size_t>(q) * D, dq_prev[r]);
            }
        }
    };

    if (qb_begin < nqb) {
        fetch(qb_begin);
        stage(0);
        if (qb_begin + 1 < nqb) fetch(qb_begin + 1);
    }
    __syncthreads();

    for (int qb = qb_begin; qb < nqb; ++qb) {
        const int b = (qb - qb_begin) & 1;
        const int q0 = qb * BM;
        // Every wave runs every block, also where all of its keys are masked (P = 0): a branch
        // around the MFMAs would make the compiler copy the dK/dV accumulators between AGPRs
        // and VGPRs on every iteration.
        f32x16 s = f32x16{};
        f32x16 dp = f32x16{};
        // S = Q K^T and dP = dO V^T: rows = queries, column = this lane's key.
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) {
            s = Elem<T>::mma(as_frag<T>(ld16(&Qs[b][l32 * RP + 16 * ks + 8 * g2])), kf[ks], s);
            dp = Elem<T>::mma(as_frag<T>(ld16(&Os[b][l32 * RP + 16 * ks + 8 * g2])), vf[ks], dp);
        }
        flush_dq();  // atomics of the previous block, behind this block's first products

        {
            const bool masked = (causal && k0 + 31 > q0) || (k0 + 31 >= N);
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const f32x4 lv = *reinterpret_cast<const f32x4*>(&Ls[b][8 * a + 4 * g2]);
                const f32x4 dv4 = *reinterpret_cast<const f32x4*>(&Ds[b][8 * a + 4 * g2]);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int r = 4 * a + u;
                    float p = fast_exp2(fmaf(s[r], c, -lv[u]));
                    if (masked && (!key_ok || (causal && key > q0 + 8 * a + 4 * g2 + u)))
                        p = 0.0f;
                    s[r] = p;
                    dp[r] = p * (dp[r] - dv4[u]);
                }
            }
            // dV^T += dO^T P and dK^T += Q^T dS: k = the block's query rows.
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const frag bp = pack_frag<T>(s[8 * j + 0], s[8 * j + 1], s[8 * j + 2], s[8 * j + 3],
                                             s[8 * j + 4], s[8 * j + 5], s[8 * j + 6], s[8 * j + 7]);
                const frag bs = pack_frag<T>(dp[8 * j + 0], dp[8 * j + 1], dp[8 * j + 2],
                                             dp[8 * j + 3], dp[8 * j + 4], dp[8 * j + 5],
                                             dp[8 * j + 6], dp[8 * j + 7]);
#pragma unroll
                for (int dt = 0; dt < D / 32; ++dt) {
                    dv[dt] = Elem<T>::mma(
                        read_tr_frag<T>(&Oc[b][16 * j * CP + 32 * dt + tr_c], CP), bp, dv[dt]);
                    dk[dt] = Elem<T>::mma(
                        read_tr_frag<T>(&Qc[b][16 * j * CP + 32 * dt + tr_c], CP), bs, dk[dt]);
                }
            }
        }
        // dS^T[key][q], rounded to T.
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            u32x2 w;
            w[0] = Elem<T>::pack2(dp[4 * a + 0], dp[4 * a + 1]);
            w[1] = Elem<T>::pack2(dp[4 * a + 2], dp[4 * a + 3]);
            st8(&St[b][(32 * wave + l32) * SP + 8 * a + 4 * g2], w);
        }
        if (qb + 1 < nqb) {
            stage(b ^ 1);
            if (qb + 2 < nqb) fetch(qb + 2);
        }
        __syncthreads();

        // dQ[q0 : q0+32, 32*dtile : +32] += dS K over this wave's share of the keys.
        f32x16 acc = f32x16{};
#pragma unroll
        for (int jj = 0; jj < Cfg::KSTEPS; ++jj) {
            const int j = jbeg + jj;
            const frag a = read_tr_frag<T>(&St[b][16 * j * SP + tr_s], SP);
            const frag bk = read_tr_frag<T>(&Kc[16 * j * CP + 32 * dtile + tr_c], CP);
            acc = Elem<T>::mma(a, bk, acc);
        }
        dq_prev = acc;
        q0_prev = q0;
    }
    flush_dq();

    if (key_ok) {
        uint16_t* krow = dK + head + static_cast<size_t>(key) * D;
        uint16_t* vrow = dV + head + static_cast<size_t>(key) * D;
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

// dQ = T(scale * dq_acc), eight elements per thread.
template <typename T>
__global__ void __launch_bounds__(256)
    dq_convert_kernel(const float* __restrict__ acc, uint16_t* __restrict__ dQ, float scale,
                      long long n8) {
    const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n8) return;
    const f32x4 a = __builtin_bit_cast(f32x4, ld16(acc + 8 * i));
    const f32x4 b = __builtin_bit_cast(f32x4, ld16(acc + 8 * i + 4));
    u32x4 w;
    w[0] = Elem<T>::pack2(a[0] * scale, a[1] * scale);
    w[1] = Elem<T>::pack2(a[2] * scale, a[3] * scale);
    w[2] = Elem<T>::pack2(b[0] * scale, b[1] * scale);
    w[3] = Elem<T>::pack2(b[2] * scale, b[3] * scale);
    st16(dQ + 8 * i, w);
}

}  // namespace dev

namespace detail {

namespace {

// Deterministic path: delta, dq_kernel, dkdv_kernel (no atomics; dQ recomputes S and dP).
template <typename T, int D>
FlashAttentionError run_backward_two_pass(const T* Q, const T* K, const T* V, const T* O,
                                          const float* L, const T* dO, T* dQ, T* dK, T* dV,
                                          int BH, int N, float scale, bool causal,
                                          hipStream_t stream) {
    using E = typename dev::Mma<T>::elem;
    const E* q = reinterpret_cast<const E*>(Q);
    const E* k = reinterpret_cast<const E*>(K);
    const E* v = reinterpret_cast<const E*>(V);
    const E* o = reinterpret_cast<const E*>(O);
    const E* go = reinterpret_cast<const E*>(dO);

    const long long rows = static_cast<long long>(BH) * N;
    StreamWorkspace ws(stream);
    FlashAttentionError err = ws.alloc(static_cast<size_t>(rows) * sizeof(float));
    if (err != FlashAttentionError::SUCCESS) return err;
    float* delta = static_cast<float*>(ws.get());

    constexpr int VEC = 16 / static_cast<int>(sizeof(E));
    constexpr int LPR = D / VEC;
    const long long dthreads = rows * LPR;
    const long long dblocks = (dthreads + 255) / 256;
    if (dblocks > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
    int tok = profile_kernel<T, D>("backward_delta", stream);
    hipLaunchKernelGGL((dev::delta_kernel<T, D>), dim3(static_cast<unsigned>(dblocks)), dim3(256),
                       0, stream, go, o, delta, nullptr, rows);
    profile_end(tok, stream);
    err = from_hip(hipGetLastError());
    if (err != FlashAttentionError::SUCCESS) return err;

    const float c = scale * dev::kLog2e;
    {
        using Cfg = dev::DqCfg<T, D>;
        const int nqb = (N + Cfg::BM - 1) / Cfg::BM;
        const long long blocks = static_cast<long long>(nqb) * BH;
        if (blocks > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
        tok = profile_kernel<T, D>("backward_dq", stream);
        hipLaunchKernelGGL((dev::dq_kernel<T, D>), dim3(static_cast<unsigned>(blocks)),
                           dim3(Cfg::kThreads), 0, stream, q, k, v, L, go, delta,
                           reinterpret_cast<E*>(dQ), N, nqb, c, scale, causal ? 1 : 0);
        profile_end(tok, stream);
        err = from_hip(hipGetLastError());
        if (err != FlashAttentionError::SUCCESS) return err;
    }
    {
        using Cfg = dev::DkvCfg<T, D>;
        const int nkb = (N + Cfg::BN - 1) / Cfg::BN;
        const long long blocks = static_cast<long long>(nkb) * BH;
        if (blocks > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
        tok = profile_kernel<T, D>("backward_dkdv", stream);
        hipLaunchKernelGGL((dev::dkdv_kernel<T, D>), dim3(static_cast<unsigned>(blocks)),
                           dim3(Cfg::kThreads), 0, stream, q, k, v, L, go, delta,
                           reinterpret_cast<E*>(dK), reinterpret_cast<E*>(dV), N, nkb, c, scale,
                           causal ? 1 : 0);
        profile_end(tok, stream);
        err = from_hip(hipGetLastError());
    }
    return err;
}

// Fused path (fp16 / bf16): delta (+ clear the fp32 dQ accumulator), bwd_fused_kernel,
// dq_convert_kernel. dQ is summed with fp32 atomics, so its last bit may differ between runs.
template <typename T, int D>
FlashAttentionError run_backward_fused(const T* Q, const T* K, const T* V, const T* O,
                                       const float* L, const T* dO, T* dQ, T* dK, T* dV, int BH,
                                       int N, float scale, bool causal, hipStream_t stream) {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(Q);
    const uint16_t* k = reinterpret_cast<const uint16_t*>(K);
    const uint16_t* v = reinterpret_cast<const uint16_t*>(V);
    const uint16_t* o = reinterpret_cast<const uint16_t*>(O);
    const uint16_t* go = reinterpret_cast<const uint16_t*>(dO);

    const long long rows = static_cast<long long>(BH) * N;
    // delta (rows floats, padded to 256 bytes) followed by the dQ accumulator (rows * D floats).
    const size_t delta_bytes = (static_cast<size_t>(rows) * sizeof(float) + 255) & ~size_t(255);
    const size_t acc_bytes = static_cast<size_t>(rows) * D * sizeof(float);
    StreamWorkspace ws(stream);
    FlashAttentionError err = ws.alloc(delta_bytes + acc_bytes);
    if (err != FlashAttentionError::SUCCESS) return err;
    float* delta = static_cast<float*>(ws.get());
    float* dq_acc = reinterpret_cast<float*>(static_cast<char*>(ws.get()) + delta_bytes);

    constexpr int LPR = D / 8;
    const long long dblocks = (rows * LPR + 255) / 256;
    using Cfg = dev::FusedCfg<D>;
    const int nkb = (N + Cfg::BN - 1) / Cfg::BN;
    const long long blocks = static_cast<long long>(nkb) * BH;
    const long long n8 = rows * D / 8;
    const long long cblocks = (n8 + 255) / 256;
    if (dblocks > 0x7fffffffLL || blocks > 0x7fffffffLL || cblocks > 0x7fffffffLL)
        return FlashAttentionError::INVALID_DIMENSION;

    int tok = profile_kernel<T, D>("backward_delta", stream);
    hipLaunchKernelGGL((dev::delta_kernel<T, D>), dim3(static_cast<unsigned>(dblocks)), dim3(256),
                       0, stream, go, o, delta, dq_acc, rows);
    profile_end(tok, stream);
    err = from_hip(hipGetLastError());
    if (err != FlashAttentionError::SUCCESS) return err;

    tok = profile_kernel<T, D>("backward_fused", stream);
    hipLaunchKernelGGL((dev::bwd_fused_kernel<T, D>), dim3(static_cast<unsigned>(blocks)),
                       dim3(Cfg::kThreads), 0, stream, q, k, v, L, go, delta, dq_acc,
                       reinterpret_cast<uint16_t*>(dK), reinterpret_cast<uint16_t*>(dV), N, nkb,
                       scale * dev::kLog2e, scale, causal ? 1 : 0);
    profile_end(tok, stream);
    err = from_hip(hipGetLastError());
    if (err != FlashAttentionError::SUCCESS) return err;

    tok = profile_kernel<T, D>("backward_dq_convert", stream);
    hipLaunchKernelGGL((dev::dq_convert_kernel<T>), dim3(static_cast<unsigned>(cblocks)),
                       dim3(256), 0, stream, dq_acc, reinterpret_cast<uint16_t*>(dQ), scale, n8);
    profile_end(tok, stream);
    return from_hip(hipGetLastError());
}

// CUFLASH_DETERMINISTIC=1 in the environment selects the atomic-free two-pass backward for
// fp16 / bf16 as well (read on every call).
bool deterministic_requested() {
    const char* e = std::getenv("CUFLASH_DETERMINISTIC");
    return e && e[0] && !(e[0] == '0' && e[1] == '\0');
}

template <typename T, int D>
FlashAttentionError run_backward(const T* Q, const T* K, const T* V, const T* O, const float* L,
                                 const T* dO, T* dQ, T* dK, T* dV, int BH, int N, float scale,
                                 bool causal, hipStream_t stream) {
    if constexpr (!std::is_same<T, float>::value) {
        if (!deterministic_requested())
            return run_backward_fused<T, D>(Q, K, V, O, L, dO, dQ, dK, dV, BH, N, scale, causal,
                                            stream);
    }
    return run_backward_two_pass<T, D>(Q, K, V, O, L, dO, dQ, dK, dV, BH, N, scale, causal,
                                       stream);
}

}  // namespace

template <typename T>
FlashAttentionError launch_backward(const T* Q, const T* K, const T* V, const T* O,
                                    const float* L, const T* dO, T* dQ, T* dK, T* dV,
                                    int batch_size, int num_heads, int seq_len, int head_dim,
                                    float scale, bool causal, hipStream_t stream) {
    const long long bh = static_cast<long long>(batch_size) * num_heads;
    if (bh > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
    const int BH = static_cast<int>(bh);
    switch (head_dim) {
        case 32:
            return run_backward<T, 32>(Q, K, V, O, L, dO, dQ, dK, dV, BH, seq_len, scale, causal,
                                       stream);
        case 64:
            return run_backward<T, 64>(Q, K, V, O, L, dO, dQ, dK, dV, BH, seq_len, scale, causal,
                                       stream);
        case 128:
            return run_backward<T, 128>(Q, K, V, O, L, dO, dQ, dK, dV, BH, seq_len, scale, causal,
                                        stream);
    }
    return FlashAttentionError::UNSUPPORTED_HEAD_DIM;
}

template FlashAttentionError launch_backward<float>(const float*, const float*, const float*,
                                                    const float*, const float*, const float*,
                                                    float*, float*, float*, int, int, int, int,
                                                    float, bool, hipStream_t);
template FlashAttentionError launch_backward<__half>(const __half*, const __half*, const __half*,
                                                     const __half*, const float*, const __half*,
                                                     __half*, __half*, __half*, int, int, int, int,
                                                     float, bool, hipStream_t);
template FlashAttentionError launch_backward<__hip_bfloat16>(
    const __hip_bfloat16*, const __hip_bfloat16*, const __hip_bfloat16*, const __hip_bfloat16*,
    const float*, const __hip_bfloat16*, __hip_bfloat16*, __hip_bfloat16*, __hip_bfloat16*, int,
    int, int, int, float, bool, hipStream_t);

}  // namespace detail
}  // namespace cuflash
