// Split-KV flash decoding for gfx950 (MI355X). No reference counterpart: the reference lists
// "FlashDecoding / Split-KV" as a roadmap item (ROADMAP.md:24-25); the merge rule is the
// reference's online-softmax update (src/kernels/impl/online_softmax.cuh:28-33).
//
// decode_split_kernel: one workgroup per (batch*head, split). The split's keys are streamed
//   once from HBM with 16-byte loads: a key row of D elements is spread over LPR = D / VEC lanes
//   (VEC = elements per 16 bytes), so one wave load covers 64 / LPR rows and every lane keeps
//   UNROLL rows of K and V in flight. Scores are reduced over the LPR lanes with DPP
//   (row-local, no LDS), each lane group folds its rows into a running (m, l, acc) state, and the
//   groups and waves are merged at the end. Output: an unnormalized fp32 partial
//   acc_s = sum_j exp2(s_j - m_s) v_j with m_s (log2 units) and l_s = sum_j exp2(s_j - m_s).
// decode_combine_kernel: per (batch*head), M = max_s m_s, l = sum_s l_s 2^(m_s - M),
//   O = sum_s acc_s 2^(m_s - M) / l, L = (M + log2 l) * ln 2.

#include "common.hpp"
#include "launch.hpp"
#include "profile.hpp"

namespace cuflash {
namespace dev {

template <typename T, int D>
struct DecCfg {
    using E = typename Mma<T>::elem;
    static constexpr int VEC = 16 / static_cast<int>(sizeof(E));
    static constexpr int LPR = D / VEC;   // lanes per key row
    static constexpr int RPW = 64 / LPR;  // rows per wave load
    static constexpr int UNROLL = 8;      // rows per lane group per iteration
    static constexpr int kWaves = 4;
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int ROWS_PER_ITER = RPW * UNROLL * kWaves;
};

// DPP lane permutations (row = 16 lanes).
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within each 8 lanes
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within each row

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of G lanes (G = 2 .. 32); every lane of the group gets the total.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (G >= 2) v += dpp<kDppXor1>(v);
    if constexpr (G >= 4) v += dpp<kDppXor2>(v);
    if constexpr (G >= 8) v += dpp<kDppHalfMirror>(v);
    if constexpr (G >= 16) v += dpp<kDppMirror>(v);
    if constexpr (G >= 32) v += xor_shuffle(v, 16);
    return v;
}

template <typename T>
__device__ __forceinline__ void unpack16(u32x4 v, float (&out)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[2 * i] = Elem<T>::to_f(static_cast<uint16_t>(v[i]));
        out[2 * i + 1] = Elem<T>::to_f(static_cast<uint16_t>(v[i] >> 16));
    }
}

// Element-wise view of a 16-byte chunk as VEC floats.
template <typename T, int VEC>
__device__ __forceinline__ void to_floats(u32x4 v, float (&out)[VEC]) {
    if constexpr (std::is_same<T, float>::value) {
        const f32x4 f = __builtin_bit_cast(f32x4, v);
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = f[i];
    } else {
        unpack16<T>(v, out);
    }
}

// exp2(x - m) that is 0 when x = -inf (also when m = -inf).
__device__ __forceinline__ float exp2_rel(float x, float m) {
    return x == -INFINITY ? 0.0f : fast_exp2(x - m);
}

template <typename T, int D>
__global__ void __launch_bounds__(256)
    decode_split_kernel(const typename Mma<T>::elem* __restrict__ Q,
                        const typename Mma<T>::elem* __restrict__ K,
                        const typename Mma<T>::elem* __restrict__ V, float* __restrict__ part_acc,
                        float2* __restrict__ part_ml, int kv_len, int chunk, int nsplit, float c) {
    using Cfg = DecCfg<T, D>;
    constexpr int VEC = Cfg::VEC;
    constexpr int LPR = Cfg::LPR;
    constexpr int RPW = Cfg::RPW;
    constexpr int U = Cfg::UNROLL;

    const int bh = blockIdx.x / nsplit;
    const int split = blockIdx.x % nsplit;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int grp = lane / LPR;   // row slot inside a wave load
    const int part = lane % LPR;  // which 16-byte chunk of the row

    const size_t head = static_cast<size_t>(bh) * kv_len * D;
    const int kbeg = split * chunk;
    const int kend = min(kv_len, kbeg + chunk);

    float qv[VEC];
    to_floats<T, VEC>(ld16(Q + static_cast<size_t>(bh) * D + part * VEC), qv);
#pragma unroll
    for (int i = 0; i < VEC; ++i) qv[i] *= c;  // scores come out in log2 units

    float m = -INFINITY;
    float l = 0.0f;
    float acc[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[i] = 0.0f;

    const typename Mma<T>::elem* Kh = K + head + part * VEC;
    const typename Mma<T>::elem* Vh = V + head + part * VEC;
    for (int base = kbeg + wave * RPW * U; base < kend; base += Cfg::ROWS_PER_ITER) {
        u32x4 kr[U], vr[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int row = base + u * RPW + grp;
            kr[u] = u32x4{0u, 0u, 0u, 0u};
            vr[u] = u32x4{0u, 0u, 0u, 0u};
            if (row < kend) {
                kr[u] = ld16(Kh + static_cast<size_t>(row) * D);
                vr[u] = ld16(Vh + static_cast<size_t>(row) * D);
            }
        }
        float s[U];
        float mblk = -INFINITY;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float kf[VEC];
            to_floats<T, VEC>(kr[u], kf);
            float dot = 0.0f;
#pragma unroll
            for (int i = 0; i < VEC; ++i) dot = fmaf(qv[i], kf[i], dot);
            dot = group_sum<LPR>(dot);
            s[u] = (base + u * RPW + grp < kend) ? dot : -INFINITY;
            mblk = fmaxf(mblk, s[u]);
        }
        const float m_new = fmaxf(m, mblk);
        const float alpha = exp2_rel(m, m_new);
        l *= alpha;
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[i] *= alpha;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float p = exp2_rel(s[u], m_new);
            float vf[VEC];
            to_floats<T, VEC>(vr[u], vf);
            l += p;
#pragma unroll
            for (int i = 0; i < VEC; ++i) acc[i] = fmaf(p, vf[i], acc[i]);
        }
        m = m_new;
    }

    // Merge the RPW row slots of the wave (lanes part, part + LPR, ...).
#pragma unroll
    for (int w = LPR; w < 64; w <<= 1) {
        const float m2 = xor_shuffle(m, w);
        const float l2 = xor_shuffle(l, w);
        const float mm = fmaxf(m, m2);
        const float f1 = exp2_rel(m, mm);
        const float f2 = exp2_rel(m2, mm);
        l = l * f1 + l2 * f2;
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[i] = acc[i] * f1 + xor_shuffle(acc[i], w) * f2;
        m = mm;
    }

    // Merge the waves through LDS.
    __shared__ float s_m[Cfg::kWaves];
    __shared__ float s_l[Cfg::kWaves];
    __shared__ __attribute__((aligned(16))) float s_acc[Cfg::kWaves][D];
    if (lane < LPR) {
#pragma unroll
        for (int i = 0; i < VEC; ++i) s_acc[wave][part * VEC + i] = acc[i];
        if (lane == 0) {
            s_m[wave] = m;
            s_l[wave] = l;
        }
    }
    __syncthreads();
    if (tid < D) {
        float mm = -INFINITY;
#pragma unroll
        for (int w = 0; w < Cfg::kWaves; ++w) mm = fmaxf(mm, s_m[w]);
        float lt = 0.0f, at = 0.0f;
#pragma unroll
        for (int w = 0; w < Cfg::kWaves; ++w) {
            const float f = exp2_rel(s_m[w], mm);
            lt += s_l[w] * f;
            at += s_acc[w][tid] * f;
        }
        const size_t slot = static_cast<size_t>(bh) * nsplit + split;
        part_acc[slot * D + tid] = at;
        if (tid == 0) part_ml[slot] = make_float2(mm, lt);
    }
}

template <typename T, int D>
__global__ void __launch_bounds__(D)
    decode_combine_kernel(const float* __restrict__ part_acc, const float2* __restrict__ part_ml,
                          typename Mma<T>::elem* __restrict__ O, float* __restrict__ L,
                          int nsplit) {
    const int bh = blockIdx.x;
    const int d = threadIdx.x;
    const float2* ml = part_ml + static_cast<size_t>(bh) * nsplit;
    const float* acc = part_acc + static_cast<size_t>(bh) * nsplit * D;
    float mm = -INFINITY;
    for (int s = 0; s < nsplit; ++s) mm = fmaxf(mm, ml[s].x);
    float lt = 0.0f, at = 0.0f;
    for (int s = 0; s < nsplit; ++s) {
        const float2 v = ml[s];
        const float f = exp2_rel(v.x, mm);
        lt += v.y * f;
        at += acc[static_cast<size_t>(s) * D + d] * f;
    }
    const float o = at / lt;
    if constexpr (std::is_same<T, float>::value) {
        O[static_cast<size_t>(bh) * D + d] = o;
    } else {
        O[static_cast<size_t>(bh) * D + d] = static_cast<uint16_t>(Elem<T>::pack2(o, 0.0f) & 0xffffu);
    }
    if (d == 0) L[bh] = (mm + fast_log2(lt)) * kLn2;
}

}  // namespace dev

namespace detail {

namespace {

int device_cu_count() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
        return 256;
    return cus;
}

// Split count: enough (batch*head, split) workgroups to give every CU several, with chunks of at
// least 512 keys; an explicit request is clamped to [1, min(1024, ceil(kv_len / 16))].
int choose_splits(int requested, int BH, int kv_len) {
    const int max_useful = std::max(1, std::min(1024, (kv_len + 15) / 16));
    if (requested > 0) return std::min(requested, max_useful);
    const int target_blocks = 8 * device_cu_count();
    int s = (target_blocks + BH - 1) / BH;
    s = std::min(s, std::max(1, kv_len / 512));
    return std::max(1, std::min(s, max_useful));
}

template <typename T, int D>
FlashAttentionError run_decode(const T* Q, const T* K, const T* V, T* O, float* L, int BH,
                               int kv_len, float scale, int num_splits, hipStream_t stream) {
    using E = typename dev::Mma<T>::elem;
    using Cfg = dev::DecCfg<T, D>;
    const int nsplit = choose_splits(num_splits, BH, kv_len);
    const int chunk = (kv_len + nsplit - 1) / nsplit;
    const long long blocks = static_cast<long long>(BH) * nsplit;
    if (blocks > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;

    const size_t acc_bytes = static_cast<size_t>(blocks) * D * sizeof(float);
    const size_t ml_bytes = static_cast<size_t>(blocks) * sizeof(float2);
    StreamWorkspace ws(stream);
    FlashAttentionError err = ws.alloc(acc_bytes + ml_bytes);
    if (err != FlashAttentionError::SUCCESS) return err;
    float* part_acc = static_cast<float*>(ws.get());
    float2* part_ml = reinterpret_cast<float2*>(static_cast<char*>(ws.get()) + acc_bytes);

    int tok = profile_kernel<T, D>("decode_split", stream);
    hipLaunchKernelGGL((dev::decode_split_kernel<T, D>), dim3(static_cast<unsigned>(blocks)),
                       dim3(Cfg::kThreads), 0, stream, reinterpret_cast<const E*>(Q),
                       reinterpret_cast<const E*>(K), reinterpret_cast<const E*>(V), part_acc,
                       part_ml, kv_len, chunk, nsplit, scale * dev::kLog2e);
    profile_end(tok, stream);
    err = from_hip(hipGetLastError());
    if (err != FlashAttentionError::SUCCESS) return err;
    tok = profile_kernel<T, D>("decode_combine", stream);
    hipLaunchKernelGGL((dev::decode_combine_kernel<T, D>), dim3(static_cast<unsigned>(BH)), dim3(D),
                       0, stream, part_acc, part_ml, reinterpret_cast<E*>(O), L, nsplit);
    profile_end(tok, stream);
    return from_hip(hipGetLastError());
}

}  // namespace

template <typename T>
FlashAttentionError launch_decode(const T* Q, const T* K, const T* V, T* O, float* L,
                                  int batch_size, int num_heads, int kv_len, int head_dim,
                                  float scale, int num_splits, hipStream_t stream) {
    const long long bh = static_cast<long long>(batch_size) * num_heads;
    if (bh > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
    const int BH = static_cast<int>(bh);
    switch (head_dim) {
        case 32: return run_decode<T, 32>(Q, K, V, O, L, BH, kv_len, scale, num_splits, stream);
        case 64: return run_decode<T, 64>(Q, K, V, O, L, BH, kv_len, scale, num_splits, stream);
        case 128: return run_decode<T, 128>(Q, K, V, O, L, BH, kv_len, scale, num_splits, stream);
    }
    return FlashAttentionError::UNSUPPORTED_HEAD_DIM;
}

template FlashAttentionError launch_decode<float>(const float*, const float*, const float*, float*,
                                                  float*, int, int, int, int, float, int,
                                                  hipStream_t);
template FlashAttentionError launch_decode<__half>(const __half*, const __half*, const __half*,
                                                   __half*, float*, int, int, int, int, float, int,
                                                   hipStream_t);
template FlashAttentionError launch_decode<__hip_bfloat16>(const __hip_bfloat16*,
                                                           const __hip_bfloat16*,
                                                           const __hip_bfloat16*, __hip_bfloat16*,
                                                           float*, int, int, int, int, float, int,
                                                           hipStream_t);

}  // namespace detail
}  // namespace cuflash
