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
// decode_mma_kernel / decode_mma_rows_kernel: the same partials for 2 to 32 query heads per
//   key/value head (fp16 / bf16) on the matrix cores, the query heads as the columns of MFMA
//   tiles; the rows kernel takes four key/value heads of a paged cache per workgroup.
// decode_combine_kernel: per (batch*head), M = max_s m_s, l = sum_s l_s 2^(m_s - M),
//   O = sum_s acc_s 2^(m_s - M) / l, L = (M + log2 l) * ln 2; one workgroup per 32 columns.

#include <mutex>

#include "common.hpp"
#include "launch.hpp"
#include "profile.hpp"
#include "softmax.hpp"
#include "tile_groups.hpp"

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

// Where the keys come from. Contiguous: K, V [B, Hkv, kv_len, D]. Paged: K, V
// [num_pages, page_size, Hkv, D] with block_table [B, max_pages] naming the page of each
// page_size keys of a sequence and seq_lens [B] its length (clamped to [0, kv_len], kv_len =
// max_pages * page_size). A workgroup serves G query heads that share one key/value head:
// query head h reads key/value head h / (H / Hkv).
struct DecodeArgs {
    const int* block_table;
    const int* seq_lens;
    int H, Hkv;
    int kv_len;
    int page_size, max_pages;
    int page_shift;  // log2(page_size) when it is a power of two, else -1
    int chunk, nsplit;
    float c;  // scale * log2(e)
};

template <typename T, int D, int G, bool PAGED>
__global__ void __launch_bounds__(256)
    decode_split_kernel(const typename Mma<T>::elem* __restrict__ Q,
                        const typename Mma<T>::elem* __restrict__ K,
                        const typename Mma<T>::elem* __restrict__ V, float* __restrict__ part_acc,
                        float2* __restrict__ part_ml, DecodeArgs a) {
    using Cfg = DecCfg<T, D>;
    constexpr int VEC = Cfg::VEC;
    constexpr int LPR = Cfg::LPR;
    constexpr int RPW = Cfg::RPW;
    // Rows in flight per lane group: fewer when the workgroup carries several query heads.
    constexpr int U = G <= 2 ? Cfg::UNROLL : Cfg::UNROLL / 2;
    constexpr int ROWS_PER_ITER = RPW * U * Cfg::kWaves;

    // blockIdx.x = ((b * Hkv + hk) * NG + g) * nsplit + split, NG = (H / Hkv) / G.
    const int hpk = a.H / a.Hkv;
    const int NG = hpk / G;
    int rest = blockIdx.x;
    const int split = rest % a.nsplit;
    rest /= a.nsplit;
    const int g = rest % NG;
    rest /= NG;
    const int hk = rest % a.Hkv;
    const int b = rest / a.Hkv;
    const int h0 = hk * hpk + g * G;  // first query head of the workgroup

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int grp = lane / LPR;   // row slot inside a wave load
    const int part = lane % LPR;  // which 16-byte chunk of the row

    const int kv_b = PAGED ? min(max(a.seq_lens[b], 0), a.kv_len) : a.kv_len;
    const int kbeg = split * a.chunk;
    const int kend = min(kv_b, kbeg + a.chunk);

    // Page of key row t and the row's offset inside it (paged cache).
    auto page_of = [&](int t) {
        const int j = a.page_shift >= 0 ? t >> a.page_shift : t / a.page_size;
        return a.block_table[static_cast<size_t>(b) * a.max_pages + j];
    };
    auto in_page = [&](int t) {
        return a.page_shift >= 0 ? t & (a.page_size - 1) : t % a.page_size;
    };
    // Element offset of key row t of this (batch, key/value head); `page` is page_of(t).
    auto row_off = [&](int t, int page) -> size_t {
        if constexpr (PAGED) {
            return ((static_cast<size_t>(page) * a.page_size + in_page(t)) * a.Hkv + hk) * D;
        } else {
            return (static_cast<size_t>(b) * a.Hkv + hk) * static_cast<size_t>(a.kv_len) * D +
                   static_cast<size_t>(t) * D;
        }
    };

    // Q: 16-bit types keep the row chunk packed for v_dot2 (the scale is applied to the dot
    // product); fp32 holds it pre-scaled.
    constexpr bool kPacked = !std::is_same<T, float>::value;
    u32x4 qp[G];
    float qv[G][VEC];
    float m[G], l[G];
    float acc[G][VEC];
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
        const size_t qrow = static_cast<size_t>(b) * a.H + h0 + gi;
        qp[gi] = ld16(Q + qrow * D + part * VEC);
        to_floats<T, VEC>(qp[gi], qv[gi]);
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
            qv[gi][i] *= a.c;  // scores come out in log2 units
            acc[gi][i] = 0.0f;
        }
        m[gi] = -INFINITY;
        l[gi] = 0.0f;
    }

    const typename Mma<T>::elem* Kp = K + part * VEC;
    const typename Mma<T>::elem* Vp = V + part * VEC;
    // Paged: the page indices of an iteration's rows are fetched one iteration ahead, so their
    // latency does not add to that of the K / V loads that depend on them.
    int pg[U];
    auto fetch_pages = [&](int bs) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int row = bs + u * RPW + grp;
            pg[u] = (PAGED && row < kend) ? page_of(row) : 0;
        }
    };
    const int first = kbeg + wave * RPW * U;
    if constexpr (PAGED) fetch_pages(first);
    for (int base = first; base < kend; base += ROWS_PER_ITER) {
        u32x4 kr[U], vr[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int row = base + u * RPW + grp;
            kr[u] = u32x4{0u, 0u, 0u, 0u};
            vr[u] = u32x4{0u, 0u, 0u, 0u};
            if (row < kend) {
                const size_t off = row_off(row, pg[u]);
                // Each key / value row is read exactly once: non-temporal loads keep the stream
                // from displacing other lines in the caches (13% more bandwidth at 32k keys).
                kr[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(Kp + off));
                vr[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(Vp + off));
            }
        }
        if constexpr (PAGED) fetch_pages(base + ROWS_PER_ITER);
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            float s[U];
            float mblk = -INFINITY;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                float dot = 0.0f;
                if constexpr (kPacked) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) dot = Elem<T>::dot2(qp[gi][j], kr[u][j], dot);
                    dot = group_sum<LPR>(dot) * a.c;
                } else {
                    float kf[VEC];
                    to_floats<T, VEC>(kr[u], kf);
#pragma unroll
                    for (int i = 0; i < VEC; ++i) dot = fmaf(qv[gi][i], kf[i], dot);
                    dot = group_sum<LPR>(dot);
                }
                s[u] = (base + u * RPW + grp < kend) ? dot : -INFINITY;
                mblk = fmaxf(mblk, s[u]);
            }
            const float m_new = fmaxf(m[gi], mblk);
            const float alpha = exp2_rel(m[gi], m_new);
            l[gi] *= alpha;
#pragma unroll
            for (int i = 0; i < VEC; ++i) acc[gi][i] *= alpha;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float p = exp2_rel(s[u], m_new);
                float vf[VEC];
                to_floats<T, VEC>(vr[u], vf);
                l[gi] += p;
#pragma unroll
                for (int i = 0; i < VEC; ++i) acc[gi][i] = fmaf(p, vf[i], acc[gi][i]);
            }
            m[gi] = m_new;
        }
    }

    // Merge the RPW row slots of the wave (lanes part, part + LPR, ...).
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
#pragma unroll
        for (int w = LPR; w < 64; w <<= 1) {
            const float m2 = xor_shuffle(m[gi], w);
            const float l2 = xor_shuffle(l[gi], w);
            const float mm = fmaxf(m[gi], m2);
            const float f1 = exp2_rel(m[gi], mm);
            const float f2 = exp2_rel(m2, mm);
            l[gi] = l[gi] * f1 + l2 * f2;
#pragma unroll
            for (int i = 0; i < VEC; ++i)
                acc[gi][i] = acc[gi][i] * f1 + xor_shuffle(acc[gi][i], w) * f2;
            m[gi] = mm;
        }
    }

    // Merge the waves through LDS.
    __shared__ float s_m[Cfg::kWaves][G];
    __shared__ float s_l[Cfg::kWaves][G];
    __shared__ __attribute__((aligned(16))) float s_acc[Cfg::kWaves][G][D];
    if (lane < LPR) {
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
#pragma unroll
            for (int i = 0; i < VEC; ++i) s_acc[wave][gi][part * VEC + i] = acc[gi][i];
            if (lane == 0) {
                s_m[wave][gi] = m[gi];
                s_l[wave][gi] = l[gi];
            }
        }
    }
    __syncthreads();
    if (tid < D) {
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            float mm = -INFINITY;
#pragma unroll
            for (int w = 0; w < Cfg::kWaves; ++w) mm = fmaxf(mm, s_m[w][gi]);
            float lt = 0.0f, at = 0.0f;
#pragma unroll
            for (int w = 0; w < Cfg::kWaves; ++w) {
                const float f = exp2_rel(s_m[w][gi], mm);
                lt += s_l[w][gi] * f;
                at += s_acc[w][gi][tid] * f;
            }
            const size_t slot = (static_cast<size_t>(b) * a.H + h0 + gi) * a.nsplit + split;
            part_acc[slot * D + tid] = at;
            if (tid == 0) part_ml[slot] = make_float2(mm, lt);
        }
    }
}

// LDS-DMA loads (common.hpp's lds_dma16_async / lds_dma16_async_s) with the non-temporal hint:
// a decode reads each key / value row once, so the stream should not displace cached lines.
// `s_nop 4` gives the five wait states that a VALU write of the base or M0 needs before the
// load reads it: the paged base comes from v_readlane / v_readfirstlane (within noise at
// config-4 size).
__device__ __forceinline__ void lds_dma16_nt(const void* src, unsigned char* lds_base) {
    asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :
                 : "v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds_address(lds_base)))
                 : "memory");
}
// A wave-uniform pointer that the compiler cannot prove uniform, read into SGPRs (lane 0's).
__device__ __forceinline__ const uint16_t* uniform_ptr(const uint16_t* p) {
    const uint64_t v = reinterpret_cast<uintptr_t>(p);
    const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
    const uint64_t hi =
        static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v >> 32)));
    return reinterpret_cast<const uint16_t*>(static_cast<uintptr_t>((hi << 32) | lo));
}
__device__ __forceinline__ void lds_dma16_nt_s(const void* sbase, unsigned voff,
                                               unsigned char* lds_base) {
    asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1 nt"
                 :
                 : "v"(voff), "s"(sbase),
                   "{m0}"(__builtin_amdgcn_readfirstlane(lds_address(lds_base)))
                 : "memory");
}

// LDS tile layouts of the matrix-core decode kernels, in TileGroups' interface (row_base of a
// K row read plus k_off(ks); tr_off of a V transpose read plus kTrRows16 per 16 keys, dtile_off
// per 32 dims and kTrHigh for its second half). decode_mma_kernel uses the forward kernels'
// groups, TileGroups<D>. The row layout of decode_mma_rows_kernel (512 / D heads per tile): key
// row r holds the 2D-byte rows of the heads side by side, 1 KB in all, chunk c of head w at r R +
// 2 D w + 16 c, with R = 1040 for K (the 16 rows of a K row read step 16 bytes through the banks)
// and 1088 for V (the 4 rows of a 32-lane transpose read step 64 bytes).
struct DecRowLayout {
    static constexpr int kRowK = 1040;
    static constexpr int kRowV = 1088;
    static constexpr int kTrRows16 = 16 * kRowV;
    static constexpr int kTrHigh = 8 * kRowV;
    static constexpr int k_off(int ks) { return ks * 32; }
    static constexpr int dtile_off(int dt) { return dt * 64; }
};

// One 32-key block of the matrix-core decode for this wave's query heads (lane l32 = head): the
// scores S^T = K Q^T, the mask past kend, the lazily rescaled softmax (m in log2 units, l this
// lane's share of the row sum), and O^T += V^T P^T. kt / vt are the block's K / V tiles; k_base
// (for even and odd k-steps) and v_off are this lane's operand offsets in layout Lay.
template <typename T, int D, class Lay>
__device__ __forceinline__ void decode_mma_block(const unsigned char* kt, const unsigned char* vt,
                                                 const int (&k_base)[2], int v_off, int key0,
                                                 int kend, int g2, float cs,
                                                 const typename Elem<T>::frag (&qf)[D / 16],
                                                 f32x16 (&o)[D / 32], float& m, float& l) {
    using frag = typename Elem<T>::frag;
    constexpr int KS = D / 16;
    constexpr int NDT = D / 32;
    constexpr int BN = 32;
    constexpr int kAhead = 3;
    f32x16 s = f32x16{};
    {
        frag fk[KS];
#pragma unroll
        for (int k = 0; k < kAhead && k < KS; ++k)
            fk[k] = as_frag<T>(ld16(kt + k_base[k & 1] + Lay::k_off(k)));
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            if (ks + kAhead < KS)
                fk[ks + kAhead] =
                    as_frag<T>(ld16(kt + k_base[(ks + kAhead) & 1] + Lay::k_off(ks + kAhead)));
            s = Elem<T>::mma(fk[ks], qf[ks], s);
        }
    }
    if (key0 + BN > kend) {
        const int lim = kend - key0 - 4 * g2;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = (8 * (r >> 2) + (r & 3) < lim) ? s[r] : -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = __builtin_elementwise_maximum(mx, s[r]);
    const float m_new = fmaxf(m, pair_max(mx) * cs);
    const bool grow = m_new > m + kLazyRescale;
    const float alpha = grow ? fast_exp2(m_new == -INFINITY ? 0.0f : m - m_new) : 1.0f;
    m = grow ? m_new : m;
    l *= alpha;
    if (__ballot(grow) != 0) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) o[dt] *= alpha;
    }
    const float m_use = (m == -INFINITY) ? 0.0f : m;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = fast_exp2(fmaf(s[r], cs, -m_use));
    float sum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; r += 2) sum += s[r] + s[r + 1];
    l += sum;
    frag p[2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
        p[h] = pack_frag<T>(s[8 * h + 0], s[8 * h + 1], s[8 * h + 2], s[8 * h + 3], s[8 * h + 4],
                            s[8 * h + 5], s[8 * h + 6], s[8 * h + 7]);
    constexpr int kMma = 2 * NDT;
    frag fv[kMma];
    auto v_frag = [&](int i) {
        const unsigned char* a0 =
            vt + v_off + (i / NDT) * Lay::kTrRows16 + Lay::dtile_off(i % NDT);
        return tr_frag_at<T>(a0, a0 + Lay::kTrHigh);
    };
#pragma unroll
    for (int k = 0; k < kAhead && k < kMma; ++k) fv[k] = v_frag(k);
#pragma unroll
    for (int i = 0; i < kMma; ++i) {
        if (i + kAhead < kMma) fv[i + kAhead] = v_frag(i + kAhead);
        o[i % NDT] = Elem<T>::mma(fv[i], p[i / NDT], o[i % NDT]);
    }
}

// ------------------------------------------------------------------------------------------
// Grouped-query decode on the matrix cores (fp16 / bf16, head_dim 32, 64, 128)
// ------------------------------------------------------------------------------------------
// With several query heads per key/value head, decode_split_kernel is bound by its vector ALU
// (per key and query head: a 16-lane dot product, its reduction and an 8-wide accumulator
// update). Here the G <= 32 query heads of one key/value head are the columns of the forward
// kernels' transposed 32 x 32 tiles: S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_32x32x16, one
// lane per query head (the lanes of columns past G carry zero queries and store nothing), so the
// vector work per key is the softmax of one score per head. One wave per (batch, key/value head,
// split) streams the split's keys in 32-key blocks through LDS-DMA double buffers in the
// forward kernels' group layout, TileGroups<D> (4-row groups at head_dim 128, 8-row groups at
// 64 and 32; K row reads and V transpose reads conflict-free), the next
// block's loads in flight while the current one is consumed; the split's chunk is a multiple
// of 32 keys, so only the last block of a sequence is partial (its rows past the end are
// clamped to the last key and masked). Paged caches (pages of a multiple of the group's rows, so
// a group never crosses a page): each group load is a scalar page base plus a fixed per-lane
// offset (rows of a page are Hkv D elements apart), with the page indices of the next block
// fetched one block ahead. Output: decode_split_kernel's partial (m, l, acc) per
// (query head, split), with m lazily rescaled as in the forward (acc and l always refer to the
// stored m, so the combine is exact).
// At head_dim 128 the LDS (34 KB per workgroup) allows four workgroups, one wave per SIMD; at
// that register budget the compiler keeps the score and O accumulators in AGPRs (16
// v_accvgpr_read per block feed the softmax, O is read back only for a rescale and at the end).
template <typename T, int D, bool PAGED>
__global__ void __launch_bounds__(64)
    decode_mma_kernel(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                      const uint16_t* __restrict__ V, float* __restrict__ part_acc,
                      float2* __restrict__ part_ml, DecodeArgs a) {
    using G = TileGroups<D>;
    constexpr int KS = D / 16;         // k-steps of the score MFMA chain
    constexpr int NDT = D / 32;        // 32-column tiles of O^T
    constexpr int BN = 32;             // keys per block
    constexpr int GR = G::kRows;       // rows per group (one load instruction)
    constexpr int GRP = G::kBytes;     // bytes per group
    constexpr int NG = BN / GR;        // groups per tile
    constexpr int TILE = NG * GRP;
    using frag = typename Elem<T>::frag;
    __shared__ __attribute__((aligned(1024))) unsigned char Kb0[TILE];
    __shared__ __attribute__((aligned(1024))) unsigned char Kb1[TILE];
    __shared__ __attribute__((aligned(1024))) unsigned char Vb0[TILE];
    __shared__ __attribute__((aligned(1024))) unsigned char Vb1[TILE];

    // blockIdx.x = (b * Hkv + hk) * nsplit + split.
    const int hpk = a.H / a.Hkv;
    int rest = blockIdx.x;
    const int split = rest % a.nsplit;
    rest /= a.nsplit;
    const int hk = rest % a.Hkv;
    const int b = rest / a.Hkv;
    const int h0 = hk * hpk;
    const int lane = threadIdx.x;
    const int l32 = lane & 31;
    const int g2 = lane >> 5;

    const int kv_b = PAGED ? min(max(a.seq_lens[b], 0), a.kv_len) : a.kv_len;
    const int kbeg = split * a.chunk;
    const int kend = min(kv_b, kbeg + a.chunk);
    const int nblk = kend > kbeg ? (kend - kbeg + BN - 1) / BN : 0;
    // Contiguous: key row t of this (batch, key/value head) at Kh + t D. Paged: at
    // ((page_of(t) page_size + t % page_size) Hkv + hk) D, consecutive rows of a page Hkv D apart.
    const uint16_t* Kh = PAGED ? K + static_cast<size_t>(hk) * D
                               : K + (static_cast<size_t>(b) * a.Hkv + hk) * static_cast<size_t>(a.kv_len) * D;
    const uint16_t* Vh = PAGED ? V + static_cast<size_t>(hk) * D
                               : V + (static_cast<size_t>(b) * a.Hkv + hk) * static_cast<size_t>(a.kv_len) * D;
    auto page_of = [&](int t) {
        const int j = a.page_shift >= 0 ? t >> a.page_shift : t / a.page_size;
        return a.block_table[static_cast<size_t>(b) * a.max_pages + j];
    };
    // Element offset of key row t from Kh / Vh; `page` is page_of(t) when PAGED.
    auto row_off = [&](int t, int page) -> size_t {
        if constexpr (PAGED) {
            const int r = a.page_shift >= 0 ? t & (a.page_size - 1) : t % a.page_size;
            return (static_cast<size_t>(page) * a.page_size + r) * static_cast<size_t>(a.Hkv) * D;
        } else {
            return static_cast<size_t>(t) * D;
        }
    };

    // Q^T: lane l32 holds query head h0 + l32 (zeros past the group), dims 16 ks + 8 g2 .. + 8.
    frag qf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (l32 < hpk) v = ld16(Q + (static_cast<size_t>(b) * a.H + h0 + l32) * D + 16 * ks + 8 * g2);
        qf[ks] = as_frag<T>(v);
    }

    // Tile loads: group g (rows key0 + GR g .. + GR - 1) by one instruction, lane i: row
    // G::ld_row(i), 16-byte chunk G::ld_col(i) / 8. Whole tiles use a scalar base per group
    // (paged: the page of group g is lane g of `pages`); the last one clamps rows to kend - 1
    // (per-lane addresses).
    const int ld_row = G::ld_row(lane);
    const int ld_col = G::ld_col(lane);
    const int row_pitch = PAGED ? a.Hkv * D : D;
    const unsigned ld_voff = static_cast<unsigned>((ld_row * row_pitch + ld_col) * 2);
    // Page indices of the groups of the block at key0, lane g holding group g (paged only).
    auto fetch_pages = [&](int key0) {
        int pg = 0;
        if constexpr (PAGED) {
            if (lane < NG && key0 + GR * lane < kend) pg = page_of(key0 + GR * lane);
        }
        return pg;
    };
    auto load_tile = [&](const uint16_t* src, int key0, unsigned char* dst, int pages) {
        if (key0 + BN <= kend) {
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                if constexpr (PAGED) {
                    // The base comes from v_readlane and the compiler cannot prove it uniform:
                    // read it into SGPRs (the load statement's wait states cover the VALU write).
                    const uint16_t* sb = src + row_off(key0 + GR * g, __builtin_amdgcn_readlane(pages, g));
                    lds_dma16_nt_s(uniform_ptr(sb), ld_voff, dst + g * GRP);
                } else {
                    lds_dma16_nt_s(src + row_off(key0 + GR * g, 0), ld_voff, dst + g * GRP);
                }
            }
        } else {
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                const int row = min(key0 + GR * g + ld_row, kend - 1);
                lds_dma16_nt(src + row_off(row, PAGED ? page_of(row) : 0) + ld_col, dst + g * GRP);
            }
        }
    };
    // Operand offsets of the group layout: K rows (lane l32 = key, chunk 2 ks + g2; the
    // head_dim-64 groups swizzle by the k-step's parity) and the V transpose reads.
    const int k_base[2] = {G::row_base(lane, 0), G::row_base(lane, 1)};
    const int v_off = G::tr_off(lane);

    f32x16 o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x16{};
    float m = -INFINITY;  // running max of s * c (log2 units), lazily raised
    float l = 0.0f;       // this lane's share of the row sum
    const float cs = fmaxf(a.c, kFltMin);  // scale 0: -inf * 0 would make the masked scores NaN

    auto block = [&](const unsigned char* kt, const unsigned char* vt, int key0) {
        decode_mma_block<T, D, G>(kt, vt, k_base, v_off, key0, kend, g2, cs, qf, o, m, l);
    };

    // Block j in Kb[j & 1] / Vb[j & 1]; block j + 1's loads are issued once block j's have
    // landed (vmcnt(0)), into the buffers block j - 1 used (its LDS reads were consumed by its
    // MFMAs). One wave per workgroup, so no barrier. (A third buffer, two blocks in flight,
    // measured slower: three workgroups per CU instead of four.) Paged: `pages` holds the page
    // indices of the next block to load, fetched with the loads of the block before it.
    int pages = fetch_pages(kbeg);
    if (nblk > 0) {
        load_tile(Kh, kbeg, Kb0, pages);
        load_tile(Vh, kbeg, Vb0, pages);
        pages = fetch_pages(kbeg + BN);
    }
    for (int j = 0; j < nblk; j += 2) {
        __builtin_amdgcn_s_waitcnt(0);
        if (j + 1 < nblk) {
            load_tile(Kh, kbeg + (j + 1) * BN, Kb1, pages);
            load_tile(Vh, kbeg + (j + 1) * BN, Vb1, pages);
            pages = fetch_pages(kbeg + (j + 2) * BN);
        }
        block(Kb0, Vb0, kbeg + j * BN);
        if (j + 1 >= nblk) break;
        __builtin_amdgcn_s_waitcnt(0);
        if (j + 2 < nblk) {
            load_tile(Kh, kbeg + (j + 2) * BN, Kb0, pages);
            load_tile(Vh, kbeg + (j + 2) * BN, Vb0, pages);
            pages = fetch_pages(kbeg + (j + 3) * BN);
        }
        block(Kb1, Vb1, kbeg + (j + 1) * BN);
    }

    // Partials of the query heads of this wave's columns: lane l32 < G holds head h0 + l32,
    // dims 32 dt + 8 q + 4 g2 .. + 3 in o[dt][4 q .. 4 q + 3].
    l = pair_sum(l);
    if (l32 < hpk) {
        const size_t slot = (static_cast<size_t>(b) * a.H + h0 + l32) * a.nsplit + split;
        float* dst = part_acc + slot * D;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
                f32x4 w;
#pragma unroll
                for (int u = 0; u < 4; ++u) w[u] = o[dt][4 * qq + u];
                st16(dst + 32 * dt + 8 * qq + 4 * g2, __builtin_bit_cast(u32x4, w));
            }
        }
        if (g2 == 0) part_ml[slot] = make_float2(m, l);
    }
}

// ------------------------------------------------------------------------------------------
// Paged grouped-query decode on the matrix cores, 1 KB of key/value heads per workgroup
// ------------------------------------------------------------------------------------------
// In the paged layout [page, key, key/value head, D] the rows of one head are 2D-byte pieces
// Hkv D 2 bytes apart, so a wave of decode_mma_kernel streams 2D bytes per key row, where the
// contiguous layout gives it 8 KB runs (head_dim 128 at config-4 size: 10% slower with one page
// per sequence, the same kernel). Here the NW = 512 / D waves of a workgroup (4 at head_dim 128,
// 8 at 64, 16 at 32) take NW adjacent key/value heads of one (batch, split): each LDS-DMA load
// fills one key row of all NW heads (1 KB contiguous in HBM and in LDS), wave w loading rows
// RPW w .. RPW w + RPW - 1 of each tile (RPW = 32 / NW), and the waves share the tiles through
// one barrier per block. The tiles use the row layout (DecRowLayout), 133 KB for the two buffers
// of K and V, one workgroup per CU; each wave runs decode_mma_block on its own head's 2D-byte
// column. A load is one key row with one scalar row index, clamped to the sequence's last key
// past its end (masked), so any page size works.
template <typename T, int D>
__global__ void __launch_bounds__(64 * (512 / D))
    decode_mma_rows_kernel(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                           const uint16_t* __restrict__ V, float* __restrict__ part_acc,
                           float2* __restrict__ part_ml, DecodeArgs a) {
    using Lay = DecRowLayout;
    constexpr int KS = D / 16;
    constexpr int NDT = D / 32;
    constexpr int BN = 32;
    constexpr int NW = 512 / D;   // waves = key/value heads per workgroup
    constexpr int RPW = BN / NW;  // rows of each tile that a wave loads
    using frag = typename Elem<T>::frag;
    __shared__ __attribute__((aligned(1024))) unsigned char Kb0[BN * Lay::kRowK];
    __shared__ __attribute__((aligned(1024))) unsigned char Kb1[BN * Lay::kRowK];
    __shared__ __attribute__((aligned(1024))) unsigned char Vb0[BN * Lay::kRowV];
    __shared__ __attribute__((aligned(1024))) unsigned char Vb1[BN * Lay::kRowV];

    // blockIdx.x = (b * (Hkv / NW) + quad) * nsplit + split; wave w: key/value head NW quad + w.
    const int hpk = a.H / a.Hkv;
    const int nquad = a.Hkv / NW;
    int rest = blockIdx.x;
    const int split = rest % a.nsplit;
    rest /= a.nsplit;
    const int quad = rest % nquad;
    const int b = rest / nquad;
    const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int hk = quad * NW + w;
    const int h0 = hk * hpk;
    const int lane = threadIdx.x & 63;
    const int l32 = lane & 31;
    const int g2 = lane >> 5;

    const int kv_b = min(max(a.seq_lens[b], 0), a.kv_len);
    const int kbeg = split * a.chunk;
    const int kend = min(kv_b, kbeg + a.chunk);
    const int nblk = kend > kbeg ? (kend - kbeg + BN - 1) / BN : 0;
    // Key row t of the NW heads: Kq + ((page_of(t) page_size + t % page_size) Hkv) D.
    const uint16_t* Kq = K + static_cast<size_t>(quad) * NW * D;
    const uint16_t* Vq = V + static_cast<size_t>(quad) * NW * D;
    auto page_of = [&](int t) {
        const int j = a.page_shift >= 0 ? t >> a.page_shift : t / a.page_size;
        return a.block_table[static_cast<size_t>(b) * a.max_pages + j];
    };
    auto row_off = [&](int t, int page) -> size_t {
        const int r = a.page_shift >= 0 ? t & (a.page_size - 1) : t % a.page_size;
        return (static_cast<size_t>(page) * a.page_size + r) * static_cast<size_t>(a.Hkv) * D;
    };

    // Q^T: lane l32 holds query head h0 + l32 (zeros past the group), dims 16 ks + 8 g2 .. + 8.
    frag qf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (l32 < hpk) v = ld16(Q + (static_cast<size_t>(b) * a.H + h0 + l32) * D + 16 * ks + 8 * g2);
        qf[ks] = as_frag<T>(v);
    }

    // Tile loads: row RPW w + i of the block at key0 (clamped to kend - 1) by one instruction,
    // lane i: the 16 bytes at 16 i of the row's 1 KB. Its page is lane i of `pages`.
    const unsigned ld_voff = static_cast<unsigned>(lane * 16);
    auto fetch_pages = [&](int key0) {
        int pg = 0;
        if (lane < RPW && key0 < kend) pg = page_of(min(key0 + RPW * w + lane, kend - 1));
        return pg;
    };
    auto load_tile = [&](const uint16_t* src, int key0, unsigned char* dst, int row_bytes,
                         int pages) {
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const int t = min(key0 + RPW * w + i, kend - 1);
            // The base comes from v_readlane and the compiler cannot prove it uniform: read it
            // into SGPRs (the load statement's wait states cover the VALU write).
            const uint16_t* sb = src + row_off(t, __builtin_amdgcn_readlane(pages, i));
            lds_dma16_nt_s(uniform_ptr(sb), ld_voff, dst + (RPW * w + i) * row_bytes);
        }
    };
    // Operand offsets in the row layout: K rows (lane l32 = key, chunk 2 ks + g2 of head w) and
    // the V transpose reads (rows 4 g2 + (lane % 16) / 4, chunks 2 ((lane / 16) % 2) +
    // (lane % 4) / 2, half lane % 2).
    const int k_off = l32 * Lay::kRowK + w * 2 * D + g2 * 16;
    const int k_base[2] = {k_off, k_off};
    const int kq = lane & 15;
    const int v_off = (4 * g2 + (kq >> 2)) * Lay::kRowV + w * 2 * D +
                      (2 * ((lane >> 4) & 1) + ((kq & 3) >> 1)) * 16 + (kq & 1) * 8;

    f32x16 o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x16{};
    float m = -INFINITY;
    float l = 0.0f;
    const float cs = fmaxf(a.c, kFltMin);  // scale 0: -inf * 0 would make the masked scores NaN

    // Block j in Kb[j & 1] / Vb[j & 1]. Each wave waits for its own loads of block j (vmcnt(0));
    // the barrier after it makes every wave's loads visible and ends every wave's reads of block
    // j - 1, whose buffers block j + 1's loads then fill. `pages` holds the page indices of this
    // wave's rows of the next block to load.
    int pages = fetch_pages(kbeg);
    if (nblk > 0) {
        load_tile(Kq, kbeg, Kb0, Lay::kRowK, pages);
        load_tile(Vq, kbeg, Vb0, Lay::kRowV, pages);
        pages = fetch_pages(kbeg + BN);
    }
    for (int j = 0; j < nblk; j += 2) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (j + 1 < nblk) {
            load_tile(Kq, kbeg + (j + 1) * BN, Kb1, Lay::kRowK, pages);
            load_tile(Vq, kbeg + (j + 1) * BN, Vb1, Lay::kRowV, pages);
            pages = fetch_pages(kbeg + (j + 2) * BN);
        }
        decode_mma_block<T, D, Lay>(Kb0, Vb0, k_base, v_off, kbeg + j * BN, kend, g2, cs, qf, o, m,
                                    l);
        if (j + 1 >= nblk) break;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (j + 2 < nblk) {
            load_tile(Kq, kbeg + (j + 2) * BN, Kb0, Lay::kRowK, pages);
            load_tile(Vq, kbeg + (j + 2) * BN, Vb0, Lay::kRowV, pages);
            pages = fetch_pages(kbeg + (j + 3) * BN);
        }
        decode_mma_block<T, D, Lay>(Kb1, Vb1, k_base, v_off, kbeg + (j + 1) * BN, kend, g2, cs, qf,
                                    o, m, l);
    }

    // Partials of this wave's query heads: lane l32 < G holds head h0 + l32, dims 32 dt + 8 q +
    // 4 g2 .. + 3 in o[dt][4 q .. 4 q + 3].
    l = pair_sum(l);
    if (l32 < hpk) {
        const size_t slot = (static_cast<size_t>(b) * a.H + h0 + l32) * a.nsplit + split;
        float* dst = part_acc + slot * D;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
                f32x4 v;
#pragma unroll
                for (int u = 0; u < 4; ++u) v[u] = o[dt][4 * qq + u];
                st16(dst + 32 * dt + 8 * qq + 4 * g2, __builtin_bit_cast(u32x4, v));
            }
        }
        if (g2 == 0) part_ml[slot] = make_float2(m, l);
    }
}

// Upper bound of the split count (choose_splits).
constexpr int kMaxSplits = 1024;

// One workgroup per (batch*head, 32-column slice of D): its 256 lanes are 8 rows of 32 columns,
// row r sums the splits r, r + 8, ... of its columns with eight loads in flight per lane, and the
// split weights 2^(m_s - M) are formed once into LDS. (One lane per column walking every split
// in sequence was latency-bound at a few heads with hundreds of splits.)
template <typename T, int D>
__global__ void __launch_bounds__(256)
    decode_combine_kernel(const float* __restrict__ part_acc, const float2* __restrict__ part_ml,
                          typename Mma<T>::elem* __restrict__ O, float* __restrict__ L,
                          int nsplit) {
    constexpr int kSlices = D / 32;
    constexpr int kRows = 8;
    constexpr int kInFlight = 8;
    __shared__ float fw[kMaxSplits];
    __shared__ float red[4];
    __shared__ float rows[kRows][33];
    const int bh = blockIdx.x / kSlices;
    const int c0 = (blockIdx.x % kSlices) * 32;
    const int t = threadIdx.x;
    const int wave = t >> 6;
    const float2* ml = part_ml + static_cast<size_t>(bh) * nsplit;
    const float* acc = part_acc + static_cast<size_t>(bh) * nsplit * D;

    float mm = -INFINITY;
    for (int s = t; s < nsplit; s += 256) mm = fmaxf(mm, ml[s].x);
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) mm = fmaxf(mm, xor_shuffle(mm, k));
    if ((t & 63) == 0) red[wave] = mm;
    __syncthreads();
    mm = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float lt = 0.0f;
    for (int s = t; s < nsplit; s += 256) {
        const float2 v = ml[s];
        const float f = exp2_rel(v.x, mm);
        fw[s] = f;
        lt += v.y * f;
    }
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) lt += xor_shuffle(lt, k);
    if ((t & 63) == 0) red[wave] = lt;
    __syncthreads();
    lt = (red[0] + red[1]) + (red[2] + red[3]);

    const int col = t & 31;
    const int row = t >> 5;
    const float* a0 = acc + c0 + col;
    float at = 0.0f;
    int s = row;
    for (; s + (kInFlight - 1) * kRows < nsplit; s += kInFlight * kRows) {
        float x[kInFlight];
#pragma unroll
        for (int u = 0; u < kInFlight; ++u) x[u] = a0[static_cast<size_t>(s + u * kRows) * D];
#pragma unroll
        for (int u = 0; u < kInFlight; ++u) at = fmaf(x[u], fw[s + u * kRows], at);
    }
    for (; s < nsplit; s += kRows) at = fmaf(a0[static_cast<size_t>(s) * D], fw[s], at);
    rows[row][col] = at;
    __syncthreads();
    if (row == 0) {
        float sum = 0.0f;
#pragma unroll
        for (int r = 0; r < kRows; ++r) sum += rows[r][col];
        // lt == 0 only when every split was empty (a paged sequence of length 0): O = 0, L = -inf.
        const float o = lt == 0.0f ? 0.0f : sum / lt;
        const size_t at_o = static_cast<size_t>(bh) * D + c0 + col;
        if constexpr (std::is_same<T, float>::value) {
            O[at_o] = o;
        } else {
            O[at_o] = static_cast<uint16_t>(Elem<T>::pack2(o, 0.0f) & 0xffffu);
        }
        if (c0 == 0 && col == 0) L[bh] = lt == 0.0f ? -INFINITY : (mm + fast_log2(lt)) * kLn2;
    }
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

// Split count: enough (batch*head, split) workgroups to give every CU per_cu, with chunks of at
// least min_chunk keys; an explicit request is clamped to [1, min(1024, ceil(kv_len / 16))]
// (1024 = dev::kMaxSplits, the combine kernel's bound).
int choose_splits(int requested, int BH, int kv_len, int min_chunk, int per_cu) {
    const int max_useful = std::max(1, std::min(dev::kMaxSplits, (kv_len + 15) / 16));
    if (requested > 0) return std::min(requested, max_useful);
    const int target_blocks = per_cu * device_cu_count();
    int s = (target_blocks + BH - 1) / BH;
    s = std::min(s, std::max(1, kv_len / min_chunk));
    return std::max(1, std::min(s, max_useful));
}

// One decode: the layout and head grouping come in `a` (chunk and nsplit are set here).
// Workgroups: one per (batch, key/value head, group of G query heads, split); partials and the
// combine: one slot per (batch, query head).
// Memory for the split partials that the caller provides instead of the stream-ordered
// workspace (ptr == nullptr: allocate one).
struct FixedScratch {
    void* ptr;
    size_t bytes;
};

// Minimum keys per split of the automatic split count (4 blocks of the matrix-core kernels):
// short sequences still spread over the chip (512-key chunks -> 128: plain decode, B = 1, 32
// heads, 1024 keys 13.6 -> 9.0 us; grouped-query, B = 1, 2 key/value heads, 32768 keys 26 ->
// 19 us; config 4's automatic 4 splits are unaffected).
constexpr int kMinChunk = 128;
// Workgroups per CU that the one-head matrix-core kernel's split count aims at: 4 (its LDS
// occupancy at head_dim 128); 8 at head_dim 32, whose 512-byte group loads need more workgroups
// in flight (16 x 8 key/value heads x 32768 keys: 130 -> 89 us; head_dim 64: 156 -> 161 us).
constexpr int mma_per_cu(int D) { return D == 32 ? 8 : 4; }
constexpr int kRowsPerCu = 1;

// MMA: the matrix-core kernels, splits of whole 32-key blocks: decode_mma_rows_kernel (paged,
// one workgroup per (batch, 512 / D key/value heads, split)) or decode_mma_kernel (one
// workgroup per (batch, key/value head, split)), each for all the query heads of its key/value
// heads; else decode_split_kernel with G query heads per workgroup.
template <typename T, int D, int G, bool PAGED, bool MMA = false>
FlashAttentionError run_decode(const T* Q, const T* K, const T* V, T* O, float* L, int B,
                               dev::DecodeArgs a, int num_splits, const FixedScratch& fixed,
                               hipStream_t stream) {
    using E = typename dev::Mma<T>::elem;
    using Cfg = dev::DecCfg<T, D>;
    // Paged caches with a multiple of 512 / D key/value heads: decode_mma_rows_kernel, one
    // workgroup per (batch, 512 / D key/value heads, split).
    constexpr int kRowHeads = 512 / D;
    const bool rows = MMA && PAGED && a.Hkv % kRowHeads == 0;
    const long long groups = static_cast<long long>(B) * (rows ? a.Hkv / kRowHeads : a.Hkv) *
                             (MMA ? 1 : (a.H / a.Hkv) / G);
    const long long bhq = static_cast<long long>(B) * a.H;
    if (groups > 0x7fffffffLL || bhq * (D / 32) > 0x7fffffffLL)
        return FlashAttentionError::INVALID_DIMENSION;
    // The one-head matrix-core kernel's workgroup is one wave: mma_per_cu(D) workgroups per CU
    // (grouped-query decode, head_dim 128, 16 x 8 key/value heads x 32768 keys: 8 -> 4 per CU,
    // 327 -> 314 us). The four-head kernel: one workgroup per CU (its LDS occupancy).
    a.nsplit = choose_splits(num_splits, static_cast<int>(groups), a.kv_len,
                             kMinChunk,
                             rows ? kRowsPerCu : (MMA ? mma_per_cu(D) : 8));
    a.chunk = (a.kv_len + a.nsplit - 1) / a.nsplit;
    if constexpr (MMA) {
        a.chunk = std::max(32, (a.chunk + 31) / 32 * 32);
        a.nsplit = std::max(1, (a.kv_len + a.chunk - 1) / a.chunk);
    }
    const long long blocks = groups * a.nsplit;
    const long long slots = bhq * a.nsplit;
    if (blocks > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;

    const size_t acc_bytes = static_cast<size_t>(slots) * D * sizeof(float);
    const size_t ml_bytes = static_cast<size_t>(slots) * sizeof(float2);
    StreamWorkspace ws(stream, true);
    void* base = fixed.ptr;
    if (base != nullptr) {
        if (acc_bytes + ml_bytes > fixed.bytes) return FlashAttentionError::OUT_OF_MEMORY;
    } else {
        FlashAttentionError err = ws.alloc(acc_bytes + ml_bytes);
        if (err != FlashAttentionError::SUCCESS) return err;
        base = ws.get();
    }
    // Every (query head, split) slot is written by the split kernel before the combine kernel
    // reads it, so neither buffer needs clearing.
    float* part_acc = static_cast<float*>(base);
    float2* part_ml = reinterpret_cast<float2*>(static_cast<char*>(base) + acc_bytes);

    ProfileEvents tok = profile_kernel<T, D>("decode_split");
    if constexpr (MMA) {
        static_assert((D == 32 || D == 64 || D == 128) && !std::is_same<T, float>::value,
                      "MMA decode shape");
        bool launched = false;
        if constexpr (PAGED) {
            if (rows) {
                launch_kernel(tok, (dev::decode_mma_rows_kernel<T, D>),
                                   dim3(static_cast<unsigned>(blocks)), dim3(64 * kRowHeads), 0,
                                   stream,
                                   reinterpret_cast<const uint16_t*>(Q),
                                   reinterpret_cast<const uint16_t*>(K),
                                   reinterpret_cast<const uint16_t*>(V), part_acc, part_ml, a);
                launched = true;
            }
        }
        if (!launched)
            launch_kernel(tok, (dev::decode_mma_kernel<T, D, PAGED>),
                               dim3(static_cast<unsigned>(blocks)), dim3(64), 0, stream,
                               reinterpret_cast<const uint16_t*>(Q),
                               reinterpret_cast<const uint16_t*>(K),
                               reinterpret_cast<const uint16_t*>(V), part_acc, part_ml, a);
    } else {
        launch_kernel(tok, (dev::decode_split_kernel<T, D, G, PAGED>),
                           dim3(static_cast<unsigned>(blocks)), dim3(Cfg::kThreads), 0, stream,
                           reinterpret_cast<const E*>(Q), reinterpret_cast<const E*>(K),
                           reinterpret_cast<const E*>(V), part_acc, part_ml, a);
    }
    FlashAttentionError err = from_hip(hipGetLastError());
    if (err != FlashAttentionError::SUCCESS) return err;
    tok = profile_kernel<T, D>("decode_combine");
    launch_kernel(tok, (dev::decode_combine_kernel<T, D>),
                       dim3(static_cast<unsigned>(bhq * (D / 32))), dim3(256), 0, stream, part_acc,
                       part_ml, reinterpret_cast<E*>(O), L, a.nsplit);
    return from_hip(hipGetLastError());
}

// fp16 / bf16 with 2 to 32 query heads per key/value head: the matrix-core kernels (below).
// Otherwise G = the largest of 8, 4, 2, 1 that divides the query heads per key/value head: each
// K/V row is then read once for G query heads.
template <typename T, int D, bool PAGED>
FlashAttentionError run_decode_grouped(const T* Q, const T* K, const T* V, T* O, float* L, int B,
                                       const dev::DecodeArgs& a, int num_splits,
                                       const FixedScratch& fx, hipStream_t stream) {
    const int hpk = a.H / a.Hkv;
    if constexpr (!std::is_same<T, float>::value) {
        // 2 to 32 query heads per key/value head: the matrix-core kernels. Paged caches: the
        // rows kernel for a multiple of 512 / D key/value heads (any page size), else the
        // one-head kernel for pages of a multiple of its group's rows (4 at head_dim 128, 8 at
        // 64 and 32) whose per-lane byte offset within a group, (rows - 1) Hkv D 2 + 256, fits
        // 32 bits.
        constexpr int kGroupRows = dev::TileGroups<D>::kRows;
        if (hpk >= 2 && hpk <= 32 &&
            (!PAGED || a.Hkv % (512 / D) == 0 ||
             (a.page_size % kGroupRows == 0 && a.Hkv <= (1 << 20))))
            return run_decode<T, D, 1, PAGED, true>(Q, K, V, O, L, B, a, num_splits, fx, stream);
    }
    if (hpk % 8 == 0)
        return run_decode<T, D, 8, PAGED>(Q, K, V, O, L, B, a, num_splits, fx, stream);
    if (hpk % 4 == 0)
        return run_decode<T, D, 4, PAGED>(Q, K, V, O, L, B, a, num_splits, fx, stream);
    if (hpk % 2 == 0)
        return run_decode<T, D, 2, PAGED>(Q, K, V, O, L, B, a, num_splits, fx, stream);
    return run_decode<T, D, 1, PAGED>(Q, K, V, O, L, B, a, num_splits, fx, stream);
}

template <typename T, bool PAGED>
FlashAttentionError run_decode_dims(const T* Q, const T* K, const T* V, T* O, float* L, int B,
                                    const dev::DecodeArgs& a, int head_dim, int num_splits,
                                    const FixedScratch& fx, hipStream_t stream) {
    switch (head_dim) {
        case 32:
            return run_decode_grouped<T, 32, PAGED>(Q, K, V, O, L, B, a, num_splits, fx, stream);
        case 64:
            return run_decode_grouped<T, 64, PAGED>(Q, K, V, O, L, B, a, num_splits, fx, stream);
        case 128:
            return run_decode_grouped<T, 128, PAGED>(Q, K, V, O, L, B, a, num_splits, fx, stream);
    }
    return FlashAttentionError::UNSUPPORTED_HEAD_DIM;
}

constexpr FixedScratch kAllocate{nullptr, 0};

dev::DecodeArgs decode_args(int num_heads, int num_kv_heads, int kv_len, float scale) {
    dev::DecodeArgs a{};
    a.H = num_heads;
    a.Hkv = num_kv_heads;
    a.kv_len = kv_len;
    a.page_size = 1;
    a.max_pages = 0;
    a.page_shift = -1;
    a.c = scale * dev::kLog2e;
    return a;
}

}  // namespace

template <typename T>
FlashAttentionError launch_decode_gqa(const T* Q, const T* K, const T* V, T* O, float* L,
                                      int batch_size, int num_heads, int num_kv_heads,
                                      int kv_len, int head_dim, float scale, int num_splits,
                                      hipStream_t stream) {
    const dev::DecodeArgs a = decode_args(num_heads, num_kv_heads, kv_len, scale);
    return run_decode_dims<T, false>(Q, K, V, O, L, batch_size, a, head_dim, num_splits,
                                     kAllocate, stream);
}

template <typename T>
FlashAttentionError launch_decode(const T* Q, const T* K, const T* V, T* O, float* L,
                                  int batch_size, int num_heads, int kv_len, int head_dim,
                                  float scale, int num_splits, hipStream_t stream) {
    return launch_decode_gqa<T>(Q, K, V, O, L, batch_size, num_heads, num_heads, kv_len,
                                head_dim, scale, num_splits, stream);
}

template <typename T>
FlashAttentionError launch_decode_paged(const T* Q, const T* K_cache, const T* V_cache, T* O,
                                        float* L, const int* block_table, const int* seq_lens,
                                        int batch_size, int num_heads, int num_kv_heads,
                                        int page_size, int max_pages_per_seq, int head_dim,
                                        float scale, int num_splits, hipStream_t stream) {
    const long long cap = static_cast<long long>(page_size) * max_pages_per_seq;
    if (cap > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
    dev::DecodeArgs a = decode_args(num_heads, num_kv_heads, static_cast<int>(cap), scale);
    a.block_table = block_table;
    a.seq_lens = seq_lens;
    a.page_size = page_size;
    a.max_pages = max_pages_per_seq;
    a.page_shift = (page_size & (page_size - 1)) == 0 ? __builtin_ctz(page_size) : -1;
    return run_decode_dims<T, true>(Q, K_cache, V_cache, O, L, batch_size, a, head_dim,
                                    num_splits, kAllocate, stream);
}

// ---------------------------------------------------------------------------------------------
// Decode without allocation (cuflash_attention_decode_noalloc_f16): the split partials live in
// `scratch`, a file-scope device array of kDecodeScratchBytes that every GPU the library runs on
// holds until the process ends. Its device address is looked up once per device with that
// device current (hipGetSymbolAddress: each GPU has its own copy at its own address); host code
// only ever passes that address, never the array's name, to kernels. Calls on one GPU share the
// array, so calls that overlap in time on one GPU (two streams, two host threads) race; calls
// ordered on one stream do not. Nothing in it has to start at zero (see run_decode).
// ---------------------------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[kDecodeScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device (looked up on the first call per device).
FlashAttentionError scratch_address(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return FlashAttentionError::CUDA_ERROR;
    }
    if (dev < 0 || dev >= kMaxScratchDevices) return FlashAttentionError::CUDA_ERROR;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            (void)hipGetLastError();
            return FlashAttentionError::CUDA_ERROR;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return FlashAttentionError::SUCCESS;
}
}  // namespace

template <typename T>
FlashAttentionError launch_decode_noalloc(const T* Q, const T* K, const T* V, T* O, float* L,
                                          int batch_size, int num_heads, int kv_len,
                                          int head_dim, float scale, int num_splits,
                                          hipStream_t stream) {
    void* ptr = nullptr;
    FlashAttentionError err = scratch_address(&ptr);
    if (err != FlashAttentionError::SUCCESS) return err;
    const dev::DecodeArgs a = decode_args(num_heads, num_heads, kv_len, scale);
    const FixedScratch fx{ptr, kDecodeScratchBytes};
    return run_decode_dims<T, false>(Q, K, V, O, L, batch_size, a, head_dim, num_splits, fx,
                                     stream);
}

template FlashAttentionError launch_decode_noalloc<__half>(const __half*, const __half*,
                                                           const __half*, __half*, float*, int,
                                                           int, int, int, float, int,
                                                           hipStream_t);

#define CUFLASH_DECODE_TYPE(T)                                                                  \
    template FlashAttentionError launch_decode<T>(const T*, const T*, const T*, T*, float*, int, \
                                                  int, int, int, float, int, hipStream_t);      \
    template FlashAttentionError launch_decode_gqa<T>(const T*, const T*, const T*, T*, float*, \
                                                      int, int, int, int, int, float, int,      \
                                                      hipStream_t);                             \
    template FlashAttentionError launch_decode_paged<T>(                                        \
        const T*, const T*, const T*, T*, float*, const int*, const int*, int, int, int, int,   \
        int, int, float, int, hipStream_t);
CUFLASH_DECODE_TYPE(float)
CUFLASH_DECODE_TYPE(__half)
CUFLASH_DECODE_TYPE(__hip_bfloat16)
#undef CUFLASH_DECODE_TYPE

}  // namespace detail
}  // namespace cuflash
