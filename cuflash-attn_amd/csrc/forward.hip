// FlashAttention forward for gfx950 (MI355X).
//
// Replaces the reference's scalar forward kernel (src/forward/flash_attention_forward_typed.cu
// :16-152) and its WMMA kernel (src/forward/flash_attention_forward_wmma.cu:30-207) with MFMA
// kernels of the same math:
//   fwd16_d128_kernel, fwd16_d64_kernel, fwd16_d256_kernel: fp16 / bf16 inputs on
//       v_mfma_f32_32x32x16_{f16,bf16}, fp32 accumulate, software-pipelined with LDS-DMA tiles
//       (head_dim 128 and 96, 64 and 32, 256; described at their definitions). P is rounded to
//       T before P*V while the row sum uses the fp32 P, as in the reference WMMA kernel
//       (forward_wmma.cu:151-156).
//   fwd32_kernel<D>, fwd32_split_kernel<D>: fp32 inputs on v_mfma_f32_32x32x2f32 (full fp32
//       products), P kept fp32 as in the reference scalar kernel (forward_typed.cu:113-129).
//
// Work decomposition: each wave owns 32 query rows of one (batch, head), a workgroup 4 or 8
// waves. The kernel streams key/value blocks through LDS;
// per block each wave computes S^T = K Q^T (A = K tile from LDS, B = Q^T held in registers for
// the whole kernel), runs the online softmax on the accumulator tile in place, and accumulates
// O^T += V^T P^T (A = V tile read with LDS transpose reads, B = P straight from the score
// registers). Each lane therefore owns one query row of O, and the softmax rescale is a per-lane
// multiply. The next K/V block is loaded (LDS-DMA for fp16 / bf16, through registers for fp32)
// while the current one is consumed.
// Blocks of one head share an XCD (item_order); causal launches process the longest query
// blocks first, non-causal ones the blocks of one head after another (equal blocks: the blocks
// of a head then run together and share their K/V rows in L2).
//
// Shapes: Q and O are [BH, Nq, D], K and V are [BH / group, Nk, D] (query head bh reads
// key/value head bh / group), L is [BH, Nq]. With a causal mask query i sees the keys
// j <= i + coff, coff = Nk - Nq >= 0 (the queries are the last Nq positions of the key
// sequence; Nq == Nk gives the usual j <= i).

#include "common.hpp"
#include "launch.hpp"
#include "profile.hpp"
#include "softmax.hpp"

namespace cuflash {
namespace dev {

// ------------------------------------------------------------------------------------------
// fp16 / bf16 kernel for head_dim 128 (the headline shape), software-pipelined
// ------------------------------------------------------------------------------------------
// The per-wave decomposition above (32 query rows per wave, S^T = K Q^T with Q^T in
// registers, O^T += V^T P^T), restructured for gfx950:
//  * a workgroup holds NW waves (32 NW query rows) and one workgroup runs per CU for NW = 8:
//    the K/V tiles a workgroup loads are shared by all its waves, and a CU's vector memory
//    path (about 64 bytes per clock) is the limit of the tile loads, so the larger workgroup
//    halves the load time per MFMA compared with two workgroups of four waves;
//  * K and V blocks of 64 keys go global -> LDS with global_load_lds_dwordx4 (no staging
//    registers, no VALU or ds_write for the copy) into double buffers, so one barrier per block
//    suffices and the next blocks load while the current one is consumed;
//  * LDS layout of a 64 x 128 tile: 16 groups of 4 rows, 1088 bytes each (1 KB + 64 bytes of
//    padding); inside a group the 16-byte chunk c of row r sits at (4 c + r % 4) * 16. One load
//    instruction fills one group (lane i: row r0 + i % 4, chunk i / 4, i.e. 1 KB of contiguous
//    global memory), and both consumers read conflict-free with immediate offsets: the K row
//    reads of S^T (16 rows, one chunk: 4 groups x 4 rows -> 16 distinct 16-byte bank slots) and
//    the V transpose reads of P V (4 rows x 4 chunks of one group: 256 contiguous bytes);
//  * the scores of block j+1 are formed by MFMA while the softmax of block j runs on the VALU
//    (two score register sets), and P V of block j follows;
//  * the lane-pair row max / sum use v_permlane32_swap instead of an LDS permute.
template <typename T, int NW, int D>
__global__ void __launch_bounds__(64 * NW, 8 / NW)
    fwd16_d128_kernel(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                      const uint16_t* __restrict__ V, uint16_t* __restrict__ O,
                      float* __restrict__ L, int Nq, int Nk, int coff, int group, int nqb,
                      float c, int causal) {
    static_assert(D == 128 || D == 96, "rows of at most 256 bytes, 4-row groups");
    constexpr int KS = D / 16;   // k-steps of a score MFMA chain
    constexpr int NDT = D / 32;  // 32-column tiles of O
    constexpr int BM = 32 * NW;  // query rows per workgroup (NW waves of 32 rows)
    constexpr int BN = 64;
    constexpr int kParts = 16 / NW;  // load instructions per wave per 64-row tile
    constexpr int GRP = 1088;              // bytes per 4-row group
    constexpr int TILE = (BN / 4) * GRP;   // bytes per 64-row tile
    using frag = typename Elem<T>::frag;
    __shared__ __attribute__((aligned(1024))) unsigned char Kb0[TILE];
    __shared__ __attribute__((aligned(1024))) unsigned char Kb1[TILE];
    __shared__ __attribute__((aligned(1024))) unsigned char Vb0[TILE];
    __shared__ __attribute__((aligned(1024))) unsigned char Vb1[TILE];

    int bh, rank;
    item_order(blockIdx.x, gridDim.x / nqb, nqb, causal == 0, bh, rank);
    const int qb = causal ? nqb - 1 - rank : rank;  // causal: longest query blocks first
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int l32 = lane & 31;
    const int g2 = lane >> 5;

    const size_t head = static_cast<size_t>(bh) * Nq * D;             // Q, O
    const size_t kv_head = static_cast<size_t>(bh / group) * Nk * D;  // K, V
    const uint16_t* Kh = K + kv_head;
    const uint16_t* Vh = V + kv_head;
    const int q0 = qb * BM + wave * 32;  // first query row of this wave
    const int q = q0 + l32;              // query row owned by this lane

    frag qf[D / 16];
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (q < Nq) v = ld16(Q + head + static_cast<size_t>(q) * D + 16 * ks + 8 * g2);
        qf[ks] = as_frag<T>(v);
    }

    const int kv_end = causal ? min(Nk, (qb + 1) * BM + coff) : Nk;
    const int nkb = (kv_end + BN - 1) / BN;

    // Loads of one 64-row tile: wave w fills groups w, w + NW, ... (kParts of them). Rows past
    // Nk are clamped to row Nk - 1 (finite values; their scores are masked). The loads are issued from
    // inline assembly, so the compiler adds no waits for them and keeps partial LDS waits for
    // the operand reads; the loop orders every LDS access itself (s_waitcnt(0) and a barrier
    // before a tile is read and before a buffer is refilled).
    // A tile that lies inside [0, Nk) is addressed as a scalar base plus a fixed per-lane offset.
    const int ld_row = lane & 3;
    // At head_dim 96 a row fills chunks 0-11 of its 256-byte slot; lanes 48-63 load chunks 0-3
    // again into the unused slots 12-15.
    const int ld_col = ((lane >> 2) % (D / 8)) * 8;
    const unsigned ld_voff = static_cast<unsigned>(((4 * wave + ld_row) * D + ld_col) * 2);
    // Part i (0..kParts-1) of a tile load: this wave's group wave + NW i.
    auto load_part = [&](const uint16_t* src, int key0, unsigned char* dst, int i) {
        if (key0 + BN <= Nk) {
            lds_dma16_async_s(src + static_cast<size_t>(key0 + 4 * NW * i) * D, ld_voff,
                              dst + (wave + NW * i) * GRP);
        } else {
            const int grp = wave + NW * i;
            const int row = min(key0 + 4 * grp + ld_row, Nk - 1);
            lds_dma16_async(src + static_cast<size_t>(row) * D + ld_col, dst + grp * GRP);
        }
    };
    auto load_tile = [&](const uint16_t* src, int key0, unsigned char* dst) {
#pragma unroll
        for (int i = 0; i < kParts; ++i) load_part(src, key0, dst, i);
    };
    // Per-lane byte offsets of the operand reads (see the layout above).
    const int k_off = (l32 >> 2) * GRP + g2 * 64 + (l32 & 3) * 16;
    const int kq = lane & 15;
    const int v_off = g2 * GRP + (2 * ((lane >> 4) & 1) + ((kq & 3) >> 1)) * 64 + (kq >> 2) * 16 +
                      (kq & 1) * 8;

    auto scores = [&](const unsigned char* kt, f32x16 (&s)[2]) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            s[t] = f32x16{};
#pragma unroll
            for (int ks = 0; ks < D / 16; ++ks)
                s[t] = Elem<T>::mma(as_frag<T>(ld16(kt + k_off + 8 * t * GRP + ks * 128)), qf[ks],
                                    s[t]);
        }
    };

    f32x16 o[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) o[dt] = f32x16{};
    float m = -INFINITY;  // running max of s * cs (log2 units)
    float l = 0.0f;       // this lane's share of the running row sum
    // Exponent scale, kept positive so that a masked score (-inf) always maps to p = 0, also
    // for scale = 0 (where FLT_MIN leaves every p at 1 and L at log(count), as with 0).
    const float cs = fmaxf(c, kFltMin);

    // Keys past Nk and, with a causal mask, keys after this lane's row get s = -inf.
    auto mask_scores = [&](f32x16 (&s)[2], int key0) {
        const int lim = min(Nk, causal ? q + 1 + coff : Nk) - key0 - 4 * g2;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int off = 32 * t + 8 * (r >> 2) + (r & 3);
                s[t][r] = off < lim ? s[t][r] : -INFINITY;
            }
        }
    };

    // Online-softmax update of (m, l) from mx, this lane's raw row max of the next block.
    // Returns whether some lane of the wave must rescale its O by alpha. The lazy rescale is
    // decided per lane with selects: m only moves when the block max exceeds it by more than
    // kLazyRescale, and O and l of that lane are scaled by the same alpha, so the result is
    // exact either way.
    auto update_max = [&](float mx, float& alpha) -> bool {
        const float m_new = fmaxf(m, pair_max(mx) * cs);
        const bool grow = m_new > m + kLazyRescale;
        const float a_raw = fast_exp2(m_new == -INFINITY ? 0.0f : m - m_new);
        alpha = grow ? a_raw : 1.0f;
        m = grow ? m_new : m;
        l *= alpha;
        return __ballot(grow) != 0;
    };

    // Operand fragment i of the score MFMAs (K rows of tile half i / 8, k-step i % 8) and of
    // the P V MFMAs (V^T for key group i / 4 and d tile i % 4).
    auto k_frag = [&](const unsigned char* kt, int i) {
        return as_frag<T>(ld16(kt + k_off + 8 * (i / KS) * GRP + (i % KS) * 128));
    };
    auto v_frag = [&](const unsigned char* vt, int i) {
        const unsigned char* a0 = vt + v_off + 4 * (i / NDT) * GRP + (i % NDT) * 256;
        return tr_frag_at<T>(a0, a0 + 2 * GRP);
    };

    // Blocks that need masking: keys past Nk, and with a causal mask the blocks that reach past
    // the last key this wave's first row sees.
    auto needs_mask = [&](int key0) {
        return key0 + BN > Nk || (causal && key0 + BN - 1 > q0 + coff);
    };

    // Exponential of score r of tile t, and the rounding of tile t's group h of eight scores
    // to T (the P operand of key group 2 t + h).
    auto exp_one = [&](f32x16 (&s)[2], int t, int r, float m_use) {
        s[t][r] = fast_exp2(fmaf(s[t][r], cs, -m_use));
    };
    auto pack_p = [&](f32x16 (&s)[2], int t, int h) {
        u32x4 pw = __builtin_bit_cast(
            u32x4, pack_frag<T>(s[t][8 * h + 0], s[t][8 * h + 1], s[t][8 * h + 2],
                                s[t][8 * h + 3], s[t][8 * h + 4], s[t][8 * h + 5],
                                s[t][8 * h + 6], s[t][8 * h + 7]));
        // Keep the exponentials where they are placed: left alone, the compiler sinks them
        // to their first use past the branches in between.
        asm volatile("" : "+v"(pw));
        return __builtin_bit_cast(frag, pw);
    };

    // One block with an explicit instruction order (the scheduling fences keep it), so that
    // each MFMA is followed by a few VALU ops that do not depend on it:
    //   phase A: the 16 MFMAs of the next block's scores (K tile kt) into s_next; after the
    //            first kDelay of them the online-softmax update with the current block's max
    //            mx_cur (formed in the previous phase B; its dependent chain of cross-lane max,
    //            compare, exp2 and ballot then overlaps MFMAs in flight instead of idling both
    //            waves of a SIMD before the barrier: config 3 1.3-3% faster, bitwise equal), then
    //            with each MFMA the exponential of one score of the current tile 0 (P groups 0
    //            and 1);
    //   phase B: the 16 MFMAs of O^T += V^T P^T (V tile vt), the first eight with the
    //            exponentials of two scores of tile 1 (P groups 2 and 3, first used by MFMA 8),
    //            each with two terms of the row sum and the max of two scores of s_next.
    // This splits the VALU work about evenly between the phases (the two waves of a SIMD run
    // the same phase at the same time). The row sum is taken over the fp32 exponentials, before
    // their rounding to T for P V, as in the reference. The next block's mask is applied
    // between the phases. Every
    // operand is read kAhead MFMAs before its product; the first V operands are read under the
    // last score MFMAs. The tile loads of the iteration (K rows from kl_key0 into kl_dst if
    // kl_do, V rows from vl_key0 into vl_dst if vl_do) are spread over the score MFMAs: issued
    // together, the loads of all waves of a CU queue up behind each other and hold back the
    // MFMAs. Returns this lane's raw row max of s_next.
    auto step = [&](f32x16 (&s)[2], const unsigned char* kt, f32x16 (&s_next)[2],
                    const unsigned char* vt, int key0_next, bool kl_do, int kl_key0,
                    unsigned char* kl_dst, bool vl_do, int vl_key0,
                    unsigned char* vl_dst, float mx_cur) -> float {
        constexpr int kAhead = 3;
        constexpr int kMma = 4 * NDT;  // MFMAs per phase (16 at head_dim 128, 12 at 96)
        constexpr int kDelay = 3;      // phase-A MFMAs before the max update
        static_assert(kAhead <= kMma, "operands read ahead within the chain");
        float m_use = 0.0f;
        frag p[4];
        frag fk[kMma];
        frag fv[kMma];
        s_next[0] = f32x16{};
        s_next[1] = f32x16{};
#pragma unroll
        for (int k = 0; k < kAhead; ++k) fk[k] = k_frag(kt, k);
#pragma unroll
        for (int i = 0; i < kMma; ++i) {
            if (i + kAhead < kMma) fk[i + kAhead] = k_frag(kt, i + kAhead);
            else fv[i + kAhead - kMma] = v_frag(vt, i + kAhead - kMma);
            s_next[i / KS] = Elem<T>::mma(fk[i], qf[i % KS], s_next[i / KS]);
            // Load slots: K part j after MFMA (j + 1) h / kParts - 1 of the first half (h = kMma
            // / 2 MFMAs), V part j at the same place in the second half.
#pragma unroll
            for (int j = 0; j < kParts; ++j) {
                constexpr int h = kMma / 2;
                if (i == (j + 1) * h / kParts - 1 && kl_do) load_part(Kh, kl_key0, kl_dst, j);
                if (i == h + (j + 1) * h / kParts - 1 && vl_do) load_part(Vh, vl_key0, vl_dst, j);
            }
            if (i == kDelay - 1) {
                // Online-softmax update with this block's max (formed in the previous phase B),
                // here where its latency overlaps the score MFMAs in flight.
                float alpha;
                if (update_max(mx_cur, alpha)) {
#pragma unroll
                    for (int dt = 0; dt < D / 32; ++dt) o[dt] *= alpha;
                }
                m_use = (m == -INFINITY) ? 0.0f : m;
            }
            if (i >= kDelay) {
                constexpr int kN = kMma - kDelay;
#pragma unroll
                for (int e = 16 * (i - kDelay) / kN; e < 16 * (i - kDelay + 1) / kN; ++e) {
                    exp_one(s, 0, e, m_use);
                    if ((e & 7) == 7) p[e >> 3] = pack_p(s, 0, e >> 3);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (needs_mask(key0_next)) mask_scores(s_next, key0_next);
        float mx = -INFINITY;
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < kMma; ++i) {
            if (i + kAhead < kMma) fv[i + kAhead] = v_frag(vt, i + kAhead);
            o[i % NDT] = Elem<T>::mma(fv[i], p[i / NDT], o[i % NDT]);
            // Tile-1 exponentials in the first half (P groups 2 and 3 are first used there by
            // MFMA kMma / 2 and 3 kMma / 4).
            if (i < kMma / 2) {
#pragma unroll
                for (int e = 32 * i / kMma; e < 32 * (i + 1) / kMma; ++e) {
                    exp_one(s, 1, e, m_use);
                    if ((e & 7) == 7) p[2 + (e >> 3)] = pack_p(s, 1, e >> 3);
                }
            }
            // Row sum of the fp32 exponentials (tile 0 in the first half, tile 1 in the second)
            // and row max of s_next, pairs k of scores.
#pragma unroll
            for (int kk = 16 * i / kMma; kk < 16 * (i + 1) / kMma; ++kk) {
                const int t = kk >> 3;
                const int r = 2 * (kk & 7);
                sum += s[t][r] + s[t][r + 1];
                mx = __builtin_elementwise_maximum(
                    __builtin_elementwise_maximum(mx, s_next[t][r]), s_next[t][r + 1]);
            }
            // Keep both chains here: left alone, the compiler sinks them to their first use.
            asm volatile("" : "+v"(sum), "+v"(mx));
            __builtin_amdgcn_sched_barrier(0);
        }
        l += sum;
        return mx;
    };

    // Block j: K_j in Kb[j & 1], V_j in Vb[j & 1]. At the top of iteration j the loads issued
    // one iteration earlier (K_{j+1}, V_j) are waited for and a barrier makes them visible and
    // retires every read of K_j and V_{j-1}; then K_{j+2} and V_{j+1} are issued into those
    // buffers during the score MFMAs. Each iteration also forms the scores of block j+1 and
    // their row max, which the next iteration applies (for the last block they come from a
    // stale buffer and the max is never used). The loop is unrolled by two so that every buffer
    // is a distinct LDS object.
    load_tile(Kh, 0, Kb0);
    load_tile(Vh, 0, Vb0);
    if (nkb > 1) load_tile(Kh, BN, Kb1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    f32x16 sa[2], sb[2];
    scores(Kb0, sa);
    if (needs_mask(0)) mask_scores(sa, 0);
    // Raw row max of the block whose scores are in the current set (step() applies it).
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = __builtin_elementwise_maximum(mx, sa[t][r]);
    }
    // Key blocks this wave computes: with a causal mask its rows see keys up to q0 + 31 + coff,
    // and up to three of the workgroup's last four blocks lie entirely past them (the keys of
    // such a block would all get p = 0). The wave leaves the compute loop after its last block
    // and runs the remaining iterations as load-only steps (its share of the tile loads, and the
    // barrier), so every wave passes the same barriers and the other waves of its SIMD get the
    // matrix unit to themselves.
    const int nkb_w = causal ? min(nkb, (q0 + 32 + coff + BN - 1) / BN) : nkb;
    int j = 0;
    for (; j < nkb_w; j += 2) {
        // ---- even block j: scores in sa, K_j in Kb0, V_j in Vb0 ----
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        mx = step(sa, Kb1, sb, Vb0, (j + 1) * BN, j + 2 < nkb, (j + 2) * BN, Kb0,
                  j + 1 < nkb, (j + 1) * BN, Vb1, mx);
        if (j + 1 >= nkb_w) {
            ++j;
            break;
        }
        // ---- odd block j + 1: scores in sb, K_{j+1} in Kb1, V_{j+1} in Vb1 ----
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        mx = step(sb, Kb0, sa, Vb1, (j + 2) * BN, j + 3 < nkb, (j + 3) * BN, Kb1,
                  j + 2 < nkb, (j + 2) * BN, Vb0, mx);
    }
    // Load-only iterations j = nkb_w .. nkb - 1 (the same buffers as the compute iterations).
    for (j = nkb_w; j < nkb; ++j) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (j + 2 < nkb) load_tile(Kh, (j + 2) * BN, (j & 1) ? Kb1 : Kb0);
        if (j + 1 < nkb) load_tile(Vh, (j + 1) * BN, (j & 1) ? Vb0 : Vb1);
    }

    // Epilogue: O = O / l, L = m + log(l) (natural log), stored with RNE. O goes through the K/V
    // buffers (two waves' rows per buffer), free once every wave is past its last block.
    l = pair_sum(l);
    static_assert(2 * staged_rows_bytes<D>() <= TILE, "two waves' O rows per K/V buffer");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    store_rows_staged<T, D>(o, 1.0f / l,
                            (wave < 2 ? Kb0 : wave < 4 ? Kb1 : wave < 6 ? Vb0 : Vb1) +
                                (wave & 1) * staged_rows_bytes<D>(),
                            O + head, q0, Nq);
    if (g2 == 0 && q < Nq) L[static_cast<size_t>(bh) * Nq + q] = (m + fast_log2(l)) * kLn2;
}

// ------------------------------------------------------------------------------------------
// fp16 / bf16 kernel for head_dim 256
// ------------------------------------------------------------------------------------------
// fwd16_d128_kernel's data path and pipeline at head_dim 256: a 4-row group holds the two
// 128-column halves of its rows one after the other, each in the 1 KB layout of the head_dim-128
// groups, plus 64 bytes of padding (so row reads and transpose reads stay conflict-free as
// there). O (8 accumulator tiles) and Q^T (16 fragments) need one workgroup of NW waves per
// CU, i.e. one wave per SIMD for NW = 4.
template <typename T, int NW>
__global__ void __launch_bounds__(64 * NW, 1)
    fwd16_d256_kernel(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                      const uint16_t* __restrict__ V, uint16_t* __restrict__ O,
                      float* __restrict__ L, int Nq, int Nk, int coff, int group, int nqb,
                      float c, int causal) {
    constexpr int D = 256;
    constexpr int BM = 32 * NW;  // query rows per workgroup (NW waves of 32 rows)
    constexpr int BN = 64;
    constexpr int kParts = 32 / NW;  // load instructions per wave per 64-row tile
    constexpr int HALF = 1024;             // bytes of one 128-column half of a 4-row group
    constexpr int GRP = 2 * HALF + 64;     // bytes per 4-row group
    constexpr int TILE = (BN / 4) * GRP;   // bytes per 64-row tile
    using frag = typename Elem<T>::frag;
    __shared__ __attribute__((aligned(1024))) unsigned char Kb0[TILE];
    __shared__ __attribute__((aligned(1024))) unsigned char Kb1[TILE];
    __shared__ __attribute__((aligned(1024))) unsigned char Vb0[TILE];
    __shared__ __attribute__((aligned(1024))) unsigned char Vb1[TILE];

    int bh, rank;
    item_order(blockIdx.x, gridDim.x / nqb, nqb, causal == 0, bh, rank);
    const int qb = causal ? nqb - 1 - rank : rank;  // causal: longest query blocks first
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int l32 = lane & 31;
    const int g2 = lane >> 5;

    const size_t head = static_cast<size_t>(bh) * Nq * D;             // Q, O
    const size_t kv_head = static_cast<size_t>(bh / group) * Nk * D;  // K, V
    const uint16_t* Kh = K + kv_head;
    const uint16_t* Vh = V + kv_head;
    const int q0 = qb * BM + wave * 32;  // first query row of this wave
    const int q = q0 + l32;              // query row owned by this lane

    frag qf[D / 16];
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (q < Nq) v = ld16(Q + head + static_cast<size_t>(q) * D + 16 * ks + 8 * g2);
        qf[ks] = as_frag<T>(v);
    }

    const int kv_end = causal ? min(Nk, (qb + 1) * BM + coff) : Nk;
    const int nkb = (kv_end + BN - 1) / BN;

    // Loads of one 64-row tile: 16 groups of 4 rows, two load instructions per group (columns
    // 0-127 and 128-255, 1 KB each, in the layout of fwd16_d128_kernel's groups). Part i of a
    // wave loads half i % 2 of group wave + NW (i / 2). Rows past Nk are clamped to row Nk - 1.
    const int ld_row = lane & 3;
    const int ld_col = (lane >> 2) * 8;
    const unsigned ld_voff = static_cast<unsigned>(((4 * wave + ld_row) * D + ld_col) * 2);
    auto load_part = [&](const uint16_t* src, int key0, unsigned char* dst, int i) {
        const int grp = wave + NW * (i >> 1);
        const int half = i & 1;
        if (key0 + BN <= Nk) {
            lds_dma16_async_s(src + static_cast<size_t>(key0 + 4 * NW * (i >> 1)) * D + 128 * half,
                              ld_voff, dst + grp * GRP + half * HALF);
        } else {
            const int row = min(key0 + 4 * grp + ld_row, Nk - 1);
            lds_dma16_async(src + static_cast<size_t>(row) * D + 128 * half + ld_col,
                            dst + grp * GRP + half * HALF);
        }
    };
    auto load_tile = [&](const uint16_t* src, int key0, unsigned char* dst) {
#pragma unroll
        for (int i = 0; i < kParts; ++i) load_part(src, key0, dst, i);
    };
    // Per-lane byte offsets of the operand reads (see the layout above).
    const int k_off = (l32 >> 2) * GRP + g2 * 64 + (l32 & 3) * 16;
    const int kq = lane & 15;
    const int v_off = g2 * GRP + (2 * ((lane >> 4) & 1) + ((kq & 3) >> 1)) * 64 + (kq >> 2) * 16 +
                      (kq & 1) * 8;

    // K row reads, k-step ks (16 columns): half ks / 8, chunk 2 (ks % 8) + lane / 32.
    auto k_addr = [&](const unsigned char* kt, int t, int ks) {
        return kt + k_off + 8 * t * GRP + (ks >> 3) * HALF + (ks & 7) * 128;
    };
    auto scores = [&](const unsigned char* kt, f32x16 (&s)[2]) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            s[t] = f32x16{};
#pragma unroll
            for (int ks = 0; ks < D / 16; ++ks)
                s[t] = Elem<T>::mma(as_frag<T>(ld16(k_addr(kt, t, ks))), qf[ks], s[t]);
        }
    };

    f32x16 o[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) o[dt] = f32x16{};
    float m = -INFINITY;  // running max of s * cs (log2 units)
    float l = 0.0f;       // this lane's share of the running row sum
    // Exponent scale, kept positive so that a masked score (-inf) always maps to p = 0, also
    // for scale = 0 (where FLT_MIN leaves every p at 1 and L at log(count), as with 0).
    const float cs = fmaxf(c, kFltMin);

    // Keys past Nk and, with a causal mask, keys after this lane's row get s = -inf.
    auto mask_scores = [&](f32x16 (&s)[2], int key0) {
        const int lim = min(Nk, causal ? q + 1 + coff : Nk) - key0 - 4 * g2;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int off = 32 * t + 8 * (r >> 2) + (r & 3);
                s[t][r] = off < lim ? s[t][r] : -INFINITY;
            }
        }
    };

    // Online-softmax update of (m, l) from mx, this lane's raw row max of the next block.
    // Returns whether some lane of the wave must rescale its O by alpha. The lazy rescale is
    // decided per lane with selects: m only moves when the block max exceeds it by more than
    // kLazyRescale, and O and l of that lane are scaled by the same alpha, so the result is
    // exact either way.
    auto update_max = [&](float mx, float& alpha) -> bool {
        const float m_new = fmaxf(m, pair_max(mx) * cs);
        const bool grow = m_new > m + kLazyRescale;
        const float a_raw = fast_exp2(m_new == -INFINITY ? 0.0f : m - m_new);
        alpha = grow ? a_raw : 1.0f;
        m = grow ? m_new : m;
        l *= alpha;
        return __ballot(grow) != 0;
    };

    // Operand fragment i of the score MFMAs (K rows of tile i / 16, k-step i % 16) and of
    // the P V MFMAs (V^T for key group i / 8 and d tile i % 8: half (i % 8) / 4).
    auto k_frag = [&](const unsigned char* kt, int i) {
        return as_frag<T>(ld16(k_addr(kt, i >> 4, i & 15)));
    };
    auto v_frag = [&](const unsigned char* vt, int i) {
        const int dt = i & 7;
        const unsigned char* a0 =
            vt + v_off + 4 * (i >> 3) * GRP + (dt >> 2) * HALF + (dt & 3) * 256;
        return tr_frag_at<T>(a0, a0 + 2 * GRP);
    };

    // Blocks that need masking: keys past Nk, and with a causal mask the blocks that reach past
    // the last key this wave's first row sees.
    auto needs_mask = [&](int key0) {
        return key0 + BN > Nk || (causal && key0 + BN - 1 > q0 + coff);
    };

    // Exponential of score r of tile t, and the rounding of tile t's group h of eight scores
    // to T (the P operand of key group 2 t + h).
    auto exp_one = [&](f32x16 (&s)[2], int t, int r, float m_use) {
        s[t][r] = fast_exp2(fmaf(s[t][r], cs, -m_use));
    };
    auto pack_p = [&](f32x16 (&s)[2], int t, int h) {
        u32x4 pw = __builtin_bit_cast(
            u32x4, pack_frag<T>(s[t][8 * h + 0], s[t][8 * h + 1], s[t][8 * h + 2],
                                s[t][8 * h + 3], s[t][8 * h + 4], s[t][8 * h + 5],
                                s[t][8 * h + 6], s[t][8 * h + 7]));
        // Keep the exponentials where they are placed: left alone, the compiler sinks them
        // to their first use past the branches in between.
        asm volatile("" : "+v"(pw));
        return __builtin_bit_cast(frag, pw);
    };

    // One block with an explicit instruction order (the scheduling fences keep it), as in
    // fwd16_d128_kernel with twice the MFMAs per phase:
    //   phase A: the 32 MFMAs of the next block's scores into s_next; every other one followed
    //            by the exponential of one score of the current tile 0 (P groups 0 and 1); the
    //            wave's 2 kParts tile-load parts after every other odd MFMA (K in the first half,
    //            V in the second);
    //   phase B: the 32 MFMAs of O^T += V^T P^T; MFMAs 0-15 carry the exponentials of tile 1
    //            (P groups 2 and 3, first used by MFMAs 16 and 24), every MFMA one term of the
    //            fp32 row sum and the max of one score of s_next.
    // Returns this lane's raw row max of s_next.
    auto step = [&](f32x16 (&s)[2], const unsigned char* kt, f32x16 (&s_next)[2],
                    const unsigned char* vt, int key0_next, bool kl_do, int kl_key0,
                    unsigned char* kl_dst, bool vl_do, int vl_key0,
                    unsigned char* vl_dst) -> float {
        constexpr int kAhead = 3;
        constexpr int kMma = 32;  // MFMAs per phase
        static_assert(kAhead <= kMma, "operands read ahead within the chain");
        const float m_use = (m == -INFINITY) ? 0.0f : m;
        frag p[4];
        frag fk[kMma];
        frag fv[kMma];
        s_next[0] = f32x16{};
        s_next[1] = f32x16{};
#pragma unroll
        for (int k = 0; k < kAhead; ++k) fk[k] = k_frag(kt, k);
#pragma unroll
        for (int i = 0; i < kMma; ++i) {
            if (i + kAhead < kMma) fk[i + kAhead] = k_frag(kt, i + kAhead);
            else fv[i + kAhead - kMma] = v_frag(vt, i + kAhead - kMma);
            s_next[i >> 4] = Elem<T>::mma(fk[i], qf[i & 15], s_next[i >> 4]);
            // Load slots: MFMAs 1, 3, 5, ...: K parts in the first half, V parts in the second.
            if (i & 1) {
                const int slot = (i & 15) >> 1;  // 0..7
                if (slot < kParts) {
                    if (i < 16 && kl_do) load_part(Kh, kl_key0, kl_dst, slot);
                    if (i >= 16 && vl_do) load_part(Vh, vl_key0, vl_dst, slot);
                }
            } else {
                exp_one(s, 0, i >> 1, m_use);
            }
            if ((i & 15) == 14) p[i >> 4] = pack_p(s, 0, i >> 4);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (needs_mask(key0_next)) mask_scores(s_next, key0_next);
        float mx = -INFINITY;
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < kMma; ++i) {
            if (i + kAhead < kMma) fv[i + kAhead] = v_frag(vt, i + kAhead);
            o[i & 7] = Elem<T>::mma(fv[i], p[i >> 3], o[i & 7]);
            if (i < 16) {
                exp_one(s, 1, i, m_use);
                if ((i & 7) == 7) p[2 + (i >> 3)] = pack_p(s, 1, i >> 3);
            }
            // Row sum of the fp32 exponentials (tile 0 in MFMAs 0-15, tile 1 in 16-31).
            sum += s[i >> 4][i & 15];
            mx = __builtin_elementwise_maximum(mx, s_next[i >> 4][i & 15]);
            // Keep both chains here: left alone, the compiler sinks them to their first use.
            asm volatile("" : "+v"(sum), "+v"(mx));
            __builtin_amdgcn_sched_barrier(0);
        }
        l += sum;
        return mx;
    };

    // Block j: K_j in Kb[j & 1], V_j in Vb[j & 1]. At the top of iteration j the loads issued
    // one iteration earlier (K_{j+1}, V_j) are waited for and a barrier makes them visible and
    // retires every read of K_j and V_{j-1}; then K_{j+2} and V_{j+1} are issued into those
    // buffers during the score MFMAs. Each iteration also forms the scores of block j+1 and their row max (for the
    // last block they come from a stale buffer and the max is replaced by -inf, which leaves
    // (m, l) unchanged). The loop is unrolled by two so that every buffer is a distinct LDS
    // object.
    load_tile(Kh, 0, Kb0);
    load_tile(Vh, 0, Vb0);
    if (nkb > 1) load_tile(Kh, BN, Kb1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    f32x16 sa[2], sb[2];
    float alpha;
    scores(Kb0, sa);
    if (needs_mask(0)) mask_scores(sa, 0);
    {
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = __builtin_elementwise_maximum(mx, sa[t][r]);
        }
        update_max(mx, alpha);  // O is still zero: nothing to rescale
    }
    // Key blocks this wave computes (see fwd16_d128_kernel): after the last one that is not
    // entirely past its rows' causal limit the wave runs load-only iterations.
    const int nkb_w = causal ? min(nkb, (q0 + 32 + coff + BN - 1) / BN) : nkb;
    int j = 0;
    for (; j < nkb_w; j += 2) {
        // ---- even block j: scores in sa, K_j in Kb0, V_j in Vb0 ----
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        float mx = step(sa, Kb1, sb, Vb0, (j + 1) * BN, j + 2 < nkb, (j + 2) * BN, Kb0,
                        j + 1 < nkb, (j + 1) * BN, Vb1);
        if (update_max(j + 1 < nkb_w ? mx : -INFINITY, alpha)) {
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) o[dt] *= alpha;
        }
        if (j + 1 >= nkb_w) {
            ++j;
            break;
        }
        // ---- odd block j + 1: scores in sb, K_{j+1} in Kb1, V_{j+1} in Vb1 ----
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        mx = step(sb, Kb0, sa, Vb1, (j + 2) * BN, j + 3 < nkb, (j + 3) * BN, Kb1,
                  j + 2 < nkb, (j + 2) * BN, Vb0);
        if (update_max(j + 2 < nkb_w ? mx : -INFINITY, alpha)) {
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) o[dt] *= alpha;
        }
    }
    for (j = nkb_w; j < nkb; ++j) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (j + 2 < nkb) load_tile(Kh, (j + 2) * BN, (j & 1) ? Kb1 : Kb0);
        if (j + 1 < nkb) load_tile(Vh, (j + 1) * BN, (j & 1) ? Vb0 : Vb1);
    }

    // Epilogue: O = O / l, L = m + log(l) (natural log), stored with RNE. O goes through the K/V
    // buffers (two waves' rows per buffer), free once every wave is past its last block.
    l = pair_sum(l);
    static_assert(NW == 4 && 2 * staged_rows_bytes<D>() <= TILE,
                  "two waves' O rows per K buffer");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    store_rows_staged<T, D>(o, 1.0f / l,
                            (wave < 2 ? Kb0 : Kb1) + (wave & 1) * staged_rows_bytes<D>(),
                            O + head, q0, Nq);
    if (g2 == 0 && q < Nq) L[static_cast<size_t>(bh) * Nq + q] = (m + fast_log2(l)) * kLn2;
}

// ------------------------------------------------------------------------------------------
// fp16 / bf16 kernel for head_dim 64: causal launches of at least as many 256-row blocks as CUs
// with fewer than 8192 keys
// ------------------------------------------------------------------------------------------
// fwd16_d128_kernel's data path and pipeline at head_dim 64: 64-key blocks in LDS-DMA double
// buffers, one workgroup of eight waves (256 query rows) per CU, the next block's scores formed
// while the current block's softmax runs. A 64-element row is 128 bytes, so one load
// instruction (64 lanes x 16 bytes) fills a group of 8 rows; the group layout is given at the
// operand offsets below (fwd16_d64_seq_kernel uses the same one; at head_dim 32 a row takes the
// first half of its 128-byte slot).
template <typename T, int NW, int D>
__global__ void __launch_bounds__(64 * NW, 8 / NW)
    fwd16_d64_kernel(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                      const uint16_t* __restrict__ V, uint16_t* __restrict__ O,
                      float* __restrict__ L, int Nq, int Nk, int coff, int group, int nqb,
                      float c, int causal) {
    static_assert(NW == 8 && D == 64, "eight waves at head_dim 64 (fwd16_d64_seq_kernel otherwise)");
    constexpr int KS = D / 16;   // k-steps of a score MFMA chain
    constexpr int NDT = D / 32;  // 32-column tiles of O
    constexpr int BM = 32 * NW;  // query rows per workgroup (NW waves of 32 rows)
    constexpr int BN = 64;
    constexpr int kParts = 8 / NW;  // load instructions per wave per 64-row tile
    constexpr int GRP = 1152;              // bytes per 8-row group
    constexpr int TILE = (BN / 8) * GRP;   // bytes per 64-row tile
    static_assert(kParts >= 1, "at most eight waves");
    using frag = typename Elem<T>::frag;
    __shared__ __attribute__((aligned(1024))) unsigned char Kb0[TILE];
    __shared__ __attribute__((aligned(1024))) unsigned char Kb1[TILE];
    __shared__ __attribute__((aligned(1024))) unsigned char Vb0[TILE];
    __shared__ __attribute__((aligned(1024))) unsigned char Vb1[TILE];

    int bh, rank;
    item_order(blockIdx.x, gridDim.x / nqb, nqb, causal == 0, bh, rank);
    const int qb = causal ? nqb - 1 - rank : rank;  // causal: longest query blocks first
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int l32 = lane & 31;
    const int g2 = lane >> 5;

    const size_t head = static_cast<size_t>(bh) * Nq * D;             // Q, O
    const size_t kv_head = static_cast<size_t>(bh / group) * Nk * D;  // K, V
    const uint16_t* Kh = K + kv_head;
    const uint16_t* Vh = V + kv_head;
    const int q0 = qb * BM + wave * 32;  // first query row of this wave
    const int q = q0 + l32;              // query row owned by this lane

    frag qf[D / 16];
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (q < Nq) v = ld16(Q + head + static_cast<size_t>(q) * D + 16 * ks + 8 * g2);
        qf[ks] = as_frag<T>(v);
    }

    const int kv_end = causal ? min(Nk, (qb + 1) * BM + coff) : Nk;
    const int nkb = (kv_end + BN - 1) / BN;

    // Loads of one 64-row tile: wave w fills groups w, w + NW, ... (kParts of them), one
    // 8-row group (1 KB) per load instruction: lane i writes slot i, i.e. chunk i / 8 of row
    // (i % 8) ^ (4 ((i >> 4) & 1)) of the group. Rows past Nk are clamped to row Nk - 1 (finite
    // values; their scores are masked). Issued from inline assembly as in fwd16_d128_kernel.
    // A tile that lies inside [0, Nk) is addressed as a scalar base plus a fixed per-lane offset.
    const int ld_row = (lane & 7) ^ (4 * ((lane >> 4) & 1));
    // At head_dim 32 a row fills chunks 0-3 of its 128-byte slot; lanes 32-63 load the same
    // chunks again into the unused slots 4-7.
    const int ld_col = ((lane >> 3) % (D / 8)) * 8;
    const unsigned ld_voff = static_cast<unsigned>(((8 * wave + ld_row) * D + ld_col) * 2);
    // Part i (0..kParts-1) of a tile load: this wave's group wave + NW i.
    auto load_part = [&](const uint16_t* src, int key0, unsigned char* dst, int i) {
        if (key0 + BN <= Nk) {
            lds_dma16_async_s(src + static_cast<size_t>(key0 + 8 * NW * i) * D, ld_voff,
                              dst + (wave + NW * i) * GRP);
        } else {
            const int grp = wave + NW * i;
            const int row = min(key0 + 8 * grp + ld_row, Nk - 1);
            lds_dma16_async(src + static_cast<size_t>(row) * D + ld_col, dst + grp * GRP);
        }
    };
    auto load_tile = [&](const uint16_t* src, int key0, unsigned char* dst) {
#pragma unroll
        for (int i = 0; i < kParts; ++i) load_part(src, key0, dst, i);
    };
    // Per-lane byte offsets of the operand reads. Chunk c of row r of a group sits at
    // 16 (8 c + (r ^ 4 ((c >> 1) & 1))): 16 rows of one chunk (K row reads) fall on 16 distinct
    // 16-byte bank slots (the 128 bytes of padding per group shift the next 8 rows by 8 slots),
    // and the 32 lanes of a V transpose read (4 rows x 8 chunk halves) on 32 distinct 8-byte
    // slots (the row swizzle moves the chunks 2-3 of a 64-byte span to the other rows).
    // K row reads: chunk 2 ks + g2, so the swizzle bit is ks & 1.
    const int k_off_even = (l32 >> 3) * GRP + g2 * 128 + (l32 & 7) * 16;
    const int k_off_odd = (l32 >> 3) * GRP + g2 * 128 + ((l32 & 7) ^ 4) * 16;
    const int kq = lane & 15;
    const int gl = (lane >> 4) & 1;
    const int v_off = (2 * gl + ((kq & 3) >> 1)) * 128 + (g2 ^ gl) * 64 + (kq >> 2) * 16 +
                      (kq & 1) * 8;
    auto k_addr = [&](const unsigned char* kt, int t, int ks) {
        return kt + ((ks & 1) ? k_off_odd : k_off_even) + 4 * t * GRP + ks * 256;
    };

    auto scores = [&](const unsigned char* kt, f32x16 (&s)[2]) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            s[t] = f32x16{};
#pragma unroll
            for (int ks = 0; ks < D / 16; ++ks)
                s[t] = Elem<T>::mma(as_frag<T>(ld16(k_addr(kt, t, ks))), qf[ks], s[t]);
        }
    };

    f32x16 o[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) o[dt] = f32x16{};
    float m = -INFINITY;  // running max of s * cs (log2 units)
    float l = 0.0f;       // this lane's share of the running row sum
    // Exponent scale, kept positive so that a masked score (-inf) always maps to p = 0, also
    // for scale = 0 (where FLT_MIN leaves every p at 1 and L at log(count), as with 0).
    const float cs = fmaxf(c, kFltMin);

    // Keys past Nk and, with a causal mask, keys after this lane's row get s = -inf.
    auto mask_scores = [&](f32x16 (&s)[2], int key0) {
        const int lim = min(Nk, causal ? q + 1 + coff : Nk) - key0 - 4 * g2;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int off = 32 * t + 8 * (r >> 2) + (r & 3);
                s[t][r] = off < lim ? s[t][r] : -INFINITY;
            }
        }
    };

    // Online-softmax update of (m, l) from mx, this lane's raw row max of the next block.
    // Returns whether some lane of the wave must rescale its O by alpha. The lazy rescale is
    // decided per lane with selects: m only moves when the block max exceeds it by more than
    // kLazyRescale, and O and l of that lane are scaled by the same alpha, so the result is
    // exact either way.
    auto update_max = [&](float mx, float& alpha) -> bool {
        const float m_new = fmaxf(m, pair_max(mx) * cs);
        const bool grow = m_new > m + kLazyRescale;
        const float a_raw = fast_exp2(m_new == -INFINITY ? 0.0f : m - m_new);
        alpha = grow ? a_raw : 1.0f;
        m = grow ? m_new : m;
        l *= alpha;
        return __ballot(grow) != 0;
    };

    // Operand fragment i of the score MFMAs (K rows of tile half i / 4, k-step i % 4) and of
    // the P V MFMAs (V^T for key group i / 2 and d tile i % 2).
    auto k_frag = [&](const unsigned char* kt, int i) {
        return as_frag<T>(ld16(k_addr(kt, i / KS, i % KS)));
    };
    auto v_frag = [&](const unsigned char* vt, int i) {
        const unsigned char* a0 = vt + v_off + 2 * (i / NDT) * GRP + (i % NDT) * 512;
        return tr_frag_at<T>(a0, a0 + GRP);
    };

    // Blocks that need masking: keys past Nk, and with a causal mask the blocks that reach past
    // the last key this wave's first row sees.
    auto needs_mask = [&](int key0) {
        return key0 + BN > Nk || (causal && key0 + BN - 1 > q0 + coff);
    };

    // Exponential of score r of tile t, and the rounding of tile t's group h of eight scores
    // to T (the P operand of key group 2 t + h).
    auto exp_one = [&](f32x16 (&s)[2], int t, int r, float m_use) {
        s[t][r] = fast_exp2(fmaf(s[t][r], cs, -m_use));
    };
    auto pack_p = [&](f32x16 (&s)[2], int t, int h) {
        u32x4 pw = __builtin_bit_cast(
            u32x4, pack_frag<T>(s[t][8 * h + 0], s[t][8 * h + 1], s[t][8 * h + 2],
                                s[t][8 * h + 3], s[t][8 * h + 4], s[t][8 * h + 5],
                                s[t][8 * h + 6], s[t][8 * h + 7]));
        // Keep the exponentials where they are placed: left alone, the compiler sinks them
        // to their first use past the branches in between.
        asm volatile("" : "+v"(pw));
        return __builtin_bit_cast(frag, pw);
    };

    // One block with an explicit instruction order (the scheduling fences keep it), as in
    // fwd16_d128_kernel with half the MFMAs per phase (the softmax work per key is the same, so
    // every MFMA carries twice the VALU work):
    //   phase A: the 8 MFMAs of the next block's scores into s_next; after the first
    //            kDelay = 2 the online-softmax update with the current block's max (as in
    //            fwd16_d128_kernel), then the exponentials of the current tile 0 spread over the
    //            remaining 6 (P groups 0 and 1); the wave's K load part after MFMA 1, its V load
    //            part after MFMA 5;
    //   phase B: the 8 MFMAs of O^T += V^T P^T; MFMAs 0-3 carry the exponentials of tile 1
    //            (P groups 2 and 3, first used by MFMAs 4 and 6), every MFMA four terms of the
    //            fp32 row sum and the max of four scores of s_next.
    // Returns this lane's raw row max of s_next.
    auto step = [&](f32x16 (&s)[2], const unsigned char* kt, f32x16 (&s_next)[2],
                    const unsigned char* vt, int key0_next, bool kl_do, int kl_key0,
                    unsigned char* kl_dst, bool vl_do, int vl_key0,
                    unsigned char* vl_dst, float mx_cur) -> float {
        constexpr int kAhead = 3;
        constexpr int kMma = 4 * NDT;  // MFMAs per phase
        static_assert(kAhead <= kMma, "operands read ahead within the chain");
        // Phase-A MFMAs before the max update, and those that carry the tile-0 exponentials.
        constexpr int kDelay = kMma / 4;
        constexpr int kN = kMma - kDelay;
        constexpr int kExpB = 16 / (kMma / 2);  // tile-1 exponentials per early phase-B MFMA
        constexpr int kQuads = 8 / kMma;        // 4-term row sum / max groups per phase-B MFMA
        float m_use = 0.0f;
        frag p[4];
        frag fk[kMma];
        frag fv[kMma];
        s_next[0] = f32x16{};
        s_next[1] = f32x16{};
#pragma unroll
        for (int k = 0; k < kAhead; ++k) fk[k] = k_frag(kt, k);
#pragma unroll
        for (int i = 0; i < kMma; ++i) {
            if (i + kAhead < kMma) fk[i + kAhead] = k_frag(kt, i + kAhead);
            else fv[i + kAhead - kMma] = v_frag(vt, i + kAhead - kMma);
            s_next[i / KS] = Elem<T>::mma(fk[i], qf[i % KS], s_next[i / KS]);
            if (i == 1 && kl_do) {
#pragma unroll
                for (int part = 0; part < kParts; ++part) load_part(Kh, kl_key0, kl_dst, part);
            }
            if (i == kMma / 2 + 1 && vl_do) {
#pragma unroll
                for (int part = 0; part < kParts; ++part) load_part(Vh, vl_key0, vl_dst, part);
            }
            if (i == kDelay - 1) {
                // Online-softmax update with this block's max (see fwd16_d128_kernel).
                float alpha;
                if (update_max(mx_cur, alpha)) {
#pragma unroll
                    for (int dt = 0; dt < D / 32; ++dt) o[dt] *= alpha;
                }
                m_use = (m == -INFINITY) ? 0.0f : m;
            }
            if (i >= kDelay) {
#pragma unroll
                for (int e = 16 * (i - kDelay) / kN; e < 16 * (i - kDelay + 1) / kN; ++e) {
                    exp_one(s, 0, e, m_use);
                    if ((e & 7) == 7) p[e >> 3] = pack_p(s, 0, e >> 3);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (needs_mask(key0_next)) mask_scores(s_next, key0_next);
        float mx = -INFINITY;
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < kMma; ++i) {
            if (i + kAhead < kMma) fv[i + kAhead] = v_frag(vt, i + kAhead);
            o[i % NDT] = Elem<T>::mma(fv[i], p[i / NDT], o[i % NDT]);
            if (i < kMma / 2) {
#pragma unroll
                for (int e = 0; e < kExpB; ++e) exp_one(s, 1, kExpB * i + e, m_use);
                if ((i + 1) * kExpB % 8 == 0)
                    p[2 + (i + 1) * kExpB / 8 - 1] = pack_p(s, 1, (i + 1) * kExpB / 8 - 1);
            }
            // Row sum of the fp32 exponentials and row max of s_next, four terms per group
            // (tile 0 in the first half of the MFMAs, tile 1 in the second).
#pragma unroll
            for (int g = 0; g < kQuads; ++g) {
                const int t = (kQuads * i + g) >> 2;
                const int r = 4 * ((kQuads * i + g) & 3);
                sum += (s[t][r] + s[t][r + 1]) + (s[t][r + 2] + s[t][r + 3]);
                mx = __builtin_elementwise_maximum(
                    __builtin_elementwise_maximum(mx, s_next[t][r]),
                    __builtin_elementwise_maximum(
                        s_next[t][r + 1],
                        __builtin_elementwise_maximum(s_next[t][r + 2], s_next[t][r + 3])));
            }
            // Keep both chains here: left alone, the compiler sinks them to their first use.
            asm volatile("" : "+v"(sum), "+v"(mx));
            __builtin_amdgcn_sched_barrier(0);
        }
        l += sum;
        return mx;
    };

    // Block j: K_j in Kb[j & 1], V_j in Vb[j & 1]. At the top of iteration j the loads issued
    // one iteration earlier (K_{j+1}, V_j) are waited for and a barrier makes them visible and
    // retires every read of K_j and V_{j-1}; then K_{j+2} and V_{j+1} are issued into those
    // buffers during the score MFMAs. Each iteration also forms the scores of block j+1 and
    // their row max, which the next iteration applies (for the last block they come from a
    // stale buffer and the max is never used). The loop is unrolled by two so that every buffer
    // is a distinct LDS object.
    load_tile(Kh, 0, Kb0);
    load_tile(Vh, 0, Vb0);
    if (nkb > 1) load_tile(Kh, BN, Kb1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    f32x16 sa[2], sb[2];
    scores(Kb0, sa);
    if (needs_mask(0)) mask_scores(sa, 0);
    // Key blocks this wave computes (see fwd16_d128_kernel): after the last one that is not
    // entirely past its rows' causal limit the wave runs load-only iterations.
    const int nkb_w = causal ? min(nkb, (q0 + 32 + coff + BN - 1) / BN) : nkb;
    int j = 0;
    {
        // Raw row max of the block whose scores are in the current set (step() applies it).
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = __builtin_elementwise_maximum(mx, sa[t][r]);
        }
        for (; j < nkb_w; j += 2) {
            // ---- even block j: scores in sa, K_j in Kb0, V_j in Vb0 ----
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            mx = step(sa, Kb1, sb, Vb0, (j + 1) * BN, j + 2 < nkb, (j + 2) * BN, Kb0,
                      j + 1 < nkb, (j + 1) * BN, Vb1, mx);
            if (j + 1 >= nkb_w) {
                ++j;
                break;
            }
            // ---- odd block j + 1: scores in sb, K_{j+1} in Kb1, V_{j+1} in Vb1 ----
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            mx = step(sb, Kb0, sa, Vb1, (j + 2) * BN, j + 3 < nkb, (j + 3) * BN, Kb1,
                      j + 2 < nkb, (j + 2) * BN, Vb0, mx);
        }
    }
    for (j = nkb_w; j < nkb; ++j) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (j + 2 < nkb) load_tile(Kh, (j + 2) * BN, (j & 1) ? Kb1 : Kb0);
        if (j + 1 < nkb) load_tile(Vh, (j + 1) * BN, (j & 1) ? Vb0 : Vb1);
    }

    // Epilogue: O = O / l, L = m + log(l) (natural log), stored with RNE. O goes through the K/V
    // buffers (two waves' rows per buffer), free once every wave is past its last block.
    l = pair_sum(l);
    static_assert(2 * staged_rows_bytes<D>() <= TILE, "two waves' O rows per K/V buffer");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    store_rows_staged<T, D>(o, 1.0f / l,
                            (wave < 2 ? Kb0 : wave < 4 ? Kb1 : wave < 6 ? Vb0 : Vb1) +
                                (wave & 1) * staged_rows_bytes<D>(),
                            O + head, q0, Nq);
    if (g2 == 0 && q < Nq) L[static_cast<size_t>(bh) * Nq + q] = (m + fast_log2(l)) * kLn2;
}

// ------------------------------------------------------------------------------------------
// fp16 / bf16 kernel for head_dim 64 and 32, four waves per SIMD
// ------------------------------------------------------------------------------------------
// fwd16_d64_kernel's tiles, operand layouts and arithmetic without its cross-block pipeline:
// each wave forms a block's scores, applies the block's max, forms the exponentials and runs the
// P V MFMAs in sequence, with one score set. That fits 128 registers, so 16 waves share a CU
// (four workgroups of four waves, or two of eight, each with 36 KB of tiles) and the SIMD
// interleaves four waves' phases instead of relying on one wave's instruction order. Eight-wave
// workgroups (256 rows) halve the tile loads per MFMA. Used for head_dim 64 launches except
// causal ones with fewer than 8192 keys (there the pipelined kernel's per-wave causal stop saves
// more) and for every launch at head_dim 32. Same products, sums and rounding in the same order
// as fwd16_d64_kernel, so the results are bitwise equal.
template <typename T, int D, int NW>
__global__ void __launch_bounds__(64 * NW, 16 / NW)
    fwd16_d64_seq_kernel(const uint16_t* __restrict__ Q, const uint16_t* __restrict__ K,
                         const uint16_t* __restrict__ V, uint16_t* __restrict__ O,
                         float* __restrict__ L, int Nq, int Nk, int coff, int group, int nqb,
                         float c, int causal) {
    static_assert(D == 64 || D == 32, "rows of at most 128 bytes");
    static_assert(NW == 4 || NW == 8, "four or eight waves");
    constexpr int KS = D / 16;   // k-steps of a score MFMA chain
    constexpr int NDT = D / 32;  // 32-column tiles of O
    constexpr int BM = 32 * NW;  // query rows per workgroup
    constexpr int BN = 64;
    constexpr int kParts = 8 / NW;         // load instructions per wave per 64-row tile
    constexpr int GRP = 1152;              // bytes per 8-row group (fwd16_d64_kernel's layout)
    constexpr int TILE = (BN / 8) * GRP;   // bytes per 64-row tile
    using frag = typename Elem<T>::frag;
    __shared__ __attribute__((aligned(1024))) unsigned char Kb0[TILE];
    __shared__ __attribute__((aligned(1024))) unsigned char Kb1[TILE];
    __shared__ __attribute__((aligned(1024))) unsigned char Vb0[TILE];
    __shared__ __attribute__((aligned(1024))) unsigned char Vb1[TILE];

    int bh, rank;
    item_order(blockIdx.x, gridDim.x / nqb, nqb, causal == 0, bh, rank);
    const int qb = causal ? nqb - 1 - rank : rank;  // causal: longest query blocks first
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
    const int l32 = lane & 31;
    const int g2 = lane >> 5;

    const size_t head = static_cast<size_t>(bh) * Nq * D;             // Q, O
    const size_t kv_head = static_cast<size_t>(bh / group) * Nk * D;  // K, V
    const uint16_t* Kh = K + kv_head;
    const uint16_t* Vh = V + kv_head;
    const int q0 = qb * BM + wave * 32;  // first query row of this wave
    const int q = q0 + l32;              // query row owned by this lane

    frag qf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (q < Nq) v = ld16(Q + head + static_cast<size_t>(q) * D + 16 * ks + 8 * g2);
        qf[ks] = as_frag<T>(v);
    }
    const int kv_end = causal ? min(Nk, (qb + 1) * BM + coff) : Nk;
    const int nkb = (kv_end + BN - 1) / BN;

    // Tile loads, operand offsets and masking exactly as in fwd16_d64_kernel.
    const int ld_row = (lane & 7) ^ (4 * ((lane >> 4) & 1));
    const int ld_col = ((lane >> 3) % (D / 8)) * 8;
    const unsigned ld_voff = static_cast<unsigned>(((8 * wave + ld_row) * D + ld_col) * 2);
    auto load_tile = [&](const uint16_t* src, int key0, unsigned char* dst) {
#pragma unroll
        for (int i = 0; i < kParts; ++i) {
            if (key0 + BN <= Nk) {
                lds_dma16_async_s(src + static_cast<size_t>(key0 + 8 * NW * i) * D, ld_voff,
                                  dst + (wave + NW * i) * GRP);
            } else {
                const int grp = wave + NW * i;
                const int row = min(key0 + 8 * grp + ld_row, Nk - 1);
                lds_dma16_async(src + static_cast<size_t>(row) * D + ld_col, dst + grp * GRP);
            }
        }
    };
    const int k_off_even = (l32 >> 3) * GRP + g2 * 128 + (l32 & 7) * 16;
    const int k_off_odd = (l32 >> 3) * GRP + g2 * 128 + ((l32 & 7) ^ 4) * 16;
    const int kq = lane & 15;
    const int gl = (lane >> 4) & 1;
    const int v_off = (2 * gl + ((kq & 3) >> 1)) * 128 + (g2 ^ gl) * 64 + (kq >> 2) * 16 +
                      (kq & 1) * 8;
    auto k_frag = [&](const unsigned char* kt, int i) {  // K rows of tile i / KS, k-step i % KS
        const int t = i / KS, ks = i % KS;
        return as_frag<T>(ld16(kt + ((ks & 1) ? k_off_odd : k_off_even) + 4 * t * GRP + ks * 256));
    };
    auto v_frag = [&](const unsigned char* vt, int i) {  // V^T, key group i / NDT, d tile i % NDT
        const unsigned char* a0 = vt + v_off + 2 * (i / NDT) * GRP + (i % NDT) * 512;
        return tr_frag_at<T>(a0, a0 + GRP);
    };

    f32x16 o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x16{};
    float m = -INFINITY;  // running max of s * cs (log2 units)
    float l = 0.0f;       // this lane's share of the running row sum
    const float cs = fmaxf(c, kFltMin);

    // One block: scores, the block's max, exponentials and row sum, then O^T += V^T P^T.
    auto block = [&](const unsigned char* kt, const unsigned char* vt, int key0) {
        constexpr int kAhead = 3;
        constexpr int kMma = 4 * NDT;  // MFMAs per chain (score tiles x k-steps = key groups x d tiles)
        static_assert(2 * KS == kMma && kAhead <= kMma, "chain lengths");
        f32x16 s[2] = {f32x16{}, f32x16{}};
        {
            frag fk[kMma];
#pragma unroll
            for (int k = 0; k < kAhead; ++k) fk[k] = k_frag(kt, k);
#pragma unroll
            for (int i = 0; i < kMma; ++i) {
                if (i + kAhead < kMma) fk[i + kAhead] = k_frag(kt, i + kAhead);
                s[i / KS] = Elem<T>::mma(fk[i], qf[i % KS], s[i / KS]);
            }
        }
        if (key0 + BN > Nk || (causal && key0 + BN - 1 > q0 + coff)) {
            const int lim = min(Nk, causal ? q + 1 + coff : Nk) - key0 - 4 * g2;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int off = 32 * t + 8 * (r >> 2) + (r & 3);
                    s[t][r] = off < lim ? s[t][r] : -INFINITY;
                }
            }
        }
        // Online-softmax update (lazy rescale, as in fwd16_d64_kernel).
        {
            float mx = -INFINITY;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = __builtin_elementwise_maximum(mx, s[t][r]);
            }
            const float m_new = fmaxf(m, pair_max(mx) * cs);
            const bool grow = m_new > m + kLazyRescale;
            const float a_raw = fast_exp2(m_new == -INFINITY ? 0.0f : m - m_new);
            const float alpha = grow ? a_raw : 1.0f;
            m = grow ? m_new : m;
            l *= alpha;
            if (__ballot(grow) != 0) {
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) o[dt] *= alpha;
            }
        }
        const float m_use = (m == -INFINITY) ? 0.0f : m;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s[t][r] = fast_exp2(fmaf(s[t][r], cs, -m_use));
        }
        frag p[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int t = g >> 1, h = g & 1;
            p[g] = pack_frag<T>(s[t][8 * h + 0], s[t][8 * h + 1], s[t][8 * h + 2], s[t][8 * h + 3],
                                s[t][8 * h + 4], s[t][8 * h + 5], s[t][8 * h + 6], s[t][8 * h + 7]);
        }
        // Row sum of the fp32 exponentials, four terms per group, in fwd16_d64_kernel's order.
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int t = i >> 2;
            const int r = 4 * (i & 3);
            sum += (s[t][r] + s[t][r + 1]) + (s[t][r + 2] + s[t][r + 3]);
        }
        l += sum;
        {
            frag fv[kMma];
#pragma unroll
            for (int k = 0; k < kAhead; ++k) fv[k] = v_frag(vt, k);
#pragma unroll
            for (int i = 0; i < kMma; ++i) {
                if (i + kAhead < kMma) fv[i + kAhead] = v_frag(vt, i + kAhead);
                o[i % NDT] = Elem<T>::mma(fv[i], p[i / NDT], o[i % NDT]);
            }
        }
    };

    // Block j in Kb[j & 1], Vb[j & 1]; the loads of block j + 1 are issued right after the
    // barrier that retires every read of block j - 1. Unrolled by two so that every buffer is a
    // distinct LDS object.
    load_tile(Kh, 0, Kb0);
    load_tile(Vh, 0, Vb0);
    for (int j = 0; j < nkb; j += 2) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (j + 1 < nkb) {
            load_tile(Kh, (j + 1) * BN, Kb1);
            load_tile(Vh, (j + 1) * BN, Vb1);
        }
        block(Kb0, Vb0, j * BN);
        if (j + 1 >= nkb) break;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (j + 2 < nkb) {
            load_tile(Kh, (j + 2) * BN, Kb0);
            load_tile(Vh, (j + 2) * BN, Vb0);
        }
        block(Kb1, Vb1, (j + 1) * BN);
    }

    // Epilogue as in fwd16_d64_kernel: O = O / l, L = m + log(l), O rows staged through LDS.
    l = pair_sum(l);
    static_assert(2 * staged_rows_bytes<D>() <= TILE, "two waves' O rows per K buffer");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    store_rows_staged<T, D>(o, 1.0f / l,
                            (wave < 2 ? Kb0 : wave < 4 ? Kb1 : wave < 6 ? Vb0 : Vb1) +
                                (wave & 1) * staged_rows_bytes<D>(),
                            O + head, q0, Nq);
    if (g2 == 0 && q < Nq) L[static_cast<size_t>(bh) * Nq + q] = (m + fast_log2(l)) * kLn2;
}

// ------------------------------------------------------------------------------------------
// fp32 kernel
// ------------------------------------------------------------------------------------------
// Two workgroups per CU, except at head_dim 256 (O, Q^T and the scores need more than the
// 256 registers per lane that two workgroups of four waves leave).
template <int D>
constexpr int fwd_min_waves() {
    return D >= 256 ? 1 : 2;
}

template <int D>
struct Fwd32Cfg {
    static constexpr int kThreads = 256;
    static constexpr int BM = 128;
    static constexpr int BN = 32;
    static constexpr int KP = D + 4;  // rows 16 bytes apart modulo 256 bytes
    static constexpr int VP = D + 8;  // the two rows read by one instruction sit 128 bytes apart
    static constexpr int kChunksPerRow = D / 4;
    static constexpr int kChunksPerThread = BN * kChunksPerRow / kThreads;
    static_assert(BN * kChunksPerRow % kThreads == 0, "tile copy must divide evenly");
};

template <int D>
__global__ void __launch_bounds__(256, (fwd_min_waves<D>()))
    fwd32_kernel(const float* __restrict__ Q, const float* __restrict__ K,
                 const float* __restrict__ V, float* __restrict__ O, float* __restrict__ L,
                 int Nq, int Nk, int coff, int group, int nqb, float c, int causal) {
    using Cfg = Fwd32Cfg<D>;
    __shared__ __attribute__((aligned(16))) float Ks[Cfg::BN * Cfg::KP];
    __shared__ __attribute__((aligned(16))) float Vs[Cfg::BN * Cfg::VP];

    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = lid / nqb;
    const int qb = causal ? nqb - 1 - lid % nqb : lid % nqb;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
    const int l32 = lane & 31;
    const int g2 = lane >> 5;

    const size_t head = static_cast<size_t>(bh) * Nq * D;             // Q, O
    const size_t kv_head = static_cast<size_t>(bh / group) * Nk * D;  // K, V
    const float* Qh = Q + head;
    const float* Kh = K + kv_head;
    const float* Vh = V + kv_head;
    const int q0 = qb * Cfg::BM + wave * 32;
    const int q = q0 + l32;

    // Q^T operand: the k index of MFMA step ks in lane half g2 is d = (D/2)*g2 + ks.
    float qf[D / 2];
#pragma unroll
    for (int i = 0; i < D / 8; ++i) {
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (q < Nq) v = __builtin_bit_cast(f32x4, ld16(Qh + static_cast<size_t>(q) * D + (D / 2) * g2 + 4 * i));
#pragma unroll
        for (int u = 0; u < 4; ++u) qf[4 * i + u] = v[u];
    }

    f32x16 o[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) o[dt] = f32x16{};
    float m = -INFINITY;
    float l = 0.0f;

    const int kv_end = causal ? min(Nk, (qb + 1) * Cfg::BM + coff) : Nk;
    const int nkb = (kv_end + Cfg::BN - 1) / Cfg::BN;

    u32x4 kreg[Cfg::kChunksPerThread];
    u32x4 vreg[Cfg::kChunksPerThread];
    auto fetch = [&](int kb) {
#pragma unroll
        for (int i = 0; i < Cfg::kChunksPerThread; ++i) {
            const int id = i * Cfg::kThreads + tid;
            const int row = id / Cfg::kChunksPerRow;
            const int col = (id % Cfg::kChunksPerRow) * 4;
            const int key = kb * Cfg::BN + row;
            if (key < Nk) {
                const size_t off = static_cast<size_t>(key) * D + col;
                kreg[i] = ld16(Kh + off);
                vreg[i] = ld16(Vh + off);
            } else {
                kreg[i] = u32x4{0u, 0u, 0u, 0u};
                vreg[i] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < Cfg::kChunksPerThread; ++i) {
            const int id = i * Cfg::kThreads + tid;
            const int row = id / Cfg::kChunksPerRow;
            const int col = (id % Cfg::kChunksPerRow) * 4;
            st16(&Ks[row * Cfg::KP + col], kreg[i]);
            st16(&Vs[row * Cfg::VP + col], vreg[i]);
        }
    };

    if (nkb > 0) fetch(0);
    for (int kb = 0; kb < nkb; ++kb) {
        __syncthreads();
        stage();
        __syncthreads();
        if (kb + 1 < nkb) fetch(kb + 1);

        const int key0 = kb * Cfg::BN;

        f32x16 s[1];
        s[0] = f32x16{};
#pragma unroll
        for (int i = 0; i < D / 8; ++i) {
            const f32x4 a4 = __builtin_bit_cast(
                f32x4, ld16(&Ks[l32 * Cfg::KP + (D / 2) * g2 + 4 * i]));
#pragma unroll
            for (int u = 0; u < 4; ++u) s[0] = mma_f32(a4[u], qf[4 * i + u], s[0]);
        }

        const bool masked = (key0 + Cfg::BN > Nk) || (causal && key0 + Cfg::BN - 1 > q0 + coff);
        float alpha;
        const bool rescale =
            masked ? softmax_step<1, true>(s, key0, q + coff, Nk, causal != 0, c, m, l, alpha)
                   : softmax_step<1, false>(s, key0, q + coff, Nk, causal != 0, c, m, l, alpha);
        if (rescale) {
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) o[dt] *= alpha;
        }

        // O^T += V^T P^T: step r contracts the two keys 8*(r/4) + 4*h + r%4 (h = lane half).
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = 8 * (r >> 2) + 4 * g2 + (r & 3);
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
                const float a = Vs[key * Cfg::VP + 32 * dt + l32];
                o[dt] = mma_f32(a, s[0][r], o[dt]);
            }
        }
    }

    l += xor_shuffle(l, 32);
    if (q < Nq) {
        const float inv = 1.0f / l;
        float* Orow = O + head + static_cast<size_t>(q) * D;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                f32x4 w;
                w[0] = o[dt][4 * a + 0] * inv;
                w[1] = o[dt][4 * a + 1] * inv;
                w[2] = o[dt][4 * a + 2] * inv;
                w[3] = o[dt][4 * a + 3] * inv;
                st16(Orow + 32 * dt + 8 * a + 4 * g2, __builtin_bit_cast(u32x4, w));
            }
        }
        if (g2 == 0) L[static_cast<size_t>(bh) * Nq + q] = (m + fast_log2(l)) * kLn2;
    }
}

// ------------------------------------------------------------------------------------------
// fp32 kernel for launches with few query blocks
// ------------------------------------------------------------------------------------------
// fwd32_kernel gives each wave 32 query rows and walks every key block of them in one wave, so a
// small launch is as long as its longest query block (config 1, causal B=2 H=8 N=1024: 128
// workgroups for 256 CUs, the last block of each head 32 key blocks long). Here a workgroup
// owns one 32-row query block and its four waves split the key blocks (wave w takes blocks
// w, w + 4, ...; with a causal mask their counts differ by at most one). Each wave stages its
// own K/V tiles through its LDS area (registers -> LDS, the next block's rows loaded during the
// current block), runs the online softmax of fwd32_kernel over its blocks and ends with a
// partial state (m_w, l_w, O_w). The partial states go through LDS and wave 0 merges them with
// the rule of the split-KV combine (online_softmax.cuh:28-33): M = max m_w,
// l = sum l_w 2^(m_w - M), O = sum O_w 2^(m_w - M) / l, L = (M + log2 l) ln 2.
template <int D>
__global__ void __launch_bounds__(256, 2)
    fwd32_split_kernel(const float* __restrict__ Q, const float* __restrict__ K,
                       const float* __restrict__ V, float* __restrict__ O, float* __restrict__ L,
                       int Nq, int Nk, int coff, int group, int nqb, int round_len, float c,
                       int causal) {
    static_assert(D == 32 || D == 64, "head_dim 32 and 64");
    constexpr int BN = 32;
    constexpr int KP = D + 4;  // rows 16 bytes apart modulo 256 bytes
    constexpr int VP = D + 8;  // the two rows read by one instruction sit 128 bytes apart
    constexpr int kChunks = BN * D / 4 / 64;    // 16-byte chunks per lane per tile
    constexpr int kWaveLds = BN * (KP + VP);    // floats per wave
    constexpr int kMerge = 32 * D + 64;         // floats per wave: O, then m and l of 32 rows
    static_assert(kMerge <= kWaveLds, "merge area inside the wave's tile area");
    __shared__ __attribute__((aligned(16))) float lds[4 * kWaveLds];

    // Blocks of one head share an XCD (xcd_remap) and causal blocks run longest first. The
    // whole grid is resident at once (at most two workgroups per CU), and the dispatcher fills
    // an XCD's CUs (round_len of them) in order, round after round, so every other round is
    // dealt in reverse: a CU then pairs a long query block with a short one.
    int lid = xcd_remap(blockIdx.x, gridDim.x);
    if (round_len > 0 && gridDim.x % kNumXcd == 0) {
        const int per_xcd = gridDim.x / kNumXcd;
        const int base = lid - lid % per_xcd;
        const int i = lid % per_xcd;
        const int r = i / round_len;
        const int pos = i % round_len;
        const int len = min(round_len, per_xcd - r * round_len);
        lid = base + r * round_len + ((r & 1) ? len - 1 - pos : pos);
    }
    const int bh = lid / nqb;
    const int qb = causal ? nqb - 1 - lid % nqb : lid % nqb;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
    const int l32 = lane & 31;
    const int g2 = lane >> 5;

    const size_t head = static_cast<size_t>(bh) * Nq * D;             // Q, O
    const size_t kv_head = static_cast<size_t>(bh / group) * Nk * D;  // K, V
    const float* Kh = K + kv_head;
    const float* Vh = V + kv_head;
    const int q0 = qb * 32;
    const int q = q0 + l32;
    float* Ks = lds + wave * kWaveLds;
    float* Vs = Ks + BN * KP;

    // Q^T operand: the k index of MFMA step ks in lane half g2 is d = (D/2)*g2 + ks.
    float qf[D / 2];
#pragma unroll
    for (int i = 0; i < D / 8; ++i) {
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (q < Nq)
            v = __builtin_bit_cast(f32x4, ld16(Q + head + static_cast<size_t>(q) * D +
                                               (D / 2) * g2 + 4 * i));
#pragma unroll
        for (int u = 0; u < 4; ++u) qf[4 * i + u] = v[u];
    }

    f32x16 o[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) o[dt] = f32x16{};
    float m = -INFINITY;
    float l = 0.0f;

    const int kv_end = causal ? min(Nk, q0 + 32 + coff) : Nk;
    const int nkb = (kv_end + BN - 1) / BN;

    u32x4 kreg[kChunks];
    u32x4 vreg[kChunks];
    auto fetch = [&](int kb) {
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int id = i * 64 + lane;
            const int row = id / (D / 4);
            const int col = (id % (D / 4)) * 4;
            const int key = kb * BN + row;
            if (key < Nk) {
                const size_t off = static_cast<size_t>(key) * D + col;
                kreg[i] = ld16(Kh + off);
                vreg[i] = ld16(Vh + off);
            } else {
                kreg[i] = u32x4{0u, 0u, 0u, 0u};
                vreg[i] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    // The wave's earlier reads of its tiles precede these writes: a wave's LDS accesses are
    // performed in order.
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int id = i * 64 + lane;
            const int row = id / (D / 4);
            const int col = (id % (D / 4)) * 4;
            st16(&Ks[row * KP + col], kreg[i]);
            st16(&Vs[row * VP + col], vreg[i]);
        }
    };

    if (wave < nkb) fetch(wave);
    for (int kb = wave; kb < nkb; kb += 4) {
        stage();
        if (kb + 4 < nkb) fetch(kb + 4);
        const int key0 = kb * BN;

        f32x16 s[1];
        s[0] = f32x16{};
#pragma unroll
        for (int i = 0; i < D / 8; ++i) {
            const f32x4 a4 = __builtin_bit_cast(f32x4, ld16(&Ks[l32 * KP + (D / 2) * g2 + 4 * i]));
#pragma unroll
            for (int u = 0; u < 4; ++u) s[0] = mma_f32(a4[u], qf[4 * i + u], s[0]);
        }

        const bool masked = (key0 + BN > Nk) || (causal && key0 + BN - 1 > q0 + coff);
        float alpha;
        const bool rescale =
            masked ? softmax_step<1, true>(s, key0, q + coff, Nk, causal != 0, c, m, l, alpha)
                   : softmax_step<1, false>(s, key0, q + coff, Nk, causal != 0, c, m, l, alpha);
        if (rescale) {
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) o[dt] *= alpha;
        }

        // O^T += V^T P^T: step r contracts the two keys 8*(r/4) + 4*h + r%4 (h = lane half).
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = 8 * (r >> 2) + 4 * g2 + (r & 3);
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
                const float a = Vs[key * VP + 32 * dt + l32];
                o[dt] = mma_f32(a, s[0][r], o[dt]);
            }
        }
    }

    // Merge of the four partial states. Each wave writes O_w in its accumulator layout
    // ([dt][r][lane]) and (m_w, l_w) of its 32 rows to the start of its own area.
    l += xor_shuffle(l, 32);
    __syncthreads();  // every wave is past its last tile reads
    float* mo = lds + wave * kWaveLds;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mo[(16 * dt + r) * 64 + lane] = o[dt][r];
    }
    if (g2 == 0) {
        mo[32 * D + l32] = m;
        mo[32 * D + 32 + l32] = l;
    }
    __syncthreads();
    if (wave != 0) return;
    float mw[4], a[4];
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        mw[w] = lds[w * kWaveLds + 32 * D + l32];
        M = fmaxf(M, mw[w]);
    }
    float lt = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        a[w] = (mw[w] == -INFINITY) ? 0.0f : fast_exp2(mw[w] - M);
        lt += a[w] * lds[w * kWaveLds + 32 * D + 32 + l32];
    }
    if (q < Nq) {
        const float inv = 1.0f / lt;
        float* Orow = O + head + static_cast<size_t>(q) * D;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                f32x4 w4;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int r = 4 * b + u;
                    float acc = 0.0f;
#pragma unroll
                    for (int w = 0; w < 4; ++w)
                        acc += a[w] * lds[w * kWaveLds + (16 * dt + r) * 64 + lane];
                    w4[u] = acc * inv;
                }
                st16(Orow + 32 * dt + 8 * b + 4 * g2, __builtin_bit_cast(u32x4, w4));
            }
        }
        if (g2 == 0) L[static_cast<size_t>(bh) * Nq + q] = (M + fast_log2(lt)) * kLn2;
    }
}

}  // namespace dev

namespace detail {

namespace {

// Query/key extents of one launch (see the shape note at the top of this file).
struct FwdShape {
    int BH;     // query heads over the batch
    int Nq;     // query rows per head
    int Nk;     // key rows per key/value head
    int group;  // query heads per key/value head
};

template <typename T, int D>
FlashAttentionError run_forward16(const T* Q, const T* K, const T* V, T* O, float* L,
                                  const FwdShape& sh, float scale, bool causal,
                                  hipStream_t stream) {
    constexpr int kWaves128 = 8;  // waves per workgroup of the head_dim 128 kernel
    constexpr int kWaves64 = 8;   // waves per workgroup of the head_dim 64 kernel
    constexpr int kWaves32 = 4;   // ... at head_dim 32, and 64/96/128 by the rules below
    constexpr int kWaves256 = 4;  // waves per workgroup of the head_dim 256 kernel
    constexpr int BM = (D == 128 || D == 96) ? 32 * kWaves128
                       : D == 64 ? 32 * kWaves64
                       : D == 32 ? 32 * kWaves32
                                  : 32 * kWaves256;
    int nqb = (sh.Nq + BM - 1) / BM;
    long long blocks = static_cast<long long>(nqb) * sh.BH;
    if (blocks > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
    const int coff = sh.Nk - sh.Nq;
    const ProfileEvents tok = profile_kernel<T, D>("forward");
    if constexpr (D == 64) {
        // Launches with at least as many 256-row blocks as CUs: eight-wave workgroups of the
        // sequential kernel (two per CU), except causal ones with fewer than 8192 keys, which
        // take the pipelined kernel and its per-wave causal stop. Smaller launches: four-wave
        // workgroups of the sequential kernel (twice the workgroups, four per CU). Measured
        // (us): config 2 93 (pipelined, four waves) -> 86 (sequential, four) -> 85 (sequential,
        // eight); causal bf16 B=2 H=16 N=4096: 86-89 pipelined, 97-100 sequential; causal
        // B=1 H=32 N=8192: 332-343 pipelined, 302-313 sequential.
        if (blocks >= compute_units() && (!causal || sh.Nk >= 8192)) {
            launch_kernel(tok, (dev::fwd16_d64_seq_kernel<T, D, kWaves64>),
                               dim3(static_cast<unsigned>(blocks)), dim3(64 * kWaves64), 0,
                               stream, reinterpret_cast<const uint16_t*>(Q),
                               reinterpret_cast<const uint16_t*>(K),
                               reinterpret_cast<const uint16_t*>(V),
                               reinterpret_cast<uint16_t*>(O), L, sh.Nq, sh.Nk, coff, sh.group,
                               nqb, scale * dev::kLog2e, causal ? 1 : 0);
        } else if (blocks >= compute_units()) {
            launch_kernel(tok, (dev::fwd16_d64_kernel<T, kWaves64, D>),
                               dim3(static_cast<unsigned>(blocks)), dim3(64 * kWaves64), 0,
                               stream, reinterpret_cast<const uint16_t*>(Q),
                               reinterpret_cast<const uint16_t*>(K),
                               reinterpret_cast<const uint16_t*>(V),
                               reinterpret_cast<uint16_t*>(O), L, sh.Nq, sh.Nk, coff, sh.group,
                               nqb, scale * dev::kLog2e, causal ? 1 : 0);
        } else {
            nqb = (sh.Nq + 32 * kWaves32 - 1) / (32 * kWaves32);
            blocks = static_cast<long long>(nqb) * sh.BH;
            if (blocks > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
            launch_kernel(tok, (dev::fwd16_d64_seq_kernel<T, D, kWaves32>),
                               dim3(static_cast<unsigned>(blocks)), dim3(64 * kWaves32), 0,
                               stream, reinterpret_cast<const uint16_t*>(Q),
                               reinterpret_cast<const uint16_t*>(K),
                               reinterpret_cast<const uint16_t*>(V),
                               reinterpret_cast<uint16_t*>(O), L, sh.Nq, sh.Nk, coff, sh.group,
                               nqb, scale * dev::kLog2e, causal ? 1 : 0);
        }
    } else if constexpr (D == 32) {
        // The sequential kernel; eight-wave workgroups under the same rule as at head_dim 64
        // (non-causal B=4 H=16 N=2048: 62.3 -> 57.7 us; causal B=2 H=16 N=4096: 68.2 us with
        // four waves, 80.4 with eight, whose masked diagonal blocks it computes).
        const long long nqb8 = (sh.Nq + 32 * kWaves64 - 1) / (32 * kWaves64);
        if (nqb8 * sh.BH >= compute_units() && (!causal || sh.Nk >= 8192)) {
            nqb = static_cast<int>(nqb8);
            blocks = nqb8 * sh.BH;
            launch_kernel(tok, (dev::fwd16_d64_seq_kernel<T, D, kWaves64>),
                               dim3(static_cast<unsigned>(blocks)), dim3(64 * kWaves64), 0,
                               stream, reinterpret_cast<const uint16_t*>(Q),
                               reinterpret_cast<const uint16_t*>(K),
                               reinterpret_cast<const uint16_t*>(V),
                               reinterpret_cast<uint16_t*>(O), L, sh.Nq, sh.Nk, coff, sh.group,
                               nqb, scale * dev::kLog2e, causal ? 1 : 0);
        } else {
            launch_kernel(tok, (dev::fwd16_d64_seq_kernel<T, D, kWaves32>),
                               dim3(static_cast<unsigned>(blocks)), dim3(64 * kWaves32), 0,
                               stream, reinterpret_cast<const uint16_t*>(Q),
                               reinterpret_cast<const uint16_t*>(K),
                               reinterpret_cast<const uint16_t*>(V),
                               reinterpret_cast<uint16_t*>(O), L, sh.Nq, sh.Nk, coff, sh.group,
                               nqb, scale * dev::kLog2e, causal ? 1 : 0);
        }
    } else if constexpr (D == 256) {
        launch_kernel(tok, (dev::fwd16_d256_kernel<T, kWaves256>),
                           dim3(static_cast<unsigned>(blocks)), dim3(64 * kWaves256), 0, stream,
                           reinterpret_cast<const uint16_t*>(Q),
                           reinterpret_cast<const uint16_t*>(K),
                           reinterpret_cast<const uint16_t*>(V), reinterpret_cast<uint16_t*>(O),
                           L, sh.Nq, sh.Nk, coff, sh.group, nqb, scale * dev::kLog2e,
                           causal ? 1 : 0);
    } else if constexpr (D == 128 || D == 96) {
        // Four-wave workgroups (128 rows, two per CU) when fewer eight-wave ones than CUs
        // would run: twice the workgroups, and two share a CU (B=1 H=3 N=1000 causal: 28.9 ->
        // 24.4 us). Larger launches keep eight waves, whose K/V tiles serve twice the rows
        // (config 3: 144.9 us against 161.6 with four).
        if (blocks < compute_units()) {
            nqb = (sh.Nq + 32 * kWaves32 - 1) / (32 * kWaves32);
            blocks = static_cast<long long>(nqb) * sh.BH;
            launch_kernel(tok, (dev::fwd16_d128_kernel<T, kWaves32, D>),
                               dim3(static_cast<unsigned>(blocks)), dim3(64 * kWaves32), 0,
                               stream, reinterpret_cast<const uint16_t*>(Q),
                               reinterpret_cast<const uint16_t*>(K),
                               reinterpret_cast<const uint16_t*>(V),
                               reinterpret_cast<uint16_t*>(O), L, sh.Nq, sh.Nk, coff, sh.group,
                               nqb, scale * dev::kLog2e, causal ? 1 : 0);
        } else {
            launch_kernel(tok, (dev::fwd16_d128_kernel<T, kWaves128, D>),
                               dim3(static_cast<unsigned>(blocks)), dim3(64 * kWaves128), 0,
                               stream, reinterpret_cast<const uint16_t*>(Q),
                               reinterpret_cast<const uint16_t*>(K),
                               reinterpret_cast<const uint16_t*>(V),
                               reinterpret_cast<uint16_t*>(O), L, sh.Nq, sh.Nk, coff, sh.group,
                               nqb, scale * dev::kLog2e, causal ? 1 : 0);
        }
    } else {
        static_assert(D == 32 || D == 64 || D == 96 || D == 128 || D == 256, "head_dim");
    }
    return from_hip(hipGetLastError());
}

template <int D>
FlashAttentionError run_forward32(const float* Q, const float* K, const float* V, float* O,
                                  float* L, const FwdShape& sh, float scale, bool causal,
                                  hipStream_t stream) {
    using Cfg = dev::Fwd32Cfg<D>;
    const int nqb = (sh.Nq + Cfg::BM - 1) / Cfg::BM;
    const long long blocks = static_cast<long long>(nqb) * sh.BH;
    if (blocks > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
    const ProfileEvents tok = profile_kernel<float, D>("forward");
    if constexpr (D <= 64) {
        // Fewer workgroups of 128 rows than two per CU: split each 32-row block's keys over
        // the four waves of a workgroup instead (fwd32_split_kernel).
        if (blocks < 2LL * compute_units()) {
            const int nqb32 = (sh.Nq + 31) / 32;
            const long long blocks32 = static_cast<long long>(nqb32) * sh.BH;
            if (blocks32 > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
            launch_kernel(tok, (dev::fwd32_split_kernel<D>), dim3(static_cast<unsigned>(blocks32)),
                               dim3(256), 0, stream, Q, K, V, O, L, sh.Nq, sh.Nk, sh.Nk - sh.Nq,
                               sh.group, nqb32, compute_units() / dev::kNumXcd,
                               scale * dev::kLog2e, causal ? 1 : 0);
            return from_hip(hipGetLastError());
        }
    }
    launch_kernel(tok, (dev::fwd32_kernel<D>), dim3(static_cast<unsigned>(blocks)),
                       dim3(Cfg::kThreads), 0, stream, Q, K, V, O, L, sh.Nq, sh.Nk,
                       sh.Nk - sh.Nq, sh.group, nqb, scale * dev::kLog2e, causal ? 1 : 0);
    return from_hip(hipGetLastError());
}

template <typename T, int D>
FlashAttentionError run_forward_d(const T* Q, const T* K, const T* V, T* O, float* L,
                                  const FwdShape& sh, float scale, bool causal,
                                  hipStream_t stream) {
    if constexpr (std::is_same<T, float>::value)
        return run_forward32<D>(Q, K, V, O, L, sh, scale, causal, stream);
    else
        return run_forward16<T, D>(Q, K, V, O, L, sh, scale, causal, stream);
}

// head_dim dispatch; `extended` admits the head dims beyond the reference's 32 / 64 / 128.
template <typename T>
FlashAttentionError run_forward(const T* Q, const T* K, const T* V, T* O, float* L,
                                const FwdShape& sh, int head_dim, bool extended, float scale,
                                bool causal, hipStream_t stream) {
    switch (head_dim) {
        case 32: return run_forward_d<T, 32>(Q, K, V, O, L, sh, scale, causal, stream);
        case 64: return run_forward_d<T, 64>(Q, K, V, O, L, sh, scale, causal, stream);
        case 128: return run_forward_d<T, 128>(Q, K, V, O, L, sh, scale, causal, stream);
        case 96:
            if (extended) return run_forward_d<T, 96>(Q, K, V, O, L, sh, scale, causal, stream);
            break;
        case 256:
            if (extended) return run_forward_d<T, 256>(Q, K, V, O, L, sh, scale, causal, stream);
            break;
    }
    return FlashAttentionError::UNSUPPORTED_HEAD_DIM;
}

}  // namespace

template <typename T>
FlashAttentionError launch_forward(const T* Q, const T* K, const T* V, T* O, float* L,
                                   int batch_size, int num_heads, int seq_len, int head_dim,
                                   float scale, bool causal, hipStream_t stream) {
    const long long bh = static_cast<long long>(batch_size) * num_heads;
    if (bh > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
    const FwdShape sh{static_cast<int>(bh), seq_len, seq_len, 1};
    return run_forward<T>(Q, K, V, O, L, sh, head_dim, false, scale, causal, stream);
}

template <typename T>
FlashAttentionError launch_forward_ext(const T* Q, const T* K, const T* V, T* O, float* L,
                                       int batch_size, int num_heads, int num_kv_heads,
                                       int q_len, int kv_len, int head_dim, float scale,
                                       bool causal, hipStream_t stream) {
    const long long bh = static_cast<long long>(batch_size) * num_heads;
    if (bh > 0x7fffffffLL) return FlashAttentionError::INVALID_DIMENSION;
    const FwdShape sh{static_cast<int>(bh), q_len, kv_len, num_heads / num_kv_heads};
    return run_forward<T>(Q, K, V, O, L, sh, head_dim, true, scale, causal, stream);
}

#define CUFLASH_FORWARD_TYPE(T)                                                                 \
    template FlashAttentionError launch_forward<T>(const T*, const T*, const T*, T*, float*,    \
                                                   int, int, int, int, float, bool,             \
                                                   hipStream_t);                                \
    template FlashAttentionError launch_forward_ext<T>(const T*, const T*, const T*, T*,        \
                                                       float*, int, int, int, int, int, int,    \
                                                       float, bool, hipStream_t);
CUFLASH_FORWARD_TYPE(float)
CUFLASH_FORWARD_TYPE(__half)
CUFLASH_FORWARD_TYPE(__hip_bfloat16)
#undef CUFLASH_FORWARD_TYPE

}  // namespace detail
}  // namespace cuflash
