#pragma once

// Online-softmax step shared by the forward kernels.
//
// Semantics follow the reference's streaming softmax (src/forward/flash_attention_forward_typed.cu
// :88-135, src/forward/flash_attention_forward_wmma.cu:126-158 and the update rule of
// src/kernels/impl/online_softmax.cuh:28-33): per query row keep a running max m and a running
// sum l of exp(s - m); when a block raises the max, rescale l and the output accumulator by
// exp(m_old - m_new); P = exp(s - m) feeds P*V; at the end O /= l and L = m + log(l).
//
// gfx950 specifics:
//  * scores live in MFMA accumulator tiles of S^T (rows = keys, column = this lane's query),
//    so a query row is owned by the lane pair (l, l^32): the row max needs one cross-half
//    exchange and the row sum is kept as a per-lane partial that is combined once at the end;
//  * the exponent runs in base 2 (v_exp_f32): m is kept as max(s) * scale * log2(e) and
//    p = exp2(s * scale * log2(e) - m), one FMA + one v_exp_f32 per score;
//  * rescaling is lazy: m is only moved when the block max exceeds it by more than
//    kLazyRescale (log2 units), so most blocks skip the O *= alpha pass. The result is exact
//    in real arithmetic (O and l always refer to the same m); P stays below 2^kLazyRescale.

#include "common.hpp"

namespace cuflash {
namespace dev {

constexpr float kLazyRescale = 8.0f;

// Masks, then folds NT score tiles (C layout of S^T for keys key0 .. key0 + 32*NT - 1) into the
// running state (m, l) of this lane's query q. On return s holds P (unnormalized, relative to
// the updated m). Returns true when the caller must multiply its output accumulator by alpha.
template <int NT, bool kMasked>
__device__ __forceinline__ bool softmax_step(f32x16 (&s)[NT], int key0, int q, int n_keys,
                                             bool causal, float c, float& m, float& l,
                                             float& alpha) {
    const int g2 = (threadIdx.x & 63) >> 5;
    if constexpr (kMasked) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = key0 + 32 * t + 8 * (r >> 2) + 4 * g2 + (r & 3);
                const bool ok = key < n_keys && (!causal || key <= q);
                s[t][r] = ok ? s[t][r] : -INFINITY;
            }
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[t][r]);
    }
    mx = fmaxf(mx, xor_shuffle(mx, 32));
    const float m_blk = (mx == -INFINITY) ? -INFINITY : mx * c;
    const float m_new = fmaxf(m, m_blk);
    const bool grow = m_new > m + kLazyRescale;
    const bool rescale = __ballot(grow) != 0;
    alpha = 1.0f;
    if (rescale) {
        alpha = (m_new == -INFINITY) ? 1.0f : fast_exp2(m - m_new);
        m = m_new;
        l *= alpha;
    }
    const float m_use = (m == -INFINITY) ? 0.0f : m;
    float sum = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float p = fast_exp2(fmaf(s[t][r], c, -m_use));
            if constexpr (kMasked) p = (s[t][r] == -INFINITY) ? 0.0f : p;
            s[t][r] = p;
            sum += p;
        }
    }
    l += sum;
    return rescale;
}

}  // namespace dev
}  // namespace cuflash
