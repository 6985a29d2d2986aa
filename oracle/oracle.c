/*
 * CPU oracle for the FlashAttention hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library,
 * and only as the checker (or, for cpu_naive_*, as the reported CPU baseline). The product
 * (libcuflash_attn.so) never calls it and has no CPU fallback.
 *
 * Contents
 *   oracle_forward         fp64 restatement of the reference's reference_attention_forward and
 *                          reference_logsumexp (tests/unit/test_forward.cu:21-69, :83-118):
 *                          O_i = sum_j softmax_j(scale * q_i.k_j) v_j, L_i = m_i + log sum_j
 *                          exp(s_ij - m_i), causal keys j > i (+ Nk - Nq) masked.
 *   oracle_backward        fp64 restatement of reference_attention_backward
 *                          (tests/unit/test_backward.cu:21-127): P, dV = P^T dO, dP = dO V^T,
 *                          D_i = sum_j P_ij dP_ij, dS = P (dP - D) (0 where masked),
 *                          dQ = scale dS K, dK = scale dS^T Q. Materializes P per head.
 *                          Q and K may differ in length (Nq <= Nk when causal), as in the
 *                          forward.
 *   oracle_backward_rows   Row-streaming form of the same gradients for selected query rows
 *                          (dQ) and key rows (dK, dV), separate query and key lengths as in
 *                          oracle_backward, O((Nq + Nk) * D) memory: first a pass computing
 *                          L_i and O_i, then D_i = dO_i . O_i (the identity the reference kernel
 *                          uses, src/backward/flash_attention_backward_typed.cu:13-34), then
 *                          P_ij = exp(s_ij - L_i).
 *   oracle_decode_partials / oracle_decode_combine
 *                          Split-KV decode restated: per chunk (m_s, l_s, acc_s) and the merge
 *                          rule of src/kernels/impl/online_softmax.cuh:28-33.
 *   cpu_naive_forward_f32 / cpu_naive_backward_f32
 *                          The reference's naive CPU attention in float arithmetic, exactly as
 *                          written in the two test files above, multithreaded over heads: the
 *                          reported CPU baseline (a port of the reference's CPU path).
 *   cpu_naive_rows_f32     The same two naive passes restricted to chosen query rows of one
 *                          head (row i's loops exactly as above, its dK / dV terms summed), so
 *                          that an evenly spread sample of a long head can be timed.
 *   cpu_naive_decode_f32   The naive forward's loops at a query length of 1 (the decode CPU
 *                          baseline; the reference has no decode path).
 *
 * The `mutation` argument (0 = none) plants a known mistake for the tests that check that the
 * pinning checks catch it; it is never non-zero outside those tests:
 *   1 = K used transposed in the score (k[d][j] instead of k[j][d], square heads only)
 *   2 = causal mask off by one (j >= i masked)
 *   3 = dS sign flipped (P (dP + D))
 *   4 = scale dropped from dK
 *   5 = max not subtracted before exp (drops the LSE shift; L = log sum exp(s))
 *   6 = dV from P instead of P^T (dV_j = sum_i P_ji dO_i)
 *   7 = causal mask aligned to the start of the key sequence (j > i) when Nq != Nk
 */

#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef int64_t i64;

/* ------------------------------------------------------------------------------------------ */
/* thread pool over an index range                                                             */
/* ------------------------------------------------------------------------------------------ */
typedef void (*range_fn)(void* ctx, i64 begin, i64 end);

typedef struct {
    range_fn fn;
    void* ctx;
    i64 begin, end;
} range_job;

static void* range_thread(void* p) {
    range_job* j = (range_job*)p;
    j->fn(j->ctx, j->begin, j->end);
    return NULL;
}

static void parallel_for(i64 n, int nthreads, range_fn fn, void* ctx) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > n) nthreads = (int)(n > 0 ? n : 1);
    if (nthreads == 1) {
        fn(ctx, 0, n);
        return;
    }
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
    range_job* jobs = (range_job*)malloc(sizeof(range_job) * (size_t)nthreads);
    for (int t = 0; t < nthreads; ++t) {
        jobs[t].fn = fn;
        jobs[t].ctx = ctx;
        jobs[t].begin = n * t / nthreads;
        jobs[t].end = n * (t + 1) / nthreads;
        pthread_create(&th[t], NULL, range_thread, &jobs[t]);
    }
    for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
}

static int masked_key(i64 i, i64 j, i64 Nq, i64 Nk, int causal, int mutation) {
    if (!causal) return 0;
    /* bottom-right aligned (j > i when Nq == Nk); mutation 7 aligns it top-left instead */
    const i64 lim = (mutation == 7) ? i : i + (Nk - Nq);
    return mutation == 2 ? (j >= lim) : (j > lim);
}

/* score s_ij = scale * sum_d q_id k_jd in fp64 */
static double score(const float* q, const float* Kh, i64 j, i64 D, i64 Nk, double scale,
                    int mutation) {
    double dot = 0.0;
    if (mutation == 1) {
        for (i64 d = 0; d < D; ++d) dot += (double)q[d] * (double)Kh[d * Nk + j];
    } else {
        const float* k = Kh + j * D;
        for (i64 d = 0; d < D; ++d) dot += (double)q[d] * (double)k[d];
    }
    return dot * scale;
}

/* ------------------------------------------------------------------------------------------ */
/* forward                                                                                     */
/* ------------------------------------------------------------------------------------------ */
typedef struct {
    const float *Q, *K, *V;
    float *O, *L;
    i64 Nq, Nk, D;
    double scale;
    int causal, mutation;
} fwd_ctx;

static void fwd_rows(void* p, i64 begin, i64 end) {
    fwd_ctx* c = (fwd_ctx*)p;
    double* s = (double*)malloc(sizeof(double) * (size_t)c->Nk);
    double* acc = (double*)malloc(sizeof(double) * (size_t)c->D);
    for (i64 r = begin; r < end; ++r) {
        const i64 bh = r / c->Nq, i = r % c->Nq;
        const float* q = c->Q + (bh * c->Nq + i) * c->D;
        const float* Kh = c->K + bh * c->Nk * c->D;
        const float* Vh = c->V + bh * c->Nk * c->D;
        double m = -INFINITY;
        for (i64 j = 0; j < c->Nk; ++j) {
            if (masked_key(i, j, c->Nq, c->Nk, c->causal, c->mutation)) {
                s[j] = -INFINITY;
                continue;
            }
            s[j] = score(q, Kh, j, c->D, c->Nk, c->scale, c->mutation);
            if (s[j] > m) m = s[j];
        }
        const double shift = (c->mutation == 5) ? 0.0 : m;
        double l = 0.0;
        for (i64 d = 0; d < c->D; ++d) acc[d] = 0.0;
        for (i64 j = 0; j < c->Nk; ++j) {
            if (s[j] == -INFINITY) continue;
            const double p = exp(s[j] - shift);
            l += p;
            const float* v = Vh + j * c->D;
            for (i64 d = 0; d < c->D; ++d) acc[d] += p * (double)v[d];
        }
        float* o = c->O + (bh * c->Nq + i) * c->D;
        for (i64 d = 0; d < c->D; ++d) o[d] = (float)(acc[d] / l);
        if (c->L) c->L[bh * c->Nq + i] = (float)(shift + log(l));
    }
    free(s);
    free(acc);
}

int oracle_forward(const float* Q, const float* K, const float* V, float* O, float* L, i64 BH,
                   i64 Nq, i64 Nk, i64 D, double scale, int causal, int nthreads, int mutation) {
    if (!Q || !K || !V || !O || BH <= 0 || Nq <= 0 || Nk <= 0 || D <= 0) return 1;
    if (causal && Nq > Nk) return 1; /* rows without any visible key */
    fwd_ctx c = {Q, K, V, O, L, Nq, Nk, D, scale, causal, mutation};
    parallel_for(BH * Nq, nthreads, fwd_rows, &c);
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* backward, materialized (direct restatement of test_backward.cu:21-127)                      */
/* Q, dO, dQ are [BH, Nq, D]; K, V, dK, dV are [BH, Nk, D]; causal masks j > i + Nk - Nq.      */
/* ------------------------------------------------------------------------------------------ */
typedef struct {
    const float *Q, *K, *V, *dO;
    float *dQ, *dK, *dV;
    i64 Nq, Nk, D;
    double scale;
    int causal, mutation;
} bwd_ctx;

static void bwd_heads(void* p, i64 begin, i64 end) {
    bwd_ctx* c = (bwd_ctx*)p;
    const i64 Nq = c->Nq, Nk = c->Nk, D = c->D;
    double* P = (double*)malloc(sizeof(double) * (size_t)(Nq * Nk));
    double* dP = (double*)malloc(sizeof(double) * (size_t)(Nq * Nk));
    for (i64 bh = begin; bh < end; ++bh) {
        const i64 qoff = bh * Nq * D, koff = bh * Nk * D;
        const float *Qh = c->Q + qoff, *Kh = c->K + koff, *Vh = c->V + koff, *dOh = c->dO + qoff;
        /* P */
        for (i64 i = 0; i < Nq; ++i) {
            double m = -INFINITY;
            double* Pi = P + i * Nk;
            for (i64 j = 0; j < Nk; ++j) {
                if (masked_key(i, j, Nq, Nk, c->causal, c->mutation)) {
                    Pi[j] = -INFINITY;
                } else {
                    Pi[j] = score(Qh + i * D, Kh, j, D, Nk, c->scale, c->mutation);
                }
                if (Pi[j] > m) m = Pi[j];
            }
            const double shift = (c->mutation == 5) ? 0.0 : m;
            double sum = 0.0;
            for (i64 j = 0; j < Nk; ++j) {
                Pi[j] = (Pi[j] == -INFINITY) ? 0.0 : exp(Pi[j] - shift);
                sum += Pi[j];
            }
            for (i64 j = 0; j < Nk; ++j) Pi[j] /= sum;
        }
        /* dV = P^T dO (mutation 6 reads P transposed, defined for Nq == Nk only) */
        for (i64 j = 0; j < Nk; ++j) {
            for (i64 d = 0; d < D; ++d) {
                double s = 0.0;
                for (i64 i = 0; i < Nq; ++i) {
                    const double pij = (c->mutation == 6) ? P[j * Nk + i] : P[i * Nk + j];
                    s += pij * (double)dOh[i * D + d];
                }
                c->dV[koff + j * D + d] = (float)s;
            }
        }
        /* dP = dO V^T */
        for (i64 i = 0; i < Nq; ++i)
            for (i64 j = 0; j < Nk; ++j) {
                double s = 0.0;
                for (i64 d = 0; d < D; ++d) s += (double)dOh[i * D + d] * (double)Vh[j * D + d];
                dP[i * Nk + j] = s;
            }
        /* dS = P (dP - D_i), D_i = sum_j P_ij dP_ij; stored in dP */
        for (i64 i = 0; i < Nq; ++i) {
            double Di = 0.0;
            for (i64 j = 0; j < Nk; ++j) Di += P[i * Nk + j] * dP[i * Nk + j];
            for (i64 j = 0; j < Nk; ++j) {
                if (masked_key(i, j, Nq, Nk, c->causal, c->mutation)) {
                    dP[i * Nk + j] = 0.0;
                } else {
                    const double diff =
                        (c->mutation == 3) ? dP[i * Nk + j] + Di : dP[i * Nk + j] - Di;
                    dP[i * Nk + j] = P[i * Nk + j] * diff;
                }
            }
        }
        /* dQ = scale dS K, dK = scale dS^T Q */
        for (i64 i = 0; i < Nq; ++i)
            for (i64 d = 0; d < D; ++d) {
                double s = 0.0;
                for (i64 j = 0; j < Nk; ++j) s += dP[i * Nk + j] * (double)Kh[j * D + d];
                c->dQ[qoff + i * D + d] = (float)(s * c->scale);
            }
        for (i64 j = 0; j < Nk; ++j)
            for (i64 d = 0; d < D; ++d) {
                double s = 0.0;
                for (i64 i = 0; i < Nq; ++i) s += dP[i * Nk + j] * (double)Qh[i * D + d];
                c->dK[koff + j * D + d] = (float)(c->mutation == 4 ? s : s * c->scale);
            }
    }
    free(P);
    free(dP);
}

int oracle_backward(const float* Q, const float* K, const float* V, const float* dO, float* dQ,
                    float* dK, float* dV, i64 BH, i64 Nq, i64 Nk, i64 D, double scale, int causal,
                    int nthreads, int mutation) {
    if (!Q || !K || !V || !dO || !dQ || !dK || !dV || BH <= 0 || Nq <= 0 || Nk <= 0 || D <= 0)
        return 1;
    if (causal && Nq > Nk) return 1; /* rows without any visible key */
    if (mutation == 6 && Nq != Nk) return 1;
    bwd_ctx c = {Q, K, V, dO, dQ, dK, dV, Nq, Nk, D, scale, causal, mutation};
    parallel_for(BH, nthreads, bwd_heads, &c);
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* backward, row-streaming (selected rows, O((Nq + Nk) * D) memory per head)                    */
/* Q, dO are [BH, Nq, D]; K, V are [BH, Nk, D]; causal masks j > i + Nk - Nq (as above).        */
/* ------------------------------------------------------------------------------------------ */
typedef struct {
    const float *Q, *K, *V, *dO;
    float *dQ, *dK, *dV;
    const i64 *qrows, *krows;
    i64 nq, nk, BH, Nq, Nk, D;
    double scale;
    int causal, mutation;
    double *Lrow, *Drow; /* [BH][Nq] */
} bwdr_ctx;

/* pass 1: L_i and D_i = dO_i . O_i for every query row of every head */
static void bwdr_stats(void* p, i64 begin, i64 end) {
    bwdr_ctx* c = (bwdr_ctx*)p;
    const i64 Nq = c->Nq, Nk = c->Nk, D = c->D;
    double* s = (double*)malloc(sizeof(double) * (size_t)Nk);
    double* acc = (double*)malloc(sizeof(double) * (size_t)D);
    for (i64 r = begin; r < end; ++r) {
        const i64 bh = r / Nq, i = r % Nq, qoff = bh * Nq * D, koff = bh * Nk * D;
        const float* q = c->Q + qoff + i * D;
        double m = -INFINITY;
        for (i64 j = 0; j < Nk; ++j) {
            s[j] = masked_key(i, j, Nq, Nk, c->causal, c->mutation)
                       ? -INFINITY
                       : score(q, c->K + koff, j, D, Nk, c->scale, c->mutation);
            if (s[j] > m) m = s[j];
        }
        const double shift = (c->mutation == 5) ? 0.0 : m;
        double l = 0.0;
        for (i64 d = 0; d < D; ++d) acc[d] = 0.0;
        for (i64 j = 0; j < Nk; ++j) {
            if (s[j] == -INFINITY) continue;
            const double pj = exp(s[j] - shift);
            l += pj;
            for (i64 d = 0; d < D; ++d) acc[d] += pj * (double)c->V[koff + j * D + d];
        }
        double Di = 0.0;
        for (i64 d = 0; d < D; ++d) Di += (double)c->dO[qoff + i * D + d] * (acc[d] / l);
        c->Lrow[r] = shift + log(l);
        c->Drow[r] = Di;
    }
    free(s);
    free(acc);
}

/* dS_ij of head bh for one (i, j) pair given the row statistics; P_ij in *P_out */
static double bwdr_ds(const bwdr_ctx* c, i64 bh, i64 i, i64 j, double* P_out) {
    const i64 D = c->D, qoff = bh * c->Nq * D, koff = bh * c->Nk * D, r = bh * c->Nq + i;
    if (masked_key(i, j, c->Nq, c->Nk, c->causal, c->mutation)) {
        *P_out = 0.0;
        return 0.0;
    }
    const double s = score(c->Q + qoff + i * D, c->K + koff, j, D, c->Nk, c->scale, c->mutation);
    const double P = exp(s - c->Lrow[r]);
    double dp = 0.0;
    for (i64 d = 0; d < D; ++d) dp += (double)c->dO[qoff + i * D + d] * (double)c->V[koff + j * D + d];
    *P_out = P;
    return P * ((c->mutation == 3) ? dp + c->Drow[r] : dp - c->Drow[r]);
}

static void bwdr_grads(void* p, i64 begin, i64 end) {
    bwdr_ctx* c = (bwdr_ctx*)p;
    const i64 D = c->D, per_head = c->nq + c->nk;
    double* acc = (double*)malloc(sizeof(double) * (size_t)(2 * D));
    for (i64 t = begin; t < end; ++t) {
        const i64 bh = t / per_head, w = t % per_head;
        const i64 qoff = bh * c->Nq * D, koff = bh * c->Nk * D;
        double P;
        if (w < c->nq) { /* dQ row */
            const i64 i = c->qrows[w];
            for (i64 d = 0; d < D; ++d) acc[d] = 0.0;
            for (i64 j = 0; j < c->Nk; ++j) {
                const double ds = bwdr_ds(c, bh, i, j, &P);
                if (ds == 0.0) continue;
                for (i64 d = 0; d < D; ++d) acc[d] += ds * (double)c->K[koff + j * D + d];
            }
            for (i64 d = 0; d < D; ++d) c->dQ[(bh * c->nq + w) * D + d] = (float)(acc[d] * c->scale);
        } else { /* dK, dV row */
            const i64 wk = w - c->nq, j = c->krows[wk];
            for (i64 d = 0; d < 2 * D; ++d) acc[d] = 0.0;
            for (i64 i = 0; i < c->Nq; ++i) {
                const double ds = bwdr_ds(c, bh, i, j, &P);
                for (i64 d = 0; d < D; ++d) {
                    acc[d] += ds * (double)c->Q[qoff + i * D + d];
                    acc[D + d] += P * (double)c->dO[qoff + i * D + d];
                }
            }
            for (i64 d = 0; d < D; ++d) {
                c->dK[(bh * c->nk + wk) * D + d] =
                    (float)(c->mutation == 4 ? acc[d] : acc[d] * c->scale);
                c->dV[(bh * c->nk + wk) * D + d] = (float)acc[D + d];
            }
        }
    }
    free(acc);
}

int oracle_backward_rows(const float* Q, const float* K, const float* V, const float* dO,
                         float* dQ, float* dK, float* dV, i64 BH, i64 Nq, i64 Nk, i64 D,
                         double scale, int causal, const i64* qrows, i64 nq, const i64* krows,
                         i64 nk, int nthreads, int mutation) {
    if (!Q || !K || !V || !dO || BH <= 0 || Nq <= 0 || Nk <= 0 || D <= 0) return 1;
    if (causal && Nq > Nk) return 1; /* rows without any visible key */
    for (i64 w = 0; w < nq; ++w)
        if (qrows[w] < 0 || qrows[w] >= Nq) return 1;
    for (i64 w = 0; w < nk; ++w)
        if (krows[w] < 0 || krows[w] >= Nk) return 1;
    bwdr_ctx c = {Q,  K,  V,  dO, dQ, dK,    dV,     qrows,    krows, nq,  nk,
                  BH, Nq, Nk, D,  scale, causal, mutation, NULL,  NULL};
    c.Lrow = (double*)malloc(sizeof(double) * (size_t)(BH * Nq));
    c.Drow = (double*)malloc(sizeof(double) * (size_t)(BH * Nq));
    if (!c.Lrow || !c.Drow) {
        free(c.Lrow);
        free(c.Drow);
        return 2;
    }
    parallel_for(BH * Nq, nthreads, bwdr_stats, &c);
    parallel_for(BH * (nq + nk), nthreads, bwdr_grads, &c);
    free(c.Lrow);
    free(c.Drow);
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* split-KV decode                                                                              */
/* ------------------------------------------------------------------------------------------ */
/* Partial state of keys [s*chunk, min(Nk, (s+1)*chunk)) for every head: m (natural log units),
 * l = sum exp(s_j - m), acc = sum exp(s_j - m) v_j. Empty chunks give m = -inf, l = 0. */
int oracle_decode_partials(const float* Q, const float* K, const float* V, i64 BH, i64 Nk, i64 D,
                           double scale, i64 nsplit, i64 chunk, double* m_out, double* l_out,
                           double* acc_out) {
    for (i64 bh = 0; bh < BH; ++bh)
        for (i64 s = 0; s < nsplit; ++s) {
            const i64 b = s * chunk, e = (b + chunk < Nk) ? b + chunk : Nk;
            const float* q = Q + bh * D;
            const float* Kh = K + bh * Nk * D;
            const float* Vh = V + bh * Nk * D;
            double m = -INFINITY, l = 0.0;
            double* acc = acc_out + (bh * nsplit + s) * D;
            for (i64 d = 0; d < D; ++d) acc[d] = 0.0;
            for (i64 j = b; j < e; ++j) {
                const double sj = score(q, Kh, j, D, Nk, scale, 0);
                if (sj > m) m = sj;
            }
            for (i64 j = b; j < e; ++j) {
                const double p = exp(score(q, Kh, j, D, Nk, scale, 0) - m);
                l += p;
                for (i64 d = 0; d < D; ++d) acc[d] += p * (double)Vh[j * D + d];
            }
            m_out[bh * nsplit + s] = m;
            l_out[bh * nsplit + s] = l;
        }
    return 0;
}

/* Merge rule of src/kernels/impl/online_softmax.cuh:28-33 applied across the splits. */
int oracle_decode_combine(const double* m_in, const double* l_in, const double* acc_in, i64 BH,
                          i64 nsplit, i64 D, float* O, float* L) {
    for (i64 bh = 0; bh < BH; ++bh) {
        double M = -INFINITY;
        for (i64 s = 0; s < nsplit; ++s)
            if (m_in[bh * nsplit + s] > M) M = m_in[bh * nsplit + s];
        double l = 0.0;
        for (i64 s = 0; s < nsplit; ++s) {
            const double ms = m_in[bh * nsplit + s];
            if (ms != -INFINITY) l += l_in[bh * nsplit + s] * exp(ms - M);
        }
        for (i64 d = 0; d < D; ++d) {
            double a = 0.0;
            for (i64 s = 0; s < nsplit; ++s) {
                const double ms = m_in[bh * nsplit + s];
                if (ms != -INFINITY) a += acc_in[(bh * nsplit + s) * D + d] * exp(ms - M);
            }
            O[bh * D + d] = (float)(a / l);
        }
        L[bh] = (float)(M + log(l));
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* naive fp32 CPU attention: the reported CPU baseline                                          */
/* ------------------------------------------------------------------------------------------ */
typedef struct {
    const float *Q, *K, *V, *dO;
    float *O, *L, *dQ, *dK, *dV;
    i64 N, D;
    float scale;
    int causal;
} naive_ctx;

/* tests/unit/test_forward.cu:21-69 (O) and :83-118 (L), float arithmetic */
static void naive_fwd_heads(void* p, i64 begin, i64 end) {
    naive_ctx* c = (naive_ctx*)p;
    const i64 N = c->N, D = c->D;
    float* scores = (float*)malloc(sizeof(float) * (size_t)N);
    for (i64 bh = begin; bh < end; ++bh) {
        const i64 off = bh * N * D;
        for (i64 i = 0; i < N; ++i) {
            float max_score = -INFINITY;
            for (i64 j = 0; j < N; ++j) {
                if (c->causal && j > i) {
                    scores[j] = -INFINITY;
                } else {
                    float dot = 0.0f;
                    for (i64 d = 0; d < D; ++d) dot += c->Q[off + i * D + d] * c->K[off + j * D + d];
                    scores[j] = dot * c->scale;
                }
                if (scores[j] > max_score) max_score = scores[j];
            }
            float sum_exp = 0.0f;
            for (i64 j = 0; j < N; ++j) {
                scores[j] = expf(scores[j] - max_score);
                sum_exp += scores[j];
            }
            for (i64 j = 0; j < N; ++j) scores[j] /= sum_exp;
            for (i64 d = 0; d < D; ++d) {
                float sum = 0.0f;
                for (i64 j = 0; j < N; ++j) sum += scores[j] * c->V[off + j * D + d];
                c->O[off + i * D + d] = sum;
            }
            if (c->L) c->L[bh * N + i] = max_score + logf(sum_exp);
        }
    }
    free(scores);
}

/* tests/unit/test_backward.cu:21-127, float arithmetic, P / dP / dS materialized per head */
static void naive_bwd_heads(void* p, i64 begin, i64 end) {
    naive_ctx* c = (naive_ctx*)p;
    const i64 N = c->N, D = c->D;
    float* P = (float*)malloc(sizeof(float) * (size_t)(N * N));
    float* dP = (float*)malloc(sizeof(float) * (size_t)(N * N));
    for (i64 bh = begin; bh < end; ++bh) {
        const i64 off = bh * N * D;
        const float *Q = c->Q + off, *K = c->K + off, *V = c->V + off, *dO = c->dO + off;
        for (i64 i = 0; i < N; ++i) {
            float max_score = -INFINITY;
            float* s = P + i * N;
            for (i64 j = 0; j < N; ++j) {
                if (c->causal && j > i) {
                    s[j] = -INFINITY;
                } else {
                    float dot = 0.0f;
                    for (i64 d = 0; d < D; ++d) dot += Q[i * D + d] * K[j * D + d];
                    s[j] = dot * c->scale;
                }
                if (s[j] > max_score) max_score = s[j];
            }
            float sum_exp = 0.0f;
            for (i64 j = 0; j < N; ++j) {
                s[j] = expf(s[j] - max_score);
                sum_exp += s[j];
            }
            for (i64 j = 0; j < N; ++j) s[j] /= sum_exp;
        }
        for (i64 j = 0; j < N; ++j)
            for (i64 d = 0; d < D; ++d) {
                float sum = 0.0f;
                for (i64 i = 0; i < N; ++i) sum += P[i * N + j] * dO[i * D + d];
                c->dV[off + j * D + d] = sum;
            }
        for (i64 i = 0; i < N; ++i)
            for (i64 j = 0; j < N; ++j) {
                float sum = 0.0f;
                for (i64 d = 0; d < D; ++d) sum += dO[i * D + d] * V[j * D + d];
                dP[i * N + j] = sum;
            }
        for (i64 i = 0; i < N; ++i) {
            float Di = 0.0f;
            for (i64 j = 0; j < N; ++j) Di += P[i * N + j] * dP[i * N + j];
            for (i64 j = 0; j < N; ++j)
                dP[i * N + j] = (c->causal && j > i) ? 0.0f : P[i * N + j] * (dP[i * N + j] - Di);
        }
        for (i64 i = 0; i < N; ++i)
            for (i64 d = 0; d < D; ++d) {
                float sum = 0.0f;
                for (i64 j = 0; j < N; ++j) sum += dP[i * N + j] * K[j * D + d];
                c->dQ[off + i * D + d] = sum * c->scale;
            }
        for (i64 j = 0; j < N; ++j)
            for (i64 d = 0; d < D; ++d) {
                float sum = 0.0f;
                for (i64 i = 0; i < N; ++i) sum += dP[i * N + j] * Q[i * D + d];
                c->dK[off + j * D + d] = sum * c->scale;
            }
    }
    free(P);
    free(dP);
}

int cpu_naive_forward_f32(const float* Q, const float* K, const float* V, float* O, float* L,
                          i64 BH, i64 N, i64 D, float scale, int causal, int nthreads) {
    naive_ctx c = {Q, K, V, NULL, O, L, NULL, NULL, NULL, N, D, scale, causal};
    parallel_for(BH, nthreads, naive_fwd_heads, &c);
    return 0;
}

int cpu_naive_backward_f32(const float* Q, const float* K, const float* V, const float* dO,
                           float* dQ, float* dK, float* dV, i64 BH, i64 N, i64 D, float scale,
                           int causal, int nthreads) {
    naive_ctx c = {Q, K, V, dO, NULL, NULL, dQ, dK, dV, N, D, scale, causal};
    parallel_for(BH, nthreads, naive_bwd_heads, &c);
    return 0;
}

/* The same naive fp32 forward and backward restricted to the query rows `rows` of one head, so
 * that a bounded, evenly spread sample of a long head can be timed. Each selected row i does
 * the work the two functions above do for it, loop for loop: the forward's score row (dot
 * products for the unmasked keys, exp and normalization over all N keys), O_i and L_i; the
 * backward's recomputed P row, dP row over all N keys, D_i, dS row, dQ_i (all N keys), and
 * row i's terms of dV (P_ij dO_i) and dK (dS_ij q_i) for every key j. Rows are split over the
 * threads; each thread sums its dK / dV terms into its own [N, D] buffers and the buffers are
 * added at the end. With every row selected the outputs equal cpu_naive_forward_f32 /
 * cpu_naive_backward_f32 up to the order of the dK / dV sums over i. */
typedef struct {
    const float *Q, *K, *V, *dO;
    const i64* rows;
    float *O, *L, *dQ, *dK, *dV;
    float* part; /* nthreads x (dK, dV) x [N, D] */
    i64 N, D, nrows;
    float scale;
    int causal, nthreads;
} naive_rows_ctx;

static void naive_rows_job(void* p, i64 begin, i64 end) {
    naive_rows_ctx* c = (naive_rows_ctx*)p;
    const i64 N = c->N, D = c->D;
    float* s = (float*)malloc(sizeof(float) * (size_t)N);
    float* dP = (float*)malloc(sizeof(float) * (size_t)N);
    for (i64 t = begin; t < end; ++t) {
        float* pk = c->part + (size_t)t * 2 * (size_t)(N * D);
        float* pv = pk + N * D;
        memset(pk, 0, sizeof(float) * (size_t)(2 * N * D));
        for (i64 r = c->nrows * t / c->nthreads; r < c->nrows * (t + 1) / c->nthreads; ++r) {
            const i64 i = c->rows[r];
            const float* qi = c->Q + i * D;
            const float* doi = c->dO + i * D;
            /* forward row (naive_fwd_heads) */
            for (int pass = 0; pass < 2; ++pass) {
                float max_score = -INFINITY;
                for (i64 j = 0; j < N; ++j) {
                    if (c->causal && j > i) {
                        s[j] = -INFINITY;
                    } else {
                        float dot = 0.0f;
                        for (i64 d = 0; d < D; ++d) dot += qi[d] * c->K[j * D + d];
                        s[j] = dot * c->scale;
                    }
                    if (s[j] > max_score) max_score = s[j];
                }
                float sum_exp = 0.0f;
                for (i64 j = 0; j < N; ++j) {
                    s[j] = expf(s[j] - max_score);
                    sum_exp += s[j];
                }
                for (i64 j = 0; j < N; ++j) s[j] /= sum_exp;
                if (pass == 0) {
                    for (i64 d = 0; d < D; ++d) {
                        float sum = 0.0f;
                        for (i64 j = 0; j < N; ++j) sum += s[j] * c->V[j * D + d];
                        c->O[r * D + d] = sum;
                    }
                    c->L[r] = max_score + logf(sum_exp);
                }
                /* pass 1 recomputes P as the naive backward does (naive_bwd_heads) */
            }
            for (i64 j = 0; j < N; ++j) {
                float sum = 0.0f;
                for (i64 d = 0; d < D; ++d) sum += doi[d] * c->V[j * D + d];
                dP[j] = sum;
            }
            float Di = 0.0f;
            for (i64 j = 0; j < N; ++j) Di += s[j] * dP[j];
            for (i64 j = 0; j < N; ++j) dP[j] = (c->causal && j > i) ? 0.0f : s[j] * (dP[j] - Di);
            for (i64 d = 0; d < D; ++d) {
                float sum = 0.0f;
                for (i64 j = 0; j < N; ++j) sum += dP[j] * c->K[j * D + d];
                c->dQ[r * D + d] = sum * c->scale;
            }
            for (i64 j = 0; j < N; ++j)
                for (i64 d = 0; d < D; ++d) {
                    pv[j * D + d] += s[j] * doi[d];
                    pk[j * D + d] += dP[j] * qi[d];
                }
        }
    }
    free(s);
    free(dP);
}

int cpu_naive_rows_f32(const float* Q, const float* K, const float* V, const float* dO,
                       const i64* rows, i64 nrows, float* O, float* L, float* dQ, float* dK,
                       float* dV, i64 N, i64 D, float scale, int causal, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > nrows) nthreads = (int)(nrows > 0 ? nrows : 1);
    float* part = (float*)malloc(sizeof(float) * (size_t)nthreads * 2 * (size_t)(N * D));
    if (!part) return 1;
    naive_rows_ctx c = {Q, K, V, dO, rows, O, L, dQ, dK, dV, part, N, D, nrows, scale, causal,
                        nthreads};
    parallel_for(nthreads, nthreads, naive_rows_job, &c);
    for (i64 e = 0; e < N * D; ++e) {
        float k = 0.0f, v = 0.0f;
        for (int t = 0; t < nthreads; ++t) {
            k += part[(size_t)t * 2 * (size_t)(N * D) + e];
            v += part[(size_t)t * 2 * (size_t)(N * D) + N * D + e];
        }
        dK[e] = k * scale;
        dV[e] = v;
    }
    free(part);
    return 0;
}

/* Naive fp32 decode: one query row per head against Nk keys with the loops of naive_fwd_heads
 * (scores, max, exp, normalization, P V), heads over the threads. The reported CPU baseline of
 * the split-KV decode (the reference has no decode path; this is its naive attention at a
 * query length of 1). */
typedef struct {
    const float *Q, *K, *V;
    float *O, *L;
    i64 Nk, D;
    float scale;
} naive_dec_ctx;

static void naive_dec_heads(void* p, i64 begin, i64 end) {
    naive_dec_ctx* c = (naive_dec_ctx*)p;
    const i64 Nk = c->Nk, D = c->D;
    float* scores = (float*)malloc(sizeof(float) * (size_t)Nk);
    for (i64 bh = begin; bh < end; ++bh) {
        const float* q = c->Q + bh * D;
        const float* Kh = c->K + bh * Nk * D;
        const float* Vh = c->V + bh * Nk * D;
        float max_score = -INFINITY;
        for (i64 j = 0; j < Nk; ++j) {
            float dot = 0.0f;
            for (i64 d = 0; d < D; ++d) dot += q[d] * Kh[j * D + d];
            scores[j] = dot * c->scale;
            if (scores[j] > max_score) max_score = scores[j];
        }
        float sum_exp = 0.0f;
        for (i64 j = 0; j < Nk; ++j) {
            scores[j] = expf(scores[j] - max_score);
            sum_exp += scores[j];
        }
        for (i64 j = 0; j < Nk; ++j) scores[j] /= sum_exp;
        for (i64 d = 0; d < D; ++d) {
            float sum = 0.0f;
            for (i64 j = 0; j < Nk; ++j) sum += scores[j] * Vh[j * D + d];
            c->O[bh * D + d] = sum;
        }
        c->L[bh] = max_score + logf(sum_exp);
    }
    free(scores);
}

int cpu_naive_decode_f32(const float* Q, const float* K, const float* V, float* O, float* L,
                         i64 BH, i64 Nk, i64 D, float scale, int nthreads) {
    naive_dec_ctx c = {Q, K, V, O, L, Nk, D, scale};
    parallel_for(BH, nthreads, naive_dec_heads, &c);
    return 0;
}
