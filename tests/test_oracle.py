"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the parity reference.

The reference holds no stored golden vectors: its tests recompute expectations at run time
from CPU restatements (tests/unit/test_forward.cu:21-118, tests/unit/test_backward.cu:21-127)
and closed forms. The oracle is therefore pinned by
  * the committed fixtures of tests/golden/ (PyTorch float64 attention + autograd);
  * closed forms: N = 1 (O = V, L = scale q.k, reference test_stress_edge_cases.cu:52-83),
    constant inputs, identical keys (uniform P), identical values, scale = 0;
  * central finite differences of the oracle's own forward (backward pinned to forward);
  * invariants: key/value permutation (non-causal), linearity in V, causal future
    independence (reference test_causal_mask.cu:22-98), N = 1 causal == non-causal
    (test_stress_edge_cases.cu:359-404), no NaN/Inf at extreme inputs
    (test_numerical_stability.cu:21-172);
  * agreement of the materialized and row-streaming backward forms, and of split-KV partials +
    combine with the forward row;
  * mutation tests: each planted mistake (oracle.c `mutation` argument) fails one check above.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

import oracle
from conftest import REPO
from cuflash_attn import synth

GOLDEN = np.load(os.path.join(REPO, "tests", "golden", "attention_cases.npz"))
NAMES = [str(n) for n in GOLDEN["names"]]


def g(name, key):
    return GOLDEN[f"{name}/{key}"]


# ------------------------------------------------------------------------------------------
# golden fixtures (torch float64)
# ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("name", NAMES)
def test_oracle_matches_golden_forward(name):
    o, lse = oracle.forward(g(name, "q"), g(name, "k"), g(name, "v"), float(g(name, "scale")),
                            bool(g(name, "causal")))
    np.testing.assert_allclose(o, g(name, "o"), rtol=0, atol=2e-6)
    np.testing.assert_allclose(lse, g(name, "lse"), rtol=0, atol=2e-6)


@pytest.mark.parametrize("name", NAMES)
def test_oracle_matches_golden_backward(name):
    args = (g(name, "q"), g(name, "k"), g(name, "v"), g(name, "do"), float(g(name, "scale")),
            bool(g(name, "causal")))
    dq, dk, dv = oracle.backward(*args)
    for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        np.testing.assert_allclose(got, g(name, key), rtol=0, atol=5e-6)
    n = g(name, "q").shape[2]
    rows = np.arange(n)
    rq, rk, rv = oracle.backward_rows(*args, rows, rows)
    for got, key in ((rq, "dq"), (rk, "dk"), (rv, "dv")):
        np.testing.assert_allclose(got, g(name, key), rtol=0, atol=5e-6)


def test_oracle_matches_golden_decode():
    o, lse = oracle.forward(g("decode", "q"), g("decode", "k"), g("decode", "v"),
                            float(g("decode", "scale")), False)
    np.testing.assert_allclose(o, g("decode", "o"), atol=2e-6)
    np.testing.assert_allclose(lse, g("decode", "lse"), atol=2e-6)


# ------------------------------------------------------------------------------------------
# closed forms
# ------------------------------------------------------------------------------------------
def rand(seed, shape, lo=-1.0, hi=1.0):
    return synth.uniform(seed, shape, lo, hi)


def n_valid(n, causal):
    return (np.arange(n) + 1.0) if causal else np.full(n, float(n))


@pytest.mark.parametrize("d", [32, 64, 128])
def test_single_key_gives_v_and_dot(d):
    q, k, v = rand(1, (2, 3, 1, d)), rand(2, (2, 3, 1, d)), rand(3, (2, 3, 1, d))
    for causal in (False, True):
        o, lse = oracle.forward(q, k, v, d ** -0.5, causal)
        np.testing.assert_allclose(o, v, atol=1e-7)
        np.testing.assert_allclose(lse[..., 0], (q * k).sum(-1)[..., 0] * d ** -0.5, atol=1e-5)


@pytest.mark.parametrize("causal", [False, True])
def test_constant_inputs(causal):
    n, d, c = 19, 64, 0.7
    x = np.full((1, 2, n, d), c, dtype=np.float32)
    o, lse = oracle.forward(x, x, x, d ** -0.5, causal)
    np.testing.assert_allclose(o, c, atol=1e-6)
    expect = c * c * d * d ** -0.5 + np.log(n_valid(n, causal))
    np.testing.assert_allclose(lse[0, 0], expect, atol=1e-5)


@pytest.mark.parametrize("causal", [False, True])
def test_identical_keys_average_values(causal):
    n, d = 23, 32
    q, v = rand(4, (1, 1, n, d)), rand(5, (1, 1, n, d))
    k = np.broadcast_to(rand(6, (1, 1, 1, d)), (1, 1, n, d)).copy()
    o, lse = oracle.forward(q, k, v, d ** -0.5, causal)
    counts = n_valid(n, causal)
    csum = np.cumsum(v[0, 0].astype(np.float64), axis=0)
    expect = csum / counts[:, None] if causal else np.broadcast_to(csum[-1] / n, (n, d))
    np.testing.assert_allclose(o[0, 0], expect, atol=1e-6)
    s = (q[0, 0].astype(np.float64) @ k[0, 0, 0].astype(np.float64)) * d ** -0.5
    np.testing.assert_allclose(lse[0, 0], s + np.log(counts), atol=1e-5)


def test_identical_values_pass_through():
    n, d = 31, 128
    q, k = rand(7, (1, 2, n, d)), rand(8, (1, 2, n, d))
    v = np.broadcast_to(rand(9, (1, 2, 1, d)), (1, 2, n, d)).copy()
    for causal in (False, True):
        o, _ = oracle.forward(q, k, v, d ** -0.5, causal)
        np.testing.assert_allclose(o, v, atol=1e-6)


def test_zero_scale_is_uniform_attention():
    n, d = 12, 64
    q, k, v = rand(10, (1, 1, n, d)), rand(11, (1, 1, n, d)), rand(12, (1, 1, n, d))
    o, lse = oracle.forward(q, k, v, 0.0, True)
    csum = np.cumsum(v[0, 0].astype(np.float64), axis=0)
    np.testing.assert_allclose(o[0, 0], csum / n_valid(n, True)[:, None], atol=1e-6)
    np.testing.assert_allclose(lse[0, 0], np.log(n_valid(n, True)), atol=1e-6)


# ------------------------------------------------------------------------------------------
# backward pinned to the forward by finite differences
# ------------------------------------------------------------------------------------------
def loss(q, k, v, do, scale, causal):
    o, _ = oracle.forward(q, k, v, scale, causal)
    return float(np.sum(o.astype(np.float64) * do))


@pytest.mark.parametrize("causal", [False, True])
def test_backward_matches_finite_differences(causal):
    shape = (1, 1, 6, 32)
    q, k, v, do = (rand(20 + i, shape) for i in range(4))
    scale = 32 ** -0.5
    dq, dk, dv = oracle.backward(q, k, v, do, scale, causal)
    rng = np.random.default_rng(0)
    h = 2e-3
    for grad, idx in ((dq, 0), (dk, 1), (dv, 2)):
        for _ in range(12):
            pos = tuple(int(rng.integers(0, s)) for s in shape)
            xs = [q.copy(), k.copy(), v.copy()]
            xs[idx][pos] += h
            up = loss(*xs, do, scale, causal)
            xs[idx][pos] -= 2 * h
            dn = loss(*xs, do, scale, causal)
            fd = (up - dn) / (2 * h)
            assert abs(fd - grad[pos]) < 2e-3, (idx, pos, fd, grad[pos])


# ------------------------------------------------------------------------------------------
# invariants
# ------------------------------------------------------------------------------------------
def test_key_value_permutation_invariance():
    n, d = 40, 64
    q, k, v = rand(30, (1, 2, n, d)), rand(31, (1, 2, n, d)), rand(32, (1, 2, n, d))
    perm = np.random.default_rng(1).permutation(n)
    o1, l1 = oracle.forward(q, k, v, d ** -0.5, False)
    o2, l2 = oracle.forward(q, k[:, :, perm], v[:, :, perm], d ** -0.5, False)
    np.testing.assert_allclose(o1, o2, atol=1e-6)
    np.testing.assert_allclose(l1, l2, atol=1e-6)


def test_linear_in_values():
    n, d = 25, 32
    q, k = rand(33, (1, 1, n, d)), rand(34, (1, 1, n, d))
    v1, v2 = rand(35, (1, 1, n, d)), rand(36, (1, 1, n, d))
    a, b = 0.75, -1.25
    o1, _ = oracle.forward(q, k, v1, d ** -0.5, True)
    o2, _ = oracle.forward(q, k, v2, d ** -0.5, True)
    o3, _ = oracle.forward(q, k, (a * v1 + b * v2).astype(np.float32), d ** -0.5, True)
    np.testing.assert_allclose(o3, a * o1 + b * o2, atol=2e-6)


def test_causal_future_independence():
    # reference tests/unit/test_causal_mask.cu:22-98: rows < N/2 ignore K, V rows >= N/2
    n, d = 16, 32
    q, k, v = rand(37, (1, 1, n, d)), rand(38, (1, 1, n, d)), rand(39, (1, 1, n, d))
    k2, v2 = k.copy(), v.copy()
    k2[:, :, n // 2:] *= 10.0
    v2[:, :, n // 2:] *= 10.0
    o1, l1 = oracle.forward(q, k, v, d ** -0.5, True)
    o2, l2 = oracle.forward(q, k2, v2, d ** -0.5, True)
    np.testing.assert_allclose(o1[:, :, : n // 2], o2[:, :, : n // 2], atol=1e-5)
    np.testing.assert_allclose(l1[:, :, : n // 2], l2[:, :, : n // 2], atol=1e-5)
    assert np.abs(o1[:, :, n // 2:] - o2[:, :, n // 2:]).max() > 1e-2


def test_single_row_causal_equals_noncausal():
    q, k, v = rand(40, (2, 2, 1, 64)), rand(41, (2, 2, 1, 64)), rand(42, (2, 2, 1, 64))
    a = oracle.forward(q, k, v, 0.125, True)
    b = oracle.forward(q, k, v, 0.125, False)
    np.testing.assert_allclose(a[0], b[0], atol=1e-7)
    np.testing.assert_allclose(a[1], b[1], atol=1e-7)


@pytest.mark.parametrize("value", [100.0, 1e-6])
def test_extreme_constants_stay_finite(value):
    # reference tests/unit/test_numerical_stability.cu:21-100
    x = np.full((1, 1, 16, 32), value, dtype=np.float32)
    o, lse = oracle.forward(x, x, x, 32 ** -0.5, False)
    assert np.isfinite(o).all() and np.isfinite(lse).all()
    np.testing.assert_allclose(o, value, rtol=1e-6)
    dq, dk, dv = oracle.backward(x, x, x, x, 32 ** -0.5, False)
    assert all(np.isfinite(t).all() for t in (dq, dk, dv))


def test_mixed_extremes_stay_finite():
    # reference tests/unit/test_numerical_stability.cu:127-172
    x = np.where(rand(43, (1, 1, 16, 32)) > 0, 50.0, -0.001).astype(np.float32)
    o, lse = oracle.forward(x, x, x, 32 ** -0.5, True)
    assert np.isfinite(o).all() and np.isfinite(lse).all()


# ------------------------------------------------------------------------------------------
# internal consistency
# ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("causal", [False, True])
def test_streaming_backward_matches_materialized(causal):
    shape = (2, 2, 45, 64)
    q, k, v, do = (synth.normal(50 + i, shape) for i in range(4))
    dq, dk, dv = oracle.backward(q, k, v, do, 0.125, causal)
    rows = np.array([0, 1, 17, 44])
    rq, rk, rv = oracle.backward_rows(q, k, v, do, 0.125, causal, rows, rows[::-1].copy())
    np.testing.assert_allclose(rq, dq[:, :, rows], atol=2e-6)
    np.testing.assert_allclose(rk, dk[:, :, rows[::-1]], atol=2e-6)
    np.testing.assert_allclose(rv, dv[:, :, rows[::-1]], atol=2e-6)


@pytest.mark.parametrize("nq,nk,causal", [(20, 53, True), (20, 53, False), (53, 20, False),
                                          (1, 9, True)])
def test_streaming_backward_matches_materialized_separate_lengths(nq, nk, causal):
    """The row-streaming form with Nq != Nk (causal mask aligned to the end of the keys) equals
    the materialized backward, which test_separate_lengths_match_torch_float64 pins."""
    d = 32
    q, do = synth.normal(70, (1, 3, nq, d)), synth.normal(71, (1, 3, nq, d))
    k, v = synth.normal(72, (1, 3, nk, d)), synth.normal(73, (1, 3, nk, d))
    dq, dk, dv = oracle.backward(q, k, v, do, 0.2, causal)
    qrows = np.arange(nq)
    krows = np.arange(nk)[::-1].copy()
    rq, rk, rv = oracle.backward_rows(q, k, v, do, 0.2, causal, qrows, krows)
    np.testing.assert_allclose(rq, dq, atol=2e-6)
    np.testing.assert_allclose(rk, dk[:, :, krows], atol=2e-6)
    np.testing.assert_allclose(rv, dv[:, :, krows], atol=2e-6)
    if causal and nq < nk:
        # a planted top-left mask changes the gradients
        mq, mk, _ = oracle.backward_rows(q, k, v, do, 0.2, causal, qrows, krows, mutation=7)
        assert max(np.abs(mq - dq).max(), np.abs(mk - dk[:, :, krows]).max()) > 1e-3


@pytest.mark.parametrize("nsplit", [1, 3, 8, 64])
def test_split_partials_combine_to_forward_row(nsplit):
    kv_len, d = 200, 64
    q = synth.normal(60, (2, 2, 1, d))
    k, v = synth.normal(61, (2, 2, kv_len, d)), synth.normal(62, (2, 2, kv_len, d))
    chunk = -(-kv_len // nsplit)
    m, l, acc = oracle.decode_partials(q, k, v, d ** -0.5, nsplit, chunk)
    o, lse = oracle.decode_combine(m, l, acc, (2, 2))
    o_ref, l_ref = oracle.forward(q, k, v, d ** -0.5, False)
    np.testing.assert_allclose(o, o_ref, atol=2e-6)
    np.testing.assert_allclose(lse, l_ref, atol=2e-6)


def test_decode_equals_last_row_of_causal_forward():
    n, d = 37, 128
    q, k, v = synth.normal(63, (1, 2, n, d)), synth.normal(64, (1, 2, n, d)), \
        synth.normal(65, (1, 2, n, d))
    o_full, l_full = oracle.forward(q, k, v, d ** -0.5, True)
    o_dec, l_dec = oracle.forward(q[:, :, -1:], k, v, d ** -0.5, True)
    np.testing.assert_allclose(o_dec[:, :, 0], o_full[:, :, -1], atol=1e-6)
    np.testing.assert_allclose(l_dec[:, :, 0], l_full[:, :, -1], atol=1e-6)


def test_naive_fp32_baseline_agrees():
    shape = (1, 3, 64, 64)
    q, k, v, do = (synth.normal(70 + i, shape) for i in range(4))
    o, lse = oracle.naive_forward_f32(q, k, v, 0.125, True)
    o_ref, l_ref = oracle.forward(q, k, v, 0.125, True)
    np.testing.assert_allclose(o, o_ref, atol=1e-5)
    np.testing.assert_allclose(lse, l_ref, atol=1e-5)
    grads = oracle.naive_backward_f32(q, k, v, do, 0.125, True)
    refs = oracle.backward(q, k, v, do, 0.125, True)
    for a, b in zip(grads, refs):
        np.testing.assert_allclose(a, b, atol=1e-4)


@pytest.mark.parametrize("causal", [True, False])
def test_naive_rows_is_the_naive_baseline_by_rows(causal):
    """The CPU baseline's row-sampled form: with every query row selected it reproduces the
    naive forward and backward (O, L, dQ bitwise: the same float loops per row; dK, dV up to
    the order of their sums over rows, on 1 and 3 threads); a subset of rows gives exactly
    those rows of O, L and dQ, and dK / dV equal to the selected rows' terms alone (checked
    against the fp64 oracle with dO zeroed on the other rows)."""
    N, D = 150, 64
    q, k, v, do = (synth.normal(90 + i, (1, 1, N, D)) for i in range(4))
    o, lse = oracle.naive_forward_f32(q, k, v, 0.125, causal)
    dq, dk, dv = oracle.naive_backward_f32(q, k, v, do, 0.125, causal)
    for nthreads in (1, 3):
        ro, rl, rdq, rdk, rdv = oracle.naive_rows_f32(q[0, 0], k[0, 0], v[0, 0], do[0, 0], 0.125,
                                                      causal, np.arange(N), nthreads=nthreads)
        np.testing.assert_array_equal(ro, o[0, 0])
        np.testing.assert_array_equal(rl, lse[0, 0])
        np.testing.assert_array_equal(rdq, dq[0, 0])
        np.testing.assert_allclose(rdk, dk[0, 0], atol=2e-6)
        np.testing.assert_allclose(rdv, dv[0, 0], atol=2e-6)
    sub = np.arange(3, N, 17)
    so, sl, sdq, sdk, sdv = oracle.naive_rows_f32(q[0, 0], k[0, 0], v[0, 0], do[0, 0], 0.125,
                                                  causal, sub, nthreads=2)
    np.testing.assert_array_equal(so, o[0, 0][sub])
    np.testing.assert_array_equal(sl, lse[0, 0][sub])
    np.testing.assert_array_equal(sdq, dq[0, 0][sub])
    # dV_j = sum_i P_ij dO_i: with dO zero off the selected rows only their terms remain.
    do_sub = np.zeros_like(do)
    do_sub[0, 0, sub] = do[0, 0, sub]
    _, _, dv_ref = oracle.backward(q, k, v, do_sub, 0.125, causal)
    np.testing.assert_allclose(sdv, dv_ref[0, 0], atol=2e-5)
    assert np.abs(sdk).max() > 0


def test_naive_decode_baseline_agrees():
    """The decode CPU baseline equals the oracle's forward at a query length of 1."""
    BH, Nk, D = 5, 700, 64
    q = synth.normal(95, (BH, D))
    k, v = synth.normal(96, (BH, Nk, D)), synth.normal(97, (BH, Nk, D))
    o, lse = oracle.naive_decode_f32(q, k, v, 0.125, nthreads=2)
    o_ref, l_ref = oracle.forward(q[:, None, None, :], k[:, None], v[:, None], 0.125, False)
    np.testing.assert_allclose(o, o_ref.reshape(BH, D), atol=2e-6)
    np.testing.assert_allclose(lse, l_ref.reshape(BH), atol=2e-6)


# ------------------------------------------------------------------------------------------
# separate query / key lengths (Q [B,H,Nq,D], K/V [B,H,Nk,D]; causal: j <= i + Nk - Nq)
# ------------------------------------------------------------------------------------------
def torch_attention_f64(q, k, v, do, scale, causal):
    """O, L, dQ, dK, dV of softmax(scale Q K^T + mask) V in float64 on the CPU (torch autograd),
    the mask written out as an explicit bottom-right aligned causal mask."""
    import torch

    tq, tk, tv = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    s = torch.matmul(tq, tk.transpose(-1, -2)) * scale
    if causal:
        nq, nk = q.shape[2], k.shape[2]
        i = torch.arange(nq)[:, None]
        j = torch.arange(nk)[None, :]
        s = s.masked_fill(j > i + (nk - nq), float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    o = torch.matmul(torch.softmax(s, dim=-1), tv)
    o.backward(torch.tensor(do, dtype=torch.float64))
    return [t.detach().numpy() for t in (o, lse, tq.grad, tk.grad, tv.grad)]


SEPARATE_LENGTHS = [(5, 37, True), (5, 37, False), (33, 100, True), (64, 71, True),
                    (40, 17, False), (1, 9, True)]


@pytest.mark.parametrize("nq,nk,causal", SEPARATE_LENGTHS)
def test_separate_lengths_match_torch_float64(nq, nk, causal):
    d = 32
    q, do = rand(70, (2, 2, nq, d)), rand(71, (2, 2, nq, d))
    k, v = rand(72, (2, 2, nk, d)), rand(73, (2, 2, nk, d))
    scale = d ** -0.5
    o_ref, l_ref, dq_ref, dk_ref, dv_ref = torch_attention_f64(q, k, v, do, scale, causal)
    o, lse = oracle.forward(q, k, v, scale, causal)
    np.testing.assert_allclose(o, o_ref, atol=2e-6)
    np.testing.assert_allclose(lse, l_ref, atol=2e-6)
    dq, dk, dv = oracle.backward(q, k, v, do, scale, causal)
    for got, ref in ((dq, dq_ref), (dk, dk_ref), (dv, dv_ref)):
        np.testing.assert_allclose(got, ref, atol=5e-6)


def suffix_identity_fails(mutation=0) -> bool:
    """Queries that are the last nq rows of an n-row sequence, attending causally to all n keys,
    give the last nq rows of the full causal attention; with dO = 0 on the first n - nq rows the
    full problem's dK, dV and last dQ rows are the gradients of the short one."""
    n, nq, d = 50, 13, 32
    q, k, v, do = (rand(80 + i, (1, 2, n, d)) for i in range(4))
    do[:, :, : n - nq] = 0.0
    scale = d ** -0.5
    o_full, l_full = oracle.forward(q, k, v, scale, True)
    o, lse = oracle.forward(q[:, :, n - nq:], k, v, scale, True, mutation=mutation)
    if not (np.allclose(o, o_full[:, :, n - nq:], atol=1e-6)
            and np.allclose(lse, l_full[:, :, n - nq:], atol=1e-6)):
        return True
    dq_full, dk_full, dv_full = oracle.backward(q, k, v, do, scale, True)
    dq, dk, dv = oracle.backward(q[:, :, n - nq:], k, v, do[:, :, n - nq:], scale, True,
                                 mutation=mutation)
    return not (np.allclose(dq, dq_full[:, :, n - nq:], atol=1e-6)
                and np.allclose(dk, dk_full, atol=1e-6) and np.allclose(dv, dv_full, atol=1e-6))


def test_suffix_queries_equal_rows_of_full_causal_attention():
    assert not suffix_identity_fails()


def test_separate_length_checks_catch_top_left_mask():
    assert suffix_identity_fails(7)
    assert not golden_fails(7)  # square heads cannot tell the two alignments apart


# ------------------------------------------------------------------------------------------
# mutation tests: every planted mistake is caught by at least one of the checks above
# ------------------------------------------------------------------------------------------
def golden_fails(mutation) -> bool:
    for name in NAMES:
        args = (g(name, "q"), g(name, "k"), g(name, "v"))
        scale, causal = float(g(name, "scale")), bool(g(name, "causal"))
        o, lse = oracle.forward(*args, scale, causal, mutation=mutation)
        if not (np.allclose(o, g(name, "o"), atol=2e-6) and np.allclose(lse, g(name, "lse"),
                                                                          atol=2e-6)):
            return True
        grads = oracle.backward(*args, g(name, "do"), scale, causal, mutation=mutation)
        for got, key in zip(grads, ("dq", "dk", "dv")):
            if not np.allclose(got, g(name, key), atol=5e-6):
                return True
    return False


def stability_fails(mutation) -> bool:
    x = np.full((1, 1, 16, 32), 100.0, dtype=np.float32)
    o, lse = oracle.forward(x, x, x, 32 ** -0.5, False, mutation=mutation)
    return not (np.isfinite(o).all() and np.isfinite(lse).all())


@pytest.mark.parametrize("mutation", [1, 2, 3, 4, 6])
def test_golden_checks_catch_planted_mistakes(mutation):
    assert golden_fails(mutation)


def test_stability_check_catches_missing_max_shift():
    # mutation 5 is exact in real arithmetic; only the extreme-value check exposes it
    assert not golden_fails(0)
    assert stability_fails(5)
    assert not stability_fails(0)
