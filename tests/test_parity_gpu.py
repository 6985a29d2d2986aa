"""GPU parity: the HIP kernels, called through the C ABI, against the fp64 CPU oracle.

Tolerances (north star): FP32 O and L within 1e-4 relative (max |diff| / max |ref|);
FP16/BF16 O, L, dQ, dK, dV within 2e-2 max-abs. The oracle runs on the same rounded inputs.
FP32 gradients are held to 1e-4 relative as well (the reference's own fp32 backward test uses
1e-3 absolute, tests/unit/test_backward.cu:202-204).
"""

from __future__ import annotations

import numpy as np
import pytest

import cuflash_attn
import oracle
from conftest import max_abs
from cuflash_attn import synth

DTYPES = ["float32", "float16", "bfloat16"]
TOL_16 = 2e-2
TOL_32 = 1e-4


def make_inputs(shape, dtype, seeds=(1, 2, 3, 4), dist="uniform", std=1.0):
    out = []
    for s in seeds:
        x = synth.uniform(s, shape) if dist == "uniform" else synth.normal(s, shape, std)
        out.append(synth.round_to(x, dtype))
    return out


def check(dtype, got, ref, what):
    if dtype == "float32":
        # Relative to the tensor's magnitude, floored at 1e-3: an exactly-zero reference (dQ at
        # N = 1, where dS = P (dP - D) = 0) leaves only fp32 rounding of dP - D (~1e-8).
        err = max_abs(got, ref) / max(float(np.max(np.abs(ref))) if np.size(ref) else 0.0, 1e-3)
        assert err <= TOL_32, f"{what}: rel err {err:.3e}"
    else:
        err = max_abs(got, ref)
        assert err <= TOL_16, f"{what}: max abs err {err:.3e}"
    return err


def run_forward(dtype, q, k, v, scale, causal):
    tq, tk, tv = (synth.to_torch(x, dtype) for x in (q, k, v))
    o, lse = cuflash_attn.flash_attention_forward(tq, tk, tv, scale=scale, causal=causal)
    return o, lse, (tq, tk, tv)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n", [1, 17, 128, 200])
def test_forward_parity(torch_gpu, dtype, d, causal, n):
    shape = (2, 3, n, d)
    q, k, v = make_inputs(shape, dtype, seeds=(1, 2, 3))
    scale = d ** -0.5
    o, lse, _ = run_forward(dtype, q, k, v, scale, causal)
    torch_gpu.cuda.synchronize()
    o_ref, l_ref = oracle.forward(q, k, v, scale, causal)
    check(dtype, synth.to_numpy(o), o_ref, "O")
    check(dtype, synth.to_numpy(lse), l_ref, "L")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n", [1, 33, 130, 300])
def test_backward_parity(torch_gpu, dtype, d, causal, n):
    shape = (1, 2, n, d)
    q, k, v, do = make_inputs(shape, dtype)
    scale = d ** -0.5
    o, lse, (tq, tk, tv) = run_forward(dtype, q, k, v, scale, causal)
    tdo = synth.to_torch(do, dtype)
    dq, dk, dv = cuflash_attn.flash_attention_backward(tq, tk, tv, o, lse, tdo, scale=scale,
                                                       causal=causal)
    torch_gpu.cuda.synchronize()
    rq, rk, rv = oracle.backward(q, k, v, do, scale, causal)
    check(dtype, synth.to_numpy(dq), rq, "dQ")
    check(dtype, synth.to_numpy(dk), rk, "dK")
    check(dtype, synth.to_numpy(dv), rv, "dV")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("kv_len", [1, 100, 1000, 4099])
@pytest.mark.parametrize("splits", [0, 1, 3, 16])
def test_decode_parity(torch_gpu, dtype, d, kv_len, splits):
    B, H = 2, 3
    q = synth.round_to(synth.normal(1, (B, H, 1, d)), dtype)
    k = synth.round_to(synth.normal(2, (B, H, kv_len, d)), dtype)
    v = synth.round_to(synth.normal(3, (B, H, kv_len, d)), dtype)
    scale = d ** -0.5
    tq, tk, tv = (synth.to_torch(x, dtype) for x in (q, k, v))
    o, lse = cuflash_attn.flash_attention_decode(tq, tk, tv, scale=scale, num_splits=splits)
    torch_gpu.cuda.synchronize()
    o_ref, l_ref = oracle.forward(q, k, v, scale, False)
    check(dtype, synth.to_numpy(o), o_ref, "O")
    check(dtype, synth.to_numpy(lse), l_ref, "L")


@pytest.mark.gpu
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("splits,kv_heads", [(1024, 2), (1000, 2), (5000, 2), (700, 1)])
def test_decode_many_splits(torch_gpu, d, splits, kv_heads):
    """The combine at 1024 splits per head (the bound of its LDS weight array; larger requests
    are clamped to it), with a remainder past its 64-split steps (1000), and the matrix-core
    grouped-query decode when a request asks for chunks shorter than its 32-key blocks (700
    splits of 16384 keys with 2 query heads per key/value head: 512 splits of 32 keys)."""
    B, H, kv_len = 1, 2, 16384
    q = synth.round_to(synth.normal(4, (B, H, 1, d)), "float16")
    k = synth.round_to(synth.normal(5, (B, kv_heads, kv_len, d)), "float16")
    v = synth.round_to(synth.normal(6, (B, kv_heads, kv_len, d)), "float16")
    tq, tk, tv = (synth.to_torch(x, "float16") for x in (q, k, v))
    o, lse = cuflash_attn.flash_attention_decode(tq, tk, tv, num_splits=splits)
    torch_gpu.cuda.synchronize()
    group = H // kv_heads
    o_ref, l_ref = oracle.forward(q, np.repeat(k, group, axis=1), np.repeat(v, group, axis=1),
                                  d ** -0.5, False)
    check("float16", synth.to_numpy(o), o_ref, "O")
    check("float16", synth.to_numpy(lse), l_ref, "L")


@pytest.mark.gpu
@pytest.mark.parametrize("d", [32, 64])
@pytest.mark.parametrize("causal", [False, True])
def test_forward_fp32_both_grids(torch_gpu, d, causal):
    """fp32 at head_dim 32/64 runs fwd32_split_kernel (key blocks split over the waves of a
    32-row workgroup) when fewer than two 128-row workgroups per CU would run, else
    fwd32_kernel. B*H = 128 heads of N = 520 give 640 of them (fwd32_kernel); 4 heads give 20
    (split kernel). Two heads of each launch are checked against the oracle."""
    for B, H in ((4, 32), (1, 4)):
        n = 520
        q, k, v = make_inputs((B, H, n, d), "float32", seeds=(5, 6, 7))
        scale = d ** -0.5
        o, lse, _ = run_forward("float32", q, k, v, scale, causal)
        torch_gpu.cuda.synchronize()
        o = synth.to_numpy(o)
        lse = synth.to_numpy(lse)
        for b, h in ((0, 0), (B - 1, H - 1)):
            o_ref, l_ref = oracle.forward(q[b:b + 1, h:h + 1], k[b:b + 1, h:h + 1],
                                          v[b:b + 1, h:h + 1], scale, causal)
            check("float32", o[b:b + 1, h:h + 1], o_ref, f"O B={B} H={H} head {(b, h)}")
            check("float32", lse[b:b + 1, h:h + 1], l_ref, f"L B={B} H={H} head {(b, h)}")


@pytest.mark.gpu
@pytest.mark.parametrize("causal", [False, True])
def test_backward_fp32_both_launches(torch_gpu, causal):
    """The fp32 backward runs dq and dkdv items in one launch (dq_dkdv_kernel) when both grids
    fit in one round of workgroups, else dq_kernel then dkdv_kernel. B*H = 128 heads of N = 520
    give 1,280 query and key blocks (two launches); 4 heads give 40 (one launch). Two heads of
    each are checked against the oracle."""
    d = 64
    for B, H in ((4, 32), (1, 4)):
        n = 520
        q, k, v, do = make_inputs((B, H, n, d), "float32", seeds=(5, 6, 7, 8))
        scale = d ** -0.5
        o, lse, (tq, tk, tv) = run_forward("float32", q, k, v, scale, causal)
        dq, dk, dv = cuflash_attn.flash_attention_backward(tq, tk, tv, o, lse,
                                                           synth.to_torch(do, "float32"),
                                                           scale=scale, causal=causal)
        torch_gpu.cuda.synchronize()
        got = [synth.to_numpy(x) for x in (dq, dk, dv)]
        for b, h in ((0, 0), (B - 1, H - 1)):
            sl = (slice(b, b + 1), slice(h, h + 1))
            ref = oracle.backward(q[sl], k[sl], v[sl], do[sl], scale, causal)
            for name, g, r in zip(("dQ", "dK", "dV"), got, ref):
                check("float32", g[sl], r, f"{name} B={B} H={H} head {(b, h)}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_forward_d64_both_workgroup_sizes(torch_gpu, dtype):
    """head_dim 64 runs four-wave workgroups (128 rows) for non-causal launches and launches
    with fewer eight-wave workgroups than CUs, eight-wave workgroups (256 rows) otherwise.
    Causal B*H = 64 heads of N = 2100 take the eight-wave kernel (576 workgroups), non-causal
    the four-wave one; two heads of each are checked against the oracle."""
    d, n = 64, 2100
    q, k, v = make_inputs((2, 32, n, d), dtype, seeds=(11, 12, 13), dist="normal")
    scale = d ** -0.5
    for causal in (True, False):
        o, lse, _ = run_forward(dtype, q, k, v, scale, causal)
        torch_gpu.cuda.synchronize()
        o = synth.to_numpy(o)
        lse = synth.to_numpy(lse)
        for b, h in ((0, 0), (1, 31)):
            sl = (slice(b, b + 1), slice(h, h + 1))
            o_ref, l_ref = oracle.forward(q[sl], k[sl], v[sl], scale, causal)
            check(dtype, o[sl], o_ref, f"O causal={causal} head {(b, h)}")
            check(dtype, lse[sl], l_ref, f"L causal={causal} head {(b, h)}")
