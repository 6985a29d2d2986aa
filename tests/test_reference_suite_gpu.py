"""The reference's GPU test suite, re-expressed against this library's C ABI.

Each test names the reference test it follows. Expected values come from the committed golden
fixtures (PyTorch float64) or the fp64 oracle, with the reference's tolerances; the reference's
own PyTorch comparison (tests/integration/test_pytorch_comparison.py:421-731) is reproduced with
PyTorch's float32 attention on the CPU as the comparison point.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

import cuflash_attn
import oracle
from conftest import REPO, max_abs
from cuflash_attn import synth

GOLDEN = np.load(os.path.join(REPO, "tests", "golden", "attention_cases.npz"))
NAMES = [str(n) for n in GOLDEN["names"]]

# Reference tolerances: test_forward.cu:169/:220/:274, test_backward.cu:202/:273,
# test_dtype.cu:102/:419/:524/:730.
def golden_tol(name, dtype, grad):
    if dtype == "float16":
        return 2e-2 if grad else 1e-2
    if dtype == "bfloat16":
        return 2e-2
    return 2e-3 if "d128" in name else 1e-3


def run(dtype, q, k, v, scale, causal, do=None):
    tq, tk, tv = (synth.to_torch(x, dtype) for x in (q, k, v))
    o, lse = cuflash_attn.flash_attention_forward(tq, tk, tv, scale=scale, causal=causal)
    grads = None
    if do is not None:
        grads = cuflash_attn.flash_attention_backward(tq, tk, tv, o, lse, synth.to_torch(do, dtype),
                                                      scale=scale, causal=causal)
    import torch

    torch.cuda.synchronize()
    out = [synth.to_numpy(o), synth.to_numpy(lse)]
    if grads is not None:
        out += [synth.to_numpy(t) for t in grads]
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_golden_cases(torch_gpu, name):
    """ForwardTest.*, BackwardTest.*, DTypeTest.* shapes (test_forward.cu:121-333,
    test_backward.cu:138-286, test_dtype.cu:24-750) against PyTorch float64."""
    dtype = str(GOLDEN[f"{name}/dtype"])
    get = lambda key: GOLDEN[f"{name}/{key}"]  # noqa: E731
    o, lse, dq, dk, dv = run(dtype, get("q"), get("k"), get("v"), float(get("scale")),
                             bool(get("causal")), get("do"))
    assert max_abs(o, get("o")) <= golden_tol(name, dtype, False)
    assert max_abs(lse, get("lse")) <= golden_tol(name, dtype, False)
    for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        assert max_abs(got, get(key)) <= golden_tol(name, dtype, True), key


@pytest.mark.gpu
def test_golden_decode(torch_gpu):
    get = lambda key: GOLDEN[f"decode/{key}"]  # noqa: E731
    tq, tk, tv = (synth.to_torch(get(x), "float16") for x in ("q", "k", "v"))
    for splits in (0, 1, 2, 7, 50):
        o, lse = cuflash_attn.flash_attention_decode(tq, tk, tv, scale=float(get("scale")),
                                                     num_splits=splits)
        torch_gpu.cuda.synchronize()
        assert max_abs(synth.to_numpy(o), get("o")) <= 1e-2
        assert max_abs(synth.to_numpy(lse), get("lse")) <= 1e-2


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_causal_future_independence(torch_gpu, dtype):
    """CausalMaskTest.FutureIndependence (test_causal_mask.cu:22-98)."""
    n, d = 16, 32
    q, k, v = (synth.round_to(synth.uniform(42 + i, (1, 1, n, d)), dtype) for i in range(3))
    k2, v2 = k.copy(), v.copy()
    k2[:, :, n // 2:] = synth.round_to(k2[:, :, n // 2:] * 10, dtype)
    v2[:, :, n // 2:] = synth.round_to(v2[:, :, n // 2:] * 10, dtype)
    o1, l1 = run(dtype, q, k, v, d ** -0.5, True)
    o2, l2 = run(dtype, q, k2, v2, d ** -0.5, True)
    assert max_abs(o1[:, :, : n // 2], o2[:, :, : n // 2]) <= 1e-5
    assert max_abs(l1[:, :, : n // 2], l2[:, :, : n // 2]) <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,tol", [("float16", 1e-2), ("bfloat16", 2e-2)])
@pytest.mark.parametrize("d", [32, 128])
def test_reduced_precision_matches_fp32(torch_gpu, dtype, tol, d):
    """DTypeTest.{FP16,BF16}{Forward,Backward}MatchesFP32 and HeadDim128 (test_dtype.cu)."""
    n = 16
    xs = [synth.round_to(synth.uniform(42 + i, (1, 1, n, d)), dtype) for i in range(4)]
    low = run(dtype, *xs[:3], d ** -0.5, False, xs[3])
    full = run("float32", *xs[:3], d ** -0.5, False, xs[3])
    for a, b in zip(low, full):
        assert max_abs(a, b) <= 2 * tol


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("kind", ["large", "small", "mixed"])
def test_numerical_stability(torch_gpu, dtype, kind):
    """NumericalStabilityTest.{LargeValues,SmallValues,MixedExtremeValues}
    (test_numerical_stability.cu:21-172): no NaN / Inf."""
    shape = (1, 1, 16, 32)
    if kind == "large":
        x = np.full(shape, 100.0, dtype=np.float32)
    elif kind == "small":
        x = np.full(shape, 1e-6, dtype=np.float32)
    else:
        x = np.where(synth.uniform(7, shape) > 0, 50.0, 0.001).astype(np.float32)
    x = synth.round_to(x, dtype)
    outs = run(dtype, x, x, x, 32 ** -0.5, kind == "mixed", x)
    for t in outs:
        assert np.isfinite(t).all()
    if kind != "mixed":
        assert max_abs(outs[0], x) <= 1e-2 * max(1.0, float(x.max()))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_single_token_causal_equals_noncausal(torch_gpu, dtype):
    """EdgeCaseTest.MinimumValidDimensions / N = 1 causal == non-causal
    (test_stress_edge_cases.cu:52-83, :359-404)."""
    xs = [synth.round_to(synth.uniform(i, (2, 3, 1, 64)), dtype) for i in (1, 2, 3, 4)]
    a = run(dtype, *xs[:3], 0.125, True, xs[3])
    b = run(dtype, *xs[:3], 0.125, False, xs[3])
    for x, y in zip(a, b):
        assert max_abs(x, y) <= 1e-5
    assert max_abs(a[0], xs[2]) <= 1e-2


@pytest.mark.gpu
def test_minimum_head_dim_causal(torch_gpu):
    """EdgeCaseTest.MinimumHeadDim (test_stress_edge_cases.cu:85-118): K = V = Q."""
    x = synth.uniform(42, (2, 4, 64, 32))
    o, lse = run("float32", x, x, x, 32 ** -0.5, True)
    o_ref, l_ref = oracle.forward(x, x, x, 32 ** -0.5, True)
    assert max_abs(o, o_ref) <= 1e-4 and max_abs(lse, l_ref) <= 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("shape,causal,bwd", [((1, 8, 8192, 128), True, False),
                                              ((1, 8, 4096, 64), True, True),
                                              ((1, 32, 512, 64), False, True)])
def test_stress_shapes(torch_gpu, shape, causal, bwd):
    """StressTest.{LargeSequenceForward,LargeSequenceBackward,MultiHeadLarge}
    (test_stress_edge_cases.cu:181-258, :320-353), fp32 as in the reference, checked on one
    head against the oracle (the reference only checks SUCCESS)."""
    d = shape[3]
    xs = [synth.uniform(123 + i, shape) for i in range(4 if bwd else 3)]
    outs = run("float32", *xs[:3], d ** -0.5, causal, xs[3] if bwd else None)
    for t in outs:
        assert np.isfinite(t).all()
    sl = (slice(0, 1), slice(shape[1] - 1, shape[1]))
    o_ref, l_ref = oracle.forward(*(x[sl] for x in xs[:3]), d ** -0.5, causal)
    assert max_abs(outs[0][sl], o_ref) <= 1e-4 * max(1.0, float(np.abs(o_ref).max()))
    if bwd:
        rows = np.arange(0, shape[2], 97)
        rq, rk, rv = oracle.backward_rows(*(x[sl] for x in xs), d ** -0.5, causal, rows, rows)
        for got, ref in ((outs[2], rq), (outs[3], rk), (outs[4], rv)):
            assert max_abs(got[sl][:, :, rows], ref) <= 1e-4 * max(1.0, float(np.abs(ref).max()))


@pytest.mark.gpu
def test_repeated_execution_no_leak(torch_gpu):
    """StressTest.RepeatedExecutionNoLeak (test_stress_edge_cases.cu:264-314)."""
    torch = torch_gpu
    shape = (2, 4, 256, 64)
    q, k, v, do = (torch.randn(shape, device="cuda") for _ in range(4))
    o, lse = cuflash_attn.flash_attention_forward(q, k, v, causal=True)
    cuflash_attn.flash_attention_backward(q, k, v, o, lse, do, causal=True)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for _ in range(100):
        o, lse = cuflash_attn.flash_attention_forward(q, k, v, causal=True)
        cuflash_attn.flash_attention_backward(q, k, v, o, lse, do, causal=True)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free0 - free1 < (1 << 20)


# ---- tests/integration/test_pytorch_comparison.py:421-731 (torch float32 on the CPU) ----
def sdpa_cpu(q, k, v, causal, grad_out=None):
    import torch
    import torch.nn.functional as F

    qc, kc, vc = (t.detach().float().cpu().requires_grad_(grad_out is not None) for t in (q, k, v))
    out = F.scaled_dot_product_attention(qc, kc, vc, scale=float(q.shape[-1] ** -0.5),
                                         is_causal=causal)
    if grad_out is None:
        return out.detach()
    out.backward(grad_out.detach().float().cpu())
    return out.detach(), qc.grad, kc.grad, vc.grad


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,tol_f,tol_b", [("float32", 1e-3, 1e-3), ("float16", 1e-2, 2e-2),
                                               ("bfloat16", 2e-2, 2e-2)])
@pytest.mark.parametrize("causal", [False, True])
def test_pytorch_comparison(torch_gpu, dtype, tol_f, tol_b, causal):
    torch = torch_gpu
    tdt = getattr(torch, dtype)
    torch.manual_seed(42)
    q, k, v, do = (torch.randn(1, 2, 32, 32, dtype=torch.float32).to(tdt).cuda()
                   for _ in range(4))
    o, lse = cuflash_attn.flash_attention_forward(q, k, v, causal=causal)
    dq, dk, dv = cuflash_attn.flash_attention_backward(q, k, v, o, lse, do, causal=causal)
    torch.cuda.synchronize()
    ref_o, rq, rk, rv = sdpa_cpu(q, k, v, causal, do)
    assert (o.float().cpu() - ref_o).abs().max().item() < tol_f
    for got, ref in ((dq, rq), (dk, rk), (dv, rv)):
        assert (got.float().cpu() - ref).abs().max().item() < tol_b


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(1, 1, 8, 32), (2, 4, 64, 64), (1, 8, 128, 64), (4, 2, 32, 128)])
def test_pytorch_comparison_shapes(torch_gpu, shape):
    torch = torch_gpu
    torch.manual_seed(42)
    q, k, v = (torch.randn(shape).cuda() for _ in range(3))
    o, _ = cuflash_attn.flash_attention_forward(q, k, v, causal=False)
    torch.cuda.synchronize()
    assert o.shape == shape and torch.isfinite(o).all()
    assert (o.cpu() - sdpa_cpu(q, k, v, False)).abs().max().item() < 1e-3


# ---- stream semantics and reproducibility ----
@pytest.mark.gpu
def test_nondefault_streams_and_reproducibility(torch_gpu):
    """Results are bitwise identical across repeats and across streams (the backward
    workspace is stream-ordered per call, reference CHANGELOG.md:44-47; no kernel uses
    atomics, so every output element has one fixed summation order)."""
    torch = torch_gpu
    shape = (2, 4, 300, 128)
    xs = [synth.to_torch(synth.round_to(synth.normal(i, shape), "bfloat16"), "bfloat16")
          for i in (1, 2, 3, 4)]
    ref = cuflash_attn.flash_attention_forward(*xs[:3], causal=True)
    ref_g = cuflash_attn.flash_attention_backward(*xs[:3], *ref, xs[3], causal=True)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    results = []
    for s in streams:
        with torch.cuda.stream(s):
            o, lse = cuflash_attn.flash_attention_forward(*xs[:3], causal=True, stream=s)
            g = cuflash_attn.flash_attention_backward(*xs[:3], o, lse, xs[3], causal=True,
                                                      stream=s)
            results.append((o, lse) + tuple(g))
    torch.cuda.synchronize()
    for res in results:
        for a, b in zip(res, tuple(ref) + tuple(ref_g)):
            assert torch.equal(a, b)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("d,n", [(64, 200), (128, 1), (128, 77), (128, 333)])
def test_backward_ragged_parity(torch_gpu, dtype, causal, d, n):
    """Backward at ragged lengths (N not a multiple of the 32-row / 128-key blocks) against
    the oracle."""
    shape = (1, 2, n, d)
    xs = [synth.round_to(synth.normal(60 + i, shape), dtype) for i in range(4)]
    o, lse, dq, dk, dv = run(dtype, *xs[:3], d ** -0.5, causal, xs[3])
    rq, rk, rv = oracle.backward(*xs, d ** -0.5, causal)
    for got, ref in ((dq, rq), (dk, rk), (dv, rv)):
        assert max_abs(got, ref) <= 2e-2


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_decode_matches_last_row_of_causal_forward(torch_gpu, dtype):
    """Split-KV decode of the last query equals row N-1 of this library's causal forward."""
    n, d = 777, 128
    xs = [synth.round_to(synth.normal(80 + i, (2, 2, n, d)), dtype) for i in range(3)]
    o_full, l_full = run(dtype, *xs, d ** -0.5, True)
    tq = synth.to_torch(np.ascontiguousarray(xs[0][:, :, -1:]), dtype)
    tk, tv = (synth.to_torch(x, dtype) for x in xs[1:])
    for splits in (1, 5, 48):
        o, lse = cuflash_attn.flash_attention_decode(tq, tk, tv, scale=d ** -0.5,
                                                     num_splits=splits)
        torch_gpu.cuda.synchronize()
        tol = 1e-4 if dtype == "float32" else 2e-2
        assert max_abs(synth.to_numpy(o)[:, :, 0], o_full[:, :, -1]) <= tol
        assert max_abs(synth.to_numpy(lse)[:, :, 0], l_full[:, :, -1]) <= max(tol, 1e-4)
