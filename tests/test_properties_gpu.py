"""The reference's RapidCheck properties, restated as seeded sweeps with a fixed example budget.

Each test draws EXAMPLES random cases from numpy's PCG64 with a fixed seed, with the generator
ranges of the reference property (rc::gen::inRange(a, b) is the half-open range [a, b)), runs the
library through the C ABI, and stops at the first failing case, naming it. The expected values
come from the fp64 oracle (the reference compares with its own CPU restatements,
tests/unit/test_forward.cu:21-69 and tests/unit/test_backward.cu:21-127).

  * ForwardProperty.NumericalEquivalence   tests/unit/test_forward.cu:339-391
  * BackwardProperty.GradientEquivalence   tests/unit/test_backward.cu:292-361
  * CausalMaskProperty.FutureIndependence  tests/unit/test_causal_mask.cu:104-174
  * DTypeProperty.FP16ClosesToFP32         tests/unit/test_dtype.cu:758-841
  * NumericalStabilityProperty.NoNaNOrInf  tests/unit/test_numerical_stability.cu:178-228

RapidCheck runs 100 cases per property by default; so do these sweeps.
"""

from __future__ import annotations

import numpy as np
import pytest

import cuflash_attn
import oracle
from conftest import max_abs
from cuflash_attn import synth

EXAMPLES = 100


def _cents(rng, shape, lo=-100, hi=100):
    """Values k * 0.01 with integer k in [lo, hi), as rc::gen::inRange(lo, hi) * 0.01f."""
    return (rng.integers(lo, hi, size=shape).astype(np.float32) * np.float32(0.01))


def _t(x, dtype="float32"):
    return synth.to_torch(x, dtype)


@pytest.mark.gpu
def test_forward_numerical_equivalence(torch_gpu):
    rng = np.random.default_rng(339)
    for case in range(EXAMPLES):
        b, h, n = int(rng.integers(1, 3)), int(rng.integers(1, 4)), int(rng.integers(1, 65))
        d = int(rng.choice([32, 64]))
        q, k, v = (_cents(rng, (b, h, n, d)) for _ in range(3))
        scale = 1.0 / np.sqrt(np.float32(d))
        o, _ = cuflash_attn.flash_attention_forward(_t(q), _t(k), _t(v), scale=float(scale),
                                                    causal=False)
        torch_gpu.cuda.synchronize()
        o_ref, _ = oracle.forward(q, k, v, float(scale), False)
        err = max_abs(synth.to_numpy(o), o_ref)
        assert err < 1e-3, f"case {case}: B={b} H={h} N={n} D={d} max|dO|={err}"


@pytest.mark.gpu
def test_backward_gradient_equivalence(torch_gpu):
    rng = np.random.default_rng(292)
    for case in range(EXAMPLES):
        h, n, d = int(rng.integers(1, 3)), int(rng.integers(1, 33)), int(rng.choice([32, 64]))
        q, k, v, do = (_cents(rng, (1, h, n, d)) for _ in range(4))
        scale = float(1.0 / np.sqrt(np.float32(d)))
        tq, tk, tv, tdo = (_t(x) for x in (q, k, v, do))
        o, lse = cuflash_attn.flash_attention_forward(tq, tk, tv, scale=scale, causal=False)
        dq, dk, dv = cuflash_attn.flash_attention_backward(tq, tk, tv, o, lse, tdo, scale=scale,
                                                           causal=False)
        torch_gpu.cuda.synchronize()
        refs = oracle.backward(q, k, v, do, scale, False)
        for name, got, ref in zip(("dQ", "dK", "dV"), (dq, dk, dv), refs):
            err = max_abs(synth.to_numpy(got), ref)
            assert err < 1e-3, f"case {case}: H={h} N={n} D={d} {name} max err {err}"


@pytest.mark.gpu
def test_causal_future_independence(torch_gpu):
    rng = np.random.default_rng(104)
    for case in range(EXAMPLES):
        n, d = int(rng.integers(4, 33)), int(rng.choice([32, 64]))
        q, k, v = (_cents(rng, (1, 1, n, d)) for _ in range(3))
        pos = int(rng.integers(0, n - 1))
        scale = float(1.0 / np.sqrt(np.float32(d)))
        o1, _ = cuflash_attn.flash_attention_forward(_t(q), _t(k), _t(v), scale=scale,
                                                     causal=True)
        k2, v2 = k.copy(), v.copy()
        k2[:, :, pos + 1:] = _cents(rng, k2[:, :, pos + 1:].shape, -1000, 1000)
        v2[:, :, pos + 1:] = _cents(rng, v2[:, :, pos + 1:].shape, -1000, 1000)
        o2, _ = cuflash_attn.flash_attention_forward(_t(q), _t(k2), _t(v2), scale=scale,
                                                     causal=True)
        torch_gpu.cuda.synchronize()
        diff = max_abs(synth.to_numpy(o1)[:, :, pos], synth.to_numpy(o2)[:, :, pos])
        assert diff < 1e-5, f"case {case}: N={n} D={d} pos={pos} changed by {diff}"


@pytest.mark.gpu
def test_fp16_close_to_fp32(torch_gpu):
    rng = np.random.default_rng(758)
    for case in range(EXAMPLES):
        n, d = int(rng.integers(4, 33)), int(rng.choice([32, 64, 128]))
        q, k, v = (_cents(rng, (1, 1, n, d)) for _ in range(3))
        scale = float(1.0 / np.sqrt(np.float32(d)))
        o32, _ = cuflash_attn.flash_attention_forward(_t(q), _t(k), _t(v), scale=scale,
                                                      causal=False)
        o16, _ = cuflash_attn.flash_attention_forward(*(_t(x, "float16") for x in (q, k, v)),
                                                      scale=scale, causal=False)
        torch_gpu.cuda.synchronize()
        diff = max_abs(synth.to_numpy(o32), synth.to_numpy(o16))
        assert diff < 1e-2, f"case {case}: N={n} D={d} max|fp32 - fp16|={diff}"


@pytest.mark.gpu
def test_no_nan_or_inf(torch_gpu):
    rng = np.random.default_rng(178)
    for case in range(EXAMPLES):
        n, d = int(rng.integers(1, 33)), int(rng.choice([32, 64]))
        xs = []
        for _ in range(3):
            mag = rng.integers(-3, 3, size=(1, 1, n, d)).astype(np.float32)
            xs.append(_cents(rng, (1, 1, n, d)) * np.power(np.float32(10.0), mag))
        scale = float(1.0 / np.sqrt(np.float32(d)))
        o, _ = cuflash_attn.flash_attention_forward(*(_t(x) for x in xs), scale=scale,
                                                    causal=False)
        torch_gpu.cuda.synchronize()
        assert np.isfinite(synth.to_numpy(o)).all(), f"case {case}: N={n} D={d}"
