"""The reference's PyTorch comparison suite (tests/integration/test_pytorch_comparison.py:421-731)
restated against this library: the same nine cases, shapes, seeds and tolerances, calling
libcuflash_attn.so through a raw ctypes binding written the way the reference's callers write
theirs (pointers as c_void_p, scale as c_float, causal as c_bool, the stream as None; reference
:37-147, :197-410). It does not use this repository's cuflash_attn helpers, so it shows that an
unchanged ctypes caller of the reference runs against the HIP build.

The expected values are torch's scaled_dot_product_attention and its autograd gradients, computed
in float32 on the CPU (the reference computes the half-precision forward references in half
precision on the GPU; float32 is the more exact reference and keeps bf16 batched products off the
GPU). Inputs are drawn on the GPU with torch.manual_seed(42) as in the reference.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

import cuflash_attn

SUCCESS = 0


class ReferenceStyleBinding:
    """argtypes exactly as the reference's CuFlashLibrary sets them."""

    def __init__(self, path: str):
        self.library = ctypes.CDLL(path)
        fwd = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 4 + [ctypes.c_float, ctypes.c_bool,
                                                          ctypes.c_void_p]
        bwd = [ctypes.c_void_p] * 9 + [ctypes.c_int] * 4 + [ctypes.c_float, ctypes.c_bool,
                                                          ctypes.c_void_p]
        for sfx in ("f32", "f16", "bf16"):
            f = getattr(self.library, f"cuflash_attention_forward_{sfx}")
            f.argtypes, f.restype = fwd, ctypes.c_int
            b = getattr(self.library, f"cuflash_attention_backward_{sfx}")
            b.argtypes, b.restype = bwd, ctypes.c_int


@pytest.fixture(scope="module")
def binding():
    import torch

    if torch.cuda.device_count() == 0:
        pytest.skip("no GPU")
    for path in cuflash_attn.candidate_library_paths():
        if os.path.exists(path):
            return ReferenceStyleBinding(path)
    pytest.fail("libcuflash_attn.so not found on the reference's search path")


def _ptr(t):
    assert t.is_cuda and t.is_contiguous()
    return ctypes.c_void_p(t.data_ptr())


_SFX = {"float32": "f32", "float16": "f16", "bfloat16": "bf16"}


def _forward(binding, q, k, v, causal):
    import torch

    b, h, n, d = q.shape
    o = torch.empty_like(q)
    l = torch.empty((b, h, n), device=q.device, dtype=torch.float32)
    fn = getattr(binding.library, f"cuflash_attention_forward_{_SFX[str(q.dtype)[6:]]}")
    status = fn(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(l), b, h, n, d,
                ctypes.c_float(float(1.0 / np.sqrt(d))), causal, None)
    torch.cuda.synchronize()
    return status, o, l


def _backward(binding, q, k, v, o, l, do, causal):
    import torch

    b, h, n, d = q.shape
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    fn = getattr(binding.library, f"cuflash_attention_backward_{_SFX[str(q.dtype)[6:]]}")
    status = fn(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(l), _ptr(do), _ptr(dq), _ptr(dk),
                _ptr(dv), b, h, n, d, ctypes.c_float(float(1.0 / np.sqrt(d))), causal, None)
    torch.cuda.synchronize()
    return status, dq, dk, dv


def _reference(q, k, v, causal, do=None):
    """float32 CPU scaled_dot_product_attention (and gradients when do is given)."""
    import torch
    import torch.nn.functional as F

    qc, kc, vc = (t.detach().float().cpu().requires_grad_(do is not None) for t in (q, k, v))
    out = F.scaled_dot_product_attention(qc, kc, vc, scale=float(1.0 / np.sqrt(q.shape[-1])),
                                         is_causal=causal)
    if do is None:
        return out.detach()
    out.backward(do.detach().float().cpu())
    return out.detach(), qc.grad, kc.grad, vc.grad


def _inputs(shape, dtype, with_grad=False):
    import torch

    torch.manual_seed(42)
    t = getattr(torch, dtype)
    xs = [torch.randn(*shape, device="cuda", dtype=t).contiguous() for _ in range(3)]
    if with_grad:
        xs.append(torch.randn(*shape, device="cuda", dtype=t).contiguous())
    return xs


def _maxdiff(a, b):
    return float((a.detach().float().cpu() - b.float()).abs().max())


# test_forward_equivalence (:421-444), test_causal_mask (:447-470), test_fp16_forward_equivalence
# (:518-541), test_fp16_causal_forward (:593-616), test_bf16_forward_equivalence (:619-646)
@pytest.mark.gpu
@pytest.mark.parametrize("dtype,shape,causal,tol", [
    ("float32", (2, 4, 64, 64), False, 1e-3),
    ("float32", (1, 2, 32, 32), True, 1e-3),
    ("float16", (1, 2, 32, 32), False, 1e-2),
    ("float16", (1, 2, 32, 32), True, 1e-2),
    ("bfloat16", (1, 2, 32, 32), False, 2e-2),
])
def test_forward_against_pytorch(binding, dtype, shape, causal, tol):
    q, k, v = _inputs(shape, dtype)
    status, o, _ = _forward(binding, q, k, v, causal)
    assert status == SUCCESS
    assert _maxdiff(o, _reference(q, k, v, causal)) < tol


# test_backward_gradients (:473-515), test_fp16_backward_equivalence (:544-590),
# test_bf16_backward_equivalence (:649-692)
@pytest.mark.gpu
@pytest.mark.parametrize("dtype,shape,tol", [
    ("float32", (1, 2, 16, 32), 1e-3),
    ("float16", (1, 1, 16, 32), 2e-2),
    ("bfloat16", (1, 1, 16, 32), 2e-2),
])
def test_backward_against_pytorch_autograd(binding, dtype, shape, tol):
    q, k, v, do = _inputs(shape, dtype, with_grad=True)
    status, o, l = _forward(binding, q, k, v, False)
    assert status == SUCCESS
    status, dq, dk, dv = _backward(binding, q, k, v, o, l, do, False)
    assert status == SUCCESS
    _, rq, rk, rv = _reference(q, k, v, False, do)
    assert _maxdiff(dq, rq) < tol
    assert _maxdiff(dk, rk) < tol
    assert _maxdiff(dv, rv) < tol


# test_different_shapes (:695-731)
@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(1, 1, 8, 32), (2, 4, 64, 64), (1, 8, 128, 64),
                                   (4, 2, 32, 128)])
def test_different_shapes(binding, shape):
    q, k, v = _inputs(shape, "float32")
    status, o, _ = _forward(binding, q, k, v, False)
    assert status == SUCCESS
    assert tuple(o.shape) == shape
    assert bool(o.isfinite().all())
    assert _maxdiff(o, _reference(q, k, v, False)) < 1e-3


@pytest.mark.gpu
def test_error_codes_through_reference_binding(binding):
    """The status codes a reference caller checks (SUCCESS = 0, non-zero otherwise)."""
    import torch

    q = torch.zeros((1, 1, 8, 48), device="cuda", dtype=torch.float32)
    status, _, _ = _forward(binding, q, q, q, False)
    assert status == 6  # UNSUPPORTED_HEAD_DIM
    err = binding.library.cuflash_error_string
    err.argtypes, err.restype = [ctypes.c_int], ctypes.c_char_p
    assert err(6).decode() == "Unsupported head_dim: must be 32, 64, or 128"
