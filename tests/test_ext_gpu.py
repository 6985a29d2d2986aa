"""GPU parity of the extended forward / backward (cuflash_attention_{forward,backward}_ext_*):
separate query and key/value lengths with a causal mask aligned to the end of the keys,
grouped-query / multi-query heads, and head_dim 96 and 256 beside 32 / 64 / 128.

Expected values come from the fp64 oracle on a per-query-head copy of K and V (each key/value
head repeated num_heads / num_kv_heads times); the expected dK and dV of a key/value head are the
sums of the copies' gradients over its query heads. The oracle's separate-length form is pinned
against torch float64 autograd with an explicit mask and against the full causal attention
(tests/test_oracle.py). Tolerances as in test_parity_gpu.py (fp32 1e-4 relative, fp16/bf16
2e-2 max-abs).
"""

from __future__ import annotations

import numpy as np
import pytest

import cuflash_attn
import oracle
from cuflash_attn import synth
from test_parity_gpu import check

DTYPES = ["float32", "float16", "bfloat16"]

# (q_len, kv_len, causal): one new token against a cache, a square head, prefill chunks whose
# causal diagonal falls inside a key block, more queries than keys (non-causal only), ragged
# lengths on both sides.
SHAPES = [(1, 300, True), (77, 77, True), (100, 333, True), (130, 64, False), (200, 513, False)]
HEADS = [(4, 4), (8, 2), (6, 1)]


def _inputs(dtype, b, h, hkv, nq, nk, d, seed):
    """Uniform [-1, 1) inputs, as in test_parity_gpu.py: the 2e-2 bound on fp16/bf16 outputs
    presumes values of that scale (a bf16 result near 4 is already rounded by up to 1.6e-2),
    and the grouped dK, dV sum num_heads / num_kv_heads heads' gradients."""
    q = synth.round_to(synth.uniform(seed, (b, h, nq, d)), dtype)
    k = synth.round_to(synth.uniform(seed + 1, (b, hkv, nk, d)), dtype)
    v = synth.round_to(synth.uniform(seed + 2, (b, hkv, nk, d)), dtype)
    do = synth.round_to(synth.uniform(seed + 3, (b, h, nq, d)), dtype)
    return q, k, v, do


def _expand(x, group):
    return np.repeat(x, group, axis=1)


def _fold(x, group):
    """[B, Hkv * group, N, D] -> [B, Hkv, N, D], summing each key/value head's query heads."""
    b, h, n, d = x.shape
    return x.reshape(b, h // group, group, n, d).sum(axis=2)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [32, 64, 96, 128, 256])
@pytest.mark.parametrize("heads,kv_heads", HEADS)
def test_forward_ext_parity(torch_gpu, dtype, d, heads, kv_heads):
    group = heads // kv_heads
    for i, (nq, nk, causal) in enumerate(SHAPES):
        q, k, v, _ = _inputs(dtype, 2, heads, kv_heads, nq, nk, d, seed=10 * i + d)
        scale = d ** -0.5
        tq, tk, tv = (synth.to_torch(x, dtype) for x in (q, k, v))
        o, lse = cuflash_attn.flash_attention_forward_ext(tq, tk, tv, scale=scale, causal=causal)
        torch_gpu.cuda.synchronize()
        o_ref, l_ref = oracle.forward(q, _expand(k, group), _expand(v, group), scale, causal)
        what = f"nq={nq} nk={nk} causal={causal}"
        check(dtype, synth.to_numpy(o), o_ref, f"O {what}")
        check(dtype, synth.to_numpy(lse), l_ref, f"L {what}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [32, 64, 96, 128, 256])
@pytest.mark.parametrize("heads,kv_heads", HEADS)
def test_backward_ext_parity(torch_gpu, dtype, d, heads, kv_heads):
    group = heads // kv_heads
    for i, (nq, nk, causal) in enumerate(SHAPES):
        q, k, v, do = _inputs(dtype, 1, heads, kv_heads, nq, nk, d, seed=10 * i + d + 5)
        scale = d ** -0.5
        tq, tk, tv, tdo = (synth.to_torch(x, dtype) for x in (q, k, v, do))
        o, lse = cuflash_attn.flash_attention_forward_ext(tq, tk, tv, scale=scale, causal=causal)
        dq, dk, dv = cuflash_attn.flash_attention_backward_ext(tq, tk, tv, o, lse, tdo,
                                                               scale=scale, causal=causal)
        torch_gpu.cuda.synchronize()
        dq_ref, dk_ref, dv_ref = oracle.backward(q, _expand(k, group), _expand(v, group), do,
                                                 scale, causal)
        what = f"nq={nq} nk={nk} causal={causal}"
        check(dtype, synth.to_numpy(dq), dq_ref, f"dQ {what}")
        check(dtype, synth.to_numpy(dk), _fold(dk_ref, group), f"dK {what}")
        check(dtype, synth.to_numpy(dv), _fold(dv_ref, group), f"dV {what}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [32, 64, 128])
def test_ext_equals_reference_entry_points_on_their_shapes(torch_gpu, dtype, d):
    """num_kv_heads == num_heads, q_len == kv_len and a reference head_dim run the same kernels
    as flash_attention_forward / _backward: the results are bitwise equal."""
    for causal in (False, True):
        q, k, v, do = _inputs(dtype, 2, 3, 3, 300, 300, d, seed=d + int(causal))
        tq, tk, tv, tdo = (synth.to_torch(x, dtype) for x in (q, k, v, do))
        o1, l1 = cuflash_attn.flash_attention_forward(tq, tk, tv, causal=causal)
        o2, l2 = cuflash_attn.flash_attention_forward_ext(tq, tk, tv, causal=causal)
        g1 = cuflash_attn.flash_attention_backward(tq, tk, tv, o1, l1, tdo, causal=causal)
        g2 = cuflash_attn.flash_attention_backward_ext(tq, tk, tv, o1, l1, tdo, causal=causal)
        torch_gpu.cuda.synchronize()
        assert torch_gpu.equal(o1, o2) and torch_gpu.equal(l1, l2)
        for a, b in zip(g1, g2):
            assert torch_gpu.equal(a, b)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_prefill_chunk_equals_rows_of_full_causal_attention(torch_gpu, dtype):
    """A chunk of queries that are the last q_len positions of the sequence gives the last rows
    of the full causal forward (same library, D = 128 kernels on both sides)."""
    n, nq, d = 1000, 136, 128
    q, k, v, _ = _inputs(dtype, 1, 8, 2, n, n, d, seed=3)
    tq, tk, tv = (synth.to_torch(x, dtype) for x in (q, k, v))
    o_full, l_full = cuflash_attn.flash_attention_forward_ext(tq, tk, tv, causal=True)
    o, lse = cuflash_attn.flash_attention_forward_ext(tq[:, :, n - nq:].contiguous(), tk, tv,
                                                      causal=True)
    torch_gpu.cuda.synchronize()
    assert float((o.float() - o_full[:, :, n - nq:].float()).abs().max()) <= 1e-2
    assert float((lse - l_full[:, :, n - nq:]).abs().max()) <= 1e-4


@pytest.mark.gpu
def test_gqa_backward_without_shares_matches_expanded_heads(torch_gpu):
    """Grouped heads whose fp32 dK/dV shares would exceed 2 GiB (64 query heads x 32768 keys)
    take the per-key/value-head dkdv items that sum the group in registers. Checked against the
    same library on K/V repeated per query head (no grouping): dQ is computed identically
    (bitwise equal), dK and dV are the sums over each group (fp32 here, one rounding there)."""
    import torch

    B, H, Hkv, nq, nk, d = 1, 64, 8, 128, 32768, 128
    group = H // Hkv
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    q, do = (torch.rand((B, H, nq, d), generator=g, device="cuda") * 2 - 1 for _ in range(2))
    k, v = (torch.rand((B, Hkv, nk, d), generator=g, device="cuda") * 2 - 1 for _ in range(2))
    q, do, k, v = (x.to(torch.bfloat16).contiguous() for x in (q, do, k, v))
    o, lse = cuflash_attn.flash_attention_forward_ext(q, k, v, causal=True)
    dq, dk, dv = cuflash_attn.flash_attention_backward_ext(q, k, v, o, lse, do, causal=True)
    ke = torch.repeat_interleave(k, group, dim=1).contiguous()
    ve = torch.repeat_interleave(v, group, dim=1).contiguous()
    o2, lse2 = cuflash_attn.flash_attention_forward_ext(q, ke, ve, causal=True)
    dq2, dk2, dv2 = cuflash_attn.flash_attention_backward_ext(q, ke, ve, o2, lse2, do,
                                                              causal=True)
    torch_gpu.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    assert torch.equal(dq, dq2)
    dk_sum = dk2.float().reshape(B, Hkv, group, nk, d).sum(2)
    dv_sum = dv2.float().reshape(B, Hkv, group, nk, d).sum(2)
    assert float((dk.float() - dk_sum).abs().max()) <= 2e-2
    assert float((dv.float() - dv_sum).abs().max()) <= 2e-2
