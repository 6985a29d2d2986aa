"""GPU parity at launch sizes that select the forward's eight-wave workgroups.

The fp16/bf16 forward at head_dim 128 and 96 runs 256-row (eight-wave) workgroups whenever
B * H * ceil(Nq / 256) is at least the number of compute units (256 on an MI355X), and four-wave
128-row ones below that; at head_dim 64 the eight-wave workgroups run for causal launches of
that size, and every other head_dim-64 launch and every head_dim-32 launch runs the sequential
four-wave kernel (four workgroups per CU), checked here at the same wide shapes. The small shapes of test_ext_gpu.py and test_parity_gpu.py all take the four-wave
path, so these tests use B = 1, H = 32 and Nq in {2000, 2049}, which reach the eight-wave kernel
with the code that only runs there: a partial last key tile (Nk not a multiple of 64), query rows
past Nq in the last workgroup, the causal offset Nk - Nq > 0 with its per-wave stop, and
grouped heads (Hkv = 8: query head h reads key/value head h / 4).

Expected values: the fp64 oracle on the per-query-head copy of K and V, on two query heads for
the forward (O and L) and on the query heads of one key/value head for the backward, dQ on
sampled rows of each of them and dK, dV (summed over the group, the gradient of the shared
input) on sampled key rows. The reference's contract for ragged and causal keys is the `valid`
predicate of src/forward/flash_attention_forward_wmma.cu:132-133. Inputs are uniform in [-1, 1)
as in test_ext_gpu.py; tolerance 2e-2 max-abs (north star, fp16/bf16).
"""

from __future__ import annotations

import numpy as np
import pytest

import cuflash_attn
import oracle
from conftest import max_abs
from cuflash_attn import synth

TOL16 = 2e-2
B, H = 1, 32
FWD_SHAPES = [(2000, 2000), (2049, 2049), (2000, 8195), (2049, 8195)]


def _inputs(dtype, hkv, nq, nk, d, seed):
    q = synth.round_to(synth.uniform(seed, (B, H, nq, d)), dtype)
    k = synth.round_to(synth.uniform(seed + 1, (B, hkv, nk, d)), dtype)
    v = synth.round_to(synth.uniform(seed + 2, (B, hkv, nk, d)), dtype)
    do = synth.round_to(synth.uniform(seed + 3, (B, H, nq, d)), dtype)
    return q, k, v, do


def _assert_eight_wave_launch(torch, nq):
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert B * H * -(-nq // 256) >= cus, "shape would select the four-wave forward"


def _rows(n, step):
    edge = [0, 1, 2, 31, 32, 63, 64, 255, 256, n - 65, n - 64, n - 33, n - 32, n - 2, n - 1]
    r = np.concatenate([np.arange(0, n, step), [x for x in edge if 0 <= x < n]])
    return np.unique(r)


def _check_forward(torch, dtype, d, hkv, causal_list, seed0):
    group = H // hkv
    for i, (nq, nk) in enumerate(FWD_SHAPES):
        _assert_eight_wave_launch(torch, nq)
        q, k, v, _ = _inputs(dtype, hkv, nq, nk, d, seed=seed0 + 10 * i)
        tq, tk, tv = (synth.to_torch(x, dtype) for x in (q, k, v))
        for causal in causal_list:
            what = f"d={d} hkv={hkv} nq={nq} nk={nk} causal={causal}"
            print(f"[wide forward] {dtype} {what}", flush=True)
            o, lse = cuflash_attn.flash_attention_forward_ext(tq, tk, tv, scale=d ** -0.5,
                                                              causal=causal)
            torch.cuda.synchronize()
            o_np, l_np = synth.to_numpy(o), synth.to_numpy(lse)
            assert np.isfinite(o_np).all() and np.isfinite(l_np).all(), what
            for h in (0, H - 1):
                kvh = h // group
                o_ref, l_ref = oracle.forward(q[:, h:h + 1], k[:, kvh:kvh + 1],
                                              v[:, kvh:kvh + 1], d ** -0.5, causal)
                assert max_abs(o_np[:, h:h + 1], o_ref) <= TOL16, f"O h={h} {what}"
                assert max_abs(l_np[:, h:h + 1], l_ref) <= TOL16, f"L h={h} {what}"


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("d", [128, 96])
@pytest.mark.parametrize("hkv", [32, 8])
def test_eight_wave_forward_d128_d96(torch_gpu, dtype, d, hkv):
    _check_forward(torch_gpu, dtype, d, hkv, (True, False), seed0=d + hkv)


@pytest.mark.gpu
@pytest.mark.parametrize("hkv", [32, 8])
def test_eight_wave_forward_d64_causal(torch_gpu, hkv):
    _check_forward(torch_gpu, "bfloat16", 64, hkv, (True,), seed0=64 + hkv)


@pytest.mark.gpu
@pytest.mark.parametrize("d,causal_list", [(64, (False,)), (32, (True, False))])
@pytest.mark.parametrize("hkv", [32, 8])
def test_sequential_forward_d64_d32_wide(torch_gpu, d, causal_list, hkv):
    _check_forward(torch_gpu, "float16", d, hkv, causal_list, seed0=700 + d + hkv)


BWD_CASES = [(2000, 2000, True), (2049, 8195, True), (2049, 8195, False)]


@pytest.mark.gpu
@pytest.mark.parametrize("d", [128, 96, 64, 32])
@pytest.mark.parametrize("hkv", [32, 8])
def test_backward_ext_at_wide_launch_sizes(torch_gpu, d, hkv):
    torch = torch_gpu
    dtype = "bfloat16"
    group = H // hkv
    scale = d ** -0.5
    for i, (nq, nk, causal) in enumerate(BWD_CASES):
        what = f"d={d} hkv={hkv} nq={nq} nk={nk} causal={causal}"
        print(f"[wide backward] {what}", flush=True)
        q, k, v, do = _inputs(dtype, hkv, nq, nk, d, seed=500 + 10 * i + d + hkv)
        tq, tk, tv, tdo = (synth.to_torch(x, dtype) for x in (q, k, v, do))
        o, lse = cuflash_attn.flash_attention_forward_ext(tq, tk, tv, scale=scale, causal=causal)
        dq, dk, dv = cuflash_attn.flash_attention_backward_ext(tq, tk, tv, o, lse, tdo,
                                                               scale=scale, causal=causal)
        torch.cuda.synchronize()
        dq_np, dk_np, dv_np = (synth.to_numpy(t) for t in (dq, dk, dv))
        for t in (dq_np, dk_np, dv_np):
            assert np.isfinite(t).all(), what
        # key/value head 1 (the second group) and its query heads
        kvh = 1
        hs = slice(kvh * group, (kvh + 1) * group)
        qrows, krows = _rows(nq, 97), _rows(nk, 89)
        ke = np.repeat(k[:, kvh:kvh + 1], group, axis=1)
        ve = np.repeat(v[:, kvh:kvh + 1], group, axis=1)
        rq, rk, rv = oracle.backward_rows(q[:, hs], ke, ve, do[:, hs], scale, causal, qrows,
                                          krows)
        assert max_abs(dq_np[:, hs][:, :, qrows], rq) <= TOL16, f"dQ {what}"
        assert max_abs(dk_np[:, kvh:kvh + 1][:, :, krows], rk.sum(axis=1, keepdims=True)) \
            <= TOL16, f"dK {what}"
        assert max_abs(dv_np[:, kvh:kvh + 1][:, :, krows], rv.sum(axis=1, keepdims=True)) \
            <= TOL16, f"dV {what}"
