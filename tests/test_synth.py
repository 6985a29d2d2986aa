"""Synthetic-input generator: determinism, distribution sanity, and RNE rounding vs PyTorch."""

from __future__ import annotations

import numpy as np
import torch

from cuflash_attn import synth


def test_stream_is_deterministic_and_chunk_independent():
    a = synth.normal(3, (5, 1000))
    b = synth.normal(3, (5000,))
    assert np.array_equal(a.ravel(), b)
    assert not np.array_equal(synth.normal(4, (5000,)), b)
    u = synth.uniform(9, (1 << 23) + 7)  # spans two generation chunks
    assert np.array_equal(u[:100], synth.uniform(9, 100))


def test_splitmix64_known_values():
    # SplitMix64 from state 0: first outputs 0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4
    bits = synth._bits(0, 0, 2)
    assert int(bits[0]) == 0xE220A8397B1DCDAF
    assert int(bits[1]) == 0x6E789E6AA1B965F4


def test_distributions():
    u = synth.uniform(1, 1 << 20)
    assert u.min() >= -1.0 and u.max() < 1.0
    assert abs(u.mean()) < 5e-3 and abs(u.var() - 1.0 / 3.0) < 5e-3
    z = synth.normal(2, 1 << 20, std=0.5)
    assert abs(z.mean()) < 3e-3 and abs(z.std() - 0.5) < 3e-3


def test_bf16_rounding_matches_torch():
    x = np.concatenate([synth.normal(5, 100000) * 1e3, np.array([0.0, -0.0, 1e-40, 3.0e38,
                                                                np.inf, -np.inf])]).astype(
        np.float32)
    ours = synth.bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    nan = synth.bf16_bits(np.array([np.nan], dtype=np.float32))
    assert synth.bf16_to_f32(nan)[0] != synth.bf16_to_f32(nan)[0]


def test_round_to_is_idempotent():
    x = synth.normal(6, 4096)
    for dt in ("float16", "bfloat16", "float32"):
        r = synth.round_to(x, dt)
        assert np.array_equal(synth.round_to(r, dt), r)
