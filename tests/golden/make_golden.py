"""Writes tests/golden/attention_cases.npz: small attention cases with expected outputs.

The expected values come from PyTorch's float64 CPU attention (explicit softmax(Q K^T * scale
+ mask) V, torch.logsumexp) and float64 autograd -- a library routine independent of this
repository's oracle. Inputs are produced by the repository's seeded generator and rounded to
the case's dtype first, so a consumer feeds exactly these float32 values to the code under
test. The shapes, seeds' roles, value ranges and tolerances mirror the reference's GPU tests
(tests/unit/test_forward.cu:121-333, tests/unit/test_backward.cu:138-286,
tests/unit/test_dtype.cu:24-750, tests/unit/test_stress_edge_cases.cu:52-118).

Run from the repository root: python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "cuflash-attn_amd"))

from cuflash_attn import synth  # noqa: E402

# name, (B, H, N, D), causal, dtype, distribution, value range/std, seed base
CASES = [
    ("fwd_basic_small", (1, 1, 8, 32), False, "float32", "uniform", 1.0, 42),
    ("fwd_causal_mh_d128", (2, 2, 16, 128), True, "float32", "uniform", 0.5, 123),
    ("fwd_lse_d64", (2, 2, 16, 64), False, "float32", "uniform", 1.0, 7),
    ("fwd_lse_causal_d32", (1, 2, 16, 32), True, "float32", "uniform", 1.0, 9),
    ("bwd_basic_small", (1, 1, 8, 32), False, "float32", "uniform", 1.0, 42),
    ("bwd_causal_d128", (1, 2, 16, 128), True, "float32", "uniform", 0.25, 7),
    ("fp16_fwd", (1, 1, 16, 32), False, "float16", "uniform", 1.0, 42),
    ("fp16_bwd", (1, 1, 8, 32), False, "float16", "uniform", 1.0, 42),
    ("bf16_fwd", (1, 1, 16, 32), False, "bfloat16", "uniform", 1.0, 42),
    ("bf16_bwd", (1, 1, 8, 32), False, "bfloat16", "uniform", 1.0, 42),
    ("ragged_n17_d64_causal", (1, 2, 17, 64), True, "float32", "normal", 1.0, 11),
    ("ragged_n33_d128", (2, 1, 33, 128), False, "bfloat16", "normal", 1.0, 13),
    ("ragged_n70_d64_causal_bf16", (1, 1, 70, 64), True, "bfloat16", "normal", 1.0, 17),
    ("min_dims_n1", (1, 1, 1, 32), False, "float32", "uniform", 1.0, 5),
]


def attention64(q, k, v, scale, causal):
    s = torch.matmul(q, k.transpose(-1, -2)) * scale
    if causal:
        n = s.shape[-1]
        mask = torch.triu(torch.ones(n, n, dtype=torch.bool), diagonal=1)
        s = s.masked_fill(mask, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v), lse


def make_case(shape, causal, dtype, dist, rng, seed):
    xs = []
    for i in range(4):
        if dist == "uniform":
            x = synth.uniform(seed + i, shape, -rng, rng)
        else:
            x = synth.normal(seed + i, shape, rng)
        xs.append(synth.round_to(x, dtype))
    q, k, v, do = (torch.from_numpy(x.astype(np.float64)).requires_grad_(True) for x in xs)
    scale = shape[3] ** -0.5
    o, lse = attention64(q, k, v, scale, causal)
    o.backward(do.detach())
    return {
        "q": xs[0], "k": xs[1], "v": xs[2], "do": xs[3],
        "o": o.detach().numpy().astype(np.float32), "lse": lse.detach().numpy().astype(np.float32),
        "dq": q.grad.numpy().astype(np.float32), "dk": k.grad.numpy().astype(np.float32),
        "dv": v.grad.numpy().astype(np.float32),
        "scale": np.float64(scale), "causal": np.int64(causal),
    }


def main():
    out = {}
    names = []
    for name, shape, causal, dtype, dist, rng, seed in CASES:
        case = make_case(shape, causal, dtype, dist, rng, seed)
        for key, val in case.items():
            out[f"{name}/{key}"] = val
        out[f"{name}/dtype"] = np.array(dtype)
        names.append(name)
    # split-KV decode case: one query against 50 keys, fp16 inputs, and its row of attention
    qd = synth.round_to(synth.normal(31, (1, 2, 1, 64)), "float16")
    kd = synth.round_to(synth.normal(32, (1, 2, 50, 64)), "float16")
    vd = synth.round_to(synth.normal(33, (1, 2, 50, 64)), "float16")
    od, ld = attention64(*(torch.from_numpy(x.astype(np.float64)) for x in (qd, kd, vd)),
                         64 ** -0.5, False)
    out.update({"decode/q": qd, "decode/k": kd, "decode/v": vd, "decode/o": od.numpy().astype(np.float32),
                "decode/lse": ld.numpy().astype(np.float32), "decode/scale": np.float64(64 ** -0.5)})
    out["names"] = np.array(names)
    path = os.path.join(HERE, "attention_cases.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(names)} cases + decode)")


if __name__ == "__main__":
    main()
