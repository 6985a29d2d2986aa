"""BF16 causal forward and backward at long sequence lengths: the stress test of the BF16 path's
accumulated error that the reference plans (ROADMAP.md:27), at 32768 to 131072 keys (config 5
stops at 16384).

A causal row i is the one-query problem over keys 0..i, so O_i, L_i and dQ_i are checked against
the fp64 oracle on that problem alone (O(i D) each): rows 0, 1, 777, N / 2, N - 2, N - 1 of both
heads, the last ones summing over every key. Key rows N - 64 .. N - 1 are seen only by the last
64 queries, so their dK and dV are checked exactly against the oracle on those 64 queries over
all keys (causal, aligned to the end of the keys). Every head is also checked through the
identities of test_configs_gpu.py (sum_j dK_j = 0, sum_j dV_j = sum_i dO_i, causal row 0).
Tolerance: the north star's 2e-2 max-abs. The errors are printed per length.
"""

from __future__ import annotations

import numpy as np
import pytest

import cuflash_attn
import oracle
from conftest import max_abs
from test_configs_gpu import TOL16, check_invariants


@pytest.mark.gpu
@pytest.mark.parametrize("n", [32768, 65536, 131072])
def test_bf16_causal_long_sequence(torch_gpu, n):
    torch = torch_gpu
    B, H, D = 1, 2, 128
    scale = D ** -0.5
    print(f"[long] N={n}", flush=True)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(n)
    q, k, v, do = (torch.randn((B, H, n, D), generator=gen, device="cuda",
                               dtype=torch.float32).to(torch.bfloat16) for _ in range(4))
    o, lse = cuflash_attn.flash_attention_forward(q, k, v, scale=scale, causal=True)
    dq, dk, dv = cuflash_attn.flash_attention_backward(q, k, v, o, lse, do, scale=scale,
                                                       causal=True)
    torch.cuda.synchronize()
    host = {name: t.float().cpu().numpy() for name, t in
            (("q", q), ("k", k), ("v", v), ("do", do), ("o", o), ("lse", lse), ("dq", dq),
             ("dk", dk), ("dv", dv))}
    del q, k, v, do, o, lse, dq, dk, dv
    torch.cuda.empty_cache()
    f64 = {name: a.astype(np.float64) for name, a in host.items()
           if name in ("q", "k", "v", "do")}

    err = {"O": 0.0, "L": 0.0, "dQ": 0.0, "dK": 0.0, "dV": 0.0}
    rel = {"dK": 0.0, "dV": 0.0}
    for h in range(H):
        for i in (0, 1, 777, n // 2, n - 2, n - 1):
            qi = f64["q"][:, h:h + 1, i:i + 1]
            doi = f64["do"][:, h:h + 1, i:i + 1]
            kk = f64["k"][:, h:h + 1, :i + 1]
            vv = f64["v"][:, h:h + 1, :i + 1]
            o_ref, l_ref = oracle.forward(qi, kk, vv, scale, False)
            dq_ref, _, _ = oracle.backward_rows(qi, kk, vv, doi, scale, False, [0], [])
            err["O"] = max(err["O"], max_abs(host["o"][:, h:h + 1, i:i + 1], o_ref))
            err["L"] = max(err["L"], max_abs(host["lse"][:, h:h + 1, i:i + 1], l_ref))
            err["dQ"] = max(err["dQ"], max_abs(host["dq"][:, h:h + 1, i:i + 1], dq_ref))
        last = slice(n - 64, n)
        _, dk_ref, dv_ref = oracle.backward_rows(
            f64["q"][:, h:h + 1, last], f64["k"][:, h:h + 1], f64["v"][:, h:h + 1],
            f64["do"][:, h:h + 1, last], scale, True, [], np.arange(n - 64, n))
        for name, got, ref in (("dK", host["dk"][:, h:h + 1, last], dk_ref),
                               ("dV", host["dv"][:, h:h + 1, last], dv_ref)):
            err[name] = max(err[name], max_abs(got, ref))
            # These rows are small (weights near 1 / N): also relative to their largest value.
            rel[name] = max(rel[name], max_abs(got, ref) / float(np.abs(ref).max()))
    print(f"[long] N={n} max errors: " + " ".join(f"{k}={v:.2e}" for k, v in err.items()) +
          " relative: " + " ".join(f"{k}={v:.2e}" for k, v in rel.items()), flush=True)
    for name, e in err.items():
        assert e <= TOL16, f"{name} {e}"
    for name, e in rel.items():
        assert e <= TOL16, f"{name} relative {e}"
    check_invariants(host["q"], host["k"], host["v"], host["o"], host["lse"], host["do"],
                     host["dq"], host["dk"], host["dv"], scale, n_tol=2e-2)
