"""Tensors past 2^31 elements: the headline path (bf16, head_dim 128, causal forward and
backward through the reference entry points) and the decodes (split-KV, grouped-query on the
matrix cores, paged).

Q, K, V, O, dO, dQ, dK and dV each hold 2 x 65568 x 128 x 128 = 2^31 + 2^20 elements (about
4.3 GB apiece, 35 GB in all), so every head from (1, 65504) on starts past element 2^31 and a
32-bit product anywhere in an offset (head, row, tile or L / (L, D) index, in the forward, the
delta pass or the fused backward) would read or write the wrong head. The inputs come from
torch's GPU generator; the heads on both sides of the boundary and the last head are copied back
and compared with the fp64 oracle on every row, to the north-star tolerance (2e-2 max-abs).
"""

from __future__ import annotations

import numpy as np
import pytest

import cuflash_attn
import oracle
from conftest import max_abs

TOL16 = 2e-2


@pytest.mark.gpu
def test_bf16_causal_fwd_bwd_past_2_31_elements(torch_gpu):
    torch = torch_gpu
    B, H, N, D = 2, 65568, 128, 128
    assert B * H * N * D > 2 ** 31 and (B * H - 64) * N * D == 2 ** 31
    scale = D ** -0.5
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(31)
    q, k, v, do = (torch.randn((B, H, N, D), device=dev, dtype=torch.bfloat16, generator=gen)
                   for _ in range(4))
    o, lse = cuflash_attn.flash_attention_forward(q, k, v, scale=scale, causal=True)
    dq, dk, dv = cuflash_attn.flash_attention_backward(q, k, v, o, lse, do, scale=scale,
                                                       causal=True)
    torch.cuda.synchronize()
    rows = np.arange(N)
    # (0, 0): the first head; (1, 65503) ends at element 2^31; (1, 65504) starts there;
    # (1, 65567): the last head.
    for b, h in ((0, 0), (1, 65503), (1, 65504), (1, H - 1)):
        host = [t[b:b + 1, h:h + 1].float().cpu().numpy().astype(np.float64)
                for t in (q, k, v, do)]
        got = [t[b:b + 1, h:h + 1].float().cpu().numpy() for t in (o, lse, dq, dk, dv)]
        o_ref, l_ref = oracle.forward(host[0], host[1], host[2], scale, True)
        assert max_abs(got[0], o_ref) <= TOL16, f"O {(b, h)}"
        assert max_abs(got[1], l_ref) <= TOL16, f"L {(b, h)}"
        rq, rk, rv = oracle.backward_rows(*host, scale, True, rows, rows)
        assert max_abs(got[2], rq) <= TOL16, f"dQ {(b, h)}"
        assert max_abs(got[3], rk) <= TOL16, f"dK {(b, h)}"
        assert max_abs(got[4], rv) <= TOL16, f"dV {(b, h)}"
    del q, k, v, do, o, lse, dq, dk, dv
    torch.cuda.empty_cache()  # 35 GB back to the device for the tests that follow


@pytest.mark.gpu
@pytest.mark.parametrize("splits", [16, 0])
def test_fp16_decode_past_2_31_elements(torch_gpu, splits):
    """Config 4's decode with one more batch row: K and V hold 17 x 32 x 32768 x 128 = 2^31 +
    2^27 elements each, so batch row 16 starts at element 2^31 (config 4 itself ends exactly
    there). Heads on both sides of the boundary and the last head against the oracle."""
    torch = torch_gpu
    B, H, LKV, D = 17, 32, 32768, 128
    assert (B - 1) * H * LKV * D == 2 ** 31
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(32)
    q = torch.randn((B, H, 1, D), device=dev, dtype=torch.float16, generator=gen)
    k = torch.randn((B, H, LKV, D), device=dev, dtype=torch.float16, generator=gen)
    v = torch.randn((B, H, LKV, D), device=dev, dtype=torch.float16, generator=gen)
    o, lse = cuflash_attn.flash_attention_decode(q, k, v, scale=D ** -0.5, num_splits=splits)
    torch.cuda.synchronize()
    for b, h in ((0, 0), (15, 31), (16, 0), (16, 31)):
        qh, kh, vh = (t[b:b + 1, h:h + 1].float().cpu().numpy().astype(np.float64)
                      for t in (q, k, v))
        o_ref, l_ref = oracle.forward(qh, kh, vh, D ** -0.5, False)
        assert max_abs(o[b:b + 1, h:h + 1].float().cpu().numpy(), o_ref) <= TOL16, f"O {(b, h)}"
        assert max_abs(lse[b:b + 1, h:h + 1].float().cpu().numpy(), l_ref) <= TOL16, f"L {(b, h)}"
    del q, k, v, o, lse
    torch.cuda.empty_cache()


@pytest.mark.gpu
def test_fp16_gqa_decode_past_2_31_elements(torch_gpu):
    """Grouped-query decode (32 query heads over 8 key/value heads: the matrix-core kernel) with
    K and V of 65 x 8 x 32768 x 128 = 2^31 + 2^25 elements each; batch row 64 starts at element
    2^31. Query heads on both sides of the boundary against the oracle."""
    torch = torch_gpu
    B, H, HKV, LKV, D = 65, 32, 8, 32768, 128
    assert (B - 1) * HKV * LKV * D == 2 ** 31
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(33)
    q = torch.randn((B, H, 1, D), device=dev, dtype=torch.float16, generator=gen)
    k = torch.randn((B, HKV, LKV, D), device=dev, dtype=torch.float16, generator=gen)
    v = torch.randn((B, HKV, LKV, D), device=dev, dtype=torch.float16, generator=gen)
    o, lse = cuflash_attn.flash_attention_decode(q, k, v, scale=D ** -0.5)
    torch.cuda.synchronize()
    for b, h in ((0, 0), (63, 31), (64, 0), (64, 31)):
        hk = h // (H // HKV)
        qh = q[b:b + 1, h:h + 1].float().cpu().numpy().astype(np.float64)
        kh, vh = (t[b:b + 1, hk:hk + 1].float().cpu().numpy().astype(np.float64) for t in (k, v))
        o_ref, l_ref = oracle.forward(qh, kh, vh, D ** -0.5, False)
        assert max_abs(o[b:b + 1, h:h + 1].float().cpu().numpy(), o_ref) <= TOL16, f"O {(b, h)}"
        assert max_abs(lse[b:b + 1, h:h + 1].float().cpu().numpy(), l_ref) <= TOL16, f"L {(b, h)}"
    del q, k, v, o, lse
    torch.cuda.empty_cache()


@pytest.mark.gpu
def test_fp16_paged_gqa_decode_past_2_31_elements(torch_gpu):
    """Paged grouped-query decode (32 query heads over 8 key/value heads, 16-key pages in
    shuffled order: the matrix-core kernel) over caches of 133120 pages x 16 x 8 x 128 = 2^31 +
    2^25 elements each: every page from 131072 on lies at or past element 2^31. Sequences whose
    pages cross that boundary against the oracle on pages gathered in block-table order."""
    torch = torch_gpu
    B, H, HKV, PAGE, MAXP, D = 65, 32, 8, 16, 2048, 128
    npages = B * MAXP
    assert (npages - 2048) * PAGE * HKV * D == 2 ** 31
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(34)
    q = torch.randn((B, H, 1, D), device=dev, dtype=torch.float16, generator=gen)
    kc = torch.randn((npages, PAGE, HKV, D), device=dev, dtype=torch.float16, generator=gen)
    vc = torch.randn((npages, PAGE, HKV, D), device=dev, dtype=torch.float16, generator=gen)
    rng = np.random.default_rng(34)
    table = rng.permutation(npages).reshape(B, MAXP).astype(np.int32)
    lens = np.full(B, MAXP * PAGE, dtype=np.int32)
    lens[7] = 20000
    ttab = torch.from_numpy(table).to(dev)
    tlen = torch.from_numpy(lens).to(dev)
    o, lse = cuflash_attn.flash_attention_decode_paged(q, kc, vc, ttab, tlen, scale=D ** -0.5)
    torch.cuda.synchronize()
    for b, h in ((0, 0), (7, 13), (64, 31)):
        n = int(lens[b])
        assert table[b, : (n + PAGE - 1) // PAGE].max() >= 131072
        hk = h // (H // HKV)
        pages = torch.from_numpy(table[b].astype(np.int64)).to(dev)
        kh, vh = (t.index_select(0, pages).reshape(MAXP * PAGE, HKV, D)[:n, hk]
                  .float().cpu().numpy().astype(np.float64) for t in (kc, vc))
        qh = q[b:b + 1, h:h + 1].float().cpu().numpy().astype(np.float64)
        o_ref, l_ref = oracle.forward(qh, kh[None, None], vh[None, None], D ** -0.5, False)
        assert max_abs(o[b:b + 1, h:h + 1].float().cpu().numpy(), o_ref) <= TOL16, f"O {(b, h)}"
        assert max_abs(lse[b:b + 1, h:h + 1].float().cpu().numpy(), l_ref) <= TOL16, f"L {(b, h)}"
    del q, kc, vc, o, lse
    torch.cuda.empty_cache()
