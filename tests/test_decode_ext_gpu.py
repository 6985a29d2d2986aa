"""GPU parity of the decode extensions (grouped-query heads, paged KV cache) against the fp64
CPU oracle, through the C ABI (cuflash_attention_decode_gqa_*, cuflash_attention_decode_paged_*).

Expected values come from oracle.forward on a contiguous, per-query-head copy of the keys and
values: for grouped-query attention each key/value head is repeated num_heads / num_kv_heads
times; for the paged cache each sequence's keys are gathered from its pages in block-table
order and cut to its length. Tolerances as in test_parity_gpu.py (fp32 1e-4 relative, fp16/bf16
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


def _expand_heads(x, group):
    """[B, Hkv, N, D] -> [B, Hkv * group, N, D]: query head h reads key/value head h // group."""
    return np.repeat(x, group, axis=1)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("heads,kv_heads", [(8, 1), (8, 2), (6, 3), (12, 2), (32, 4), (16, 16),
                                            (32, 1), (64, 1)])
@pytest.mark.parametrize("kv_len", [1, 77, 1500])
def test_decode_gqa_parity(torch_gpu, dtype, d, heads, kv_heads, kv_len):
    """Query heads per key/value head: 1 (plain), 2 to 32 (the matrix-core kernels for fp16 /
    bf16: 32 fills every column of their tiles), 64 (past them: the vector kernel)."""
    B = 2
    q = synth.round_to(synth.normal(11, (B, heads, 1, d)), dtype)
    k = synth.round_to(synth.normal(12, (B, kv_heads, kv_len, d)), dtype)
    v = synth.round_to(synth.normal(13, (B, kv_heads, kv_len, d)), dtype)
    scale = d ** -0.5
    tq, tk, tv = (synth.to_torch(x, dtype) for x in (q, k, v))
    for splits in (0, 5):
        o, lse = cuflash_attn.flash_attention_decode(tq, tk, tv, scale=scale, num_splits=splits)
        torch_gpu.cuda.synchronize()
        group = heads // kv_heads
        o_ref, l_ref = oracle.forward(q, _expand_heads(k, group), _expand_heads(v, group), scale,
                                      False)
        check(dtype, synth.to_numpy(o), o_ref, f"O splits={splits}")
        check(dtype, synth.to_numpy(lse), l_ref, f"L splits={splits}")


def _paged_case(dtype, d, B, heads, kv_heads, page_size, max_pages, seq_lens, seed):
    """A shuffled page pool holding each sequence's keys, its block table, and the contiguous
    per-sequence keys and values the oracle sees."""
    rng = np.random.default_rng(seed)
    num_pages = B * max_pages + 3
    k_pool = synth.round_to(synth.normal(seed + 1, (num_pages, page_size, kv_heads, d)), dtype)
    v_pool = synth.round_to(synth.normal(seed + 2, (num_pages, page_size, kv_heads, d)), dtype)
    table = rng.permutation(num_pages)[: B * max_pages].reshape(B, max_pages).astype(np.int32)
    seqs = []
    for b in range(B):
        n = int(min(max(seq_lens[b], 0), page_size * max_pages))
        kk = k_pool[table[b]].reshape(max_pages * page_size, kv_heads, d)[:n]
        vv = v_pool[table[b]].reshape(max_pages * page_size, kv_heads, d)[:n]
        seqs.append((np.ascontiguousarray(kk.transpose(1, 0, 2)),
                     np.ascontiguousarray(vv.transpose(1, 0, 2))))
    return k_pool, v_pool, table, seqs


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("heads,kv_heads", [(4, 4), (8, 2), (8, 1)])
@pytest.mark.parametrize("page_size", [16, 64])
def test_decode_paged_parity(torch_gpu, dtype, d, heads, kv_heads, page_size):
    import torch

    B, max_pages = 4, 9
    # A full table, a partial last page, a single key, a length past the capacity (clamped).
    seq_lens = [max_pages * page_size, 3 * page_size + 5, 1, max_pages * page_size + 40]
    k_pool, v_pool, table, seqs = _paged_case(dtype, d, B, heads, kv_heads, page_size,
                                              max_pages, seq_lens, seed=20 + d + page_size)
    q = synth.round_to(synth.normal(31, (B, heads, 1, d)), dtype)
    scale = d ** -0.5
    tq, tk, tv = (synth.to_torch(x, dtype) for x in (q, k_pool, v_pool))
    ttab = torch.from_numpy(table).to(tq.device)
    tlen = torch.tensor(seq_lens, dtype=torch.int32, device=tq.device)
    group = heads // kv_heads
    for splits in (0, 1, 7):
        o, lse = cuflash_attn.flash_attention_decode_paged(tq, tk, tv, ttab, tlen, scale=scale,
                                                           num_splits=splits)
        torch.cuda.synchronize()
        o, lse = synth.to_numpy(o), synth.to_numpy(lse)
        for b in range(B):
            kb, vb = seqs[b]
            o_ref, l_ref = oracle.forward(q[b:b + 1], _expand_heads(kb[None], group),
                                          _expand_heads(vb[None], group), scale, False)
            check(dtype, o[b:b + 1], o_ref, f"O b={b} splits={splits}")
            check(dtype, lse[b:b + 1], l_ref, f"L b={b} splits={splits}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("heads,kv_heads", [(8, 4), (64, 8), (24, 12), (16, 2), (32, 1)])
@pytest.mark.parametrize("page_size", [4, 12, 6, 1])
def test_decode_paged_matrix_core_pages(torch_gpu, dtype, heads, kv_heads, page_size):
    """fp16/bf16 head_dim 128 with 2 to 32 query heads per key/value head runs on the matrix
    cores: with 4, 8 or 12 key/value heads the four-head kernel at every page size (one key row
    per load; 12: three workgroups per key row), with 1 or 2 the one-head kernel on pages of a multiple of 4 keys (4: one 4-row group
    per page; 12: not a power of two) and the vector kernel otherwise (6, 1). Lengths: several
    32-key blocks and splits, a partial last block, one key, an empty sequence."""
    import torch

    B, d, max_pages = 5, 128, (1200 + page_size - 1) // page_size
    seq_lens = [max_pages * page_size, 1000, 33, 1, 0]
    k_pool, v_pool, table, seqs = _paged_case(dtype, d, B, heads, kv_heads, page_size, max_pages,
                                              seq_lens, seed=60 + page_size)
    q = synth.round_to(synth.normal(61, (B, heads, 1, d)), dtype)
    tq, tk, tv = (synth.to_torch(x, dtype) for x in (q, k_pool, v_pool))
    ttab = torch.from_numpy(table).to(tq.device)
    tlen = torch.tensor(seq_lens, dtype=torch.int32, device=tq.device)
    group = heads // kv_heads
    for splits in (0, 3, 16):
        o, lse = cuflash_attn.flash_attention_decode_paged(tq, tk, tv, ttab, tlen,
                                                           num_splits=splits)
        torch.cuda.synchronize()
        o, lse = synth.to_numpy(o), synth.to_numpy(lse)
        for b in range(B):
            if seq_lens[b] == 0:
                assert np.all(o[b] == 0.0) and np.all(np.isneginf(lse[b]))
                continue
            kb, vb = seqs[b]
            o_ref, l_ref = oracle.forward(q[b:b + 1], _expand_heads(kb[None], group),
                                          _expand_heads(vb[None], group), d ** -0.5, False)
            check(dtype, o[b:b + 1], o_ref, f"O b={b} splits={splits}")
            check(dtype, lse[b:b + 1], l_ref, f"L b={b} splits={splits}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("d", [32, 64])
@pytest.mark.parametrize("group", [2, 8])
@pytest.mark.parametrize("page_size", [1, 6, 16])
def test_decode_paged_rows_kernel_head_dims(torch_gpu, dtype, d, group, page_size):
    """Paged grouped-query decode with 512 / d key/value heads (8 at head_dim 64, 16 at 32): the
    kernel whose loads read one key row of all of them (1 KB) per instruction, at any page size.
    Lengths as in test_decode_paged_matrix_core_pages."""
    import torch

    kv_heads = 512 // d
    heads = group * kv_heads
    B, max_pages = 5, (1200 + page_size - 1) // page_size
    seq_lens = [max_pages * page_size, 1000, 33, 1, 0]
    k_pool, v_pool, table, seqs = _paged_case(dtype, d, B, heads, kv_heads, page_size, max_pages,
                                              seq_lens, seed=70 + d + page_size)
    q = synth.round_to(synth.normal(71, (B, heads, 1, d)), dtype)
    tq, tk, tv = (synth.to_torch(x, dtype) for x in (q, k_pool, v_pool))
    ttab = torch.from_numpy(table).to(tq.device)
    tlen = torch.tensor(seq_lens, dtype=torch.int32, device=tq.device)
    for splits in (0, 3):
        o, lse = cuflash_attn.flash_attention_decode_paged(tq, tk, tv, ttab, tlen,
                                                           num_splits=splits)
        torch.cuda.synchronize()
        o, lse = synth.to_numpy(o), synth.to_numpy(lse)
        for b in range(B):
            if seq_lens[b] == 0:
                assert np.all(o[b] == 0.0) and np.all(np.isneginf(lse[b]))
                continue
            kb, vb = seqs[b]
            o_ref, l_ref = oracle.forward(q[b:b + 1], _expand_heads(kb[None], group),
                                          _expand_heads(vb[None], group), d ** -0.5, False)
            check(dtype, o[b:b + 1], o_ref, f"O b={b} splits={splits}")
            check(dtype, lse[b:b + 1], l_ref, f"L b={b} splits={splits}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_decode_paged_empty_sequence(torch_gpu, dtype):
    """A sequence of length 0 (or negative) gives O = 0 and L = -inf; the others are unaffected."""
    import torch

    B, heads, kv_heads, d, page_size, max_pages = 3, 4, 2, 128, 16, 4
    seq_lens = [0, 37, -5]
    k_pool, v_pool, table, seqs = _paged_case(dtype, d, B, heads, kv_heads, page_size, max_pages,
                                              seq_lens, seed=5)
    q = synth.round_to(synth.normal(6, (B, heads, 1, d)), dtype)
    tq, tk, tv = (synth.to_torch(x, dtype) for x in (q, k_pool, v_pool))
    ttab = torch.from_numpy(table).to(tq.device)
    tlen = torch.tensor(seq_lens, dtype=torch.int32, device=tq.device)
    o, lse = cuflash_attn.flash_attention_decode_paged(tq, tk, tv, ttab, tlen, num_splits=3)
    torch.cuda.synchronize()
    o, lse = synth.to_numpy(o), synth.to_numpy(lse)
    for b in (0, 2):
        assert np.all(o[b] == 0.0)
        assert np.all(np.isneginf(lse[b]))
    kb, vb = seqs[1]
    o_ref, l_ref = oracle.forward(q[1:2], _expand_heads(kb[None], 2), _expand_heads(vb[None], 2),
                                  d ** -0.5, False)
    check(dtype, o[1:2], o_ref, "O")
    check(dtype, lse[1:2], l_ref, "L")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("scale", [0.0, 1e-6, 10.0])
def test_decode_matrix_core_edge_scales(torch_gpu, dtype, d, scale):
    """The matrix-core decode kernels at scales validation accepts beyond head_dim^-0.5: zero
    (uniform attention over the keys; a masked key's -inf score times the scale must not become
    NaN), tiny and large. Grouped-query contiguous with a key count that leaves a partial last
    32-key block (decode_mma_kernel), one-head paged (decode_mma_kernel, 2 key/value heads) and
    four-head paged (decode_mma_rows_kernel, 8 key/value heads) with short sequences."""
    import torch

    B, heads, kv_heads, n = 2, 16, 4, 77
    q = synth.round_to(synth.normal(81, (B, heads, 1, d)), dtype)
    k = synth.round_to(synth.normal(82, (B, kv_heads, n, d)), dtype)
    v = synth.round_to(synth.normal(83, (B, kv_heads, n, d)), dtype)
    tq, tk, tv = (synth.to_torch(x, dtype) for x in (q, k, v))
    for splits in (0, 2):
        o, lse = cuflash_attn.flash_attention_decode(tq, tk, tv, scale=scale, num_splits=splits)
        torch.cuda.synchronize()
        o_ref, l_ref = oracle.forward(q, _expand_heads(k, heads // kv_heads),
                                      _expand_heads(v, heads // kv_heads), scale, False)
        check(dtype, synth.to_numpy(o), o_ref, f"O contiguous splits={splits}")
        check(dtype, synth.to_numpy(lse), l_ref, f"L contiguous splits={splits}")

    for kvh, page_size in ((2, 16), (8, 16)):
        hq = 4 * kvh
        seq_lens = [45, 1, 100]
        max_pages = 7
        k_pool, v_pool, table, seqs = _paged_case(dtype, d, len(seq_lens), hq, kvh, page_size,
                                                  max_pages, seq_lens, seed=90 + kvh)
        qp = synth.round_to(synth.normal(91, (len(seq_lens), hq, 1, d)), dtype)
        tqp, tkp, tvp = (synth.to_torch(x, dtype) for x in (qp, k_pool, v_pool))
        ttab = torch.from_numpy(table).to(tqp.device)
        tlen = torch.tensor(seq_lens, dtype=torch.int32, device=tqp.device)
        o, lse = cuflash_attn.flash_attention_decode_paged(tqp, tkp, tvp, ttab, tlen,
                                                           scale=scale, num_splits=0)
        torch.cuda.synchronize()
        o, lse = synth.to_numpy(o), synth.to_numpy(lse)
        for b in range(len(seq_lens)):
            kb, vb = seqs[b]
            o_ref, l_ref = oracle.forward(qp[b:b + 1], _expand_heads(kb[None], 4),
                                          _expand_heads(vb[None], 4), scale, False)
            check(dtype, o[b:b + 1], o_ref, f"O paged kv_heads={kvh} b={b}")
            check(dtype, lse[b:b + 1], l_ref, f"L paged kv_heads={kvh} b={b}")


@pytest.mark.gpu
def test_decode_gqa_matches_mha_on_repeated_heads(torch_gpu):
    """Grouped-query decode equals the plain decode of the head-repeated keys and values (same
    library, same split count) up to rounding: the grouped path (four query heads per key/value
    head, fp16, head_dim 128) runs the matrix-core kernel, which rounds P to fp16 for P V and
    rescales in 32-key blocks, where the plain kernel keeps P in fp32."""
    import torch

    B, heads, kv_heads, d, n = 2, 16, 4, 128, 3000
    q = synth.round_to(synth.normal(41, (B, heads, 1, d)), "float16")
    k = synth.round_to(synth.normal(42, (B, kv_heads, n, d)), "float16")
    v = synth.round_to(synth.normal(43, (B, kv_heads, n, d)), "float16")
    tq, tk, tv = (synth.to_torch(x, "float16") for x in (q, k, v))
    o1, l1 = cuflash_attn.flash_attention_decode(tq, tk, tv, num_splits=8)
    tk4 = torch.repeat_interleave(tk, heads // kv_heads, dim=1).contiguous()
    tv4 = torch.repeat_interleave(tv, heads // kv_heads, dim=1).contiguous()
    o2, l2 = cuflash_attn.flash_attention_decode(tq, tk4, tv4, num_splits=8)
    torch.cuda.synchronize()
    assert float((o1.float() - o2.float()).abs().max()) <= 1e-3
    assert float((l1 - l2).abs().max()) <= 1e-5
