"""cuflash_attention_decode_noalloc_f16: decode whose split partials live in the library's fixed
per-GPU device array instead of an allocated workspace.

It runs the kernels of cuflash_attention_decode_f16 with the same split count, so its O and L
must equal that entry point's bitwise (and therefore meet the 2e-2 fp16 bar against the oracle
that test_parity_gpu.py and test_configs_gpu.py hold decode_f16 to). Two calls in a row, the
second smaller, check that a call does not depend on what the previous one left in the array;
a request larger than the array returns OUT_OF_MEMORY with no device work.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import cuflash_attn
import oracle
from conftest import max_abs
from cuflash_attn import synth

SCRATCH_BYTES = 32 << 20


def _noalloc(lib):
    fn = lib.library.cuflash_attention_decode_noalloc_f16
    fn.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 4 + [ctypes.c_float, ctypes.c_int,
                                                                ctypes.c_void_p]
    fn.restype = ctypes.c_int
    return fn


def _inputs(torch, b, h, kv_len, d, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    q = torch.randn((b, h, 1, d), generator=g, device="cuda", dtype=torch.float32).half()
    k = torch.randn((b, h, kv_len, d), generator=g, device="cuda", dtype=torch.float16)
    v = torch.randn((b, h, kv_len, d), generator=g, device="cuda", dtype=torch.float16)
    return q, k, v


def _both(torch, lib, q, k, v, splits):
    """O, L from decode_f16 and from decode_noalloc_f16 on the same inputs and stream."""
    b, h, _, d = q.shape
    kv_len = k.shape[2]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    outs = []
    for fn in (lib.fn("decode", "f16"), _noalloc(lib)):
        o = torch.full_like(q, float("nan"))
        lse = torch.full((b, h, 1), float("nan"), device="cuda", dtype=torch.float32)
        st = fn(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), b, h,
                kv_len, d, d ** -0.5, splits, stream)
        assert st == 0, lib.error_string(st)
        outs.append((o, lse))
    torch.cuda.synchronize()
    return outs


@pytest.mark.gpu
def test_noalloc_decode_equals_decode_on_two_calls(torch_gpu, lib):
    torch = torch_gpu
    # call 1: config 4's shape at 64 splits (16.3 MiB of partials); call 2: a smaller decode
    cases = [(16, 32, 32768, 128, 64, 1), (2, 4, 777, 64, 16, 2)]
    for b, h, kv_len, d, splits, seed in cases:
        print(f"[noalloc] B={b} H={h} kv_len={kv_len} D={d} splits={splits}", flush=True)
        q, k, v = _inputs(torch, b, h, kv_len, d, seed)
        (o1, l1), (o2, l2) = _both(torch, lib, q, k, v, splits)
        assert torch.equal(o1, o2) and torch.equal(l1, l2)
        assert bool(torch.isfinite(o2.float()).all()) and bool(torch.isfinite(l2).all())
        qh, kh, vh = (synth.to_numpy(x[:1, :1]) for x in (q, k, v))
        o_ref, l_ref = oracle.forward(qh, kh, vh, d ** -0.5, False)
        assert max_abs(synth.to_numpy(o2[:1, :1]), o_ref) <= 2e-2
        assert max_abs(synth.to_numpy(l2[:1, :1]), l_ref) <= 2e-2
        del q, k, v
        torch.cuda.empty_cache()


@pytest.mark.gpu
def test_noalloc_decode_rejects_partials_beyond_the_array(torch_gpu, lib):
    torch = torch_gpu
    # 64 heads x 1024 splits x (128 + 2) x 4 bytes = 34.1 MB > 32 MiB
    b, h, kv_len, d, splits = 1, 64, 16384, 128, 1024
    assert b * h * splits * (d + 2) * 4 > SCRATCH_BYTES
    q, k, v = _inputs(torch, b, h, kv_len, d, 3)
    o = torch.full_like(q, 7.0)
    lse = torch.full((b, h, 1), 7.0, device="cuda", dtype=torch.float32)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    st = _noalloc(lib)(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), b,
                       h, kv_len, d, d ** -0.5, splits, stream)
    assert st == cuflash_attn.OUT_OF_MEMORY, lib.error_string(st)
    torch.cuda.synchronize()
    assert bool((o == 7.0).all()) and bool((lse == 7.0).all()), "a kernel ran"
    # 512 splits fit (17.0 MB) and match decode_f16
    (o1, l1), (o2, l2) = _both(torch, lib, q, k, v, 512)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_noalloc_validation_matches_decode(lib):
    """Validation errors come back before any device work, as for decode_f16."""
    buf = (ctypes.c_float * 16)()
    p = ctypes.addressof(buf)
    fn = _noalloc(lib)
    ref = lib.fn("decode", "f16")
    cases = [
        (None, p, p, p, p, 1, 1, 8, 64, 0.1, 0),   # null Q
        (p, p, p, p, p, 0, 1, 8, 64, 0.1, 0),      # batch 0
        (p, p, p, p, p, 1, 1, 8, 80, 0.1, 0),      # head_dim 80
        (p, p, p, p, p, 1, 1, 8, 64, -1.0, 0),     # negative scale
        (p, p, p, p, p, 1, 1, 8, 64, 0.1, -1),     # negative splits
    ]
    for args in cases:
        got = fn(*args, None)
        assert got != 0 and got == ref(*args, None), args


@pytest.mark.gpu
def test_noalloc_decode_in_a_captured_graph(torch_gpu, lib):
    """The entry point that allocates nothing, captured in a HIP graph (torch.cuda.CUDAGraph: its
    two kernels, no allocation and no memset) and replayed three times, with new queries written
    into its input and a synchronization between the replays; every replay equals
    cuflash_attention_decode_f16 run eagerly on the same inputs, bitwise."""
    torch = torch_gpu
    b, h, kv_len, d, splits = 2, 8, 4096, 128, 16
    q, k, v = _inputs(torch, b, h, kv_len, d, 11)
    o = torch.full_like(q, float("nan"))
    lse = torch.full((b, h, 1), float("nan"), device="cuda", dtype=torch.float32)
    fn = _noalloc(lib)

    def launch():
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        st = fn(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), b, h,
                kv_len, d, d ** -0.5, splits, stream)
        assert st == 0, lib.error_string(st)

    # Warm-up on a side stream (the first call on a device looks up the array's address).
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch()
    g = torch.Generator(device="cuda")
    for rep in range(3):
        print(f"[noalloc graph] replay {rep}", flush=True)
        g.manual_seed(100 + rep)
        q.copy_(torch.randn(q.shape, generator=g, device="cuda", dtype=torch.float32).half())
        o.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        (o_ref, l_ref), _ = _both(torch, lib, q, k, v, splits)
        assert torch.equal(o, o_ref) and torch.equal(lse, l_ref), f"replay {rep}"
    del graph
