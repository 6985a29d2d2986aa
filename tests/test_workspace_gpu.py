"""The stream-ordered workspace's failure path on the GPU.

The reference maps a failed stream-ordered allocation of its backward workspace to
OUT_OF_MEMORY (src/backward/flash_attention_backward_typed.cu:380-384, AsyncFloatBuffer). This
library's StreamWorkspace does the same for every launcher that needs one; these tests make the
request larger than the device and check the status, that no kernel ran (the outputs keep their
sentinel values), and that the library and the device work normally afterwards.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import cuflash_attn
import oracle
from conftest import max_abs
from cuflash_attn import synth


@pytest.mark.gpu
def test_decode_workspace_larger_than_the_device_returns_out_of_memory(torch_gpu, lib):
    torch = torch_gpu
    _, total = torch.cuda.mem_get_info()
    # Grouped-query decode of H query heads over one key/value head of kv_len keys: the split
    # partials take H * splits * (D + 2) fp32 while the inputs stay small. An explicit request
    # is clamped to ceil(kv_len / 16) splits, so kv_len = 16384 keeps all 1024.
    D, kv_len, splits = 128, 16384, 1024
    per_head = splits * (D + 2) * 4
    H = ((2 * total) // per_head + 7) // 8 * 8
    assert H * per_head > total and H < 2 ** 31
    print(f"[oom] H={H} workspace={H * per_head / 2**30:.1f} GiB device={total / 2**30:.1f} GiB",
          flush=True)
    q = torch.zeros((1, H, 1, D), dtype=torch.float16, device="cuda")
    k = torch.zeros((1, 1, kv_len, D), dtype=torch.float16, device="cuda")
    v = torch.zeros_like(k)
    o = torch.full((1, H, 1, D), 7.0, dtype=torch.float16, device="cuda")
    lse = torch.full((1, H, 1), 7.0, dtype=torch.float32, device="cuda")
    fn = lib.fn("decode_gqa", "f16")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    status = fn(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), 1, H, 1,
                kv_len, D, D ** -0.5, splits, stream)
    assert status == cuflash_attn.OUT_OF_MEMORY, (status, lib.error_string(status))
    assert lib.error_string(status) == "Out of memory: insufficient GPU memory"
    torch.cuda.synchronize()
    assert bool((o == 7.0).all()) and bool((lse == 7.0).all()), "a kernel ran"
    del q, k, v, o, lse
    torch.cuda.empty_cache()

    # the next call on the same stream works and is correct
    qh = synth.round_to(synth.normal(5, (1, 4, 1, D)), "float16")
    kh, vh = (synth.round_to(synth.normal(s, (1, 4, 700, D)), "float16") for s in (6, 7))
    od, ld = cuflash_attn.flash_attention_decode(*(synth.to_torch(x, "float16")
                                                   for x in (qh, kh, vh)), num_splits=16)
    torch.cuda.synchronize()
    o_ref, l_ref = oracle.forward(qh, kh, vh, D ** -0.5, False)
    assert max_abs(synth.to_numpy(od), o_ref) <= 2e-2
    assert max_abs(synth.to_numpy(ld), l_ref) <= 2e-2
    assert np.isfinite(synth.to_numpy(ld)).all()


def _bwd_case(torch, n, seed, h=4):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    q, k, v, do = (torch.randn((1, h, n, 128), generator=g, device="cuda").to(torch.bfloat16)
                   for _ in range(4))
    return q, k, v, do


@pytest.mark.gpu
def test_cached_workspace_grows_and_is_reused_in_stream_order(torch_gpu):
    """The backward's and decode's workspaces are one cached buffer per stream: calls of
    growing and shrinking size on one stream, back to back with no synchronization, give the
    results of the same calls made one at a time with a synchronization after each."""
    torch = torch_gpu
    sizes = [64, 2048, 300, 4096, 1000]
    cases = [_bwd_case(torch, n, 30 + i) for i, n in enumerate(sizes)]
    ref = []
    for q, k, v, do in cases:
        o, lse = cuflash_attn.flash_attention_forward(q, k, v, causal=True)
        g = cuflash_attn.flash_attention_backward(q, k, v, o, lse, do, causal=True)
        torch.cuda.synchronize()
        ref.append((o, lse) + tuple(g))
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        got = []
        for q, k, v, do in cases:
            o, lse = cuflash_attn.flash_attention_forward(q, k, v, causal=True)
            got.append((o, lse) + tuple(cuflash_attn.flash_attention_backward(
                q, k, v, o, lse, do, causal=True)))
        # decode partials share the stream's buffer: small, large, small
        dec = []
        for bh, kv_len, splits in ((2, 512, 4), (64, 32768, 64), (4, 100, 2)):
            g = torch.Generator(device="cuda")
            g.manual_seed(kv_len)
            qd = torch.randn((1, bh, 1, 128), generator=g, device="cuda").half()
            kd = torch.randn((1, bh, kv_len, 128), generator=g, device="cuda").half()
            vd = torch.randn((1, bh, kv_len, 128), generator=g, device="cuda").half()
            dec.append(((qd, kd, vd, splits),
                        cuflash_attn.flash_attention_decode(qd, kd, vd, num_splits=splits)))
    torch.cuda.synchronize()
    for r, g in zip(ref, got):
        for a, b in zip(r, g):
            assert torch.equal(a, b)
    for (args, (o, lse)) in dec:
        o2, l2 = cuflash_attn.flash_attention_decode(*args[:3], num_splits=args[3])
        torch.cuda.synchronize()
        assert torch.equal(o, o2) and torch.equal(lse, l2)


@pytest.mark.gpu
def test_concurrent_host_threads_on_one_stream(torch_gpu):
    """Host threads that call the backward on the same stream at the same time, with different
    workspace sizes (so the stream's cached buffer grows while other calls use it), get the
    results of serial calls. ctypes releases the interpreter lock during each call."""
    import threading

    torch = torch_gpu
    sizes = [128, 4096, 512, 2048, 256, 3000]
    cases = [_bwd_case(torch, n, 60 + i, h=8) for i, n in enumerate(sizes)]
    fwd = []
    for q, k, v, do in cases:
        fwd.append(cuflash_attn.flash_attention_forward(q, k, v, causal=True))
    torch.cuda.synchronize()
    ref = []
    for (q, k, v, do), (o, lse) in zip(cases, fwd):
        ref.append(cuflash_attn.flash_attention_backward(q, k, v, o, lse, do, causal=True))
        torch.cuda.synchronize()
    lib = cuflash_attn.load_library()
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    outs = [[torch.empty_like(c[0]) for _ in range(3)] for c in cases]
    errors = []

    def worker(i):
        q, k, v, do = cases[i]
        o, lse = fwd[i]
        fn = lib.fn("backward", "bf16")
        for _ in range(5):
            st = fn(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                    do.data_ptr(), outs[i][0].data_ptr(), outs[i][1].data_ptr(),
                    outs[i][2].data_ptr(), 1, 8, q.shape[2], 128, 128 ** -0.5, True, sp)
            if st != 0:
                errors.append((i, st))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(cases))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for r, g in zip(ref, outs):
        for a, b in zip(r, g):
            assert torch.equal(a, b)


@pytest.mark.gpu
def test_many_streams_past_the_cache_bound_and_release(torch_gpu):
    """Ten streams whose decode partials need a 34 MB workspace each: the cached buffers stop at
    256 MiB per device, so the later streams run with per-call workspaces. Every stream's result
    equals the serial call's; cuflash_release_workspaces() then returns 0 and calls made
    afterwards (which cache afresh) give the same results again."""
    torch = torch_gpu
    lib = cuflash_attn.load_library()
    H, kv_len, D, splits = 1024, 1024, 128, 64  # partials 1024 * 64 * 130 * 4 B = 34 MB
    g = torch.Generator(device="cuda")
    g.manual_seed(77)
    q = torch.randn((1, H, 1, D), generator=g, device="cuda").half()
    k = torch.randn((1, H, kv_len, D), generator=g, device="cuda").half()
    v = torch.randn((1, H, kv_len, D), generator=g, device="cuda").half()
    o_ref, l_ref = cuflash_attn.flash_attention_decode(q, k, v, num_splits=splits)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(10)]
    outs = []
    for s in streams:
        with torch.cuda.stream(s):
            outs.append(cuflash_attn.flash_attention_decode(q, k, v, num_splits=splits))
    torch.cuda.synchronize()
    for o, lse in outs:
        assert torch.equal(o, o_ref) and torch.equal(lse, l_ref)
    assert lib.library.cuflash_release_workspaces() == 0
    for s in streams[:3]:
        with torch.cuda.stream(s):
            o, lse = cuflash_attn.flash_attention_decode(q, k, v, num_splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref) and torch.equal(lse, l_ref)
    assert lib.library.cuflash_release_workspaces() == 0


@pytest.mark.gpu
def test_release_while_other_threads_call(torch_gpu):
    """cuflash_release_workspaces() from one host thread while four others run decodes on their
    own streams: every release returns 0 or CUDA_ERROR (a buffer in use by a call is kept), and
    every decode result equals the serial call's."""
    import threading

    torch = torch_gpu
    lib = cuflash_attn.load_library()
    H, kv_len, D, splits = 64, 2048, 128, 16
    g = torch.Generator(device="cuda")
    g.manual_seed(78)
    q = torch.randn((2, H, 1, D), generator=g, device="cuda").half()
    k = torch.randn((2, H, kv_len, D), generator=g, device="cuda").half()
    v = torch.randn((2, H, kv_len, D), generator=g, device="cuda").half()
    o_ref, l_ref = cuflash_attn.flash_attention_decode(q, k, v, num_splits=splits)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(4)]
    outs = [[(torch.empty_like(o_ref), torch.empty_like(l_ref)) for _ in range(20)]
            for _ in streams]
    fn = lib.fn("decode", "f16")
    errors, codes = [], []
    done = threading.Event()

    def worker(i):
        sp = streams[i].cuda_stream
        for o, lse in outs[i]:
            st = fn(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), 2, H,
                    kv_len, D, D ** -0.5, splits, sp)
            if st != 0:
                errors.append((i, st))

    def releaser():
        while not done.is_set():
            codes.append(lib.library.cuflash_release_workspaces())

    rel = threading.Thread(target=releaser)
    rel.start()
    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(streams))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    done.set()
    rel.join()
    torch.cuda.synchronize()
    assert not errors, errors
    assert codes and set(codes) <= {0, 4}, sorted(set(codes))
    for per_stream in outs:
        for o, lse in per_stream:
            assert torch.equal(o, o_ref) and torch.equal(lse, l_ref)
    assert lib.library.cuflash_release_workspaces() == 0
