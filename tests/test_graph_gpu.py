"""HIP graph capture of the allocating entry points: forward + backward, and the plain,
grouped-query and paged decodes.

Each captured sequence is replayed three times with new inputs written between the replays (the
program's own eager work and a synchronization between them), and every replay is compared
bitwise with the same calls run eagerly on the same inputs (the kernels are deterministic).
Inside a capture the library takes per-call workspaces, a stream-ordered allocation and free that
the graph records, instead of the capturing stream's cached buffer, which later calls could
replace while the graph still refers to it. The kernels record no memset.
"""

from __future__ import annotations

import pytest


def _capture(torch, fn):
    """Warm-up on a side stream, then capture fn() into a graph."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    return graph


def _refill(torch, tensors, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    for t in tensors:
        t.copy_(torch.randn(t.shape, generator=g, device="cuda", dtype=torch.float32).to(t.dtype))


@pytest.mark.gpu
def test_forward_backward_in_a_captured_graph(torch_gpu):
    import cuflash_attn

    torch = torch_gpu
    B, H, N, D = 1, 4, 1024, 128
    q, k, v, do = (torch.empty((B, H, N, D), device="cuda", dtype=torch.bfloat16)
                   for _ in range(4))
    _refill(torch, (q, k, v, do), 1)
    static = {}

    def step():
        o, lse = cuflash_attn.flash_attention_forward(q, k, v, causal=True)
        dq, dk, dv = cuflash_attn.flash_attention_backward(q, k, v, o, lse, do, causal=True)
        static["out"] = (o, lse, dq, dk, dv)

    graph = _capture(torch, step)
    for rep in range(3):
        print(f"[graph fwd+bwd] replay {rep}", flush=True)
        _refill(torch, (q, k, v, do), 10 + rep)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in static["out"]]
        o, lse = cuflash_attn.flash_attention_forward(q, k, v, causal=True)
        ref = [o, lse, *cuflash_attn.flash_attention_backward(q, k, v, o, lse, do, causal=True)]
        torch.cuda.synchronize()
        for name, a, b in zip(("O", "L", "dQ", "dK", "dV"), got, ref):
            assert torch.equal(a, b), f"replay {rep}: {name}"
    del graph


@pytest.mark.gpu
def test_decodes_in_a_captured_graph(torch_gpu):
    import cuflash_attn

    torch = torch_gpu
    B, H, HKV, L, D, page = 2, 16, 4, 3000, 128, 16
    q = torch.empty((B, H, 1, D), device="cuda", dtype=torch.float16)
    k, v = (torch.empty((B, H, L, D), device="cuda", dtype=torch.float16) for _ in range(2))
    kg, vg = (torch.empty((B, HKV, L, D), device="cuda", dtype=torch.float16) for _ in range(2))
    maxp = (L + page - 1) // page
    kp, vp = (torch.empty((B * maxp, page, HKV, D), device="cuda", dtype=torch.float16)
              for _ in range(2))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    table = torch.randperm(B * maxp, generator=gen, device="cuda").to(torch.int32)
    table = table.reshape(B, maxp).contiguous()
    lens = torch.tensor([L, L - 777], dtype=torch.int32, device="cuda")
    inputs = (q, k, v, kg, vg, kp, vp)
    _refill(torch, inputs, 2)
    static = {}

    def calls():
        return [*cuflash_attn.flash_attention_decode(q, k, v, num_splits=16),
                *cuflash_attn.flash_attention_decode(q, kg, vg),
                *cuflash_attn.flash_attention_decode_paged(q, kp, vp, table, lens)]

    def step():
        static["out"] = calls()

    graph = _capture(torch, step)
    for rep in range(3):
        print(f"[graph decode] replay {rep}", flush=True)
        _refill(torch, inputs, 20 + rep)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in static["out"]]
        ref = calls()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(got, ref)):
            assert torch.equal(a, b), f"replay {rep}: output {i}"
    del graph
