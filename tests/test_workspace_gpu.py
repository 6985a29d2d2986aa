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
