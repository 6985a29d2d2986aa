"""The library's host code on the GPU under AddressSanitizer and UndefinedBehaviorSanitizer.

build/sanitize/host_sanitizer_driver (tests/cpp/host_sanitizer_driver.cpp, built by
`cuflash-attn_amd/build.py --sanitize`) links build/sanitize/libcuflash_attn.so, whose host code
is compiled with -fsanitize=address,undefined and whose gfx950 code is the release code. It runs
every entry point on small shapes against a naive attention, the per-stream workspace cache on
several streams and host threads (with cuflash_release_workspaces() called meanwhile), the
profiling hook and the allocation-free decode. A sanitizer report or a failed check fails the
test. The CPU-only half (every validation path) is tests/test_host_sanitizers.py.
"""

from __future__ import annotations

import os
import subprocess

import pytest

from conftest import REPO

BINARY = os.path.join(REPO, "build", "sanitize", "host_sanitizer_driver")


@pytest.mark.gpu
def test_gpu_paths_under_host_asan_ubsan():
    import torch

    if torch.cuda.device_count() == 0:  # does not initialize the GPU in this process
        pytest.skip("no GPU")
    assert os.path.exists(BINARY), "run `python cuflash-attn_amd/build.py --sanitize` first"
    env = dict(os.environ)
    env.update({
        # leaks: the HIP runtime keeps allocations until exit; link order: a preloaded library
        # may precede the runtime, which the program itself links
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=0:verify_asan_link_order=0",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
    })
    proc = subprocess.run([BINARY], capture_output=True, text=True, timeout=240, env=env,
                          close_fds=True)
    out = proc.stdout + proc.stderr
    print(out[-3000:])
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-6000:]
    assert proc.returncode == 0, out[-6000:]
    assert " 0 failed" in out, out[-4000:]
