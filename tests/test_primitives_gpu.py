"""GPU tests of the primitive layer cuflash::kernels::* (matmul, online softmax, tile I/O).

The checks live in tests/cpp/test_primitives.cpp, a C++ program built with the library
(cuflash-attn_amd/build.py -> build/test_primitives) that calls the C++ API the way the
reference's tests/unit/test_{matmul,online_softmax,tile_io}.cu do, with their shapes, inputs
and tolerances. Each group runs in its own process and must report zero failures.
"""

from __future__ import annotations

import os
import subprocess

import pytest

from conftest import REPO

BINARY = os.path.join(REPO, "build", "test_primitives")


def _gpu_count() -> int:
    import torch

    return torch.cuda.device_count()  # does not initialize the GPU in this process


@pytest.mark.gpu
@pytest.mark.parametrize("group", ["matmul", "softmax", "tile"])
def test_primitive_group(group):
    if _gpu_count() == 0:
        pytest.skip("no GPU")
    assert os.path.exists(BINARY), "build/test_primitives is missing: run cuflash-attn_amd/build.py"
    proc = subprocess.run([BINARY, group], capture_output=True, text=True, timeout=120,
                          close_fds=True)
    out = proc.stdout + proc.stderr
    assert proc.returncode == 0, out[-4000:]
    assert " 0 failed" in out, out[-4000:]
