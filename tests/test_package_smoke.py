"""Installed-package check (host only): build.py --install into a temporary prefix, then a CMake
consumer (tests/package_smoke, as the reference's tests/package_smoke) finds the package with
find_package(cuflash_attn CONFIG), links cuflash::cuflash_attn and runs a validation-only call."""

from __future__ import annotations

import importlib.util
import os
import shutil
import subprocess

import pytest

from conftest import REPO

SMOKE = os.path.join(REPO, "tests", "package_smoke")


def _build_module():
    spec = importlib.util.spec_from_file_location(
        "cuflash_build", os.path.join(REPO, "cuflash-attn_amd", "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.skipif(shutil.which("cmake") is None, reason="cmake not available")
def test_installed_package_is_found_and_links(tmp_path):
    build = _build_module()
    if not os.path.exists(build.LIB_PATH):
        pytest.skip("library not built")
    prefix = tmp_path / "prefix"
    build.install(str(prefix), verbose=False)
    assert (prefix / "include" / "cuflash" / "flash_attention.h").exists()
    assert (prefix / "include" / "cuflash" / "kernels" / "tile_io.cuh").exists()
    assert (prefix / "lib" / "libcuflash_attn.so").exists()
    bdir = tmp_path / "build"
    env = dict(os.environ, CXX=shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
    cfg = subprocess.run(["cmake", "-S", SMOKE, "-B", str(bdir), f"-DCMAKE_PREFIX_PATH={prefix}",
                          "-DCMAKE_BUILD_TYPE=Release"], capture_output=True, text=True, env=env,
                         timeout=300)
    assert cfg.returncode == 0, cfg.stdout[-3000:] + cfg.stderr[-3000:]
    bld = subprocess.run(["cmake", "--build", str(bdir), "-j", "4"], capture_output=True,
                         text=True, timeout=300)
    assert bld.returncode == 0, bld.stdout[-3000:] + bld.stderr[-3000:]
    run = subprocess.run([str(bdir / "cuflash_attn_package_smoke")], capture_output=True,
                         text=True, timeout=60)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.strip() == "Success 0.6.0"
