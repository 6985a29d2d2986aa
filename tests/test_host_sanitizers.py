"""The CPU suite again, against the library built with the host code under AddressSanitizer and
UndefinedBehaviorSanitizer (the reference's ENABLE_ASAN / ENABLE_UBSAN builds,
CMakeLists.txt:32-33, 100-114, 175-184). No GPU is used.

build.py --sanitize compiles every source with `-Xarch_host -fsanitize=address` and
`-Xarch_host -fsanitize=undefined` (unrecoverable), so the host side of the library is
instrumented: the C ABI and its validation (api.cpp), the profiling hook (profile.cpp), the
workspace cache (workspace.cpp) and the host code of the kernel sources up to their first HIP
call. The gfx950 code objects are the release ones. The suite runs in a child process that
preloads clang's ASan runtime (Python itself is not instrumented) and selects the sanitized
library through $CUFLASH_LIB, with leak detection off (the interpreter keeps its allocations
until exit) and every report fatal. Without a GPU the host paths reached are those of the CPU
suite: symbol exports, error strings, every validation path of every entry point, library
search and loading.
"""

from __future__ import annotations

import os
import subprocess
import sys

import pytest

from conftest import PKG, REPO

CHILD = os.environ.get("CUFLASH_SANITIZER_RUN") == "1"


def _sanitized_library():
    sys.path.insert(0, PKG)
    import build as cuflash_build  # cuflash-attn_amd/build.py

    lib = cuflash_build.SANITIZE_LIB
    srcs = [os.path.join(cuflash_build.CSRC, s) for s in os.listdir(cuflash_build.CSRC)]
    srcs += [os.path.join(REPO, "include", "cuflash", f)
             for f in os.listdir(os.path.join(REPO, "include", "cuflash")) if f.endswith(".h")]
    newest = max(os.path.getmtime(p) for p in srcs if os.path.isfile(p))
    if not os.path.exists(lib) or os.path.getmtime(lib) < newest:
        cuflash_build.build_sanitized(jobs=4, verbose=False)
    return lib, cuflash_build.sanitizer_runtime()


@pytest.mark.skipif(CHILD, reason="this is the sanitized run itself")
def test_cpu_suite_under_host_asan_ubsan():
    lib, runtime = _sanitized_library()
    syms = subprocess.run(["nm", "-D", lib], capture_output=True, text=True, check=True).stdout
    assert "__asan_report_load" in syms and "__ubsan_handle_" in syms, "not instrumented"
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": runtime,
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=0",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
        "CUFLASH_LIB": lib,
        "CUFLASH_SANITIZER_RUN": "1",
    })
    proc = subprocess.run(
        [sys.executable, "-m", "pytest", os.path.join(REPO, "tests"), "-q", "-m", "not gpu",
         "-p", "no:cacheprovider"],
        cwd=REPO, env=env, capture_output=True, text=True, timeout=900)
    out = proc.stdout + proc.stderr
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert proc.returncode == 0, out[-4000:]
    assert " passed" in out
