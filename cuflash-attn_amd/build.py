"""Builds libcuflash_attn.so for gfx950 with hipcc.

The shared library lands in <repo>/build/libcuflash_attn.so, the first path the reference's test
caller searches (tests/integration/test_pytorch_comparison.py:158-180), with hidden default
visibility so that only the CUFLASH_EXPORT symbols are exported (reference CMakeLists.txt:60-72).
build/release/libcuflash_attn.so, a relative symbolic link to it, is the first path of the
reference's example caller (examples/python_binding.py:25-48), which does not look in build/.

Usage: python cuflash-attn_amd/build.py [--jobs N] [--install PREFIX]

--install PREFIX also installs the package the way the reference's CMake install does
(CMakeLists.txt:268-315): headers under PREFIX/include, the library under PREFIX/lib, and a
CMake package config under PREFIX/lib/cmake/cuflash_attn so that find_package(cuflash_attn
CONFIG) provides the imported target cuflash::cuflash_attn.
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_ROOT, "include")
BUILD_DIR = os.path.join(REPO_ROOT, "build")
LIB_NAME = "libcuflash_attn.so"
LIB_PATH = os.path.join(BUILD_DIR, LIB_NAME)
# build/release/ is where examples/python_binding.py:28 looks first (its CMake release preset).
RELEASE_LINK = os.path.join(BUILD_DIR, "release", LIB_NAME)

SOURCES = ["api.cpp", "profile.cpp", "workspace.cpp", "forward.hip", "backward.hip", "decode.hip",
           "primitives.hip"]
# C++ test programs linked against the library (sources under tests/cpp, binaries in build/).
TEST_PROGRAMS = {"test_primitives": "test_primitives.cpp"}
TEST_SRC = os.path.join(REPO_ROOT, "tests", "cpp")

# Packed-FP32 VALU forms are disabled for all device code (v_pk_{add,mul,fma}_f32).
COMMON_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-fvisibility-inlines-hidden",
    "-DCUFLASH_BUILDING_SHARED",
    "-I" + INCLUDE,
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# Per-source additions. forward.hip: LLVM's AMDGPU register-pressure trackers in the machine
# scheduler. Measured bitwise equal, 1-3% faster for the sequential head_dim-64 forward and level
# at head_dim 128; in backward.hip the same option spills fewer registers but ran 1% slower.
SOURCE_FLAGS = {
    "forward.hip": ["-mllvm", "-amdgpu-use-amdgpu-trackers=1"],
}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm is required to build libcuflash_attn)")
    return path


def _compile(src: str, obj: str) -> None:
    cmd = [hipcc(), "-x", "hip", *COMMON_FLAGS, *SOURCE_FLAGS.get(src, []), "-c",
           os.path.join(CSRC, src), "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stdout}\n{proc.stderr}")


def build(jobs: int = 4, verbose: bool = True) -> str:
    """Compiles every source and links build/libcuflash_attn.so. Returns the library path."""
    obj_dir = os.path.join(BUILD_DIR, "obj")
    os.makedirs(obj_dir, exist_ok=True)
    objs = [os.path.join(obj_dir, s.rsplit(".", 1)[0] + ".o") for s in SOURCES]
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        futures = [pool.submit(_compile, s, o) for s, o in zip(SOURCES, objs)]
        for f in futures:
            f.result()
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    _link_release()
    if verbose:
        print(f"built {LIB_PATH}")
    for name, src in TEST_PROGRAMS.items():
        out = os.path.join(BUILD_DIR, name)
        cmd = [hipcc(), "-x", "hip", "--offload-arch=gfx950", "-O2", "-std=c++17",
               "-I" + INCLUDE, os.path.join(TEST_SRC, src), "-x", "none", LIB_PATH,
               "-Wl,-rpath,$ORIGIN", "-o", out + ".tmp"]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{proc.stdout}\n{proc.stderr}")
        os.replace(out + ".tmp", out)
        if verbose:
            print(f"built {out}")
    return LIB_PATH


SANITIZE_DIR = os.path.join(BUILD_DIR, "sanitize")
SANITIZE_LIB = os.path.join(SANITIZE_DIR, LIB_NAME)
# AddressSanitizer + UndefinedBehaviorSanitizer on the host code only (the reference's
# ENABLE_ASAN / ENABLE_UBSAN options, CMakeLists.txt:32-33, 100-114): each -fsanitize= goes to
# the host compilation through -Xarch_host, so the gfx950 code objects are built exactly as in
# the release library. The library links the shared sanitizer runtime; a process that loads it
# must preload that runtime (sanitizer_runtime()).
SANITIZE_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                  "-Xarch_host", "-fno-sanitize-recover=undefined",
                  "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-g"]


def sanitizer_runtime() -> str:
    """ROCm's clang AddressSanitizer runtime (it carries the UBSan handlers as well)."""
    out = subprocess.run([hipcc(), "--print-file-name=libclang_rt.asan-x86_64.so"],
                         capture_output=True, text=True).stdout.strip()
    if not out or not os.path.exists(out):
        import glob

        hits = glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so")
        if not hits:
            raise RuntimeError("clang AddressSanitizer runtime not found")
        out = hits[0]
    return out


def build_sanitized(jobs: int = 4, verbose: bool = True) -> str:
    """The library with the host code under ASan + UBSan, in build/sanitize/. Returns its path."""
    obj_dir = os.path.join(SANITIZE_DIR, "obj")
    os.makedirs(obj_dir, exist_ok=True)
    objs = [os.path.join(obj_dir, s.rsplit(".", 1)[0] + ".o") for s in SOURCES]

    def comp(src, obj):
        cmd = [hipcc(), "-x", "hip", *COMMON_FLAGS, *SOURCE_FLAGS.get(src, []), *SANITIZE_FLAGS,
               "-c", os.path.join(CSRC, src), "-o", obj]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{proc.stdout}\n{proc.stderr}")

    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        for f in [pool.submit(comp, s, o) for s, o in zip(SOURCES, objs)]:
            f.result()
    tmp = SANITIZE_LIB + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-Xarch_host",
           "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined", "-Xarch_host",
           "-shared-libasan", *objs, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, SANITIZE_LIB)
    if verbose:
        print(f"built {SANITIZE_LIB}")
    # The GPU-side exercise of the sanitized host code (tests/cpp/host_sanitizer_driver.cpp),
    # itself instrumented and linked against the shared sanitizer runtime next to the library.
    runtime_dir = os.path.dirname(sanitizer_runtime())
    out = os.path.join(SANITIZE_DIR, "host_sanitizer_driver")
    cmd = [hipcc(), "-x", "hip", "--offload-arch=gfx950", "-O1", "-std=c++17", *SANITIZE_FLAGS,
           "-I" + INCLUDE, os.path.join(TEST_SRC, "host_sanitizer_driver.cpp"), "-x", "none",
           SANITIZE_LIB, "-Xarch_host", "-shared-libasan", "-Wl,-rpath,$ORIGIN",
           "-Wl,-rpath," + runtime_dir, "-lpthread", "-o", out + ".tmp"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for host_sanitizer_driver.cpp:\n{proc.stdout}\n{proc.stderr}")
    os.replace(out + ".tmp", out)
    if verbose:
        print(f"built {out}")
    return SANITIZE_LIB


def _link_release() -> None:
    """Points build/release/libcuflash_attn.so at ../libcuflash_attn.so (relative, so the link
    stays valid when the tree is copied elsewhere)."""
    os.makedirs(os.path.dirname(RELEASE_LINK), exist_ok=True)
    tmp = RELEASE_LINK + ".tmp"
    if os.path.lexists(tmp):
        os.remove(tmp)
    os.symlink(os.path.join("..", LIB_NAME), tmp)
    os.replace(tmp, RELEASE_LINK)


_CONFIG = """# cuflash_attn CMake package (installed by cuflash-attn_amd/build.py --install).
# Imported target cuflash::cuflash_attn: the prebuilt libcuflash_attn.so for gfx950 and its
# headers; consumers also get the HIP host runtime (hip::host) that the headers use.
include(CMakeFindDependencyMacro)
find_dependency(hip CONFIG PATHS /opt/rocm /opt/rocm/lib/cmake/hip)
get_filename_component(_cuflash_prefix "${CMAKE_CURRENT_LIST_DIR}/../../.." ABSOLUTE)
if(NOT TARGET cuflash::cuflash_attn)
  add_library(cuflash::cuflash_attn SHARED IMPORTED)
  set_target_properties(cuflash::cuflash_attn PROPERTIES
    IMPORTED_LOCATION "${_cuflash_prefix}/lib/libcuflash_attn.so"
    IMPORTED_SONAME "libcuflash_attn.so"
    INTERFACE_INCLUDE_DIRECTORIES "${_cuflash_prefix}/include"
    INTERFACE_LINK_LIBRARIES "hip::host")
endif()
unset(_cuflash_prefix)
"""

_CONFIG_VERSION = """set(PACKAGE_VERSION "@VERSION@")
if(PACKAGE_FIND_VERSION VERSION_GREATER PACKAGE_VERSION)
  set(PACKAGE_VERSION_COMPATIBLE FALSE)
else()
  set(PACKAGE_VERSION_COMPATIBLE TRUE)
  if(PACKAGE_FIND_VERSION STREQUAL PACKAGE_VERSION)
    set(PACKAGE_VERSION_EXACT TRUE)
  endif()
endif()
"""


def install(prefix: str, verbose: bool = True) -> str:
    """Copies the built library and the public headers under `prefix` and writes the CMake
    package config. Returns the config directory."""
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build first")
    inc_dst = os.path.join(prefix, "include", "cuflash")
    shutil.copytree(os.path.join(INCLUDE, "cuflash"), inc_dst, dirs_exist_ok=True)
    lib_dir = os.path.join(prefix, "lib")
    os.makedirs(lib_dir, exist_ok=True)
    shutil.copy2(LIB_PATH, os.path.join(lib_dir, LIB_NAME))
    cfg_dir = os.path.join(lib_dir, "cmake", "cuflash_attn")
    os.makedirs(cfg_dir, exist_ok=True)
    with open(os.path.join(INCLUDE, "cuflash", "version.h")) as f:
        version = next(line.split('"')[1] for line in f if line.startswith("#define CUFLASH_VERSION "))
    with open(os.path.join(cfg_dir, "cuflash_attnConfig.cmake"), "w") as f:
        f.write(_CONFIG)
    with open(os.path.join(cfg_dir, "cuflash_attnConfigVersion.cmake"), "w") as f:
        f.write(_CONFIG_VERSION.replace("@VERSION@", version))
    if verbose:
        print(f"installed into {prefix}")
    return cfg_dir


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--install", metavar="PREFIX", default=None)
    ap.add_argument("--sanitize", action="store_true",
                    help="build build/sanitize/libcuflash_attn.so, host code under ASan + UBSan")
    args = ap.parse_args()
    try:
        if args.sanitize:
            build_sanitized(args.jobs)
            sys.exit(0)
        build(args.jobs)
        if args.install:
            install(args.install)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
