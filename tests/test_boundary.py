"""C-ABI boundary checks that need no GPU.

Mirrors the host-only parts of the reference's tests: tests/integration/test_api_smoke.cpp:11-41
(validation errors returned before any device work), tests/unit/test_error_handling.cu:21-253
(error codes and exact strings) and tests/unit/test_stress_edge_cases.cu:124-175. Every call
here fails validation, so the library returns before its first HIP call.
"""

from __future__ import annotations

import ctypes
import math
import os
import re
import subprocess

import pytest

import cuflash_attn
from conftest import REPO

HEADER = os.path.join(REPO, "include", "cuflash", "flash_attention.h")

# The default search order is only what decides the library when $CUFLASH_LIB (the reference
# caller's override, test_pytorch_comparison.py:158-180) does not name one, as in the run of
# this suite against the sanitizer build (tests/test_host_sanitizers.py).
default_search_only = pytest.mark.skipif(
    bool(os.environ.get("CUFLASH_LIB")),
    reason="$CUFLASH_LIB names the library; the default search order is checked without it")


def _declared_c_symbols():
    text = open(HEADER).read()
    c_part = text[text.index('extern "C"'):]
    return sorted(set(re.findall(r"CUFLASH_EXPORT\s+[\w\s\*]+?\b(cuflash_\w+)\s*\(", c_part)))


@default_search_only
def test_library_loads_from_reference_search_path(lib):
    assert lib.path.endswith(os.path.join("build", "libcuflash_attn.so"))
    assert lib.version() == "0.6.0"


def test_every_declared_symbol_is_exported(lib):
    declared = _declared_c_symbols()
    assert len(declared) == 27, declared
    out = subprocess.run(["nm", "-D", "--defined-only", lib.path], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    for sym in declared:
        assert sym in exported, sym
        assert getattr(lib.library, sym) is not None
    assert set(declared) == set(cuflash_attn.EXPORTED_SYMBOLS)


def test_only_the_public_api_is_exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", "-C", lib.path], capture_output=True,
                         text=True, check=True).stdout
    names = [line.split(" ", 2)[-1] for line in out.splitlines() if " T " in line]
    for n in names:
        assert n.startswith("cuflash"), n  # C ABI or the cuflash:: C++ API, nothing internal


# Reference src/api/flash_attention_api.cu:21-42, checked verbatim by test_error_handling.cu:236-250.
EXPECTED_STRINGS = {
    0: "Success",
    1: "Invalid dimension: dimensions must be positive",
    2: "Dimension mismatch: Q, K, V tensors have incompatible shapes",
    3: "Null pointer: input or output pointer is null",
    4: "CUDA error occurred",
    5: "Out of memory: insufficient GPU memory",
    6: "Unsupported head_dim: must be 32, 64, or 128",
    7: "Unsupported data type",
    8: "Unknown error",
    -1: "Unknown error",
}


@pytest.mark.parametrize("code", sorted(EXPECTED_STRINGS))
def test_error_strings(lib, code):
    assert lib.error_string(code) == EXPECTED_STRINGS[code]


# Host buffers stand in for device pointers: validation never dereferences them.
_BUF = (ctypes.c_float * 16)()
P = ctypes.addressof(_BUF)


def _fwd(lib, sfx, ptrs, b=1, h=1, n=16, d=32, scale=1.0, causal=False):
    return lib.fn("forward", sfx)(*ptrs, b, h, n, d, scale, causal, None)


def _bwd(lib, sfx, ptrs, b=1, h=1, n=16, d=32, scale=1.0, causal=False):
    return lib.fn("backward", sfx)(*ptrs, b, h, n, d, scale, causal, None)


@pytest.mark.parametrize("sfx", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("null_idx", range(5))
def test_forward_null_pointers(lib, sfx, null_idx):
    ptrs = [P] * 5
    ptrs[null_idx] = None
    assert _fwd(lib, sfx, ptrs) == cuflash_attn.NULL_POINTER


@pytest.mark.parametrize("sfx", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("null_idx", range(9))
def test_backward_null_pointers(lib, sfx, null_idx):
    ptrs = [P] * 9
    ptrs[null_idx] = None
    assert _bwd(lib, sfx, ptrs) == cuflash_attn.NULL_POINTER


@pytest.mark.parametrize("dims", [(0, 1, 16, 32), (-1, 1, 16, 32), (1, 0, 16, 32),
                                  (1, 1, 0, 32), (1, 1, 16, 0), (1, 1, -5, 64)])
@pytest.mark.parametrize("sfx", ["f32", "f16", "bf16"])
def test_invalid_dimensions(lib, sfx, dims):
    b, h, n, d = dims
    assert _fwd(lib, sfx, [P] * 5, b, h, n, d) == cuflash_attn.INVALID_DIMENSION
    assert _bwd(lib, sfx, [P] * 9, b, h, n, d) == cuflash_attn.INVALID_DIMENSION


@pytest.mark.parametrize("d", [48, 256, 16, 96, 1])
def test_unsupported_head_dim(lib, d):
    for sfx in ("f32", "f16", "bf16"):
        assert _fwd(lib, sfx, [P] * 5, d=d) == cuflash_attn.UNSUPPORTED_HEAD_DIM
        assert _bwd(lib, sfx, [P] * 9, d=d) == cuflash_attn.UNSUPPORTED_HEAD_DIM


@pytest.mark.parametrize("scale", [math.nan, math.inf, -math.inf, -1.0, -1e-30])
def test_invalid_scale(lib, scale):
    for sfx in ("f32", "f16", "bf16"):
        assert _fwd(lib, sfx, [P] * 5, scale=scale) == cuflash_attn.INVALID_DIMENSION
        assert _bwd(lib, sfx, [P] * 9, scale=scale) == cuflash_attn.INVALID_DIMENSION


def test_validation_order_matches_reference(lib):
    # null beats bad dims (flash_attention_api.cu:49-55)
    assert _fwd(lib, "f32", [None] + [P] * 4, b=0) == cuflash_attn.NULL_POINTER
    # bad dims beat bad head_dim (:53-59)
    assert _fwd(lib, "f32", [P] * 5, b=0, d=48) == cuflash_attn.INVALID_DIMENSION
    # bad head_dim beats bad scale (:57-63)
    assert _fwd(lib, "f32", [P] * 5, d=48, scale=math.nan) == cuflash_attn.UNSUPPORTED_HEAD_DIM
    # backward checks gradient pointers before the forward-side ones (:74-78)
    assert _bwd(lib, "f32", [None] * 9, d=48) == cuflash_attn.NULL_POINTER
    assert _bwd(lib, "f32", [P] * 5 + [None] + [P] * 3, b=-1) == cuflash_attn.NULL_POINTER


def test_decode_validation(lib):
    dec = lib.fn("decode", "f16")
    assert dec(None, P, P, P, P, 1, 1, 16, 32, 1.0, 0, None) == cuflash_attn.NULL_POINTER
    assert dec(P, P, P, P, P, 1, 1, 0, 32, 1.0, 0, None) == cuflash_attn.INVALID_DIMENSION
    assert dec(P, P, P, P, P, 1, 1, 16, 48, 1.0, 0, None) == cuflash_attn.UNSUPPORTED_HEAD_DIM
    assert dec(P, P, P, P, P, 1, 1, 16, 32, math.nan, 0, None) == cuflash_attn.INVALID_DIMENSION
    assert dec(P, P, P, P, P, 1, 1, 16, 32, 1.0, -1, None) == cuflash_attn.INVALID_DIMENSION


def test_decode_gqa_validation(lib):
    """Grouped-query decode: the decode checks, then num_kv_heads > 0 and a divisor of num_heads
    (DIMENSION_MISMATCH otherwise). Every case returns before any GPU work."""
    dec = lib.fn("decode_gqa", "bf16")
    #            Q     K  V  O  L  B  H  Hkv kv  D   scale splits
    assert dec(None, P, P, P, P, 1, 8, 2, 16, 64, 1.0, 0, None) == cuflash_attn.NULL_POINTER
    assert dec(P, P, P, P, P, 1, 8, 2, 0, 64, 1.0, 0, None) == cuflash_attn.INVALID_DIMENSION
    assert dec(P, P, P, P, P, 1, 8, 0, 16, 64, 1.0, 0, None) == cuflash_attn.INVALID_DIMENSION
    assert dec(P, P, P, P, P, 1, 8, 3, 16, 64, 1.0, 0, None) == cuflash_attn.DIMENSION_MISMATCH
    assert dec(P, P, P, P, P, 1, 8, 2, 16, 96, 1.0, 0, None) == cuflash_attn.UNSUPPORTED_HEAD_DIM
    assert dec(P, P, P, P, P, 1, 8, 2, 16, 64, -1.0, 0, None) == cuflash_attn.INVALID_DIMENSION
    assert dec(P, P, P, P, P, 1, 8, 2, 16, 64, 1.0, -2, None) == cuflash_attn.INVALID_DIMENSION


def test_decode_paged_validation(lib):
    """Paged decode: every pointer including block_table and seq_lens non-null, page_size and
    max_pages_per_seq positive and their product an int, then the grouped-query checks."""
    dec = lib.fn("decode_paged", "f16")
    #            Q  K  V  O  L  tab lens B  H  Hkv page maxp D  scale splits
    ok = (P, P, P, P, P, P, P, 2, 8, 8, 16, 4, 128, 1.0, 0, None)
    def call(**kw):
        names = ["q", "k", "v", "o", "l", "tab", "lens", "b", "h", "hkv", "page", "maxp", "d",
                 "scale", "splits", "stream"]
        args = dict(zip(names, ok))
        args.update(kw)
        return dec(*[args[n] for n in names])
    assert call(tab=None) == cuflash_attn.NULL_POINTER
    assert call(lens=None) == cuflash_attn.NULL_POINTER
    assert call(o=None) == cuflash_attn.NULL_POINTER
    assert call(page=0) == cuflash_attn.INVALID_DIMENSION
    assert call(maxp=-1) == cuflash_attn.INVALID_DIMENSION
    assert call(page=1 << 16, maxp=1 << 16) == cuflash_attn.INVALID_DIMENSION
    assert call(b=0) == cuflash_attn.INVALID_DIMENSION
    assert call(hkv=3) == cuflash_attn.DIMENSION_MISMATCH
    assert call(d=16) == cuflash_attn.UNSUPPORTED_HEAD_DIM
    assert call(scale=math.inf) == cuflash_attn.INVALID_DIMENSION
    assert call(splits=-1) == cuflash_attn.INVALID_DIMENSION


@pytest.mark.parametrize("sfx", ["f32", "f16", "bf16"])
def test_ext_validation(lib, sfx):
    """Extended forward / backward: the forward checks in order (null pointers, dimensions
    including num_kv_heads and both lengths, head_dim in {32, 64, 96, 128, 256}, scale), then
    the head grouping and, with a causal mask, q_len <= kv_len (DIMENSION_MISMATCH); the
    backward checks its gradient pointers first. Every case returns before any GPU work."""
    fwd = lib.fn("forward_ext", sfx)
    bwd = lib.fn("backward_ext", sfx)
    names = ["b", "h", "hkv", "nq", "nk", "d", "scale", "causal"]
    ok = dict(b=1, h=8, hkv=2, nq=16, nk=40, d=96, scale=1.0, causal=True)

    def f(ptrs=None, **kw):
        a = dict(ok, **kw)
        return fwd(*(ptrs or [P] * 5), *[a[n] for n in names], None)

    def g(ptrs=None, **kw):
        a = dict(ok, **kw)
        return bwd(*(ptrs or [P] * 9), *[a[n] for n in names], None)

    for call, n in ((f, 5), (g, 9)):
        for i in range(n):
            ptrs = [P] * n
            ptrs[i] = None
            assert call(ptrs) == cuflash_attn.NULL_POINTER
        for dims in (dict(b=0), dict(h=-1), dict(hkv=0), dict(nq=0), dict(nk=-3), dict(d=0)):
            assert call(**dims) == cuflash_attn.INVALID_DIMENSION
        for d in (16, 48, 80, 160, 512):
            assert call(d=d) == cuflash_attn.UNSUPPORTED_HEAD_DIM
        for scale in (math.nan, -1.0):
            assert call(scale=scale) == cuflash_attn.INVALID_DIMENSION
        assert call(hkv=3) == cuflash_attn.DIMENSION_MISMATCH
        assert call(nq=41, nk=40) == cuflash_attn.DIMENSION_MISMATCH
        # order: null before dims, dims before head_dim, head_dim before scale, scale before
        # the grouping
        assert call([None] + [P] * (n - 1), b=0) == cuflash_attn.NULL_POINTER
        assert call(b=0, d=48) == cuflash_attn.INVALID_DIMENSION
        assert call(d=48, scale=math.nan) == cuflash_attn.UNSUPPORTED_HEAD_DIM
        assert call(scale=math.nan, hkv=3) == cuflash_attn.INVALID_DIMENSION
    # q_len > kv_len is fine without a causal mask (checked up to the launch on the GPU tests)
    assert g([P] * 5 + [None] + [P] * 3, b=-1) == cuflash_attn.NULL_POINTER


def test_candidate_paths_follow_reference_order(monkeypatch):
    monkeypatch.setenv("CUFLASH_LIB", "/nonexistent/libcuflash_attn.so")
    paths = cuflash_attn.candidate_library_paths()
    assert paths[0] == "/nonexistent/libcuflash_attn.so"
    assert paths[1] == os.path.join(REPO, "build", "libcuflash_attn.so")
    assert paths[2].endswith(os.path.join("build", "default", "libcuflash_attn.so"))


def test_missing_library_fails_loudly():
    with pytest.raises(OSError):
        cuflash_attn.load_library("/nonexistent/libcuflash_attn.so")


# The primitive layer cuflash::kernels::* (include/cuflash/kernels/*.cuh): every instantiation the
# reference library exports (src/kernels/matmul.cu:236-319, tile_io.cu:229-287,
# online_softmax.cu:160-246) must be exported, with the HIP stream type.
MATMUL_SHAPES = [(64, 64, 32), (32, 32, 32), (64, 64, 64), (32, 32, 128), (64, 64, 128),
                 (32, 64, 32), (32, 64, 64), (64, 32, 64)]
TILE_SHAPES = [(64, 64), (64, 32), (32, 32), (32, 64), (32, 128), (64, 128)]


def _primitive_signatures():
    f, s = "ihipStream_t*", "int, int, int, int, int"
    sigs = []
    for m, n, k in MATMUL_SHAPES:
        for op in ("matmul_ABt", "matmul_AB", "matmul_AB_acc", "matmul_AtB"):
            sigs.append(f"cuflash::kernels::{op}<{m}, {n}, {k}>(float const*, float const*, "
                        f"float*, float, {f})")
    for r, c in TILE_SHAPES:
        sigs += [f"cuflash::kernels::load_tile<{r}, {c}>(float const*, float*, {s}, {f})",
                 f"cuflash::kernels::load_tile<{r}, {c}>(__half const*, float*, {s}, {f})",
                 f"cuflash::kernels::store_tile<{r}, {c}>(float const*, float*, {s}, {f})",
                 f"cuflash::kernels::store_tile<{r}, {c}>(float const*, __half*, {s}, {f})"]
    sigs.append(f"cuflash::kernels::load_store_tile_roundtrip<64, 64>(float const*, float*, {s}, "
                f"{f})")
    sigs += [f"cuflash::kernels::online_softmax_init(float*, float*, int, {f})",
             f"cuflash::kernels::online_softmax_update(float const*, float const*, float*, "
             f"float*, int, {f})",
             f"cuflash::kernels::online_softmax_finalize(float const*, float const*, float*, "
             f"float*, int, {f})",
             f"cuflash::kernels::online_softmax_forward(float const*, float*, float*, int, int, "
             f"int, {f})"]
    return sigs


def test_primitive_layer_is_exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", "-C", lib.path], capture_output=True,
                         text=True, check=True).stdout
    exported = set()
    for line in out.splitlines():
        parts = line.split(" ", 2)
        if len(parts) == 3 and parts[1] in ("T", "W"):
            exported.add(parts[2].replace("cuflash::FlashAttentionError ", ""))
    sigs = _primitive_signatures()
    assert len(sigs) == 61
    missing = [s for s in sigs if s not in exported]
    assert not missing, missing


def test_primitive_headers_declare_the_reference_api():
    """Every primitive the reference declares (include/cuflash/kernels/*.cuh) is declared here
    under the same name and header file name."""
    names = {"matmul.cuh": ["matmul_ABt", "matmul_AB", "matmul_AB_acc", "matmul_AtB"],
             "online_softmax.cuh": ["online_softmax_init", "online_softmax_update",
                                    "online_softmax_finalize", "online_softmax_forward",
                                    "warp_reduce_max", "warp_reduce_sum"],
             "tile_io.cuh": ["load_tile", "store_tile", "load_store_tile_roundtrip"]}
    for header, fns in names.items():
        text = open(os.path.join(REPO, "include", "cuflash", "kernels", header)).read()
        assert "namespace kernels" in text
        for fn in fns:
            assert re.search(r"\b" + fn + r"\(", text), (header, fn)


# The library search list of the reference's example caller (examples/python_binding.py:25-48),
# restated as data: paths relative to the repository root that holds examples/, then the system
# library directories. It does not look in build/ itself.
EXAMPLE_SEARCH = ("build/release/libcuflash_attn.so", "build/debug/libcuflash_attn.so",
                  "/usr/local/lib/libcuflash_attn.so", "/usr/lib/libcuflash_attn.so")


@default_search_only
def test_example_caller_search_path_finds_the_library(lib):
    found = None
    for p in EXAMPLE_SEARCH:
        path = p if os.path.isabs(p) else os.path.join(REPO, p)
        if os.path.exists(path):
            found = path
            break
    assert found == os.path.join(REPO, "build", "release", "libcuflash_attn.so")
    assert os.path.realpath(found) == os.path.realpath(lib.path)
    handle = ctypes.CDLL(found)
    for sym in ("cuflash_attention_forward_f32", "cuflash_attention_backward_f32",
                "cuflash_error_string"):
        assert getattr(handle, sym) is not None
    handle.cuflash_error_string.restype = ctypes.c_char_p
    assert handle.cuflash_error_string(0) == b"Success"


@default_search_only
def test_test_caller_search_path_finds_the_library(lib):
    # tests/integration/test_pytorch_comparison.py:158-180 without $CUFLASH_LIB: build/ first.
    presets = ("default", "release", "release-fast-math", "minimal", "Release", "Debug")
    order = [os.path.join(REPO, "build", "libcuflash_attn.so")]
    order += [os.path.join(REPO, "build", d, "libcuflash_attn.so") for d in presets]
    first = next(p for p in order if os.path.exists(p))
    assert first == lib.path
