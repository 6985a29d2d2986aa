"""Python binding of libcuflash_attn.so (MI355X / gfx950).

Mirrors the reference's ctypes caller (tests/integration/test_pytorch_comparison.py:37-194 and
examples/python_binding.py:51-180): the same library search order ($CUFLASH_LIB, then
build/libcuflash_attn.so and the build/<preset>/ directories), the same argtypes for the six
C-ABI entry points, and status codes equal to cuflash::FlashAttentionError. On top of that it
offers tensor-level helpers for PyTorch-ROCm tensors that allocate the outputs and enqueue on
torch's current HIP stream.

There is no fallback: if the library is missing, load_library() raises.
"""

from __future__ import annotations

import ctypes
import os
import sys
from typing import Optional, Sequence

SUCCESS = 0
INVALID_DIMENSION = 1
DIMENSION_MISMATCH = 2
NULL_POINTER = 3
CUDA_ERROR = 4
OUT_OF_MEMORY = 5
UNSUPPORTED_HEAD_DIM = 6
UNSUPPORTED_DTYPE = 7

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_ROOT = os.path.dirname(os.path.dirname(_PKG_DIR))

_DTYPE_SUFFIX = {"float32": "f32", "float16": "f16", "bfloat16": "bf16"}


class CuFlashError(RuntimeError):
    """Raised by the tensor helpers when a C-ABI call returns a non-zero status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"cuflash error {code}: {message}")
        self.code = code


def candidate_library_paths() -> Sequence[str]:
    """Search order of the reference's test_pytorch_comparison.py:158-180."""
    build_dir = os.path.join(REPO_ROOT, "build")
    out = []
    explicit = os.environ.get("CUFLASH_LIB")
    if explicit:
        out.append(explicit)
    name = "libcuflash_attn.so"
    out.append(os.path.join(build_dir, name))
    for preset in ("default", "release", "release-fast-math", "minimal", "Release", "Debug"):
        out.append(os.path.join(build_dir, preset, name))
    return out


_FWD_ARGS = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 4 + [ctypes.c_float, ctypes.c_bool,
                                                          ctypes.c_void_p]
_BWD_ARGS = [ctypes.c_void_p] * 9 + [ctypes.c_int] * 4 + [ctypes.c_float, ctypes.c_bool,
                                                          ctypes.c_void_p]
_DEC_ARGS = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 4 + [ctypes.c_float, ctypes.c_int,
                                                          ctypes.c_void_p]
_DEC_GQA_ARGS = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 5 + [ctypes.c_float, ctypes.c_int,
                                                              ctypes.c_void_p]
_DEC_PAGED_ARGS = [ctypes.c_void_p] * 7 + [ctypes.c_int] * 6 + [ctypes.c_float, ctypes.c_int,
                                                                ctypes.c_void_p]
_FWD_EXT_ARGS = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 6 + [ctypes.c_float, ctypes.c_bool,
                                                              ctypes.c_void_p]
_BWD_EXT_ARGS = [ctypes.c_void_p] * 9 + [ctypes.c_int] * 6 + [ctypes.c_float, ctypes.c_bool,
                                                              ctypes.c_void_p]

EXPORTED_SYMBOLS = (
    "cuflash_attention_forward_f32", "cuflash_attention_forward_f16",
    "cuflash_attention_forward_bf16", "cuflash_attention_backward_f32",
    "cuflash_attention_backward_f16", "cuflash_attention_backward_bf16",
    "cuflash_attention_decode_f32", "cuflash_attention_decode_f16",
    "cuflash_attention_decode_bf16", "cuflash_attention_decode_gqa_f32",
    "cuflash_attention_decode_gqa_f16", "cuflash_attention_decode_gqa_bf16",
    "cuflash_attention_decode_paged_f32", "cuflash_attention_decode_paged_f16",
    "cuflash_attention_decode_paged_bf16", "cuflash_attention_forward_ext_f32",
    "cuflash_attention_forward_ext_f16", "cuflash_attention_forward_ext_bf16",
    "cuflash_attention_backward_ext_f32", "cuflash_attention_backward_ext_f16",
    "cuflash_attention_backward_ext_bf16", "cuflash_error_string", "cuflash_version",
    "cuflash_profile_enable", "cuflash_profile_report", "cuflash_attention_decode_noalloc_f16",
    "cuflash_release_workspaces",
)


class CuFlashLibrary:
    """ctypes view of libcuflash_attn.so with argtypes set (reference CuFlashLibrary)."""

    def __init__(self, library: ctypes.CDLL):
        self.library = library
        self.path = getattr(library, "_name", "")
        for sfx in ("f32", "f16", "bf16"):
            fwd = getattr(library, f"cuflash_attention_forward_{sfx}")
            fwd.argtypes, fwd.restype = _FWD_ARGS, ctypes.c_int
            bwd = getattr(library, f"cuflash_attention_backward_{sfx}")
            bwd.argtypes, bwd.restype = _BWD_ARGS, ctypes.c_int
            dec = getattr(library, f"cuflash_attention_decode_{sfx}")
            dec.argtypes, dec.restype = _DEC_ARGS, ctypes.c_int
            gqa = getattr(library, f"cuflash_attention_decode_gqa_{sfx}")
            gqa.argtypes, gqa.restype = _DEC_GQA_ARGS, ctypes.c_int
            paged = getattr(library, f"cuflash_attention_decode_paged_{sfx}")
            paged.argtypes, paged.restype = _DEC_PAGED_ARGS, ctypes.c_int
            fwd_ext = getattr(library, f"cuflash_attention_forward_ext_{sfx}")
            fwd_ext.argtypes, fwd_ext.restype = _FWD_EXT_ARGS, ctypes.c_int
            bwd_ext = getattr(library, f"cuflash_attention_backward_ext_{sfx}")
            bwd_ext.argtypes, bwd_ext.restype = _BWD_EXT_ARGS, ctypes.c_int
        noalloc = library.cuflash_attention_decode_noalloc_f16
        noalloc.argtypes, noalloc.restype = _DEC_ARGS, ctypes.c_int
        library.cuflash_error_string.argtypes = [ctypes.c_int]
        library.cuflash_error_string.restype = ctypes.c_char_p
        library.cuflash_version.argtypes = []
        library.cuflash_version.restype = ctypes.c_char_p
        library.cuflash_profile_enable.argtypes = [ctypes.c_int]
        library.cuflash_profile_enable.restype = None
        library.cuflash_profile_report.argtypes = [ctypes.c_char_p, ctypes.c_int]
        library.cuflash_profile_report.restype = ctypes.c_int
        library.cuflash_release_workspaces.argtypes = []
        library.cuflash_release_workspaces.restype = ctypes.c_int

    def error_string(self, code: int) -> str:
        return self.library.cuflash_error_string(int(code)).decode()

    def version(self) -> str:
        return self.library.cuflash_version().decode()

    def profile_enable(self, enabled: bool) -> None:
        self.library.cuflash_profile_enable(1 if enabled else 0)

    def profile_report(self) -> dict:
        """{label: (launches, total_ms)} for the kernels launched since the last report."""
        buf = ctypes.create_string_buffer(1 << 16)
        self.library.cuflash_profile_report(buf, len(buf))
        out = {}
        for line in buf.value.decode().splitlines():
            label, count, ms = line.split("\t")
            out[label] = (int(count), float(ms))
        return out

    def fn(self, kind: str, suffix: str):
        return getattr(self.library, f"cuflash_attention_{kind}_{suffix}")


_CACHED: Optional[CuFlashLibrary] = None


def load_library(path: Optional[str] = None) -> CuFlashLibrary:
    """Loads libcuflash_attn.so (first hit of the search order). Raises when it is missing."""
    global _CACHED
    if path is None and _CACHED is not None:
        return _CACHED
    tried = [path] if path else list(candidate_library_paths())
    errors = []
    for p in tried:
        if not os.path.exists(p):
            errors.append(f"{p}: missing")
            continue
        try:
            lib = CuFlashLibrary(ctypes.CDLL(p))
        except OSError as e:
            errors.append(f"{p}: {e}")
            continue
        if path is None:
            _CACHED = lib
        return lib
    raise OSError("libcuflash_attn.so not found; build it with "
                  "`python cuflash-attn_amd/build.py`. Tried:\n  " + "\n  ".join(errors))


# ---------------------------------------------------------------------------------------------
# PyTorch tensor helpers (device memory and streams come from PyTorch-ROCm)
# ---------------------------------------------------------------------------------------------

def _torch():
    import torch  # noqa: WPS433 (imported lazily: the ctypes layer itself needs no torch)

    return torch


def _suffix(t) -> str:
    name = str(t.dtype).replace("torch.", "")
    if name not in _DTYPE_SUFFIX:
        raise CuFlashError(UNSUPPORTED_DTYPE, f"unsupported dtype {t.dtype}")
    return _DTYPE_SUFFIX[name]


def _check(tensors, dtype):
    for t in tensors:
        if not t.is_cuda:
            raise ValueError("tensors must be on the GPU")
        if not t.is_contiguous():
            raise ValueError("tensors must be contiguous")
        if t.dtype != dtype:
            raise ValueError("all tensors must share one dtype")


def _stream_ptr(stream=None):
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _raise(lib: CuFlashLibrary, status: int):
    if status != SUCCESS:
        raise CuFlashError(status, lib.error_string(status))


def flash_attention_forward(q, k, v, scale: Optional[float] = None, causal: bool = False,
                            out=None, lse=None, stream=None, lib: Optional[CuFlashLibrary] = None):
    """O, L = attention(q, k, v) for [B, H, N, D] tensors; L is float32 [B, H, N]."""
    torch = _torch()
    lib = lib or load_library()
    _check((q, k, v), q.dtype)
    B, H, N, D = q.shape
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k, v must have the same shape")
    scale = float(D ** -0.5) if scale is None else float(scale)
    out = torch.empty_like(q) if out is None else out
    lse = torch.empty((B, H, N), device=q.device, dtype=torch.float32) if lse is None else lse
    status = lib.fn("forward", _suffix(q))(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                           out.data_ptr(), lse.data_ptr(), B, H, N, D, scale,
                                           bool(causal), _stream_ptr(stream))
    _raise(lib, status)
    return out, lse


def flash_attention_backward(q, k, v, o, lse, do, scale: Optional[float] = None,
                             causal: bool = False, stream=None,
                             lib: Optional[CuFlashLibrary] = None):
    """dQ, dK, dV for [B, H, N, D] tensors given O and the float32 logsumexp L."""
    torch = _torch()
    lib = lib or load_library()
    _check((q, k, v, o, do), q.dtype)
    B, H, N, D = q.shape
    scale = float(D ** -0.5) if scale is None else float(scale)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    status = lib.fn("backward", _suffix(q))(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                            o.data_ptr(), lse.data_ptr(), do.data_ptr(),
                                            dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, H, N,
                                            D, scale, bool(causal), _stream_ptr(stream))
    _raise(lib, status)
    return dq, dk, dv


def _ext_shapes(q, k, v):
    if q.dim() != 4 or k.dim() != 4 or v.shape != k.shape:
        raise ValueError("expected q [B,H,Nq,D] and k, v [B,Hkv,Nk,D]")
    B, H, Nq, D = q.shape
    if k.shape[0] != B or k.shape[3] != D:
        raise ValueError("q and k, v differ in batch or head_dim")
    return B, H, k.shape[1], Nq, k.shape[2], D


def flash_attention_forward_ext(q, k, v, scale: Optional[float] = None, causal: bool = False,
                                out=None, lse=None, stream=None,
                                lib: Optional[CuFlashLibrary] = None):
    """Forward with q [B, H, Nq, D] and k, v [B, Hkv, Nk, D] (Hkv a divisor of H; query head h
    reads key/value head h // (H // Hkv)), D in {32, 64, 96, 128, 256}; a causal mask lets
    query i see keys j <= i + Nk - Nq (cuflash_attention_forward_ext_*).
    -> O [B, H, Nq, D], L float32 [B, H, Nq]."""
    torch = _torch()
    lib = lib or load_library()
    _check((q, k, v), q.dtype)
    B, H, Hkv, Nq, Nk, D = _ext_shapes(q, k, v)
    scale = float(D ** -0.5) if scale is None else float(scale)
    out = torch.empty_like(q) if out is None else out
    lse = torch.empty((B, H, Nq), device=q.device, dtype=torch.float32) if lse is None else lse
    status = lib.fn("forward_ext", _suffix(q))(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                               out.data_ptr(), lse.data_ptr(), B, H, Hkv, Nq,
                                               Nk, D, scale, bool(causal), _stream_ptr(stream))
    _raise(lib, status)
    return out, lse


def flash_attention_backward_ext(q, k, v, o, lse, do, scale: Optional[float] = None,
                                 causal: bool = False, stream=None,
                                 lib: Optional[CuFlashLibrary] = None):
    """dQ [B, H, Nq, D], dK, dV [B, Hkv, Nk, D] for the shapes of flash_attention_forward_ext
    (dK, dV of a key/value head summed over its query heads; cuflash_attention_backward_ext_*)."""
    torch = _torch()
    lib = lib or load_library()
    _check((q, k, v, o, do), q.dtype)
    B, H, Hkv, Nq, Nk, D = _ext_shapes(q, k, v)
    scale = float(D ** -0.5) if scale is None else float(scale)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    status = lib.fn("backward_ext", _suffix(q))(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                                o.data_ptr(), lse.data_ptr(), do.data_ptr(),
                                                dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, H,
                                                Hkv, Nq, Nk, D, scale, bool(causal),
                                                _stream_ptr(stream))
    _raise(lib, status)
    return dq, dk, dv


def flash_attention_decode(q, k, v, scale: Optional[float] = None, num_splits: int = 0,
                           out=None, lse=None, stream=None,
                           lib: Optional[CuFlashLibrary] = None):
    """Split-KV decode: q [B, H, 1, D], k/v [B, Hkv, Lkv, D] -> O [B, H, 1, D], L [B, H, 1].
    Hkv == H calls cuflash_attention_decode_*, a divisor of H (grouped-query / multi-query
    attention: query head h reads key/value head h // (H // Hkv)) cuflash_attention_decode_gqa_*."""
    torch = _torch()
    lib = lib or load_library()
    _check((q, k, v), q.dtype)
    B, H, one, D = q.shape
    if one != 1 or k.dim() != 4 or k.shape[0] != B or k.shape[3] != D or v.shape != k.shape:
        raise ValueError("decode expects q [B,H,1,D] and k, v [B,Hkv,Lkv,D]")
    Hkv, kv_len = k.shape[1], k.shape[2]
    scale = float(D ** -0.5) if scale is None else float(scale)
    out = torch.empty_like(q) if out is None else out
    lse = torch.empty((B, H, 1), device=q.device, dtype=torch.float32) if lse is None else lse
    if Hkv == H:
        status = lib.fn("decode", _suffix(q))(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                              out.data_ptr(), lse.data_ptr(), B, H, kv_len, D,
                                              scale, int(num_splits), _stream_ptr(stream))
    else:
        status = lib.fn("decode_gqa", _suffix(q))(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                                  out.data_ptr(), lse.data_ptr(), B, H, Hkv,
                                                  kv_len, D, scale, int(num_splits),
                                                  _stream_ptr(stream))
    _raise(lib, status)
    return out, lse


def flash_attention_decode_paged(q, k_cache, v_cache, block_table, seq_lens,
                                 scale: Optional[float] = None, num_splits: int = 0, out=None,
                                 lse=None, stream=None, lib: Optional[CuFlashLibrary] = None):
    """Split-KV decode over a paged cache: q [B, H, 1, D]; k_cache, v_cache
    [num_pages, page_size, Hkv, D]; block_table [B, max_pages] int32 (page of keys
    [p * page_size, (p + 1) * page_size) of each sequence); seq_lens [B] int32.
    -> O [B, H, 1, D], L [B, H, 1] (cuflash_attention_decode_paged_*)."""
    torch = _torch()
    lib = lib or load_library()
    _check((q, k_cache, v_cache), q.dtype)
    B, H, one, D = q.shape
    if (one != 1 or k_cache.dim() != 4 or k_cache.shape[3] != D or v_cache.shape != k_cache.shape
            or block_table.dim() != 2 or block_table.shape[0] != B
            or tuple(seq_lens.shape) != (B,)):
        raise ValueError("paged decode expects q [B,H,1,D], k/v cache [P,page,Hkv,D], "
                         "block_table [B,max_pages], seq_lens [B]")
    if block_table.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise TypeError("block_table and seq_lens must be int32")
    if not (block_table.is_contiguous() and seq_lens.is_contiguous()):
        raise ValueError("block_table and seq_lens must be contiguous")
    page_size, Hkv = k_cache.shape[1], k_cache.shape[2]
    scale = float(D ** -0.5) if scale is None else float(scale)
    out = torch.empty_like(q) if out is None else out
    lse = torch.empty((B, H, 1), device=q.device, dtype=torch.float32) if lse is None else lse
    status = lib.fn("decode_paged", _suffix(q))(q.data_ptr(), k_cache.data_ptr(),
                                                v_cache.data_ptr(), out.data_ptr(),
                                                lse.data_ptr(), block_table.data_ptr(),
                                                seq_lens.data_ptr(), B, H, Hkv, page_size,
                                                block_table.shape[1], D, scale, int(num_splits),
                                                _stream_ptr(stream))
    _raise(lib, status)
    return out, lse


__all__ = [
    "CuFlashError", "CuFlashLibrary", "EXPORTED_SYMBOLS", "load_library",
    "candidate_library_paths", "flash_attention_forward", "flash_attention_backward",
    "flash_attention_forward_ext", "flash_attention_backward_ext", "flash_attention_decode",
    "flash_attention_decode_paged", "SUCCESS", "INVALID_DIMENSION", "DIMENSION_MISMATCH",
    "NULL_POINTER", "CUDA_ERROR", "OUT_OF_MEMORY", "UNSUPPORTED_HEAD_DIM", "UNSUPPORTED_DTYPE",
]

if sys.version_info < (3, 8):  # pragma: no cover
    raise RuntimeError("python >= 3.8 required")
