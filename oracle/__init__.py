"""CPU oracle for the FlashAttention hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module,
and only as the checker (or, for the naive fp32 functions, as the reported CPU baseline).
The product library (build/libcuflash_attn.so) never calls it and has no CPU fallback.

The arithmetic lives in oracle.c (fp64 restatements of the reference's CPU attention in
tests/unit/test_forward.cu:21-118 and tests/unit/test_backward.cu:21-127); this file is a
ctypes wrapper over numpy arrays laid out [B, H, N, D] (float32, C-contiguous).

The reference (CUDA-only) cannot be compiled here, so there is no oracle/_ref build; the oracle
is pinned by closed forms, finite differences, invariants, torch's float64 attention and the
committed fixtures (tests/test_oracle.py).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_DIR, "_build", "liboracle.so")
_lib = None

_i64 = ctypes.c_int64
_fp = ctypes.POINTER(ctypes.c_float)
_dp = ctypes.POINTER(ctypes.c_double)
_ip = ctypes.POINTER(ctypes.c_int64)


def build() -> str:
    """Compiles oracle.c with the committed Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", _DIR], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    lib.oracle_forward.argtypes = [_fp, _fp, _fp, _fp, _fp, _i64, _i64, _i64, _i64,
                                   ctypes.c_double, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.oracle_backward.argtypes = [_fp, _fp, _fp, _fp, _fp, _fp, _fp, _i64, _i64, _i64, _i64,
                                    ctypes.c_double, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.oracle_backward_rows.argtypes = [_fp, _fp, _fp, _fp, _fp, _fp, _fp, _i64, _i64, _i64,
                                         _i64, ctypes.c_double, ctypes.c_int, _ip, _i64, _ip,
                                         _i64, ctypes.c_int, ctypes.c_int]
    lib.oracle_decode_partials.argtypes = [_fp, _fp, _fp, _i64, _i64, _i64, ctypes.c_double,
                                           _i64, _i64, _dp, _dp, _dp]
    lib.oracle_decode_combine.argtypes = [_dp, _dp, _dp, _i64, _i64, _i64, _fp, _fp]
    lib.cpu_naive_forward_f32.argtypes = [_fp, _fp, _fp, _fp, _fp, _i64, _i64, _i64,
                                          ctypes.c_float, ctypes.c_int, ctypes.c_int]
    lib.cpu_naive_backward_f32.argtypes = [_fp, _fp, _fp, _fp, _fp, _fp, _fp, _i64, _i64, _i64,
                                           ctypes.c_float, ctypes.c_int, ctypes.c_int]
    lib.cpu_naive_rows_f32.argtypes = [_fp, _fp, _fp, _fp, _ip, _i64, _fp, _fp, _fp, _fp, _fp,
                                       _i64, _i64, ctypes.c_float, ctypes.c_int, ctypes.c_int]
    lib.cpu_naive_decode_f32.argtypes = [_fp, _fp, _fp, _fp, _fp, _i64, _i64, _i64,
                                         ctypes.c_float, ctypes.c_int]
    _lib = lib
    return lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray):
    if a.dtype == np.float32:
        return a.ctypes.data_as(_fp)
    if a.dtype == np.float64:
        return a.ctypes.data_as(_dp)
    if a.dtype == np.int64:
        return a.ctypes.data_as(_ip)
    raise TypeError(a.dtype)


def default_threads() -> int:
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


def forward(q, k, v, scale: float, causal: bool, nthreads: int | None = None, mutation: int = 0):
    """O [B,H,Nq,D] and L [B,H,Nq] in fp64 arithmetic (reference test_forward.cu:21-118).

    K and V may have a different key count Nk (decode); causal masks keys j > i + Nk - Nq.
    """
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, Nq, D = q.shape
    Nk = k.shape[2]
    assert k.shape == (B, H, Nk, D) and v.shape == k.shape
    o = np.empty_like(q)
    lse = np.empty((B, H, Nq), dtype=np.float32)
    rc = _load().oracle_forward(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), B * H, Nq, Nk, D,
                                float(scale), int(bool(causal)), nthreads or default_threads(),
                                mutation)
    assert rc == 0
    return o, lse


def backward(q, k, v, do, scale: float, causal: bool, nthreads: int | None = None,
             mutation: int = 0):
    """dQ, dK, dV in fp64 arithmetic, P materialized (reference test_backward.cu:21-127).

    K and V may have a different key count Nk; causal masks keys j > i + Nk - Nq (Nq <= Nk).
    """
    q, k, v, do = _f32(q), _f32(k), _f32(v), _f32(do)
    B, H, Nq, D = q.shape
    Nk = k.shape[2]
    assert k.shape == (B, H, Nk, D) and v.shape == k.shape and do.shape == q.shape
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(k)
    rc = _load().oracle_backward(_ptr(q), _ptr(k), _ptr(v), _ptr(do), _ptr(dq), _ptr(dk),
                                 _ptr(dv), B * H, Nq, Nk, D, float(scale), int(bool(causal)),
                                 nthreads or default_threads(), mutation)
    assert rc == 0
    return dq, dk, dv


def backward_rows(q, k, v, do, scale: float, causal: bool, q_rows, k_rows,
                  nthreads: int | None = None, mutation: int = 0):
    """Row-streaming gradients: dQ at q_rows [B,H,len(q_rows),D]; dK, dV at k_rows.

    K and V may have a different key count Nk than Q's Nq (causal masks j > i + Nk - Nq, as in
    backward); q_rows index [0, Nq), k_rows index [0, Nk).
    """
    q, k, v, do = _f32(q), _f32(k), _f32(v), _f32(do)
    B, H, Nq, D = q.shape
    Nk = k.shape[2]
    assert k.shape == (B, H, Nk, D) and v.shape == k.shape and do.shape == q.shape
    qr = np.ascontiguousarray(q_rows, dtype=np.int64)
    kr = np.ascontiguousarray(k_rows, dtype=np.int64)
    dq = np.zeros((B, H, len(qr), D), dtype=np.float32)
    dk = np.zeros((B, H, len(kr), D), dtype=np.float32)
    dv = np.zeros((B, H, len(kr), D), dtype=np.float32)
    dummy_i = np.zeros(1, dtype=np.int64)
    rc = _load().oracle_backward_rows(
        _ptr(q), _ptr(k), _ptr(v), _ptr(do), _ptr(dq), _ptr(dk), _ptr(dv), B * H, Nq, Nk, D,
        float(scale), int(bool(causal)), _ptr(qr if len(qr) else dummy_i), len(qr),
        _ptr(kr if len(kr) else dummy_i), len(kr), nthreads or default_threads(), mutation)
    assert rc == 0
    return dq, dk, dv


def decode_partials(q, k, v, scale: float, nsplit: int, chunk: int):
    """Per-split (m, l, acc) of the split-KV decode, natural-log units, fp64."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, _, D = q.shape
    Nk = k.shape[2]
    m = np.empty((B * H, nsplit), dtype=np.float64)
    l = np.empty((B * H, nsplit), dtype=np.float64)
    acc = np.empty((B * H, nsplit, D), dtype=np.float64)
    _load().oracle_decode_partials(_ptr(q), _ptr(k), _ptr(v), B * H, Nk, D, float(scale), nsplit,
                                   chunk, _ptr(m), _ptr(l), _ptr(acc))
    return m, l, acc


def decode_combine(m, l, acc, out_shape):
    """Merges split partials (online-softmax rule) into O [B,H,1,D] and L [B,H,1]."""
    m = np.ascontiguousarray(m, dtype=np.float64)
    l = np.ascontiguousarray(l, dtype=np.float64)
    acc = np.ascontiguousarray(acc, dtype=np.float64)
    BH, nsplit, D = acc.shape
    o = np.empty((BH, D), dtype=np.float32)
    lse = np.empty((BH,), dtype=np.float32)
    _load().oracle_decode_combine(_ptr(m), _ptr(l), _ptr(acc), BH, nsplit, D, _ptr(o), _ptr(lse))
    B, H = out_shape[:2]
    return o.reshape(B, H, 1, D), lse.reshape(B, H, 1)


def naive_forward_f32(q, k, v, scale: float, causal: bool, nthreads: int | None = None):
    """The reference's naive CPU attention in float arithmetic (the reported CPU baseline)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, N, D = q.shape
    o = np.empty_like(q)
    lse = np.empty((B, H, N), dtype=np.float32)
    _load().cpu_naive_forward_f32(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), B * H, N, D,
                                  float(scale), int(bool(causal)), nthreads or default_threads())
    return o, lse


def naive_backward_f32(q, k, v, do, scale: float, causal: bool, nthreads: int | None = None):
    """The reference's naive CPU backward in float arithmetic (the reported CPU baseline)."""
    q, k, v, do = _f32(q), _f32(k), _f32(v), _f32(do)
    B, H, N, D = q.shape
    dq, dk, dv = np.empty_like(q), np.empty_like(q), np.empty_like(q)
    _load().cpu_naive_backward_f32(_ptr(q), _ptr(k), _ptr(v), _ptr(do), _ptr(dq), _ptr(dk),
                                   _ptr(dv), B * H, N, D, float(scale), int(bool(causal)),
                                   nthreads or default_threads())
    return dq, dk, dv


def naive_rows_f32(q, k, v, do, scale: float, causal: bool, rows, nthreads: int | None = None):
    """The naive fp32 forward + backward of one head ([N, D] arrays) restricted to query rows
    `rows`: O [len(rows), D], L [len(rows)], dQ [len(rows), D], and the selected rows' summed
    terms of dK and dV [N, D] (the CPU baseline's bounded sample of a long head)."""
    q, k, v, do = _f32(q), _f32(k), _f32(v), _f32(do)
    N, D = q.shape
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    r = rows.size
    o, dq = np.empty((r, D), np.float32), np.empty((r, D), np.float32)
    lse = np.empty((r,), np.float32)
    dk, dv = np.empty_like(q), np.empty_like(q)
    rc = _load().cpu_naive_rows_f32(_ptr(q), _ptr(k), _ptr(v), _ptr(do), _ptr(rows), r, _ptr(o),
                                    _ptr(lse), _ptr(dq), _ptr(dk), _ptr(dv), N, D, float(scale),
                                    int(bool(causal)), nthreads or default_threads())
    assert rc == 0
    return o, lse, dq, dk, dv


def naive_decode_f32(q, k, v, scale: float, nthreads: int | None = None):
    """Naive fp32 decode: q [BH, D], k / v [BH, Nk, D] -> O [BH, D], L [BH] (the decode CPU
    baseline)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    BH, Nk, D = k.shape
    o = np.empty((BH, D), np.float32)
    lse = np.empty((BH,), np.float32)
    _load().cpu_naive_decode_f32(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), BH, Nk, D,
                                 float(scale), nthreads or default_threads())
    return o, lse
