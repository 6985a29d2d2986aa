"""Seeded synthetic inputs for tests and benchmarks.

A counter-based SplitMix64 stream: value i of seed s is mix(s + (i + 1) * 0x9E3779B97F4A7C15),
the i-th output of Steele/Lea/Flood's SplitMix64 generator started at state s. Uniforms take
the top 53 bits; normals use the Box-Muller transform on consecutive pairs. The stream depends
only on (seed, index), so it is reproducible on any machine and independent of numpy's or
torch's generators. Reduced-precision inputs are rounded to nearest-even (float16 via numpy,
bfloat16 by the bit rule below), as the reference's conversions do
(src/kernels/impl/type_adapter.cuh:18-32).
"""

from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _bits(seed: int, start: int, n: int) -> np.ndarray:
    idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix(np.uint64(seed) + idx * _GAMMA)


def uniform(seed: int, shape, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    """i.i.d. uniform [lo, hi) float32 values."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    for s in range(0, n, _CHUNK):
        m = min(_CHUNK, n - s)
        u = (_bits(seed, s, m) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))
        out[s:s + m] = (lo + (hi - lo) * u).astype(np.float32)
    return out.reshape(shape)


def normal(seed: int, shape, std: float = 1.0) -> np.ndarray:
    """i.i.d. N(0, std^2) float32 values (Box-Muller on pairs of the stream)."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    for s in range(0, n, _CHUNK):
        m = min(_CHUNK, n - s)
        pairs = (m + 1) // 2
        b = _bits(seed, s, 2 * pairs)  # chunk starts are even, so pairs stay aligned
        u1 = ((b[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / (1 << 53))
        u2 = (b[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))
        r = np.sqrt(-2.0 * np.log(u1))
        z = np.empty(2 * pairs, dtype=np.float64)
        z[0::2] = r * np.cos(2.0 * np.pi * u2)
        z[1::2] = r * np.sin(2.0 * np.pi * u2)
        out[s:s + m] = (std * z[:m]).astype(np.float32)
    return out.reshape(shape)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even, NaN kept quiet."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = (u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))) >> np.uint32(16)
    nan = np.isnan(x)
    out = rounded.astype(np.uint16)
    out[nan] = np.uint16(0x7FC0)
    return out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values rounded to `dtype` ("float32" | "float16" | "bfloat16"), as float32."""
    if dtype == "float32":
        return np.asarray(x, dtype=np.float32)
    if dtype == "float16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        return bf16_to_f32(bf16_bits(x))
    raise ValueError(dtype)


def to_torch(x: np.ndarray, dtype: str, device="cuda"):
    """float32 numpy values (already representable in `dtype`) -> torch tensor on `device`."""
    import torch

    if dtype == "float32":
        t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    elif dtype == "float16":
        t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32).astype(np.float16))
    elif dtype == "bfloat16":
        t = torch.from_numpy(bf16_bits(x).view(np.int16)).view(torch.bfloat16)
    else:
        raise ValueError(dtype)
    return t.to(device).contiguous()


def to_numpy(t) -> np.ndarray:
    """torch tensor (any of the three dtypes, any device) -> float32 numpy."""
    import torch

    return t.detach().to(device="cpu", dtype=torch.float32).contiguous().numpy()
