"""Seeded synthetic inputs shared by the tests and the benchmark.

SplitMix64 (Steele, Lea and Flood, "Fast splittable pseudorandom number generators", OOPSLA 2014) gives the
uniform stream; normals come from the Box-Muller transform evaluated in double precision. Values are produced
as float32 and narrowed to bfloat16 / float16 with round-to-nearest-even, the same narrowing Frame's dtype
bridge uses, so CPU and GPU runs see bit-identical inputs.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _splitmix64(seed: int, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (np.arange(1, n + 1, dtype=np.uint64) * _GOLDEN)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    """n doubles in [lo, hi)."""
    u = (_splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    return lo + (hi - lo) * u


def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """n doubles ~ N(mean, std^2) by Box-Muller on pairs of uniforms."""
    m = (n + 1) // 2
    u = uniform(seed, 2 * m)
    u1 = 1.0 - u[0::2]  # (0, 1]
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return mean + std * z[:n]


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round-to-nearest-even, NaN forced quiet (sign kept)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    with np.errstate(over="ignore"):
        r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    r = np.where(nan, (u >> np.uint32(16)) | np.uint32(0x40), r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_f16_bits(a: np.ndarray) -> np.ndarray:
    """float32 -> float16 bit patterns (IEEE round-to-nearest-even; NaN made the canonical quiet NaN)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        h = a.astype(np.float16).view(np.uint16)
    nan = np.isnan(a)
    sign = (a.view(np.uint32) >> np.uint32(16)).astype(np.uint16) & np.uint16(0x8000)
    return np.where(nan, sign | np.uint16(0x7E00), h).astype(np.uint16)


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def to_storage(values_f32: np.ndarray, dtype: int) -> np.ndarray:
    """float32 values -> storage array for dtype code (0 f32, 2 f16, 3 bf16)."""
    if dtype == 0:
        return np.ascontiguousarray(values_f32, dtype=np.float32)
    if dtype == 3:
        return f32_to_bf16_bits(values_f32)
    if dtype == 2:
        return f32_to_f16_bits(values_f32)
    raise ValueError(f"unsupported dtype code {dtype}")


def to_float(storage: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == 0:
        return np.asarray(storage, dtype=np.float32)
    if dtype == 3:
        return bf16_bits_to_f32(storage)
    if dtype == 2:
        return f16_bits_to_f32(storage)
    raise ValueError(f"unsupported dtype code {dtype}")


def tensor(seed: int, shape, dtype: int, dist: str = "normal", scale: float = 1.0) -> np.ndarray:
    """Seeded tensor in storage form. dist: 'normal' (N(0, scale^2)) or 'uniform' (U(-scale, scale))."""
    n = int(np.prod(shape)) if len(shape) else 1
    if dist == "normal":
        v = normal(seed, n, 0.0, scale)
    elif dist == "uniform":
        v = uniform(seed, n, -scale, scale)
    elif dist == "zeros":
        v = np.zeros(n)
    else:
        raise ValueError(dist)
    return to_storage(v.astype(np.float32).reshape(shape), dtype)
