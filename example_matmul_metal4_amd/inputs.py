"""Seeded synthetic inputs for the benchmark and examples (numpy, vectorised).

SplitMix64(seed) -> fp64 uniform / Box-Muller normal -> fp32 -> round-to-nearest-even to f16 or
bf16. Output i of SplitMix64 depends only on seed + (i + 1) * 0x9e3779b97f4a7c15, so the whole
stream is computed at once. The values follow the same recipe as the test oracle's generator;
numpy's vectorised log/cos/sin may differ from the C library's in the last bit for rare inputs,
which changes nothing about the workload.
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (np.arange(1, n + 1, dtype=np.uint64) * _GAMMA)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def _unit(z: np.ndarray) -> np.ndarray:
    return (z >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def to_dtype(x32: np.ndarray, dtype: str) -> np.ndarray:
    """fp32 -> f16 (numpy float16) or bf16 (uint16 bits), round to nearest even."""
    x32 = np.ascontiguousarray(x32, np.float32)
    if dtype == "f16":
        return x32.astype(np.float16)
    u = x32.view(np.uint32).astype(np.uint64)
    u = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return u.astype(np.uint16)


def uniform(seed: int, shape, lo: float, hi: float, dtype: str = "f16") -> np.ndarray:
    n = int(np.prod(shape))
    x = (lo + (hi - lo) * _unit(splitmix64(seed, n))).astype(np.float32)
    return to_dtype(x, dtype).reshape(shape)


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0, dtype: str = "f16") -> np.ndarray:
    n = int(np.prod(shape))
    pairs = (n + 1) // 2
    z = splitmix64(seed, 2 * pairs)
    u1 = 1.0 - _unit(z[0::2])
    u2 = _unit(z[1::2])
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(2 * pairs, np.float64)
    out[0::2] = mean + std * r * np.cos(2.0 * np.pi * u2)
    out[1::2] = mean + std * r * np.sin(2.0 * np.pi * u2)
    return to_dtype(out[:n].astype(np.float32), dtype).reshape(shape)
