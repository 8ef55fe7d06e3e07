"""Deterministic, portable synthetic inputs (weights, token ids, labels).

SplitMix64 streams (Steele, Lea & Flood, "Fast splittable pseudorandom number
generators", OOPSLA 2014): the same integers on every platform and in every
language, unlike ``std::*_distribution``.  Uniforms take the top 24 bits
(``u = (x >> 40) * 2**-24``, exact in float32); normals use Box-Muller in
double precision, rounded once to float32.
"""
from __future__ import annotations

import zlib

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z):
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def stream_seed(seed: int, name: str) -> int:
    """Independent stream per (seed, name)."""
    with np.errstate(over="ignore"):
        s = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) ^ np.uint64(zlib.crc32(name.encode()))
        return int(_mix(np.array([s], dtype=np.uint64))[0])


def raw(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """n consecutive SplitMix64 outputs of the stream starting at `seed`."""
    with np.errstate(over="ignore"):
        k = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        return _mix(np.uint64(seed) + k * _GOLDEN)


def uniform01(seed: int, n: int) -> np.ndarray:
    """float64 uniforms in [0, 1) with 24 random bits."""
    return (raw(seed, n) >> np.uint64(40)).astype(np.float64) * (2.0 ** -24)


def uniform(seed: int, n: int, lo: float, hi: float) -> np.ndarray:
    return (lo + (hi - lo) * uniform01(seed, n)).astype(np.float32)


def normal(seed: int, n: int, std: float = 1.0) -> np.ndarray:
    u = uniform01(seed, 2 * n).reshape(n, 2)
    z = np.sqrt(-2.0 * np.log1p(-u[:, 0])) * np.cos(2.0 * np.pi * u[:, 1])
    return (z * std).astype(np.float32)


def xavier_uniform(seed: int, fan_in: int, fan_out: int) -> np.ndarray:
    a = np.sqrt(6.0 / (fan_in + fan_out))
    return uniform(seed, fan_in * fan_out, -a, a)


def token_ids(seed: int, n: int, vocab: int) -> np.ndarray:
    """floor(u * vocab) as float32 (ids travel as floats through the ABI)."""
    return np.floor(uniform01(seed, n) * vocab).astype(np.float32)


def one_hot(ids: np.ndarray, classes: int) -> np.ndarray:
    y = np.zeros((ids.size, classes), dtype=np.float32)
    y[np.arange(ids.size), ids.astype(np.int64)] = 1.0
    return y.ravel()
