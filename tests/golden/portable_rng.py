"""Portable seeded N(0,1) generator for the golden fixtures.

splitmix64 (Steele, Lea, Flood, "Fast splittable pseudorandom number
generators", OOPSLA 2014) produces 64-bit words; the top 53 bits become
uniforms in (0, 1]; Box-Muller in f64 turns pairs of uniforms into normals,
which are rounded once to f32. Everything is integer or correctly rounded f64
arithmetic in numpy, so every machine produces the same f32 bits, and the
fixtures only need to store a seed and a digest of the inputs.
"""
from __future__ import annotations

import hashlib

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int) -> np.ndarray:
    """The first n outputs of splitmix64 started at `seed`."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + _GAMMA * np.arange(1, n + 1, dtype=np.uint64)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def normal_f32(seed: int, n: int) -> np.ndarray:
    """n standard normals (f32) from splitmix64 + Box-Muller."""
    m = (n + 1) // 2
    words = splitmix64(seed, 2 * m)
    u = ((words >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return z[:n].astype(np.float32)


def permutation(seed: int, n: int) -> np.ndarray:
    """A permutation of range(n): argsort of n splitmix64 words (ties impossible
    in practice; stable sort makes the result deterministic regardless)."""
    return np.argsort(splitmix64(seed, n), kind="stable").astype(np.int64)


def digest(*arrays: np.ndarray) -> str:
    """sha256 over the raw bytes of the arrays, in order."""
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()
