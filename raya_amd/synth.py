"""Seeded synthetic inputs for the benchmark workloads.

SplitMix64 (Steele, Lea and Flood, OOPSLA 2014) gives 64-bit words; the top 53
bits make a uniform double in [0, 1); Box-Muller turns pairs into N(0, 1)
(rounded to f32).  The seed of stream s of workload c is 1000 * c + s:
0/1/2 = Q/K/V, 3 = valid lengths, 4 = outliers, 5 = weights, 6 = token ids.
Everything is vectorised numpy, generated in chunks so that large tensors do
not need temporaries of their full size.
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def splitmix64(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Outputs start .. start+n-1 of SplitMix64 seeded with `seed`."""
    with np.errstate(over="ignore"):
        i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Doubles in [0, 1) from the top 53 bits."""
    return (splitmix64(seed, n, start) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def normal(seed: int, n: int) -> np.ndarray:
    """n i.i.d. N(0, 1) values as float32 (Box-Muller on consecutive pairs)."""
    out = np.empty(n, dtype=np.float32)
    pairs = (n + 1) // 2
    for p0 in range(0, pairs, _CHUNK):
        p1 = min(pairs, p0 + _CHUNK)
        u = uniform(seed, 2 * (p1 - p0), 2 * p0)
        r = np.sqrt(-2.0 * np.log1p(-u[0::2]))
        th = (2.0 * np.pi) * u[1::2]
        z = np.empty(2 * (p1 - p0), dtype=np.float64)
        z[0::2] = r * np.cos(th)
        z[1::2] = r * np.sin(th)
        lo = 2 * p0
        hi = min(n, 2 * p1)
        out[lo:hi] = z[: hi - lo]
    return out


def integers(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    """n integers uniform in [lo, hi] inclusive."""
    u = uniform(seed, n)
    return (lo + np.floor(u * (hi - lo + 1))).astype(np.int64)


def with_outliers(x: np.ndarray, seed: int, p: float = 0.01, factor: float = 20.0) -> np.ndarray:
    """Scales each element by `factor` with probability p (in place)."""
    flat = x.reshape(-1)
    for s in range(0, flat.size, _CHUNK):
        e = min(flat.size, s + _CHUNK)
        hit = uniform(seed, e - s, s) < p
        flat[s:e][hit] *= np.float32(factor)
    return x


def workload_seed(config: int, stream: int) -> int:
    return 1000 * config + stream
