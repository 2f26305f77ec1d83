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


# ---------------------------------------------------------------------------
# The reference bench's inputs: xorshift64 (shifts 13, 7, 17) seeded with
# seed * 0x9E3779B97F4A7C15 | 1; each value is the top 24 bits of the state
# after a step, as u / 2^24, mapped to 2u - 1 in [-1, 1)
# (crates/raya-kernels/tests/common/mod.rs:6-18; q, k, v use seeds 42, 43, 44
# in benches/local_attention.rs:95).
#
# One xorshift step is linear over GF(2)^64, so the sequence is produced in
# parallel: `lanes` independent states start `chunk` steps apart (state
# advanced with T^chunk, T the step's 64x64 bit matrix) and all lanes step
# together with vectorised numpy.

_MASK64 = (1 << 64) - 1


def _xs_step(s: int) -> int:
    s ^= (s << 13) & _MASK64
    s ^= s >> 7
    s ^= (s << 17) & _MASK64
    return s


def _apply(cols, s: int) -> int:
    """Bit matrix (column j = image of bit j) applied to state s."""
    r = 0
    j = 0
    while s:
        if s & 1:
            r ^= cols[j]
        s >>= 1
        j += 1
    return r


def _power(cols, e: int):
    """Columns of the matrix raised to the power e."""
    result = [1 << j for j in range(64)]
    base = list(cols)
    while e:
        if e & 1:
            result = [_apply(base, c) for c in result]
        base = [_apply(base, c) for c in base]
        e >>= 1
    return result


def xorshift_uniform(seed: int, n: int, lanes: int = 4096) -> np.ndarray:
    """n values of the reference bench's generator, as float32 in [-1, 1)."""
    if n <= 0:
        return np.empty(0, dtype=np.float32)
    s0 = ((seed * 0x9E3779B97F4A7C15) & _MASK64) | 1
    lanes = max(1, min(lanes, n))
    chunk = (n + lanes - 1) // lanes
    step = [_xs_step(1 << j) for j in range(64)]
    jump = _power(step, chunk)
    starts = [s0]
    for _ in range(lanes - 1):
        starts.append(_apply(jump, starts[-1]))
    s = np.array(starts, dtype=np.uint64)
    vals = np.empty((chunk, lanes), dtype=np.float32)
    with np.errstate(over="ignore"):
        for i in range(chunk):
            s ^= s << np.uint64(13)
            s ^= s >> np.uint64(7)
            s ^= s << np.uint64(17)
            vals[i] = (s >> np.uint64(40)).astype(np.float32)
    u = vals.T.reshape(-1)[:n] * np.float32(1.0 / (1 << 24))
    return np.float32(2.0) * u - np.float32(1.0)
