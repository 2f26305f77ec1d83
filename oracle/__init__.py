"""CPU oracle for the block-local attention hot path (TEST INFRASTRUCTURE ONLY).

This package is the checker.  Only the test suite, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it: to check the HIP
path's results, or to time the reference algorithm on the host.  The product
(``raya_amd`` and ``libraya_hip.so``) never imports it and never falls back to
it.

The C sources (``attention.c``, ``gemm.c``, ``ops.c``) restate the reference's
Rust algorithms and cite the file:line each follows; ``oracle.h`` lists how
every function is pinned.  This module is a thin ctypes/numpy wrapper.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

MASK_BLOCK3, MASK_WINDOW64, MASK_FULL, MASK_SLIDING, MASK_BLOCKDIAG = 0, 1, 2, 3, 4

_u64, _i32, _f32, _dbl = ctypes.c_uint64, ctypes.c_int, ctypes.c_float, ctypes.c_double
_fp = ctypes.POINTER(ctypes.c_float)
_ip = ctypes.POINTER(ctypes.c_int32)


def build() -> str:
    """Compile liboracle.so with the committed Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_key_range.argtypes = [_i32, _u64, _u64, _u64, _u64,
                                       ctypes.POINTER(_u64), ctypes.POINTER(_u64)]
        L.oracle_allows.argtypes = [_i32, _u64, _u64, _u64, _u64]
        L.oracle_allows.restype = _i32
        att = [_u64, _u64, _u64, _i32, _u64, _u64, _u64, _f32, _fp, _fp, _fp, _fp]
        L.oracle_naive_attend.argtypes = att
        L.oracle_dense_attend.argtypes = att
        L.oracle_naive_attend_batched.argtypes = [_u64, _u64, _u64, _u64, _i32, _u64, _u64,
                                                  _ip, _f32, _fp, _fp, _fp, _fp]
        L.oracle_tiled_attend_batched.argtypes = [_u64, _u64, _u64, _u64, _i32, _u64, _u64,
                                                  _ip, _f32, _fp, _fp, _fp, _fp, _i32, _i32]
        L.oracle_tiled_attend_batched.restype = _i32
        L.oracle_cpu_has_avx2_fma.restype = _i32
        L.oracle_matmul_nt.argtypes = [_fp, _fp, _fp, _u64, _u64, _u64]
        L.oracle_matmul_nt_threaded.argtypes = [_fp, _fp, _fp, _u64, _u64, _u64, _i32]
        L.oracle_erf.argtypes = [_dbl]
        L.oracle_erf.restype = _dbl
        L.oracle_gelu.argtypes = [_f32]
        L.oracle_gelu.restype = _f32
        L.oracle_gelu_vec.argtypes = [_fp, _fp, _u64]
        L.oracle_layer_norm.argtypes = [_fp, _fp, _fp, _fp, _f32, _u64, _u64]
        L.oracle_softmax.argtypes = [_fp, _u64]
        L.oracle_rope.argtypes = [_fp, _u64, _u64, _u64, _f32]
        L.oracle_rand_vec.argtypes = [_u64, _u64, _fp]
        L.oracle_lcg_fill.argtypes = [_u64, ctypes.c_uint32, _fp]
        _lib = L
    return _lib


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)


def _c32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def key_range(kind: int, i: int, valid_len: int, block: int = 128, window: int = 0):
    lo, hi = _u64(), _u64()
    lib().oracle_key_range(kind, block, window, i, valid_len, ctypes.byref(lo), ctypes.byref(hi))
    return lo.value, hi.value


def allows(kind: int, i: int, j: int, block: int = 128, window: int = 0) -> bool:
    return bool(lib().oracle_allows(kind, block, window, i, j))


def naive_attend(q, k, v, kind, valid_len, scale, block=128, window=0):
    """Naive::attend on one sequence; q/k/v are [heads, seq, head_dim]."""
    q, k, v = _c32(q), _c32(k), _c32(v)
    h, s, d = q.shape
    out = np.empty_like(q)
    lib().oracle_naive_attend(h, s, d, kind, block, window, valid_len, scale,
                              _f(q), _f(k), _f(v), _f(out))
    return out


def dense_attend(q, k, v, kind, valid_len, scale, block=128, window=0):
    q, k, v = _c32(q), _c32(k), _c32(v)
    h, s, d = q.shape
    out = np.empty_like(q)
    lib().oracle_dense_attend(h, s, d, kind, block, window, valid_len, scale,
                              _f(q), _f(k), _f(v), _f(out))
    return out


def naive_attend_batched(q, k, v, kind, valid_lens, scale, block=128, window=0):
    """q/k/v are [batch, heads, seq, head_dim]; valid_lens is [batch]."""
    q, k, v = _c32(q), _c32(k), _c32(v)
    b, h, s, d = q.shape
    vl = np.ascontiguousarray(valid_lens, dtype=np.int32)
    out = np.empty_like(q)
    lib().oracle_naive_attend_batched(b, h, s, d, kind, block, window, vl.ctypes.data_as(_ip),
                                      scale, _f(q), _f(k), _f(v), _f(out))
    return out


def tiled_attend_batched(q, k, v, kind, valid_lens, scale, block=128, window=0,
                         threads=1, backend=1, out=None):
    """The Tiled CPU algorithm; returns (out, backend_used)."""
    q, k, v = _c32(q), _c32(k), _c32(v)
    b, h, s, d = q.shape
    vl = np.ascontiguousarray(valid_lens, dtype=np.int32)
    if out is None:
        out = np.empty_like(q)
    used = lib().oracle_tiled_attend_batched(b, h, s, d, kind, block, window,
                                             vl.ctypes.data_as(_ip), scale, _f(q), _f(k), _f(v),
                                             _f(out), threads, backend)
    return out, used


def cpu_has_avx2_fma() -> bool:
    return bool(lib().oracle_cpu_has_avx2_fma())


def matmul_nt(a, b, threads: int = 1):
    a, b = _c32(a), _c32(b)
    m, k = a.shape
    n = b.shape[0]
    out = np.empty((m, n), dtype=np.float32)
    if threads > 1:
        lib().oracle_matmul_nt_threaded(_f(out), _f(a), _f(b), m, n, k, threads)
    else:
        lib().oracle_matmul_nt(_f(out), _f(a), _f(b), m, n, k)
    return out


def erf(x: float) -> float:
    return lib().oracle_erf(x)


def gelu(x: float) -> float:
    return lib().oracle_gelu(x)


def gelu_array(x) -> np.ndarray:
    x = _c32(x)
    out = np.empty_like(x)
    lib().oracle_gelu_vec(_f(out), _f(x), x.size)
    return out


def layer_norm(x, weight, bias, eps):
    x = _c32(x)
    d = x.shape[-1]
    rows = x.size // d
    w = _c32(weight)
    out = np.empty_like(x)
    bb = _c32(bias) if bias is not None else None
    bp = _f(bb) if bb is not None else None
    lib().oracle_layer_norm(_f(out), _f(x), _f(w), bp, eps, rows, d)
    return out


def softmax(x):
    x = _c32(x).copy()
    lib().oracle_softmax(_f(x), x.size)
    return x


def rope(x, theta):
    """Rotate-half RoPE in place on a copy of [heads, seq, head_dim]."""
    x = _c32(x).copy()
    h, s, d = x.shape
    lib().oracle_rope(_f(x), h, s, d, theta)
    return x


def rand_vec(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().oracle_rand_vec(n, seed, _f(out))
    return out


def lcg_fill(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().oracle_lcg_fill(n, seed, _f(out))
    return out


def qkv(heads: int, seq: int, head_dim: int, seed: int):
    """qkv(shape, seed) of crates/raya-kernels/tests/common/mod.rs:20-27."""
    n = heads * seq * head_dim
    shp = (heads, seq, head_dim)
    return (rand_vec(n, seed).reshape(shp), rand_vec(n, seed + 1).reshape(shp),
            rand_vec(n, seed + 2).reshape(shp))
