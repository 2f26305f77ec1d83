"""Pins the CPU oracle's GEMM and scalar ops (known answers of the reference's tests)."""
import math

import numpy as np
import pytest

import oracle


def test_matmul_nt_hand_values():
    """gemm_reference.rs:4-12."""
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[1, 0, -1], [2, 1, 0.5]], np.float32)
    assert np.array_equal(oracle.matmul_nt(a, b), np.array([[-2, 5.5], [-2, 16]], np.float32))


def test_matmul_nt_empty_k_is_zero():
    """gemm_reference.rs:14-21."""
    out = oracle.matmul_nt(np.zeros((2, 0), np.float32), np.zeros((3, 0), np.float32))
    assert out.shape == (2, 3) and (out == 0).all()


def test_matmul_nt_nan_and_inf():
    """gemm_edges.rs:26-51."""
    out = oracle.matmul_nt(np.array([[np.nan, 1]], np.float32), np.ones((2, 2), np.float32))
    assert np.isnan(out).all()
    out = oracle.matmul_nt(np.array([[np.inf, 1]], np.float32), np.array([[1, 0], [-1, 0]], np.float32))
    assert out[0, 0] == np.inf and out[0, 1] == -np.inf
    out = oracle.matmul_nt(np.array([[np.inf, 1]], np.float32), np.array([[0, 1], [1, 1]], np.float32))
    assert np.isnan(out[0, 0]) and out[0, 1] == np.inf


def test_matmul_nt_within_the_reordering_bound_of_float64():
    """specs/009 bound: |out - exact| <= k * 2^-24 * sum|a_t b_t| for sequential f32 sums."""
    rng = np.random.default_rng(0)
    for m, n, k in ((1, 1, 1), (3, 5, 7), (17, 9, 33), (64, 64, 64), (130, 31, 257)):
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((n, k)).astype(np.float32)
        got = oracle.matmul_nt(a, b).astype(np.float64)
        exact = a.astype(np.float64) @ b.astype(np.float64).T
        bound = k * 2.0 ** -24 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64).T)
        assert (np.abs(got - exact) <= bound + 1e-30).all()
        # the threaded variant is the same per-row loop
        assert np.array_equal(oracle.matmul_nt(a, b, threads=4), got.astype(np.float32))


def test_erf_known_values():
    """crates/raya-core/tests/ops.rs:9-25."""
    for x, want in ((0.0, 0.0), (0.5, 0.5204998778130465), (1.0, 0.8427007929497149),
                    (2.0, 0.9953222650189527), (2.5, 0.999593047982555),
                    (3.0, 0.9999779095030014), (4.0, 0.9999999845827421)):
        assert abs(oracle.erf(x) - want) < 1e-12 and abs(oracle.erf(-x) + want) < 1e-12
        assert abs(oracle.erf(x) - math.erf(x)) < 1e-12
    assert oracle.erf(7.0) == 1.0 and oracle.erf(-7.0) == -1.0
    assert abs(oracle.erf(2.5 - 1e-9) - oracle.erf(2.5 + 1e-9)) < 1e-8


def test_gelu_is_exact_not_tanh():
    """ops.rs:33-43."""
    assert oracle.gelu(0.0) == 0.0
    assert abs(oracle.gelu(1.0) - 0.84134475) < 1e-7
    assert abs(oracle.gelu(-1.0) + 0.15865525) < 1e-7
    assert abs(oracle.gelu(1.0) - 0.841192) > 1e-4
    assert abs(oracle.gelu(-10.0)) < 1e-12 and abs(oracle.gelu(10.0) - 10.0) < 1e-6


def test_layer_norm_biased_variance():
    """ops.rs:45-59."""
    x = np.array([[1, 2, 3, 4], [10, 10, 10, 10]], np.float32)
    out = oracle.layer_norm(x, np.ones(4, np.float32), None, 0.0)
    assert np.abs(out[0] - np.array([-1.3416408, -0.4472136, 0.4472136, 1.3416408])).max() < 1e-6
    out = oracle.layer_norm(x, np.full(4, 2.0, np.float32), np.full(4, 0.5, np.float32), 1e-5)
    assert np.abs(out[1] - 0.5).max() < 1e-6


def test_softmax_shift_invariance():
    """ops.rs:61-74."""
    a = oracle.softmax(np.array([1, 2, 3], np.float32))
    b = oracle.softmax(np.array([1001, 1002, 1003], np.float32))
    assert abs(a.sum() - 1) < 1e-6 and np.abs(a - b).max() < 1e-6
    assert np.array_equal(oracle.softmax(np.array([0.5, -1e4], np.float32)), np.array([1, 0], np.float32))


def test_rope_rotate_half():
    """ops.rs:76-92."""
    x = oracle.rope(np.array([1, 0, 0, 0, 1, 0, 0, 0], np.float32).reshape(1, 2, 4), 10000.0).ravel()
    assert np.array_equal(x[:4], np.array([1, 0, 0, 0], np.float32))
    assert abs(x[4] - np.cos(np.float32(1))) < 1e-6 and abs(x[6] - np.sin(np.float32(1))) < 1e-6
    assert abs(x[5]) < 1e-7 and abs(x[7]) < 1e-7
    y = oracle.rope(np.array([0, 1, 0, 0, 0, 1, 0, 0], np.float32).reshape(1, 2, 4), 10000.0).ravel()
    assert abs(y[5] - np.cos(np.float32(0.01))) < 1e-6 and abs(y[7] - np.sin(np.float32(0.01))) < 1e-6
    assert abs((x[4:] ** 2).sum() - 1) < 1e-6


def _folded_layernorm_f32(h, w, mode: str):
    """LayerNorm(h) W^T (gain 1) folded into one f32 product as the GEMM computes it:
    statistics in f64 rounded to f32 (mean = hi + lo); the operands enter as h - c and the
    rest of the mean comes out afterwards, y = rstd (acc - ((hi - c) + lo) colsum).  c = 0
    for every row ("after"), c = hi for every row ("centre"), or the GEMM's rule ("rows"):
    c = hi for rows with |hi| rstd > 1, else 0."""
    h64 = h.astype(np.float64)
    mean, rstd = h64.mean(1), (1.0 / np.sqrt(h64.var(1) + 1e-12)).astype(np.float32)
    hi = mean.astype(np.float32)
    lo = (mean - hi).astype(np.float32)
    if mode == "after":
        c = np.zeros_like(hi)
    elif mode == "centre":
        c = hi
    else:
        c = np.where(np.abs(hi) * rstd > 1, hi, np.float32(0))
    colsum = w.astype(np.float64).sum(1).astype(np.float32)
    acc = (h - c[:, None]) @ w.T
    rest = (hi - c) + lo
    return rstd[:, None] * (acc - rest[:, None] * colsum[None, :])


@pytest.mark.parametrize("offset", [0.0, 0.9, 1.1, 10.0, 100.0])
def test_folded_layernorm_bar_separates_the_folds(offset):
    """The bar of the device test of the folded LayerNorm (1e-5 against LayerNorm then
    matmul_nt) passes the GEMM's per-row rule at every offset, including rows on either
    side of its one-sigma threshold, and fails the fold that subtracts mean * colsum after
    the product once rows sit 100 sigma from zero: the test tells them apart."""
    rng = np.random.default_rng(3)
    h = (offset + rng.standard_normal((64, 768))).astype(np.float32)
    w = (0.02 * rng.standard_normal((256, 768))).astype(np.float32)
    want = oracle.matmul_nt(oracle.layer_norm(h, np.ones(768, np.float32), None, np.float32(1e-12)), w,
                            threads=8)
    for mode in ("rows", "centre"):
        err = np.abs(_folded_layernorm_f32(h, w, mode) - want).max()
        assert err <= 1e-5, (mode, err)
    after = np.abs(_folded_layernorm_f32(h, w, "after") - want).max()
    if offset >= 100:
        assert after > 1e-5, after
    elif offset <= 1.1:
        assert after <= 5e-6, after  # within the threshold the mean may come out afterwards
