"""Parity of the MFMA GEMM with the oracle's Reference::matmul_nt, through the C ABI.

Bar (specs/009-gemm-backend-comparison/spec.md:24): every element within
2 * k * 2^-24 * sum_t |a_t b_t| of the sequential f32 result; hand values and
NaN/Inf propagation exact, as the reference's tests pin them.
"""
import numpy as np
import pytest
import torch

import oracle
import raya_amd as R
from raya_amd import _capi as C

pytestmark = pytest.mark.gpu


def bound(a, b):
    k = a.shape[1]
    return 2 * k * 2.0 ** -24 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64).T)


def run(gemm, a, b):
    m, k = a.shape
    n = b.shape[0]
    out = np.full((m, n), 3.0, np.float32)
    gemm.matmul_nt(out.reshape(-1), a.reshape(-1), b.reshape(-1), m, n, k)
    return out


def test_hand_values(hip_gemm):
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[1, 0, -1], [2, 1, 0.5]], np.float32)
    assert np.array_equal(run(hip_gemm, a, b), np.array([[-2, 5.5], [-2, 16]], np.float32))


def test_empty_k_overwrites_with_zeros(hip_gemm):
    out = np.full(6, 5.0, np.float32)
    hip_gemm.matmul_nt(out, np.zeros(0, np.float32), np.zeros(0, np.float32), 2, 3, 0)
    assert (out == 0).all()


def test_nan_and_inf_propagate(hip_gemm):
    assert np.isnan(run(hip_gemm, np.array([[np.nan, 1]], np.float32), np.ones((2, 2), np.float32))).all()
    out = run(hip_gemm, np.array([[np.inf, 1]], np.float32), np.array([[1, 0], [-1, 0]], np.float32))
    assert out[0, 0] == np.inf and out[0, 1] == -np.inf
    out = run(hip_gemm, np.array([[np.inf, 1]], np.float32), np.array([[0, 1], [1, 1]], np.float32))
    assert np.isnan(out[0, 0]) and out[0, 1] == np.inf


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (3, 5, 7), (17, 9, 33), (64, 64, 64), (130, 31, 257),
                                   (256, 2304, 768), (300, 768, 3072), (129, 6144, 768),
                                   # k = 16, 32, 48: one, two and three 16-deep slabs in the LDS ring
                                   (70, 40, 16), (70, 40, 32), (200, 130, 48)])
def test_within_the_reordering_bound(hip_gemm, m, n, k):
    rng = np.random.default_rng(m * 7 + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = (0.02 * rng.standard_normal((n, k))).astype(np.float32)
    got = run(hip_gemm, a, b).astype(np.float64)
    want = oracle.matmul_nt(a, b, threads=8).astype(np.float64)
    assert (np.abs(got - want) <= bound(a, b)).all()


def test_mfma_accumulation_is_full_fp32(hip_gemm):
    """The MFMA path is no less accurate than sequential fp32: against a float64
    product, its RMS error (relative to sum|a b|) is at most twice that of
    Reference::matmul_nt.  A reduced-precision product (tf32, bf16 splits)
    would be orders of magnitude worse."""
    rng = np.random.default_rng(11)
    m, n, k = 512, 384, 768
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k)).astype(np.float32)
    exact = a.astype(np.float64) @ b.astype(np.float64).T
    scale = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64).T
    e_gpu = np.abs(run(hip_gemm, a, b) - exact) / scale
    e_seq = np.abs(oracle.matmul_nt(a, b, threads=8) - exact) / scale
    rms_gpu, rms_seq = np.sqrt((e_gpu ** 2).mean()), np.sqrt((e_seq ** 2).mean())
    print(f"rms relative error: mfma {rms_gpu:.3g}, sequential {rms_seq:.3g}")
    assert rms_gpu <= 2 * rms_seq


def _dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


@pytest.mark.parametrize("act", ["none", "gelu", "relu", "geglu"])
@pytest.mark.parametrize("residual", [False, True])
@pytest.mark.parametrize("k", [136, 128])
def test_device_epilogues(hip_gemm, act, residual, k):
    """bias + activation (+ residual) against the oracle's matmul_nt and scalar ops, on both
    kernels (k = 128: the LDS-ring kernel; k = 136: the general one)."""
    rng = np.random.default_rng(5)
    m, n = 200, 96
    rows_b = 2 * n if act == "geglu" else n
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = (0.1 * rng.standard_normal((rows_b, k))).astype(np.float32)
    bias = rng.standard_normal(rows_b).astype(np.float32)
    res = rng.standard_normal((m, n)).astype(np.float32)
    y = oracle.matmul_nt(a, b) + bias
    if act == "gelu":
        want = oracle.gelu_array(y)
    elif act == "relu":
        want = np.maximum(y, 0)
    elif act == "geglu":
        want = oracle.gelu_array(y[:, :n]) * y[:, n:]
    else:
        want = y
    if residual:
        want = want + res
    code = {"none": C.RAYA_EPI_NONE, "gelu": C.RAYA_EPI_GELU, "relu": C.RAYA_EPI_RELU,
            "geglu": C.RAYA_EPI_GEGLU}[act]
    out = _dev(res) if residual else torch.full((m, n), 9.0, device="cuda")
    hip_gemm.matmul_nt_device(out, _dev(a), _dev(b), bias=_dev(bias), activation=code,
                              residual=out if residual else None)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.abs(got - want).max() < 1e-4 * max(1.0, float(np.abs(want).max()))


@pytest.mark.parametrize("act", ["none", "gelu", "geglu"])
@pytest.mark.parametrize("residual", [False, True])
def test_strided_out_vector_and_scalar_epilogues_agree(hip_gemm, act, residual):
    """n = 70 inside rows of 72 floats takes the float4 (LDS-staged) epilogue, with a
    partial last float4; rows of 70 floats take the per-element one.  Both give the
    same bits, and the two columns past n are left alone."""
    rng = np.random.default_rng(13)
    m, n, k = 150, 70, 64
    code = {"none": C.RAYA_EPI_NONE, "gelu": C.RAYA_EPI_GELU, "geglu": C.RAYA_EPI_GEGLU}[act]
    rows_b = 2 * n if act == "geglu" else n
    a = _dev(rng.standard_normal((m, k)).astype(np.float32))
    b = _dev((0.1 * rng.standard_normal((rows_b, k))).astype(np.float32))
    bias = _dev(rng.standard_normal(rows_b).astype(np.float32))
    res = rng.standard_normal((m, n)).astype(np.float32)
    outs = []
    for ld in (72, 70):
        buf = torch.full((m, ld), 9.0, device="cuda")
        out = buf[:, :n]
        if residual:
            out.copy_(_dev(res))
        hip_gemm.matmul_nt_device(out, a, b, bias=bias, activation=code,
                                  residual=out if residual else None)
        torch.cuda.synchronize()
        outs.append(buf.cpu().numpy())
    assert np.array_equal(outs[0][:, :n], outs[1])
    assert (outs[0][:, n:] == 9.0).all()
    y = oracle.matmul_nt(a.cpu().numpy(), b.cpu().numpy()) + bias.cpu().numpy()
    want = {"none": lambda: y, "gelu": lambda: oracle.gelu_array(y),
            "geglu": lambda: oracle.gelu_array(y[:, :n]) * y[:, n:]}[act]()
    if residual:
        want = want + res
    assert np.abs(outs[1] - want).max() < 1e-4 * max(1.0, float(np.abs(want).max()))


def test_random_sweep_of_shapes_and_epilogues(hip_gemm):
    """40 random device GEMMs against the oracle's Reference::matmul_nt: m, n, k from 1 to
    several hundred (k a multiple of 16 in half of them, the LDS-ring kernel), every
    activation, optional bias and residual, and row strides larger than n in a third of them.
    The bound is the reordering bound above, carried through the epilogue (GELU's slope is
    at most 1.13; GeGLU's product takes each factor's error times the other factor)."""
    rng = np.random.default_rng(77)
    acts = ["none", "gelu", "relu", "geglu"]
    for case in range(40):
        m, n = int(rng.integers(1, 600)), int(rng.integers(1, 400))
        k = 16 * int(rng.integers(1, 40)) if case % 2 == 0 else int(rng.integers(1, 400))
        act = acts[case % 4]
        rows_b = 2 * n if act == "geglu" else n
        has_bias, has_res = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
        ld = n + (4 * int(rng.integers(1, 4)) if case % 3 == 0 else 0)
        print(f"case {case}: m{m} n{n} k{k} {act} bias {has_bias} residual {has_res} ld {ld}", flush=True)
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = (0.1 * rng.standard_normal((rows_b, k))).astype(np.float32)
        bias = rng.standard_normal(rows_b).astype(np.float32) if has_bias else np.zeros(rows_b, np.float32)
        res = rng.standard_normal((m, n)).astype(np.float32)
        y = oracle.matmul_nt(a, b).astype(np.float64) + bias
        err = bound(a, b) + 1e-7 * np.abs(y)
        if act == "geglu":
            x, g = y[:, :n], y[:, n:]
            gx = oracle.gelu_array(x.astype(np.float32)).astype(np.float64)
            want = gx * g
            err = 1.13 * err[:, :n] * np.abs(g) + np.abs(gx) * err[:, n:] + 1e-6 * np.abs(want)
        elif act == "gelu":
            want = oracle.gelu_array(y.astype(np.float32)).astype(np.float64)
            err = 1.13 * err + 1e-6 * np.abs(want)
        elif act == "relu":
            want = np.maximum(y, 0)
        else:
            want = y
        if has_res:
            want = want + res
        buf = torch.full((m, ld), 9.0, device="cuda")
        out = buf[:, :n]
        if has_res:
            out.copy_(_dev(res))
        code = {"none": C.RAYA_EPI_NONE, "gelu": C.RAYA_EPI_GELU, "relu": C.RAYA_EPI_RELU,
                "geglu": C.RAYA_EPI_GEGLU}[act]
        hip_gemm.matmul_nt_device(out, _dev(a), _dev(b), bias=_dev(bias) if has_bias else None,
                                  activation=code, residual=out if has_res else None)
        torch.cuda.synchronize()
        got = buf.cpu().numpy()
        diff = np.abs(got[:, :n].astype(np.float64) - want)
        tol = 2 * err + 1e-6 * (1 + np.abs(want))
        assert (diff <= tol).all(), (case, float((diff - tol).max()))
        assert (got[:, n:] == 9.0).all()


@pytest.mark.parametrize("shape", ["qkv", "wo", "geglu", "mlp_wo"])
def test_encoder_shapes_at_the_forward_row_count(hip_gemm, shape):
    """The four encoder projections at the measured forward's M = 21,405 packed tokens
    (167 whole 128-row tiles and a last one of 29 rows), with the epilogue each takes in the
    forward.  Every output element is held to the reordering bound around a float64 product
    computed on the device (the bound is what the sequential fp32 result itself meets), carried
    through GeGLU as in the sweep above.  The residual shapes pass `out` as their own residual,
    as the forward does."""
    m = 21405
    n, k, act, residual = {"qkv": (2304, 768, C.RAYA_EPI_NONE, False), "wo": (768, 768, C.RAYA_EPI_NONE, True),
                           "geglu": (3072, 768, C.RAYA_EPI_GEGLU, False),
                           "mlp_wo": (768, 3072, C.RAYA_EPI_NONE, True)}[shape]
    rows_b = 2 * n if act == C.RAYA_EPI_GEGLU else n
    gen = torch.Generator(device="cuda").manual_seed(2024)
    a = torch.randn(m, k, device="cuda", generator=gen)
    b = 0.02 * torch.randn(rows_b, k, device="cuda", generator=gen)
    res = torch.randn(m, n, device="cuda", generator=gen) if residual else None
    out = res.clone() if residual else torch.full((m, n), 9.0, device="cuda")
    hip_gemm.matmul_nt_device(out, a, b, activation=act, residual=out if residual else None)
    torch.cuda.synchronize()
    a64, b64 = a.double(), b.double()
    y = a64 @ b64.T
    err = 2 * k * 2.0 ** -24 * (a64.abs() @ b64.abs().T)
    if act == C.RAYA_EPI_GEGLU:
        x, g = y[:, :n], y[:, n:]
        gx = torch.nn.functional.gelu(x)  # exact erf form, float64
        want = gx * g
        err = 1.13 * err[:, :n] * g.abs() + gx.abs() * err[:, n:] + 1e-6 * want.abs()
    else:
        want = y
    if residual:
        want = want + res.double()
    diff = (out.double() - want).abs()
    tol = err + 1e-6 * (1 + want.abs())
    worst = float((diff - tol).max())
    print(f"{shape}: max |diff| {float(diff.max()):.3g}, worst margin {worst:.3g}")
    assert worst <= 0, worst
