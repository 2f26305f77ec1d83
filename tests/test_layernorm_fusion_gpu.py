"""Residual + LayerNorm across two GEMMs, through the C ABI: a residual GEMM writes its rows'
64-column chunk statistics (raya_gemm_epilogue.out_row_stats), raya_row_norm_stats turns them
into each row's mean and 1/sqrt(var + eps), and the next GEMM normalises its A rows on the fly
(in_row_stats, the norm's gain folded into the weight's columns).  This is the pre-LN encoder
step h += x Wo^T; LayerNorm(h) Wi^T of encoder::layer (crates/raya-core/src/encoder.rs:127-146).

Oracle: ops::layer_norm (crates/raya-core/src/ops.rs:51-74: f64 mean and biased variance, the
mean subtracted before scaling, the result rounded to f32 and times the gain) followed by the
sequential-f32 Reference::matmul_nt (crates/raya-kernels/src/gemm.rs:22-37).

Every other residual row carries an offset of 0.5, 10, 100 or 1000 times its spread, the
rows between stay around zero.  Subtracting mean * colsum(g W) after the contraction loses
|mean| / sigma of the product's digits (1.6e-4 at 100 sigma on these shapes): the GEMM
centres the rows more than one sigma from zero and takes the others' means out afterwards,
and both kinds share every workgroup here.  The bar is the forward goldens' 1e-5 per stage
(crates/raya-cli/tests/forward_golden.rs:21-22) on outputs of order one.
"""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

EPS = 1e-12
M, D, KIN = 1000, 768, 256


def _dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")


def residual_rows(rng, offset):
    """h = res + x Wo^T on the device with its chunk statistics; the even rows of res are
    offset by +-offset (times 0.5..1.5) around N(0, 1), the odd rows are not."""
    sign = np.where(rng.random(M) < 0.5, -1.0, 1.0)
    shift = offset * sign * (0.5 + rng.random(M)) * (np.arange(M) % 2 == 0)
    res = (shift[:, None] + rng.standard_normal((M, D))).astype(np.float32)
    x = (0.5 * rng.standard_normal((M, KIN))).astype(np.float32)
    wo = (0.02 * rng.standard_normal((D, KIN))).astype(np.float32)
    return res, x, wo


@pytest.mark.parametrize("offset", [0.5, 10.0, 100.0, 1000.0])
def test_layernorm_across_gemms_matches_the_oracle(hip_gemm, offset):
    rng = np.random.default_rng(int(offset) + 7)
    res, x, wo = residual_rows(rng, offset)
    print(f"row offset {offset:g} sigma: residual GEMM [{M}, {D}] from k = {KIN}", flush=True)
    h = torch.empty((M, D), device="cuda:0")
    chunks = torch.full((M, D // 64, 4), float("nan"), device="cuda:0")
    res_d = _dev(res)
    hip_gemm.matmul_nt_device(h, _dev(x), _dev(wo), residual=res_d, out_row_stats=chunks)
    rows = torch.full((M, 4), float("nan"), device="cuda:0")
    hip_gemm.row_norm_stats(chunks, rows, EPS)
    torch.cuda.synchronize()
    hh = h.cpu().numpy()

    # the residual add itself: the oracle's product plus res, within one unit in the last place
    want_h = oracle.matmul_nt(x, wo, threads=8) + res
    assert (np.abs(hh - want_h) <= np.spacing(np.abs(want_h)) + 1e-6).all()

    # the row statistics against f64 over the device's own rows
    st = rows.cpu().numpy().astype(np.float64)
    h64 = hh.astype(np.float64)
    mean, sd = h64.mean(1), h64.std(1)
    err_mean = np.abs(st[:, 0] + st[:, 1] - mean) / sd
    err_rstd = np.abs(st[:, 2] * np.sqrt(sd ** 2 + EPS) - 1.0)
    print(f"  mean error {err_mean.max():.1e} sigma, rstd relative error {err_rstd.max():.1e}")
    assert err_mean.max() <= 1e-6 and err_rstd.max() <= 1e-6
    assert (st[:, 3] == 0).all()

    gain = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    ln = oracle.layer_norm(hh, gain, None, np.float32(EPS))
    # QKV-shaped (plain) and GeGLU-shaped products of the normalised rows
    wqkv = (0.02 * rng.standard_normal((3 * D, D))).astype(np.float32)
    wi = (0.02 * rng.standard_normal((2 * 512, D))).astype(np.float32)
    for name, w, act in (("qkv", wqkv, 0), ("geglu", wi, 3)):
        n = w.shape[0] // (2 if act == 3 else 1)
        out = torch.full((M, n), float("nan"), device="cuda:0")
        folded = _dev(w * gain[None, :])
        sums = torch.empty(w.shape[0], device="cuda:0")
        hip_gemm.weight_row_sums(folded, sums)
        hip_gemm.matmul_nt_device(out, h, folded, activation=act, in_row_stats=rows, in_weight_sums=sums)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        prod = oracle.matmul_nt(ln, w, threads=8)
        want = prod if act == 0 else oracle.gelu_array(prod[:, :n]) * prod[:, n:]
        err = float(np.abs(got - want).max())
        print(f"  {name}: max-abs {err:.2e} against LayerNorm then matmul_nt")
        assert err <= 1e-5, (name, err)
        want_sums = (w * gain[None, :]).astype(np.float64).sum(1)
        assert np.abs(sums.cpu().numpy() - want_sums).max() <= 1e-7 * np.abs(want_sums).max()


def test_row_statistics_argument_checks(hip_gemm):
    """Shapes the ring kernel cannot take are refused before any launch."""
    from raya_amd import UnsupportedError

    a = torch.zeros((8, 24), device="cuda:0")
    b = torch.zeros((64, 24), device="cuda:0")
    out = torch.zeros((8, 64), device="cuda:0")
    with pytest.raises(UnsupportedError):  # k = 24 is not a multiple of 16
        hip_gemm.matmul_nt_device(out, a, b, out_row_stats=torch.zeros((8, 1, 4), device="cuda:0"))
    a = torch.zeros((8, 32), device="cuda:0")
    b = torch.zeros((96, 32), device="cuda:0")
    out = torch.zeros((8, 96), device="cuda:0")
    with pytest.raises(Exception):  # n = 96 has a partial chunk
        hip_gemm.matmul_nt_device(out, a, b, out_row_stats=torch.zeros((8, 1, 4), device="cuda:0"))
    b = torch.zeros((64, 32), device="cuda:0")
    out = torch.zeros((8, 64), device="cuda:0")
    with pytest.raises(Exception):  # row statistics without the weight's row sums
        hip_gemm.matmul_nt_device(out, a, b, in_row_stats=torch.zeros((8, 4), device="cuda:0"))
