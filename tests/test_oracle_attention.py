"""Pins the CPU oracle's attention before it is trusted as the checker.

Sources of truth, none of them a retyping of the oracle's own loop:
* the reference's golden tensors block_local_L256 (q, k, v, `reference`,
  `kernel`), checked as crates/raya-kernels/tests/goldens.rs:35-80 does;
* the reference's dense brute force (tests/common/mod.rs:39-84), restated in
  C as oracle_dense_attend, at the reference's 1e-6 (tests/oracle.rs:7-32);
* torch's scaled_dot_product_attention in float64 with an explicit boolean
  mask built from the mask definitions (an independent library routine);
* invariants of the reference's tests: exact masks (masking.rs:20-61),
  exact-zero padding (masking.rs:63-91), extreme logits (masking.rs:93-125),
  single valid row (masks_edges.rs:90-107).
"""
import json
import math
import os

import numpy as np
import pytest
import torch
from safetensors.numpy import load_file

import oracle
from tests.conftest import GOLDEN

B3, W64, FULL, SL, BD = (oracle.MASK_BLOCK3, oracle.MASK_WINDOW64, oracle.MASK_FULL,
                         oracle.MASK_SLIDING, oracle.MASK_BLOCKDIAG)


def scale_of(d):
    return float(np.float32(1.0) / np.sqrt(np.float32(d)))


def allowed_matrix(kind, seq, valid, block=128, window=0):
    """Boolean [seq, seq] mask from the mask definitions (attention.rs:62-69)."""
    i = np.arange(seq)[:, None]
    j = np.arange(seq)[None, :]
    if kind == B3:
        m = np.abs(i // 128 - j // 128) <= 1
    elif kind == W64:
        m = np.abs(i - j) <= 64
    elif kind == FULL:
        m = np.ones((seq, seq), bool)
    elif kind == SL:
        m = np.abs(i - j) <= window
    else:
        m = (i // block) == (j // block)
    return m & (i < valid) & (j < valid)


def sdpa_reference(q, k, v, kind, valid, block=128, window=0):
    """torch SDPA in float64; rows with no allowed key are zero."""
    h, s, d = q.shape
    m = torch.from_numpy(allowed_matrix(kind, s, valid, block, window))
    qt, kt, vt = (torch.from_numpy(x.astype(np.float64)) for x in (q, k, v))
    out = torch.nn.functional.scaled_dot_product_attention(
        qt, kt, vt, attn_mask=m, scale=scale_of(d))
    empty = ~m.any(dim=1)
    out[:, empty, :] = 0.0
    return out.numpy()


def golden():
    d = os.path.join(GOLDEN, "block_local_L256")
    meta = json.load(open(os.path.join(d, "meta.json")))
    t = load_file(os.path.join(d, "tensors.safetensors"))
    return meta, t


def test_golden_meta_is_the_block_local_case():
    meta, t = golden()
    assert meta["pattern"] == "block_local" and meta["scale"] == "1/sqrt(head_dim)"
    assert meta["block"] == 128 and meta["tolerance"] == 1e-5
    assert t["q"].shape == (1, meta["heads"], meta["length"], meta["head_dim"])


@pytest.mark.parametrize("which", ["reference", "kernel"])
def test_naive_and_tiled_match_the_golden(which):
    """goldens.rs:35-80: Naive and Tiled (Block3) vs both golden outputs at 1e-5."""
    _, t = golden()
    q, k, v = t["q"][0], t["k"][0], t["v"][0]
    h, s, d = q.shape
    want = t[which][0]
    naive = oracle.naive_attend(q, k, v, B3, s, scale_of(d))
    assert np.abs(naive - want).max() < 1e-5
    for backend in (0, 1):
        tiled, _ = oracle.tiled_attend_batched(q[None], k[None], v[None], B3, [s], scale_of(d),
                                               threads=2, backend=backend)
        assert np.abs(tiled[0] - want).max() < 1e-5


@pytest.mark.parametrize("mistake", ["swap_qk_for_v", "no_scale", "window_not_block", "shift_keys"])
def test_planted_mistakes_fail_the_golden(mistake):
    """Plausible slips in an attention restatement all miss the golden by far more than 1e-5."""
    _, t = golden()
    q, k, v = t["q"][0], t["k"][0], t["v"][0]
    s, d = q.shape[1], q.shape[2]
    if mistake == "swap_qk_for_v":
        got = oracle.naive_attend(q, v, k, B3, s, scale_of(d))
    elif mistake == "no_scale":
        got = oracle.naive_attend(q, k, v, B3, s, 1.0)
    elif mistake == "window_not_block":
        got = oracle.naive_attend(q, k, v, W64, s, scale_of(d))
    else:
        got = oracle.naive_attend(q, np.roll(k, 1, axis=1), v, B3, s, scale_of(d))
    assert np.abs(got - t["reference"][0]).max() > 1e-3


def test_key_range_matches_the_reference_examples():
    """masks_dense.rs:93-98 and attention.rs:48-59 at block edges."""
    assert oracle.key_range(SL, 2, 40, window=8) == (0, 11)
    assert oracle.key_range(FULL, 5, 7) == (0, 7)
    assert oracle.allows(SL, 20, 12, window=8) and oracle.allows(SL, 20, 28, window=8)
    assert not oracle.allows(SL, 20, 11, window=8) and not oracle.allows(SL, 20, 29, window=8)
    assert oracle.key_range(B3, 0, 1000) == (0, 256)
    assert oracle.key_range(B3, 128, 1000) == (0, 384)
    assert oracle.key_range(B3, 300, 1000) == (128, 512)
    assert oracle.key_range(B3, 300, 400) == (128, 400)
    assert oracle.key_range(W64, 10, 1000) == (0, 75)
    assert oracle.key_range(W64, 100, 120) == (36, 120)
    assert oracle.key_range(BD, 70, 1000, block=64) == (64, 128)
    assert oracle.key_range(BD, 70, 100, block=64) == (64, 100)


@pytest.mark.parametrize("kind,block,window", [(B3, 128, 0), (W64, 128, 0), (FULL, 128, 0),
                                               (SL, 128, 5), (SL, 128, 0), (BD, 64, 0),
                                               (BD, 128, 0), (BD, 7, 0)])
def test_key_range_is_exactly_the_allowed_interval(kind, block, window):
    """key_range and allows are two statements of one mask: they must agree on every (i, j)."""
    seq = 300
    for valid in (300, 263, 129, 1, 0):
        m = allowed_matrix(kind, seq, valid, block, window)
        for i in range(seq):
            lo, hi = oracle.key_range(kind, i, valid, block=block, window=window)
            row = np.zeros(seq, bool)
            row[lo:hi] = True
            if i < valid:
                assert (row == m[i]).all(), (i, valid)


@pytest.mark.parametrize("kind", [B3, W64])
def test_naive_matches_the_dense_reference(kind):
    """oracle.rs:7-32: seq {1,7,127,128,129,257}, (H,D) in {(1,8),(3,64)}, valid variants, 1e-6."""
    for seq in (1, 7, 127, 128, 129, 257):
        for heads, d in ((1, 8), (3, 64)):
            for valid in (seq, max(seq - 37, 0), seq // 2):
                q, k, v = oracle.qkv(heads, seq, d, 11 + seq)
                got = oracle.naive_attend(q, k, v, kind, valid, scale_of(d))
                want = oracle.dense_attend(q, k, v, kind, valid, scale_of(d))
                assert np.abs(got - want).max() < 1e-6, (seq, heads, d, valid)


@pytest.mark.parametrize("kind,block,window", [(B3, 128, 0), (W64, 128, 0), (FULL, 128, 0),
                                               (SL, 128, 8), (SL, 128, 0), (SL, 128, 500),
                                               (BD, 64, 0), (BD, 128, 0), (BD, 48, 0)])
def test_naive_matches_torch_sdpa_in_float64(kind, block, window):
    for seq, valid, heads, d in ((300, 300, 2, 64), (300, 217, 2, 16), (40, 23, 2, 16), (3, 1, 1, 8)):
        q, k, v = oracle.qkv(heads, seq, d, 1000 + seq)
        got = oracle.naive_attend(q, k, v, kind, valid, scale_of(d), block=block, window=window)
        want = sdpa_reference(q, k, v, kind, valid, block, window)
        assert np.abs(got - want).max() < 2e-6, (seq, valid, d)


def test_full_and_sliding_match_the_dense_softmax():
    """masks_dense.rs:64-76 with its LCG inputs."""
    for kind, w in ((FULL, 0), (SL, 8), (SL, 0), (SL, 500)):
        for seq, valid in ((40, 40), (40, 23), (3, 1)):
            n = 2 * seq * 16
            q = oracle.lcg_fill(n, 1).reshape(2, seq, 16)
            k = oracle.lcg_fill(n, 2).reshape(2, seq, 16)
            v = oracle.lcg_fill(n, 3).reshape(2, seq, 16)
            got = oracle.naive_attend(q, k, v, kind, valid, 0.25, window=w)
            want = oracle.dense_attend(q, k, v, kind, valid, 0.25, window=w)
            assert np.abs(got - want).max() < 1e-5


@pytest.mark.parametrize("kind,block", [(B3, 128), (W64, 128), (BD, 64)])
def test_masks_are_exact(kind, block):
    """masking.rs:20-61: with V one-hot on key j, out[i][0] > 0 exactly when (i, j) is allowed."""
    seq, d = 300, 8
    q = oracle.rand_vec(seq * d, 5).reshape(1, seq, d)
    k = oracle.rand_vec(seq * d, 6).reshape(1, seq, d)
    for j in (0, 1, 63, 64, 65, 127, 128, 129, 191, 255, 256, 299):
        v = np.zeros((1, seq, d), np.float32)
        v[0, j, 0] = 1.0
        out = oracle.naive_attend(q, k, v, kind, seq, scale_of(d), block=block)
        for i in range(seq):
            assert (out[0, i, 0] > 0) == oracle.allows(kind, i, j, block=block), (i, j)


def test_padding_and_empty_rows_are_exact_zeros():
    """masking.rs:63-91."""
    q, k, v = oracle.qkv(2, 200, 16, 9)
    for kind in (B3, W64, BD):
        for valid in (0, 1, 150):
            out = oracle.naive_attend(q, k, v, kind, valid, scale_of(16), block=64)
            assert (out[:, valid:, :] == 0).all()
            assert np.isfinite(out).all()
            tiled, _ = oracle.tiled_attend_batched(q[None], k[None], v[None], kind, [valid],
                                                   scale_of(16), block=64, threads=2)
            assert (tiled[0, :, valid:, :] == 0).all()


def test_single_valid_row_is_its_value_row():
    """masks_edges.rs:90-107: softmax over one key is 1."""
    q = oracle.lcg_fill(40, 31).reshape(1, 5, 8)
    k = oracle.lcg_fill(40, 32).reshape(1, 5, 8)
    v = oracle.lcg_fill(40, 33).reshape(1, 5, 8)
    for kind, w in ((FULL, 0), (SL, 2)):
        out = oracle.naive_attend(q, k, v, kind, 1, scale_of(8), window=w)
        assert np.abs(out[0, 0] - v[0, 0]).max() < 1e-6
        assert (out[0, 1:] == 0).all()


def test_extreme_logits_are_stable():
    """masking.rs:93-125: q, k scaled by 400 (scores ~1e4): finite, tiled == naive at 1e-5."""
    q, k, v = oracle.qkv(2, 300, 64, 21)
    q, k = q * 400.0, k * 400.0
    for kind in (B3, W64):
        want = oracle.naive_attend(q, k, v, kind, 300, scale_of(64))
        assert np.isfinite(want).all()
        got, _ = oracle.tiled_attend_batched(q[None], k[None], v[None], kind, [300], scale_of(64),
                                             threads=2)
        assert np.abs(got[0] - want).max() < 1e-5


@pytest.mark.parametrize("kind", [B3, W64])
def test_tiled_matches_naive_at_edge_lengths_and_padding(kind):
    """equivalence.rs:29-75."""
    cases = [(s, s, 3 if s < 1000 else 2) for s in (1, 127, 128, 129, 1000, 2048)]
    cases += [(300, 263, 2), (1000, 963, 2), (256, 1, 2), (256, 0, 2), (129, 128, 2)]
    for seq, valid, heads in cases:
        q, k, v = oracle.qkv(heads, seq, 64, 100 + seq)
        want = oracle.naive_attend(q, k, v, kind, valid, scale_of(64))
        for backend in (0, 1):
            got, _ = oracle.tiled_attend_batched(q[None], k[None], v[None], kind, [valid],
                                                 scale_of(64), threads=1, backend=backend)
            assert np.abs(got[0] - want).max() < 1e-5, (seq, valid, backend)


def test_tiled_is_bit_identical_across_thread_counts():
    """equivalence.rs:114-129."""
    q, k, v = oracle.qkv(4, 700, 64, 800)
    for kind in (B3, W64, BD):
        one, _ = oracle.tiled_attend_batched(q[None], k[None], v[None], kind, [650], scale_of(64),
                                             block=64, threads=1)
        four, _ = oracle.tiled_attend_batched(q[None], k[None], v[None], kind, [650], scale_of(64),
                                              block=64, threads=4)
        assert np.array_equal(one, four)


def test_tiled_other_head_dims():
    """equivalence.rs:77-112: D in {8, 40, 96}."""
    for d in (8, 40, 96):
        q, k, v = oracle.qkv(2, 300, d, 100 + 300)
        for kind in (B3, W64):
            want = oracle.naive_attend(q, k, v, kind, 300, scale_of(d))
            got, _ = oracle.tiled_attend_batched(q[None], k[None], v[None], kind, [300],
                                                 scale_of(d), threads=1)
            assert np.abs(got[0] - want).max() < 1e-5


def test_generators_reproduce_their_recurrences():
    """rand_vec (tests/common/mod.rs:6-18) and fill (masks_dense.rs:5-13) recomputed with ints."""
    mask = (1 << 64) - 1
    s = ((42 * 0x9E3779B97F4A7C15) & mask) | 1
    want = []
    for _ in range(8):
        s ^= (s << 13) & mask
        s ^= s >> 7
        s ^= (s << 17) & mask
        want.append(2.0 * np.float32((s >> 40) / float(1 << 24)) - 1.0)
    assert np.array_equal(oracle.rand_vec(8, 42), np.array(want, np.float32))
    s, want = 7, []
    for _ in range(8):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        want.append(np.float32((s >> 8) / float(1 << 24)) - np.float32(0.5))
    assert np.array_equal(oracle.lcg_fill(8, 7), np.array(want, np.float32))
    assert math.isclose(scale_of(64), 0.125)
