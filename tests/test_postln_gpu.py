"""The post-LN encoder layer (raya_postln_layer_forward) against the oracle's restatement,
which tests/test_oracle_postln.py pins to torch's nn.TransformerEncoderLayer in float64.

* The configuration itself: 16 sequences of 1024 tokens, hidden 768 = 12 x 64, GELU 3072,
  eps 1e-12, N(0, 0.02) weights, zero biases, gain 1 and shift 0, N(0, 1) inputs,
  BlockDiag(64); sequences 0 and 15 through the oracle at max-abs 1e-4 and rel-L2 1e-5.
* Smaller layers with random biases, gains and shifts, padding and the other masks, head dims
  32 and 64, at max-abs 1e-5 on the valid rows."""
import numpy as np
import pytest
import torch

import oracle
from oracle import forward as F
from raya_amd import Mask
from raya_amd import workloads as W
from raya_amd.layers import PostLNLayer

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.sqrt(((got - want) ** 2).sum() / (want ** 2).sum()))


@pytest.mark.timeout(900)
def test_the_postln_workload_matches_the_oracle():
    spec = W.POSTLN_LAYER
    x, valid, w = W.postln_inputs(spec)
    print(f"post-LN layer: B={x.shape[0]} L={x.shape[1]} d={x.shape[2]}", flush=True)
    layer = PostLNLayer({k: dev(v) for k, v in w.items()}, spec["heads"], spec["eps"], Mask.block_diag(spec["block"]))
    out = layer.forward(dev(x), dev(valid)).cpu().numpy()
    assert np.isfinite(out).all()
    F.GEMM_THREADS = 16
    for i in (0, 15):
        want = F.postln_layer(x[i], int(valid[i]), w, spec["heads"], spec["eps"], oracle.MASK_BLOCKDIAG, spec["block"])
        err, rel = float(np.abs(out[i] - want).max()), rel_l2(out[i], want)
        print(f"  sequence {i}: max-abs {err:.2e} rel-L2 {rel:.2e}", flush=True)
        assert err <= 1e-4 and rel <= 1e-5, (i, err, rel)


SMALL = [
    # (d, heads, ffn, seq, valid lengths, mask, oracle kind, arg)
    (128, 4, 256, 300, [300, 173, 1], Mask.block_diag(64), oracle.MASK_BLOCKDIAG, 64),
    (128, 2, 192, 260, [260, 200], Mask.BLOCK3, oracle.MASK_BLOCK3, 0),
    (256, 4, 512, 190, [190, 64, 131], Mask.WINDOW64, oracle.MASK_WINDOW64, 0),
    (64, 2, 128, 77, [77, 50], Mask.sliding(7), oracle.MASK_SLIDING, 7),
]


@pytest.mark.parametrize("d,heads,ffn,seq,valids,mask,kind,arg", SMALL)
def test_small_layers_with_biases_match_the_oracle(d, heads, ffn, seq, valids, mask, kind, arg):
    rng = np.random.default_rng(d + seq)
    f32 = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    w = {"wqkv": 0.1 * f32(3 * d, d), "bqkv": 0.1 * f32(3 * d), "wo": 0.1 * f32(d, d), "bo": 0.1 * f32(d),
         "w1": 0.1 * f32(ffn, d), "b1": 0.1 * f32(ffn), "w2": 0.1 * f32(d, ffn), "b2": 0.1 * f32(d),
         "ln1_w": 1 + 0.1 * f32(d), "ln1_b": 0.1 * f32(d), "ln2_w": 1 + 0.1 * f32(d), "ln2_b": 0.1 * f32(d)}
    b = len(valids)
    x = f32(b, seq, d)
    valid = np.array(valids, np.int32)
    layer = PostLNLayer({k: dev(v) for k, v in w.items()}, heads, 1e-5, mask)
    out = layer.forward(dev(x), dev(valid)).cpu().numpy()
    for i in range(b):
        v = int(valid[i])
        want = F.postln_layer(x[i], v, w, heads, 1e-5, kind, arg)
        err = float(np.abs(out[i, :v] - want[:v]).max())
        assert err <= 1e-5, (i, err)
