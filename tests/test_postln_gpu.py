"""The post-LN encoder layer (raya_postln_layer_forward) against the oracle's restatement,
which tests/test_oracle_postln.py pins to torch's nn.TransformerEncoderLayer in float64.

* The configuration itself: 16 sequences of 1024 tokens, hidden 768 = 12 x 64, GELU 3072,
  eps 1e-12, N(0, 0.02) weights, zero biases, gain 1 and shift 0, N(0, 1) inputs,
  BlockDiag(64); sequences 0 and 15 through the oracle at max-abs 1e-4 and rel-L2 1e-5, and
  the whole batch against torch's float64 layer on the device at the same bars.
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


@pytest.mark.timeout(600)
def test_the_postln_workload_whole_batch_against_torch_float64():
    """Every token of all 16 sequences of the measured configuration against torch's own
    nn.TransformerEncoderLayer(norm_first=False, activation="gelu") evaluated in float64 on
    the device with the same weights and a BlockDiag(64) attention mask: max-abs 1e-4 and
    rel-L2 1e-5 over the whole batch."""
    spec = W.POSTLN_LAYER
    x, valid, w = W.postln_inputs(spec)
    b, s, d = x.shape
    layer = PostLNLayer({k: dev(v) for k, v in w.items()}, spec["heads"], spec["eps"], Mask.block_diag(spec["block"]))
    out = layer.forward(dev(x), dev(valid)).double()
    ref = torch.nn.TransformerEncoderLayer(d, spec["heads"], dim_feedforward=spec["ffn"], dropout=0.0,
                                           activation="gelu", layer_norm_eps=spec["eps"], batch_first=True,
                                           norm_first=False, dtype=torch.float64, device="cuda")
    t = lambda a: dev(np.asarray(a, np.float64))  # noqa: E731
    with torch.no_grad():
        ref.self_attn.in_proj_weight.copy_(t(w["wqkv"]))
        ref.self_attn.in_proj_bias.copy_(t(w["bqkv"]))
        ref.self_attn.out_proj.weight.copy_(t(w["wo"]))
        ref.self_attn.out_proj.bias.copy_(t(w["bo"]))
        ref.linear1.weight.copy_(t(w["w1"]))
        ref.linear1.bias.copy_(t(w["b1"]))
        ref.linear2.weight.copy_(t(w["w2"]))
        ref.linear2.bias.copy_(t(w["b2"]))
        ref.norm1.weight.copy_(t(w["ln1_w"]))
        ref.norm1.bias.copy_(t(w["ln1_b"]))
        ref.norm2.weight.copy_(t(w["ln2_w"]))
        ref.norm2.bias.copy_(t(w["ln2_b"]))
        ref.train()  # dropout is 0; train mode keeps the plain (non-fused) path
        i = torch.arange(s, device="cuda")
        blocks = (i[:, None] // spec["block"]) == (i[None, :] // spec["block"])
        mask = torch.zeros(s, s, dtype=torch.float64, device="cuda").masked_fill(~blocks, float("-inf"))
        assert bool((torch.from_numpy(valid) == s).all())  # the configuration has no padding
        want = torch.cat([ref(t(x[j:j + 4]), src_mask=mask) for j in range(0, b, 4)])
    diff = out - want
    err, rel = float(diff.abs().max()), float(diff.norm() / want.norm())
    print(f"whole batch: max-abs {err:.2e} rel-L2 {rel:.2e}", flush=True)
    assert err <= 1e-4 and rel <= 1e-5, (err, rel)
