"""The oracle's post-LN layer (oracle.forward.postln_layer) against torch's
nn.TransformerEncoderLayer(norm_first=False, activation="gelu", dropout=0) in float64: the same
composition (LayerNorm after each residual add, biases, erf GELU, q/k/v stacked in one
projection with heads as contiguous column slices, scale 1/sqrt(head_dim)), evaluated
independently.  A planted mistake (pre-LN order, no 1/sqrt(head_dim), swapped k and v) misses
by far more than the bar."""
import numpy as np
import pytest
import torch

import oracle
from oracle import forward as F


def make(d, heads, ffn, seed, biases=True):
    rng = np.random.default_rng(seed)
    w = {"wqkv": 0.1 * rng.standard_normal((3 * d, d)), "wo": 0.1 * rng.standard_normal((d, d)),
         "w1": 0.1 * rng.standard_normal((ffn, d)), "w2": 0.1 * rng.standard_normal((d, ffn)),
         "ln1_w": 1 + 0.1 * rng.standard_normal(d), "ln2_w": 1 + 0.1 * rng.standard_normal(d)}
    if biases:
        w.update({"bqkv": 0.1 * rng.standard_normal(3 * d), "bo": 0.1 * rng.standard_normal(d),
                  "b1": 0.1 * rng.standard_normal(ffn), "b2": 0.1 * rng.standard_normal(d),
                  "ln1_b": 0.1 * rng.standard_normal(d), "ln2_b": 0.1 * rng.standard_normal(d)})
    return {k: v.astype(np.float32) for k, v in w.items()}


def torch_layer(x, valid, w, heads, eps, allowed):
    """nn.TransformerEncoderLayer in float64 on one sequence; `allowed[i, j]` is the mask."""
    d = x.shape[1]
    ffn = w["w1"].shape[0]
    layer = torch.nn.TransformerEncoderLayer(d, heads, dim_feedforward=ffn, dropout=0.0, activation="gelu",
                                             layer_norm_eps=eps, batch_first=True, norm_first=False,
                                             dtype=torch.float64)
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731
    zero = lambda n: torch.zeros(n, dtype=torch.float64)  # noqa: E731
    with torch.no_grad():
        layer.self_attn.in_proj_weight.copy_(t(w["wqkv"]))
        layer.self_attn.in_proj_bias.copy_(t(w["bqkv"]) if "bqkv" in w else zero(3 * d))
        layer.self_attn.out_proj.weight.copy_(t(w["wo"]))
        layer.self_attn.out_proj.bias.copy_(t(w["bo"]) if "bo" in w else zero(d))
        layer.linear1.weight.copy_(t(w["w1"]))
        layer.linear1.bias.copy_(t(w["b1"]) if "b1" in w else zero(ffn))
        layer.linear2.weight.copy_(t(w["w2"]))
        layer.linear2.bias.copy_(t(w["b2"]) if "b2" in w else zero(d))
        layer.norm1.weight.copy_(t(w["ln1_w"]))
        layer.norm1.bias.copy_(t(w["ln1_b"]) if "ln1_b" in w else zero(d))
        layer.norm2.weight.copy_(t(w["ln2_w"]))
        layer.norm2.bias.copy_(t(w["ln2_b"]) if "ln2_b" in w else zero(d))
        layer.train()  # dropout is 0; train mode keeps the plain (non-fused) path
        seq = x.shape[0]
        keep = torch.from_numpy(allowed.copy())
        keep[:, valid:] = False
        mask = torch.zeros(seq, seq, dtype=torch.float64).masked_fill(~keep, float("-inf"))
        out = layer(t(x)[None], src_mask=mask)[0]
    return out.numpy()


def allowed_matrix(kind, seq, arg):
    i = np.arange(seq)[:, None]
    j = np.arange(seq)[None, :]
    if kind == oracle.MASK_BLOCKDIAG:
        return i // arg == j // arg
    if kind == oracle.MASK_BLOCK3:
        return np.abs(i // 128 - j // 128) <= 1
    if kind == oracle.MASK_WINDOW64:
        return np.abs(i - j) <= 64
    return np.abs(i - j) <= arg  # Sliding(arg)


CASES = [
    # (d, heads, ffn, seq, valid, kind, arg, eps, biases)
    (64, 2, 128, 150, 150, oracle.MASK_BLOCKDIAG, 16, 1e-12, False),
    (64, 4, 96, 260, 200, oracle.MASK_BLOCK3, 0, 1e-5, True),
    (96, 3, 192, 170, 131, oracle.MASK_WINDOW64, 0, 1e-6, True),
    (64, 2, 64, 90, 77, oracle.MASK_SLIDING, 5, 1e-5, True),
]


@pytest.mark.parametrize("d,heads,ffn,seq,valid,kind,arg,eps,biases", CASES)
def test_postln_layer_matches_torch(d, heads, ffn, seq, valid, kind, arg, eps, biases):
    w = make(d, heads, ffn, seed=d + seq, biases=biases)
    x = np.random.default_rng(seq).standard_normal((seq, d)).astype(np.float32)
    got = F.postln_layer(x, valid, w, heads, eps, kind, arg)
    want = torch_layer(x, valid, w, heads, eps, allowed_matrix(kind, seq, arg))
    err = np.abs(got[:valid] - want[:valid]).max()
    assert err < 2e-5, err


def test_planted_mistakes_miss():
    d, heads, ffn, seq, valid = 64, 2, 128, 130, 130
    w = make(d, heads, ffn, seed=3)
    x = np.random.default_rng(4).standard_normal((seq, d)).astype(np.float32)
    want = torch_layer(x, valid, w, heads, 1e-5, allowed_matrix(oracle.MASK_BLOCK3, seq, 0))
    good = F.postln_layer(x, valid, w, heads, 1e-5, oracle.MASK_BLOCK3, 0)
    assert np.abs(good - want).max() < 2e-5
    swapped = dict(w)
    swapped["wqkv"] = np.concatenate([w["wqkv"][:d], w["wqkv"][2 * d:], w["wqkv"][d:2 * d]])
    swapped["bqkv"] = np.concatenate([w["bqkv"][:d], w["bqkv"][2 * d:], w["bqkv"][d:2 * d]])
    assert np.abs(F.postln_layer(x, valid, swapped, heads, 1e-5, oracle.MASK_BLOCK3, 0) - want).max() > 1e-2
    unscaled = dict(w)  # q scaled up by sqrt(head_dim): the 1/sqrt(head_dim) dropped
    unscaled["wqkv"] = w["wqkv"].copy()
    unscaled["bqkv"] = w["bqkv"].copy()
    unscaled["wqkv"][:d] *= np.float32(np.sqrt(d // heads))
    unscaled["bqkv"][:d] *= np.float32(np.sqrt(d // heads))
    assert np.abs(F.postln_layer(x, valid, unscaled, heads, 1e-5, oracle.MASK_BLOCK3, 0) - want).max() > 1e-2
    pre = oracle.layer_norm(x, w["ln1_w"], w["ln1_b"], np.float32(1e-5))  # pre-LN order
    pre_ln = x + F.linear(F.attend(F.linear(pre, w["wqkv"], w["bqkv"]), heads, d // heads, None,
                                   oracle.MASK_BLOCK3, 0, valid), w["wo"], w["bo"])
    assert np.abs(pre_ln - want).max() > 1e-2
