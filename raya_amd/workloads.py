"""The measured workloads: attention batches, the 12-layer encoder batch and the
single block-local layer, with their seeded inputs and algorithmic work.

Every workload is named by what it is.  The attention lines are one kernel
launch over a whole batch; the encoder lines are the decision-model forward of
crates/raya-core/src/model.rs:261-348 on a synthetic ModernBERT-base checkpoint.
Inputs come from ``raya_amd.synth`` (SplitMix64 + Box-Muller, seed
1000 * c + stream for workload family c; the reference bench's own shapes use its
xorshift U[-1, 1] with seeds 42/43/44, crates/raya-kernels/benches/local_attention.rs:90-97).
"""
from __future__ import annotations

import numpy as np

from . import synth

REF_BLOCK, REF_WINDOW = 128, 64  # attention.rs:4, :6


def _attn(family, batch, heads, seq, mask, valid, outliers=False, data="normal"):
    return {"family": family, "batch": batch, "heads": heads, "seq": seq, "head_dim": 64,
            "mask": mask, "valid": valid, "outliers": outliers, "data": data}


ATTENTION = {
    # BlockDiag(b): each query sees its own b-token block
    "attn_b32_h12_l2048_d64_blockdiag64": _attn(2, 32, 12, 2048, ("block_diag", 64), (512, 2048)),
    "attn_b1_h12_l512_d64_blockdiag64": _attn(1, 1, 12, 512, ("block_diag", 64), (512, 512)),
    "attn_b4_h12_l16384_d64_blockdiag128": _attn(5, 4, 12, 16384, ("block_diag", 128), (8192, 16384),
                                                 outliers=True),
    # the reference's own masks at the same shapes: Block3 = own 128-block and both neighbours
    "attn_b32_h12_l2048_d64_block3": _attn(2, 32, 12, 2048, ("block3",), (512, 2048)),
    "attn_b1_h12_l512_d64_block3": _attn(1, 1, 12, 512, ("block3",), (512, 512)),
    "attn_b4_h12_l16384_d64_block3": _attn(5, 4, 12, 16384, ("block3",), (8192, 16384), outliers=True),
    # the reference bench's shapes and inputs (16 heads, one sequence, no padding, xorshift
    # U[-1, 1] from seeds 42/43/44; benches/local_attention.rs:21-22, 90-97)
    **{f"refbench_h16_l{n}_d64_{m}": _attn(0, 1, 16, n, (m,), (n, n), data="xorshift")
       for n in (2048, 4096, 8192) for m in ("block3", "window64")},
}
DEFAULT_ATTENTION = "attn_b32_h12_l2048_d64_blockdiag64"

ENCODER = {
    # 12-layer ModernBERT-base decision model, batch of 64 sequences of up to 512 tokens
    "workload": "encoder_b64_l512_12x768_geglu",
    "family": 4, "batch": 64, "seq": 512, "valid": (128, 512), "cls_id": 101,
    "ids": (1000, 30522), "markers": [1, 2], "qtype": 0,
}
ENCODER_WEIGHT_SEED = 1000 * ENCODER["family"] + 5

LAYER = {
    # one local (block-local) layer of the same model on 16 sequences of 1024 valid tokens
    "workload": "encoder_layer_b16_l1024_768_geglu_blockdiag64",
    "family": 3, "batch": 16, "seq": 1024, "valid": (1024, 1024), "cls_id": 101,
    "ids": (1000, 30522), "markers": [1, 2], "qtype": 0, "block": 64,
}


def mask_name(mask) -> str:
    return f"block_diag({mask[1]})" if mask[0] == "block_diag" else mask[0]


def key_pairs(mask, v: int) -> int:
    """Sum over rows i < v of |key_range(i, v)| (attention.rs:48-59, plus BlockDiag(b))."""
    if mask[0] == "block_diag":
        b = mask[1]
        return b * b * (v // b) + (v % b) ** 2
    i = np.arange(v, dtype=np.int64)
    if mask[0] == "block3":
        blk = i // REF_BLOCK
        lo, hi = np.maximum(blk - 1, 0) * REF_BLOCK, (blk + 2) * REF_BLOCK
    elif mask[0] == "window64":
        lo, hi = np.maximum(i - REF_WINDOW, 0), i + REF_WINDOW + 1
    else:
        raise ValueError(mask)
    return int((np.minimum(hi, v) - np.minimum(lo, v)).sum())


def algorithmic(valid, heads, head_dim, seq, mask):
    """FLOP = 4 D H sum_b sum_{i<v_b} |keys(i)|; bytes = Q, K, V valid rows read once + all
    output rows written (fp32)."""
    keys = sum(key_pairs(mask, int(v)) for v in valid)
    flops = 4 * head_dim * heads * keys
    nbytes = 4 * (3 * heads * head_dim * int(sum(int(v) for v in valid))
                  + len(valid) * heads * seq * head_dim)
    return flops, nbytes


def attention_inputs(wl):
    """(q, k, v) as [B, H, L, D] float32 and the int32 valid lengths of workload `wl`."""
    c, b, h, s, d = wl["family"], wl["batch"], wl["heads"], wl["seq"], wl["head_dim"]
    lo, hi = wl["valid"]
    n = b * h * s * d
    qkv = []
    for i in range(3):
        if wl["data"] == "xorshift":
            x = synth.xorshift_uniform(42 + i, n).reshape(b, h, s, d)
        else:
            x = synth.normal(synth.workload_seed(c, i), n).reshape(b, h, s, d)
        if wl["outliers"]:
            synth.with_outliers(x, synth.workload_seed(c, 4) + 10 * i)
        qkv.append(x)
    if lo == hi:
        valid = np.full(b, lo, np.int32)
    else:
        valid = synth.integers(synth.workload_seed(c, 3), b, lo, hi).astype(np.int32)
    return qkv, valid


def encoder_inputs(spec):
    """(ids [B, L] uint32, valid [B], marker_pos [B, K], marker_mask [B, K], qtype [B]) of an
    encoder workload: token ids uniform in [1000, 30522) with the CLS id first, markers at
    positions 1 and 2, question type 0."""
    c, b, s = spec["family"], spec["batch"], spec["seq"]
    lo, hi = spec["valid"]
    valid = synth.integers(synth.workload_seed(c, 3), b, lo, hi).astype(np.uint64)
    a, z = spec["ids"]
    ids = synth.integers(synth.workload_seed(c, 6), b * s, a, z - 1).astype(np.uint32).reshape(b, s)
    ids[:, 0] = spec["cls_id"]
    k = len(spec["markers"])
    pos = np.tile(np.array(spec["markers"], np.uint64), (b, 1))
    mask = np.ones((b, k), np.uint8)
    qtype = np.full(b, spec["qtype"], np.uint64)
    return ids, valid, pos, mask, qtype


POSTLN_LAYER = {
    # one post-LN encoder layer as BERT writes it: hidden 768 = 12 x 64, GELU feed-forward 3072,
    # LayerNorm eps 1e-12, weights N(0, 0.02), zero biases, LayerNorm gain 1 and shift 0,
    # inputs N(0, 1), 16 sequences of 1024 valid tokens, BlockDiag(64) attention
    "workload": "postln_layer_b16_l1024_768_gelu3072_blockdiag64",
    "family": 3, "batch": 16, "seq": 1024, "hidden": 768, "heads": 12, "ffn": 3072, "eps": 1e-12,
    "block": 64, "std": 0.02,
}


def postln_flops(spec, valid) -> tuple[int, int]:
    """(GEMM FLOP, attention FLOP) of one post-LN layer over the valid tokens: 2 d (3d + d + 2F)
    per token, and 4 D H per allowed (query, key) pair under BlockDiag(block)."""
    d, f, h = spec["hidden"], spec["ffn"], spec["heads"]
    tokens = int(sum(int(v) for v in valid))
    gemm = tokens * 2 * d * (3 * d + d + 2 * f)
    attn = 4 * (d // h) * h * sum(key_pairs(("block_diag", spec["block"]), int(v)) for v in valid)
    return gemm, attn


def postln_inputs(spec):
    """(x [B, L, d] float32, valid [B] int32, weights) of a post-LN layer workload: x N(0, 1)
    (stream 0 of the family), the four weight matrices N(0, std) (streams 5, 7, 8, 9), zero
    biases, LayerNorm gains 1 and shifts 0."""
    c, b, s, d, f = spec["family"], spec["batch"], spec["seq"], spec["hidden"], spec["ffn"]
    x = synth.normal(synth.workload_seed(c, 0), b * s * d).reshape(b, s, d)
    valid = np.full(b, s, np.int32)
    std = np.float32(spec["std"])
    w = {}
    for name, shape, stream in (("wqkv", (3 * d, d), 5), ("wo", (d, d), 7), ("w1", (f, d), 8), ("w2", (d, f), 9)):
        w[name] = (synth.normal(synth.workload_seed(c, stream), shape[0] * shape[1]) * std).reshape(shape)
    w.update({"bqkv": np.zeros(3 * d, np.float32), "bo": np.zeros(d, np.float32), "b1": np.zeros(f, np.float32),
              "b2": np.zeros(d, np.float32), "ln1_w": np.ones(d, np.float32), "ln1_b": np.zeros(d, np.float32),
              "ln2_w": np.ones(d, np.float32), "ln2_b": np.zeros(d, np.float32)})
    return x, valid, w
