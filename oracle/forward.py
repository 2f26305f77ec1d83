"""CPU restatement of raya-core's reference forward pass (TEST INFRASTRUCTURE ONLY).

The decision model of crates/raya-core: ModernBERT encoder (embed, pre-LN layers
with RoPE and GeGLU, final norm), type embedding, nn.TransformerEncoderLayer head
layers, marker scorer, score features and act head.  Numerics follow the reference:
fp32 storage, sequential-f32 GEMMs (oracle.matmul_nt), LayerNorm statistics and
GELU in f64 (oracle.layer_norm / oracle.gelu_array), Naive attention
(oracle.naive_attend), RoPE with f32 angles (oracle.rope).

Pinned by the four forward goldens of tests/data (short, medium, padded,
fastpath_off; crates/raya-cli/tests/forward_golden.rs) at 1e-5 per stage and 1e-6
for probabilities and features, and by the padding-invariance property of
forward_golden.rs:238-262.  Only the test suite uses this module.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field

import numpy as np

import oracle

HEAD_EPS = np.float32(1e-5)  # head.rs:8, torch's default layer_norm_eps
GEMM_THREADS = 4  # host threads of the sequential-f32 GEMM (results do not depend on it)


# --- configuration (crates/raya-core/src/config/{encoder,agent,mod}.rs) -----------------------

@dataclass
class Config:
    hidden: int
    inter: int
    layers: int
    heads: int
    global_every: int
    local_attention: int
    global_theta: float
    local_theta: float
    norm_eps: float
    vocab: int
    head_layers: int
    n_act: int

    @property
    def head_heads(self) -> int:  # config/mod.rs:63-78
        return max(1, self.hidden // 64)

    def is_global(self, layer: int) -> bool:  # config/encoder.rs:39-41
        return layer % self.global_every == 0


def rope_thetas(enc: dict) -> tuple[float, float]:
    """config/encoder.rs:201-218: per-layer-type rope_parameters, else the flat 4.x keys,
    else rope_parameters.rope_theta."""
    rp = enc.get("rope_parameters") or {}
    flat = rp.get("rope_theta")

    def pick(typed, legacy):
        if typed and typed.get("rope_theta") is not None:
            return typed["rope_theta"]
        return legacy if legacy is not None else flat

    return (pick(rp.get("full_attention"), enc.get("global_rope_theta")),
            pick(rp.get("sliding_attention"), enc.get("local_rope_theta")))


def load_config(checkpoint_dir: str) -> Config:
    enc = json.load(open(os.path.join(checkpoint_dir, "encoder", "config.json")))
    agent = json.load(open(os.path.join(checkpoint_dir, "rl_agent_config.json")))
    g, l = rope_thetas(enc)
    return Config(hidden=enc["hidden_size"], inter=enc["intermediate_size"],
                  layers=enc["num_hidden_layers"], heads=enc["num_attention_heads"],
                  global_every=enc["global_attn_every_n_layers"],
                  local_attention=enc["local_attention"], global_theta=g, local_theta=l,
                  norm_eps=enc["norm_eps"], vocab=enc["vocab_size"],
                  head_layers=agent.get("head_layers", 2),
                  n_act=len(agent.get("act_costs", {})) + 1)


def load_weights(path: str) -> dict[str, np.ndarray]:
    from safetensors.numpy import load_file

    return {k: np.ascontiguousarray(v.astype(np.float32)) for k, v in load_file(path).items()}


# --- building blocks ------------------------------------------------------------------------

def linear(x, w, b=None):
    """ops::linear (ops.rs:91-109): sequential-f32 matmul_nt, then the bias in f32."""
    out = oracle.matmul_nt(x, w, threads=GEMM_THREADS)
    if b is not None:
        out += b
    return out


def split_qkv(qkv, heads, hd):
    """encoder::split_qkv (encoder.rs:36-53): [seq, 3, heads, hd] -> 3 x [heads, seq, hd]."""
    seq = qkv.shape[0]
    t = qkv.reshape(seq, 3, heads, hd).transpose(1, 2, 0, 3)
    return [np.ascontiguousarray(t[i]) for i in range(3)]


def attend(qkv, heads, hd, theta, kind, arg, valid_len):
    """encoder::attend (encoder.rs:57-92) with the Naive kernel."""
    q, k, v = split_qkv(qkv, heads, hd)
    if theta is not None:
        q = oracle.rope(q, np.float32(theta))
        k = oracle.rope(k, np.float32(theta))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    # the oracle takes a BlockDiag width as `block`, a Sliding half-width as `window`
    if kind == oracle.MASK_BLOCKDIAG:
        out = oracle.naive_attend(q, k, v, kind, valid_len, scale, block=arg)
    else:
        out = oracle.naive_attend(q, k, v, kind, valid_len, scale, window=arg)
    seq = qkv.shape[0]
    return np.ascontiguousarray(out.transpose(1, 0, 2).reshape(seq, heads * hd))


def postln_layer(x, valid_len: int, w: dict, heads: int, eps: float, kind: int, arg: int):
    """One post-LN encoder layer on one sequence (x: [seq, hidden] float32), the layer of
    raya_postln_layer_forward, restated with the reference's building blocks: sequential-f32
    linear with bias (ops.rs:91-109), Naive attention without RoPE (naive.rs:13-65), LayerNorm
    with f64 statistics (ops.rs:51-74) and erf GELU (ops.rs:7-38).  `w` holds wqkv [3d, d]
    (q, k, v stacked), wo [d, d], w1 [F, d], w2 [d, F], ln1_w/ln2_w [d] and optional biases
    bqkv, bo, b1, b2, ln1_b, ln2_b.  Rows at or beyond valid_len attend to nothing."""
    x = np.asarray(x, np.float32)
    d = x.shape[1]
    hd = d // heads
    eps = np.float32(eps)
    qkv = linear(x, w["wqkv"], w.get("bqkv"))
    ctx = attend(qkv, heads, hd, None, kind, arg, valid_len)
    y1 = oracle.layer_norm(x + linear(ctx, w["wo"], w.get("bo")), w["ln1_w"], w.get("ln1_b"), eps)
    f = oracle.gelu_array(linear(y1, w["w1"], w.get("b1")))
    return oracle.layer_norm(y1 + linear(f, w["w2"], w.get("b2")), w["ln2_w"], w.get("ln2_b"), eps)


def f32_sum(xs) -> np.float32:
    acc = np.float32(0.0)
    for x in xs:
        acc = np.float32(acc + np.float32(x))
    return acc


def softmax(x):
    return oracle.softmax(np.asarray(x, np.float32))


def features(p, valid_markers):
    """head::features (head.rs:70-92)."""
    k = np.float32(max(valid_markers, 2))
    ent = -f32_sum(np.float32(x) * np.log(np.maximum(np.float32(x), np.float32(1e-9)))
                   for x in p) / np.log(k)
    top1 = top2 = np.float32(-np.inf)
    for x in p:
        if x > top1:
            top2, top1 = top1, x
        elif x > top2:
            top2 = x
    if len(p) < 2:
        top2 = np.float32(0.0)
    return np.array([top1, top1 - top2, ent, k / np.float32(255.0)], np.float32)


# --- the forward pass -----------------------------------------------------------------------

@dataclass
class Output:
    logits: np.ndarray
    probabilities: np.ndarray
    act_logits: np.ndarray
    features: np.ndarray
    pooled: np.ndarray
    trace: dict = field(default_factory=dict)


def forward(cfg: Config, w: dict, ids, valid_len: int, marker_pos, marker_mask, qtype: int,
            local_mask=(oracle.MASK_SLIDING, None)) -> Output:
    """Network::forward (model.rs:261-348) on one sequence, recording the stages under the
    golden names.  `local_mask` overrides the local layers' mask (kind, arg); the default is
    the reference's Sliding(local_attention / 2)."""
    d, eps = cfg.hidden, np.float32(cfg.norm_eps)
    ids = np.asarray(ids, np.int64)
    seq = len(ids)
    tr = {}

    h = oracle.layer_norm(w["encoder.embeddings.tok_embeddings.weight"][ids],
                          w["encoder.embeddings.norm.weight"], None, eps)
    tr["embedding_output"] = h.copy()
    for i in range(cfg.layers):
        p = f"encoder.layers.{i}"
        normed = h.copy() if i == 0 else oracle.layer_norm(h, w[f"{p}.attn_norm.weight"], None, eps)
        qkv = linear(normed, w[f"{p}.attn.Wqkv.weight"])
        if cfg.is_global(i):
            theta, kind, arg = cfg.global_theta, oracle.MASK_FULL, 0
        else:
            theta = cfg.local_theta
            kind, arg = local_mask
            if arg is None:
                arg = cfg.local_attention // 2
        ctx = attend(qkv, cfg.heads, d // cfg.heads, theta, kind, arg, valid_len)
        h = h + linear(ctx, w[f"{p}.attn.Wo.weight"])
        normed = oracle.layer_norm(h, w[f"{p}.mlp_norm.weight"], None, eps)
        wi = linear(normed, w[f"{p}.mlp.Wi.weight"])
        gated = oracle.gelu_array(wi[:, :cfg.inter]) * wi[:, cfg.inter:]
        h = h + linear(gated, w[f"{p}.mlp.Wo.weight"])
        tr[f"encoder_layer_{i:02d}"] = h.copy()
    h = oracle.layer_norm(h, w["encoder.final_norm.weight"], None, eps)
    tr["encoder_final_norm"] = h.copy()
    tr["encoder_output"] = h.copy()
    add = w["type_emb.weight"][qtype]
    tr["type_emb_add"] = add.reshape(1, d).copy()
    h = h + add
    tr["head_input"] = h.copy()
    hh = cfg.head_heads
    for i in range(cfg.head_layers):
        p = f"head.layers.{i}"
        normed = oracle.layer_norm(h, w[f"{p}.norm1.weight"], w[f"{p}.norm1.bias"], HEAD_EPS)
        qkv = linear(normed, w[f"{p}.self_attn.in_proj_weight"], w[f"{p}.self_attn.in_proj_bias"])
        ctx = attend(qkv, hh, d // hh, None, oracle.MASK_FULL, 0, valid_len)
        h = h + linear(ctx, w[f"{p}.self_attn.out_proj.weight"], w[f"{p}.self_attn.out_proj.bias"])
        normed = oracle.layer_norm(h, w[f"{p}.norm2.weight"], w[f"{p}.norm2.bias"], HEAD_EPS)
        hidden = np.maximum(linear(normed, w[f"{p}.linear1.weight"], w[f"{p}.linear1.bias"]),
                            np.float32(0.0))
        h = h + linear(hidden, w[f"{p}.linear2.weight"], w[f"{p}.linear2.bias"])
        tr[f"head_layer_{i:02d}"] = h.copy()

    states = np.ascontiguousarray(h[np.asarray(marker_pos, np.int64)])
    tr["marker_states"] = states.copy()
    normed = oracle.layer_norm(states, w["scorer.0.weight"], w["scorer.0.bias"], HEAD_EPS)
    hidden = oracle.gelu_array(linear(normed, w["scorer.1.weight"], w["scorer.1.bias"]))
    logits = linear(hidden, w["scorer.3.weight"], w["scorer.3.bias"])[:, 0].copy()
    logits[~np.asarray(marker_mask, bool)] = np.float32(-1e4)
    tr["logits"] = logits.copy()
    probs = softmax(logits)
    tr["probabilities"] = probs.copy()
    feats = features(probs, int(np.count_nonzero(marker_mask)))
    tr["act_features"] = feats.copy()
    pooled = h[0].copy()
    tr["pooled"] = pooled.copy()
    act_in = np.concatenate([pooled, feats]).reshape(1, d + 4)
    hidden = oracle.gelu_array(linear(act_in, w["act_head.0.weight"], w["act_head.0.bias"]))
    act_logits = linear(hidden, w["act_head.2.weight"], w["act_head.2.bias"])[0]
    tr["act_logits"] = act_logits.copy()
    return Output(logits, probs, act_logits, feats, pooled, tr)


def expected_names(cfg: Config) -> list[tuple[str, tuple]]:
    """raya-weights' expected parameter set (crates/raya-weights/src/mapping.rs:42-143):
    (laya name, shape) in mapping order."""
    d, i = cfg.hidden, cfg.inter
    out = [("encoder.embeddings.tok_embeddings.weight", (cfg.vocab, d)),
           ("encoder.embeddings.norm.weight", (d,))]
    for n in range(cfg.layers):
        p = f"encoder.layers.{n}"
        if n > 0:
            out.append((f"{p}.attn_norm.weight", (d,)))
        out += [(f"{p}.attn.Wqkv.weight", (3 * d, d)), (f"{p}.attn.Wo.weight", (d, d)),
                (f"{p}.mlp_norm.weight", (d,)), (f"{p}.mlp.Wi.weight", (2 * i, d)),
                (f"{p}.mlp.Wo.weight", (d, i))]
    out.append(("encoder.final_norm.weight", (d,)))
    for n in range(cfg.head_layers):
        p = f"head.layers.{n}"
        out += [(f"{p}.self_attn.in_proj_weight", (3 * d, d)),
                (f"{p}.self_attn.in_proj_bias", (3 * d,)),
                (f"{p}.self_attn.out_proj.weight", (d, d)), (f"{p}.self_attn.out_proj.bias", (d,)),
                (f"{p}.linear1.weight", (4 * d, d)), (f"{p}.linear1.bias", (4 * d,)),
                (f"{p}.linear2.weight", (d, 4 * d)), (f"{p}.linear2.bias", (d,)),
                (f"{p}.norm1.weight", (d,)), (f"{p}.norm1.bias", (d,)),
                (f"{p}.norm2.weight", (d,)), (f"{p}.norm2.bias", (d,))]
    out += [("type_emb.weight", (3, d)), ("scorer.0.weight", (d,)), ("scorer.0.bias", (d,)),
            ("scorer.1.weight", (d, d)), ("scorer.1.bias", (d,)), ("scorer.3.weight", (1, d)),
            ("scorer.3.bias", (1,)), ("act_head.0.weight", (256, d + 4)),
            ("act_head.0.bias", (256,)), ("act_head.2.weight", (cfg.n_act, 256)),
            ("act_head.2.bias", (cfg.n_act,)), ("temperature", (3,))]
    return out
