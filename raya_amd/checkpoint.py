"""Synthetic checkpoints in the layout raya-core and raya-weights read.

A checkpoint directory holds ``encoder/config.json`` (a ModernBertConfig),
``rl_agent_config.json`` and ``model.safetensors`` (crates/raya-weights/src/store.rs:234-239).
``write_synthetic`` fills every parameter the config implies — names and shapes from
the library's ``raya_expected_params`` (mapping.rs:19-143) — with seeded
N(0, std) weights (numpy's PCG64 generator: 137M values in about a second), LayerNorm
weights of one and zero biases, as used for the throughput runs.
"""
from __future__ import annotations

import ctypes
import json
import os

import numpy as np

from . import _capi as C
from .model import _check

# ModernBERT-base: 12 layers of 768 = 12 x 64, GeGLU 3072, global layer every 3rd with the
# full-attention RoPE base, local layers a 128-token window.
MODERNBERT_BASE = {
    "hidden_size": 768, "intermediate_size": 3072, "num_hidden_layers": 12,
    "num_attention_heads": 12, "global_attn_every_n_layers": 3, "local_attention": 128,
    "max_position_embeddings": 4096, "vocab_size": 30522, "norm_eps": 1e-12,
    "norm_bias": False, "attention_bias": False, "mlp_bias": False,
    "hidden_activation": "gelu", "pad_token_id": 0, "cls_token_id": 101,
    "rope_parameters": {"full_attention": {"rope_theta": 160000.0},
                        "sliding_attention": {"rope_theta": 10000.0}},
}


def expected_params(checkpoint_dir: str) -> list[tuple[str, tuple[int, ...]]]:
    """(name, shape) of every parameter the config in checkpoint_dir implies, in order."""
    n = ctypes.c_uint64()
    _check(C.lib().raya_expected_params(checkpoint_dir.encode(), None, 0, ctypes.byref(n)))
    buf = (C.ParamEntryC * n.value)()
    _check(C.lib().raya_expected_params(checkpoint_dir.encode(), buf, n.value, ctypes.byref(n)))
    return [(e.name.decode(), tuple(e.shape[i] for i in range(e.ndim))) for e in buf]


def write_config(checkpoint_dir: str, encoder: dict, agent: dict) -> None:
    os.makedirs(os.path.join(checkpoint_dir, "encoder"), exist_ok=True)
    with open(os.path.join(checkpoint_dir, "encoder", "config.json"), "w") as f:
        json.dump(encoder, f, indent=1)
    with open(os.path.join(checkpoint_dir, "rl_agent_config.json"), "w") as f:
        json.dump(agent, f, indent=1)


def write_synthetic(checkpoint_dir: str, encoder: dict | None = None, agent: dict | None = None,
                    seed: int = 0, std: float = 0.02) -> str:
    """Writes a full checkpoint; returns the weights path."""
    from safetensors.numpy import save_file

    encoder = dict(MODERNBERT_BASE if encoder is None else encoder)
    agent = {"head_layers": 0, "act_costs": {"abstain": 0.1}} if agent is None else agent
    write_config(checkpoint_dir, encoder, agent)
    tensors = {}
    rng = np.random.default_rng(seed)
    for name, shape in expected_params(checkpoint_dir):
        n = int(np.prod(shape))
        if name.endswith("norm.weight") or name.endswith(("norm1.weight", "norm2.weight")) \
                or name == "scorer.0.weight" or name == "temperature":
            x = np.ones(n, np.float32)
        elif name.endswith("bias"):
            x = np.zeros(n, np.float32)
        else:
            x = rng.standard_normal(n, dtype=np.float32)
            x *= np.float32(std)
        tensors[name] = x.reshape(shape)
    path = os.path.join(checkpoint_dir, "model.safetensors")
    save_file(tensors, path)
    return path
