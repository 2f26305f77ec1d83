"""The oracle's forward pass against the reference's four forward goldens.

Mirrors crates/raya-cli/tests/forward_golden.rs: every stage on the valid rows at
1e-5 (probabilities and features at 1e-6), padding invariance, and planted
mistakes that must miss the goldens.
"""
import json
import os

import numpy as np
import pytest

import oracle
from oracle import forward as F

FWD = os.path.join(os.path.dirname(__file__), "golden", "forward")
LAYER_TOL, PROB_TOL = 1e-5, 1e-6
CASES = ["short", "medium", "padded", "fastpath_off"]


def load_case(name):
    from safetensors.numpy import load_file

    meta = json.load(open(os.path.join(FWD, name, "meta.json")))
    cfg = F.load_config(os.path.normpath(os.path.join(FWD, name, meta["config_dir"])))
    w = F.load_weights(os.path.normpath(os.path.join(FWD, name, meta["weights_file"])))
    g = load_file(os.path.join(FWD, name, "tensors.safetensors"))
    return cfg, w, g, meta["input"]["unpadded_length"]


def stages(cfg):
    v = [("embedding_output", LAYER_TOL)]
    v += [(f"encoder_layer_{i:02d}", LAYER_TOL) for i in range(cfg.layers)]
    v += [(n, LAYER_TOL) for n in ("encoder_final_norm", "encoder_output", "type_emb_add",
                                   "head_input")]
    v += [(f"head_layer_{i:02d}", LAYER_TOL) for i in range(cfg.head_layers)]
    v += [("marker_states", LAYER_TOL), ("logits", LAYER_TOL), ("probabilities", PROB_TOL),
          ("act_features", PROB_TOL), ("pooled", LAYER_TOL), ("act_logits", LAYER_TOL)]
    return v


def run_case(cfg, w, g, valid, **kw):
    return F.forward(cfg, w, g["input_ids"][0], valid, g["marker_pos"][0], g["marker_mask"][0],
                     int(g["qtype"][0]), **kw)


def compare(cfg, g, valid, trace):
    """(name, max abs diff over valid rows, tolerance) per stage."""
    seq = g["input_ids"].shape[1]
    rows = []
    for name, tol in stages(cfg):
        want = g[name].astype(np.float32)
        got = trace[name].reshape(want.shape)
        if want.ndim == 3 and want.shape[1] == seq:
            want, got = want[:, :valid], got[:, :valid]
        rows.append((name, float(np.abs(got - want).max()), tol))
    return rows


@pytest.mark.parametrize("case", CASES)
def test_oracle_forward_matches_golden(case):
    cfg, w, g, valid = load_case(case)
    out = run_case(cfg, w, g, valid)
    rows = compare(cfg, g, valid, out.trace)
    bad = [r for r in rows if r[1] > r[2]]
    assert not bad, f"{case}: {bad}"


def test_padding_does_not_change_valid_rows():
    cfg, w, g, valid = load_case("padded")
    ids = g["input_ids"][0]
    assert len(ids) > valid
    args = (g["marker_pos"][0], g["marker_mask"][0], int(g["qtype"][0]))
    a = F.forward(cfg, w, ids, valid, *args)
    b = F.forward(cfg, w, ids[:valid], valid, *args)
    for name in ("embedding_output", "encoder_layer_00", "encoder_layer_02", "head_layer_00"):
        assert np.abs(a.trace[name][:valid] - b.trace[name][:valid]).max() <= 1e-5
    for name in ("logits", "probabilities", "act_logits", "pooled"):
        assert np.abs(a.trace[name] - b.trace[name]).max() <= 1e-5


@pytest.mark.parametrize("mistake", ["no_rope", "window_full", "swap_thetas", "gelu_gate"])
def test_planted_mistakes_miss_the_golden(mistake, monkeypatch):
    """Plausible slips in a forward restatement: each misses the golden by over 10x the 1e-5
    stage tolerance."""
    cfg, w, g, valid = load_case("medium")
    kw = {}
    if mistake == "no_rope":
        monkeypatch.setattr(oracle, "rope", lambda x, theta: np.asarray(x, np.float32).copy())
    elif mistake == "window_full":
        kw["local_mask"] = (oracle.MASK_FULL, 0)
    elif mistake == "swap_thetas":
        cfg.global_theta, cfg.local_theta = cfg.local_theta, cfg.global_theta
    else:
        real = oracle.gelu_array
        monkeypatch.setattr(oracle, "gelu_array", lambda x: x if x.shape[-1] == cfg.inter else real(x))
    out = run_case(cfg, w, g, valid, **kw)
    worst = max(d for _, d, _ in compare(cfg, g, valid, out.trace))
    assert worst > 10 * LAYER_TOL, mistake


def test_expected_parameter_set_matches_the_fixture_files():
    """mapping.rs's expected names and shapes are exactly what the fixture weights hold."""
    for cfgdir, wfile in (("fixture-h64", "weights-h64.safetensors"),
                          ("fixture-h128", "weights-h128.safetensors")):
        cfg = F.load_config(os.path.join(FWD, cfgdir))
        w = F.load_weights(os.path.join(FWD, wfile))
        exp = dict(F.expected_names(cfg))
        assert set(exp) == set(w)
        for name, shape in exp.items():
            assert tuple(w[name].shape) == shape, name
