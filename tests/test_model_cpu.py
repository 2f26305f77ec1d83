"""The decision model's host side on the CPU: config and weights loading with the
reference's error reports, and input checks, all before any GPU work.

Follows crates/raya-core/tests/config.rs, crates/raya-weights/tests/load_negative.rs
and Network::check (crates/raya-core/src/model.rs:221-258).
"""
import json
import os
import shutil
import struct

import numpy as np
import pytest

from raya_amd import model as M
from tests.conftest import GOLDEN

FWD = os.path.join(GOLDEN, "forward")
H64 = os.path.join(FWD, "fixture-h64")
W64 = os.path.join(FWD, "weights-h64.safetensors")


def load64():
    return M.Model.load(H64, W64)


def test_fixture_configs_load_with_their_weights():
    for cfg, w, d in (("fixture-h64", "weights-h64.safetensors", 64),
                      ("fixture-h128", "weights-h128.safetensors", 128)):
        info = M.Model.load(os.path.join(FWD, cfg), os.path.join(FWD, w)).info
        assert info["hidden_size"] == d and info["num_hidden_layers"] == 3
        assert (info["global_rope_theta"], info["local_rope_theta"]) == (160000.0, 10000.0)
        assert (info["head_layers"], info["head_heads"], info["head_ffn"]) == (1, max(1, d // 64), 4 * d)
        assert info["n_act"] == 2 and info["local_attention"] == 16


def test_h128_config_does_not_match_h64_weights():
    with pytest.raises(M.WeightsError) as e:
        M.Model.load(os.path.join(FWD, "fixture-h128"), W64)
    assert "encoder.embeddings.tok_embeddings.weight: expected [231, 128], found [231, 64]" in str(e.value)


def _config_dir(tmp_path, enc_edit=None, agent_edit=None):
    d = tmp_path / "ckpt"
    shutil.copytree(H64, d)
    enc = json.load(open(d / "encoder" / "config.json"))
    agent = json.load(open(d / "rl_agent_config.json"))
    if enc_edit:
        enc_edit(enc)
    if agent_edit:
        agent_edit(agent)
    json.dump(enc, open(d / "encoder" / "config.json", "w"))
    json.dump(agent, open(d / "rl_agent_config.json", "w"))
    return str(d)


def _field(err) -> str:
    text = str(err.value)
    assert text.startswith("invalid config: `"), text
    return text.split("`")[1]


@pytest.mark.parametrize("key", ["hidden_size", "intermediate_size", "num_hidden_layers",
                                 "num_attention_heads", "norm_eps", "vocab_size"])
def test_missing_required_field_names_the_key(tmp_path, key):
    d = _config_dir(tmp_path, enc_edit=lambda e: e.pop(key))
    with pytest.raises(M.ConfigError) as err:
        M.Model.load(d, W64)
    assert _field(err) == key


def test_missing_rope_theta_names_the_key(tmp_path):
    def edit(e):
        e["rope_parameters"].pop("sliding_attention")
    with pytest.raises(M.ConfigError) as err:
        M.Model.load(_config_dir(tmp_path, enc_edit=edit), W64)
    assert _field(err) == "local_rope_theta"


def test_rope_parameters_forms(tmp_path):
    def edit(e):
        e.pop("rope_parameters")
        e["global_rope_theta"], e["local_rope_theta"] = 123.0, 45.0
    info = M.Model.load(_config_dir(tmp_path, enc_edit=edit), W64).info
    assert (info["global_rope_theta"], info["local_rope_theta"]) == (123.0, 45.0)


def test_wrong_types_name_the_key(tmp_path):
    with pytest.raises(M.ConfigError) as err:
        M.Model.load(_config_dir(tmp_path / "a", enc_edit=lambda e: e.update(hidden_size="64")), W64)
    assert _field(err) == "hidden_size"
    with pytest.raises(M.ConfigError) as err:
        M.Model.load(_config_dir(tmp_path / "b", agent_edit=lambda a: a.update(temperature=[1, "x", 1])),
                     W64)
    assert _field(err) == "temperature"


@pytest.mark.parametrize("edit,field", [
    (lambda e: e.update(num_attention_heads=3), "hidden_size"),
    (lambda e: e.update(local_attention=0), "local_attention"),
    (lambda e: e.update(norm_eps=0.0), "norm_eps"),
])
def test_inconsistent_fields_are_rejected(tmp_path, edit, field):
    with pytest.raises(M.ConfigError) as err:
        M.Model.load(_config_dir(tmp_path, enc_edit=edit), W64)
    assert _field(err) == field


def test_bad_temperature_and_bias_flags(tmp_path):
    with pytest.raises(M.ConfigError) as err:
        M.Model.load(_config_dir(tmp_path / "a", agent_edit=lambda a: a.update(temperature=[1.0, 1.0])),
                     W64)
    assert _field(err) == "temperature"
    with pytest.raises(M.UnimplementedError, match="mlp_bias=true"):
        M.Model.load(_config_dir(tmp_path / "b", enc_edit=lambda e: e.update(mlp_bias=True)), W64)
    with pytest.raises(M.UnimplementedError, match="hidden_activation `relu`"):
        M.Model.load(_config_dir(tmp_path / "c", enc_edit=lambda e: e.update(hidden_activation="relu")),
                     W64)


def test_missing_directory_is_an_io_error(tmp_path):
    with pytest.raises(M.ConfigError, match="cannot read"):
        M.Model.load(str(tmp_path / "nope"))


def _tensors():
    from safetensors.numpy import load_file

    return dict(load_file(W64))


def _save(tmp_path, tensors, name="w.safetensors"):
    from safetensors.numpy import save_file

    p = str(tmp_path / name)
    save_file(tensors, p)
    return p


def test_weights_report_missing_unused_and_shapes(tmp_path):
    t = _tensors()
    t.pop("temperature")
    with pytest.raises(M.WeightsError) as e:
        M.Model.load(H64, _save(tmp_path, t, "a.safetensors"))
    assert "missing tensors:\n    temperature" in str(e.value)
    t = _tensors()
    t.pop("type_emb.weight")
    t["bogus.weight"] = np.zeros(3, np.float32)
    with pytest.raises(M.WeightsError) as e:
        M.Model.load(H64, _save(tmp_path, t, "b.safetensors"))
    text = str(e.value)
    assert "missing tensors:\n    type_emb.weight" in text and "unexpected tensors:\n    bogus.weight" in text
    t = _tensors()
    t["type_emb.weight"] = np.ascontiguousarray(t["type_emb.weight"].T)
    with pytest.raises(M.WeightsError, match=r"type_emb.weight: expected \[3, 64\], found \[64, 3\]"):
        M.Model.load(H64, _save(tmp_path, t, "c.safetensors"))


def test_unsupported_dtype_is_unimplemented(tmp_path):
    t = _tensors()
    t["temperature"] = t["temperature"].astype(np.float64)
    with pytest.raises(M.UnimplementedError, match=r"temperature \(F64\)"):
        M.Model.load(H64, _save(tmp_path, t))


def test_truncated_and_junk_files(tmp_path):
    raw = open(W64, "rb").read()
    trunc = tmp_path / "trunc.safetensors"
    trunc.write_bytes(raw[: len(raw) // 2])
    with pytest.raises(M.WeightsError, match="invalid weights file"):
        M.Model.load(H64, str(trunc))
    junk = tmp_path / "junk.safetensors"
    junk.write_bytes(b"\x05\x00\x00\x00\x00\x00\x00\x00{abc}")
    with pytest.raises(M.WeightsError, match="invalid weights file"):
        M.Model.load(H64, str(junk))


def test_duplicate_key_is_reported(tmp_path):
    """store.rs:239-281: a name twice in the header is reported, not silently overwritten."""
    raw = open(W64, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    header = raw[8:8 + n].decode()
    entry = json.loads(header)["temperature"]
    body = header.rstrip()
    assert body.endswith("}")
    dup = body[:-1] + ',"temperature":' + json.dumps(entry) + "}"
    dup_b = dup.encode()
    dup_b += b" " * ((8 - len(dup_b) % 8) % 8)
    p = tmp_path / "dup.safetensors"
    p.write_bytes(struct.pack("<Q", len(dup_b)) + dup_b + raw[8 + n:])
    with pytest.raises(M.WeightsError) as e:
        M.Model.load(H64, str(p))
    assert "duplicate tensors:\n    temperature" in str(e.value)
    assert "missing" not in str(e.value)


def test_half_precision_weights_load(tmp_path):
    t = {k: v.astype(np.float16) for k, v in _tensors().items()}
    assert M.Model.load(H64, _save(tmp_path, t)).info["hidden_size"] == 64


@pytest.mark.parametrize("change,message", [
    (dict(ids=[1, 2, 231]), "token id 231 is outside the vocabulary of 231"),
    (dict(valid=0), "valid_len 0 is not in 1..=3"),
    (dict(valid=4), "valid_len 4 is not in 1..=3"),
    (dict(pos=[3], mask=[True]), "marker position 3 is outside the sequence (valid_len 3, length 3)"),
    (dict(valid=2, pos=[2], mask=[True]), "marker position 2 is outside the sequence (valid_len 2, length 3)"),
    (dict(pos=[0], mask=[False]), "no valid marker"),
    (dict(qtype=3), "qtype 3 is not 0, 1 or 2"),
])
def test_input_checks_match_network_check(change, message):
    m = load64()
    kw = dict(ids=[1, 2, 3], valid=3, pos=[0], mask=[True], qtype=0)
    kw.update(change)
    inp = M.ForwardInput(np.array(kw["ids"]), kw["valid"], np.array(kw["pos"]),
                         np.array(kw["mask"]), kw["qtype"])
    with pytest.raises(M.InputError) as e:
        m.forward(inp)
    assert str(e.value) == "invalid input: " + message


def test_invalid_marker_may_sit_on_padding():
    """A masked-out marker beyond valid_len (but inside the sequence) is accepted by the
    check; without a GPU the call then fails at the device, not at the check."""
    m = load64()
    inp = M.ForwardInput(np.array([1, 2, 3]), 2, np.array([0, 2]), np.array([True, False]), 0)
    try:
        m.forward(inp)
    except M.InputError as e:  # pragma: no cover - would be a check bug
        raise AssertionError(str(e))
    except Exception:
        pass


def test_expected_params_follow_the_mapping():
    """raya_expected_params lists mapping.rs's names and shapes in order, the same set the
    fixture weights hold (and the oracle's restatement of the mapping)."""
    from oracle import forward as F
    from raya_amd import checkpoint

    for cfg_dir in ("fixture-h64", "fixture-h128"):
        got = checkpoint.expected_params(os.path.join(FWD, cfg_dir))
        want = F.expected_names(F.load_config(os.path.join(FWD, cfg_dir)))
        assert got == [(n, tuple(s)) for n, s in want]


def test_synthetic_checkpoint_round_trips(tmp_path):
    """A written checkpoint loads, with the shapes the config implies."""
    from raya_amd import checkpoint

    enc = dict(checkpoint.MODERNBERT_BASE, hidden_size=128, num_attention_heads=2,
               intermediate_size=256, num_hidden_layers=2, vocab_size=500)
    checkpoint.write_synthetic(str(tmp_path), encoder=enc, seed=1)
    info = M.Model.load(str(tmp_path)).info
    assert (info["hidden_size"], info["num_hidden_layers"], info["n_act"]) == (128, 2, 2)
    assert info["norm_eps"] == 1e-12 and info["head_layers"] == 0


def test_profiling_level_is_checked_and_starts_empty():
    m = load64()
    assert m.stage_times() == []
    for level in (0, 1, 2):
        m.set_profiling(level)
        assert m.stage_times() == []
    for bad in (-1, 3):
        with pytest.raises(M.InputError, match="profiling level"):
            m.set_profiling(bad)
