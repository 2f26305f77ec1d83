"""Bench metadata: the cases of crates/raya-kernels/src/meta.rs:106-182, restated for
raya_amd.meta, plus the build stamp of the library (raya_build_info)."""
import json
import re

import pytest

from raya_amd import meta


def test_serialises_every_field():
    m = meta.collect(2, None, use_env=False)
    text = json.dumps(m)
    for key in ("label", "cpu_model", "logical_cpus", "physical_cpus", "threads", "features",
                "backend", "build_flags", "compiler", "git_commit", "timestamp", "gpu"):
        assert key in m, key
    assert json.loads(text)["threads"] == 2
    assert m["backend"] == "hip-gfx950" and "stage-timing" in m["features"]
    assert re.fullmatch(r"unix:\d+", m["timestamp"])


@pytest.mark.parametrize("env", [None, "", "0", "yes"])
def test_label_never_claims_hardware_without_the_env_var(env):
    label = meta.collect(1, env, use_env=False)["label"]
    assert label == meta.LABEL_UNLABELED and "cloud-agent" not in label


@pytest.mark.parametrize("env", ["cloud", "Cloud-Agent", "cloud-agent ", "true", "2", "target machine"])
def test_unknown_values_are_unlabeled_not_cloud(env):
    assert meta.label_for(env) == meta.LABEL_UNLABELED


def test_cloud_agent_value_gives_the_cloud_label():
    assert meta.label_for("cloud-agent") == meta.LABEL_CLOUD
    assert meta.LABEL_CLOUD == "cloud-agent hardware, indicative only"


def test_label_is_serialised_verbatim():
    assert json.loads(json.dumps(meta.collect(1, None, use_env=False)))["label"] == meta.LABEL_UNLABELED
    assert meta.LABEL_UNLABELED == "unlabeled machine, indicative only"


def test_label_is_target_machine_when_env_is_one():
    assert meta.label_for("1") == meta.LABEL_TARGET


def test_env_var_is_read_by_default(monkeypatch):
    monkeypatch.setenv("RAYA_TARGET_MACHINE", "cloud-agent")
    assert meta.collect(1)["label"] == meta.LABEL_CLOUD
    monkeypatch.delenv("RAYA_TARGET_MACHINE")
    assert meta.collect(1)["label"] == meta.LABEL_UNLABELED


def test_build_stamp():
    b = meta.build_info()
    assert b["arch"] == "gfx950"
    assert b["commit"] == "unknown" or re.fullmatch(r"[0-9a-f]{40}", b["commit"])
    assert "--offload-arch=gfx950" in b["flags"] and "-packed-fp32-ops" in b["flags"]
    assert b["compiler"].startswith("HIP version") or b["compiler"] == "unknown"


@pytest.mark.parametrize("value,want", [("4", 4), (" 8 ", 8), ("+3", 3), ("12\n", 12)])
def test_raya_threads_parses_like_threads_rs(value, want):
    """threads.rs:3-9: RAYA_THREADS when it parses to a positive usize."""
    assert meta.default_threads(value) == want


@pytest.mark.parametrize("value", ["0", "-2", "abc", "4.0", "1_000", "", "0x10", "٣"])
def test_raya_threads_falls_back_to_physical_cores(value):
    """Anything else (zero, signs, non-digits, Python-only integer spellings) falls back to the
    physical cores this process may run on."""
    assert meta.default_threads(value) == meta.default_threads(use_env=False) >= 1


def test_raya_threads_env(monkeypatch):
    monkeypatch.setenv("RAYA_THREADS", "5")
    assert meta.default_threads() == 5
    monkeypatch.delenv("RAYA_THREADS")
    assert meta.default_threads() == meta.default_threads(use_env=False)
