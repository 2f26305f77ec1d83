"""Edge cases of the decision-model forward, as the reference's own tests state them
(crates/raya-core/tests/forward_edges.rs, forward_tiny.rs), on a small random model,
for both the oracle (CPU) and the device forward (GPU).

Markers: an invalid marker gets logit -1e4 and probability 0 and leaves the valid
markers' outputs as if it were absent; features count valid markers only.  Shapes:
a one-token sequence runs; valid_len 1 inside a padded sequence equals the one-token
sequence; padding after valid_len changes nothing.  qtype selects its type-embedding
row.  Tracing (and on the device, batching) changes no number.
"""
import math

import numpy as np
import pytest

from oracle import forward as F
from raya_amd import model as M
from tests.test_model_gpu import make_model

TOL = 1e-6


@pytest.fixture(scope="module")
def random_model(tmp_path_factory):
    return make_model(tmp_path_factory.mktemp("edges"), 64, 2, layers=3, head_layers=2)


class Run:
    """One backend: run(ids, valid, pos, mask, qtype) -> (outputs, {stage: rows})."""

    def __init__(self, kind, cfg, cdir, w):
        self.kind, self.cfg, self.w = kind, cfg, w
        self.model = M.Model.load(cdir) if kind == "device" else None

    def __call__(self, ids, valid, pos, mask, qtype=0):
        pos, mask = np.array(pos), np.array(mask, bool)
        if self.kind == "oracle":
            out = F.forward(self.cfg, self.w, ids, valid, pos, mask, qtype)
            return out, out.trace
        tr = M.Trace()
        out = self.model.forward(M.ForwardInput(ids, valid, pos, mask, qtype), trace=tr)
        stages = {}
        for name in tr.names():
            shape, arr = tr.get(name)
            stages[name] = arr.reshape(shape[1:])  # the batch of one
        return out, stages


@pytest.fixture(params=["oracle", pytest.param("device", marks=pytest.mark.gpu)])
def run(request, random_model):
    cfg, cdir, w = random_model
    return Run(request.param, cfg, cdir, w)


def ids_of(n, seed=1):
    return np.random.default_rng(seed).integers(1, 300, size=n).astype(np.uint32)


def close(a, b, tol=TOL):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    assert a.shape == b.shape and np.abs(a - b).max() <= tol, (a, b)


def test_a_leading_invalid_marker_leaves_the_valid_ones_unchanged(run):
    """forward_edges.rs:50-62"""
    ids = ids_of(12)
    full, _ = run(ids, 12, [5, 8], [True, True])
    out, _ = run(ids, 12, [2, 5, 8], [False, True, True])
    assert out.logits[0] == np.float32(-1e4) and out.probabilities[0] == 0.0
    close(out.logits[1:], full.logits)
    close(out.probabilities[1:], full.probabilities)
    close(out.features, full.features)
    assert abs(float(out.probabilities.sum()) - 1.0) < 1e-6


def test_an_invalid_marker_in_the_middle_keeps_slots_aligned(run):
    """forward_edges.rs:64-78"""
    ids = ids_of(12)
    packed, _ = run(ids, 12, [2, 8], [True, True])
    out, _ = run(ids, 12, [2, 5, 8], [True, False, True])
    assert out.logits[1] == np.float32(-1e4) and out.probabilities[1] == 0.0
    close(out.logits[[0, 2]], packed.logits)
    close(out.probabilities[[0, 2]], packed.probabilities)
    close(out.features, packed.features)


def test_the_shortest_sequence_runs(run):
    """forward_edges.rs:79-88"""
    out, _ = run(ids_of(1), 1, [0], [True])
    assert np.isfinite(out.logits).all() and np.isfinite(out.pooled).all()
    assert np.isfinite(out.act_logits).all()
    assert out.probabilities.tolist() == [1.0]


def test_valid_len_one_inside_a_longer_padded_sequence_matches_seq_one(run):
    """forward_edges.rs:89-98"""
    ids = ids_of(6)
    short, _ = run(ids[:1], 1, [0], [True])
    padded, _ = run(ids, 1, [0], [True])
    close(padded.logits, short.logits)
    close(padded.pooled, short.pooled)
    close(padded.act_logits, short.act_logits)


def test_qtype_selects_its_type_embedding_row(run):
    """forward_edges.rs:99-121"""
    ids, pos, mask = ids_of(9), [1, 4, 6], [True] * 3
    out2, tr = run(ids, 9, pos, mask, qtype=2)
    assert np.isfinite(out2.logits).all() and np.isfinite(out2.act_logits).all()
    te = run.w["type_emb.weight"]
    assert te.shape == (3, run.cfg.hidden)
    close(np.asarray(tr["type_emb_add"]).reshape(-1), te[2], 0.0)
    out0, _ = run(ids, 9, pos, mask, qtype=0)
    out1, _ = run(ids, 9, pos, mask, qtype=1)
    assert not np.array_equal(out2.logits, out0.logits)
    assert not np.array_equal(out2.logits, out1.logits)
    assert not np.array_equal(out0.logits, out1.logits)


def _entropy(p):
    return -sum(x * math.log(max(x, 1e-9)) for x in p) / math.log(len(p))


def test_features_for_four_options_follow_the_formula(run):
    """forward_edges.rs:122-138: top1, top1 - top2, normalised entropy, k / 255."""
    out, _ = run(ids_of(12), 12, [1, 3, 5, 7], [True] * 4)
    p = out.probabilities.astype(np.float64)
    assert p.shape == (4,) and abs(p.sum() - 1.0) < 1e-6
    s = np.sort(p)[::-1]
    assert abs(out.features[0] - s[0]) < 1e-7
    assert abs(out.features[1] - (s[0] - s[1])) < 1e-7
    assert abs(out.features[2] - _entropy(p)) < 1e-6
    assert 0.0 < out.features[2] <= 1.0 + 1e-6
    assert abs(out.features[3] - 4.0 / 255.0) < 1e-9


def test_features_count_valid_markers_only(run):
    """forward_edges.rs:139-148"""
    out, _ = run(ids_of(12), 12, [1, 3, 5, 7], [True, False, True, True])
    assert out.probabilities[1] == 0.0
    assert abs(out.features[3] - 3.0 / 255.0) < 1e-9
    p = out.probabilities[[0, 2, 3]].astype(np.float64)
    assert abs(out.features[2] - _entropy(p)) < 1e-6


def test_a_single_marker_follows_the_single_option_rule(run):
    """forward_tiny.rs:92-107"""
    out, _ = run(ids_of(8), 8, [3], [True])
    assert out.probabilities.tolist() == [1.0]
    assert out.features[0] == 1.0 and out.features[1] == 1.0
    assert abs(out.features[2]) < 1e-7
    assert abs(out.features[3] - 2.0 / 255.0) < 1e-9


def test_padding_after_valid_len_changes_nothing(run):
    """forward_tiny.rs:109-133, on the logits and the head layer's valid rows."""
    ids = ids_of(14)
    a, full = run(ids, 9, [1, 6], [True, True])
    b, cut = run(ids[:9], 9, [1, 6], [True, True])
    close(a.logits, b.logits)
    close(np.asarray(full["head_layer_00"])[:9], np.asarray(cut["head_layer_00"])[:9])


@pytest.mark.gpu
def test_tracing_and_batching_change_no_number(random_model):
    """forward_tiny.rs:72-90 on the device, plus: a sequence in a batch equals it alone."""
    cfg, cdir, w = random_model
    model = M.Model.load(cdir)
    ids = ids_of(20)
    args = (ids, 20, np.array([2, 9, 15]), np.ones(3, bool), 1)
    plain = model.forward(M.ForwardInput(*args))
    traced = model.forward(M.ForwardInput(*args), trace=M.Trace())
    for f in ("logits", "probabilities", "act_logits", "features", "pooled"):
        assert np.array_equal(getattr(plain, f), getattr(traced, f)), f
    other = ids_of(20, seed=2)
    batch = model.forward_batch(np.stack([other, ids]), [13, 20], np.array([[1, 5, 7], [2, 9, 15]]),
                                np.ones((2, 3), bool), [0, 1])
    close(batch.act_logits[1], plain.act_logits)
    close(batch.logits[1], plain.logits)
