"""The measured encoder workloads themselves against the oracle's Network::forward
(crates/raya-core/src/model.rs:261-348), through the C ABI, at their full sizes.

* One block-local encoder layer: ModernBERT-base width (768 = 12 x 64, GeGLU 3072,
  LayerNorm eps 1e-12), N(0, 0.02) weights and norms of one, BlockDiag(64) on the local
  layer, 16 sequences of 1,024 valid tokens.  The model has two layers: layer 0 is the
  global (Full) layer every ModernBERT stack starts with, layer 1 the block-local layer
  whose output is compared.
* The full 12-layer forward of the bench: the bench's own synthetic checkpoint (vocab
  30,522, max positions 4,096, weight seed and token ids as the bench draws them), 64
  sequences of up to 512 tokens with the bench's valid lengths; every traced stage and
  every output of three sequences (the first, the longest and the shortest).

The GPU runs the whole batch; the oracle runs the compared sequences one at a time.  The
bar is the fp32 one, max-abs 1e-4 and rel-L2 1e-5 on every stage and output; the
probabilities within 5e-6, which is what 1e-5 on the logits allows
(|dp_i| <= p_i (1 - p_i) |dz_i - dz_j|)."""
import os

import numpy as np
import pytest

import oracle
from oracle import forward as F
from raya_amd import Mask, checkpoint
from raya_amd import model as M
from raya_amd import workloads as W

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2, PROB_ABS = 1e-4, 1e-5, 5e-6


def _threads():
    return max(1, min(16, len(os.sched_getaffinity(0))))


def _compare(name, got, want, worst):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (name, got.shape, want.shape)
    err = np.abs(got - want)
    rel = float(np.sqrt((err ** 2).sum() / max(float((want ** 2).sum()), 1e-30)))
    mx = float(err.max()) if err.size else 0.0
    worst[name] = max(worst.get(name, (0.0, 0.0)), (mx, rel))
    if name in ("probabilities", "act_features"):
        assert mx <= PROB_ABS, (name, mx)
    else:
        assert mx <= MAX_ABS and rel <= REL_L2, (name, mx, rel)


def _check_sequence(tr, i, v, want, worst, seq):
    """Every stage of sequence i of a batched trace against the oracle's own trace."""
    for name, ref in want.trace.items():
        _, arr = tr.get(name)
        got = arr[i]
        if got.ndim == 2 and got.shape[0] == seq:  # [seq, d] stages: the valid rows
            got = got[:v]
        _compare(name, got.reshape(np.asarray(ref).shape), ref, worst)


@pytest.mark.timeout(900)
def test_block_local_layer_workload(tmp_path):
    """16 x 1,024 tokens through a 768-wide layer with BlockDiag(64), as the bench's layer
    line runs it; sequences 0 and 15 against the oracle at every stage."""
    spec = W.LAYER
    enc = dict(checkpoint.MODERNBERT_BASE)
    enc["num_hidden_layers"] = 2
    ckpt = str(tmp_path / "layer")
    checkpoint.write_synthetic(ckpt, encoder=enc, seed=1000 * spec["family"] + 5)
    model = M.Model.load(ckpt)
    ids, valid, pos, mask, qtype = W.encoder_inputs(spec)
    assert ids.shape == (16, 1024) and (valid == 1024).all()
    print(f"layer workload: B={len(valid)} L={ids.shape[1]} block_diag({spec['block']})", flush=True)
    tr = M.Trace()
    out = model.forward_batch(ids, valid, pos, mask, qtype, trace=tr,
                              local_mask=Mask.block_diag(spec["block"]))
    cfg = F.load_config(ckpt)
    w = F.load_weights(os.path.join(ckpt, "model.safetensors"))
    F.GEMM_THREADS = _threads()
    worst = {}
    for i in (0, 15):
        v = int(valid[i])
        want = F.forward(cfg, w, ids[i, :v], v, pos[i], mask[i], int(qtype[i]),
                         local_mask=(oracle.MASK_BLOCKDIAG, spec["block"]))
        _check_sequence(tr, i, v, want, worst, ids.shape[1])
        _compare("act_logits", out.act_logits[i], want.act_logits, worst)
        _compare("pooled", out.pooled[i], want.pooled, worst)
    print({k: f"{a:.1e}/{r:.1e}" for k, (a, r) in worst.items()}, flush=True)
    assert {"encoder_layer_01", "pooled", "act_logits"} <= set(worst)


@pytest.mark.timeout(900)
def test_twelve_layer_encoder_workload(tmp_path):
    """The bench's encoder line: its checkpoint and batch, 64 sequences on the GPU; three of
    them through the oracle, every stage and output compared."""
    spec = W.ENCODER
    ckpt = str(tmp_path / "enc")
    checkpoint.write_synthetic(ckpt, seed=W.ENCODER_WEIGHT_SEED)
    model = M.Model.load(ckpt)
    info = model.info
    assert (info["num_hidden_layers"], info["hidden_size"]) == (12, 768)
    ids, valid, pos, mask, qtype = W.encoder_inputs(spec)
    assert ids.shape == (64, 512)
    picks = sorted({0, int(np.argmax(valid)), int(np.argmin(valid))})
    print(f"encoder workload: B={len(valid)} L={ids.shape[1]} valid {int(valid.min())}..{int(valid.max())}, "
          f"checking sequences {picks}", flush=True)
    tr = M.Trace()
    out = model.forward_batch(ids, valid, pos, mask, qtype, trace=tr)
    plain = model.forward_batch(ids, valid, pos, mask, qtype)  # no trace: the bench's own call
    for f in ("logits", "probabilities", "act_logits", "features", "pooled"):
        assert np.array_equal(getattr(out, f), getattr(plain, f)), f
    cfg = F.load_config(ckpt)
    w = F.load_weights(os.path.join(ckpt, "model.safetensors"))
    F.GEMM_THREADS = _threads()
    worst = {}
    for i in picks:
        v = int(valid[i])
        want = F.forward(cfg, w, ids[i, :v], v, pos[i], mask[i], int(qtype[i]))
        _check_sequence(tr, i, v, want, worst, ids.shape[1])
        for f, name in (("logits", "logits"), ("probabilities", "probabilities"),
                        ("act_logits", "act_logits"), ("features", "act_features"), ("pooled", "pooled")):
            _compare(name, getattr(out, f)[i], getattr(want, f), worst)
        print(f"  sequence {i} (valid {v}) done", flush=True)
    print({k: f"{a:.1e}/{r:.1e}" for k, (a, r) in worst.items()}, flush=True)
    assert {f"encoder_layer_{i:02d}" for i in range(12)} <= set(worst)


@pytest.mark.timeout(600)
def test_twelve_layer_encoder_batch_order_and_size(tmp_path):
    """Whole-batch properties of the bench's 12-layer forward (all 64 sequences): reversing
    the batch reverses every output bit for bit (each sequence's rows, tiles and statistics
    are computed the same wherever it sits in the packed batch, so nothing leaks between
    sequences); and each group of 8 sequences run on its own (a smaller grid, where the
    attention may take its other kernel) agrees with the batch of 64 at the fp32 bar."""
    spec = W.ENCODER
    ckpt = str(tmp_path / "enc")
    checkpoint.write_synthetic(ckpt, seed=W.ENCODER_WEIGHT_SEED)
    model = M.Model.load(ckpt)
    ids, valid, pos, mask, qtype = W.encoder_inputs(spec)
    fields = ("logits", "probabilities", "act_logits", "features", "pooled")
    out = model.forward_batch(ids, valid, pos, mask, qtype)
    rev = slice(None, None, -1)
    back = model.forward_batch(ids[rev], valid[rev], pos[rev], mask[rev], qtype[rev])
    for f in fields:
        assert np.array_equal(getattr(back, f)[rev], getattr(out, f)), f
    worst = {}
    for g0 in range(0, len(valid), 8):
        part = slice(g0, g0 + 8)
        sub = model.forward_batch(ids[part], valid[part], pos[part], mask[part], qtype[part])
        for f in fields:
            name = "act_features" if f == "features" else f
            _compare(name, getattr(sub, f), getattr(out, f)[part], worst)
    print({k: f"{a:.1e}/{r:.1e}" for k, (a, r) in worst.items()}, flush=True)


@pytest.mark.timeout(600)
def test_split_k_forward_matches_the_unsplit_batch(tmp_path):
    """One sequence alone (few rows: every encoder GEMM and the act head split K into partial
    tiles and a reducing launch) against the same sequence inside the bench's batch of 64
    (thousands of rows: no GEMM splits), every output at the fp32 bar; and the split forward
    run twice gives the same bits (the partials are summed in a fixed order)."""
    spec = W.ENCODER
    ckpt = str(tmp_path / "enc")
    checkpoint.write_synthetic(ckpt, seed=W.ENCODER_WEIGHT_SEED)
    model = M.Model.load(ckpt)
    ids, valid, pos, mask, qtype = W.encoder_inputs(spec)
    batch = model.forward_batch(ids, valid, pos, mask, qtype)
    fields = ("logits", "probabilities", "act_logits", "features", "pooled")
    worst = {}
    for i in sorted({0, int(np.argmax(valid)), int(np.argmin(valid))}):
        one = slice(i, i + 1)
        alone = model.forward_batch(ids[one], valid[one], pos[one], mask[one], qtype[one])
        again = model.forward_batch(ids[one], valid[one], pos[one], mask[one], qtype[one])
        for f in fields:
            assert np.array_equal(getattr(alone, f), getattr(again, f)), f
            _compare("act_features" if f == "features" else f, getattr(alone, f)[0], getattr(batch, f)[i], worst)
    print({k: f"{a:.1e}/{r:.1e}" for k, (a, r) in worst.items()}, flush=True)
