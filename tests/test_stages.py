"""Stage timing of the attention kernel: Tiled::attend_with_stages and StageTimes
(crates/raya-kernels/src/tiled/mod.rs:61-126, tiled/stages.rs:3-31), test model
crates/raya-kernels/tests/stages.rs:7-32.

CPU: the StageTimes arithmetic and the argument checks, which run before any GPU work.
GPU: shares sum to 100, the tile count equals the kernel's tile schedule, and the
instrumented kernel's outputs equal the plain kernel's bit for bit.
"""
import ctypes

import numpy as np
import pytest

import raya_amd as R
from raya_amd import _capi as C
from raya_amd import synth


def test_percentages_are_none_when_nothing_was_timed():
    assert R.StageTimes().percentages() is None
    assert R.StageTimes(load_wait=5, tiles=3).percentages() is None


def test_percentages_and_merge():
    a = R.StageTimes(qk=30, softmax=50, pv=20, load_wait=1000, tiles=2)
    a.merge(R.StageTimes(qk=10, softmax=10, pv=80, load_wait=7, tiles=5))
    assert (a.qk, a.softmax, a.pv, a.load_wait, a.tiles) == (40, 60, 100, 1007, 7)
    qk, sm, pv = a.percentages()
    assert (qk, sm, pv) == (20.0, 30.0, 50.0)  # load_wait is not a share


def test_bad_arguments_are_errors_before_gpu_work():
    k = R.HipAttention()
    shape = R.AttnShape(1, 4, 8)
    ok = np.zeros(32, np.float32)
    p = R.AttnParams.new(R.Mask.WINDOW64, 4, 8)
    with pytest.raises(R.LengthError) as e:
        k.attend_with_stages(shape, p, np.zeros(3, np.float32), ok, ok, ok.copy())
    assert str(e.value) == "buffer `q` has length 3, expected 32"
    with pytest.raises(R.ShapeError):
        k.attend_with_stages(shape, p.replace(valid_len=5), ok, ok, ok, ok.copy())
    with pytest.raises(R.UnsupportedError):
        k.attend_with_stages(shape, p.replace(block=64), ok, ok, ok, ok.copy())
    s = C.AttnShapeC(1, 4, 8)
    cp = C.AttnParamsC(p.mask.kind, p.scale, 0, p.block, 4)
    buf = ctypes.c_void_p(ok.ctypes.data)
    assert C.lib().raya_attend_with_stages(ctypes.byref(s), ctypes.byref(cp), buf, 32, buf, 32, buf, 32,
                                           buf, 32, None) == C.RAYA_ERR_SHAPE
    desc = C.AttnBatchC(1, 1, 4, 8, p.mask.kind, p.scale, 0, p.block,
                        C.AttnLayoutC(), C.AttnLayoutC(), C.AttnLayoutC(), C.AttnLayoutC())
    assert C.lib().raya_attend_batched_stages(ctypes.byref(desc), buf, buf, buf, buf, buf, None,
                                              None) == C.RAYA_ERR_SHAPE


def test_empty_shape_times_nothing():
    e = np.zeros(0, np.float32)
    t = R.HipAttention().attend_with_stages(R.AttnShape(2, 0, 8), R.AttnParams.new(R.Mask.BLOCK3, 0, 8),
                                            e, e, e, e)
    assert t == R.StageTimes() and t.percentages() is None


# --- on the GPU --------------------------------------------------------------------------

def scheduled_tiles(mask: R.Mask, seq: int, valids, heads: int, rows: int = 64) -> int:
    """Tiles of 16 query rows x 64 keys the kernel computes: per workgroup of `rows`
    rows, the 64-key tiles spanning the rows' key ranges; per group of 16 rows (a wave,
    or with 16-row items the whole workgroup), those tiles that meet the group's keys."""
    def kr(i, valid):
        r = mask.key_range(i, valid)
        return r.start, r.stop

    n = 0
    for valid in valids:
        for q0 in range(0, seq, rows):
            if q0 >= valid:
                continue
            k_lo, k_hi = kr(q0, valid)[0], kr(min(q0 + rows, valid) - 1, valid)[1]
            for kt in range(k_lo, k_hi, 64):
                for w in range(rows // 16):
                    qw = q0 + 16 * w
                    if qw >= valid:
                        continue
                    first, last = kr(qw, valid), kr(min(qw + 15, valid - 1), valid)
                    n += kt < last[1] and kt + 64 > first[0]
    return n * heads


@pytest.fixture(params=["64", "16"], ids=["items64", "items16"])
def item_rows(request, monkeypatch):
    """Both attention kernels: 64-row items, and 16-row items with each tile's keys split
    over the waves (forced with RAYA_ATTN_ITEMS)."""
    monkeypatch.setenv("RAYA_ATTN_ITEMS", request.param)
    return int(request.param)


@pytest.mark.gpu
@pytest.mark.parametrize("mask", [R.Mask.WINDOW64, R.Mask.BLOCK3], ids=["window64", "block3"])
def test_stage_percentages_sum_to_one_hundred_when_timed(hip_attention, mask, item_rows):
    """stages.rs:7-32 on its shape (2 heads, L=512, D=64)."""
    shape = R.AttnShape(2, 512, 64)
    params = R.AttnParams.new(mask, 512, 64)
    q, k, v = (synth.xorshift_uniform(4 + i, shape.numel()) for i in range(3))
    out = np.zeros(shape.numel(), np.float32)
    times = hip_attention.attend_with_stages(shape, params, q, k, v, out)
    print(mask.name(), times, times.percentages(), flush=True)
    a, b, c = times.percentages()
    assert abs(a + b + c - 100.0) < 1e-6
    assert times.qk > 0 and times.softmax > 0 and times.pv > 0 and times.load_wait > 0
    assert times.tiles == scheduled_tiles(mask, 512, [512], 2, item_rows)
    plain = np.full(shape.numel(), 3.0, np.float32)
    hip_attention.attend(shape, params, q, k, v, plain)
    assert np.array_equal(out, plain)


@pytest.mark.gpu
def test_batched_stages_accumulate_and_match_the_plain_kernel(hip_attention, item_rows):
    """H=12, L=2048, D=64, BlockDiag(64), padded valid lengths; two launches into one
    total (StageTimes::merge), outputs bit-identical to raya_attend_batched."""
    import torch

    b, h, s, d = 3, 12, 2048, 64
    q, k, v = (torch.from_numpy(synth.normal(50 + i, b * h * s * d).reshape(b, h, s, d)).cuda()
               for i in range(3))
    valid_np = np.array([2048, 1000, 513], np.int32)
    valid = torch.from_numpy(valid_np).cuda()
    mask = R.Mask.block_diag(64)
    plain = torch.empty_like(q)
    hip_attention.attend_batched(q, k, v, plain, valid, mask)
    one = hip_attention.attend_batched_stages(q, k, v, torch.empty_like(q), valid, mask)
    assert one.tiles == scheduled_tiles(mask, s, valid_np.tolist(), h, item_rows)
    stages = torch.zeros(5, dtype=torch.int64, device="cuda")
    timed = torch.full_like(q, 9.0)
    for _ in range(2):
        hip_attention.attend_batched(q, k, v, timed, valid, mask, stages=stages)
    torch.cuda.synchronize()
    total = R.StageTimes(*stages.cpu().tolist())
    print("block_diag64 b3", one, one.percentages(), flush=True)
    assert total.tiles == 2 * one.tiles
    assert total.qk > one.qk and total.pv > one.pv
    assert torch.equal(timed, plain)
