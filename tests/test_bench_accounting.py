"""bench.py's algorithmic work: FLOP and bytes per launch against a brute-force count of
allowed (query, key) pairs through the host mirror of Mask::key_range (attention.rs:48-59)."""
import json
import subprocess
import sys

import numpy as np
import pytest

import bench
from raya_amd import Mask
from raya_amd import workloads as W
from tests.conftest import ROOT


def brute_pairs(mask, v):
    return sum(len(mask.key_range(i, v)) for i in range(v))


@pytest.mark.parametrize("spec,mask", [(("block_diag", 64), Mask.block_diag(64)),
                                       (("block_diag", 128), Mask.block_diag(128)),
                                       (("block3",), Mask.BLOCK3), (("window64",), Mask.WINDOW64)])
@pytest.mark.parametrize("v", [0, 1, 63, 64, 65, 127, 128, 129, 300, 512, 1000, 2048])
def test_key_pairs_match_key_range(spec, mask, v):
    assert W.key_pairs(spec, v) == brute_pairs(mask, v)


def test_algorithmic_flop_and_bytes():
    valid = np.array([512, 700, 2048], np.int32)
    h, d, s = 12, 64, 2048
    flops, nbytes = W.algorithmic(valid, h, d, s, ("block_diag", 64))
    pairs = sum(brute_pairs(Mask.block_diag(64), int(v)) for v in valid)
    assert flops == 4 * d * h * pairs
    assert nbytes == 4 * (3 * h * d * int(valid.sum()) + len(valid) * h * s * d)


def test_headline_workload_figures():
    """The default workload's per-launch figures quoted in the profiles."""
    from raya_amd import synth

    wl = W.ATTENTION[W.DEFAULT_ATTENTION]
    lo, hi = wl["valid"]  # the valid lengths make_inputs draws, without the Q/K/V tensors
    valid = synth.integers(synth.workload_seed(wl["family"], 3), wl["batch"], lo, hi)
    flops, nbytes = W.algorithmic(valid, wl["heads"], wl["head_dim"], wl["seq"], wl["mask"])
    assert (flops, nbytes) == (7_387_216_896, 550_548_480)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], cwd=ROOT, capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr
