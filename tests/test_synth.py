"""Seeded input generators: published vectors, definitions on small cases, committed KATs."""
import json
import math
import os

import numpy as np
import pytest

from raya_amd import synth

KAT = os.path.join(os.path.dirname(__file__), "golden", "synth", "kat.json")


def test_splitmix64_published_vector():
    # Seed 1234567: the check values published with the reference implementation
    # of SplitMix64 (Vigna, splitmix64.c) and Java's SplittableRandom.
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423,
            4593380528125082431, 16408922859458223821]
    assert [int(x) for x in synth.splitmix64(1234567, 5)] == want


def test_splitmix64_offsets_are_a_window_of_the_stream():
    whole = synth.splitmix64(99, 40)
    assert np.array_equal(synth.splitmix64(99, 15, start=25), whole[25:])


def test_normal_is_box_muller_on_uniform_pairs():
    u = synth.uniform(11, 10)
    z = synth.normal(11, 9)  # odd n keeps the first of the last pair
    for p in range(5):
        r = math.sqrt(-2.0 * math.log1p(-u[2 * p]))
        th = 2.0 * math.pi * u[2 * p + 1]
        assert z[2 * p] == np.float32(r * math.cos(th))
        if 2 * p + 1 < 9:
            assert z[2 * p + 1] == np.float32(r * math.sin(th))


def test_normal_moments():
    z = synth.normal(3, 1 << 20).astype(np.float64)
    assert abs(z.mean()) < 5e-3 and abs(z.var() - 1.0) < 5e-3


def test_integers_are_inclusive_and_uniform():
    x = synth.integers(5, 200000, 3, 6)
    assert x.min() == 3 and x.max() == 6
    counts = np.bincount(x - 3) / x.size
    assert np.all(np.abs(counts - 0.25) < 0.01)


def _xorshift_scalar(seed, n):
    """The bench generator one step at a time (crates/raya-kernels/tests/common/mod.rs:6-18)."""
    m = (1 << 64) - 1
    s = ((seed * 0x9E3779B97F4A7C15) & m) | 1
    out = []
    for _ in range(n):
        s ^= (s << 13) & m
        s ^= s >> 7
        s ^= (s << 17) & m
        out.append(np.float32(2.0) * np.float32((s >> 40) / (1 << 24)) - np.float32(1.0))
    return np.array(out, np.float32)


@pytest.mark.parametrize("n,lanes", [(1, 4096), (7, 3), (1000, 4096), (5000, 64), (12345, 100)])
def test_xorshift_jump_ahead_matches_stepping(n, lanes):
    assert np.array_equal(synth.xorshift_uniform(42, n, lanes), _xorshift_scalar(42, n))


def test_xorshift_range():
    x = synth.xorshift_uniform(43, 1 << 16)
    assert x.min() >= -1.0 and x.max() < 1.0 and abs(float(x.mean())) < 0.01


def test_committed_known_answers():
    kat = json.load(open(KAT))
    for seed, vals in kat["splitmix64"].items():
        assert [str(int(x)) for x in synth.splitmix64(int(seed), 8)] == vals
    for seed, vals in kat["normal"].items():
        assert synth.normal(int(seed), 8).tolist() == vals
    assert synth.integers(2003, 8, 512, 2048).tolist() == kat["integers"]["2003 [512, 2048]"]
    assert synth.integers(5003, 8, 8192, 16384).tolist() == kat["integers"]["5003 [8192, 16384]"]
    for seed, vals in kat["xorshift_uniform"].items():
        assert synth.xorshift_uniform(int(seed), 8).tolist() == vals
