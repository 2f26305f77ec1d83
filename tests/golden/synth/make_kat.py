"""Writes the known-answer vectors of the seeded input generators (kat.json).

The first 8 outputs of each stream, so any other implementation of the
generators (a host binding in another language) can check that it draws the
same inputs.  Run from the repository root: python tests/golden/synth/make_kat.py
"""
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
sys.path.insert(0, ROOT)

from raya_amd import synth  # noqa: E402


def main():
    kat = {"splitmix64": {}, "normal": {}, "integers": {}, "xorshift_uniform": {}}
    for c in (1, 2, 3, 4, 5):
        for s in range(7):
            seed = synth.workload_seed(c, s)
            kat["splitmix64"][str(seed)] = [str(int(x)) for x in synth.splitmix64(seed, 8)]
            kat["normal"][str(seed)] = [float(x) for x in synth.normal(seed, 8)]
    kat["integers"]["2003 [512, 2048]"] = [int(x) for x in synth.integers(2003, 8, 512, 2048)]
    kat["integers"]["5003 [8192, 16384]"] = [int(x) for x in synth.integers(5003, 8, 8192, 16384)]
    for seed in (42, 43, 44):
        kat["xorshift_uniform"][str(seed)] = [float(x) for x in synth.xorshift_uniform(seed, 8)]
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kat.json")
    with open(path, "w") as f:
        json.dump(kat, f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
