"""The config-1 fixture (written by the compiled reference) regenerates from
its seed, and the oracle restatement reproduces it exactly."""
from pathlib import Path

import numpy as np

from hs_data import config1_inputs
from golden.make_golden import digest

FIXTURE = Path(__file__).resolve().parent / "golden" / "config1.npz"


def load():
    return np.load(FIXTURE, allow_pickle=False)


def test_inputs_regenerate():
    g = load()
    q, k, outliers = config1_inputs(0, int(g["n"]))
    assert str(g["inputs_sha256"]) == digest(q, k)
    assert np.array_equal(outliers, g["outliers"])


def test_oracle_reproduces_fixture(port):
    g = load()
    n = int(g["n"])
    q, k, _ = config1_inputs(0, n)
    raw = port.score(q, k.reshape(-1), n)
    assert np.array_equal(raw, g["raw"])
    scaled = port.scale(raw)
    assert np.array_equal(scaled, g["scaled"])
    rc, kk, ids, counts, tied = port.select(scaled, 32, n, n, float(g["alpha"]), float(g["ratio"]))
    assert rc == 0 and kk == int(g["k"]) and tied == int(g["boundary_tied_heads"])
    assert np.array_equal(ids, g["ids"]) and np.array_equal(counts, g["counts"])
