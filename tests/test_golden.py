"""The oracle and the synthetic generator reproduce the committed golden
fixtures (tests/golden/make_golden.py) exactly.  CPU only."""
import os
import sys

import numpy as np
import pytest

import synth

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import make_golden  # noqa: E402

CASES = [("c0_tiny.npz", "c0_tiny", None),
         ("c1_20b_decode_first8.npz", "c1_20b_decode", np.arange(8))]


@pytest.mark.parametrize("fname,cfg,rows", CASES)
def test_golden(fname, cfg, rows):
    g = np.load(os.path.join(HERE, fname))
    d = synth.make_data(cfg)
    assert bytes(g["digest"]).decode() == make_golden.digest(d), "synthetic inputs changed"
    now = make_golden.golden(d, rows)
    for k in g.files:
        if k in now:
            assert np.array_equal(g[k], now[k]), f"{fname}:{k} differs"


def test_golden_routing_invariants():
    g = np.load(os.path.join(HERE, "c1_20b_decode_first8.npz"))
    ti = g["topk_i"]
    assert all(len(set(r)) == len(r) for r in ti)                      # distinct experts
    assert g["counts"].sum() == ti.size                                # every slot routed
    for e in range(len(g["counts"])):
        rows = g["row_token"][g["offsets"][e]:g["offsets"][e + 1]]
        assert np.all(np.diff(rows) > 0)                               # token-ascending
    w = synth.bf16_to_f32(g["topk_w"])
    assert np.allclose(w.sum(axis=1), 1.0, atol=2e-2)
    assert np.all(np.diff(w, axis=1) <= 0)                             # descending scores
