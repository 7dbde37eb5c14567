"""GPU parity of the per-expert tile switch (GPTOSS_MOE_FLAG_TILE_SWITCH,
path "switch"): experts of 128 rows or more run on the large-M GEMM's
128-row tiles reading the packed weights, the others on the streamed GEMM,
in one forward call.  Against the oracle at the layer tolerance, on
configurations whose experts fall on both sides of the switch; where no
expert reaches it (or the shape is below the large-M GEMM's 256 minimum)
the call is bit-identical to the default path.  Collected after the other
GPU tests: this path has not run on a GPU yet."""
import numpy as np
import pytest

import oracle
import synth
from parity import assert_close

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("gpu")]


def _run(name, path, rows=None, tokens=None):
    import torch
    import gptoss_moe
    d = synth.make_data(name, tokens=tokens)
    layer = gptoss_moe.MoeLayer.from_numpy(d, device="cuda:0")
    layer.drop_unpacked()  # the switch reads only the packed copy
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16 if a.dtype == np.uint16 else a.dtype)).to("cuda:0")
    x = dev(d.x)
    fi = None if d.forced_i is None else dev(d.forced_i)
    fw = None if d.forced_w is None else dev(d.forced_w)
    out = layer.forward(x, forced_i=fi, forced_w=fw, path=path)
    torch.cuda.synchronize()
    counts = layer.views(d.cfg.tokens)["counts"]
    return d, out.cpu().numpy().view(np.uint16), counts


@pytest.mark.parametrize("name", ["t_large_m", "c2_20b_zipf"])
def test_switch_matches_oracle(name):
    d, got, counts = _run(name, "switch")
    assert (counts >= 128).any() and (counts < 128).any(), counts   # both GEMMs take part
    ref = oracle.moe_forward(d, forced=d.forced_i is not None)
    assert_close(got, ref["e_agg"], f"tile switch {name}")


def test_switch_prefill_sampled():
    """c3b (120B, 4096 tokens): 256 sampled rows against the oracle."""
    d, got, counts = _run("c3b_120b_prefill", "switch")
    assert (counts >= 128).any()
    rows = np.random.default_rng(5).choice(d.cfg.tokens, 256, replace=False)
    ref = oracle.moe_forward(d, forced=d.forced_i is not None, rows=rows)
    assert_close(got[rows], ref["e_agg"], "tile switch c3b (256 sampled rows)")


@pytest.mark.parametrize("name", ["c0_tiny", "c1_20b_decode"])
def test_switch_inactive_is_the_default(name):
    """c0: below the large-M GEMM's shape minimum; c1: no expert reaches 128
    rows.  The call is the default path, bit for bit."""
    _, a, counts = _run(name, "switch")
    _, b, _ = _run(name, "auto")
    assert np.array_equal(a, b)
