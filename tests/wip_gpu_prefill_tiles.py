"""GPU parity of 128-row tiles on the streamed GEMM
(GPTOSS_MOE_FLAG_PREFILL_TILES, path "prefill").  Every output row meets the
same MFMAs in the same k order as with the default 64-row tiles (a tile only
holds more row groups), so the call must be bit-identical to the default
path: on tiles of 1-128 rows (c2's Zipf counts, t_large_m's 300-row experts
cut into 128-row tiles and a remainder), at decode (c1: one tile per expert
below 64 rows) and at prefill (c3b), plus the oracle at c3b on sampled rows.
Collected after the other GPU tests: this kernel has not run on a GPU yet."""
import numpy as np
import pytest

import oracle
from parity import assert_close
from wip_gpu_tile_switch import _run

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("gpu")]


@pytest.mark.parametrize("name", ["c0_tiny", "c1_20b_decode", "c2_20b_zipf", "t_large_m"])
def test_prefill_tiles_bit_identical(name):
    _, a, counts = _run(name, "prefill")
    _, b, _ = _run(name, "auto")
    assert np.array_equal(a, b), (name, int((a != b).sum()))


def test_prefill_tiles_c3b_sampled():
    d, got, counts = _run("c3b_120b_prefill", "prefill")
    _, want_default, _ = _run("c3b_120b_prefill", "auto")
    assert np.array_equal(got, want_default)
    rows = np.random.default_rng(7).choice(d.cfg.tokens, 256, replace=False)
    ref = oracle.moe_forward(d, forced=d.forced_i is not None, rows=rows)
    assert_close(got[rows], ref["e_agg"], "128-row tiles c3b (256 sampled rows)")
