"""GPU parity of the streamed GEMM's prefetching consumers
(GPTOSS_MOE_FLAG_STAGE_PREFETCH, path "prefetch"; with
GPTOSS_MOE_FLAG_WIDE_CONSUMERS, 4 column tiles per wave, paths "wide" on
64-row and "wide_prefill" on 128-row tiles).  The consumers run the same
MFMAs in the same k order as the default ones (only the LDS reads move
earlier, and a wave owns more column tiles), so the call must be
bit-identical to the default path: at every
tile height 1-64 rows (c2's Zipf counts, t_odd_n's 5 experts, c1's ~32-row
experts), with a 64-k last stage (K = 2880) and without one (c0, K = 128;
t_large_m, K = 384 and 320), plus the oracle at c1 and c2.
Kept uncollected until it has passed on a GPU once."""
import numpy as np
import pytest

import oracle
from parity import assert_close
from wip_gpu_tile_switch import _run

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("gpu")]


@pytest.mark.parametrize("path", ["prefetch", "wide", "wide_prefill", "wpf", "wide_wpf"])
@pytest.mark.parametrize("name", ["c0_tiny", "t_odd_n", "t_large_m", "c1_20b_decode", "c2_20b_zipf",
                                  "c3a_120b_decode"])
def test_prefetch_bit_identical(name, path):
    print(f"{path} vs default: {name}", flush=True)
    _, a, _ = _run(name, path)
    _, b, _ = _run(name, "auto")
    assert np.array_equal(a, b), (name, int((a != b).sum()))


@pytest.mark.parametrize("path", ["prefetch", "wide"])
@pytest.mark.parametrize("name", ["c1_20b_decode", "c2_20b_zipf"])
def test_prefetch_matches_oracle(name, path):
    print(f"{path} vs oracle: {name}", flush=True)
    d, got, _ = _run(name, path)
    ref = oracle.moe_forward(d, forced=d.forced_i is not None)
    assert_close(got, ref["e_agg"], f"{path} {name}")


def test_wide_prefill_c3b_sampled():
    print("wide_prefill vs default and oracle: c3b", flush=True)
    d, got, _ = _run("c3b_120b_prefill", "wide_prefill")
    _, want_default, _ = _run("c3b_120b_prefill", "auto")
    assert np.array_equal(got, want_default)
    rows = np.random.default_rng(11).choice(d.cfg.tokens, 256, replace=False)
    ref = oracle.moe_forward(d, forced=d.forced_i is not None, rows=rows)
    assert_close(got[rows], ref["e_agg"], "wide consumers, 128-row tiles, c3b (256 sampled rows)")
