"""Parity of the HIP path (through the C ABI) against the CPU oracle.

Bit-exact: MXFP4 dequantisation, router logits (pinned fp32 order), top-k
indices, per-expert counts, offsets and the compact row map.  Within
tolerance: router weights (1 bf16 ulp: device expf vs libm expf) and layer
outputs (tests/parity.py).
"""
import numpy as np
import pytest

import oracle
import synth
from packing import pack_expected
from parity import assert_close, compare

pytestmark = pytest.mark.gpu


def _dev(a, device):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to(device)


def _host16(t):
    return t.cpu().numpy().view(np.uint16)


_CACHE = {}


def _data(name, tokens=None):
    key = (name, tokens)
    if key not in _CACHE:
        _CACHE.clear()
        _CACHE[key] = synth.make_data(name, tokens=tokens)
    return _CACHE[key]


# ---------------------------------------------------------------- dequant --
def test_dequant_all_codes_all_scales(gpu):
    import gptoss_moe
    # every byte value (two nibbles) under every e8m0 scale
    packed = np.tile(np.arange(256, dtype=np.uint8), 256)      # 65536 B = 131072 elements
    scales = np.repeat(np.arange(256, dtype=np.uint8), 16)     # one scale per 32 elements
    n = packed.size * 2
    got = _host16(gptoss_moe.dequant_mxfp4(_dev(packed, gpu), _dev(scales, gpu), 1, 1, n))[0]
    want = oracle.dequant(packed, scales, n)
    gf, wf = synth.bf16_to_f32(got), synth.bf16_to_f32(want)
    both_nan = np.isnan(gf) & np.isnan(wf)
    bad = (got != want) & ~both_nan
    if bad.any():
        i = np.flatnonzero(bad)[:8]
        detail = [(int(k), int(scales[k // 32]), int((packed[k // 2] >> (4 * (k & 1))) & 15),
                   hex(got[k]), hex(want[k])) for k in i]
        pytest.fail(f"{bad.sum()} dequant mismatches (elem, e8m0, code, got, want): {detail}")


@pytest.mark.parametrize("e_range", [(120, 129), (1, 255)])
def test_dequant_expert_segment(gpu, e_range):
    import gptoss_moe
    rng = np.random.default_rng(7)
    E, N, K = 2, 5760, 2880
    packed = rng.integers(0, 256, E * N * K // 2, dtype=np.uint8)
    scales = rng.integers(e_range[0], e_range[1], E * N * K // 32, dtype=np.uint8)
    got = _host16(gptoss_moe.dequant_mxfp4(_dev(packed, gpu), _dev(scales, gpu), E, N, K))
    for e in range(E):
        want = oracle.dequant(packed[e * N * K // 2:(e + 1) * N * K // 2],
                              scales[e * N * K // 32:(e + 1) * N * K // 32], N * K)
        assert np.array_equal(got[e], want), f"expert {e}: {(got[e] != want).sum()} mismatches"


def test_dequant_odd_tail(gpu):
    import gptoss_moe
    rng = np.random.default_rng(3)
    n = 1000 * 7 + 3  # not a multiple of 8, odd element count
    packed = rng.integers(0, 256, (n + 1) // 2, dtype=np.uint8)
    scales = rng.integers(118, 131, (n + 31) // 32, dtype=np.uint8)
    got = _host16(gptoss_moe.dequant_mxfp4(_dev(packed, gpu), _dev(scales, gpu), 1, 1, n))[0]
    assert np.array_equal(got, oracle.dequant(packed, scales, n))


# ---------------------------------------------------------------- routing --
ROUTE_CASES = ["c0_tiny", "c1_20b_decode", "c2_20b_zipf", "c3a_120b_decode"]


@pytest.mark.parametrize("name", ROUTE_CASES)
def test_routing_bit_exact(gpu, name):
    import gptoss_moe
    d = _data(name)
    c = d.cfg
    layer = gptoss_moe.MoeLayer.from_numpy(d, device=gpu)
    x = _dev(d.x, gpu)
    fi = None if d.forced_i is None else _dev(d.forced_i, gpu)
    fw = None if d.forced_w is None else _dev(d.forced_w, gpu)
    layer.route(x, fi, fw)
    v = layer.views(c.tokens)
    if d.forced_i is None:
        lg = oracle.router_logits(d.x, d.router_w)
        assert np.array_equal(v["logits"], lg), f"logits: {(v['logits'] != lg).sum()} differ"
        ti, tw = oracle.topk_softmax(lg, d.router_b, c.top_k)
    else:
        ti, tw = d.forced_i, d.forced_w
    assert np.array_equal(v["topk_i"], ti), f"topk_i: {(v['topk_i'] != ti).sum()} differ"
    ulps = np.abs(v["topk_w"].astype(np.int32) - tw.astype(np.int32))
    assert ulps.max() <= 1, f"topk_w off by {ulps.max()} ulp"
    ref = oracle.route_index(ti, v["topk_w"], c.n_experts)
    for k in ("counts", "offsets", "local_ids", "row_token", "row_weight"):
        assert np.array_equal(v[k], ref[k]), f"{k} differs"
    assert int(v["status"][0]) == ref["dropped"] == 0


def test_routing_invalid_and_duplicate_slots(gpu):
    import gptoss_moe
    d = _data("c0_tiny")
    c = d.cfg
    layer = gptoss_moe.MoeLayer.from_numpy(d, device=gpu)
    fi = np.array([[0, 1], [1, 1], [3, -1], [2, 7], [0, 3], [3, 0], [2, 2], [1, 0]], np.int32)
    fw = synth.f32_to_bf16(np.full((c.tokens, c.top_k), 0.5, np.float32))
    layer.route(_dev(d.x, gpu), _dev(fi, gpu), _dev(fw, gpu))
    v = layer.views(c.tokens)
    ref = oracle.route_index(fi, fw, c.n_experts)
    for k in ("counts", "offsets", "local_ids", "row_token", "row_weight"):
        assert np.array_equal(v[k], ref[k]), f"{k} differs"
    assert int(v["status"][0]) == ref["dropped"] == 4


# ---------------------------------------------------------------- forward --
def _forward(d, gpu, rows_check=None, residual=False, path="auto", pack=True):
    import gptoss_moe
    c = d.cfg
    layer = gptoss_moe.MoeLayer.from_numpy(d, device=gpu, pack=pack)
    x = _dev(d.x, gpu)
    fi = None if d.forced_i is None else _dev(d.forced_i, gpu)
    fw = None if d.forced_w is None else _dev(d.forced_w, gpu)
    out = layer.forward(x, forced_i=fi, forced_w=fw, path=path)
    got = _host16(out)
    ref = oracle.moe_forward(d, forced=d.forced_i is not None, rows=rows_check)
    sel = slice(None) if rows_check is None else rows_check
    m = assert_close(got[sel], ref["e_agg"], c.name)
    return layer, got, ref, m


@pytest.mark.parametrize("name", ["c0_tiny", "c1_20b_decode", "c2_20b_zipf"])
def test_forward_matches_oracle(gpu, name):
    d = _data(name)
    _, _, _, m = _forward(d, gpu)
    print(name, m)


def test_forward_120b_decode(gpu):
    d = _data("c3a_120b_decode")
    _, _, _, m = _forward(d, gpu)
    print(m)


@pytest.mark.parametrize("name,path", [("t_large_m", "auto"), ("t_large_m", "small"),
                                       ("c1_20b_decode", "large"), ("c2_20b_zipf", "large")])
def test_forward_gemm_paths(gpu, name, path):
    """Both grouped-GEMM paths against the oracle: the large-M path on ragged
    128-row tiles (t_large_m), on small experts (c1) and on skewed routing with
    multi-tile experts (c2); the small-M path where large-M would run."""
    d = _data(name)
    _, _, _, m = _forward(d, gpu, path=path)
    print(name, path, m)


@pytest.mark.parametrize("name", ["c0_tiny", "t_large_m", "t_odd_n", "c1_20b_decode"])
def test_forward_small_m_unpacked(gpu, name):
    """The LDS-staged small-M GEMM on the original weight layout (no packed copy)."""
    d = _data(name)
    _, _, _, m = _forward(d, gpu, path="small", pack=False)
    print(name, m)


@pytest.mark.parametrize("name", ["t_odd_n", "t_large_m"])
def test_forward_direct_ragged(gpu, name):
    """The direct GEMM on packed weights where N is not a multiple of the
    256-row weight block and K not a multiple of the 256-k stage, and (t_large_m)
    experts of several 64-row tiles."""
    d = _data(name)
    _, _, _, m = _forward(d, gpu)
    print(name, m)


@pytest.mark.parametrize("name", ["c0_tiny", "t_odd_n"])
def test_pack_layout_bit_exact(gpu, name):
    """gptoss_moe_pack_weights moves bytes only: its output equals a numpy
    permutation of the MXFP4 nibbles and scales, with zero padding past K."""
    import gptoss_moe
    d = _data(name)
    c = d.cfg
    layer = gptoss_moe.MoeLayer.from_numpy(d, device=gpu)
    got = layer.tensors["packed"].cpu().numpy()
    H, D = c.hidden, c.intermediate
    o = 0
    for wq, ws, n, k, mlp1 in ((d.w1, d.s1, 2 * D, H, True), (d.w2, d.s2, H, D, False)):
        ew, es = pack_expected(np.ascontiguousarray(wq).reshape(-1),
                                np.ascontiguousarray(ws).reshape(-1), n, k, mlp1)
        assert np.array_equal(got[o:o + ew.size], ew), "nibbles"
        o = -(-(o + ew.size) // 256) * 256
        assert np.array_equal(got[o:o + es.size], es), "scales"
        o = -(-(o + es.size) // 256) * 256
    assert o == got.size


def test_forward_120b_prefill_sampled(gpu):
    d = _data("c3b_120b_prefill")
    rows = np.random.default_rng(11).choice(d.cfg.tokens, 256, replace=False)
    rows.sort()
    _, _, _, m = _forward(d, gpu, rows_check=rows)
    print(m)


def test_reduction_bit_exact_given_slots(gpu):
    """The weighted k-way reduction reproduces the oracle's fmaf order on the
    MLP2 rows the GPU produced."""
    d = _data("c1_20b_decode")
    layer, got, _, _ = _forward(d, gpu)
    v = layer.views(d.cfg.tokens)
    T, K, H = d.cfg.tokens, d.cfg.top_k, d.cfg.hidden
    w = synth.bf16_to_f32(v["topk_w"])
    y = synth.bf16_to_f32(v["slots"])
    acc = np.zeros((T, H), np.float32)
    for j in range(K):
        live = (v["local_ids"][:, j] >= 0)[:, None]
        # w*y is exact in fp32 for bf16 operands, so fmaf == one rounding of acc + w*y
        acc = np.where(live, (acc + w[:, j:j + 1] * y[:, j, :]).astype(np.float32), acc)
    assert np.array_equal(got, synth.f32_to_bf16(acc))


def test_act_matches_oracle(gpu):
    """SwiGLU output rows (MLP2 input) against the oracle's."""
    d = _data("c1_20b_decode")
    layer, _, ref, _ = _forward(d, gpu)
    v = layer.views(d.cfg.tokens)
    _, act = oracle.moe_experts(d, d.x, v["topk_i"], v["topk_w"], want_act=True)
    m = compare(v["act"], act)
    assert m["rel_l2"] <= 1e-2 and m["frac_exact"] > 0.99, m


def test_forward_repeatable_and_residual(gpu):
    import torch
    import gptoss_moe
    d = _data("c1_20b_decode")
    layer = gptoss_moe.MoeLayer.from_numpy(d, device=gpu)
    x = _dev(d.x, gpu)
    a = layer.forward(x).clone()
    b = layer.forward(x).clone()
    # the k-way reduction has a fixed order: repeated calls are bit-identical
    assert np.array_equal(_host16(a), _host16(b))
    base = _dev(synth.f32_to_bf16(np.random.default_rng(5).standard_normal(
        d.x.shape).astype(np.float32)), gpu)
    y = base.clone()
    layer.forward(x, out=y, residual=True)
    want = oracle.residual_add(_host16(base), _host16(a))
    assert np.array_equal(_host16(y), want)
    torch.cuda.synchronize()


@pytest.mark.parametrize("path", ["auto", "small"])
def test_forward_sequence_of_batch_sizes(gpu, path):
    """One workspace, batches of changing size in a row: the routing
    histogram is cleared by each call for the next (more than one histogram
    block at 1000 tokens; the LDS-staged path also gathers with several
    workgroups per block)."""
    import gptoss_moe
    d = synth.make_data("c1_20b_decode", tokens=1000)
    c = d.cfg
    layer = gptoss_moe.MoeLayer.from_numpy(d, device=gpu)
    x = _dev(d.x, gpu)
    for n in (1000, 17, 300, 1000, 64):
        out = layer.forward(x[:n], path=path)
        v = layer.views(n)
        lg = oracle.router_logits(d.x[:n], d.router_w)
        ti, _ = oracle.topk_softmax(lg, d.router_b, c.top_k)
        assert np.array_equal(v["topk_i"], ti), f"{n} tokens: topk_i differs"
        ref = oracle.route_index(ti, v["topk_w"], c.n_experts)
        for k in ("counts", "offsets", "local_ids", "row_token", "row_weight"):
            assert np.array_equal(v[k], ref[k]), f"{n} tokens: {k} differs"
    rows = np.arange(0, 64, 5)  # the last call's tokens are rows 0..63 of d.x
    ref = oracle.moe_forward(d, forced=False, rows=rows)
    assert_close(_host16(out)[rows], ref["e_agg"], "c1 64 tokens after a sequence")


@pytest.mark.parametrize("tokens", [1, 3, 17])
def test_forward_small_batches(gpu, tokens):
    d = synth.make_data("c1_20b_decode", tokens=tokens)
    _forward(d, gpu)


def test_forward_one_hot_expert(gpu):
    """All tokens on the same experts: counts > 64 -> several M tiles, and
    empty experts."""
    d = synth.make_data("c1_20b_decode", tokens=200)
    c = d.cfg
    d.forced_i = np.tile(np.array([[5, 9, 1, 30]], np.int32), (c.tokens, 1))
    d.forced_w = synth.f32_to_bf16(np.tile(np.array([[0.4, 0.3, 0.2, 0.1]], np.float32),
                                           (c.tokens, 1)))
    _forward(d, gpu)


def test_rmsnorm_bit_exact(gpu):
    import gptoss_moe
    rng = np.random.default_rng(2)
    x = synth.f32_to_bf16(rng.standard_normal((64, 2880)).astype(np.float32) * 3)
    w = synth.f32_to_bf16(1 + 0.1 * rng.standard_normal(2880).astype(np.float32))
    got = _host16(gptoss_moe.rmsnorm(_dev(x, gpu), _dev(w, gpu)))
    assert np.array_equal(got, oracle.rmsnorm(x, w))


@pytest.mark.parametrize("name", ["c1_20b_decode", "c0_tiny", "c3a_120b_decode"])
def test_layer_matches_oracle(gpu, name):
    """moe_gpu at TP = 1: RMSNorm -> MoE -> residual add, in place."""
    import torch
    import gptoss_moe
    d = _data(name)
    rng = np.random.default_rng(9)
    rms_w = synth.f32_to_bf16(1 + 0.1 * rng.standard_normal(d.cfg.hidden).astype(np.float32))
    layer = gptoss_moe.MoeLayer.from_numpy(d, device=gpu)
    x = _dev(d.x, gpu)
    t_scratch = torch.empty_like(x)
    layer.layer(x, _dev(rms_w, gpu), t_scratch=t_scratch)
    t = oracle.rmsnorm(d.x, rms_w)
    # the RMSNorm fused into the router kernel is bit-exact
    assert np.array_equal(_host16(t_scratch), t)
    e = oracle.moe_forward(d, x_norm=t, forced=False)["e_agg"]
    want = oracle.residual_add(d.x, e)
    assert_close(_host16(x), want, "layer")


def test_layer_prefill_sampled(gpu):
    """The layer at 4096 tokens (8 tokens per router workgroup): the fused
    RMSNorm bit-exact on every row, the output on sampled rows."""
    import torch
    import gptoss_moe
    d = _data("c3b_120b_prefill")
    rng = np.random.default_rng(10)
    rms_w = synth.f32_to_bf16(1 + 0.1 * rng.standard_normal(d.cfg.hidden).astype(np.float32))
    layer = gptoss_moe.MoeLayer.from_numpy(d, device=gpu)
    x = _dev(d.x, gpu)
    t_scratch = torch.empty_like(x)
    layer.layer(x, _dev(rms_w, gpu), t_scratch=t_scratch)
    t = oracle.rmsnorm(d.x, rms_w)
    assert np.array_equal(_host16(t_scratch), t)
    rows = np.sort(rng.choice(d.cfg.tokens, 128, replace=False))
    e = oracle.moe_forward(d, x_norm=t, forced=False, rows=rows)["e_agg"]
    assert_close(_host16(x)[rows], oracle.residual_add(d.x[rows], e), "layer c3b")


def test_zero_tokens_is_noop(gpu):
    import torch
    import gptoss_moe
    d = _data("c0_tiny")
    layer = gptoss_moe.MoeLayer.from_numpy(d, device=gpu)
    x = torch.empty((0, d.cfg.hidden), dtype=torch.int16, device=gpu)
    layer.forward(x)


# ------------------------------------------------------ MXFP4 quantiser --
def _quant_case(seed):
    rng = np.random.default_rng(seed)
    return np.concatenate([
        rng.standard_normal(32 * 4096).astype(np.float32) * np.float32(10.0) ** rng.integers(-3, 4, 32 * 4096),
        (rng.integers(-24, 25, 32 * 512) * 0.25).astype(np.float32) * np.float32(2.0) ** rng.integers(-4, 5, 32 * 512),
        np.zeros(64, np.float32),
        np.ldexp(rng.standard_normal(64), -140).astype(np.float32),
        np.array([np.nan, 1.0, -np.nan, 3.0] * 8, np.float32),
        rng.standard_normal(77).astype(np.float32)]).astype(np.float32)


@pytest.mark.parametrize("seed", [0, 1])
def test_quantize_mxfp4_bit_exact(gpu, seed):
    """gptoss_moe_quantize_mxfp4 against the oracle byte for byte: magnitudes
    1e-3..1e3, exact ties at code midpoints, zero and denormal blocks, NaN, a
    ragged tail."""
    import torch
    import gptoss_moe
    v = _quant_case(seed)
    p, s = gptoss_moe.quantize_mxfp4(torch.from_numpy(v).to(gpu))
    wp, ws = oracle.quantize_mxfp4(v)
    assert np.array_equal(s.cpu().numpy(), ws)
    assert np.array_equal(p.cpu().numpy(), wp)


def test_quantize_mxfp4_round_trip_gpu(gpu):
    """Quantise on the GPU, dequantise with the GEMMs' conversion: the result is
    the oracle's dequantisation of the oracle's quantisation, bit for bit."""
    import torch
    import gptoss_moe
    v = _quant_case(7)[:32 * 4096]
    p, s = gptoss_moe.quantize_mxfp4(torch.from_numpy(v).to(gpu))
    got = _host16(gptoss_moe.dequant_mxfp4(p, s, 1, 1, v.size))
    wp, ws = oracle.quantize_mxfp4(v)
    assert np.array_equal(got.reshape(-1), oracle.dequant(wp, ws, v.size).reshape(-1))


def test_quantize_mxfp4_infinities(gpu):
    """A block holding +-Inf: frexp of Inf gives exponent 0 in the C library,
    so the scale is 2^-3; Inf itself becomes code 0 (every distance is
    infinite) and the block's finite values saturate to +-6.  The device
    library must agree byte for byte."""
    import torch
    import gptoss_moe
    v = np.array([np.inf, -np.inf, 1.0, -1.0, 100.0] + [0.5] * 27 + [2.0] * 32, np.float32)
    p, s = gptoss_moe.quantize_mxfp4(torch.from_numpy(v).to(gpu))
    wp, ws = oracle.quantize_mxfp4(v)
    assert np.array_equal(s.cpu().numpy(), ws)
    assert np.array_equal(p.cpu().numpy(), wp)
