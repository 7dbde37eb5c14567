"""Pins the CPU oracle (oracle/moe_oracle.c) against things it does not
restate: closed forms, brute force, float64 arithmetic and the reference's
own tables.  CPU only.

The reference ships no golden vectors for the MoE path; its MXFP4 table and
nibble order are fixed by export_model_bin/gpt-oss-20b/export_model_bin.py:66-123
(FP4_VALUES, lut[low nibble] -> even element, ldexp by scale - 127) and
getp-csrc/memory/mxfp4.hpp:7-57 (same table, scale = bits e << 23).
"""
import numpy as np
import pytest
import torch

import oracle
import synth
from synth import bf16_to_f32, f32_to_bf16

# export_model_bin.py:66-83, written out independently of the oracle's table
FP4_VALUES = [+0.0, +0.5, +1.0, +1.5, +2.0, +3.0, +4.0, +6.0,
              -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def torch_bf16(a32):
    """Round-to-nearest-even fp32 -> bf16 by torch (independent of ours)."""
    return torch.from_numpy(np.asarray(a32, np.float32)).to(torch.bfloat16).view(
        torch.int16).numpy().view(np.uint16)


# ----------------------------------------------------------------- bf16 --
def test_f2bf_matches_torch_rounding():
    rng = np.random.default_rng(0)
    v = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 1e3,
        # exact halfway cases in both parities
        ((np.arange(1000, dtype=np.uint32) << 16) | 0x8000).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38], np.float32),
    ])
    ours = np.array([oracle.lib().orc_f2bf(float(x)) for x in v[:2000]], np.uint16)
    assert np.array_equal(ours, torch_bf16(v[:2000]))
    assert np.array_equal(f32_to_bf16(v), torch_bf16(v))
    nan = f32_to_bf16(np.array([np.nan], np.float32))
    assert np.isnan(bf16_to_f32(nan))[0]


# -------------------------------------------------------------- dequant --
def test_dequant_closed_form_all_codes_all_scales():
    codes = np.arange(256, dtype=np.uint8)           # every nibble pair
    packed = np.tile(codes, 256)
    scales = np.repeat(np.arange(256, dtype=np.uint8), 16)
    n = packed.size * 2
    got = oracle.dequant(packed, scales, n)
    # element i: byte i // 2, low nibble for even i; scale i // 32
    i = np.arange(n)
    nib = (packed[i // 2] >> (4 * (i & 1))) & 0xF
    e = scales[i // 32].astype(np.int64)
    val = np.array([FP4_VALUES[c] for c in nib], np.float64)
    mid = (e >= 1) & (e <= 254)
    # e in [1, 254]: the exporter's ldexp(lut, e - 127) (export_model_bin.py:95-121)
    with np.errstate(over="ignore"):  # 6 * 2^127 overflows to inf, as in fp32
        want_mid = torch_bf16(np.ldexp(val[mid], e[mid] - 127).astype(np.float32))
    assert np.array_equal(got[mid], want_mid)
    # e = 0: mxfp4.hpp:53 builds X from the bits (0 << 23) = +0.0, so code * 0.0
    z = e == 0
    assert np.array_equal(got[z], np.where(nib[z] >= 8, 0x8000, 0x0000).astype(np.uint16))
    # e = 255: X = +Inf: +-Inf, NaN for the two zero codes
    inf = e == 255
    gi = bf16_to_f32(got[inf])
    zc = (nib[inf] & 7) == 0
    assert np.isnan(gi[zc]).all()
    assert np.array_equal(gi[~zc], np.where(nib[inf][~zc] >= 8, -np.inf, np.inf))


def test_dequant_nibble_order():
    # byte 0x21: element 0 = code 1 (0.5), element 1 = code 2 (1.0); scale 127 -> X = 1
    packed = np.array([0x21, 0xF8] + [0] * 14, np.uint8)
    got = bf16_to_f32(oracle.dequant(packed, np.array([127], np.uint8), 32))
    assert list(got[:4]) == [0.5, 1.0, -0.0, -6.0]


# --------------------------------------------------------------- router --
def _router_f32_emulation(x, wr):
    """The pinned fp32 order written with numpy float32: 16 partials over
    k = 128 i + 8 l + j, then an xor butterfly.  bf16 x bf16 products are exact
    in fp32, so fmaf(a, b, acc) == float32(acc + a*b)."""
    xf, wf = bf16_to_f32(x), bf16_to_f32(wr)
    T, H = xf.shape
    E = wf.shape[0]
    prod = xf[:, None, :] * wf[None, :, :]       # exact, [T][E][H]
    p = np.zeros((T, E, 16), np.float32)
    for base in range(0, H, 128):
        for j in range(8):
            k = base + 8 * np.arange(16) + j
            ok = k < H
            add = np.zeros((T, E, 16), np.float32)
            add[:, :, ok] = prod[:, :, k[ok]]
            p = (p + add).astype(np.float32)
    lanes = np.arange(16)
    for s in (8, 4, 2, 1):
        p = (p + p[:, :, lanes ^ s]).astype(np.float32)
    return f32_to_bf16(p[:, :, 0])


@pytest.mark.parametrize("H,E", [(128, 4), (2880, 32)])
def test_router_logits(H, E):
    rng = np.random.default_rng(H + E)
    x = f32_to_bf16(rng.standard_normal((6, H)).astype(np.float32))
    wr = f32_to_bf16(rng.standard_normal((E, H)).astype(np.float32) * 0.02)
    got = oracle.router_logits(x, wr)
    # the pinned fp32 order, restated with numpy
    assert np.array_equal(got, _router_f32_emulation(x, wr))
    # and within one bf16 ulp of the float64 dot product
    exact = bf16_to_f32(x).astype(np.float64) @ bf16_to_f32(wr).astype(np.float64).T
    ulp = np.abs(exact) * 2.0 ** -7
    assert np.all(np.abs(bf16_to_f32(got) - exact) <= ulp + 1e-30)


# ---------------------------------------------------------------- top-k --
def _scores(logits, bias):
    return (bf16_to_f32(logits) + bf16_to_f32(bias)[None, :]).astype(np.float32)


@pytest.mark.parametrize("E,K", [(4, 2), (32, 4), (128, 4), (256, 8), (100, 3)])
def test_topk_brute_force(E, K):
    rng = np.random.default_rng(E * 10 + K)
    T = 64
    # coarse bf16 values make exact ties frequent
    logits = f32_to_bf16(np.round(rng.standard_normal((T, E)) * 4).astype(np.float32) / 4)
    bias = f32_to_bf16(np.round(rng.standard_normal(E) * 2).astype(np.float32) / 4)
    ti, tw = oracle.topk_softmax(logits, bias, K)
    s = _scores(logits, bias)
    for t in range(T):
        # distinct values here are >= 1/4 apart, so the eps rule reduces to
        # exact ties -> lower index: a sort by (-score, index)
        order = sorted(range(E), key=lambda i: (-s[t, i], i))[:K]
        assert list(ti[t]) == order
        sel = s[t, order].astype(np.float64)
        w = np.exp(sel - sel.max())
        w /= w.sum()
        assert np.all(np.abs(tw[t].astype(np.int32) - torch_bf16(w.astype(np.float32)).astype(
            np.int32)) <= 1)


def test_topk_epsilon_tie_rule():
    # scores 1.0 (index 0) and 1.0 + 2^-23 (index 1): within eps = 1e-6 relative,
    # so the lower index wins (moe.hpp:333-342); with a gap of 2^-19 it does not.
    logits = f32_to_bf16(np.array([[1.0, 1.0, -5.0, -5.0]], np.float32))
    for gap, first in ((2.0 ** -23, 0), (2.0 ** -19, 1)):
        bias = f32_to_bf16(np.array([0.0, gap, 0.0, 0.0], np.float32))
        ti, _ = oracle.topk_softmax(logits, bias, 2)
        assert ti[0, 0] == first and set(ti[0]) == {0, 1}


# ---------------------------------------------------------------- index --
def test_route_index_against_sort():
    rng = np.random.default_rng(4)
    T, K, E = 300, 4, 32
    ti = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
    tw = f32_to_bf16(rng.random((T, K)).astype(np.float32))
    r = oracle.route_index(ti, tw, E)
    flat_e = ti.ravel()
    flat_t = np.repeat(np.arange(T), K)
    order = np.lexsort((flat_t, flat_e))            # by expert, then token
    assert np.array_equal(r["counts"], np.bincount(flat_e, minlength=E))
    assert np.array_equal(r["offsets"], np.concatenate([[0], np.cumsum(r["counts"])]))
    assert np.array_equal(r["row_token"], flat_t[order])
    lid = np.empty(T * K, np.int64)
    lid[order] = np.arange(T * K)
    assert np.array_equal(r["local_ids"].ravel(), lid)
    assert r["dropped"] == 0


def test_route_index_drops_invalid_and_duplicate_slots():
    ti = np.array([[0, 0], [1, 5], [-1, 2]], np.int32)
    tw = f32_to_bf16(np.ones((3, 2), np.float32))
    r = oracle.route_index(ti, tw, 4)
    assert r["dropped"] == 3
    assert list(r["counts"]) == [1, 1, 1, 0]
    assert list(r["local_ids"].ravel()) == [0, -1, 1, -1, -1, 2]


# -------------------------------------------------------------- experts --
def _moe_float64(d, x, ti, tw):
    """The getp MoE restated with numpy float64 dot products and the same bf16
    rounding points (MLP1 out, SwiGLU out, MLP2 out, final)."""
    c = d.cfg
    H, D, E, K = c.hidden, c.intermediate, c.n_experts, c.top_k
    lut = np.array(FP4_VALUES)

    def deq(packed, scales, e, n):
        p = packed[e * n // 2:(e + 1) * n // 2]
        s = scales[e * n // 32:(e + 1) * n // 32].astype(np.int64)
        v = np.empty(n)
        v[0::2] = lut[p & 15]
        v[1::2] = lut[p >> 4]
        return np.ldexp(v, np.repeat(s, 32) - 127)

    bf = lambda a: bf16_to_f32(torch_bf16(np.asarray(a, np.float32))).astype(np.float64)
    xf = bf16_to_f32(x).astype(np.float64)
    b1, b2 = bf16_to_f32(d.b1).astype(np.float64), bf16_to_f32(d.b2).astype(np.float64)
    out = np.zeros((x.shape[0], H))
    for t in range(x.shape[0]):
        acc = np.float32(0)
        ys = []
        for j in range(K):
            e = ti[t, j]
            W1 = deq(d.w1, d.s1, e, 2 * D * H).reshape(2 * D, H)
            h = bf(W1 @ xf[t] + b1[e])
            g, u = np.clip(h[0::2], -7, 7), np.clip(h[1::2], -7, 7)
            a = bf(g / (1 + np.exp(-1.702 * g)) * (u + 1))
            W2 = deq(d.w2, d.s2, e, H * D).reshape(H, D)
            ys.append(bf(W2 @ a + b2[e]))
        w = bf16_to_f32(tw[t]).astype(np.float64)
        out[t] = sum(w[j] * ys[j] for j in range(K))
    return out


def test_moe_experts_against_float64_restatement():
    d = synth.make_data("c0_tiny")
    ti, tw = oracle.topk_softmax(oracle.router_logits(d.x, d.router_w), d.router_b, 2)
    got = bf16_to_f32(oracle.moe_experts(d, d.x, ti, tw)).astype(np.float64)
    want = _moe_float64(d, d.x, ti, tw)
    rel = np.abs(got - want) / np.maximum(np.abs(want), np.sqrt(np.mean(want ** 2)))
    # bf16 output rounding (2^-8) plus rare one-ulp flips of intermediates
    assert rel.max() < 2e-2, rel.max()
    assert np.median(rel) < 2e-3


def test_getp_and_cpu_engine_semantics_agree():
    """The CPU engine's fp32 path (run.cpp:657-748) and the getp path agree
    within the layer tolerance on the same weights."""
    from parity import compare
    d = synth.make_data("c0_tiny")
    eng = oracle.Fp32Engine(d)
    xf = bf16_to_f32(d.x)
    cpu = np.stack([eng.token(xf[t]) for t in range(d.cfg.tokens)])
    getp = oracle.moe_forward(d, forced=False)["e_agg"]
    m = compare(f32_to_bf16(cpu), getp)
    assert m["max_abs_norm"] <= 2e-2 and m["rel_l2"] <= 1e-2, m


def test_rmsnorm_against_float64():
    rng = np.random.default_rng(8)
    x = f32_to_bf16(rng.standard_normal((16, 2880)).astype(np.float32) * 5)
    w = f32_to_bf16(1 + 0.1 * rng.standard_normal(2880).astype(np.float32))
    got = bf16_to_f32(oracle.rmsnorm(x, w)).astype(np.float64)
    xf = bf16_to_f32(x).astype(np.float64)
    want = bf16_to_f32(w) * xf / np.sqrt(np.mean(xf ** 2, axis=1, keepdims=True) + 1e-5)
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -8 * 1.01 + 1e-30)


def test_residual_add():
    a = f32_to_bf16(np.array([1.0, 2.0, -3.0, 1e4], np.float32))
    b = f32_to_bf16(np.array([0.5, 2.0 ** -9, 3.0, 1.0], np.float32))
    got = bf16_to_f32(oracle.residual_add(a, b))
    big = float(bf16_to_f32(a)[3])  # bf16(1e4) = 9984; + 1 rounds back to it
    assert list(got) == [1.5, 2.0, 0.0, big]


# ------------------------------------------------------ MXFP4 quantiser --
E2M1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], np.float32)


def _unpack(packed, n):
    b = packed.astype(np.uint8)
    nib = np.empty(b.size * 2, np.uint8)
    nib[0::2] = b & 0xF
    nib[1::2] = b >> 4
    return nib[:n]


def _quant_inputs(seed):
    rng = np.random.default_rng(seed)
    parts = [rng.standard_normal(32 * 64).astype(np.float32) * np.float32(10.0) ** rng.integers(-3, 4, 32 * 64),
             (rng.integers(-24, 25, 32 * 16) * 0.25).astype(np.float32),      # ties at code midpoints
             np.zeros(32, np.float32),                                          # all-zero block
             np.ldexp(rng.standard_normal(32), -140).astype(np.float32),       # denormal block
             rng.standard_normal(45).astype(np.float32)]                       # ragged tail
    return np.concatenate(parts).astype(np.float32)


def test_quantize_scale_rule():
    """Scale byte = clip(floor(log2 max|v|) - 2 + 127, 0, 255), 127 for a zero
    block (numpy frexp restatement, mxfp4.hpp:183-193)."""
    v = _quant_inputs(1)
    packed, scales = oracle.quantize_mxfp4(v)
    nb = (v.size + 31) // 32
    vv = np.zeros(nb * 32, np.float32)
    vv[:v.size] = v
    m = np.abs(vv.reshape(nb, 32)).max(axis=1)
    _, e = np.frexp(m)
    want = np.where(m > 0, np.clip(e - 3 + 127, 0, 255), 127).astype(np.uint8)
    assert np.array_equal(scales, want)


def test_quantize_nearest_code_first_index_ties():
    """Each code is the first argmin of |v / 2^exp - E2M1[c]| (the reference's
    strict-< scan keeps the lower index on ties), NaN -> 0.  exp is the
    unclamped ilogb(max|v|) - 2: for a block of denormals it lies below -127,
    the stored scale byte clamps to 0, and the codes still use 2^exp (the
    reference's behaviour, mxfp4.hpp:188-201)."""
    v = _quant_inputs(2)
    v[5] = np.nan
    packed, scales = oracle.quantize_mxfp4(v)
    nb = scales.size
    vv = np.zeros(nb * 32, np.float32)
    vv[:v.size] = v
    m = np.nanmax(np.abs(vv.reshape(nb, 32)), axis=1)
    _, e = np.frexp(m)
    ex = np.where(m > 0, e - 3, 0)
    X = np.ldexp(np.float32(1), ex).astype(np.float32)
    x = (vv.reshape(nb, 32) / X[:, None]).reshape(-1)
    with np.errstate(invalid="ignore"):
        d = np.abs(x[:, None] - E2M1[None, :])
    d = np.where(np.isnan(d), np.inf, d)
    want = d.argmin(axis=1).astype(np.uint8)
    got = _unpack(packed, nb * 32)
    assert np.array_equal(got, want)
    assert got[5] == 0


def test_quantize_round_trip_exact():
    """Blocks built from E2M1 codes whose largest magnitude is 4 or 6 at a
    scale come back unchanged (-0 comes back as +0)."""
    rng = np.random.default_rng(3)
    nb = 200
    codes = rng.integers(0, 16, (nb, 32)).astype(np.uint8)
    codes[:, 0] = rng.choice([6, 7, 14, 15], nb)  # |4| or |6| in every block
    sc = rng.integers(100, 150, nb).astype(np.uint8)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8).reshape(-1)
    vals = oracle.dequant_f32(packed, sc, nb * 32)
    p2, s2 = oracle.quantize_mxfp4(vals)
    assert np.array_equal(s2, sc)
    want = np.where(codes.reshape(-1) == 8, 0, codes.reshape(-1))
    assert np.array_equal(_unpack(p2, nb * 32), want)
