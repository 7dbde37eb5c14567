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


# ------------------------------------------ MXFP8 activations (FP4 variant) --
# OCP FP8 e4m3 known answers (bias 7, no infinities, 0x7f NaN): 0x38 = 1.0,
# 0x7e = 448 (largest), 0x08 = 2^-6 (smallest normal), 0x01 = 2^-9.
def test_e4m3_known_values():
    t = oracle.e4m3_decode_table()
    assert t[0x38] == 1.0 and t[0x7E] == 448.0 and t[0x08] == 2.0 ** -6 and t[0x01] == 2.0 ** -9
    assert t[0xB8] == -1.0 and t[0x00] == 0.0 and np.signbit(t[0x80])
    pos = t[:0x7F]
    assert np.all(np.diff(pos) > 0)  # codes 0..126 ascend


def _e4m3_nearest_even(v):
    """Brute force: the nearest of the 127 non-negative e4m3 values, ties to
    the even code (last mantissa bit 0), sign applied after."""
    t = oracle.e4m3_decode_table()[:0x7F].astype(np.float64)
    a = np.abs(v.astype(np.float64))[:, None]
    d = np.abs(t[None, :] - a)
    best = d.min(axis=1, keepdims=True)
    cand = d == best
    code = np.where(cand.sum(1) > 1, np.argmax(cand & (np.arange(127) % 2 == 0)[None, :], 1),
                    np.argmax(cand, 1)).astype(np.uint8)
    return code | np.where(np.signbit(v), 0x80, 0).astype(np.uint8)


def _qa_pos(k):
    """Byte of k within a row: 1 KB per 512-k stage, the MFMA A-operand order."""
    j, kk = k // 512, k % 512
    kp, kin = kk // 128, kk % 128
    return j * 1024 + kp * 128 + 32 * ((kin % 64) // 16) + 16 * (kin // 64) + kin % 16


def test_quantize_act_rounding_brute_force():
    """Groups whose max is in [128, 256) have e = 0, so hi codes are e4m3_rne(x)
    itself: checked against the brute-force nearest-even code, including every
    tie between neighbouring codes."""
    rng = np.random.default_rng(3)
    t = oracle.e4m3_decode_table()[:0x7E].astype(np.float64)
    mids = (t[:-1] + t[1:]) / 2
    vals = np.concatenate([mids, rng.uniform(-250, 250, 4000), rng.uniform(-0.02, 0.02, 1000)])
    vals = bf16_to_f32(f32_to_bf16(vals.astype(np.float32)))
    vals = vals[np.abs(vals) < 255]
    n = vals.size // 31 * 31
    blocks = vals[:n].reshape(-1, 31)
    x = np.concatenate([np.full((blocks.shape[0], 1), 255.0, np.float32), blocks], 1).reshape(1, -1)
    K = x.shape[1] // 64 * 64
    x = f32_to_bf16(x[:, :K])
    q, s = oracle.quantize_act(x, 1)
    xf = bf16_to_f32(x)[0]
    got = q[0, _qa_pos(np.arange(K))]
    assert np.array_equal(got, _e4m3_nearest_even(xf))
    assert np.all(s[0, :] [np.arange(0, s.shape[1], 32)] == 127)


def test_quantize_act_scale_rule_and_layout():
    """Scale e = floor(log2 max|x|) - 7 (hi byte e + 127, lo e + 123), 0 for
    an all-zero group, clamped at -123; group b's byte sits at 4 (b % 4) +
    (b % 16) // 4 of its stage; codes follow the stated byte order."""
    K = 1024
    amax = [1.0, 3.0, 0.0, 2.0 ** -130, 1000.0, 2.0 ** 100] + [0.5] * 26
    x = np.zeros((1, K), np.float32)
    for b, a in enumerate(amax):
        x[0, 32 * b + (b % 32)] = a
    x = f32_to_bf16(x)
    q, s = oracle.quantize_act(x, 2)
    for b, a in enumerate(amax):
        if a == 0.0:
            e = 0
        else:
            ab = float(bf16_to_f32(f32_to_bf16(np.array([a], np.float32)))[0])
            e = max(int(np.floor(np.log2(ab))) - 7, -123)
        j, bs = b // 16, b % 16
        at = j * 32 + 4 * (bs % 4) + bs // 4
        assert s[0, at] == e + 127 and s[0, at + 16] == e + 123, (b, a)
    # the only nonzero hi code of group b is at k = 32 b + b % 32
    hi = q[0].reshape(-1, 2, 512)[:, 0, :].reshape(-1)
    nz = [int(i // 512) * 1024 + int(i % 512) for i in np.nonzero(hi)[0]]
    want = sorted(_qa_pos(32 * b + (b % 32)) for b, a in enumerate(amax) if a != 0.0)
    assert sorted(nz) == want


def test_quantize_act_two_terms_error_bound():
    """hi + lo reproduces x to within 2^-9 of its group's max scale 2^(e+7)
    (the rounding of lo), and exactly when x has at most 7 significant bits."""
    rng = np.random.default_rng(4)
    v = rng.standard_normal((8, 2880)) * np.exp2(rng.integers(-20, 21, (8, 1)) + rng.standard_normal((8, 2880)) * 2)
    x = f32_to_bf16(v.astype(np.float32))
    q, s = oracle.quantize_act(x, 2)
    y = oracle.dequant_act(q, s, 2880).astype(np.float64)
    xf = bf16_to_f32(x).astype(np.float64)
    g = np.abs(xf).reshape(8, -1, 32).max(2)
    lim = np.repeat(np.exp2(np.floor(np.log2(np.maximum(g, 1e-300)))), 32, axis=1) * 2.0 ** -9
    assert np.all(np.abs(y - xf) <= lim)
    x7 = f32_to_bf16((np.round(rng.uniform(-127, 127, (4, 512))) * 2.0 ** -3).astype(np.float32))
    q7, s7 = oracle.quantize_act(x7, 2)
    assert np.array_equal(oracle.dequant_act(q7, s7, 512), bf16_to_f32(x7))


def test_moe_forward_act_quant_two_terms_close_to_bf16():
    """The variant's expected output with two terms stays within the layer
    tolerance of the bf16 path's (the oracle, not the GPU)."""
    from parity import compare
    d = synth.make_data("c0_tiny")
    a = oracle.moe_forward(d, forced=False)["e_agg"]
    b = oracle.moe_forward(d, forced=False, act_quant=2)["e_agg"]
    m = compare(b, a)
    assert m["rel_l2"] < 1e-3, m


# ------------------------------------------ router order vs exact scores --
@pytest.mark.parametrize("cfg", ["c1_20b_decode", "c3a_120b_decode", "c3b_120b_prefill"])
def test_router_selection_vs_exact_scores(cfg):
    """The pinned-order router (bf16 logits, then the reference's top-k)
    against top-k on float64-exact scores over the benchmark inputs: the
    expert sets may differ only where the float64 scores of the swapped
    experts lie within one bf16 ulp of the logits (the reference's own bf16
    logits cannot order them either).  Records how many tokens differ."""
    import synth
    x, wr, br = synth.make_router_inputs(cfg)
    K = synth.CONFIGS[cfg].top_k
    logits = oracle.router_logits(x, wr)
    ti, _ = oracle.topk_softmax(logits, br, K)
    exact = synth.router_scores_f64(x, wr, br)
    logit64 = exact - bf16_to_f32(br).astype(np.float64)[None, :]
    order = np.argsort(-exact, axis=1, kind="stable")[:, :K]
    n_diff = 0
    for t in range(x.shape[0]):
        a, b = set(ti[t].tolist()), set(order[t].tolist())
        if a == b:
            continue
        n_diff += 1
        # every swapped expert scores within one bf16 ulp (of the larger of
        # its logit and the K-th expert's) of the exact K-th score
        k_e = order[t, K - 1]
        kth = exact[t, k_e]
        for e in a ^ b:
            mag = max(abs(logit64[t, e]), abs(logit64[t, k_e]), 1e-30)
            ulp = 2.0 ** (np.floor(np.log2(mag)) - 7)
            assert abs(exact[t, e] - kth) <= ulp, (cfg, t, sorted(a), sorted(b), e)
    # near-ties are rare: a small fraction of tokens
    assert n_diff <= max(2, x.shape[0] // 50), (cfg, n_diff)
    print(f"{cfg}: {n_diff} of {x.shape[0]} tokens select a different expert set than exact scores")
