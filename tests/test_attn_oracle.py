"""Pins the decode-attention oracle (oracle/attn_oracle.c) against things it
does not restate: numpy's fp16 rounding, closed forms of the quantiser and of
softmax attention, a float64 textbook attention over the token history
(independent of the cache's ring addressing), and brute force for the
reference GPU kernel's dropped-token rule.  CPU only."""
import numpy as np
import pytest

import oracle
from attn_cases import HD, KV, N_HEADS, N_KV, make_case, oracle_out
from synth import bf16_to_f32, f32_to_bf16


# ----------------------------------------------------------------- fp16 --
def test_f2h_matches_numpy_rounding():
    rng = np.random.default_rng(1)
    v = np.concatenate([
        rng.standard_normal(3000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 3000),
        # exact halfway cases between fp16 neighbours, both parities, normal and subnormal
        (np.arange(1, 600, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24),
        (np.float32(1.0) + (np.arange(0, 600, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10)),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, np.inf, -np.inf,
                  2.0 ** -25, 2.0 ** -25 * 1.0001, 2.0 ** -14, 2.0 ** -14 * (1 - 2 ** -12)],
                 np.float32),
    ]).astype(np.float32)
    ours = np.array([oracle.f2h(x) for x in v], np.uint16)
    with np.errstate(over="ignore"):  # 1e6 -> inf, as the conversion does
        want = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, want)
    back = np.array([oracle.lib().orc_h2f(int(h)) for h in want], np.float32)
    assert np.array_equal(back, want.view(np.float16).astype(np.float32))


# --------------------------------------------------- KV quantisation --
def test_kv_quantize_power_of_two_rows_are_exact():
    """Row max 127 * 2^j: the inverse scale 127 / safe is exactly 2^-j, so
    code = rint(x / 2^j): integers map to themselves and halves to the even
    neighbour (rint, not round-half-away)."""
    for j in (-6, 0, 3):
        c = 2.0 ** j
        k = np.concatenate([np.arange(-127, 128), np.arange(-20, 20) + 0.5, [127.0]])
        x = f32_to_bf16((k[:KV] if k.size >= KV else np.resize(k, KV)).astype(np.float32) * c)
        x = x.reshape(1, KV)
        q, s = oracle.kv_quantize_rows(x)
        kv = bf16_to_f32(x)[0] / c
        want = np.where(np.abs(kv - np.trunc(kv)) == 0.5,
                        2 * np.round(kv / 2), np.round(kv))  # ties to even
        assert np.array_equal(q[0].astype(np.float64), want)
        assert s[0] == np.float32(c).astype(np.float16).view(np.uint16)


def test_kv_quantize_properties():
    rng = np.random.default_rng(2)
    x = f32_to_bf16((rng.standard_normal((200, KV)) * np.exp(rng.normal(0, 3, (200, 1))))
                    .astype(np.float32))
    q, s = oracle.kv_quantize_rows(x)
    xf = bf16_to_f32(x).astype(np.float64)
    amax = np.abs(xf).max(axis=1)
    sf = s.view(np.float16).astype(np.float64)
    safe = np.maximum(amax, 1e-6)
    # the stored scale is fp16(safe / 127): within fp16 half-ulp of it
    assert np.all(np.abs(sf - safe / 127) <= np.abs(safe / 127) * 2.0 ** -11 + 2.0 ** -25)
    # the largest element maps to +-127; codes stay in [-127, 127]
    i = np.abs(xf).argmax(axis=1)
    assert np.array_equal(np.abs(q[np.arange(200), i]), np.full(200, 127))
    assert q.min() >= -127
    # each code is the nearest integer to x * 127 / safe
    assert np.all(np.abs(q - xf * 127 / safe[:, None]) <= 0.5 + 1e-5)
    # sign symmetry
    qn, sn = oracle.kv_quantize_rows(x ^ np.uint16(0x8000))
    assert np.array_equal(qn, -q) and np.array_equal(sn, s)
    # an all-zero row keeps the 1e-6 floor and zero codes
    qz, sz = oracle.kv_quantize_rows(np.zeros((1, KV), np.uint16))
    assert not qz.any() and sz[0] == np.float16(np.float32(1e-6) / np.float32(127)).view(np.uint16)


# ---------------------------------------------------------- attention --
def textbook(c, prefix_rule=0):
    """float64 softmax attention with a sink over the token history itself
    (no cache rows): keys and values are the int8-dequantised rows, or the
    bf16 rows where the prefix rule says so."""
    out = np.zeros((c.B, N_HEADS, HD))
    for b in range(c.B):
        pos = int(c.pos[b])
        n = pos + 1
        kq, ks = oracle.kv_quantize_rows(c.k_hist[b][:n])
        vq, vs = oracle.kv_quantize_rows(c.v_hist[b][:n])
        K = kq.astype(np.float64) * ks.view(np.float16).astype(np.float64)[:, None]
        V = vq.astype(np.float64) * vs.view(np.float16).astype(np.float64)[:, None]
        if not c.even() and c.keep:
            use = np.arange(n) < c.keep if prefix_rule == 1 else np.full(n, pos < c.keep)
            K[use] = bf16_to_f32(c.k_hist[b][:n][use])
            V[use] = bf16_to_f32(c.v_hist[b][:n][use])
        t0 = max(0, pos - c.window + 1) if (c.even() and c.window) else 0
        q = bf16_to_f32(c.q[b]).astype(np.float64)
        for h in range(N_HEADS):
            g = h // (N_HEADS // N_KV)
            s = K[t0:, g * HD:(g + 1) * HD] @ q[h] / 8.0
            s = np.append(s, float(bf16_to_f32(c.sinks[h:h + 1])[0]))
            p = np.exp(s - s.max())
            p /= p.sum()
            out[b, h] = p[:-1] @ V[t0:, g * HD:(g + 1) * HD]
    return out


CASES = [
    dict(layer_idx=0, pos=[0, 5, 127, 128, 300]),            # even: ring wrap, window edges
    dict(layer_idx=1, pos=[0, 15, 16, 40, 129]),             # odd: bf16 while pos < 16
    dict(layer_idx=3, pos=[3, 200], keep=128),               # the C4 prefix length
    dict(layer_idx=2, pos=[64, 1000], window=128),
]


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("rule", [0, 1])
def test_attention_matches_float64_textbook(case, rule):
    c = make_case(100 + case, **CASES[case])
    got = oracle_out(c, prefix_rule=rule)
    want = textbook(c, prefix_rule=rule)
    err = np.abs(got - want).max()
    assert err <= 2e-6 * max(1.0, np.abs(want).max()), err


def test_attention_closed_form_uniform_keys():
    """Zero keys: every attended token weighs 1 and the sink e^sink, so
    out = sum(V over the window) / (n + e^sink).  Even layer at pos 300:
    exactly tokens 173..300 (n = 128); odd layer: tokens 0..pos."""
    for layer, pos, n in ((0, 300, 128), (0, 50, 51), (1, 300, 301)):
        c = make_case(7, layer_idx=layer, pos=[pos], kscale=0.0, keep=0,
                      cap=128 if layer == 0 else 301)
        got = oracle_out(c)[0]
        vq, vs = oracle.kv_quantize_rows(c.v_hist[0])
        V = vq.astype(np.float64) * vs.view(np.float16).astype(np.float64)[:, None]
        sinks = bf16_to_f32(c.sinks).astype(np.float64)
        for h in (0, 9, 63):
            g = h // 8
            want = V[pos - n + 1:pos + 1, g * HD:(g + 1) * HD].sum(0) / (n + np.exp(sinks[h]))
            np.testing.assert_allclose(got[h], want, rtol=1e-5, atol=1e-6)


def test_attention_one_hot_follows_gqa_head():
    """A key aligned with the query at one token and zero elsewhere, with a
    very negative sink: each head returns that token's value row of its own
    KV head (h // 8), so a wrong head grouping or token index fails."""
    c = make_case(11, layer_idx=1, pos=[40], keep=0, sink_scale=0.0)
    c.sinks[:] = f32_to_bf16(np.full(N_HEADS, -80.0, np.float32))
    kh = np.zeros((41, KV), np.float32)
    qf = np.zeros((N_HEADS, HD), np.float32)
    for g in range(N_KV):
        kh[17 + g, g * HD] = 64.0          # KV head g peaks at token 17 + g
    qf[:, 0] = 64.0
    c.k_hist[0] = f32_to_bf16(kh)
    c.q[0] = f32_to_bf16(qf)
    from attn_cases import write_caches
    write_caches(c)
    got = oracle_out(c)[0]
    vq, vs = oracle.kv_quantize_rows(c.v_hist[0])
    V = vq.astype(np.float64) * vs.view(np.float16).astype(np.float64)[:, None]
    for h in range(N_HEADS):
        g = h // 8
        np.testing.assert_allclose(got[h], V[17 + g, g * HD:(g + 1) * HD], rtol=1e-6, atol=1e-7)


def test_prefix_rule_sources():
    """Odd layer, keep 16.  Rule 0 at pos 10 and rule 1 at any pos read the
    bf16 rows for t < 16; rule 0 at pos >= 16 reads only int8 rows."""
    for pos, rule, bf16_upto in ((10, 0, 11), (10, 1, 11), (40, 0, 0), (40, 1, 16)):
        c = make_case(13, layer_idx=1, pos=[pos], keep=16, kscale=0.0)
        got = oracle_out(c, prefix_rule=rule)[0]
        vq, vs = oracle.kv_quantize_rows(c.v_hist[0])
        V = vq.astype(np.float64) * vs.view(np.float16).astype(np.float64)[:, None]
        V[:bf16_upto] = bf16_to_f32(c.v_hist[0][:bf16_upto])
        sinks = bf16_to_f32(c.sinks).astype(np.float64)
        want = V[:, 0:HD].sum(0) / (pos + 1 + np.exp(sinks[0]))
        np.testing.assert_allclose(got[0], want, rtol=1e-5, atol=1e-6)


def test_phi_semantics_brute_force():
    """The reference GPU kernel's rule (phi_splits = 4): inside each of 4
    contiguous splits a token whose score is <= running max - 8 weighs 0.
    Brute force: find those tokens from the float64 scores, then take the
    exact softmax over the rest (plus the sink)."""
    c = make_case(17, layer_idx=1, pos=[257], keep=0, qscale=3.0)
    got = oracle_out(c, phi_splits=4)[0]
    exact = oracle_out(c, phi_splits=0)[0]
    pos = 257
    n = pos + 1
    kq, ks = oracle.kv_quantize_rows(c.k_hist[0])
    vq, vs = oracle.kv_quantize_rows(c.v_hist[0])
    K = kq.astype(np.float64) * ks.view(np.float16).astype(np.float64)[:, None]
    V = vq.astype(np.float64) * vs.view(np.float16).astype(np.float64)[:, None]
    q = bf16_to_f32(c.q[0]).astype(np.float64)
    sinks = bf16_to_f32(c.sinks).astype(np.float64)
    dropped_any = False
    for h in range(N_HEADS):
        g = h // 8
        s = K[:, g * HD:(g + 1) * HD] @ q[h] / 8.0
        keep = np.ones(n, bool)
        for w in range(4):
            m = -np.inf
            for t in range(n * w // 4, n * (w + 1) // 4):
                m = max(m, s[t])
                keep[t] = s[t] - m > -8.0
        dropped_any |= not keep.all()
        sk = np.append(s[keep], sinks[h])
        p = np.exp(sk - sk.max())
        p /= p.sum()
        want = p[:-1] @ V[keep, g * HD:(g + 1) * HD]
        np.testing.assert_allclose(got[h], want, rtol=2e-4, atol=2e-5)
    assert dropped_any                      # the case exercises the rule
    assert np.abs(got - exact).max() > 0    # and it differs from run.cpp's math


@pytest.mark.parametrize("case", range(len(CASES)))
def test_bf16_cache_matches_float64_textbook(case):
    """The 20B path's bf16 cache: the textbook over the history's own bf16
    rows (no quantisation), with the window on even layers."""
    from attn_cases import oracle_out_bf16
    c = make_case(200 + case, **CASES[case])
    got = oracle_out_bf16(c)
    want = np.zeros((c.B, N_HEADS, HD))
    for b in range(c.B):
        pos = int(c.pos[b])
        t0 = max(0, pos - c.window + 1) if (c.even() and c.window) else 0
        K = bf16_to_f32(c.k_hist[b][t0:pos + 1]).astype(np.float64)
        V = bf16_to_f32(c.v_hist[b][t0:pos + 1]).astype(np.float64)
        q = bf16_to_f32(c.q[b]).astype(np.float64)
        for h in range(N_HEADS):
            g = h // 8
            s = np.append(K[:, g * HD:(g + 1) * HD] @ q[h] / 8.0, float(bf16_to_f32(c.sinks[h:h + 1])[0]))
            p = np.exp(s - s.max())
            p /= p.sum()
            want[b, h] = p[:-1] @ V[:, g * HD:(g + 1) * HD]
    assert np.abs(got - want).max() <= 2e-6 * max(1.0, np.abs(want).max())
