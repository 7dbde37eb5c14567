"""Pins the decoder-step pieces of the oracle (oracle/attn_oracle.c): the
RoPE/YaRN tables, the QKV bias + rotary split, the output-projection
epilogue, the dense bf16 GEMM and greedy sampling, against float64
formulas, closed forms and numpy/torch routines they do not share.  CPU
only."""
import math

import numpy as np
import torch

import oracle
from synth import bf16_to_f32, f32_to_bf16


def torch_bf16(a32):
    return torch.from_numpy(np.asarray(a32, np.float32)).to(torch.bfloat16).view(
        torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------------ RoPE --
def yarn_float64(n_pos, base=150000.0, d=64, s=32.0, ctx=4096.0, beta=32.0, alpha=1.0):
    """YaRN (NTK-by-parts) in float64, from its definition: dimension pair
    i rotates at base^(-2i/d); pairs whose wavelength is below
    ctx / beta (fast) keep it, pairs above ctx / alpha (slow) are divided by
    s, a linear ramp in between; magnitudes carry 0.1 ln s + 1."""
    i = np.arange(d // 2, dtype=np.float64)
    freq = base ** (2 * i / d)
    low = d / 2 * math.log(ctx / (beta * 2 * math.pi)) / math.log(base)
    high = d / 2 * math.log(ctx / (alpha * 2 * math.pi)) / math.log(base)
    ramp = np.clip((i - low) / (high - low), 0, 1)
    inv = (1 / (s * freq)) * ramp + (1 / freq) * (1 - ramp)
    conc = 0.1 * math.log(s) + 1
    ang = np.arange(n_pos, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang) * conc, np.sin(ang) * conc, inv, conc, low, high


def test_rope_table_matches_yarn_definition():
    c, s = oracle.rope_table(1024)
    wc, ws, inv, conc, low, high = yarn_float64(1024)
    # fp32 angle pos * inv_freq: absolute error grows with pos (~pos * 2^-24)
    tol = 1024 * 2.0 ** -23 * conc + 1e-6
    assert np.abs(c - wc).max() < tol and np.abs(s - ws).max() < tol
    # position 0: cos = concentration, sin = 0
    assert np.allclose(c[0], np.float32(0.1 * math.log(32.0) + 1.0), rtol=1e-7) and not s[0].any()
    # cos^2 + sin^2 = concentration^2 at every position
    assert np.allclose(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2, conc ** 2, rtol=1e-5)
    # the bands: fast pairs (i <= low) rotate at base^(-2i/d), slow pairs (i >= high) s times slower
    i = np.arange(32)
    fast, slow = i <= math.floor(low), i >= math.ceil(high)
    assert fast.sum() >= 8 and slow.sum() >= 10
    plain = 150000.0 ** (-2 * i / 64)
    assert np.allclose(inv[fast], plain[fast]) and np.allclose(inv[slow], plain[slow] / 32)
    ang1 = np.arctan2(s[1].astype(np.float64), c[1].astype(np.float64))
    assert np.allclose(ang1[fast], plain[fast], rtol=1e-5)
    assert np.allclose(ang1[slow], plain[slow] / 32, rtol=1e-5)


def test_rope_table_without_scaling_is_plain_rope():
    c, s = oracle.rope_table(16, base=10000.0, scaling=1.0)
    ang = np.arange(16)[:, None] * 10000.0 ** (-np.arange(32) / 32.0)
    assert np.abs(c - np.cos(ang)).max() < 1e-5 and np.abs(s - np.sin(ang)).max() < 1e-5


# -------------------------------------------------------- QKV split + rope --
def _rand_bf16(rng, shape, sigma=1.0):
    return f32_to_bf16((rng.standard_normal(shape) * sigma).astype(np.float32))


def test_qkv_bias_rope_closed_forms():
    rng = np.random.default_rng(3)
    B, W = 3, (64 + 16) * 64
    qkv = _rand_bf16(rng, (B, W))
    bias = _rand_bf16(rng, W, 0.1)
    pre = bf16_to_f32(torch_bf16(bf16_to_f32(qkv) + bf16_to_f32(bias)[None]))   # bf16(x + b)
    # identity table: cos 1, sin 0 -> q, k, v are the biased inputs, bit for bit
    one, zero = np.ones((4, 32), np.float32), np.zeros((4, 32), np.float32)
    q, k, v = oracle.qkv_bias_rope(qkv, bias, one, zero, np.array([0, 1, 3], np.int32))
    assert np.array_equal(bf16_to_f32(q).reshape(B, -1), pre[:, :4096])
    assert np.array_equal(bf16_to_f32(k), pre[:, 4096:4608])
    assert np.array_equal(bf16_to_f32(v), pre[:, 4608:])
    # a quarter turn: (a, b) -> (-b, a) exactly
    q, k, _ = oracle.qkv_bias_rope(qkv, bias, zero, one, np.array([0, 0, 0], np.int32))
    x = pre[:, :4096].reshape(B, 64, 64)
    assert np.array_equal(bf16_to_f32(q)[:, :, :32], -x[:, :, 32:])
    assert np.array_equal(bf16_to_f32(q)[:, :, 32:], x[:, :, :32])


def test_qkv_bias_rope_is_a_rotation():
    """With the real tables, each pair (i, i + 32) of a head is rotated by the
    table's angle at the sequence's own position and scaled by the
    concentration: compare with float64 complex multiplication."""
    rng = np.random.default_rng(4)
    B, W = 4, 80 * 64
    qkv = _rand_bf16(rng, (B, W))
    bias = _rand_bf16(rng, W, 0.1)
    cos, sin = oracle.rope_table(1024)
    pos = np.array([0, 7, 500, 1023], np.int32)
    q, k, _ = oracle.qkv_bias_rope(qkv, bias, cos, sin, pos)
    pre = bf16_to_f32(torch_bf16(bf16_to_f32(qkv) + bf16_to_f32(bias)[None])).astype(np.float64)
    for name, got, lo, nh in (("q", bf16_to_f32(q).reshape(B, -1), 0, 64), ("k", bf16_to_f32(k), 4096, 8)):
        x = pre[:, lo:lo + nh * 64].reshape(B, nh, 64)
        z = (x[..., :32] + 1j * x[..., 32:]) * (cos[pos] + 1j * sin[pos]).astype(np.complex128)[:, None, :]
        want = np.concatenate([z.real, z.imag], -1).reshape(B, -1)
        err = np.abs(got - want) / np.maximum(np.abs(want), 1e-3)
        assert np.quantile(err, 0.999) <= 2.0 ** -8, name      # bf16 rounding of the result


# ------------------------------------------------ epilogue, GEMM, argmax --
def test_bias_residual_closed_form():
    rng = np.random.default_rng(5)
    x, p = _rand_bf16(rng, (5, 256)), _rand_bf16(rng, (5, 256))
    b = _rand_bf16(rng, 256)
    got = oracle.bias_residual(x, p, b)
    t = bf16_to_f32(torch_bf16(bf16_to_f32(p) + bf16_to_f32(b)[None]))
    want = torch_bf16(t + bf16_to_f32(x))
    assert np.array_equal(got, want)


def test_matmul_bf16_against_float64():
    rng = np.random.default_rng(6)
    a, w = _rand_bf16(rng, (7, 320)), _rand_bf16(rng, (33, 320))
    got = bf16_to_f32(oracle.matmul_bf16(a, w))
    want = bf16_to_f32(a).astype(np.float64) @ bf16_to_f32(w).astype(np.float64).T
    # bf16 rounding of the exact product sum
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -8 + 1e-30)
    assert np.array_equal(oracle.matmul_bf16(a, w), torch_bf16(want.astype(np.float32)))


def test_argmax_first_of_ties():
    rng = np.random.default_rng(7)
    logits = _rand_bf16(rng, (6, 1000))
    logits[1, [17, 400, 999]] = f32_to_bf16(np.array([50.0] * 3, np.float32))   # a three-way tie
    logits[2, :] = f32_to_bf16(np.full(1000, -3.0, np.float32))                 # all equal
    got = oracle.argmax_bf16(logits)
    assert np.array_equal(got, np.argmax(bf16_to_f32(logits), axis=1))
    assert got[1] == 17 and got[2] == 0
