"""Seeded decode-attention cases for the tests: a token history of bf16 K/V
rows, written into the reference's logical caches exactly as its decode
loop writes them one token at a time (quantize_kv_cache_kernel_impl,
attention.hpp:536-652; rows by getp_run.cpp:2195-2230), plus the query,
sinks and positions.  Uses the oracle's quantiser: test infrastructure."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

import oracle
from synth import f32_to_bf16

N_HEADS, N_KV, HD = 64, 8, 64
KV = N_KV * HD


@dataclass
class AttnCase:
    layer_idx: int
    window: int          # sliding window of even layers (0: none)
    keep: int            # bf16-kept tokens of odd layers
    cap: int             # cache rows of this layer
    pos: np.ndarray      # int32 [B]
    q: np.ndarray        # bf16 [B][N_HEADS][HD]
    k_hist: list         # per sequence: bf16 [pos + 1][KV], the keys written so far
    v_hist: list
    sinks: np.ndarray    # bf16 [N_HEADS]
    kq: np.ndarray = None  # int8 [B][cap][KV]
    vq: np.ndarray = None
    ks: np.ndarray = None  # fp16 bits [B][cap]
    vs: np.ndarray = None
    kb: np.ndarray = None  # bf16 [B][keep][KV]
    vb: np.ndarray = None

    @property
    def B(self):
        return len(self.pos)

    def even(self):
        return (self.layer_idx & 1) == 0

    def row_of(self, t):
        return t % self.window if self.even() and self.window > 0 else t


def write_caches(c: AttnCase) -> AttnCase:
    """Replay every token's cache update in position order."""
    B = c.B
    c.kq = np.zeros((B, c.cap, KV), np.int8)
    c.vq = np.zeros((B, c.cap, KV), np.int8)
    c.ks = np.zeros((B, c.cap), np.uint16)
    c.vs = np.zeros((B, c.cap), np.uint16)
    c.kb = np.zeros((B, max(c.keep, 1), KV), np.uint16)
    c.vb = np.zeros((B, max(c.keep, 1), KV), np.uint16)
    for b in range(B):
        n = int(c.pos[b]) + 1
        kq, ks = oracle.kv_quantize_rows(c.k_hist[b][:n])
        vq, vs = oracle.kv_quantize_rows(c.v_hist[b][:n])
        for t in range(n):               # later tokens overwrite ring rows
            r = c.row_of(t)
            c.kq[b, r], c.ks[b, r] = kq[t], ks[t]
            c.vq[b, r], c.vs[b, r] = vq[t], vs[t]
            if not c.even() and t < c.keep:
                c.kb[b, t] = c.k_hist[b][t]
                c.vb[b, t] = c.v_hist[b][t]
    return c


def make_case(seed, *, layer_idx, pos, window=128, keep=16, cap=None, kscale=1.0,
              vscale=1.0, qscale=1.0, sink_scale=1.0) -> AttnCase:
    rng = np.random.default_rng(seed)
    pos = np.asarray(pos, np.int32)
    if cap is None:
        cap = window if (layer_idx & 1) == 0 and window > 0 else int(pos.max()) + 1
    B = len(pos)
    k_hist, v_hist = [], []
    for b in range(B):
        n = int(pos[b]) + 1
        # per-token magnitudes vary, so per-token scales differ
        mag = np.exp(rng.normal(0, 0.5, size=(n, 1))).astype(np.float32)
        k_hist.append(f32_to_bf16(rng.standard_normal((n, KV)).astype(np.float32) * mag * kscale))
        v_hist.append(f32_to_bf16(rng.standard_normal((n, KV)).astype(np.float32) * mag * vscale))
    q = f32_to_bf16(rng.standard_normal((B, N_HEADS, HD)).astype(np.float32) * qscale)
    sinks = f32_to_bf16(rng.standard_normal(N_HEADS).astype(np.float32) * sink_scale)
    c = AttnCase(layer_idx, window, keep, cap, pos, q, k_hist, v_hist, sinks)
    return write_caches(c)


def oracle_out(c: AttnCase, prefix_rule=0, phi_splits=0):
    return oracle.attn_decode(c.q, c.kq, c.vq, c.ks, c.vs, c.kb if c.keep else None,
                              c.vb if c.keep else None, c.sinks, c.pos, n_kv_heads=N_KV,
                              layer_idx=c.layer_idx, sliding_window=c.window, keep=c.keep,
                              prefix_rule=prefix_rule, phi_splits=phi_splits)


def bf16_caches(c: AttnCase):
    """The 20B path's caches (update_kv_cache_kernel, attention.hpp:756-778):
    the bf16 rows themselves at the same rows as the int8 codes.  Returns
    (kc, vc) bf16 [B][cap][KV]."""
    kc = np.zeros((c.B, c.cap, KV), np.uint16)
    vc = np.zeros((c.B, c.cap, KV), np.uint16)
    for b in range(c.B):
        for t in range(int(c.pos[b]) + 1):
            r = c.row_of(t)
            kc[b, r], vc[b, r] = c.k_hist[b][t], c.v_hist[b][t]
    return kc, vc


def oracle_out_bf16(c: AttnCase, phi_splits=0):
    kc, vc = bf16_caches(c)
    return oracle.attn_decode(c.q, None, None, None, None, kc, vc, c.sinks, c.pos, n_kv_heads=N_KV,
                              layer_idx=c.layer_idx, sliding_window=c.window, keep=0,
                              phi_splits=phi_splits, cache_bf16=True)
