"""The decode step of gpt-oss (forward_batch_gpu, getp-csrc/getp_run.cpp:
3260-3409, attention_gpu_120b :2181-2481, moe_gpu :2540-2887) composed from the
oracle's restatements, with the KV caches in the reference's logical layout (int8 codes, or the
20B path's bf16 rows when cfg.cache_kind is 1).
Test infrastructure."""
from __future__ import annotations

import numpy as np

import oracle
from attn_cases import KV


class OracleDecoder:
    def __init__(self, cfg, n_seqs, w, moe_data):
        self.cfg, self.B, self.w, self.moe = cfg, n_seqs, w, moe_data
        self.cos, self.sin = oracle.rope_table(cfg.max_ctx, base=cfg.rope_theta,
                                               scaling=cfg.rope_scaling,
                                               init_ctx=cfg.initial_context_length)
        self.caps = [cfg.sliding_window if (l % 2 == 0 and cfg.sliding_window > 0) else cfg.max_ctx
                     for l in range(cfg.n_layers)]
        B = n_seqs
        self.kq = [np.zeros((B, c, KV), np.int8) for c in self.caps]
        self.vq = [np.zeros((B, c, KV), np.int8) for c in self.caps]
        self.ks = [np.zeros((B, c), np.uint16) for c in self.caps]
        self.vs = [np.zeros((B, c), np.uint16) for c in self.caps]
        keep = max(cfg.keep, 1)
        self.kb = [np.zeros((B, keep, KV), np.uint16) for _ in self.caps]
        self.vb = [np.zeros((B, keep, KV), np.uint16) for _ in self.caps]
        # the 20B path's bf16 cache (update_kv_cache_kernel, attention.hpp:756-778)
        self.bf16_cache = getattr(cfg, "cache_kind", 0) == 1
        self.kc = [np.zeros((B, c, KV), np.uint16) for c in self.caps]
        self.vc = [np.zeros((B, c, KV), np.uint16) for c in self.caps]

    def kv_update(self, l, k, v, pos):
        """quantize_kv_cache_kernel_{int8,bf16} (attention.hpp:536-652)."""
        cfg = self.cfg
        kq, ks = oracle.kv_quantize_rows(k)
        vq, vs = oracle.kv_quantize_rows(v)
        for b, p in enumerate(pos):
            p = int(p)
            ring = l % 2 == 0 and cfg.sliding_window > 0
            if p < 0 or (not ring and p >= self.caps[l]):
                continue
            r = p % cfg.sliding_window if ring else p
            self.kc[l][b, r], self.vc[l][b, r] = k[b], v[b]
            self.kq[l][b, r], self.ks[l][b, r] = kq[b], ks[b]
            self.vq[l][b, r], self.vs[l][b, r] = vq[b], vs[b]
            if l % 2 == 1 and p < cfg.keep:
                self.kb[l][b, p], self.vb[l][b, p] = k[b], v[b]

    def attention_half(self, l, x, pos, q=None, k=None, v=None):
        """RMSNorm, QKV, RoPE, cache update, attention, output projection and
        residual; q/k/v may be given (then the cache is fed those)."""
        w, cfg = self.w, self.cfg
        out = {}
        out["t"] = t = oracle.rmsnorm(x, w["rms_attn"][l])
        out["qkv"] = qkv = oracle.matmul_bf16(t, w["w_qkv"][l])
        rq, rk, rv = oracle.qkv_bias_rope(qkv, w["b_qkv"][l], self.cos, self.sin, pos)
        out["q"], out["k"], out["v"] = rq, rk, rv
        q = rq if q is None else q
        self.kv_update(l, rk if k is None else k, rv if v is None else v, pos)
        keep = cfg.keep if l % 2 == 1 else 0
        if self.bf16_cache:
            o32 = oracle.attn_decode(q, None, None, None, None, self.kc[l], self.vc[l], w["sinks"][l], pos,
                                     n_kv_heads=8, layer_idx=l, sliding_window=cfg.sliding_window, keep=0,
                                     cache_bf16=True)
        else:
            o32 = oracle.attn_decode(q, self.kq[l], self.vq[l], self.ks[l], self.vs[l],
                                     self.kb[l] if keep else None, self.vb[l] if keep else None,
                                     w["sinks"][l], pos, n_kv_heads=8, layer_idx=l,
                                     sliding_window=cfg.sliding_window, keep=cfg.keep,
                                     prefix_rule=cfg.prefix_rule)
        from synth import f32_to_bf16
        out["o"] = o = f32_to_bf16(o32)
        out["proj"] = proj = oracle.matmul_bf16(o.reshape(self.B, -1), w["w_o"][l])
        out["x_attn"] = oracle.bias_residual(x, proj, w["b_o"][l])
        return out

    def moe_half(self, l, x):
        t = oracle.rmsnorm(x, self.w["rms_ffn"][l])
        e = oracle.moe_forward(self.moe[l], x_norm=t, forced=False)["e_agg"]
        return oracle.residual_add(x, e)

    def head(self, x):
        t = oracle.rmsnorm(x, self.w["rms_out"])
        logits = oracle.matmul_bf16(t, self.w["out"])
        return logits, oracle.argmax_bf16(logits)

    def step(self, tokens, pos):
        x = np.ascontiguousarray(self.w["emb"][tokens])
        for l in range(self.cfg.n_layers):
            x = self.attention_half(l, x, pos)["x_attn"]
            x = self.moe_half(l, x)
        return self.head(x)
