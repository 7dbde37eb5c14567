"""Writes the golden fixtures under tests/golden/ from the seeded synthetic
layers (gpt-oss_amd/synth.py) and the CPU oracle.

The reference holds no golden vectors for its MoE path, so these fixtures are
regression pins of the oracle, which tests/test_oracle.py pins independently
(closed forms, brute force, float64).  Each fixture stores a digest of the
inputs it was made from, so a change of the generator is caught too.

    python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "gpt-oss_amd"), os.path.join(ROOT, "oracle")]

import oracle  # noqa: E402
import synth  # noqa: E402


def digest(d) -> str:
    h = hashlib.sha256()
    for a in (d.x, d.router_w, d.router_b, d.w1, d.s1, d.b1, d.w2, d.s2, d.b2):
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def golden(d, rows=None):
    x = d.x if rows is None else d.x[rows]
    lg = oracle.router_logits(x, d.router_w)
    ti, tw = oracle.topk_softmax(lg, d.router_b, d.cfg.top_k)
    idx = oracle.route_index(ti, tw, d.cfg.n_experts)
    e_agg, act = oracle.moe_experts(d, x, ti, tw, want_act=True)
    eng = oracle.Fp32Engine(d)
    xf = synth.bf16_to_f32(x)
    cpu = np.stack([eng.token(xf[t]) for t in range(x.shape[0])])
    out = {"digest": np.frombuffer(digest(d).encode(), np.uint8), "logits": lg, "topk_i": ti,
           "topk_w": tw, "e_agg": e_agg, "cpu_fp32_e_agg": cpu,
           "act": act[:int(idx["offsets"][-1])]}
    out.update({k: v for k, v in idx.items() if k != "dropped"})
    return out


def main():
    d0 = synth.make_data("c0_tiny")
    np.savez_compressed(os.path.join(HERE, "c0_tiny.npz"), **golden(d0))
    d1 = synth.make_data("c1_20b_decode")
    g1 = golden(d1, rows=np.arange(8))
    g1.pop("act")
    np.savez_compressed(os.path.join(HERE, "c1_20b_decode_first8.npz"), **g1)


if __name__ == "__main__":
    main()
