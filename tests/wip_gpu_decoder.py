"""GPU parity of the decode step (gpt-oss_amd/decoder.py) against the
oracle's composition of the reference's decode step (tests/decoder_ref.py),
at a small shape (2 layers, hidden 256, 8 experts, vocabulary 512, a
32-row window, 16 bf16-kept tokens) over 40 teacher-forced steps:
  - op by op, every op fed the GPU's own inputs: RMSNorm, the QKV bias +
    RoPE split, the output-projection epilogue and greedy sampling
    bit-exact; the library GEMMs within one bf16 rounding; the attention
    and the MoE layer within the layer tolerance; the KV caches bit-exact
    after all 40 steps;
  - end to end (the oracle running on its own values) at the last step,
    logits within 5e-2 relative L2 (the per-op tolerances compound over
    two layers)."""
import numpy as np
import pytest
import torch

import decoder as dec
import gptoss_attn as ga
import oracle
import parity
from attn_layout import to_logical
from decoder_ref import OracleDecoder
from synth import bf16_to_f32

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("gpu")]

CFG = dec.DecoderConfig(hidden=256, intermediate=256, n_experts=8, top_k=4, n_layers=2, vocab=512,
                        max_ctx=64, sliding_window=32, keep=16, prefix_rule=ga.PREFIX_MIXED)
B, STEPS = 3, 40


def gemm_close(got, want, what):
    g = bf16_to_f32(got).astype(np.float64)
    w = bf16_to_f32(want).astype(np.float64)
    # fp32 accumulation against a double one: at most one bf16 rounding apart
    assert np.all(np.abs(g - w) <= np.abs(w) * 2.0 ** -7 + 1e-3 * np.abs(w).max()), what


@pytest.fixture(scope="module")
def model():
    w, moe = dec.make_host_weights(CFG)
    return w, moe


def test_decoder_ops_match_oracle(model):
    w, moe = model
    gpu = dec.from_host(CFG, B, w, moe)
    ref = OracleDecoder(CFG, B, w, moe)
    rng = np.random.default_rng(11)
    tokens = rng.integers(0, CFG.vocab, size=(STEPS, B)).astype(np.int32)
    for s in range(STEPS):
        pos = np.full(B, s, np.int32)
        trace = []
        nxt = gpu.step(torch.from_numpy(tokens[s]).cuda(), torch.from_numpy(pos).cuda(), trace=trace)
        torch.cuda.synchronize()
        for l, tr in enumerate(trace):
            if s == 0 and l == 0:
                assert np.array_equal(tr["x_in"], w["emb"][tokens[s]]), "embedding gather"
            assert np.array_equal(tr["t"], oracle.rmsnorm(tr["x_in"], w["rms_attn"][l])), (s, l, "rmsnorm")
            gemm_close(tr["qkv"], oracle.matmul_bf16(tr["t"], w["w_qkv"][l]), (s, l, "qkv"))
            rq, rk, rv = oracle.qkv_bias_rope(tr["qkv"], w["b_qkv"][l], ref.cos, ref.sin, pos)
            assert np.array_equal(tr["q"], rq.reshape(tr["q"].shape)), (s, l, "q")
            assert np.array_equal(tr["k"], rk) and np.array_equal(tr["v"], rv), (s, l, "k, v")
            # the oracle's caches take the GPU's k, v; its attention the GPU's q
            ref.kv_update(l, tr["k"], tr["v"], pos)
            keep = CFG.keep if l % 2 else 0
            o = oracle.attn_decode(tr["q"], ref.kq[l], ref.vq[l], ref.ks[l], ref.vs[l],
                                   ref.kb[l] if keep else None, ref.vb[l] if keep else None,
                                   w["sinks"][l], pos, n_kv_heads=8, layer_idx=l,
                                   sliding_window=CFG.sliding_window, keep=CFG.keep,
                                   prefix_rule=CFG.prefix_rule)
            from synth import f32_to_bf16
            m = parity.assert_close(tr["o"], f32_to_bf16(o), f"decoder attention step {s} layer {l}")
            assert m["rel_l2"] <= 4e-3, m
            gemm_close(tr["proj"], oracle.matmul_bf16(tr["o"].reshape(B, -1), w["w_o"][l]), (s, l, "o-proj"))
            assert np.array_equal(tr["x_attn"], oracle.bias_residual(tr["x_in"], tr["proj"], w["b_o"][l]))
            parity.assert_close(tr["x_out"], ref.moe_half(l, tr["x_attn"]), f"decoder moe step {s} layer {l}")
        logits = gpu.logits.view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(nxt.cpu().numpy(), oracle.argmax_bf16(logits)), (s, "argmax")
    # caches after 40 steps: bit-exact in the reference's logical layout
    for l in range(CFG.n_layers):
        kq, vq, ks, vs, kb, vb = gpu.kv.layer_slabs(l)
        for b in range(B):
            lk, lv = to_logical(kq[b], vq[b], gpu.kv.caps[l])
            assert np.array_equal(lk, ref.kq[l][b]) and np.array_equal(lv, ref.vq[l][b]), (l, b)
            assert np.array_equal(ks[b], ref.ks[l][b]) and np.array_equal(vs[b], ref.vs[l][b])
            if l % 2:
                bk, bv = to_logical(kb[b], vb[b], CFG.keep)
                assert np.array_equal(bk, ref.kb[l][b]) and np.array_equal(bv, ref.vb[l][b])


@pytest.mark.parametrize("kind", [ga.CACHE_INT8, ga.CACHE_BF16])
def test_decoder_end_to_end(model, kind):
    """Both cache kinds: C4's int8 cache and the 20B path's bf16 rows."""
    import dataclasses
    cfg = dataclasses.replace(CFG, cache_kind=kind)
    w, moe = model
    gpu = dec.from_host(cfg, B, w, moe)
    ref = OracleDecoder(cfg, B, w, moe)
    rng = np.random.default_rng(12)
    tokens = rng.integers(0, CFG.vocab, size=(STEPS, B)).astype(np.int32)
    for s in range(STEPS):
        pos = np.full(B, s, np.int32)
        gpu.step(torch.from_numpy(tokens[s]).cuda(), torch.from_numpy(pos).cuda())
        want, _ = ref.step(tokens[s], pos)
    torch.cuda.synchronize()
    got = gpu.logits.view(torch.int16).cpu().numpy().view(np.uint16)
    m = parity.compare(got, want)
    parity.RECORD.append({"what": f"decoder end to end, last step, cache kind {kind}", **{k: m[k] for k in ("max_abs", "max_abs_norm", "rel_l2", "frac_exact")}})
    assert m["finite"] and m["rel_l2"] <= 5e-2, m


def test_decoder_graph_replays_match_eager(model):
    """The whole step captured as a HIP graph: each replay, with eager steps
    of other positions in between, gives the eager step's logits bit for bit
    (the cache update at the replayed position rewrites the same rows)."""
    w, moe = model
    gpu = dec.from_host(CFG, B, w, moe)
    rng = np.random.default_rng(13)
    for s in range(10):
        gpu.step(torch.from_numpy(rng.integers(0, CFG.vocab, B).astype(np.int32)).cuda(),
                 torch.full((B,), s, dtype=torch.int32, device="cuda"))
    tokens = torch.from_numpy(rng.integers(0, CFG.vocab, B).astype(np.int32)).cuda()
    pos = torch.full((B,), 10, dtype=torch.int32, device="cuda")
    graph = dec.capture_step(gpu, tokens, pos)
    gpu.step(tokens, pos)
    want = gpu.logits.clone()
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gpu.logits, want), f"replay {r}"
        # eager work of another position between replays (rows past 10 are not attended at 10)
        gpu.step(tokens, torch.full((B,), 11 + r, dtype=torch.int32, device="cuda"))
        torch.cuda.synchronize()
