"""GPU parity of the decode attention (libgptoss_attn.so through its C ABI)
against the oracle (oracle/attn_oracle.c):
  - the KV-cache update is bit-exact: int8 codes, fp16 scales and bf16 rows,
    read back in the reference's logical layout;
  - decode outputs are within the layer tolerance (max-abs 2e-2 normalised,
    relative L2 1e-2) of the oracle's run.cpp semantics, and within 4e-3
    relative L2, with and without the token split;
  - at the C4 shape (512 sequences, context 1024) sampled sequences match
    the oracle, the split and unsplit paths agree, and skipped sequences
    give zeros."""
import numpy as np
import pytest
import torch

import gptoss_attn as ga
import oracle
import parity
from attn_cases import KV, make_case, oracle_out
from attn_layout import to_logical
from synth import bf16_to_f32, f32_to_bf16

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("gpu")]

TIGHT_REL_L2 = 4e-3


def _dev(a, dtype=torch.int16):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16 if dtype == torch.int16 else
                                                         np.int32)).to("cuda:0")


def replay(c, rule, cache_kind=ga.CACHE_INT8):
    """Write the case's token history into a fresh KvCache one decode step at
    a time (sequences already at their position are skipped, pos = -1)."""
    maxpos = int(c.pos.max())
    max_ctx = c.cap if not c.even() else 16 * ((maxpos + 16) // 16)
    kc = ga.KvCache(c.B, c.layer_idx + 1, max_ctx, sliding_window=c.window, keep=c.keep,
                    prefix_rule=rule, cache_kind=cache_kind)
    for t in range(maxpos + 1):
        pos = np.where(c.pos >= t, t, -1).astype(np.int32)
        k = np.zeros((c.B, KV), np.uint16)
        v = np.zeros((c.B, KV), np.uint16)
        for b in range(c.B):
            if c.pos[b] >= t:
                k[b], v[b] = c.k_hist[b][t], c.v_hist[b][t]
        kc.kv_update(c.layer_idx, _dev(k), _dev(v), _dev(pos, torch.int32))
    torch.cuda.synchronize()
    return kc


CASES = {
    "even_ring": dict(layer_idx=0, pos=[0, 5, 127, 128, 300, 1000]),
    "odd_keep16": dict(layer_idx=1, pos=[0, 15, 16, 40, 129, 511]),
    "odd_keep128": dict(layer_idx=3, pos=[3, 127, 128, 200], keep=128),
    "odd_nokeep": dict(layer_idx=5, pos=[1, 64, 300], keep=0),
}


@pytest.mark.parametrize("name", sorted(CASES))
@pytest.mark.parametrize("rule", [0, 1])
def test_kv_update_bit_exact_and_decode(name, rule):
    kw = dict(CASES[name])
    if kw["layer_idx"] % 2:
        kw["cap"] = 16 * ((max(kw["pos"]) + 16) // 16)
    c = make_case(500 + sorted(CASES).index(name), **kw)
    kc = replay(c, rule)
    kq, vq, ks, vs, kb, vb = kc.layer_slabs(c.layer_idx)
    for b in range(c.B):
        lk, lv = to_logical(kq[b], vq[b], c.cap)
        assert np.array_equal(lk, c.kq[b]), f"key codes of sequence {b}"
        assert np.array_equal(lv, c.vq[b]), f"value codes of sequence {b}"
        assert np.array_equal(ks[b], c.ks[b]) and np.array_equal(vs[b], c.vs[b]), f"scales {b}"
        if c.keep and c.layer_idx % 2:
            bk, bv = to_logical(kb[b], vb[b], c.keep)
            assert np.array_equal(bk, c.kb[b]) and np.array_equal(bv, c.vb[b]), f"bf16 rows {b}"
    want = f32_to_bf16(oracle_out(c, prefix_rule=rule))
    q = _dev(c.q)
    sinks = _dev(c.sinks)
    pos = _dev(c.pos, torch.int32)
    for split in (False, True):
        out = kc.decode(c.layer_idx, q, sinks, pos, split=split)
        got = out.view(torch.int16).cpu().numpy().view(np.uint16)
        m = parity.assert_close(got, want, f"attn {name} rule {rule} split {split}")
        assert m["rel_l2"] <= TIGHT_REL_L2, m


def test_c4_shape_sampled():
    """512 sequences at context 1024 (one even and one odd layer, bf16 rows
    for the first 128 tokens): the history is generated on the device, 12
    sampled sequences are checked against the oracle; split and unsplit
    decodes agree; a sequence at pos = -1 gets zeros."""
    B, ctx, keep = 512, 1024, 128
    g = torch.Generator(device="cuda:0").manual_seed(1234)
    kc = ga.KvCache(B, 2, ctx, sliding_window=128, keep=keep, prefix_rule=ga.PREFIX_MIXED)
    pos = torch.full((B,), ctx - 1, dtype=torch.int32, device="cuda:0")
    pos[7] = 517
    pos[300] = 64
    hist = {}
    sample = [0, 7, 63, 64, 128, 255, 300, 301, 400, 448, 500, 511]
    for t in range(ctx):
        step = torch.where(pos >= t, torch.full_like(pos, t), torch.full_like(pos, -1))
        mag = torch.exp(0.5 * torch.randn((B, 1), generator=g, device="cuda:0"))
        k = (torch.randn((B, KV), generator=g, device="cuda:0") * mag).to(torch.bfloat16)
        v = (torch.randn((B, KV), generator=g, device="cuda:0") * mag).to(torch.bfloat16)
        for layer in (0, 1):
            kc.kv_update(layer, k, v, step)
        hist[t] = (k[sample].view(torch.int16).cpu().numpy().view(np.uint16),
                   v[sample].view(torch.int16).cpu().numpy().view(np.uint16))
    q = (torch.randn((B, 64, 64), generator=g, device="cuda:0")).to(torch.bfloat16)
    sinks = torch.randn(64, generator=g, device="cuda:0").to(torch.bfloat16)
    pos_np = pos.cpu().numpy()
    from attn_cases import AttnCase, write_caches
    for layer in (0, 1):
        out = kc.decode(layer, q, sinks, pos, split=False)
        out_s = kc.decode(layer, q, sinks, pos, split=True)
        torch.cuda.synchronize()
        a = bf16_to_f32(out.view(torch.int16).cpu().numpy().view(np.uint16))
        b2 = bf16_to_f32(out_s.view(torch.int16).cpu().numpy().view(np.uint16))
        # no split is needed at this size: both launches are the same kernel
        assert np.array_equal(a, b2)
        c = AttnCase(layer, 128, keep, 128 if layer == 0 else ctx, pos_np[sample],
                     q[sample].view(torch.int16).cpu().numpy().view(np.uint16),
                     [np.stack([hist[t][0][i] for t in range(pos_np[s] + 1)]) for i, s in enumerate(sample)],
                     [np.stack([hist[t][1][i] for t in range(pos_np[s] + 1)]) for i, s in enumerate(sample)],
                     sinks.view(torch.int16).cpu().numpy().view(np.uint16))
        write_caches(c)
        want = f32_to_bf16(oracle_out(c, prefix_rule=ga.PREFIX_MIXED))
        got = f32_to_bf16(a[sample])
        m = parity.assert_close(got, want, f"attn c4 layer {layer} (12 sampled sequences)")
        assert m["rel_l2"] <= TIGHT_REL_L2, m
    # a skipped sequence decodes to zeros
    pos[5] = -1
    out = kc.decode(1, q, sinks, pos, split=False)
    assert not out[5].float().abs().sum().item()


def test_small_batch_split_matches_unsplit():
    """One and three sequences at context 1024: the split path (16 splits
    and a combine) agrees with the single-wave path within fp32 rounding."""
    c = make_case(77, layer_idx=1, pos=[1023, 700, 31], keep=16, cap=1024)
    kc = replay(c, 0)
    assert kc.ws_bytes > 0
    q, sinks, pos = _dev(c.q), _dev(c.sinks), _dev(c.pos, torch.int32)
    a = kc.decode(1, q, sinks, pos, split=False).float().cpu().numpy()
    b = kc.decode(1, q, sinks, pos, split=True).float().cpu().numpy()
    assert np.max(np.abs(a - b)) <= 2 ** -7 * max(1.0, np.abs(a).max())
    want = f32_to_bf16(oracle_out(c, prefix_rule=0))
    parity.assert_close(f32_to_bf16(b), want, "attn split 1024")


@pytest.mark.parametrize("kind", [0, 1])
def test_cpp_attention_shim(tmp_path, kind):
    """The attention shim from C++ (tests/cpp/attn_gpu_test.cpp over
    gpt-oss_amd/csrc/attn_gpu_shim.hpp, the reference's state member names):
    40 steps of 2 layers (a 32-row ring, 16 bf16-kept tokens, the mixed
    rule), with the int8 cache (attention_gpu_120b) and the bf16 cache
    (attention_gpu), the last step's outputs against the oracle, and the
    same step run as two row ranges (row_offset) bit-identical to the whole
    batch."""
    import os
    import subprocess
    from attn_cases import AttnCase, write_caches
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    exe = os.path.join(root, "gpt-oss_amd", "bin", "attn_gpu_test")
    assert os.path.exists(exe), "build it with __graft_entry__.build()"
    B, L, max_seq, window, keep, rule, T = 4, 2, 64, 32, 16, 1, 40
    rng = np.random.default_rng(21)
    mag = np.exp(rng.normal(0, 0.5, size=(T, B, 1))).astype(np.float32)
    kh = f32_to_bf16(rng.standard_normal((T, B, KV)).astype(np.float32) * mag)
    vh = f32_to_bf16(rng.standard_normal((T, B, KV)).astype(np.float32) * mag)
    q = f32_to_bf16(rng.standard_normal((B, 64, 64)).astype(np.float32))
    sinks = f32_to_bf16(rng.standard_normal((L, 64)).astype(np.float32))
    inp = tmp_path / "in.bin"
    with open(inp, "wb") as f:
        f.write(np.array([B, L, max_seq, window, keep, rule, T, kind], np.int32).tobytes())
        for t in range(T):
            f.write(kh[t].tobytes())
            f.write(vh[t].tobytes())
        f.write(q.tobytes())
        f.write(sinks.tobytes())
    outp = tmp_path / "out.bin"
    r = subprocess.run([exe, str(inp), str(outp)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0
    out = np.fromfile(outp, np.uint16).reshape(2, L, B, 64, 64)
    assert np.array_equal(out[0], out[1]), "row ranges differ from the whole batch"
    for l in range(L):
        c = AttnCase(l, window, keep, window if l % 2 == 0 else max_seq, np.full(B, T - 1, np.int32), q,
                     [kh[:, b] for b in range(B)], [vh[:, b] for b in range(B)], sinks[l])
        write_caches(c)
        if kind == 1:  # attention_gpu's bf16 cache
            from attn_cases import oracle_out_bf16
            want = f32_to_bf16(oracle_out_bf16(c))
        else:
            want = f32_to_bf16(oracle_out(c, prefix_rule=rule))
        m = parity.assert_close(out[0, l], want, f"attention shim from C++, layer {l}, cache kind {kind}")
        assert m["rel_l2"] <= TIGHT_REL_L2, m


@pytest.mark.parametrize("name", sorted(CASES))
def test_bf16_cache(name):
    """The reference's 20B path: bf16 rows in the cache (no quantisation),
    written bit for bit, and the decode against the oracle's bf16 mode."""
    from attn_cases import bf16_caches, oracle_out_bf16
    kw = dict(CASES[name])
    if kw["layer_idx"] % 2:
        kw["cap"] = 16 * ((max(kw["pos"]) + 16) // 16)
    c = make_case(700 + sorted(CASES).index(name), **kw)
    kc = replay(c, 0, cache_kind=ga.CACHE_BF16)
    kslab, vslab, _, _, _, _ = kc.layer_slabs(c.layer_idx)
    ref_k, ref_v = bf16_caches(c)
    for b in range(c.B):
        lk, lv = to_logical(kslab[b], vslab[b], c.cap)
        assert np.array_equal(lk, ref_k[b]) and np.array_equal(lv, ref_v[b]), f"rows of sequence {b}"
    want = f32_to_bf16(oracle_out_bf16(c))
    q, sinks, pos = _dev(c.q), _dev(c.sinks), _dev(c.pos, torch.int32)
    for split in (False, True):
        got = kc.decode(c.layer_idx, q, sinks, pos, split=split).view(torch.int16).cpu().numpy().view(np.uint16)
        m = parity.assert_close(got, want, f"attn bf16 cache {name} split {split}")
        assert m["rel_l2"] <= TIGHT_REL_L2, m
