"""CPU mirror of the decode-attention kernels (gptoss_attn.hip) at the lane
level: the cache update's stores, the decode kernel's loads, its
matrix-instruction operand layout (v_mfma_f32_16x16x32_bf16: lane l supplies
A[l % 16][8 (l / 16) + j] and B[8 (l / 16) + j][l % 16], and receives
D[4 (l / 16) + i][l % 16]) and its online softmax, checked against the
oracle.  A wrong tile order, lane mapping, mask or split bound fails here
without a GPU, and every offset is checked against its buffer."""
import numpy as np
import pytest

import oracle
from attn_cases import N_HEADS, make_case, oracle_out
from attn_layout import HD, KV, N_KV, TILE, from_logical, key_offset, to_logical, value_offset
from synth import bf16_to_f32, f32_to_bf16

LANE = np.arange(64)
C, G = LANE % 16, LANE // 16
LOG2E = np.float32(1.4426950408889634)


def test_layout_maps_are_bijections():
    rows = 48
    r, gd = np.meshgrid(np.arange(rows), np.arange(KV), indexing="ij")
    for f in (key_offset, value_offset):
        o = f(r, gd // HD, gd % HD).ravel()
        assert np.array_equal(np.sort(o), np.arange(rows * KV))


def test_kv_update_lane_stores_match_layout():
    """kv_update_kernel: lane l stores key bytes (r % 16) * 64 + d0 .. +7 and
    value bytes v_tile_off(r, d0 + j) of tile ((r / 16) * 8 + l / 8)."""
    for r in (0, 5, 16, 127, 1000):
        tile = ((r >> 4) * N_KV + (LANE >> 3)) * TILE
        d0 = 8 * (LANE & 7)
        for j in range(8):
            d = d0 + j
            g = LANE >> 3
            assert np.array_equal(tile + (r & 15) * 64 + d, key_offset(r, g, d))
            vt = (d & 15) * 64 + ((r & 15) >> 2) * 16 + (d >> 4) * 4 + (r & 3)
            assert np.array_equal(tile + vt, value_offset(r, g, d))


def mfma(a_lanes, b_lanes, acc):
    """A 16x16 matrix instruction on per-lane operands [64][kpl] (values as
    floats): v_mfma_f32_16x16x32_bf16 (kpl 8) or v_mfma_i32_16x16x64_i8
    (kpl 16, integer values, exact in float64)."""
    kpl = a_lanes.shape[1]
    A = np.zeros((16, 4 * kpl), np.float64)
    B = np.zeros((4 * kpl, 16), np.float64)
    for l in range(64):
        A[l % 16, kpl * (l // 16):kpl * (l // 16) + kpl] = a_lanes[l]
        B[kpl * (l // 16):kpl * (l // 16) + kpl, l % 16] = b_lanes[l]
    D = A @ B
    out = acc.astype(np.float64).copy()
    for l in range(64):
        out[l] += D[4 * (l // 16):4 * (l // 16) + 4, l % 16]
    return out


def split_query(qf_lanes):
    """The decode kernel's int8 query: per head (lane column), E = 14 -
    frexp exponent of the head's max |q|, Q = rint(q 2^E) = 256 hi + lo.
    Returns hi, lo [64][16] and 2^-E log2(e) / 8 per lane."""
    qm = np.abs(qf_lanes).max(1)
    qm = np.maximum(qm, qm[LANE ^ 16])
    qm = np.maximum(qm, qm[LANE ^ 32])
    E = 14 - np.frexp(qm)[1]
    Q = np.rint(np.ldexp(qf_lanes.astype(np.float64), E[:, None])).astype(np.int64)
    hi = (Q + 128) >> 8
    lo = Q - (hi << 8)
    assert np.abs(Q).max() <= 1 << 14
    assert hi.min() >= -128 and hi.max() <= 127 and lo.min() >= -128 and lo.max() <= 127
    qf = np.ldexp(np.float32(0.125) * LOG2E, -E).astype(np.float32)
    return hi.astype(np.float64), lo.astype(np.float64), qf


def bf16r(x):
    return bf16_to_f32(f32_to_bf16(np.asarray(x, np.float32)))


def decode_mirror(c, S, rule, bufs, bf16cache=False):
    """attn_decode_kernel + attn_combine_kernel for case c with S splits over
    whole cache buffers (library_buffers); each sequence's slabs are found
    with the kernel's base formulas."""
    B = c.B
    out = np.zeros((B, N_HEADS, HD), np.float32)
    for b in range(B):
        kv0, s0 = b * bufs["bks"] + bufs["lko"], b * bufs["bss"] + bufs["lso"]
        n = c.cap * KV
        if bf16cache:   # the cache's own rows: codes buffers hold bf16, slab b bks + lko
            slab_k = slab_v = None
            kb_slab, vb_slab = bufs["kc"][kv0:kv0 + n], bufs["vc"][kv0:kv0 + n]
            ksf = vsf = None
        else:
            slab_k, slab_v = bufs["kc"][kv0:kv0 + n], bufs["vc"][kv0:kv0 + n]
            kp = (b * bufs["n_layers"] + c.layer_idx) * c.keep * KV   # kept-token slab
            kb_slab, vb_slab = bufs["kb"][kp:kp + c.keep * KV], bufs["vb"][kp:kp + c.keep * KV]
            ksf = bufs["ks"][s0:s0 + c.cap].view(np.float16).astype(np.float32)
            vsf = bufs["vs"][s0:s0 + c.cap].view(np.float16).astype(np.float32)
        pos = int(c.pos[b])
        ring = c.even() and c.window > 0
        nvalid = min(pos + 1, c.window) if ring else pos + 1
        nblk = (nvalid + 15) >> 4
        nb16 = 0
        if bf16cache:
            nb16 = nblk                     # every block: the cache's own bf16 rows
        elif not c.even() and c.keep > 0:
            nb16 = (nblk if pos < c.keep else 0) if rule == 0 else min(nblk, c.keep >> 4)
        for kvh in range(N_KV):
            parts = []
            for s in range(S):
                blk0, blk1 = nblk * s // S, nblk * (s + 1) // S
                qv = np.zeros((64, 16), np.float32)
                heads = kvh * 8 + C
                m = C < 8
                qf = bf16_to_f32(c.q[b]).astype(np.float32)
                for l in range(64):
                    if m[l]:
                        qv[l] = qf[heads[l], 16 * G[l]:16 * G[l] + 16]
                q0, q1 = qv[:, :8], qv[:, 8:]
                qhi, qlo, qfac = split_query(qv)
                M = np.full(64, -np.inf, np.float32)
                Ls = np.zeros(64, np.float32)
                O = np.zeros((4, 64, 4), np.float32)

                def block_ops(pair_blk, bf16, two, sub):
                    """Operands of block pair_blk + sub of the pair at pair_blk."""
                    blk = pair_blk + sub
                    t = (blk * N_KV + kvh) * TILE
                    if bf16:
                        ko = t + C * 64 + 16 * G
                        assert ko.max() + 16 <= kb_slab.size
                        kk = np.stack([bf16_to_f32(kb_slab[o:o + 16]) for o in ko])
                        vv = np.stack([bf16_to_f32(vb_slab[o:o + 16]) for o in ko])
                        ksc = np.full((64, 4), np.float32(0.125) * LOG2E, np.float32)
                        vsc = np.ones((64, 4), np.float32)
                    else:
                        ko = t + C * 64 + 16 * G
                        assert ko.max() + 16 <= slab_k.size
                        kk = np.stack([slab_k[o:o + 16] for o in ko]).astype(np.float32)
                        vv = np.stack([slab_v[o:o + 16] for o in ko]).astype(np.float32)
                        # scales through the stage's scale lanes: lane sl < 32 loads
                        # 4 B of (key if sl < 16 else value) scales of block
                        # blk + ((sl >> 3) & 1) at byte (sl & 7) * 4
                        sl = np.arange(32)
                        src_blk = pair_blk + ((sl >> 3) & 1) if two else np.full(32, pair_blk)
                        src = src_blk * 16 + (sl & 7) * 2          # first half of the 4 bytes
                        assert src.max() + 2 <= c.cap
                        stage = np.where(sl[:, None] < 16, ksf[np.stack([src, src + 1], 1)],
                                         vsf[np.stack([src, src + 1], 1)]).ravel()
                        # lane (c, g) reads 8 B at 8g (+32 second block, +64 values)
                        half = (32 if sub else 0)
                        ks_l = np.stack([stage[(half + 8 * g) // 2:(half + 8 * g) // 2 + 4] for g in G])
                        vs_l = np.stack([stage[(64 + half + 8 * g) // 2:(64 + half + 8 * g) // 2 + 4] for g in G])
                        ksc = ks_l * qfac[:, None]
                        vsc = vs_l
                    # value operand per dim tile: elements dt * 4 + i
                    vop = [vv[:, 4 * dt:4 * dt + 4] for dt in range(4)]
                    return kk[:, :8], kk[:, 8:], vop, ksc.astype(np.float32), vsc.astype(np.float32)

                def step(blk, nb, bf16):
                    nonlocal M, Ls, O
                    A = block_ops(blk, bf16, nb > 1, 0)
                    Bo = block_ops(blk, bf16, True, 1) if nb > 1 else None

                    def scores(X):
                        if bf16:
                            return mfma(X[1], q1, mfma(X[0], q0, np.zeros((64, 4)))).astype(np.float32)
                        kk = np.concatenate([X[0], X[1]], 1)        # the tile's 16 raw bytes
                        si = mfma(kk, qhi, np.zeros((64, 4))) * 256 + mfma(kk, qlo, np.zeros((64, 4)))
                        assert np.abs(si).max() < 2 ** 31
                        return si.astype(np.float32)                # int32 -> float, nearest
                    s0 = scores(A)
                    s1 = scores(Bo) if Bo else np.zeros((64, 4), np.float32)
                    row0 = blk * 16 + 4 * G
                    ok = np.zeros((64, 8), bool)
                    sv = np.full((64, 8), -np.inf, np.float32)
                    for i in range(4):
                        ok[:, i] = row0 + i < nvalid
                        ok[:, 4 + i] = (nb > 1) & (row0 + 16 + i < nvalid)
                        sv[:, i] = np.where(ok[:, i], s0[:, i] * A[3][:, i], -np.inf)
                        if Bo:
                            sv[:, 4 + i] = np.where(ok[:, 4 + i], s1[:, i] * Bo[3][:, i], -np.inf)
                    bm = sv.max(1)
                    bm = np.maximum(bm, bm[LANE ^ 16])
                    bm = np.maximum(bm, bm[LANE ^ 32])
                    mn = np.maximum(M, bm)
                    alpha = np.exp2(M - mn)
                    p = np.exp2(sv - mn[:, None])
                    Ls = Ls * alpha + p.sum(1)
                    M = mn
                    vsc = np.concatenate([A[4], Bo[4] if Bo else np.zeros((64, 4), np.float32)], 1)
                    pop = bf16r(np.where(ok, p * vsc, 0))
                    ar = np.stack([alpha[4 * G + i] for i in range(4)], 1)
                    for dt in range(4):
                        va = A[2][dt]
                        vb = Bo[2][dt] if Bo else np.zeros((64, 4), np.float32)
                        vop = np.concatenate([va, vb], 1)
                        if bf16:
                            vop = np.where(ok, vop, 0)
                        O[dt] = mfma(pop, vop, O[dt] * ar).astype(np.float32)

                e16 = min(blk1, nb16)
                for blk in range(blk0, e16, 2):
                    step(blk, min(2, e16 - blk), True)
                for blk in range(max(blk0, nb16), blk1, 2):
                    step(blk, min(2, blk1 - blk), False)
                L = Ls + Ls[LANE ^ 16]
                L = L + L[LANE ^ 32]
                # partial: m, l of heads 0..7, O rows 4g + i for g < 2
                o_rows = np.zeros((8, HD), np.float32)
                for l in range(32):
                    for dt in range(4):
                        for i in range(4):
                            o_rows[4 * G[l] + i, 16 * dt + C[l]] = O[dt][l, i]
                parts.append((M[:8].copy(), L[:8].copy(), o_rows))
            mm = np.max([p[0] for p in parts], 0)
            Lt = np.zeros(8, np.float32)
            ot = np.zeros((8, HD), np.float32)
            for pm, pl, po in parts:
                w = np.exp2(pm - mm)
                Lt += pl * w
                ot += po * w[:, None]
            sk = bf16_to_f32(c.sinks[kvh * 8:kvh * 8 + 8]) * LOG2E
            mf = np.maximum(mm, sk)
            al = np.exp2(mm - mf)
            f = al / (Lt * al + np.exp2(sk - mf))
            out[b, kvh * 8:kvh * 8 + 8] = ot * f[:, None]
    return out


def library_buffers(c, kc=None, vc=None, lead=48, tail=32, seed=0):
    """Whole cache buffers as the library holds them: per sequence `lead`
    rows of other layers, this layer's cap rows in the library's layout, then
    `tail` rows, all other memory random (a wrong base reads garbage); the
    kept-token buffer [B][n_layers][keep][KV] with this layer at its index.
    kc, vc: bf16 logical caches [B][cap][KV] for the bf16 cache kind."""
    rng = np.random.default_rng(seed)
    B, cap = c.B, c.cap
    rows = lead + cap + tail
    n_layers = c.layer_idx + 2
    bf = kc is not None
    dt = np.uint16 if bf else np.int8
    big = lambda n: rng.integers(-100, 100, n).astype(dt) if not bf else \
        f32_to_bf16(rng.standard_normal(n).astype(np.float32) * 50)
    out = {"bks": rows * KV, "lko": lead * KV, "bss": rows, "lso": lead, "n_layers": n_layers,
           "kc": big(B * rows * KV), "vc": big(B * rows * KV),
           # garbage fp16 scales (1 .. 4) outside the layer's rows
           "ks": rng.integers(0x3C00, 0x4400, B * rows).astype(np.uint16),
           "vs": rng.integers(0x3C00, 0x4400, B * rows).astype(np.uint16)}
    keep = max(c.keep, 1)
    out["kb"] = f32_to_bf16(rng.standard_normal(B * n_layers * keep * KV).astype(np.float32) * 50)
    out["vb"] = f32_to_bf16(rng.standard_normal(B * n_layers * keep * KV).astype(np.float32) * 50)
    for b in range(B):
        k, v = from_logical(kc[b], vc[b]) if bf else from_logical(c.kq[b], c.vq[b])
        o = b * out["bks"] + out["lko"]
        out["kc"][o:o + cap * KV], out["vc"][o:o + cap * KV] = k, v
        if bf:
            continue
        so = b * out["bss"] + out["lso"]
        out["ks"][so:so + cap], out["vs"][so:so + cap] = c.ks[b], c.vs[b]
        if c.keep:
            kb, vb = from_logical(c.kb[b], c.vb[b])
            kp = (b * n_layers + c.layer_idx) * c.keep * KV
            out["kb"][kp:kp + c.keep * KV], out["vb"][kp:kp + c.keep * KV] = kb, vb
    return out


@pytest.mark.parametrize("layer,pos,keep,S,rule", [
    (0, [0, 17, 200], 16, 1, 0),
    (0, [127, 5], 16, 3, 0),
    (1, [9, 40], 16, 1, 0),
    (1, [9, 40, 70], 16, 2, 1),
    (3, [130], 128, 4, 1),
])
def test_decode_mirror_matches_oracle(layer, pos, keep, S, rule):
    c = make_case(31 + layer, layer_idx=layer, pos=pos, keep=keep,
                  cap=None if layer % 2 == 0 else 16 * ((max(pos) + 16) // 16))
    bufs = library_buffers(c, seed=layer)
    # round trip of the layout helpers
    for b in range(c.B):
        o = b * bufs["bks"] + bufs["lko"]
        lk, lv = to_logical(bufs["kc"][o:o + c.cap * KV], bufs["vc"][o:o + c.cap * KV], c.cap)
        assert np.array_equal(lk, c.kq[b]) and np.array_equal(lv, c.vq[b])
    got = decode_mirror(c, S, rule, bufs)
    want = oracle_out(c, prefix_rule=rule)
    err = np.abs(got - want)
    assert err.max() <= 2e-2 * max(1.0, np.abs(want).max()), err.max()
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 4e-3, rel



@pytest.mark.parametrize("layer,pos,S", [(0, [0, 17, 200], 1), (0, [127, 5], 3), (1, [9, 40, 70], 2),
                                         (3, [130], 4)])
def test_decode_mirror_bf16_cache(layer, pos, S):
    """The bf16 cache (the reference's 20B path): every block through the
    bf16 path from the cache's layer slab, against the oracle's bf16 mode."""
    from attn_cases import bf16_caches, oracle_out_bf16
    c = make_case(51 + layer, layer_idx=layer, pos=pos, keep=16,
                  cap=None if layer % 2 == 0 else 16 * ((max(pos) + 16) // 16))
    kc, vc = bf16_caches(c)
    got = decode_mirror(c, S, 0, library_buffers(c, kc, vc, seed=layer), bf16cache=True)
    want = oracle_out_bf16(c)
    err = np.abs(got - want)
    assert err.max() <= 2e-2 * max(1.0, np.abs(want).max()), err.max()
    assert np.linalg.norm(got - want) / np.linalg.norm(want) < 4e-3
