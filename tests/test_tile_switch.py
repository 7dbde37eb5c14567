"""CPU checks of the per-expert tile switch (GPTOSS_MOE_FLAG_TILE_SWITCH):
the streamed GEMM's tile list leaves out experts with big_rows rows or more
(build_tiles), and the large-M GEMM's packed loader fills its LDS stage with
exactly what its reference-layout loader fills it with, for every expert,
weight block and stage, MLP1 (gate/up rows) and MLP2, K a multiple of 128
or not.  The index arithmetic restates large_m_gemm_kernel's issue() and
write() with numpy over the 512 threads."""
import numpy as np
import pytest

from packing import pack_expected
from test_addressing import build_tiles as place_tiles

LBN, LBK = 256, 128


@pytest.mark.parametrize("seed", range(4))
def test_streamed_tiles_leave_out_big_experts(seed):
    """build_tiles with big_rows: experts at or above it get no tile, the
    others are placed as before (a balanced bijection)."""
    rng = np.random.default_rng(300 + seed)
    E = int(rng.choice([32, 128]))
    counts = rng.integers(0, 400, E)
    big = 128
    kept = np.where(counts >= big, 0, counts)           # what build_tiles tiles
    placed, xcount, unit_xcd = place_tiles(kept, tile_rows=64)
    assert sorted(placed) == list(range(sum((c + 63) // 64 for c in kept)))
    assert all(counts[e] < big for e, _ in placed.values())
    assert max(xcount) - min(xcount) <= 2
    # the large-M GEMM's own list takes exactly the others, in 128-row tiles
    large = [(e, m) for e in range(E) if counts[e] >= big for m in range(-(-counts[e] // 128))]
    assert sum(min(128, counts[e] - 128 * m) for e, m in large) + sum(kept) == counts.sum()


def lrow(r, mlp1):
    return ((r & 1) << 7) | (r >> 1) if mlp1 else r


def stage_reference(wq, ws, e, nb, j, N, K, mlp1):
    """LDS weights (bytes [256 rows][64]) and scale words [256] the
    reference-layout loader writes for (expert, block, stage); rows past N
    masked out of the comparison by `valid`."""
    KS = K // 32
    b = np.zeros((256, 4, 16), np.uint8)   # LDS row R, 16-byte unit u (before the swizzle)
    for q in range(1024):
        r0, u = q >> 2, q & 3
        row = min(nb * LBN + r0, N - 1)
        kb = min(j * 64 + 16 * u, K // 2 - 16)
        ok = nb * LBN + r0 < N and j * LBK + 32 * u < K
        src = (e * N + row) * (K // 2) + kb
        b[lrow(r0, mlp1), u] = wq[src:src + 16] if ok else 0
    s = np.zeros(256, np.uint32)
    for tid in range(256):
        row = min(nb * LBN + tid, N - 1)
        o = (e * N + row) * KS + min(4 * j, KS - 4)
        sv = int.from_bytes(bytes(ws[o:o + 4]), "little")
        ng = KS - 4 * j
        if ng < 4:
            sv = (sv >> (8 * (4 - ng))) & (0xFFFF if ng >= 2 else 0)
        s[lrow(tid, mlp1)] = sv
    valid = np.array([nb * LBN + r < N for r in range(256)])
    vrows = np.zeros(256, bool)
    for r in range(256):
        vrows[lrow(r, mlp1)] = valid[r]
    return b, s, vrows


def stage_packed(pw, ps, e, nb, j, N, K, mlp1, bounds):
    """The same from the packed copy: thread q loads lane entry q & 63 of
    packed column tile 16 nb + (q >> 6) (16 B at ((e CT + ct) KP + j) KB +
    16 (q & 63)) and writes its dword u to unit u, dword (q >> 4) & 3 of LDS
    row R(t, n); scale thread tid reads the packed word of tile tid >> 4,
    row tid & 15."""
    CT, KP = N // 16, -(-K // LBK)
    b = np.zeros((256, 4, 16), np.uint8)
    for q in range(1024):
        t, n, gq = q >> 6, q & 15, (q >> 4) & 3
        ct = min(nb * 16 + t, CT - 1)
        off = ((e * CT + ct) * KP + j) * 1024 + 16 * (q & 63)
        bounds.append((off, 16, pw.size))
        v = pw[off:off + 16] if nb * 16 + t < CT else np.zeros(16, np.uint8)
        R = ((t & 1) << 7) + 16 * (t >> 1) + n if mlp1 else 16 * t + n
        for u in range(4):
            b[R, u, 4 * gq:4 * gq + 4] = v[4 * u:4 * u + 4]
    s = np.zeros(256, np.uint32)
    for tid in range(256):
        t, n = tid >> 4, tid & 15
        ct = min(nb * 16 + t, CT - 1)
        off = ((e * KP + j) * CT + ct) * 64 + 4 * n
        bounds.append((off, 4, ps.size))
        R = ((t & 1) << 7) + 16 * (t >> 1) + n if mlp1 else 16 * t + n
        s[R] = int.from_bytes(bytes(ps[off:off + 4]), "little") if nb * 16 + t < CT else 0
    return b, s


@pytest.mark.parametrize("N,K,mlp1", [(512, 384, True), (256, 320, False), (640, 256, True),
                                      (384, 448, False), (768, 2880, True)])
def test_packed_loader_fills_the_same_stage(N, K, mlp1):
    rng = np.random.default_rng(N + K)
    E = 2
    wq = rng.integers(0, 256, E * N * K // 2, dtype=np.uint8)
    ws = rng.integers(100, 140, E * N * K // 32, dtype=np.uint8)
    pw, ps = pack_expected(wq, ws, N, K, mlp1)
    bounds = []
    for e in range(E):
        for nb in range(-(-N // LBN)):
            for j in range(-(-K // LBK)):
                rb, rs, valid = stage_reference(wq, ws, e, nb, j, N, K, mlp1)
                pb, pss = stage_packed(pw, ps, e, nb, j, N, K, mlp1, bounds)
                assert np.array_equal(rb[valid], pb[valid]), (e, nb, j)
                assert np.array_equal(rs[valid], pss[valid]), (e, nb, j)
                assert not pb[~valid].any() and not pss[~valid].any()
    for off, size, total in bounds:
        assert 0 <= off and off + size <= total
