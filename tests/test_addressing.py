"""Bounds of every global load the grouped GEMM issues, evaluated on the CPU
for many shapes (regression test: a clamp that went negative for K < 256
once put a scale load outside its buffer).  The index arithmetic below is
the kernel's (gpt-oss_amd/csrc/gptoss_moe.hip, gemm_wproducer,
gemm_aloader and scale_block_load), vectorised over lanes, stages and rows."""
import numpy as np
import pytest

BLOCK_N = 256
STAGE_K = 256


def wproducer_loads(N, K):
    """Byte offsets of the weight producer's 16-byte nibble loads into one
    expert's N*K/2 bytes (gemm_wproducer, 4 producers of 64 rows: lane l loads
    row 64 p + 32 hh + 8 t + (l >> 3), chunk l & 7; invalid halves read row 0)."""
    nst = (K + STAGE_K - 1) // STAGE_K
    nblk = (N + BLOCK_N - 1) // BLOCK_N
    q = []
    lane = np.arange(64)
    rr, ch = lane >> 3, lane & 7
    for nb in range(nblk):
        for p in range(4):
            for j in range(nst):
                k = np.minimum(j * STAGE_K + 32 * ch, K - 32)
                for hh in range(2):
                    row0 = nb * BLOCK_N + 64 * p + 32 * hh
                    wvalid = row0 < N
                    el0 = np.where(wvalid, row0 + rr, 0) * K + k
                    for t in range(4):
                        q.append((el0 + t * 8 * K) // 2)
    return np.concatenate(q)


def scale_block_loads(N, K):
    """Byte offsets of the consumers' 16-byte loads of one item's scale block
    (scale_block_load: 512 consumer threads x 3 loads, clamped to the block)."""
    out = []
    tid = np.arange(512)
    for nb in range((N + BLOCK_N - 1) // BLOCK_N):
        nrows = min(BLOCK_N, N - nb * BLOCK_N)
        length = nrows * (K // 32)
        # the block must fit the LDS copy the consumers read from
        assert length <= 3 * 512 * 16
        for u in range(3):
            out.append(nb * BLOCK_N * (K // 32) + np.minimum(16 * (tid + 512 * u), length - 16))
    return np.concatenate(out)


def aloader_loads(K, row0, rows):
    """Element offsets of the activation loader's 8-element loads (gemm_aloader:
    instruction i of loader p covers rows 4 i + 2 p + (l >> 5), unit l & 31;
    rows past the tile repeat its last row)."""
    nst = (K + STAGE_K - 1) // STAGE_K
    lane = np.arange(64)
    out = []
    for p in range(2):
        for j in range(nst):
            k = np.minimum(j * STAGE_K + 8 * (lane & 31), K - 8)
            for i in range(8):
                row = np.minimum(4 * i + 2 * p + (lane >> 5), rows - 1)
                out.append((row0 + row) * K + k)
    return np.concatenate(out)


@pytest.mark.parametrize("N,K", [(256, 128), (128, 128), (64, 64), (5760, 2880), (2880, 2880),
                                 (128, 64), (192, 320), (320, 192), (6144, 3072), (3072, 3072)])
def test_weight_and_scale_loads_in_bounds(N, K):
    q = wproducer_loads(N, K)
    s = scale_block_loads(N, K)
    # 16-byte loads inside the expert's N*K/2 nibble bytes and N*K/32 scale bytes
    assert q.min() >= 0 and (q + 16).max() <= N * K // 2
    assert (q % 16 == 0).all()
    assert s.min() >= 0 and (s + 16).max() <= N * K // 32
    assert (s % 16 == 0).all()


@pytest.mark.parametrize("K", [64, 128, 192, 2880])
@pytest.mark.parametrize("rows", [1, 15, 16, 31, 32])
def test_activation_loads_in_bounds(K, rows):
    P = 97  # compact rows in the buffer; the tile is the last `rows` of them
    row0 = P - rows
    a = aloader_loads(K, row0, rows)
    assert a.min() >= 0 and (a + 8).max() <= P * K  # 8 bf16 per load
    assert (a % 8 == 0).all()


def n_mod8(n, x):
    return (n - 1 - x) // 8 + 1 if n > x else 0


def build_tiles(counts, tile_rows=32):
    """The placement of build_tiles (gptoss_moe.hip): returns {pos: (e, m)} and
    per-XCD (start, count)."""
    nt = [(c + tile_rows - 1) // tile_rows for c in counts]
    n2 = [t // 2 for t in nt]
    n1 = [t % 2 for t in nt]
    U2, U1 = sum(n2), sum(n1)
    xcount = [2 * n_mod8(U2, x) + n_mod8(U2 + U1, x) - n_mod8(U2, x) for x in range(8)]
    xstart = list(np.concatenate([[0], np.cumsum(xcount)[:-1]]))
    placed, unit_xcd = {}, {}
    r2 = r1 = 0
    for e, t in enumerate(nt):
        for m in range(t):
            u = m // 2
            if u < n2[e]:
                rank = r2 + u
                x, pos = rank & 7, 2 * (rank // 8) + (m & 1)
            else:
                rank = U2 + r1
                x = rank & 7
                pos = 2 * n_mod8(U2, x) + n_mod8(rank, x) - n_mod8(U2, x)
            assert 0 <= pos < xcount[x]
            assert xstart[x] + pos not in placed
            placed[xstart[x] + pos] = (e, m)
            unit_xcd.setdefault((e, u), set()).add(x)
        r2 += n2[e]
        r1 += n1[e]
    return placed, xcount, unit_xcd


@pytest.mark.parametrize("seed", range(6))
def test_tile_placement_is_a_balanced_bijection(seed):
    rng = np.random.default_rng(seed)
    E = int(rng.choice([4, 32, 128, 256]))
    counts = rng.integers(0, 200 if seed % 2 else 70, E)
    counts[rng.random(E) < 0.2] = 0
    placed, xcount, unit_xcd = build_tiles(counts)
    total = sum((c + 31) // 32 for c in counts)
    assert sorted(placed) == list(range(total))
    assert max(xcount) - min(xcount) <= 2
    assert all(len(v) == 1 for v in unit_xcd.values())  # a unit's tiles share an XCD


# ------------------------------------------------------------ large-M GEMM --
LBN, LBK = 256, 128


def large_m_weight_loads(N, K):
    """large_m_gemm_kernel issue(): per thread 2 x 16-byte nibble loads (block
    row q >> 2, unit q & 3 of the stage's 64-byte row chunk) and one 4-byte scale
    read as two halfwords (waves 0..3: block row tid, groups 4 j .. 4 j + 3)."""
    nst = (K + LBK - 1) // LBK
    KS = K // 32
    q, s = [], []
    tid = np.arange(512)
    for nb in range((N + LBN - 1) // LBN):
        for j in range(nst):
            for i in range(2):
                qq = tid + 512 * i
                row = np.minimum(nb * LBN + (qq >> 2), N - 1)
                kb = np.minimum(j * (LBK // 2) + 16 * (qq & 3), K // 2 - 16)
                q.append(row * (K // 2) + kb)
            row = np.minimum(nb * LBN + tid[:256], N - 1)
            s.append(row * KS + min(4 * j, KS - 4))
    return np.concatenate(q), np.concatenate(s)


@pytest.mark.parametrize("N,K", [(5760, 2880), (2880, 2880), (640, 384), (384, 320), (512, 256),
                                 (6144, 3072)])
def test_large_m_loads_in_bounds(N, K):
    q, s = large_m_weight_loads(N, K)
    assert q.min() >= 0 and (q + 16).max() <= N * K // 2 and (q % 16 == 0).all()
    # 4 scale bytes inside the expert's N*K/32, 2-byte aligned (two halfword loads)
    assert s.min() >= 0 and (s + 4).max() <= N * K // 32 and (s % 2 == 0).all()


# ------------------------------------------------- direct GEMM (packed) --
DBN, DTR, DWAVES, DSK = 256, 64, 8, 512  # weight rows per item, tile rows, waves, k per stage
DCH = DSK // 128                          # 16-byte weight chunks per lane, tile and stage


def direct_weight_loads(N, K, E):
    """direct_gemm_kernel issue_w(): per lane 2 tiles x DCH 16-byte nibble
    loads (uint4 index) per stage, for every expert, weight block, wave and
    stage; and issue_lds()'s scale loads (uint4 index, waves 0..3)."""
    CT, KP, KQ = N // 16, -(-K // 128), -(-K // 512)
    nst = -(-K // DSK)
    lane = np.arange(64)
    w_idx, s_idx = [], []
    for e in (0, E - 1):
        for nb in range(-(-N // DBN)):
            for j in range(nst):
                for w in range(DWAVES):
                    for t in range(2):
                        tile = e * CT + min(nb * (DBN // 16) + 2 * w + t, CT - 1)
                        for h in range(DCH):
                            w_idx.append((tile * KP + min(DCH * j + h, KP - 1)) * 64 + lane)
                for w in range(4):
                    ct = np.minimum(nb * (DBN // 16) + 4 * w + (lane >> 4), CT - 1)
                    s_idx.append(((e * CT + ct) * KQ + j) * 16 + (lane & 15))
    return np.concatenate(w_idx), np.concatenate(s_idx)


@pytest.mark.parametrize("N,K", [(256, 128), (128, 128), (192, 448), (896, 192), (5760, 2880),
                                 (2880, 2880), (128, 64), (6144, 3072), (64, 3072)])
def test_direct_weight_loads_in_bounds(N, K):
    E = 3
    w_idx, s_idx = direct_weight_loads(N, K, E)
    # packed sizes per expert: N * ceil(K/128) * 64 nibble bytes, N * ceil(K/512) * 16 scale bytes
    assert w_idx.min() >= 0 and (w_idx.max() + 1) * 16 <= E * N * -(-K // 128) * 64
    assert s_idx.min() >= 0 and (s_idx.max() + 1) * 16 <= E * N * -(-K // 512) * 16


def direct_activation_loads(K, rows, j):
    """issue_lds(): for every wave and its loads, the LDS row it fills (64
    units of 16 B, lane l at unit 64 q + l) and the byte offsets (from the
    tile's first row) its lanes read; rows at or past the tile's 16-row
    padding are not loaded."""
    lane = np.arange(64)
    rpad = (rows + 15) & ~15
    units, offs = [], []
    for w in range(DWAVES):
        for i in range(DTR * (DSK // 8) // 64 // DWAVES):
            q = (DTR * (DSK // 8) // 64 // DWAVES) * w + i
            if q >= rpad:
                continue
            u = lane ^ (q & 15)
            units.append(64 * q + lane)
            offs.append(np.minimum(q, rows - 1) * 2 * K + 2 * np.minimum(j * DSK + 8 * u, K - 8))
    return np.concatenate(units), np.concatenate(offs), rpad


@pytest.mark.parametrize("K", [64, 128, 448, 2880])
@pytest.mark.parametrize("rows", [1, 16, 17, 33, 63, 64])
def test_direct_activation_loads(K, rows):
    for j in range(-(-K // DSK)):
        units, offs, rpad = direct_activation_loads(K, rows, j)
        # every LDS unit of the rows the MFMAs read is written exactly once
        assert np.array_equal(np.sort(units), np.arange(rpad * 64))
        # reads stay inside the tile's rows
        assert offs.min() >= 0 and (offs + 16).max() <= rows * 2 * K
        assert (offs % 16 == 0).all()
        # the consumer's fragment (row r, unit U) sits at LDS unit r*64 + (U ^ (r & 15)):
        # the loader put source row r (clamped), k unit U there
        got = np.full(DTR * 64, -1, np.int64)
        got[units] = offs
        r = np.repeat(np.arange(rpad), 64)
        U = np.tile(np.arange(64), rpad)
        pos = r * 64 + (U ^ (r & 15))
        want = np.minimum(r, rows - 1) * 2 * K + 2 * np.minimum(j * DSK + 8 * U, K - 8)
        assert np.array_equal(got[pos], want)
        # the consumer's address form: lane part + 64 (ks ^ (n >> 2)) + m * 16 KB
        n = r & 15
        ks, g = U >> 2, U & 3
        m = r >> 4
        assert np.array_equal(16 * pos, 16 * (n * 64 + (g ^ (n & 3))) + 64 * (ks ^ (n >> 2)) + m * 16384)


@pytest.mark.parametrize("N", [128, 192, 384, 5760, 2880])
def test_direct_aux_loads(N):
    """Bias pairs (waves 4, 5: 4 bytes at element min(256 nb + 128 h + 2 l, N - 2))
    stay inside the expert's N biases; slot loads stay inside the tile."""
    lane = np.arange(64)
    for nb in range(-(-N // DBN)):
        for h in range(2):
            b = np.minimum(nb * DBN + 128 * h + 2 * lane, N - 2)
            assert b.min() >= 0 and b.max() + 2 <= N
            row = nb * DBN + 128 * h + 2 * lane
            ok = row < N
            assert np.array_equal(b[ok], row[ok])
    for rows in (1, 40, 64):
        s = np.minimum(lane, rows - 1)
        assert s.max() < rows


@pytest.mark.parametrize("seed", range(4))
def test_tile_placement_64_rows(seed):
    rng = np.random.default_rng(100 + seed)
    E = int(rng.choice([4, 32, 128]))
    counts = rng.integers(0, 150, E)
    placed, xcount, unit_xcd = build_tiles(counts, tile_rows=64)
    assert sorted(placed) == list(range(sum((c + 63) // 64 for c in counts)))
    assert max(xcount) - min(xcount) <= 2


# ------------------------------------------------------------ work items --
def item_map(ntx, nblk, Gx):
    """ItemMap.init / ItemMap.at for one XCD: workgroup w runs items
    ii = w + i Gx (i < n_items), item ii = (tile ii / nblk, block ii % nblk)."""
    items_x = ntx * nblk
    per_wg = []
    for w in range(Gx):
        n_items = (items_x - w + Gx - 1) // Gx if items_x > w else 0
        got = []
        for i in range(n_items):
            ii = w + i * Gx
            tli = ii // nblk
            got.append((tli, ii - tli * nblk))
        per_wg.append(got)
    return per_wg


@pytest.mark.parametrize("ntx,nblk,Gx", [(4, 23, 32), (4, 12, 32), (16, 23, 32), (1, 1, 32),
                                         (0, 12, 32), (3, 45, 64), (33, 12, 32), (5, 7, 3)])
def test_items_cover_every_tile_block_once(ntx, nblk, Gx):
    per_wg = item_map(ntx, nblk, Gx)
    flat = [it for got in per_wg for it in got]
    assert sorted(flat) == [(t, b) for t in range(ntx) for b in range(nblk)]
    # tile-major: the workgroups' first items are consecutive blocks of the first tiles
    first = [got[0] for got in per_wg if got]
    assert first == sorted(first)
    # balanced: item counts per workgroup differ by at most one
    n = [len(got) for got in per_wg]
    assert max(n) - min(n) <= 1


# ------------------------------------------------- index_kernel counter --
def index_grid_arrivals(G, n_blk):
    """index_kernel's grid (G, n_blk + 1): workgroup (g, b) returns at once
    when it is a planner (b == n_blk) with g > 0; all others reach the
    histogram-clearing counter."""
    return [(g, b) for b in range(n_blk + 1) for g in range(G) if not (b == n_blk and g > 0)]


@pytest.mark.parametrize("G,n_blk", [(1, 1), (1, 64), (2, 3), (64, 4), (256, 1), (8, 64)])
def test_index_done_counter_clears_once_and_resets(G, n_blk):
    """The done counter (hdr[HDR_DONE]) counts arrivals; the arrival that
    reads index_arrivals(G, n_blk) - 1 = G * n_blk is the last, clears the
    histogram and resets the counter to 0 for the next call, whatever grid
    that call has."""
    counter = 0
    for grid in ((G, n_blk), (max(1, G // 2), n_blk + 1), (1, 1)):
        arrivals = index_grid_arrivals(*grid)
        expected = grid[0] * grid[1] + 1  # index_arrivals()
        assert len(arrivals) == expected
        lasts = 0
        for _ in arrivals:  # any order: one fetch_add each
            old = counter
            counter += 1
            if old == expected - 1:
                lasts += 1
                counter = 0  # the last workgroup resets it
        assert lasts == 1 and counter == 0
