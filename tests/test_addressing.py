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
