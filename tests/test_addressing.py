"""Bounds of every global load the grouped GEMM issues, evaluated on the CPU
for many shapes (regression test: a clamp that went negative for K < 256
once put a scale load outside its buffer).  The index arithmetic below is
the kernel's (gpt-oss_amd/csrc/gptoss_moe.hip, gemm_wproducer and
aload_stage), vectorised over lanes, stages and rows."""
import numpy as np
import pytest

BLOCK_N = 128
STAGE_K = 256


def wproducer_loads(N, K):
    """(byte offsets into one expert's nibbles, byte offsets into its scales)."""
    nst = (K + STAGE_K - 1) // STAGE_K
    nblk = (N + BLOCK_N - 1) // BLOCK_N
    q, s = [], []
    lane = np.arange(64)
    rr, ch = lane >> 3, lane & 7
    for nb in range(nblk):
        for p in range(2):
            for j in range(nst):
                k = np.minimum(j * STAGE_K + 32 * ch, K - 32)
                for hh in range(2):
                    row0 = nb * BLOCK_N + (2 * p + hh) * 32
                    wvalid = row0 < N
                    el0 = np.where(wvalid, row0 + rr, 0) * K + k
                    for t in range(4):
                        q.append((el0 + t * 8 * K) // 2)
                srow = np.minimum(nb * BLOCK_N + 64 * p + lane, N - 1)
                for m in range(4):
                    s.append(srow * (K // 32) + np.minimum(j * 8 + 2 * m, K // 32 - 2))
    return np.concatenate(q), np.concatenate(s)


def aloader_loads(K, row0, rows, P):
    nst = (K + STAGE_K - 1) // STAGE_K
    lane = np.arange(64)
    out = []
    for p in range(2):
        for j in range(nst):
            k = np.minimum(j * STAGE_K + 8 * (lane & 31), K - 8)
            for i in range(16):
                row = np.minimum(32 * p + 2 * i + (lane >> 5), rows - 1)
                out.append((row0 + row) * K + k)
    return np.concatenate(out)


@pytest.mark.parametrize("N,K", [(256, 128), (128, 128), (64, 64), (5760, 2880), (2880, 2880),
                                 (128, 64), (192, 320), (320, 192)])
def test_weight_and_scale_loads_in_bounds(N, K):
    q, s = wproducer_loads(N, K)
    # 16-byte nibble loads inside the expert's N*K/2 bytes, 2-byte scale loads
    # inside its N*K/32 bytes and 2-byte aligned
    assert q.min() >= 0 and (q + 16).max() <= N * K // 2
    assert (q % 16 == 0).all()
    assert s.min() >= 0 and (s + 2).max() <= N * K // 32
    assert (s % 2 == 0).all()


@pytest.mark.parametrize("K", [64, 128, 192, 2880])
@pytest.mark.parametrize("rows", [1, 15, 16, 33, 64])
def test_activation_loads_in_bounds(K, rows):
    P = 97  # compact rows in the buffer; the tile is the last `rows` of them
    row0 = P - rows
    a = aloader_loads(K, row0, rows, P)
    assert a.min() >= 0 and (a + 8).max() <= P * K  # 8 bf16 per load
    assert (a % 8 == 0).all()
