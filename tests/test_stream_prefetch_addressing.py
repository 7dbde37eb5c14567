"""CPU check of the prefetching consumers' LDS read addresses
(stream_gemm_kernel with consumer kind 2 or 4: s_read_k and its
lds_read2st64_if / lds_read2_if / lds_read_b128_if helpers) against the
default consumer's (s_compute), which has passed its GPU parity tests.

For every lane, consumer, column tile, k step and row group, the byte
offsets the new path's instructions read (base register plus the
instruction's immediate in its own units: 256 B for ds_read2st64_b32, 4 B
for ds_read2_b32, bytes for ds_read_b128) must equal the offsets the default
consumer reads for the same operand."""
import numpy as np
import pytest

LANE = np.arange(64)
N16, G4 = LANE & 15, LANE >> 4
W_TILE = 64 * 16            # SWSlotR::w[j]: 64 lanes x 16 B
SC_OFF = 16 * W_TILE        # offsetof(SWSlotR, sc)
ROWGROUP = 16 * 256         # SASlotR::a: 16 rows of 256 B


def default_offsets(c, t, ks, m):
    """s_compute<MT, NKS, R> of default consumer c (2 column tiles): the
    bytes of the nibble dword, the e8m0 word and the activation fragment."""
    w = ((2 * c + t) * 64 + LANE) * 16 + 4 * ks          # wv[t][ks] of ws.w[2c + t][lane]
    sc = SC_OFF + 4 * ((2 * c + t) * 16 + N16)           # ws.sc words[(2c + t) * 16 + n]
    a = N16 * 256 + m * ROWGROUP + ((4 * ks + G4) ^ N16) * 16   # arow + m * 4096 + uo
    return w, sc, a


def prefetch_offsets(CT, c, t, ks, m):
    """s_read_k<R, CT, kSc> of prefetching consumer c: tile t (0 .. CT - 1)."""
    wa = (CT * c * 64 + LANE) * 16 + 4 * ks
    sa = SC_OFF + 4 * ((CT * c) * 16 + N16)
    aa = N16 * 256 + ((4 * ks + G4) ^ N16) * 16
    # r.w[t / 2][t & 1]: ds_read2st64_b32 offset0 / offset1 = (0, 4) for tiles
    # 0, 1 and (8, 12) for tiles 2, 3, in units of 256 B
    st64 = [(0, 4), (8, 12)][t // 2][t & 1]
    w = wa + 256 * st64
    # r.sc[t / 2][t & 1]: ds_read2_b32 offsets (0, 16) and (32, 48), 4 B units
    r2 = [(0, 16), (32, 48)][t // 2][t & 1]
    sc = sa + 4 * r2
    # r.a[m]: ds_read_b128 offset m * 4096 (s_read_act)
    a = aa + m * 4096
    return w, sc, a


@pytest.mark.parametrize("CT", [2, 4])
@pytest.mark.parametrize("R", [64, 128])
def test_prefetch_reads_what_the_default_reads(CT, R):
    if CT == 2 and R == 128:
        pytest.skip("kind 2 runs on 64-row tiles only")
    for c in range(16 // CT):
        for t in range(CT):
            # the default consumer owning the same column tile
            cd, td = divmod(CT * c + t, 2)
            for ks in range(4):
                for m in range(R // 16):
                    got = prefetch_offsets(CT, c, t, ks, m)
                    want = default_offsets(cd, td, ks, m)
                    for g, w_, what in zip(got, want, ("nibbles", "e8m0", "activations")):
                        assert np.array_equal(g, w_), (CT, R, c, t, ks, m, what)


def test_immediates_fit_their_fields():
    # ds_read2st64_b32 / ds_read2_b32 offsets are 8-bit fields, ds_read_b128's
    # a 16-bit byte offset
    assert max(12, 48) < 256
    assert 7 * 4096 < 65536


@pytest.mark.parametrize("CT", [2, 4])
def test_reads_stay_in_their_slot(CT):
    """Every byte read lies inside the weight slot's w / sc arrays or the
    activation slot of a 128-row tile (the larger of the two)."""
    for c in range(16 // CT):
        for t in range(CT):
            for ks in range(4):
                for m in range(8 if CT == 4 else 4):
                    w, sc, a = prefetch_offsets(CT, c, t, ks, m)
                    assert w.min() >= 0 and (w + 4).max() <= SC_OFF
                    assert sc.min() >= SC_OFF and (sc + 4).max() <= SC_OFF + 1024
                    assert a.min() >= 0 and (a + 16).max() <= 128 * 256


def test_offsets_match_the_kernel_source():
    """The immediates restated above are the ones s_read_k passes (read from
    the kernel source, so that an edit there cannot drift from this check)."""
    import os
    import re
    src = open(os.path.join(os.path.dirname(__file__), "..", "gpt-oss_amd", "csrc", "gptoss_moe.hip")).read()
    body = src[src.index("__device__ __forceinline__ int s_read_k("):]
    body = body[:body.index("\n}\n")]
    st64 = re.findall(r"lds_read2st64_if<(\d+), (\d+)>\(r\.w\[(\d)\]", body)
    r2 = re.findall(r"lds_read2_if<(\d+), (\d+)>\(r\.sc\[(\d)\]", body)
    assert sorted((int(h), int(a), int(b)) for a, b, h in st64) == [(0, 0, 4), (1, 8, 12)]
    assert sorted((int(h), int(a), int(b)) for a, b, h in r2) == [(0, 0, 16), (1, 32, 48)]
    act = src[src.index("__device__ __forceinline__ void s_read_act("):]
    act = act[:act.index("\n}\n")]
    assert "lds_read_b128_if<M, M * 4096>(a[M], aa, mt)" in act
    # the address bases
    assert "(CT * c * 64 + lane) * 16 + 4 * ks" in body
    assert "4u * (uint32_t)((CT * c) * 16 + n)" in body
    assert "(n * 256 + ((4 * ks + g) ^ n) * 16)" in body


@pytest.mark.parametrize("H,D,E", [(2880, 2880, 32), (2880, 2880, 128), (128, 128, 4), (192, 448, 5),
                                   (384, 320, 6)])
def test_weight_prefetch_reads_stay_in_the_packed_copy(H, D, E):
    """weight_prefetch_kernel: the last uint4 it reads of the nibbles and of
    the e8m0 blocks lies inside MLP1's packed regions (pk_w_expert /
    pk_s_expert bytes per expert), whatever S in 1 .. KP."""
    N, K = 2 * D, H
    CT, KP = N // 16, -(-K // 128)
    w_bytes = E * N * KP * 64                  # pk_w_expert(N, K) per expert
    s_bytes = E * N * (-(-K // 512)) * 16      # pk_s_expert(N, K) per expert
    for S in {1, KP // 2 or 1, KP}:
        per_w, per_s = S * 64, S * CT * 4
        last_w = (E * CT - 1) * KP * 64 + per_w - 1
        last_s = (E - 1) * KP * CT * 4 + per_s - 1
        assert 16 * (last_w + 1) <= w_bytes
        assert 16 * (last_s + 1) <= s_bytes
        # and the ranges are what the GEMM's producers read first: tile j of
        # expert e, stages kp < S
        e, j = E - 1, CT - 1
        assert ((e * CT + j) * KP + 0) * 64 == (e * CT + j) * KP * 64
