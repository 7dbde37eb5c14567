"""The packed weight layout of gptoss_moe_pack_weights (format 0, the
streamed GEMM's) as a numpy permutation.  Test infrastructure."""
import numpy as np


def pack_expected(wq, ws, n, k, mlp1):
    """Packed nibbles and scales of one matrix [E][n][k] laid out as the
    streamed GEMM reads them: nibbles [E][n/16][kp][g][16 rows][q][4 B] with
    byte 64 kp + 16 q + 4 g of the row, scales [E][kp][n/16][16 rows][4]
    (k groups 4 kp .. 4 kp + 3), then zeros to the region size
    E * n * ceil(k/512) * 16.  Zero past K.  The nibbles of a group whose
    e8m0 byte is 0 keep only their sign bits (+-0, as the reference's code *
    0.0), so that the GEMMs need no fix-up."""
    e = wq.shape[0] // (n * k // 2)
    kp, kq, ks = -(-k // 128), -(-k // 512), k // 32
    pr = np.arange(n)
    src = ((pr & ~31) + 2 * (pr & 15) + ((pr >> 4) & 1)) if mlp1 else pr
    w = np.zeros((e, n, kp * 64), np.uint8)
    w[:, :, :k // 2] = wq.reshape(e, n, k // 2)[:, src]
    # a zero e8m0 byte: its 32 elements (16 bytes) keep only their sign bits
    zero = np.repeat(ws.reshape(e, n, ks)[:, src] == 0, 16, axis=2)
    w[:, :, :k // 2][zero] &= 0x88
    w = w.reshape(e, n // 16, 16, kp, 4, 4, 4).transpose(0, 1, 3, 5, 2, 4, 6)
    s = np.zeros((e, n, kp * 4), np.uint8)
    s[:, :, :ks] = ws.reshape(e, n, ks)[:, src]
    s = s.reshape(e, n // 16, 16, kp, 4).transpose(0, 3, 1, 2, 4).reshape(-1)
    s = np.concatenate([s, np.zeros(e * n * kq * 16 - s.size, np.uint8)])
    return w.reshape(-1), s
