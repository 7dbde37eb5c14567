"""The decode-attention cache layout of gptoss_attn.h as numpy index maps:
converting the library's blocked caches to the reference's logical
[row][kv_dim] form and back.  Test infrastructure."""
import numpy as np

N_KV, HD, KV, TILE = 8, 64, 512, 1024


def key_offset(r, g, d):
    """Offset inside a layer slab of key (row r, KV head g, dim d)."""
    return ((r // 16) * N_KV + g) * TILE + (r % 16) * 64 + d


def value_offset(r, g, d):
    return ((r // 16) * N_KV + g) * TILE + (d % 16) * 64 + ((r % 16) // 4) * 16 + (d // 16) * 4 + r % 4


def _maps(rows):
    r, gd = np.meshgrid(np.arange(rows), np.arange(KV), indexing="ij")
    g, d = gd // HD, gd % HD
    return key_offset(r, g, d), value_offset(r, g, d)


def to_logical(slab_k, slab_v, rows):
    """Library slabs (flat, rows * 512 elements) -> logical [rows][512]."""
    ko, vo = _maps(rows)
    return slab_k[ko], slab_v[vo]


def from_logical(k, v):
    rows = k.shape[0]
    ko, vo = _maps(rows)
    sk = np.zeros(rows * KV, k.dtype)
    sv = np.zeros(rows * KV, v.dtype)
    sk[ko] = k
    sv[vo] = v
    return sk, sv
