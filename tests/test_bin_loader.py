"""The checkpoint loader (gptoss_moe_bin_*): header and offsets on the CPU,
argument errors before any device call; the GPU test is in
tests/test_gpu_bin_loader.py."""
import ctypes
import os

import numpy as np
import pytest

import binfile


def _lib():
    import gptoss_moe
    return gptoss_moe


def test_read_config_and_offsets(tmp_path):
    g = _lib()
    p = str(tmp_path / "tiny.bin")
    tag = lambda name, shape: np.full(shape, 0, np.float32)
    c = dict(binfile.TINY)
    idx = {n: i for i, (n, _) in enumerate(binfile.array_shapes(c))}

    def fill(name, shape):  # value = 1000 * array index + layer (or 0 for unlayered arrays)
        a = np.full(shape, 1000.0 * idx[name], np.float32)
        if len(shape) >= 2 and name not in ("token_embedding_table", "out"):
            a += np.arange(shape[0], dtype=np.float32).reshape((-1,) + (1,) * (len(shape) - 1))
        return a
    arrays = binfile.write_bin(p, c, fill)
    cfg = g.read_bin_config(p)
    for k in binfile.CONFIG_FIELDS:
        assert getattr(cfg, k) == pytest.approx(c[k])
    raw = np.fromfile(p, np.uint8)
    for l in range(c["n_layers"]):
        o = g.bin_layer_offsets(cfg, l)
        assert o.file_bytes == raw.size
        for name, field in (("rms_ffn_w", "rms_ffn_w"), ("w_router", "w_router"),
                            ("b_router", "b_router"), ("w_mlp1", "w_mlp1"), ("b_mlp1", "b_mlp1"),
                            ("w_mlp2", "w_mlp2"), ("b_mlp2", "b_mlp2")):
            off = getattr(o, field)
            n = arrays[name][l].size
            got = raw[off:off + 4 * n].view(np.float32)
            assert np.array_equal(got, arrays[name][l].reshape(-1)), (l, name)
    with pytest.raises(g.MoeError):
        g.bin_layer_offsets(cfg, c["n_layers"])


def test_loader_argument_errors(tmp_path):
    g = _lib()
    lib = g.load_library()
    p = str(tmp_path / "t.bin")
    c = dict(binfile.TINY)
    binfile.write_bin(p, c, lambda n, s: np.zeros(s, np.float32))
    short = str(tmp_path / "short.bin")
    with open(p, "rb") as f, open(short, "wb") as o:
        o.write(f.read()[:4096])
    dst = g.BinDest(*([16] * 9))  # never dereferenced: every case fails before device work
    buf = ctypes.c_void_p(16)
    cases = [(b"/nonexistent.bin", 0, 1 << 20), (short.encode(), 0, 1 << 20),
             (p.encode(), 3, 1 << 20), (p.encode(), -1, 1 << 20), (p.encode(), 0, 1000),
             (p.encode(), 0, 4100)]
    for path, layer, nbytes in cases:
        rc = lib.gptoss_moe_load_bin_layer(path, layer, ctypes.byref(dst), buf, buf, nbytes, None)
        assert rc == g.ERR_INVALID_ARG, (path, layer, nbytes, rc)
    cfg = g.BinConfig()
    assert lib.gptoss_moe_bin_read_config(b"/nonexistent.bin", ctypes.byref(cfg)) == g.ERR_INVALID_ARG


def test_from_bin_checks_header_before_allocating(tmp_path, monkeypatch):
    """MoeLayer.from_bin validates the header (supported shape) and the file
    size it implies before it sizes any device buffer: a truncated file or
    an unsupported shape raises MoeError, and torch.empty is never reached."""
    g = _lib()
    import torch

    def no_alloc(*a, **k):
        raise AssertionError("device allocation before the header was checked")
    monkeypatch.setattr(torch, "empty", no_alloc)
    c = dict(binfile.TINY)
    p = str(tmp_path / "t.bin")
    binfile.write_bin(p, c, lambda n, s: np.zeros(s, np.float32))
    short = str(tmp_path / "short.bin")
    with open(p, "rb") as f, open(short, "wb") as o:
        o.write(f.read()[:-4])
    with pytest.raises(g.MoeError) as e:
        g.MoeLayer.from_bin(short, 0, max_tokens=4)
    assert e.value.rc == g.ERR_INVALID_ARG
    for bad in (dict(hidden_dim=100), dict(intermediate_dim=96), dict(experts_per_token=9),
                dict(n_experts=0)):
        cb = dict(c, **bad)
        pb = str(tmp_path / "bad.bin")
        try:
            binfile.write_bin(pb, cb, lambda n, s: np.zeros(s, np.float32))
        except ValueError:
            continue
        with pytest.raises(g.MoeError):
            g.MoeLayer.from_bin(pb, 0, max_tokens=4)
