"""The original-checkpoint reader (gpt-oss_amd/checkpoint.py) on a synthetic
safetensors checkpoint with the reference exporter's tensor names and shapes
(export_model_bin.py:41-62): MoE matrices byte for byte, their values equal
to the exporter's dequantisation (restated below from export_model_bin.py:
86-123, closed form: LUT[low nibble] at even and LUT[high nibble] at odd
elements, times 2^(scale - 127)), the other tensors rounded to bf16, config
parsing and error paths."""
import numpy as np
import pytest
import torch

import checkpoint as ck
import decoder as dec
import oracle
from ckpt_fixture import SMALL, write
from synth import f32_to_bf16

FP4 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
               np.float32)


def exporter_dequant(blocks: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """dequantize_fp4 of the exporter in float32: [..., G, 16] bytes and
    [..., G] scales -> [..., G * 32] values."""
    lo, hi = FP4[blocks & 15], FP4[blocks >> 4]
    v = np.empty(blocks.shape[:-1] + (32,), np.float32)
    v[..., 0::2], v[..., 1::2] = lo, hi
    with np.errstate(over="ignore"):  # scales near 254 overflow to inf, as in the exporter
        v = np.ldexp(v, (scales.astype(np.int32) - 127)[..., None]).astype(np.float32)
    return v.reshape(blocks.shape[:-2] + (-1,))


@pytest.fixture(scope="module")
def small(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    t = write(str(d))
    return str(d), t


def test_moe_layer_bytes_and_bf16(small):
    path, t = small
    c = ck.Checkpoint(path)
    assert c.n_layers() == SMALL["num_hidden_layers"]
    H, D, E = SMALL["hidden_size"], SMALL["intermediate_size"], SMALL["num_experts"]
    for l in range(2):
        a = c.moe_layer(l)
        m = f"block.{l}.mlp."
        assert (a["hidden"], a["intermediate"], a["n_experts"]) == (H, D, E)
        assert a["w1"].size == E * 2 * D * H // 2 and a["w1_scales"].size == E * 2 * D * H // 32
        assert np.array_equal(a["w1"], t[m + "mlp1_weight.blocks"].numpy().reshape(-1))
        assert np.array_equal(a["w2_scales"], t[m + "mlp2_weight.scales"].numpy().reshape(-1))
        assert np.array_equal(a["b1"], t[m + "mlp1_bias"].view(torch.int16).numpy().view(np.uint16))
        assert np.array_equal(a["router_w"], t[m + "gate.weight"].view(torch.int16).numpy().view(np.uint16))
        # fp32 norm scale: round to nearest even, by an independent restatement
        assert np.array_equal(a["rms_ffn_w"], f32_to_bf16(t[m + "norm.scale"].numpy()))


@pytest.mark.parametrize("mat", ["mlp1", "mlp2"])
def test_values_equal_the_exporters_dequant(small, mat):
    """The library's dequantisation of the bytes taken (the oracle's, pinned
    against all 16 codes x 256 scales elsewhere) equals the exporter's bf16
    values element for element."""
    path, t = small
    a = ck.Checkpoint(path).moe_layer(1)
    blk = t[f"block.1.mlp.{mat}_weight.blocks"].numpy()
    scl = t[f"block.1.mlp.{mat}_weight.scales"].numpy()
    want = f32_to_bf16(exporter_dequant(blk, scl)).reshape(-1)
    key = "w1" if mat == "mlp1" else "w2"
    got = oracle.dequant(a[key], a[key + "_scales"], want.size)
    assert np.array_equal(got, want)


def test_every_code_and_scale_against_the_exporter():
    """All 16 codes x scales 1..254: the library's layout read by the oracle
    gives the exporter's value; scales 0 and 255 are where they part (the
    library's 0 and inf against ldexp's)."""
    codes = np.arange(256, dtype=np.uint8)              # both nibbles over all pairs
    for s in range(256):
        blk = codes.reshape(16, 16)                     # 16 blocks of 16 bytes = 16 x 32 values
        scl = np.full(16, s, np.uint8)
        want = f32_to_bf16(exporter_dequant(blk, scl)).reshape(-1)
        got = oracle.dequant(blk.reshape(-1), scl, want.size)
        if 1 <= s <= 254:
            assert np.array_equal(got, want), s
        elif s == 0:
            assert (got & 0x7FFF == 0).all()            # +-0
            nz = exporter_dequant(blk, np.full(16, 127, np.uint8)).reshape(-1) != 0
            assert (want[nz] & 0x7FFF != 0).all() and (want[~nz] & 0x7FFF == 0).all()


def test_sharded_directory(tmp_path):
    t = write(str(tmp_path), shards=3)
    c = ck.Checkpoint(str(tmp_path))
    assert set(c.keys()) == set(t)
    a = c.moe_layer(0)
    assert np.array_equal(a["w2"], t["block.0.mlp.mlp2_weight.blocks"].numpy().reshape(-1))


def test_decoder_config_and_weights(small):
    path, t = small
    cfg = dec.config_from_json(ck.read_config(path), max_ctx=64, keep=16)
    assert (cfg.hidden, cfg.intermediate, cfg.n_experts, cfg.top_k, cfg.n_layers, cfg.vocab) == \
        (128, 128, 4, 2, 2, 96)
    assert (cfg.sliding_window, cfg.rope_theta, cfg.rope_scaling, cfg.initial_context_length) == \
        (32, 150000.0, 32.0, 4096.0)
    w = dec.checkpoint_host_weights(ck.Checkpoint(path), cfg)
    bits = lambda x: x.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(w["emb"], bits(t["embedding.weight"]))
    assert np.array_equal(w["out"], bits(t["unembedding.weight"]))
    assert np.array_equal(w["rms_out"], f32_to_bf16(t["norm.scale"].numpy()))
    for l in range(2):
        a = f"block.{l}.attn."
        assert np.array_equal(w["w_qkv"][l], bits(t[a + "qkv.weight"]))
        assert np.array_equal(w["b_qkv"][l], bits(t[a + "qkv.bias"]))
        assert np.array_equal(w["w_o"][l], bits(t[a + "out.weight"]))
        assert np.array_equal(w["b_o"][l], bits(t[a + "out.bias"]))
        assert np.array_equal(w["sinks"][l], bits(t[a + "sinks"]))
        assert np.array_equal(w["rms_attn"][l], f32_to_bf16(t[a + "norm.scale"].numpy()))
        assert np.array_equal(w["rms_ffn"][l], f32_to_bf16(t[f"block.{l}.mlp.norm.scale"].numpy()))
    # the shapes make_host_weights gives the decoder
    ref, _ = dec.make_host_weights(cfg)
    for k in w:
        if isinstance(w[k], list):
            assert [x.shape for x in w[k]] == [x.shape for x in ref[k]], k
        else:
            assert w[k].shape == ref[k].shape, k


def test_errors(small, tmp_path):
    path, t = small
    c = ck.Checkpoint(path)
    with pytest.raises(KeyError):
        c.moe_layer(5)
    with pytest.raises(ValueError):
        c.bf16("embedding.weight", (1, 2))
    bad = dict(SMALL, num_key_value_heads=4)
    with pytest.raises(ValueError):
        dec.config_from_json(bad)
    with pytest.raises(FileNotFoundError):
        ck.Checkpoint(str(tmp_path))
    # MXFP4 blocks whose shape does not match the biases
    from safetensors.torch import save_file
    t2 = dict(t)
    t2["block.0.mlp.mlp1_weight.scales"] = t["block.0.mlp.mlp1_weight.scales"][:, :-1].contiguous()
    save_file({k: v.contiguous() for k, v in t2.items()}, str(tmp_path / "m.safetensors"))
    with pytest.raises(ValueError):
        ck.Checkpoint(str(tmp_path / "m.safetensors")).moe_layer(0)
