"""GPU runs of weights read from a synthetic original-format checkpoint
(gpt-oss_amd/checkpoint.py; tests/ckpt_fixture.py): one MoE layer
(MoeLayer.from_checkpoint, config-0 shape) against the oracle on the same
bytes, and the decode step (decoder.from_checkpoint) against the oracle's
composition over 12 teacher-forced steps."""
import numpy as np
import pytest
import torch

import checkpoint as ck
import decoder as dec
import gptoss_moe as gm
import oracle
import parity
import synth
from ckpt_fixture import SMALL, write
from decoder_ref import OracleDecoder

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("gpu")]


def moe_data(a, top_k, tokens):
    c = synth.MoeConfig("checkpoint", a["hidden"], a["intermediate"], a["n_experts"], top_k, tokens,
                        "router", 0)
    return synth.MoeData(c, None, a["router_w"], a["router_b"], a["w1"], a["w1_scales"], a["b1"], a["w2"],
                         a["w2_scales"], a["b2"])


def test_moe_layer_from_checkpoint(tmp_path):
    cfg = dict(SMALL, hidden_size=128, intermediate_size=128, num_experts=4, experts_per_token=2)
    write(str(tmp_path), cfg, scale_lo=118, scale_hi=127)
    T = 8
    lay = gm.MoeLayer.from_checkpoint(str(tmp_path), 1, T, drop_unpacked=True)
    a = ck.Checkpoint(str(tmp_path)).moe_layer(1)
    rng = np.random.default_rng(5)
    x = synth.f32_to_bf16(rng.standard_normal((T, 128)).astype(np.float32))
    out = lay.forward(torch.from_numpy(x.view(np.int16)).cuda())
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    want = oracle.moe_forward(moe_data(a, 2, T), x_norm=x, forced=False)["e_agg"]
    parity.assert_close(got, want, "MoE layer from a checkpoint")


def test_decoder_from_checkpoint(tmp_path):
    cfg = dict(SMALL, hidden_size=256, intermediate_size=256, num_experts=8, experts_per_token=4,
               vocab_size=512)
    write(str(tmp_path), cfg, scale_lo=118, scale_hi=126)
    B, steps = 3, 12
    gpu = dec.from_checkpoint(str(tmp_path), B, max_ctx=64, keep=16)
    c = ck.Checkpoint(str(tmp_path))
    w = dec.checkpoint_host_weights(c, gpu.cfg)
    ref = OracleDecoder(gpu.cfg, B, w, [moe_data(c.moe_layer(l), 4, B) for l in range(2)])
    rng = np.random.default_rng(9)
    tokens = rng.integers(0, 512, size=(steps, B)).astype(np.int32)
    for s in range(steps):
        pos = np.full(B, s, np.int32)
        gpu.step(torch.from_numpy(tokens[s]).cuda(), torch.from_numpy(pos).cuda())
        want, _ = ref.step(tokens[s], pos)
    torch.cuda.synchronize()
    got = gpu.logits.view(torch.int16).cpu().numpy().view(np.uint16)
    m = parity.compare(got, want)
    assert m["finite"] and m["rel_l2"] <= 5e-2, m
