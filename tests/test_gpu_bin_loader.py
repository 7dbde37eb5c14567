"""gptoss_moe_load_bin_layer on the GPU: a tiny checkpoint in the reference's
fp32 format, loaded through a 64 KB staging (many chunks), gives the same bytes
as the oracle's MXFP4 quantiser and bf16 rounding of the same arrays, and the
loaded layer matches the oracle forward."""
import numpy as np
import pytest

import binfile
import oracle
import synth
from parity import assert_close

pytestmark = pytest.mark.gpu


def test_load_bin_layer_bytes_and_forward(gpu, tmp_path):
    import torch
    import gptoss_moe
    p = str(tmp_path / "tiny.bin")
    c = dict(binfile.TINY)
    arrays = binfile.write_bin(p, c, binfile.random_fill(5))
    l = 1
    layer = gptoss_moe.MoeLayer.from_bin(p, l, max_tokens=48, device=gpu, stage_bytes=64 << 10)
    t = {k: v.cpu().numpy() for k, v in layer.tensors.items()}
    w1p, w1s = oracle.quantize_mxfp4(arrays["w_mlp1"][l].reshape(-1))
    w2p, w2s = oracle.quantize_mxfp4(arrays["w_mlp2"][l].reshape(-1))
    assert np.array_equal(t["w1"], w1p) and np.array_equal(t["w1_scales"], w1s)
    assert np.array_equal(t["w2"], w2p) and np.array_equal(t["w2_scales"], w2s)
    bf = lambda a: synth.f32_to_bf16(a.reshape(-1))
    for key, name in (("b1", "b_mlp1"), ("b2", "b_mlp2"), ("router_w", "w_router"),
                      ("router_b", "b_router"), ("rms_ffn_w", "rms_ffn_w")):
        assert np.array_equal(t[key].view(np.uint16), bf(arrays[name][l])), key
    # the loaded layer against the oracle on the same quantised weights
    H, D, E, K = c["hidden_dim"], c["intermediate_dim"], c["n_experts"], c["experts_per_token"]
    cfg = synth.MoeConfig("bin_tiny", H, D, E, K, 48, "router", 0)
    rng = np.random.default_rng(7)
    d = synth.MoeData(cfg=cfg, x=synth.f32_to_bf16(rng.standard_normal((48, H)).astype(np.float32)),
                      router_w=bf(arrays["w_router"][l]).reshape(E, H), router_b=bf(arrays["b_router"][l]),
                      w1=w1p, s1=w1s, b1=bf(arrays["b_mlp1"][l]), w2=w2p, s2=w2s,
                      b2=bf(arrays["b_mlp2"][l]), forced_i=None, forced_w=None)
    x = torch.from_numpy(d.x.view(np.int16)).to(gpu)
    out = layer.forward(x)
    got = out.cpu().numpy().view(np.uint16)
    assert_close(got, oracle.moe_forward(d, forced=False)["e_agg"], "bin layer")
