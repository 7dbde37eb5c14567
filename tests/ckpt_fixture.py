"""A small synthetic checkpoint in the original gpt-oss safetensors format
(tensor names and shapes of export_model_bin.py:41-62 and :86-123; MXFP4
`.blocks` [E][N][K/32][16] and `.scales` [E][N][K/32]) plus its config.json.
Test infrastructure."""
from __future__ import annotations

import json
import os

import numpy as np

SMALL = {"vocab_size": 96, "hidden_size": 128, "num_experts": 4, "experts_per_token": 2,
         "intermediate_size": 128, "num_hidden_layers": 2, "head_dim": 64, "num_attention_heads": 64,
         "num_key_value_heads": 8, "sliding_window": 32, "initial_context_length": 4096,
         "rope_theta": 150000.0, "rope_scaling_factor": 32.0, "swiglu_limit": 7.0}


def tensors(cfg=SMALL, seed=7, scale_lo=118, scale_hi=131):
    """name -> torch tensor.  Norm scales are fp32 (rounded to bf16 on read),
    everything else floating is bf16."""
    import torch
    g = torch.Generator().manual_seed(seed)
    H, D, E, V, L = (cfg[k] for k in ("hidden_size", "intermediate_size", "num_experts", "vocab_size",
                                        "num_hidden_layers"))
    NH, NKV, HD = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]
    bf = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)
    f32 = lambda *s: 1.0 + 0.1 * torch.randn(*s, generator=g)
    u8 = lambda lo, hi, *s: torch.randint(lo, hi, s, generator=g, dtype=torch.uint8)
    t = {"embedding.weight": bf(V, H), "unembedding.weight": bf(V, H), "norm.scale": f32(H)}
    q = (NH + 2 * NKV) * HD
    for l in range(L):
        a, m = f"block.{l}.attn.", f"block.{l}.mlp."
        t.update({a + "norm.scale": f32(H), a + "qkv.weight": bf(q, H), a + "qkv.bias": bf(q),
                  a + "out.weight": bf(H, NH * HD), a + "out.bias": bf(H), a + "sinks": bf(NH),
                  m + "norm.scale": f32(H), m + "gate.weight": bf(E, H), m + "gate.bias": bf(E),
                  m + "mlp1_weight.blocks": u8(0, 256, E, 2 * D, H // 32, 16),
                  m + "mlp1_weight.scales": u8(scale_lo, scale_hi, E, 2 * D, H // 32),
                  m + "mlp1_bias": bf(E, 2 * D),
                  m + "mlp2_weight.blocks": u8(0, 256, E, H, D // 32, 16),
                  m + "mlp2_weight.scales": u8(scale_lo, scale_hi, E, H, D // 32),
                  m + "mlp2_bias": bf(E, H)})
    return t


def write(dirname, cfg=SMALL, shards=1, **kw):
    """config.json + model*.safetensors (tensors dealt round robin over
    `shards` files); returns the tensors."""
    from safetensors.torch import save_file
    t = tensors(cfg, **kw)
    os.makedirs(dirname, exist_ok=True)
    names = sorted(t)
    for s in range(shards):
        save_file({n: t[n].contiguous() for n in names[s::shards]},
                  os.path.join(dirname, f"model-{s:05d}.safetensors"))
    with open(os.path.join(dirname, "config.json"), "w") as f:
        json.dump(cfg, f)
    return t
