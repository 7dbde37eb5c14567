"""Weights from the original gpt-oss checkpoint (safetensors) in this
library's layouts, without the reference's detour through an fp32 `.bin`.

The reference's exporter (export_model_bin/gpt-oss-20b/export_model_bin.py:
86-123) dequantises each `X.blocks` / `X.scales` pair to bf16 as
LUT[nibble] * 2^(scale - 127), low nibble = even element, and writes every
tensor as fp32; the runtime then rounds to bf16 (20B) or re-quantises the MoE
matrices with its frexp rule (120B, mxfp4.hpp:139-217).  The checkpoint's
MXFP4 tensors already are this library's MoE layout (include/gptoss_moe.h):
`blocks` [E][N][K/32][16] is the nibble array [E][N][K/2] (low nibble first)
and `scales` [E][N][K/32] the e8m0 array, one byte per 32 elements.  So the
MoE matrices are taken byte for byte: the values the GEMMs compute with are
exactly the exporter's bf16 values for every code and every scale 1..254
(LUT * 2^(s - 127) is a bf16 number there, or overflows to inf in both).
Scale 0 reads as 0 and 255 as inf in the library (mxfp4.hpp:42-57), where
the exporter's ldexp gives LUT * 2^-127 and LUT * 2^128.  Every other tensor
is rounded to bf16 (round to nearest even), as the runtime does with the
exporter's fp32.

Tensor names are the checkpoint's (the exporter's CATEGORIES,
export_model_bin.py:41-62): `embedding.weight`, `unembedding.weight`,
`norm.scale`, and per layer `block.{l}.attn.{norm.scale, qkv.weight,
qkv.bias, out.weight, out.bias, sinks}` and `block.{l}.mlp.{norm.scale,
gate.weight, gate.bias, mlp1_weight.blocks, mlp1_weight.scales, mlp1_bias,
mlp2_weight.blocks, mlp2_weight.scales, mlp2_bias}`.  The config is the
checkpoint's config.json (the exporter's KEYS, :33-39).
"""
from __future__ import annotations

import glob
import json
import os
from typing import Dict, List

import numpy as np

MOE_KEYS = ("gate.weight", "gate.bias", "mlp1_weight.blocks", "mlp1_weight.scales", "mlp1_bias",
            "mlp2_weight.blocks", "mlp2_weight.scales", "mlp2_bias")


def _bf16_bits(t) -> np.ndarray:
    """A floating torch tensor as bf16 bits (uint16), rounded to nearest even."""
    import torch
    if t.dtype != torch.bfloat16:
        if not t.dtype.is_floating_point:
            raise ValueError(f"expected a floating tensor, got {t.dtype}")
        t = t.to(torch.float32).to(torch.bfloat16)
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


class Checkpoint:
    """Read access to one checkpoint: a .safetensors file, or a directory
    whose *.safetensors files together hold the tensors."""

    def __init__(self, path: str):
        from safetensors import safe_open
        files: List[str] = sorted(glob.glob(os.path.join(path, "*.safetensors"))) \
            if os.path.isdir(path) else [path]
        if not files:
            raise FileNotFoundError(f"no .safetensors file in {path}")
        self._handles = [safe_open(f, framework="pt", device="cpu") for f in files]
        self._where: Dict[str, object] = {}
        for h in self._handles:
            for k in h.keys():
                self._where[k] = h

    def keys(self):
        return self._where.keys()

    def tensor(self, name: str):
        h = self._where.get(name)
        if h is None:
            raise KeyError(f"checkpoint has no tensor {name!r}")
        return h.get_tensor(name)

    def bf16(self, name: str, shape=None) -> np.ndarray:
        a = _bf16_bits(self.tensor(name))
        if shape is not None and tuple(a.shape) != tuple(shape):
            raise ValueError(f"{name}: shape {tuple(a.shape)}, expected {tuple(shape)}")
        return a

    def n_layers(self) -> int:
        n = 0
        while f"block.{n}.mlp.gate.weight" in self._where:
            n += 1
        return n

    def moe_layer(self, layer: int) -> dict:
        """Layer `layer`'s MoE weights in include/gptoss_moe.h's layouts (numpy):
        router_w bf16 [E][H], router_b bf16 [E], w1 uint8 [E*2D*H/2], w1_scales
        uint8 [E*2D*H/32], b1 bf16 [E][2D], w2 / w2_scales / b2 likewise for
        [E][H][D], rms_ffn_w bf16 [H]; plus the shape (hidden, intermediate,
        n_experts)."""
        p = f"block.{layer}.mlp."
        wr = self.bf16(p + "gate.weight")
        E, H = wr.shape
        b1 = self.bf16(p + "mlp1_bias")
        if b1.ndim != 2 or b1.shape[0] != E or b1.shape[1] % 2:
            raise ValueError(f"{p}mlp1_bias: shape {b1.shape}")
        D = b1.shape[1] // 2
        out = {"router_w": wr, "router_b": self.bf16(p + "gate.bias", (E,)), "b1": b1,
               "b2": self.bf16(p + "mlp2_bias", (E, H)), "rms_ffn_w": self.bf16(p + "norm.scale", (H,)),
               "hidden": H, "intermediate": D, "n_experts": E}
        for tag, n, k in (("1", 2 * D, H), ("2", H, D)):
            blk = self.tensor(f"{p}mlp{tag}_weight.blocks")
            scl = self.tensor(f"{p}mlp{tag}_weight.scales")
            if tuple(blk.shape) != (E, n, k // 32, 16) or tuple(scl.shape) != (E, n, k // 32):
                raise ValueError(f"{p}mlp{tag}_weight: blocks {tuple(blk.shape)}, scales "
                                 f"{tuple(scl.shape)}, expected ({E}, {n}, {k // 32}, 16) / ({E}, {n}, {k // 32})")
            out["w" + tag] = blk.contiguous().view(-1).numpy().view(np.uint8).copy()
            out["w" + tag + "_scales"] = scl.contiguous().view(-1).numpy().view(np.uint8).copy()
        return out

    def attention_layer(self, layer: int, hidden: int, n_heads: int, n_kv: int, head_dim: int) -> dict:
        """Layer `layer`'s attention weights (bf16 bits): rms_attn [H], w_qkv
        [(NH + 2 NKV) HD][H], b_qkv, w_o [H][NH HD], b_o [H], sinks [NH]."""
        p = f"block.{layer}.attn."
        q = (n_heads + 2 * n_kv) * head_dim
        return {"rms_attn": self.bf16(p + "norm.scale", (hidden,)),
                "w_qkv": self.bf16(p + "qkv.weight", (q, hidden)), "b_qkv": self.bf16(p + "qkv.bias", (q,)),
                "w_o": self.bf16(p + "out.weight", (hidden, n_heads * head_dim)),
                "b_o": self.bf16(p + "out.bias", (hidden,)), "sinks": self.bf16(p + "sinks", (n_heads,))}


def read_config(path: str) -> dict:
    """config.json (a file, or the checkpoint directory holding it)."""
    if os.path.isdir(path):
        path = os.path.join(path, "config.json")
    with open(path) as f:
        return json.load(f)
