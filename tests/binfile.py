"""Writer of small checkpoints in the reference's fp32 .bin format, for the
loader tests: the Config header (run.cpp:25-45) then the fp32 arrays in the
order memory_map_weights reads them (run.cpp:206-247).  Each array is filled
by `fill(name, shape)` so a test can recognise what it reads back."""
import struct

import numpy as np

CONFIG_FIELDS = ("vocab_size", "hidden_dim", "n_experts", "experts_per_token", "intermediate_dim",
                 "n_layers", "head_dim", "n_attn_heads", "n_kv_heads", "seq_len",
                 "initial_context_length", "rope_theta", "rope_scaling_factor", "sliding_window",
                 "swiglu_limit")


def array_shapes(c):
    V, H, E, D, L = c["vocab_size"], c["hidden_dim"], c["n_experts"], c["intermediate_dim"], c["n_layers"]
    hd, nh, nkv = c["head_dim"], c["n_attn_heads"], c["n_kv_heads"]
    qkv = hd * nh + 2 * hd * nkv
    return [("token_embedding_table", (V, H)), ("out", (V, H)), ("rms_attn_w", (L, H)),
            ("rms_ffn_w", (L, H)), ("rms_out_w", (H,)), ("w_qkv", (L, H, qkv)), ("b_qkv", (L, qkv)),
            ("w_o", (L, hd * nh, H)), ("b_o", (L, H)), ("attn_sinks", (L, nh)),
            ("w_router", (L, E, H)), ("b_router", (L, E)), ("w_mlp1", (L, E, 2 * D, H)),
            ("b_mlp1", (L, E, 2 * D)), ("w_mlp2", (L, E, H, D)), ("b_mlp2", (L, E, H))]


def write_bin(path, c, fill):
    hdr = struct.pack("<11i2fif", *[c[k] for k in CONFIG_FIELDS])
    arrays = {}
    with open(path, "wb") as f:
        f.write(hdr)
        for name, shape in array_shapes(c):
            a = np.ascontiguousarray(fill(name, shape), dtype=np.float32)
            assert a.shape == tuple(shape)
            arrays[name] = a
            f.write(a.tobytes())
    return arrays


TINY = {"vocab_size": 16, "hidden_dim": 128, "n_experts": 4, "experts_per_token": 2,
        "intermediate_dim": 192, "n_layers": 3, "head_dim": 64, "n_attn_heads": 2, "n_kv_heads": 1,
        "seq_len": 64, "initial_context_length": 64, "rope_theta": 150000.0,
        "rope_scaling_factor": 32.0, "sliding_window": 128, "swiglu_limit": 7.0}


def random_fill(seed):
    rng = np.random.default_rng(seed)

    def fill(name, shape):
        scale = {"w_mlp1": 0.05, "w_mlp2": 0.05, "w_router": 0.1}.get(name, 0.2)
        v = rng.standard_normal(shape) * scale
        if name == "rms_ffn_w":
            v = 1 + v
        return v.astype(np.float32)
    return fill
