"""ctypes bindings of the CPU oracle (moe_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product path never uses it.
bf16 values are uint16 bit patterns; all arrays are C-contiguous numpy.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float

_SIGS = {
    "orc_f2bf": (ctypes.c_uint16, [_F]),
    "orc_bf2f": (_F, [ctypes.c_uint16]),
    "orc_dequant_mxfp4": (None, [_P, _P, _I64, _P]),
    "orc_dequant_mxfp4_f32": (None, [_P, _P, _I64, _P]),
    "orc_quantize_mxfp4": (None, [_P, _I64, _P, _P]),
    "orc_router_logits": (None, [_P, _P, _I, _I, _I, _P]),
    "orc_topk_softmax": (None, [_P, _P, _I, _I, _I, _P, _P]),
    "orc_route_index": (_I, [_P, _P, _I, _I, _I, _P, _P, _P, _P, _P]),
    "orc_moe_experts": (None, [_I, _I, _I, _I, _F, _F, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I,
                               _P, _P]),
    "orc_rmsnorm": (None, [_P, _P, _I, _I, _P]),
    "orc_residual_add": (None, [_P, _P, _I64]),
    "orc_moe_forward": (None, [_I, _I, _I, _I, _F, _F, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I,
                               _P, _P, _P, _P, _P, _P]),
    "orc_moe_forward_aq": (None, [_I, _I, _I, _I, _F, _F, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I,
                                  _P, _P, _P, _P, _P, _P, _I]),
    "orc_quantize_act": (None, [_P, _I, _I, _I, _P, _P]),
    "orc_dequant_act": (None, [_P, _P, _I, _I, _P]),
    "orc_e4m3_dec": (_F, [ctypes.c_uint8]),
    "orc_moe_fp32_token": (None, [_I, _I, _I, _I, _F, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "orc_num_threads": (_I, []),
    "orc_f2h": (ctypes.c_uint16, [_F]),
    "orc_h2f": (_F, [ctypes.c_uint16]),
    "orc_kv_quantize_row": (None, [_P, _I, _P, _P]),
    "orc_attn_decode": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I,
                             _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "orc_rope_table": (_I, [_F, _I, _F, _F, _I, _P, _P]),
    "orc_qkv_bias_rope": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P]),
    "orc_bias_residual": (None, [_P, _P, _P, _I, _I]),
    "orc_matmul_bf16": (None, [_P, _P, _I, _I, _I, _P]),
    "orc_argmax_bf16": (None, [_P, _I, _I, _P]),
}

_lib = None
NATIVE_PATH = os.path.join(_HERE, "_native", "liboracle_native.so")


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def use_native() -> bool:
    """Build the -march=native copy for this host (the reference's runomp
    flags) and load it instead of the portable one; False if it cannot be
    built here.  Call before any other oracle function."""
    global LIB_PATH
    if _lib is not None:
        raise RuntimeError("oracle library already loaded")
    r = subprocess.run(["make", "-s", "-B", "-C", _HERE, "native"], capture_output=True, text=True)
    if r.returncode != 0 or not os.path.exists(NATIVE_PATH):
        return False
    LIB_PATH = NATIVE_PATH
    return True


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        for n, (r, a) in _SIGS.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def dequant(packed, scales, n: int) -> np.ndarray:
    packed, scales = _c(packed, np.uint8), _c(scales, np.uint8)
    out = np.empty(n, np.uint16)
    lib().orc_dequant_mxfp4(_p(packed), _p(scales), n, _p(out))
    return out


def dequant_f32(packed, scales, n: int) -> np.ndarray:
    packed, scales = _c(packed, np.uint8), _c(scales, np.uint8)
    out = np.empty(n, np.float32)
    lib().orc_dequant_mxfp4_f32(_p(packed), _p(scales), n, _p(out))
    return out


def quantize_mxfp4(src):
    """fp32 [n] -> (packed uint8 [ceil(n/32)*16], scales uint8 [ceil(n/32)])."""
    s = _c(src, np.float32).reshape(-1)
    nb = (s.size + 31) // 32
    packed = np.zeros(nb * 16, np.uint8)
    scales = np.zeros(nb, np.uint8)
    lib().orc_quantize_mxfp4(_p(s), s.size, _p(packed), _p(scales))
    return packed, scales


def quantize_act(x, terms: int):
    """bf16 [rows][K] -> MXFP8 activations of the FP4-MFMA variant:
    (q uint8 [rows][ceil(K/512)*1024], s uint8 [rows][ceil(K/512)*32])."""
    x = _c(x, np.uint16)
    rows, K = x.shape
    KS = (K + 511) // 512
    q = np.empty((rows, KS * 1024), np.uint8)
    s = np.empty((rows, KS * 32), np.uint8)
    lib().orc_quantize_act(_p(x), rows, K, terms, _p(q), _p(s))
    return q, s


def dequant_act(q, s, K: int) -> np.ndarray:
    q, s = _c(q, np.uint8), _c(s, np.uint8)
    rows = q.shape[0]
    out = np.empty((rows, K), np.float32)
    lib().orc_dequant_act(_p(q), _p(s), rows, K, _p(out))
    return out


def e4m3_decode_table() -> np.ndarray:
    return np.array([lib().orc_e4m3_dec(c) for c in range(256)], np.float32)


def router_logits(x, wr) -> np.ndarray:
    x, wr = _c(x, np.uint16), _c(wr, np.uint16)
    T, H = x.shape
    E = wr.shape[0]
    out = np.empty((T, E), np.uint16)
    lib().orc_router_logits(_p(x), _p(wr), T, H, E, _p(out))
    return out


def topk_softmax(logits, bias, K: int):
    logits, bias = _c(logits, np.uint16), _c(bias, np.uint16)
    T, E = logits.shape
    ti = np.empty((T, K), np.int32)
    tw = np.empty((T, K), np.uint16)
    lib().orc_topk_softmax(_p(logits), _p(bias), T, E, K, _p(ti), _p(tw))
    return ti, tw


def route_index(ti, tw, E: int) -> dict:
    ti, tw = _c(ti, np.int32), _c(tw, np.uint16)
    T, K = ti.shape
    counts = np.empty(E, np.int32)
    offsets = np.empty(E + 1, np.int32)
    local_ids = np.empty((T, K), np.int32)
    row_token = np.empty(T * K + 1, np.int32)
    row_w = np.empty(T * K + 1, np.float32)
    dropped = lib().orc_route_index(_p(ti), _p(tw), T, K, E, _p(counts), _p(offsets),
                                    _p(local_ids), _p(row_token), _p(row_w))
    P = int(offsets[E])
    return {"counts": counts, "offsets": offsets, "local_ids": local_ids,
            "row_token": row_token[:P], "row_weight": row_w[:P], "dropped": dropped}


def moe_experts(d, x_norm, ti, tw, want_act=False):
    c = d.cfg
    x_norm = _c(x_norm, np.uint16)
    ti, tw = _c(ti, np.int32), _c(tw, np.uint16)
    T = x_norm.shape[0]
    out = np.empty((T, c.hidden), np.uint16)
    act = np.empty((T * c.top_k, c.intermediate), np.uint16) if want_act else None
    lib().orc_moe_experts(c.hidden, c.intermediate, c.n_experts, c.top_k, 7.0, 1.702,
                          _p(x_norm), _p(d.w1), _p(d.s1), _p(d.b1), _p(d.w2), _p(d.s2),
                          _p(d.b2), _p(ti), _p(tw), T, _p(out), _p(act))
    return (out, act) if want_act else out


def moe_forward(d, x_norm=None, forced=True, rows=None, act_quant=0):
    """getp-semantics MoE of a synth.MoeData layer.  Returns dict with
    e_agg, logits (router runs only), topk_i, topk_w.  `rows` selects a
    subset of tokens (each token's result depends on that token only).
    act_quant 1 / 2: the expert GEMMs see their activations as the FP4-MFMA
    variant quantises them (one / two MXFP8 terms)."""
    c = d.cfg
    x = d.x if x_norm is None else x_norm
    fi, fw = (d.forced_i, d.forced_w) if forced else (None, None)
    if rows is not None:
        x = x[rows]
        if fi is not None:
            fi, fw = fi[rows], fw[rows]
    x = _c(x, np.uint16)
    T = x.shape[0]
    E, K = c.n_experts, c.top_k
    e_agg = np.empty((T, c.hidden), np.uint16)
    lg = np.zeros((T, E), np.uint16)
    ti = np.empty((T, K), np.int32)
    tw = np.empty((T, K), np.uint16)
    if fi is not None:
        fi, fw = _c(fi, np.int32), _c(fw, np.uint16)
    lib().orc_moe_forward_aq(c.hidden, c.intermediate, E, K, 7.0, 1.702, _p(x), _p(d.router_w),
                             _p(d.router_b), _p(d.w1), _p(d.s1), _p(d.b1), _p(d.w2), _p(d.s2),
                             _p(d.b2), T, _p(fi), _p(fw), _p(e_agg), _p(lg), _p(ti), _p(tw),
                             act_quant)
    return {"e_agg": e_agg, "logits": lg if fi is None else None, "topk_i": ti, "topk_w": tw}


def rmsnorm(x, w) -> np.ndarray:
    x, w = _c(x, np.uint16), _c(w, np.uint16)
    out = np.empty_like(x)
    lib().orc_rmsnorm(_p(x), _p(w), x.shape[0], x.shape[1], _p(out))
    return out


def residual_add(x, e) -> np.ndarray:
    x = _c(x, np.uint16).copy()
    e = _c(e, np.uint16)
    lib().orc_residual_add(_p(x), _p(e), x.size)
    return x


class Fp32Engine:
    """The CPU engine's MoE block (run.cpp:657-748) over fp32 weights that are
    the exact dequantisation of a synth.MoeData layer."""

    def __init__(self, d):
        from synth import bf16_to_f32  # noqa: E402 (package dir on sys.path)
        c = d.cfg
        self.c = c
        H, D, E = c.hidden, c.intermediate, c.n_experts
        self.wr = bf16_to_f32(d.router_w).copy()
        self.br = bf16_to_f32(d.router_b).copy()
        self.w1 = dequant_f32(d.w1, d.s1, E * 2 * D * H)
        self.b1 = bf16_to_f32(d.b1).copy()
        self.w2 = dequant_f32(d.w2, d.s2, E * H * D)
        self.b2 = bf16_to_f32(d.b2).copy()
        self.scratch = np.empty(2 * D + 3 * D + H + E + 16, np.float32)

    def token(self, x_row_f32: np.ndarray) -> np.ndarray:
        c = self.c
        x = _c(x_row_f32, np.float32)
        out = np.empty(c.hidden, np.float32)
        lib().orc_moe_fp32_token(c.hidden, c.intermediate, c.n_experts, c.top_k, 7.0, _p(x),
                                 _p(self.wr), _p(self.br), _p(self.w1), _p(self.b1), _p(self.w2),
                                 _p(self.b2), _p(out), _p(self.scratch))
        return out


def num_threads() -> int:
    return lib().orc_num_threads()


# ------------------------------------------------------------ attention --

def f2h(x: float) -> int:
    return int(lib().orc_f2h(float(x)))


def kv_quantize_rows(x):
    """bf16 rows [n][kv_dim] -> (int8 codes [n][kv_dim], fp16 scale bits [n])
    (attention.hpp:582-628)."""
    x = _c(x, np.uint16)
    n, kv = x.shape
    q = np.empty((n, kv), np.int8)
    s = np.empty(n, np.uint16)
    L = lib()
    for i in range(n):
        L.orc_kv_quantize_row(_p(x[i]), kv, _p(q[i]), _p(s[i:i + 1]))
    return q, s


def attn_decode(q, kq, vq, ks, vs, kb, vb, sinks, pos, *, n_kv_heads: int, layer_idx: int,
                sliding_window: int, keep: int, prefix_rule: int = 0,
                phi_splits: int = 0, cache_bf16: bool = False) -> np.ndarray:
    """Decode attention over logical caches (attn_oracle.c): q bf16
    [B][n_heads][hd]; kq/vq int8 [B][cap][kv_dim]; ks/vs fp16 bits [B][cap];
    kb/vb bf16 [B][keep][kv_dim] or None; sinks bf16 [n_heads]; pos int32 [B].
    cache_bf16: kb/vb are the whole bf16 caches [B][cap][kv_dim] (kq..vs
    unused, may be None).  Returns fp32 [B][n_heads][hd]."""
    q = _c(q, np.uint16)
    B, NH, HD = q.shape
    if cache_bf16:
        cap = kb.shape[1]
        kq = vq = np.zeros((1,), np.int8)
        ks = vs = np.zeros((1,), np.uint16)
    else:
        cap = kq.shape[1]
    kq, vq = _c(kq, np.int8), _c(vq, np.int8)
    ks, vs = _c(ks, np.uint16), _c(vs, np.uint16)
    kb = None if kb is None else _c(kb, np.uint16)
    vb = None if vb is None else _c(vb, np.uint16)
    sinks, pos = _c(sinks, np.uint16), _c(pos, np.int32)
    out = np.empty((B, NH, HD), np.float32)
    rc = lib().orc_attn_decode(B, NH, n_kv_heads, HD, cap, layer_idx, sliding_window, keep,
                               prefix_rule, phi_splits, int(cache_bf16), _p(q), _p(kq), _p(vq), _p(ks), _p(vs),
                               _p(kb), _p(vb), _p(sinks), _p(pos), _p(out))
    if rc != 0:
        raise ValueError("orc_attn_decode: shape outside the restatement")
    return out


def rope_table(n_pos: int, base=150000.0, head_dim=64, scaling=32.0, init_ctx=4096.0):
    """cos, sin fp32 [n_pos][head_dim / 2] (run.cpp:422-503); gpt-oss
    defaults: rope_theta 150000, scaling factor 32, initial context 4096."""
    c = np.empty((n_pos, head_dim // 2), np.float32)
    s = np.empty_like(c)
    if lib().orc_rope_table(base, head_dim, scaling, init_ctx, n_pos, _p(c), _p(s)) != 0:
        raise ValueError("rope parameters fail run.cpp's assertion")
    return c, s


def qkv_bias_rope(qkv, bias, cos, sin, pos, nq=64, nkv=8, hd=64):
    qkv, bias = _c(qkv, np.uint16), _c(bias, np.uint16)
    cos, sin, pos = _c(cos, np.float32), _c(sin, np.float32), _c(pos, np.int32)
    B = qkv.shape[0]
    q = np.empty((B, nq, hd), np.uint16)
    k = np.empty((B, nkv * hd), np.uint16)
    v = np.empty((B, nkv * hd), np.uint16)
    lib().orc_qkv_bias_rope(_p(qkv), _p(bias), _p(cos), _p(sin), _p(pos), B, nq, nkv, hd, _p(q),
                            _p(k), _p(v))
    return q, k, v


def bias_residual(x, proj, bias):
    x = np.array(x, np.uint16, copy=True, order="C")
    proj, bias = _c(proj, np.uint16), _c(bias, np.uint16)
    lib().orc_bias_residual(_p(x), _p(proj), _p(bias), x.shape[0], x.shape[1])
    return x


def matmul_bf16(a, w):
    a, w = _c(a, np.uint16), _c(w, np.uint16)
    out = np.empty((a.shape[0], w.shape[0]), np.uint16)
    lib().orc_matmul_bf16(_p(a), _p(w), a.shape[0], w.shape[0], a.shape[1], _p(out))
    return out


def argmax_bf16(logits):
    logits = _c(logits, np.uint16)
    out = np.empty(logits.shape[0], np.int32)
    lib().orc_argmax_bf16(_p(logits), logits.shape[0], logits.shape[1], _p(out))
    return out
