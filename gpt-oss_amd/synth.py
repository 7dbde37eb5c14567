"""Seeded synthetic MoE layers for the configurations the benchmark and the
parity tests use.  Pure numpy; bf16 values are carried as uint16 bit patterns.

Distributions (one fixed seed per configuration, 0x6F550000 + index):
  x        bf16 ~ N(0, 1)                     [T][H]
  router_w bf16 ~ N(0, 0.02)                  [E][H]
  router_b bf16 ~ N(0, 0.01)                  [E]
  w1, w2   uniform random E2M1 codes, two per byte (low nibble = even element)
  scales   e8m0 uniform in [120, 128]
  b1, b2   bf16 ~ N(0, 0.01)
Routing: "router" (the layer's own router), or forced: "uniform" (k distinct
experts uniformly at random) / "zipf" (k distinct experts drawn without
replacement with p(e) ~ (rank(e)+1)^-1.2 over a seeded permutation of the
experts); forced weights are the softmax, over the chosen experts, of the
router scores (float64 x . Wr^T + b), rounded to bf16.
"""
from __future__ import annotations

import dataclasses

import numpy as np

SWIGLU_LIMIT = 7.0
SWIGLU_ALPHA = 1.702


@dataclasses.dataclass(frozen=True)
class MoeConfig:
    name: str
    hidden: int
    intermediate: int
    n_experts: int
    top_k: int
    tokens: int
    routing: str  # "router" | "uniform" | "zipf"
    seed: int

    @property
    def pairs(self) -> int:
        return self.tokens * self.top_k


CONFIGS = {
    "c0_tiny": MoeConfig("c0_tiny", 128, 128, 4, 2, 8, "router", 0x6F550000),
    "c1_20b_decode": MoeConfig("c1_20b_decode", 2880, 2880, 32, 4, 256, "router", 0x6F550001),
    "c2_20b_zipf": MoeConfig("c2_20b_zipf", 2880, 2880, 32, 4, 512, "zipf", 0x6F550002),
    "c3a_120b_decode": MoeConfig("c3a_120b_decode", 2880, 2880, 128, 4, 1024, "uniform", 0x6F550003),
    "c3b_120b_prefill": MoeConfig("c3b_120b_prefill", 2880, 2880, 128, 4, 4096, "router", 0x6F550004),
    # test-only: many rows per expert at a small shape (large-M GEMM path, ragged tiles)
    "t_large_m": MoeConfig("t_large_m", 384, 320, 6, 2, 700, "router", 0x6F550010),
    # test-only: H = 1.5 weight blocks of 128 rows, D = 3.5 packed k groups of 128
    "t_odd_n": MoeConfig("t_odd_n", 192, 448, 5, 2, 40, "router", 0x6F550011),
}


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even, NaN kept quiet."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x0040).astype(np.uint16)
    return r


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


@dataclasses.dataclass
class MoeData:
    cfg: MoeConfig
    x: np.ndarray          # uint16 [T][H]
    router_w: np.ndarray   # uint16 [E][H]
    router_b: np.ndarray   # uint16 [E]
    w1: np.ndarray         # uint8  [E * 2D*H/2]
    s1: np.ndarray         # uint8  [E * 2D*H/32]
    b1: np.ndarray         # uint16 [E][2D]
    w2: np.ndarray         # uint8  [E * H*D/2]
    s2: np.ndarray         # uint8  [E * H*D/32]
    b2: np.ndarray         # uint16 [E][H]
    forced_i: np.ndarray | None = None  # int32 [T][k]
    forced_w: np.ndarray | None = None  # uint16 [T][k]

    @property
    def weight_bytes(self) -> int:
        return sum(a.nbytes for a in (self.w1, self.s1, self.b1, self.w2, self.s2, self.b2))


def _normal_bf16(rng: np.random.Generator, shape, sigma: float) -> np.ndarray:
    return f32_to_bf16(rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma))


def make_weights(rng: np.random.Generator, H: int, D: int, E: int):
    n1 = 2 * D * H
    n2 = H * D
    w1 = rng.integers(0, 256, size=E * n1 // 2, dtype=np.uint8)
    s1 = rng.integers(120, 129, size=E * n1 // 32, dtype=np.uint8)
    b1 = _normal_bf16(rng, (E, 2 * D), 0.01)
    w2 = rng.integers(0, 256, size=E * n2 // 2, dtype=np.uint8)
    s2 = rng.integers(120, 129, size=E * n2 // 32, dtype=np.uint8)
    b2 = _normal_bf16(rng, (E, H), 0.01)
    return w1, s1, b1, w2, s2, b2


def router_scores_f64(x: np.ndarray, wr: np.ndarray, br: np.ndarray) -> np.ndarray:
    return bf16_to_f32(x).astype(np.float64) @ bf16_to_f32(wr).astype(np.float64).T + \
        bf16_to_f32(br).astype(np.float64)[None, :]


def forced_routing(rng: np.random.Generator, scores: np.ndarray, K: int, kind: str):
    T, E = scores.shape
    if kind == "uniform":
        p = None
    elif kind == "zipf":
        perm = rng.permutation(E)
        p = np.empty(E)
        p[perm] = 1.0 / np.arange(1, E + 1) ** 1.2
        p /= p.sum()
    else:
        raise ValueError(kind)
    idx = np.empty((T, K), dtype=np.int32)
    for t in range(T):
        idx[t] = rng.choice(E, size=K, replace=False, p=p)
    sel = np.take_along_axis(scores, idx.astype(np.int64), axis=1)
    sel = np.exp(sel - sel.max(axis=1, keepdims=True))
    w = sel / sel.sum(axis=1, keepdims=True)
    return idx, f32_to_bf16(w.astype(np.float32))


def make_router_inputs(cfg: MoeConfig | str):
    """x, router weight and router bias of make_data(cfg), without the expert
    weights (the same generator stream: these are drawn first)."""
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    rng = np.random.Generator(np.random.PCG64(cfg.seed))
    H, E, T = cfg.hidden, cfg.n_experts, cfg.tokens
    x = _normal_bf16(rng, (T, H), 1.0)
    wr = _normal_bf16(rng, (E, H), 0.02)
    br = _normal_bf16(rng, (E,), 0.01)
    return x, wr, br


def make_data(cfg: MoeConfig | str, tokens: int | None = None) -> MoeData:
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    if tokens is not None:
        cfg = dataclasses.replace(cfg, tokens=tokens)
    rng = np.random.Generator(np.random.PCG64(cfg.seed))
    H, D, E, K, T = cfg.hidden, cfg.intermediate, cfg.n_experts, cfg.top_k, cfg.tokens
    x = _normal_bf16(rng, (T, H), 1.0)
    wr = _normal_bf16(rng, (E, H), 0.02)
    br = _normal_bf16(rng, (E,), 0.01)
    w1, s1, b1, w2, s2, b2 = make_weights(rng, H, D, E)
    d = MoeData(cfg, x, wr, br, w1, s1, b1, w2, s2, b2)
    if cfg.routing != "router":
        d.forced_i, d.forced_w = forced_routing(rng, router_scores_f64(x, wr, br), K, cfg.routing)
    return d


def algorithmic_bytes(cfg: MoeConfig, active_experts: int | None = None) -> int:
    """HBM bytes one layer call must move at minimum: the active experts'
    MXFP4 weights + scales + biases, the router, activations in and out."""
    H, D, E, T = cfg.hidden, cfg.intermediate, cfg.n_experts, cfg.tokens
    act = E if active_experts is None else active_experts
    per_expert = (2 * D * H) // 2 + (2 * D * H) // 32 + (H * D) // 2 + (H * D) // 32 + 2 * (2 * D + H)
    return act * per_expert + 2 * H * E + 2 * E + 2 * T * H + 2 * T * H


def algorithmic_flops(cfg: MoeConfig, pairs: int | None = None) -> int:
    H, D, E, T = cfg.hidden, cfg.intermediate, cfg.n_experts, cfg.tokens
    p = cfg.pairs if pairs is None else pairs
    return p * (2 * H * 2 * D + 2 * D * H) + T * 2 * H * E
