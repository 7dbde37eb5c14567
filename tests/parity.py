"""Shared comparison helpers for the parity tests."""
import numpy as np

from synth import bf16_to_f32

# Layer-output tolerance of the target (fp32 accumulate, bf16 out): max-abs
# 2e-2 and relative L2 1e-2.  With the benchmark's weight distributions the
# output magnitude is ~1e3 (one bf16 ulp there is 4-64), so the max-abs bound
# is applied to |got - want| / max(1, rms(want), |want|) elementwise: an
# absolute bound for O(1) outputs, a relative one for large ones.
MAX_ABS = 2e-2
REL_L2 = 1e-2


def compare(got_bf16, want_bf16):
    g = bf16_to_f32(np.asarray(got_bf16).view(np.uint16)).astype(np.float64)
    w = bf16_to_f32(np.asarray(want_bf16).view(np.uint16)).astype(np.float64)
    assert g.shape == w.shape
    d = np.abs(g - w)
    scale = max(1.0, float(np.sqrt(np.mean(w * w)))) if w.size else 1.0
    norm = d / np.maximum(scale, np.abs(w))
    return {
        "max_abs": float(d.max()) if d.size else 0.0,
        "max_abs_norm": float(norm.max()) if d.size else 0.0,
        "rel_l2": float(np.linalg.norm(g - w) / max(np.linalg.norm(w), 1e-30)),
        "frac_exact": float(np.mean(d == 0)) if d.size else 1.0,
        "scale": scale,
        "finite": bool(np.isfinite(g).all()),
    }


# Every layer-output comparison of the session (name, absolute max-abs,
# normalised max-abs, rel-L2); tests/conftest.py writes them to
# gpurun_out/parity_metrics.json after a GPU session.
RECORD = []


def assert_close(got_bf16, want_bf16, what=""):
    m = compare(got_bf16, want_bf16)
    RECORD.append({"what": what, "max_abs": m["max_abs"], "max_abs_norm": m["max_abs_norm"],
                   "rel_l2": m["rel_l2"], "frac_exact": m["frac_exact"]})
    assert m["finite"], f"{what}: non-finite output"
    assert m["max_abs_norm"] <= MAX_ABS and m["rel_l2"] <= REL_L2, (
        f"{what}: max_abs {m['max_abs']:.4g} (normalised {m['max_abs_norm']:.4g} <= {MAX_ABS}), "
        f"rel_l2 {m['rel_l2']:.4g} (<= {REL_L2}); {m}")
    return m
