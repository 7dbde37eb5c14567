"""gptoss_moe_forward_noalloc (the entry point that allocates nothing and
works in the library's per-GPU device array) against gptoss_moe_forward on
a caller workspace: bit-identical outputs and routing, on two calls in a
row, the second with fewer tokens (the array keeps the first call's
contents)."""
import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu


def _dev(a, device):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to(device)


@pytest.mark.parametrize("path", ["auto", "small"])
def test_noalloc_matches_workspace_entry(gpu, path):
    import torch
    import gptoss_moe
    d = synth.make_data("c1_20b_decode")
    layer = gptoss_moe.MoeLayer.from_numpy(d, device=gpu)
    x = _dev(d.x, gpu)
    for T in (256, 37):  # second call smaller
        xs = x[:T].contiguous()
        want = layer.forward(xs, path=path)
        got = torch.full_like(xs, 0x7FC1)  # NaN pattern: every element must be written
        layer.forward_noalloc(xs, got, path=path)
        torch.cuda.synchronize()
        w = want.cpu().numpy().view(np.uint16)
        g = got.cpu().numpy().view(np.uint16)
        n_bad = int((w != g).sum())
        print(f"noalloc path={path} T={T}: {n_bad} differing elements", flush=True)
        assert n_bad == 0


def test_noalloc_forced_routing_and_residual(gpu):
    import torch
    import gptoss_moe
    d = synth.make_data("c2_20b_zipf")
    layer = gptoss_moe.MoeLayer.from_numpy(d, device=gpu)
    x = _dev(d.x, gpu)
    fi = _dev(d.forced_i, gpu)
    fw = _dev(d.forced_w, gpu)
    for T in (512, 100):
        xs, fis, fws = x[:T].contiguous(), fi[:T].contiguous(), fw[:T].contiguous()
        base = _dev(d.x[::-1][:T].copy(), gpu)
        want = base.clone()
        layer.forward(xs, want, fis, fws, residual=True)
        got = base.clone()
        layer.forward_noalloc(xs, got, fis, fws, residual=True)
        torch.cuda.synchronize()
        assert torch.equal(want, got), f"T={T}"
