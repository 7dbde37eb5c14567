"""HIP-graph capture of the forward call (the serving-loop use: one capture,
many replays).  A call allocates nothing, issues no memset and does not
synchronise, and each call's index kernel clears the routing histogram for
the next, so a captured forward must replay exactly what an eager call
computes, also when eager calls of other sizes run on the same workspace
between replays.  Every replay is checked bit for bit against the eager
result on the same inputs (the path is deterministic)."""
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


@pytest.mark.parametrize("name,path", [("c1_20b_decode", "auto"), ("c2_20b_zipf", "auto"),
                                       ("c0_tiny", "small"), ("c1_20b_decode", "fp4")])
def test_graph_replays_match_eager(gpu, name, path):
    import torch
    import gptoss_moe
    d = synth.make_data(name)
    T = d.cfg.tokens
    layer = gptoss_moe.MoeLayer.from_numpy(d, device=gpu, pack_fp4=path == "fp4")
    x = _dev(d.x, gpu)
    fi = None if d.forced_i is None else _dev(d.forced_i, gpu)
    fw = None if d.forced_w is None else _dev(d.forced_w, gpu)
    x_other = x[torch.randperm(T, generator=torch.Generator().manual_seed(5)).to(gpu)].contiguous()

    want = layer.forward(x, forced_i=fi, forced_w=fw, path=path).clone()
    want_other = layer.forward(x_other, forced_i=fi, forced_w=fw, path=path).clone()

    xin = x.clone()
    out = torch.empty_like(x)
    graph = layer.capture_forward(xin, out, fi, fw, path=path)
    for rep in range(3):
        # eager calls of other sizes on the same workspace between replays
        n = max(1, T // (rep + 2))
        layer.forward(x_other[:n], forced_i=None if fi is None else fi[:n],
                      forced_w=None if fw is None else fw[:n], path=path)
        torch.cuda.synchronize()
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep} differs from the eager forward"
    # the graph reads the captured input buffer: new contents, new result
    xin.copy_(x_other)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want_other), "replay on new inputs differs from the eager forward"
