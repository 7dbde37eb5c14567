import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "gpt-oss_amd"), os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI on cuda:0)")


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def pytest_sessionfinish(session, exitstatus):
    """After a session that compared layer outputs (the GPU parity tests),
    keep their absolute and normalised max-abs and rel-L2 beside the pass
    line: gpurun_out/parity_metrics.json (the folder a GPU run returns)."""
    try:
        import json
        import parity
    except ImportError:
        return
    if not parity.RECORD:
        return
    out = os.path.join(ROOT, "gpurun_out")
    os.makedirs(out, exist_ok=True)
    with open(os.path.join(out, "parity_metrics.json"), "w") as f:
        json.dump(parity.RECORD, f, indent=1)
