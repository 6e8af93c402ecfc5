import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    """The GPU device. GPU tests fail (not skip) when no GPU is visible, so a
    missing device or library never passes silently on the GPU box."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    return torch.device("cuda:0")


def close(actual, expected, atol=2e-2, rtol=1e-2, what=""):
    """fp16/bf16 output tolerance of the north star: atol 2e-2 / rtol 1e-2."""
    import torch

    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    ok = torch.isclose(a, e, atol=atol, rtol=rtol)
    if not bool(ok.all()):
        bad = (~ok).nonzero()[:5].tolist()
        diff = (a - e).abs().max().item()
        raise AssertionError(f"{what}: {int((~ok).sum())} mismatches, max abs diff {diff}, first at {bad}")
