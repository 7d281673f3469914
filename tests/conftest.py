import pathlib
import sys

import pytest

REPO = pathlib.Path(__file__).resolve().parent.parent
PKG = REPO / "ltx-nv_amd"
GOLDEN = REPO / "tests" / "golden"
for p in (str(REPO), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); parity tests of the HIP kernels")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


# Tolerance of the elementwise bf16 outputs against the fp32-accumulated oracle.
RTOL = 1e-2
ATOL = 4e-3


def assert_close_bf16(got, want, rtol=RTOL, atol=ATOL, what=""):
    """|got - want| <= atol + rtol*|want| elementwise (both compared in fp32)."""
    import torch

    g = got.detach().float().cpu()
    w = want.detach().float().cpu()
    assert g.shape == w.shape, f"{what}: shape {tuple(g.shape)} vs {tuple(w.shape)}"
    d = (g - w).abs()
    bad = d > atol + rtol * w.abs()
    if bool(bad.any()) or bool(torch.isnan(g).any() != torch.isnan(w).any()):
        i = int(torch.argmax((d - (atol + rtol * w.abs())).flatten()))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{d.numel()} outside {atol}+{rtol}|x|; worst at {i}: "
            f"got {g.flatten()[i].item()} want {w.flatten()[i].item()}"
        )
    return d


def bf16_from_bits(a):
    import numpy as np
    import torch

    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)
