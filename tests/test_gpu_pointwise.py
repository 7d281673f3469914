"""Parity of GELU-tanh, gated residual at the config-3 shapes, and the Euler /
x0 updates (GPU)."""

import numpy as np
import pytest
import torch

from conftest import assert_close_bf16
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bf(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def test_config3_gelu_full_shape():
    """h [6144, 16384] ~ N(0,1)."""
    import ltxk

    h = bf((6144, 16384), 50)
    y = ltxk.gelu_tanh(h.to(DEV))
    d = assert_close_bf16(y, O.gelu_tanh(h), what="gelu config3")
    assert (d == 0).float().mean() > 0.99


def test_gelu_range_tails_and_odd_sizes():
    import ltxk

    x = torch.linspace(-12, 12, 200003).to(torch.bfloat16)  # n % 8 != 0: scalar tail
    assert_close_bf16(ltxk.gelu_tanh(x.to(DEV)), O.gelu_tanh(x), what="gelu range")
    special = torch.tensor([0.0, -0.0, 1e-30, -1e-30, 60.0, -60.0, float("inf"), float("-inf")],
                           dtype=torch.bfloat16)
    got = ltxk.gelu_tanh(special.to(DEV)).cpu().float()
    assert got[0] == 0 and got[4] == 60.0 and abs(got[5]) == 0 and got[6] == float("inf")
    for n in (1, 7, 8, 9, 4095):
        t = bf((n,), n)
        assert_close_bf16(ltxk.gelu_tanh(t.to(DEV)), O.gelu_tanh(t), what=f"gelu n={n}")
    # in place
    t = bf((3, 1000), 51)
    td = t.to(DEV)
    ltxk.gelu_tanh(td, out=td)
    assert_close_bf16(td, O.gelu_tanh(t), what="gelu in place")


def test_config3_gated_residual_full_shape():
    """x, f [6144, 4096] ~ N(0,1), gate [4096] ~ N(0, 0.02^2): out = x + gate*f."""
    import ltxk

    x, f = bf((6144, 4096), 52), bf((6144, 4096), 53)
    gate = bf((4096,), 54, 0.02)
    out = ltxk.gated_residual(x.to(DEV), f.to(DEV), ltxk.AdaRef(gate.to(DEV), 0))
    assert torch.equal(out.cpu(), O.gated_residual(x, f, gate))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_euler_update(dtype):
    import ltxk

    g = torch.Generator().manual_seed(55)
    x = torch.randn(1003, generator=g).to(dtype)
    v = torch.randn(1003, generator=g).to(dtype)
    xd = x.to(DEV)
    ltxk.euler_update(xd, v.to(DEV), -0.125)
    if dtype == torch.float32:
        assert np.array_equal(xd.cpu().numpy(), O.euler_update_f32(x.numpy(), v.numpy(), -0.125))
    else:
        want = (x.float() + (v.float() * -0.125)).to(torch.bfloat16)
        assert torch.equal(xd.cpu(), want)


def test_euler_step_and_x0_match_reference_formula():
    import ltxk

    s, d = bf((2, 6144, 128), 56), bf((2, 6144, 128), 57)
    for sigma, dt in ((1.0, -0.05), (0.5, -0.125), (0.1, -0.1)):
        got = ltxk.euler_step(s.to(DEV), d.to(DEV), sigma, dt).cpu()
        assert torch.equal(got, O.euler_step(s, d, sigma, dt)), (sigma, dt)
    ts_tok = torch.rand(2, 6144, 1, generator=torch.Generator().manual_seed(58))
    ts_bat = torch.tensor([0.5, 0.25]).view(2, 1, 1)
    for ts in (ts_tok, ts_bat):
        got = ltxk.x0(s.to(DEV), d.to(DEV), ts.to(DEV)).cpu()
        assert torch.equal(got, O.x0(s, d, ts))
