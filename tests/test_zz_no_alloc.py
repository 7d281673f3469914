"""ltxk_guide_noalloc (the library's own partial-sum array, no workspace
argument) against ltxk_guide with a caller workspace, through the C ABI:
denoised, the per-pass x0 and the Euler-stepped latent must be bit-equal,
on two calls in a row, the second with a smaller input (so the second call
reads only partials it wrote itself)."""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _call(lib, fn, rows, dim, seed, rescale):
    import ltxk

    g = torch.Generator(device=DEV).manual_seed(seed)
    lat = torch.randn(rows, dim, device=DEV, generator=g).to(torch.bfloat16)
    vel = torch.randn(4, rows, dim, device=DEV, generator=g).to(torch.bfloat16)
    ts = torch.rand(4, rows, 1, device=DEV, generator=g) * 0.9 + 0.05
    den = torch.empty_like(lat)
    x0 = torch.empty_like(vel)
    nxt = torch.empty_like(lat)
    gp = ltxk.Guidance(3.0, 1.0, 3.0, rescale)
    stream = torch.cuda.current_stream().cuda_stream
    args = [den.data_ptr(), x0.data_ptr(), nxt.data_ptr(), lat.data_ptr(), vel.data_ptr(), ts.data_ptr(), rows, 1,
            rows, dim, ctypes.byref(gp), ctypes.c_float(0.7), ctypes.c_float(-0.05)]
    if fn == "ws":
        nb = int(lib.ltxk_guide_workspace_bytes(rows * dim))
        ws = torch.empty(max(nb, 8), dtype=torch.uint8, device=DEV)
        rc = lib.ltxk_guide(*args, ws.data_ptr(), nb, stream)
    else:
        rc = lib.ltxk_guide_noalloc(*args, stream)
    assert rc == 0, ltxk.last_error()
    torch.cuda.synchronize()
    return den, x0, nxt


@pytest.mark.parametrize("rescale", [0.7, 0.0])
def test_noalloc_matches_workspace_entry(rescale):
    import ltxk

    lib = ltxk.load()
    # a large call first, then a smaller one: the partials of the first stay in
    # the shared array, and the second must neither read nor need them
    for rows, dim, seed in ((6144, 128, 1), (300, 64, 2)):
        want = _call(lib, "ws", rows, dim, seed, rescale)
        got = _call(lib, "noalloc", rows, dim, seed, rescale)
        for name, a, b in zip(("denoised", "x0", "next"), got, want):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"{name} differs at {rows}x{dim}"

