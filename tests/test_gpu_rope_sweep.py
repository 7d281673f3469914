"""Seeded sweep of ltxk_qk_norm_rope's launch shapes (GPU): head counts and
head sizes that select every thread-per-row geometry, no / full / compact
(1 or 3 axis) tables, with and without the q/k norm weights, q alone, q and
k of different lengths, and q and k sharing tables (the paired path).  Each
case against the oracle's fp32 norm + rotation on the same (full) tables,
within 1e-2 relative + 4e-3 absolute."""

import random

import pytest
import torch

from conftest import assert_close_bf16
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cases(n=30, seed=11):
    rng = random.Random(seed)
    out = []
    while len(out) < n:
        heads = rng.choice([1, 2, 4, 8, 16, 32])
        dh = rng.choice([16, 32, 64, 128])
        if heads * dh > 4096:
            continue
        tables = rng.choice(["none", "full", "compact1", "compact3"])
        grid = rng.choice([(1, 1, 1), (2, 3, 5), (3, 10, 10), (2, 16, 24)])
        out.append((rng.choice([1, 2]), heads, dh, tables, grid, rng.choice([False, True]),
                    rng.choice(["none", "other", "paired"]), rng.randrange(1 << 16)))
    return out


def _tables(kind, b, grid, d, heads):
    """(ltxk pe argument, full cos, full sin on the CPU) for `kind` on a grid."""
    import ltx_nn

    if kind == "none":
        return None, None, None
    f, h, w = grid
    if kind.endswith("3"):
        pos, max_pos = O.video_positions(b, f, h, w, 24.0), [20, 2048, 2048]
    else:
        pos, max_pos = O.audio_positions(b, f * h * w), [f * h * w]
    pos = pos.to(DEV)
    c, s = ltx_nn.precompute_freqs_cis(pos, d, torch.bfloat16, max_pos=max_pos, num_attention_heads=heads)
    if kind == "full":
        return (c, s), c.cpu(), s.cpu()
    cp = ltx_nn.precompute_freqs_cis_compact(pos, d, torch.bfloat16, max_pos=max_pos, num_attention_heads=heads)
    return cp, c.cpu(), s.cpu()


@pytest.mark.parametrize("b,heads,dh,tables,grid,weights,kmode,seed", _cases())
def test_qk_norm_rope_sweep(b, heads, dh, tables, grid, weights, kmode, seed):
    import ltxk

    d = heads * dh
    t = grid[0] * grid[1] * grid[2]
    g = torch.Generator().manual_seed(seed)
    bf = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)  # noqa: E731
    q = bf(b, t, d)
    wq = bf(d) if weights else None
    pe, c, s = _tables(tables, b, grid, d, heads)
    what = f"b={b} heads={heads} dh={dh} tables={tables} grid={grid} weights={weights} k={kmode}"
    k = wk = kpe = kc = ks = None
    if kmode == "paired":
        k, wk, kpe, kc, ks = bf(b, t, d), bf(d) if weights else None, pe, c, s
    elif kmode == "other":
        kgrid = (1, 2, 3)
        k, wk = bf(b, 6, d), bf(d) if weights else None
        kpe, kc, ks = _tables(tables, b, kgrid, d, heads)
    qd = q.to(DEV)
    kd = k.to(DEV) if k is not None else None
    ltxk.qk_norm_rope(qd, kd, heads, dh, q_weight=None if wq is None else wq.to(DEV),
                      k_weight=None if wk is None else wk.to(DEV), q_pe=pe, k_pe=kpe)
    assert_close_bf16(qd, O.qk_norm_rope(q, wq, c, s), what="q " + what)
    if k is not None:
        assert_close_bf16(kd, O.qk_norm_rope(k, wk, kc, ks), what="k " + what)
