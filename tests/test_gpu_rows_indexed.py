"""Indexed AdaLN operands (GPU): one embedding row per distinct timestep and a
per-token int32 index (ltxk_ada.emb_index), as LTXModel builds them for a
keyframe-conditioned step, in every row kernel and launch form.  Each output
equals the same kernel fed the per-token embeddings the index stands for (the
reference's layout, ltx_dit.py:146-150) bit for bit, and the oracle within the
bf16 bar; indexes outside [0, rows) read the last row (the kernels clamp)."""

import random

import pytest
import torch

from conftest import assert_close_bf16
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bf(shape, gen, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.bfloat16)


def _cases(n=16, seed=11):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        d = rng.choice([64, 520, 2048, 3072, 4096])
        b = rng.choice([1, 1, 2, 3])
        t = rng.choice([5, 17, 126, 700]) if d <= 2048 else rng.choice([5, 126, 300])
        out.append((b, t, d, rng.choice(["norm", "norm2", "add", "add2", "residual", "modulate"]), rng.randrange(1 << 16)))
    return out


@pytest.mark.parametrize("b,t,d,op,seed", _cases())
def test_indexed_operands_equal_per_token_operands(b, t, d, op, seed):
    import ltxk

    g = torch.Generator().manual_seed(seed)
    n, u = 9, 3                                     # table rows; distinct timesteps
    table = bf((n, d), g, 0.05)
    rows = bf((1, u, n * d), g, 0.05)              # the de-duplicated embeddings
    idx = torch.randint(0, u, (b * t,), generator=g, dtype=torch.int32)
    idx[:: max(1, (b * t) // 7)] = u + 5            # out of range: clamped to the last row
    idx[1::11] = -3
    clamped = torch.where((idx < 0) | (idx >= u), torch.full_like(idx, u - 1), idx)
    per_tok = rows[0, clamped.long()].reshape(b, t, n * d)   # what the index stands for
    index = ltxk.TimestepIndex(idx.to(DEV), u)
    tab, rdev, pdev = table.to(DEV), rows.to(DEV), per_tok.to(DEV)

    def ind(row):
        return ltxk.AdaRef(tab, row, rdev, index=index)

    def tok(row):
        return ltxk.AdaRef(tab, row, pdev)

    def val(row):
        return O.ada_value(table, row, per_tok, b, t)

    x, f = bf((b, t, d), g), bf((b, t, d), g)
    xd, fd = x.to(DEV), f.to(DEV)
    if op in ("norm", "norm2"):
        two = op == "norm2"
        a = ltxk.norm_modulate(xd, shift=ind(1), scale=ind(0), shift2=ind(3) if two else None,
                               scale2=ind(2) if two else None)
        w = ltxk.norm_modulate(xd, shift=tok(1), scale=tok(0), shift2=tok(3) if two else None,
                               scale2=tok(2) if two else None)
        a, w = (a if two else (a,)), (w if two else (w,))
        want = [O.norm_modulate(x, val(1), val(0))] + ([O.norm_modulate(x, val(3), val(2))] if two else [])
    elif op in ("add", "add2"):
        two = op == "add2"
        kw = dict(shift2=ind(7), scale2=ind(6)) if two else {}
        a = ltxk.add_norm_modulate(xd.clone(), fd, gate=ind(5), shift=ind(1), scale=ind(0), **kw)
        kw = dict(shift2=tok(7), scale2=tok(6)) if two else {}
        w = ltxk.add_norm_modulate(xd.clone(), fd, gate=tok(5), shift=tok(1), scale=tok(0), **kw)
        xo, y = O.add_norm_modulate(x, f, val(5), None, val(1), val(0))
        want = [xo, y] + ([O.norm_modulate(xo, val(7), val(6))] if two else [])
    elif op == "residual":
        a = (ltxk.gated_residual(xd, fd, gate=ind(4)),)
        w = (ltxk.gated_residual(xd, fd, gate=tok(4)),)
        want = [O.gated_residual(x, f, val(4))]
    else:
        a = (ltxk.modulate(xd, ind(1), ind(0)),)
        w = (ltxk.modulate(xd, tok(1), tok(0)),)
        want = [O.modulate(x, val(1), val(0))]
    assert len(a) == len(w) == len(want)
    for i, (got, same, ref) in enumerate(zip(a, w, want)):
        assert torch.equal(got.view(torch.int16), same.view(torch.int16)), (op, i)
        assert_close_bf16(got.cpu(), ref, what=f"{op} output {i} {b}x{t}x{d}")
