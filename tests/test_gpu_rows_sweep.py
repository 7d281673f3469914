"""Seeded sweep of the row kernels' launch shapes (GPU): norm_modulate and
add_norm_modulate, one and two outputs, over row widths that select every
kernel form (partial rows, whole-workgroup rows, full C x 2048 rows), batch
counts on both sides of the segmented kernel's limit, token counts below and
above the resident workgroup count, and every modulation operand kind
(absent, table only, timestep row only, both; per batch item or per token).
Each case against the oracle within 1e-2 relative + 4e-3 absolute."""

import random

import pytest
import torch

from conftest import assert_close_bf16
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cases(n=40, seed=7):
    rng = random.Random(seed)
    widths = [8, 24, 64, 520, 1024, 2048, 3072, 4096, 6144, 8192, 16384]
    out = []
    for _ in range(n):
        d = rng.choice(widths)
        b = rng.choice([1, 1, 1, 2, 3, 66])
        t = rng.choice([1, 3, 17, 126, 513, 700]) if d <= 4096 else rng.choice([1, 5, 130])
        if b == 66:
            t = rng.choice([1, 2, 3])
        kinds = [rng.choice(["none", "tab", "emb", "both"]) for _ in range(5)]
        out.append((b, t, d, rng.choice([False, True]), rng.choice([False, True]), tuple(kinds), rng.randrange(1 << 16)))
    return out


def _operand(kind, row, table, emb_b, emb_t, per_token, b, t):
    """(ltxk operand, oracle value) for one modulation row of the given kind."""
    import ltxk

    if kind == "none":
        return None, None
    emb = emb_t if per_token else emb_b
    d = table.shape[-1]
    if kind == "tab":
        return ltxk.AdaRef(table.to(DEV), row), O.ada_value(table, row, None, b, t)
    if kind == "emb":
        zero = torch.zeros_like(table)
        return ltxk.AdaRef(None, row, emb.to(DEV), dim=d), O.ada_value(zero, row, emb, b, t)
    return ltxk.AdaRef(table.to(DEV), row, emb.to(DEV)), O.ada_value(table, row, emb, b, t)


@pytest.mark.parametrize("b,t,d,dual,per_token,kinds,seed", _cases())
def test_row_kernels_sweep(b, t, d, dual, per_token, kinds, seed):
    import ltxk

    g = torch.Generator().manual_seed(seed)
    bf = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(torch.bfloat16)  # noqa: E731
    x, f = bf(b, t, d), bf(b, t, d)
    table = bf(5, d, sc=0.05)
    emb_b, emb_t = bf(b, 1, 5 * d, sc=0.05), bf(b, t, 5 * d, sc=0.05)
    ops = [_operand(k, r, table, emb_b, emb_t, per_token, b, t) for r, k in enumerate(kinds)]
    (gate, wgate), (sh, wsh), (sc, wsc), (sh2, wsh2), (sc2, wsc2) = ops
    what = f"{b}x{t}x{d} dual={dual} per_token={per_token} kinds={kinds}"

    if dual:
        y1, y2 = ltxk.norm_modulate(x.to(DEV), shift=sh, scale=sc, shift2=sh2 or ltxk.AdaRef(table.to(DEV), 3),
                                    scale2=sc2)
        wsh2 = wsh2 if sh2 is not None else O.ada_value(table, 3, None, b, t)
        assert_close_bf16(y1, O.norm_modulate(x, wsh, wsc), what="norm_modulate y " + what)
        assert_close_bf16(y2, O.norm_modulate(x, wsh2, wsc2), what="norm_modulate y2 " + what)
    else:
        y = ltxk.norm_modulate(x.to(DEV), shift=sh, scale=sc)
        assert_close_bf16(y, O.norm_modulate(x, wsh, wsc), what="norm_modulate " + what)

    mask = (torch.arange(b) % 2 == 0).to(torch.bfloat16) if b > 1 else None
    args = dict(gate=gate, mask=None if mask is None else mask.to(DEV), shift=sh, scale=sc)
    if dual:
        args.update(shift2=sh2 or ltxk.AdaRef(table.to(DEV), 3), scale2=sc2)
        xo, y, y2 = ltxk.add_norm_modulate(x.to(DEV), f.to(DEV), **args)
    else:
        xo, y = ltxk.add_norm_modulate(x.to(DEV), f.to(DEV), **args)
    wxo, wy = O.add_norm_modulate(x, f, wgate, mask, wsh, wsc)
    assert torch.equal(xo.cpu(), wxo), "residual " + what
    assert_close_bf16(y, wy, what="add_norm_modulate y " + what)
    if dual:
        assert_close_bf16(y2, O.norm_modulate(wxo, wsh2, wsc2), what="add_norm_modulate y2 " + what)
