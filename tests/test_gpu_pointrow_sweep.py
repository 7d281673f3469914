"""Seeded sweep of the row-wise elementwise entry points (GPU): head_gate (token-
major, contiguous (B, H, T, Dh) and transposed-view inputs; with and without
logits; with the perturbation blend), gated_residual (every gate kind, per batch
item or per token, with and without the batch mask) and modulate.  Each case
against the oracle within 1e-2 relative + 4e-3 absolute."""

import random

import pytest
import torch

from conftest import assert_close_bf16
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cases(n=30, seed=23):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        heads, dh = rng.choice([(1, 8), (4, 64), (32, 64), (32, 128), (2, 128), (16, 16)])
        out.append((rng.choice([1, 2, 3]), rng.choice([1, 7, 126, 300]), heads, dh,
                    rng.choice(["tokens", "bhtd", "view"]), rng.choice([False, True]), rng.choice([False, True]),
                    rng.choice(["none", "tab", "emb", "both"]), rng.choice([False, True]), rng.randrange(1 << 16)))
    return out


@pytest.mark.parametrize("b,t,heads,dh,layout,logits,blend,gkind,per_token,seed", _cases())
def test_pointrow_sweep(b, t, heads, dh, layout, logits, blend, gkind, per_token, seed):
    import ltxk

    g = torch.Generator().manual_seed(seed)
    bf = lambda *s, sc=1.0: (torch.randn(*s, generator=g) * sc).to(torch.bfloat16)  # noqa: E731
    d = heads * dh
    what = f"b={b} t={t} heads={heads} dh={dh} layout={layout} logits={logits} blend={blend} gate={gkind}"

    # head gate
    attn = bf(b, t, d)
    lg = bf(b, t, heads) if logits else None
    v = bf(b, t, d) if blend else None
    mask = (torch.arange(b) % 2 == 1).to(torch.bfloat16) if blend else None
    if layout == "tokens":
        a_dev = attn.to(DEV)
    elif layout == "bhtd":
        a_dev = attn.view(b, t, heads, dh).transpose(1, 2).contiguous().to(DEV)
    else:
        a_dev = attn.to(DEV).view(b, t, heads, dh).transpose(1, 2)
    got = ltxk.head_gate(a_dev, None if lg is None else lg.to(DEV), v=None if v is None else v.to(DEV),
                         mask=None if mask is None else mask.to(DEV), heads=heads)
    src = attn if v is None else torch.where(mask.view(b, 1, 1) != 0, attn, v)
    want = O.head_gate(src, lg, heads) if lg is not None else src
    assert_close_bf16(got.reshape(b, t, d), want, what="head_gate " + what)

    # gated residual and modulate with every operand kind
    x, f = bf(b, t, d), bf(b, t, d)
    table = bf(3, d, sc=0.05)
    emb = bf(b, t if per_token else 1, 3 * d, sc=0.05)
    zero = torch.zeros_like(table)

    def operand(row):
        if gkind == "none":
            return None, None
        if gkind == "tab":
            return ltxk.AdaRef(table.to(DEV), row), O.ada_value(table, row, None, b, t)
        if gkind == "emb":
            return ltxk.AdaRef(None, row, emb.to(DEV), dim=d), O.ada_value(zero, row, emb, b, t)
        return ltxk.AdaRef(table.to(DEV), row, emb.to(DEV)), O.ada_value(table, row, emb, b, t)

    (gate, wgate), (sh, wsh), (sc, wsc) = operand(0), operand(1), operand(2)
    rmask = (torch.arange(b) % 2 == 0).to(torch.bfloat16) if b > 1 else None
    got = ltxk.gated_residual(x.to(DEV), f.to(DEV), gate=gate, mask=None if rmask is None else rmask.to(DEV))
    assert torch.equal(got.cpu(), O.gated_residual(x, f, wgate, rmask)), "gated_residual " + what
    got = ltxk.modulate(x.to(DEV), sh, sc)
    assert_close_bf16(got, O.modulate(x, wsh, wsc), what="modulate " + what)
