"""Parity of the row kernels (norm/modulate/residual/head gate) with the oracle (GPU).

Inputs are seeded bf16 tensors made on the CPU, copied to the device; the
oracle evaluates the same formula in fp32 on the CPU and rounds once.
Tolerance: 1e-2 relative + 4e-3 absolute per element (bf16 outputs)."""

import pytest
import torch

from conftest import assert_close_bf16
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bf(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def test_config1_rmsnorm_modulate_full_shape():
    """x [6144, 4096] ~ N(0,1) (seed 0); shift, scale [4096] ~ N(0, 0.02^2) (seed 1)."""
    import ltxk

    x = bf((6144, 4096), 0)
    g = torch.Generator().manual_seed(1)
    shift = (torch.randn(4096, generator=g) * 0.02).to(torch.bfloat16)
    scale = (torch.randn(4096, generator=g) * 0.02).to(torch.bfloat16)
    y = ltxk.norm_modulate(x.to(DEV), shift=ltxk.AdaRef(shift.to(DEV), 0), scale=ltxk.AdaRef(scale.to(DEV), 0))
    want = O.norm_modulate(x, shift, scale)
    d = assert_close_bf16(y, want, what="config1")
    # fp32 single rounding on both sides: nearly every element identical
    assert (d == 0).float().mean() > 0.99


@pytest.mark.parametrize("b,t,d", [(1, 5, 8), (2, 33, 64), (1, 126, 2048), (3, 17, 3072), (1, 4, 8192),
                                   (2, 7, 24), (1, 300, 4096), (1, 2, 16384), (3, 41, 1024), (2, 9, 512),
                                   (5, 3, 128), (70, 3, 2048), (65, 2, 4096)])
def test_norm_modulate_shapes_per_token_and_broadcast(b, t, d):
    import ltxk

    x = bf((b, t, d), 2)
    table = bf((9, d), 3, 0.05)
    emb_tok = bf((b, t, 9 * d), 4, 0.05)    # per-token timestep embedding
    emb_bat = bf((b, 1, 9 * d), 5, 0.05)    # one row per batch item
    for emb in (emb_tok, emb_bat):
        sh = ltxk.AdaRef(table.to(DEV), 0, emb.to(DEV))
        sc = ltxk.AdaRef(table.to(DEV), 1, emb.to(DEV))
        y = ltxk.norm_modulate(x.to(DEV), shift=sh, scale=sc)
        want = O.norm_modulate(x, O.ada_value(table, 0, emb, b, t), O.ada_value(table, 1, emb, b, t))
        assert_close_bf16(y, want, what=f"norm_modulate {b}x{t}x{d}")


@pytest.mark.parametrize("t,d", [(1100, 2048), (600, 4096), (3, 8192), (513, 16384)])
def test_single_item_full_rows_operand_kinds(t, d):
    """One batch item, rows of whole workgroups (d = 2048 .. 16384), more or
    fewer rows than resident workgroups: shift absent / table only / table and
    embedding, scale embedding only / table and embedding."""
    import ltxk

    x = bf((1, t, d), 50)
    table = bf((4, d), 51, 0.05)
    emb = bf((1, 1, 4 * d), 52, 0.05)
    etab = torch.zeros(4, d, dtype=torch.bfloat16)
    cases = [
        (None, ltxk.AdaRef(None, 1, emb.to(DEV), dim=d), None, O.ada_value(etab, 1, emb, 1, t)),
        (ltxk.AdaRef(table.to(DEV), 0), ltxk.AdaRef(table.to(DEV), 1, emb.to(DEV)),
         O.ada_value(table, 0, None, 1, t), O.ada_value(table, 1, emb, 1, t)),
        (ltxk.AdaRef(table.to(DEV), 2, emb.to(DEV)), None, O.ada_value(table, 2, emb, 1, t), None),
    ]
    for sh, sc, wsh, wsc in cases:
        y = ltxk.norm_modulate(x.to(DEV), shift=sh, scale=sc)
        assert_close_bf16(y, O.norm_modulate(x, wsh, wsc), what=f"norm_modulate 1x{t}x{d}")
    # two outputs of add_norm_modulate: absent gate (1), a gate with a zero
    # mask, absent second shift
    f = bf((1, t, d), 53)
    A = lambda r: ltxk.AdaRef(table.to(DEV), r, emb.to(DEV))  # noqa: E731
    ov = lambda r: O.ada_value(table, r, emb, 1, t)  # noqa: E731
    for gate, mask, wgate in ((None, None, None), (A(3), torch.zeros(1, dtype=torch.bfloat16), ov(3))):
        m = None if mask is None else mask.to(DEV)
        xo, y, y2 = ltxk.add_norm_modulate(x.to(DEV), f.to(DEV), gate=gate, mask=m, shift=A(0), scale=A(1),
                                           shift2=None, scale2=A(2))
        wxo, wy = O.add_norm_modulate(x, f, wgate, mask, ov(0), ov(1))
        assert torch.equal(xo.cpu(), wxo)
        assert_close_bf16(y, wy, what=f"add_norm_modulate y 1x{t}x{d}")
        assert_close_bf16(y2, O.norm_modulate(wxo, None, ov(2)), what=f"add_norm_modulate y2 1x{t}x{d}")


def test_norm_modulate_dual_output_and_layernorm():
    import ltxk

    x = bf((2, 50, 1024), 6)
    table = bf((5, 1024), 7, 0.05)
    emb = bf((2, 1, 4 * 1024), 8, 0.05)
    T = lambda r: ltxk.AdaRef(table.to(DEV), r, emb.to(DEV))  # noqa: E731
    y1, y2 = ltxk.norm_modulate(x.to(DEV), shift=T(1), scale=T(0), shift2=T(3), scale2=T(2))
    av = lambda r: O.ada_value(table[:4], r, emb, 2, 50)  # noqa: E731
    assert_close_bf16(y1, O.norm_modulate(x, av(1), av(0)), what="dual y1")
    assert_close_bf16(y2, O.norm_modulate(x, av(3), av(2)), what="dual y2")
    # LayerNorm (output head): shift/scale = sst rows + the same embedded row
    sst = bf((2, 1024), 9, 0.05)
    e1 = bf((2, 50, 1024), 10, 0.05)
    y = ltxk.norm_modulate(x.to(DEV), shift=ltxk.AdaRef(sst.to(DEV), 0, e1.to(DEV), 0),
                           scale=ltxk.AdaRef(sst.to(DEV), 1, e1.to(DEV), 0), layer=True)
    want = O.norm_modulate(x, O.ada_value(sst, 0, e1, 2, 50), O.ada_value(torch.stack([sst[1], sst[1]]), 0, e1, 2, 50),
                           layer=True)
    assert_close_bf16(y, want, what="layer norm head")


@pytest.mark.parametrize("b,t,d", [(2, 40, 2048), (3, 11, 3072), (1, 513, 4096), (70, 2, 4096)])
def test_dual_outputs_on_whole_workgroup_rows(b, t, d):
    """Two modulations of one normalised row (norm_modulate shift2/scale2 and
    add_norm_modulate's y2) on rows a whole workgroup owns: full rows
    (d = 2048, 4096), partial rows (3072), more rows than resident workgroups
    (513), and more batch items than the segmented kernel takes (70)."""
    import ltxk

    x, f = bf((b, t, d), 40), bf((b, t, d), 41)
    table = bf((9, d), 42, 0.05)
    emb = bf((b, 1, 9 * d), 43, 0.05)
    A = lambda r: ltxk.AdaRef(table.to(DEV), r, emb.to(DEV))  # noqa: E731
    ov = lambda r: O.ada_value(table, r, emb, b, t)  # noqa: E731
    y1, y2 = ltxk.norm_modulate(x.to(DEV), shift=A(0), scale=A(1), shift2=A(3), scale2=A(4))
    assert_close_bf16(y1, O.norm_modulate(x, ov(0), ov(1)), what="norm_modulate y")
    assert_close_bf16(y2, O.norm_modulate(x, ov(3), ov(4)), what="norm_modulate y2")
    xo, y, y2 = ltxk.add_norm_modulate(x.to(DEV), f.to(DEV), gate=A(2), shift=A(6), scale=A(7), shift2=A(3),
                                       scale2=A(4))
    wxo, wy = O.add_norm_modulate(x, f, ov(2), None, ov(6), ov(7))
    assert torch.equal(xo.cpu(), wxo)
    assert_close_bf16(y, wy, what="add_norm_modulate y")
    assert_close_bf16(y2, O.norm_modulate(wxo, ov(3), ov(4)), what="add_norm_modulate y2")


@pytest.mark.parametrize("b,t,d,dual", [(1, 9000, 2048, False), (2, 8500, 4096, True), (4, 6144, 4096, False),
                                         (3, 4500, 3072, True)])
def test_wave_rows_walk_more_rows_than_two_per_wave(b, t, d, dual):
    """The one-wave-per-row norm_modulate on items of more rows than two per
    resident wave (the per-chunk refill of a wave's third row and beyond),
    on several batch items (the modulation staged per item), full and partial
    rows, one and two outputs."""
    import ltxk

    x = bf((b, t, d), 60)
    table = bf((9, d), 61, 0.05)
    emb = bf((b, 1, 9 * d), 62, 0.05)
    A = lambda r: ltxk.AdaRef(table.to(DEV), r, emb.to(DEV))  # noqa: E731
    ov = lambda r: O.ada_value(table, r, emb, b, t)  # noqa: E731
    if dual:
        y1, y2 = ltxk.norm_modulate(x.to(DEV), shift=A(0), scale=A(1), shift2=A(3), scale2=A(4))
        assert_close_bf16(y2, O.norm_modulate(x, ov(3), ov(4)), what=f"y2 {b}x{t}x{d}")
    else:
        y1 = ltxk.norm_modulate(x.to(DEV), shift=A(0), scale=A(1))
    d1 = assert_close_bf16(y1, O.norm_modulate(x, ov(0), ov(1)), what=f"y {b}x{t}x{d}")
    assert (d1 == 0).float().mean() > 0.99


def test_rms_norm_with_weight():
    import ltxk

    x, w = bf((2, 9, 4096), 11), bf((4096,), 12)
    assert_close_bf16(ltxk.rms_norm(x.to(DEV), w.to(DEV)), O.rms_norm(x, w), what="rms_norm w")
    assert_close_bf16(ltxk.rms_norm(x.to(DEV)), O.rms_norm(x), what="rms_norm")


@pytest.mark.parametrize("with_mask", [False, True])
@pytest.mark.parametrize("b,t,d", [(2, 129, 4096), (2, 33, 1024), (2, 7, 64), (2, 50, 2048), (2, 21, 3072)])
def test_add_norm_modulate(with_mask, b, t, d):
    import ltxk

    x, f = bf((b, t, d), 13), bf((b, t, d), 14)
    table = bf((9, d), 15, 0.05)
    emb = bf((b, 1, 9 * d), 16, 0.05)
    mask = torch.tensor([1.0, 0.0], dtype=torch.bfloat16) if with_mask else None
    emb_tok = bf((b, t, 9 * d), 26, 0.05)  # per-token embedding: the per-row kernel
    A_tok = lambda r: ltxk.AdaRef(table.to(DEV), r, emb_tok.to(DEV))  # noqa: E731
    xo_t, y_t = ltxk.add_norm_modulate(x.to(DEV), f.to(DEV), gate=A_tok(2), shift=A_tok(6), scale=A_tok(7))
    ot = lambda r: O.ada_value(table, r, emb_tok, b, t)  # noqa: E731
    wxo_t, wy_t = O.add_norm_modulate(x, f, ot(2), None, ot(6), ot(7))
    assert torch.equal(xo_t.cpu(), wxo_t)
    assert_close_bf16(y_t, wy_t, what="add_norm_modulate per-token y")
    A = lambda r: ltxk.AdaRef(table.to(DEV), r, emb.to(DEV))  # noqa: E731
    xo, y = ltxk.add_norm_modulate(x.to(DEV), f.to(DEV), gate=A(2), mask=None if mask is None else mask.to(DEV),
                                   shift=A(6), scale=A(7))
    ov = lambda r: O.ada_value(table, r, emb, b, t)  # noqa: E731
    wxo, wy = O.add_norm_modulate(x, f, ov(2), mask, ov(6), ov(7))
    assert torch.equal(xo.cpu(), wxo)  # residual: same single rounding
    assert_close_bf16(y, wy, what="add_norm_modulate y")
    # residual only, in place
    xd = x.to(DEV)
    ltxk.add_norm_modulate(xd, f.to(DEV), gate=A(2), norm=False, x_out=xd)
    assert torch.equal(xd.cpu(), O.gated_residual(x, f, ov(2)))


def test_modulate_gated_residual_context_shapes():
    import ltxk

    ctx = bf((2, 1024, 4096), 17)
    psst = bf((2, 4096), 18, 0.05)
    pts = bf((2, 1, 2 * 4096), 19, 0.05)
    enc = ltxk.modulate(ctx.to(DEV), ltxk.AdaRef(psst.to(DEV), 0, pts.to(DEV)),
                        ltxk.AdaRef(psst.to(DEV), 1, pts.to(DEV)))
    want = O.modulate(ctx, O.ada_value(psst, 0, pts, 2, 1024), O.ada_value(psst, 1, pts, 2, 1024))
    assert torch.equal(enc.cpu(), want)
    x, f = bf((3, 77, 2048), 20), bf((3, 77, 2048), 21)
    gate_tab = bf((5, 2048), 22, 0.05)
    gate_ts = bf((3, 77, 2048), 23, 0.05)
    mask = torch.tensor([1.0, 0.0, 1.0], dtype=torch.bfloat16)
    out = ltxk.gated_residual(x.to(DEV), f.to(DEV), ltxk.AdaRef(gate_tab.to(DEV), 4, gate_ts.to(DEV), 0),
                              mask.to(DEV))
    gv = O.ada_value(gate_tab[4:], 0, gate_ts, 3, 77)
    assert torch.equal(out.cpu(), O.gated_residual(x, f, gv, mask))
    assert torch.equal(ltxk.gated_residual(x.to(DEV), f.to(DEV)).cpu(), O.gated_residual(x, f))
    # broadcast gate (one row per batch item) and per-batch context modulation at other widths
    for d in (1024, 64, 4096):
        xs, fs = bf((3, 21, d), 27), bf((3, 21, d), 28)
        tab = bf((9, d), 29, 0.05)
        eb = bf((3, 1, 9 * d), 30, 0.05)
        got = ltxk.gated_residual(xs.to(DEV), fs.to(DEV), ltxk.AdaRef(tab.to(DEV), 5, eb.to(DEV)), mask.to(DEV))
        assert torch.equal(got.cpu(), O.gated_residual(xs, fs, O.ada_value(tab, 5, eb, 3, 21), mask))
        got = ltxk.modulate(xs.to(DEV), ltxk.AdaRef(tab.to(DEV), 3, eb.to(DEV)), ltxk.AdaRef(tab.to(DEV), 4, eb.to(DEV)))
        assert torch.equal(got.cpu(), O.modulate(xs, O.ada_value(tab, 3, eb, 3, 21), O.ada_value(tab, 4, eb, 3, 21)))


@pytest.mark.parametrize("h,dh,t", [(32, 128, 300), (32, 64, 126), (4, 16, 9)])
def test_head_gate_token_major_and_bhtd(h, dh, t):
    import ltxk

    b = 2
    attn_bhtd = bf((b, h, t, dh), 24)
    logits = bf((b, t, h), 25, 2.0)
    tok = attn_bhtd.transpose(1, 2).reshape(b, t, h * dh).contiguous()
    want = O.head_gate(tok, logits, h)
    got4 = ltxk.head_gate(attn_bhtd.to(DEV), logits.to(DEV))
    got3 = ltxk.head_gate(tok.to(DEV), logits.to(DEV))
    assert_close_bf16(got4, want, what="head_gate bhtd")
    assert torch.equal(got4.cpu(), got3.cpu())
    # a transposed view of a (B, T, H, D) buffer, as some attention kernels return
    bthd = attn_bhtd.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)
    assert torch.equal(ltxk.head_gate(bthd, logits.to(DEV)).cpu(), got4.cpu())


def test_rows_zero_and_shape_errors():
    import ltxk

    x = torch.empty(0, 4096, device=DEV, dtype=torch.bfloat16)
    assert ltxk.norm_modulate(x).shape == (0, 4096)
    with pytest.raises(ValueError, match="width"):
        ltxk.norm_modulate(torch.zeros(4, 64, device=DEV, dtype=torch.bfloat16),
                           shift=ltxk.AdaRef(torch.zeros(2, 128, device=DEV, dtype=torch.bfloat16), 0))
    with pytest.raises(RuntimeError, match="multiple of 8"):
        ltxk.norm_modulate(torch.zeros(4, 12, device=DEV, dtype=torch.bfloat16))


def test_head_gate_with_perturbation_blend_and_without_logits():
    """attn*m + v*(1-m) per batch item (ltx_nn.py:229-230), then the gate (231-235)."""
    import ltxk

    b, h, t, dh = 4, 4, 33, 32
    attn = bf((b, t, h, dh), 31).transpose(1, 2)       # SDPA's (B,T,H,D) buffer as (B,H,T,D)
    v = bf((b, t, h * dh), 32)
    logits = bf((b, t, h), 33, 2.0)
    keep = torch.tensor([1.0, 1.0, 0.0, 1.0], dtype=torch.bfloat16)
    tok = attn.transpose(1, 2).reshape(b, t, h * dh)
    blended = (tok.float() * keep.float().view(-1, 1, 1) + v.float() * (1 - keep.float().view(-1, 1, 1)))
    got = ltxk.head_gate(attn.to(DEV), logits.to(DEV), v=v.to(DEV), mask=keep.to(DEV))
    assert_close_bf16(got, O.head_gate(blended.to(torch.bfloat16), logits, h), what="blend + gate")
    assert torch.equal(got[2].cpu(), O.head_gate(v[2:3], logits[2:3], h)[0])
    # no gate: the plain head merge (and blend)
    got = ltxk.head_gate(attn.to(DEV), None, v=v.to(DEV), mask=keep.to(DEV))
    assert torch.equal(got.cpu(), blended.to(torch.bfloat16))
    # all perturbed: gate applied to v itself
    got = ltxk.head_gate(v.to(DEV), logits.to(DEV))
    assert torch.equal(got.cpu(), O.head_gate(v, logits, h))


@pytest.mark.parametrize("b,t,d,layers", [(1, 1024, 4096, 48), (2, 37, 2048, 5), (3, 8, 64, 1), (1, 6, 136, 3)])
def test_modulate_layers_equals_per_layer_modulate(b, t, d, layers):
    """Every block's context modulation from one launch: layer l equals
    ltxk.modulate with block l's prompt table (bit for bit) and the oracle's
    modulate of the materialised table + prompt-timestep rows."""
    import ltxk

    ctx = bf((b, t, d), 60)
    tabs = bf((layers, 2, d), 61, 0.05)
    pts = bf((b, 1, 2 * d), 62, 0.05)
    cd, td, pd = ctx.to(DEV), tabs.to(DEV), pts.to(DEV)
    out = ltxk.modulate_layers(cd, ltxk.AdaRef(td, 0, pd), ltxk.AdaRef(td, 1, pd), layers)
    assert out.shape == (layers, b, t, d)
    for layer in sorted({0, layers // 2, layers - 1}):
        one = ltxk.modulate(cd, ltxk.AdaRef(td[layer].contiguous(), 0, pd), ltxk.AdaRef(td[layer].contiguous(), 1, pd))
        assert torch.equal(out[layer], one), layer
        want = O.modulate(ctx, O.ada_value(tabs[layer], 0, pts, b, t), O.ada_value(tabs[layer], 1, pts, b, t))
        assert torch.equal(out[layer].cpu(), want), layer
    # no embedding: the tables alone; no operands at all: a copy per layer
    out = ltxk.modulate_layers(cd, ltxk.AdaRef(td, 0), ltxk.AdaRef(td, 1), layers)
    assert torch.equal(out[-1].cpu(), O.modulate(ctx, tabs[-1, 0], tabs[-1, 1]))
    out = ltxk.modulate_layers(cd, None, None, 2)
    assert torch.equal(out[1], cd)


def test_modulate_layers_per_layer_embeddings_through_the_c_abi():
    """emb_layer_stride != 0 (each layer its own embedding rows), through the C
    entry point directly: layer l equals modulate with layer l's rows."""
    import ctypes

    import ltxk

    layers, b, t, d = 4, 2, 24, 256
    ctx = bf((b, t, d), 66).to(DEV)
    tabs = bf((layers, 2, d), 67, 0.05).to(DEV)
    embs = bf((layers, b, 1, 2 * d), 68, 0.05).to(DEV)
    out = torch.empty(layers, b, t, d, device=DEV, dtype=torch.bfloat16)
    sh = ltxk.AdaRef(tabs, 0, embs[0]).struct(b, t)
    sc = ltxk.AdaRef(tabs, 1, embs[0]).struct(b, t)
    rc = ltxk.load().ltxk_modulate_layers(out.data_ptr(), ctx.data_ptr(), layers, b * t, t, d, ctypes.byref(sh),
                                          ctypes.byref(sc), 2 * d, b * 2 * d,
                                          torch.cuda.current_stream().cuda_stream)
    assert rc == 0, ltxk.last_error()
    for layer in range(layers):
        tab = tabs[layer].contiguous()
        want = ltxk.modulate(ctx, ltxk.AdaRef(tab, 0, embs[layer]), ltxk.AdaRef(tab, 1, embs[layer]))
        assert torch.equal(out[layer], want), layer
    # strides that are not whole 16-byte chunks are refused
    rc = ltxk.load().ltxk_modulate_layers(out.data_ptr(), ctx.data_ptr(), layers, b * t, t, d, ctypes.byref(sh),
                                          ctypes.byref(sc), 2 * d + 4, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == ltxk.E_ALIGN


def test_modulate_layers_per_token_and_indexed_embeddings():
    """Embedding rows that vary per token (per-token rows, or an index into
    de-duplicated rows) take the per-row form: still equal to modulate."""
    import ltxk

    layers, b, t, d = 3, 2, 40, 512
    ctx = bf((b, t, d), 69).to(DEV)
    tabs = bf((layers, 2, d), 70, 0.05).to(DEV)
    per_tok = bf((b, t, 2 * d), 71, 0.05).to(DEV)
    out = ltxk.modulate_layers(ctx, ltxk.AdaRef(tabs, 0, per_tok), ltxk.AdaRef(tabs, 1, per_tok), layers)
    rows = bf((1, 3, 2 * d), 72, 0.05).to(DEV)
    index = ltxk.TimestepIndex(torch.randint(0, 3, (b * t,), dtype=torch.int32).to(DEV), 3)
    outi = ltxk.modulate_layers(ctx, ltxk.AdaRef(tabs, 0, rows, index=index),
                                ltxk.AdaRef(tabs, 1, rows, index=index), layers)
    for layer in range(layers):
        tab = tabs[layer].contiguous()
        assert torch.equal(out[layer], ltxk.modulate(ctx, ltxk.AdaRef(tab, 0, per_tok), ltxk.AdaRef(tab, 1, per_tok)))
        assert torch.equal(outi[layer], ltxk.modulate(ctx, ltxk.AdaRef(tab, 0, rows, index=index),
                                                      ltxk.AdaRef(tab, 1, rows, index=index)))


def test_modulate_layers_rejects_bad_tables():
    import ltxk

    x = bf((1, 8, 64), 63).to(DEV)
    with pytest.raises(ValueError):
        ltxk.modulate_layers(x, ltxk.AdaRef(bf((2, 64), 64).to(DEV), 0), None, 3)   # not (layers, n, D)
    with pytest.raises(ValueError):
        ltxk.modulate_layers(x, ltxk.AdaRef(bf((2, 2, 64), 65).to(DEV), 0), None, 3)  # 2 layers, not 3
