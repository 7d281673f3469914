"""Parity of ltxk_qk_norm_rope (split RoPE, optional weighted RMSNorm) (GPU):
against the reference's own RoPE vectors and against the oracle."""

import numpy as np
import pytest
import torch

from conftest import GOLDEN, assert_close_bf16, bf16_from_bits
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
ROPE = np.load(GOLDEN / "rope_golden.npz")


def bf(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("name", ["video", "video_small", "audio", "cross"])
def test_rope_on_reference_vectors(name):
    import ltx_nn

    x = bf16_from_bits(ROPE[f"{name}_x"])
    c, s = bf16_from_bits(ROPE[f"{name}_cos"]), bf16_from_bits(ROPE[f"{name}_sin"])
    ref = bf16_from_bits(ROPE[f"{name}_rot"])
    got = ltx_nn.apply_split_rotary_emb(x.to(DEV), (c.to(DEV), s.to(DEV))).cpu()
    # fp32 single rounding: equal to the oracle
    assert torch.equal(got, O.apply_rope(x, c, s))
    # and within the reference's own eager-bf16 rounding of its output
    assert_close_bf16(got, ref, atol=2.0**-5, rtol=2.0**-6, what="vs reference eager rotation")


def test_tables_built_on_device_match_reference():
    import ltx_nn

    for name in ("video", "audio", "cross"):
        meta = ROPE[f"{name}_meta"]
        dim, heads = int(meta[0]), int(meta[1])
        max_pos = [int(m) for m in meta[2:]]
        pos = torch.from_numpy(ROPE[f"{name}_positions"]).to(DEV)
        c, s = ltx_nn.precompute_freqs_cis(pos, dim, torch.bfloat16, max_pos=max_pos, num_attention_heads=heads)
        gc, gs = bf16_from_bits(ROPE[f"{name}_cos"]), bf16_from_bits(ROPE[f"{name}_sin"])
        # device cos/sin may round a handful of entries differently from the CPU library
        for got, want in ((c.cpu(), gc), (s.cpu(), gs)):
            assert (got.view(torch.int16) == want.view(torch.int16)).float().mean() > 0.999
            assert (got.float() - want.float()).abs().max() <= 2.0**-8


def _video_tables(t_grid, h_grid, w_grid, dim=4096, heads=32, fps=24.0):
    pos = O.video_positions(1, t_grid, h_grid, w_grid, fps)
    return O.rope_tables(pos, dim, heads, [20, 2048, 2048])


def test_config2_video_qk_rope_full_shape():
    """q, k [1, 32, 6144, 128] bf16 (token-major [6144, 4096]), 16x16x24 grid, theta 1e4."""
    import ltxk

    c, s = _video_tables(16, 16, 24)
    q, k = bf((1, 6144, 4096), 30), bf((1, 6144, 4096), 31)
    qd, kd = q.to(DEV), k.to(DEV)
    pe = (c.to(DEV), s.to(DEV))
    ltxk.qk_norm_rope(qd, kd, 32, 128, q_pe=pe, k_pe=pe)   # shared tables: paired launch
    assert torch.equal(qd.cpu(), O.apply_rope(q, c, s))
    assert torch.equal(kd.cpu(), O.apply_rope(k, c, s))


@pytest.mark.parametrize("form", ["grid_bounds", "fp32_grid"])
def test_config2_other_table_forms_full_shape(form):
    """Config 2 at full shape on its other table forms: positions as grid
    bounds (i, i+1) normalised by max_pos (16, 16, 24), and the model's
    positions on the fp32 frequency grid (checkpoints without float64
    frequencies).  The oracle's tables applied on the GPU rotate exactly as the
    oracle does; the tables built on the device are within the device's
    cos/sin rounding of the oracle's, and their compact form rotates exactly as
    their full form."""
    import ltx_nn
    import ltxk

    if form == "grid_bounds":
        grid = torch.stack(torch.meshgrid(torch.arange(16.0), torch.arange(16.0), torch.arange(24.0),
                                          indexing="ij")).reshape(3, -1)
        pos, mp, dp = torch.stack([grid, grid + 1], dim=-1).unsqueeze(0).contiguous(), [16, 16, 24], True
    else:
        pos, mp, dp = O.video_positions(1, 16, 16, 24, 24.0), [20, 2048, 2048], False
    c, s = O.rope_tables(pos, 4096, 32, mp, double_precision=dp)
    dc, ds = ltx_nn.precompute_freqs_cis(pos.to(DEV), 4096, torch.bfloat16, max_pos=mp, num_attention_heads=32,
                                         double_precision=dp)
    # the device's cos/sin round a few large angles (up to 1e4*pi/2 rad) one bf16 ulp
    # away from the CPU library's; a wrong position, scale or layout is O(1)
    for got, want in ((dc.cpu(), c), (ds.cpu(), s)):
        assert (got.view(torch.int16) == want.view(torch.int16)).float().mean() > 0.99
        assert (got.float() - want.float()).abs().max() <= 2.0**-8
    q, k = bf((1, 6144, 4096), 34), bf((1, 6144, 4096), 35)
    qd, kd = q.to(DEV), k.to(DEV)
    pe = (c.to(DEV), s.to(DEV))
    ltxk.qk_norm_rope(qd, kd, 32, 128, q_pe=pe, k_pe=pe)
    assert torch.equal(qd.cpu(), O.apply_rope(q, c, s))
    assert torch.equal(kd.cpu(), O.apply_rope(k, c, s))
    cp = ltx_nn.precompute_freqs_cis_compact(pos.to(DEV), 4096, torch.bfloat16, max_pos=mp, num_attention_heads=32,
                                             double_precision=dp)
    qd, kd = q.to(DEV), k.to(DEV)
    ltxk.qk_norm_rope(qd, kd, 32, 128, None, None, cp, cp)
    assert torch.equal(qd.cpu(), O.apply_rope(q, dc.cpu(), ds.cpu()))
    assert torch.equal(kd.cpu(), O.apply_rope(k, dc.cpu(), ds.cpu()))


def test_config2_audio_rope():
    """Audio q/k [1, 32, 126, 64] with positions 0..125 (1D RoPE)."""
    import ltxk

    pos = torch.arange(126, dtype=torch.float32).view(1, 1, 126, 1).expand(1, 1, 126, 2).contiguous()
    c, s = O.rope_tables(pos, 2048, 32, [126])
    q, k = bf((1, 126, 2048), 32), bf((1, 126, 2048), 33)
    qd, kd = q.to(DEV), k.to(DEV)
    ltxk.qk_norm_rope(qd, kd, 32, 64, q_pe=(c.to(DEV), s.to(DEV)), k_pe=(c.to(DEV), s.to(DEV)))
    assert torch.equal(qd.cpu(), O.apply_rope(q, c, s))
    assert torch.equal(kd.cpu(), O.apply_rope(k, c, s))


@pytest.mark.parametrize("b,tq,tk,heads,dh", [(1, 300, 300, 32, 128), (2, 77, 77, 32, 64), (1, 6144, 126, 32, 64),
                                              (2, 40, 13, 4, 16), (1, 9, 9, 1, 256)])
def test_qk_norm_rope_with_weights(b, tq, tk, heads, dh):
    import ltxk

    d = heads * dh
    q, k = bf((b, tq, d), 34), bf((b, tk, d), 35)
    wq, wk = bf((d,), 36), bf((d,), 37)
    posq = torch.rand(b, 1, tq, 2, generator=torch.Generator().manual_seed(38)) * 20
    posk = torch.rand(b, 1, tk, 2, generator=torch.Generator().manual_seed(39)) * 20
    cq, sq = O.rope_tables(posq, d, heads, [20])
    ck, sk = O.rope_tables(posk, d, heads, [20])
    qd, kd = q.to(DEV), k.to(DEV)
    ltxk.qk_norm_rope(qd, kd, heads, dh, wq.to(DEV), wk.to(DEV), (cq.to(DEV), sq.to(DEV)), (ck.to(DEV), sk.to(DEV)))
    assert_close_bf16(qd, O.qk_norm_rope(q, wq, cq, sq), what="q")
    assert_close_bf16(kd, O.qk_norm_rope(k, wk, ck, sk), what="k")
    # shared tables for q and k of equal length take the paired path
    if tq == tk:
        qd, kd = q.to(DEV), k.to(DEV)
        ltxk.qk_norm_rope(qd, kd, heads, dh, wq.to(DEV), wk.to(DEV), (cq.to(DEV), sq.to(DEV)),
                          (cq.to(DEV), sq.to(DEV)))
        assert_close_bf16(kd, O.qk_norm_rope(k, wk, cq, sq), what="k paired")


def test_qk_norm_without_rope_text_cross():
    """Text cross-attention: q [6144, 4096] and k [1024, 4096] normed, no RoPE."""
    import ltxk

    q, k = bf((1, 6144, 4096), 40), bf((1, 1024, 4096), 41)
    wq, wk = bf((4096,), 42), bf((4096,), 43)
    qd, kd = q.to(DEV), k.to(DEV)
    ltxk.qk_norm_rope(qd, kd, 32, 128, wq.to(DEV), wk.to(DEV))
    assert_close_bf16(qd, O.rms_norm(q, wq), what="q norm")
    assert_close_bf16(kd, O.rms_norm(k, wk), what="k norm")


@pytest.mark.parametrize("tq,tk,dim,wq,wk", [(1, 0, 4096, True, False), (5, 3, 2048, True, False),
                                             (6144, 1024, 4096, False, False), (20007, 7, 2048, True, True),
                                             (7, 4100, 4096, False, True)])
def test_qk_norm_without_rope_wave_rows(tq, tk, dim, wq, wk):
    """The one-wave-per-row q/k norm (rows of 2048 or 4096, no tables): q
    rows then k rows in one launch, a wave taking up to five rows (20007 +
    7), q alone, fewer rows than a workgroup's waves; a weighted operand
    against the oracle's fp32 RMSNorm, an unweighted one left unchanged bit
    for bit (no normalisation, as the one-pass kernel does)."""
    import ltxk

    q = bf((1, tq, dim), 50 + tq)
    k = bf((1, tk, dim), 51 + tk) if tk else None
    w1 = bf((dim,), 52).to(DEV) if wq else None
    w2 = bf((dim,), 53).to(DEV) if wk else None
    qd = q.to(DEV)
    kd = k.to(DEV) if k is not None else None
    ltxk.qk_norm_rope(qd, kd, dim // 128, 128, w1, w2)
    for got, x, w, what in ((qd, q, w1, "q"), (kd, k, w2, "k")):
        if got is None:
            continue
        if w is None:
            assert torch.equal(got.cpu().view(torch.int16), x.view(torch.int16)), what
        else:
            assert_close_bf16(got.cpu(), O.rms_norm(x, w.cpu()), what=what)


def test_apply_split_rotary_emb_bhtd_input():
    import ltx_nn

    c, s = _video_tables(2, 2, 2, dim=256, heads=2)
    x = bf((1, 8, 256), 44)
    x4 = x.view(1, 8, 2, 128).transpose(1, 2)  # (B, H, T, D)
    got = ltx_nn.apply_split_rotary_emb(x4.to(DEV), (c.to(DEV), s.to(DEV)))
    assert got.shape == (1, 2, 8, 128)
    assert torch.equal(got.transpose(1, 2).reshape(1, 8, 256).cpu(), O.apply_rope(x, c, s))


def _both_forms(pos, dim, heads, max_pos):
    import ltx_nn

    pos = pos.to(DEV)
    full = ltx_nn.precompute_freqs_cis(pos, dim, torch.bfloat16, max_pos=max_pos, num_attention_heads=heads)
    compact = ltx_nn.precompute_freqs_cis_compact(pos, dim, torch.bfloat16, max_pos=max_pos,
                                                  num_attention_heads=heads)
    return full, compact


def _same_but_sum_order(got, want, min_equal, what=""):
    """What two kernels that differ only in the order their norm sums a row's
    squares may differ by: 1/rms in its last fp32 bit.  That moves each of
    an output's two rotation terms by about 2^-23 of itself, so every bf16 of
    got is want or one of its neighbours or, where the two terms cancel to
    near zero, within 2^-16 of its row's largest output; and at least
    min_equal of them are bit-equal.  A wrong table entry, sign or partner
    moves an output by the size of its row's values."""
    def key(t):  # bf16 bits -> integers in the order of the values (+0 and -0 both 0)
        i = t.view(torch.int16).to(torch.int32)
        return torch.where(i >= 0, i, -(i & 0x7FFF))
    d = (key(got) - key(want)).abs()
    diff = (got.float() - want.float()).abs()
    near = diff <= want.float().abs().amax(dim=-1, keepdim=True) * 2.0 ** -16
    bad = (d > 1) & ~near
    eq = float((d == 0).float().mean())
    assert not bool(bad.any()) and eq >= min_equal, \
        f"{what}: {int(bad.sum())} outputs off by more, max {int(d.max())} ulp, {eq:.4f} bit-equal"


@pytest.mark.parametrize("case", ["video_paired", "video_two_fps", "audio", "cross", "mixed_forms",
                                  "video_4096_odd_tokens", "video_4096_two_fps", "video_3072", "cross_4096"])
def test_compact_tables_give_full_table_results(case):
    """The compact per-axis form of the tables rotates bit-identically to the
    full (B, H, T, Dh/2) tables, on every launch shape: paired q/k (self
    attention), one launch with different tables (cross), and q and k in
    different table forms (two launches); the wave-token and contiguous-chunk
    pair kernels and the wave-row kernel (2048-wide rows, 64-wide heads) up to
    their norm's summation order (one bf16 ulp, more only where an output's two
    terms cancel) and within the parity bound of the oracle.  Rows of
    2048 < D <= 4096 take the
    two-tokens-per-workgroup kernel: odd token counts (a last workgroup with
    one token), batch items whose neighbouring tokens share no axis row, rows
    narrower than the workgroup, and q/k of different token counts."""
    import ltxk

    if case == "video_paired":
        pos, dim, heads, mp, b = O.video_positions(1, 16, 16, 24, 24.0), 4096, 32, [20, 2048, 2048], 1
    elif case == "video_two_fps":
        pos = torch.cat([O.video_positions(1, 3, 4, 5, 24.0), O.video_positions(1, 3, 4, 5, 25.0)])
        dim, heads, mp, b = 512, 4, [20, 2048, 2048], 2
    elif case == "video_4096_odd_tokens":
        pos, dim, heads, mp, b = O.video_positions(1, 3, 5, 7, 24.0), 4096, 32, [20, 2048, 2048], 1
    elif case == "video_4096_two_fps":
        pos = torch.cat([O.video_positions(1, 3, 4, 5, 24.0), O.video_positions(1, 3, 4, 5, 25.0)])
        dim, heads, mp, b = 4096, 32, [20, 2048, 2048], 2
    elif case == "video_3072":
        pos, dim, heads, mp, b = O.video_positions(1, 2, 5, 5, 24.0), 3072, 24, [20, 2048, 2048], 1
    elif case == "audio":
        pos = torch.arange(126, dtype=torch.float32).view(1, 1, 126, 1).expand(1, 1, 126, 2).contiguous()
        dim, heads, mp, b = 2048, 32, [126], 1
    elif case == "cross_4096":
        pos, dim, heads, mp, b = O.video_positions(1, 4, 6, 7, 24.0)[:, 0:1], 4096, 32, [20], 1
    else:
        pos, dim, heads, mp, b = O.video_positions(1, 16, 16, 24, 24.0)[:, 0:1], 2048, 32, [20], 1
    t = pos.shape[2]
    full, compact = _both_forms(pos, dim, heads, mp)
    q, k = bf((b, t, dim), 50), bf((b, t, dim), 51)
    wq, wk = bf((dim,), 52).to(DEV), bf((dim,), 53).to(DEV)
    if case in ("cross", "mixed_forms", "cross_4096"):
        # k: the audio time axis (126 tokens), q: the video time axis
        apos = (torch.arange(126, dtype=torch.float32) / 25.0).view(1, 1, 126, 1).expand(1, 1, 126, 2).contiguous()
        afull, acompact = _both_forms(apos, dim, heads, mp)
        k = bf((1, 126, dim), 54)
        kf, kc = afull, (afull if case == "mixed_forms" else acompact)
        qc = compact
    else:
        kf, kc, qc = full, compact, compact
    want_q, want_k = q.to(DEV), k.to(DEV)
    ltxk.qk_norm_rope(want_q, want_k, heads, dim // heads, wq, wk, full, kf)
    got_q, got_k = q.to(DEV), k.to(DEV)
    ltxk.qk_norm_rope(got_q, got_k, heads, dim // heads, wq, wk, qc, kc)
    if dim == 2048 and dim // heads == 64:
        # 2048-wide rows with 64-wide heads on compact tables take the wave-token
        # or contiguous-chunk kernel (a self-attention pair) or the wave-row
        # kernel (q and k with their own tables, or q alone): the same rotation
        # arithmetic, but the norm sums the squares in another order, so 1/rms
        # can differ in its last bit
        for got, want, x, w, tab in ((got_q, want_q, q, wq, full), (got_k, want_k, k, wk, kf)):
            _same_but_sum_order(got, want, min_equal=0.95, what=case)
            assert_close_bf16(got.cpu(), O.qk_norm_rope(x, w.cpu(), tab[0].cpu(), tab[1].cpu()), what=case)
    else:
        assert torch.equal(got_q.view(torch.int16), want_q.view(torch.int16))
        assert torch.equal(got_k.view(torch.int16), want_k.view(torch.int16))
    # without the norm weights (apply_split_rotary_emb's form)
    import ltx_nn
    x = bf((b, t, dim), 55).to(DEV)
    assert torch.equal(ltx_nn.apply_split_rotary_emb(x, compact).view(torch.int16),
                       ltx_nn.apply_split_rotary_emb(x, full).view(torch.int16))


@pytest.mark.parametrize("dims", [(4096, 32), (3072, 24)])
def test_compact_tables_without_norm_weights(dims):
    """RoPE alone (config 2's op: no q/k norm) on compact tables equals the full
    tables bit for bit, on the two-token kernel's variant without reductions."""
    import ltxk

    dim, heads = dims
    pos = O.video_positions(1, 3, 5, 7, 24.0)
    full, compact = _both_forms(pos, dim, heads, [20, 2048, 2048])
    t = pos.shape[2]
    q, k = bf((1, t, dim), 70), bf((1, t, dim), 71)
    want_q, want_k = q.to(DEV), k.to(DEV)
    ltxk.qk_norm_rope(want_q, want_k, heads, dim // heads, None, None, full, full)
    got_q, got_k = q.to(DEV), k.to(DEV)
    ltxk.qk_norm_rope(got_q, got_k, heads, dim // heads, None, None, compact, compact)
    assert torch.equal(got_q.view(torch.int16), want_q.view(torch.int16))
    assert torch.equal(got_k.view(torch.int16), want_k.view(torch.int16))
    assert_close_bf16(got_q.cpu(), O.apply_rope(q, *[c.cpu() for c in full]), what="rope q")


@pytest.mark.parametrize("paired", [True, False])
def test_compact_index_outside_the_tables_is_clamped(paired):
    """A caller's compact index outside [0, table_rows) reads the last table row
    (the kernels clamp it; the Python binding refuses such an index before the
    launch, so this goes through the C entry point): the streaming pair kernel
    (paired, 4096-wide rows) and the one-pass kernel (q alone)."""
    import ctypes

    import ltx_nn
    import ltxk

    pos = O.video_positions(1, 3, 5, 7, 24.0).to(DEV)
    cp = ltx_nn.precompute_freqs_cis_compact(pos, 4096, torch.bfloat16, max_pos=[20, 2048, 2048],
                                             num_attention_heads=32)
    t, rows = pos.shape[2], cp.rows
    bad = cp.index.clone()
    flat = bad.view(-1)
    flat[::5] = rows + 3
    flat[2::9] = -2
    clamped = torch.where((bad < 0) | (bad >= rows), torch.full_like(bad, rows - 1), bad)
    q, k = bf((1, t, 4096), 80).to(DEV), bf((1, t, 4096), 81).to(DEV)
    wq, wk = bf((4096,), 82).to(DEV), bf((4096,), 83).to(DEV)
    lib = ltxk.load()
    stream = torch.cuda.current_stream().cuda_stream

    def run(index):
        qo, ko = q.clone(), k.clone()
        sq = ltxk.QK(qo.data_ptr(), wq.data_ptr(), cp.cos.data_ptr(), cp.sin.data_ptr(), 1, t, 0, index.data_ptr(),
                     cp.n_axes, rows)
        sk = ltxk.QK(ko.data_ptr(), wk.data_ptr(), cp.cos.data_ptr(), cp.sin.data_ptr(), 1, t, 0, index.data_ptr(),
                     cp.n_axes, rows)
        rc = lib.ltxk_qk_norm_rope(ctypes.byref(sq), ctypes.byref(sk) if paired else None, 32, 128,
                                   ctypes.c_float(1e-6), stream)
        assert rc == 0, ltxk.last_error()
        return qo, ko

    qb, kb = run(bad)
    qc, kc = run(clamped)
    assert torch.equal(qb.view(torch.int16), qc.view(torch.int16))
    assert torch.equal(kb.view(torch.int16), kc.view(torch.int16))
    with pytest.raises(ValueError):  # the binding checks a caller's index range
        ltxk.CompactRope(cp.cos, cp.sin, bad, cp.shape)


@pytest.mark.parametrize("b,tq,tk", [(1, 6144, 126), (1, 1, 1), (1, 1, 0), (1, 3, 700), (1, 10007, 300), (1, 126, 6144),
                                     (2, 1536, 126), (3, 77, 0)])
@pytest.mark.parametrize("weights", [True, False])
def test_wave_row_kernel_cross_rows(b, tq, tk, weights):
    """q and k of 2048-wide rows with 64-wide heads, each with its own one-axis
    compact tables and token count (the A2V q + audio k form of a cross
    attention, and q alone), take the one-wave-per-row kernel: one row, fewer
    rows than a workgroup's waves, more rows than the launch's waves (10,307:
    a wave takes up to three), more k rows than q rows, two and three batch
    items with their own positions; against the oracle's
    fp32 norm + rotation on the full tables (the launch on the full tables
    too) and, without norm weights (rotation only), bit-equal to the
    full-table kernel."""
    import ltx_nn
    import ltxk

    # batch item i's positions shifted by i (each item reads its own table rows)
    vpos = ((torch.arange(tq, dtype=torch.float32) / 24.0).view(1, 1, tq, 1)
            + torch.arange(b, dtype=torch.float32).view(b, 1, 1, 1)).expand(b, 1, tq, 2).contiguous().to(DEV)
    qf = ltx_nn.precompute_freqs_cis(vpos, 2048, torch.bfloat16, max_pos=[20], num_attention_heads=32)
    qc = ltx_nn.precompute_freqs_cis_compact(vpos, 2048, torch.bfloat16, max_pos=[20], num_attention_heads=32)
    seed = 150 + tq + tk + b
    q = bf((b, tq, 2048), seed)
    wq = bf((2048,), seed + 2).to(DEV) if weights else None
    wk = bf((2048,), seed + 3).to(DEV) if weights else None
    what = f"b={b} tq={tq} tk={tk} weights={weights}"
    print(what, flush=True)
    got_q, want_q = q.to(DEV), q.to(DEV)
    if tk:
        apos = ((torch.arange(tk, dtype=torch.float32) / 25.0).view(1, 1, tk, 1)
                + 0.5 * torch.arange(b, dtype=torch.float32).view(b, 1, 1, 1)).expand(b, 1, tk, 2).contiguous().to(DEV)
        kf = ltx_nn.precompute_freqs_cis(apos, 2048, torch.bfloat16, max_pos=[20], num_attention_heads=32)
        kc = ltx_nn.precompute_freqs_cis_compact(apos, 2048, torch.bfloat16, max_pos=[20], num_attention_heads=32)
        k = bf((b, tk, 2048), seed + 1)
        got_k, want_k = k.to(DEV), k.to(DEV)
        ltxk.qk_norm_rope(got_q, got_k, 32, 64, wq, wk, qc, kc)
        ltxk.qk_norm_rope(want_q, want_k, 32, 64, wq, wk, qf, kf)
        pairs = ((got_q, want_q, q, wq, qf, "q"), (got_k, want_k, k, wk, kf, "k"))
    else:
        ltxk.qk_norm_rope(got_q, None, 32, 64, wq, None, qc, None)
        ltxk.qk_norm_rope(want_q, None, 32, 64, wq, None, qf, None)
        pairs = ((got_q, want_q, q, wq, qf, "q"),)
    for got, want, x, w, tab, name in pairs:
        oracle = O.qk_norm_rope(x, None if w is None else w.cpu(), tab[0].cpu(), tab[1].cpu())
        assert_close_bf16(got.cpu(), oracle, what=f"{name} {what}")
        assert_close_bf16(want.cpu(), oracle, what=f"{name} full tables {what}")
        if weights:
            _same_but_sum_order(got, want, min_equal=0.95, what=f"{name} {what}")
        else:
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"{name} {what}"


@pytest.mark.parametrize("b,grid,axes", [(1, (1, 1, 1), 1), (1, (5, 1, 1), 1), (1, (126, 1, 1), 1),
                                         (2, (7, 1, 1), 1), (1, (16, 16, 24), 1), (1, (10007, 1, 1), 1),
                                         (1, (3, 5, 7), 3), (2, (2, 4, 5), 3), (1, (16, 16, 24), 3)])
@pytest.mark.parametrize("weights", [True, False])
def test_pair_kernels_2048_rows(b, grid, axes, weights):
    """Self-attention q/k pairs of 2048-wide rows with 64-wide heads (the A2V
    q + V2A k pair, audio self-attention): one table axis on the wave-token
    kernel, three on the contiguous-chunk kernel; against the oracle's fp32
    norm + rotation on the full tables, and without norm weights (rotation
    only) bit-equal to the full-table kernel, for one token, fewer tokens than
    a workgroup's waves, more tokens than the launch's waves (6144, 10007:
    a wave takes two and three tokens), two batch items."""
    import ltx_nn
    import ltxk

    f, h, w = grid
    t = f * h * w
    if axes == 1:
        pos, mp = O.audio_positions(b, t), [t]
    else:
        pos, mp = O.video_positions(b, f, h, w, 24.0), [20, 2048, 2048]
    full, compact = _both_forms(pos, 2048, 32, mp)
    seed = 90 + t + b
    q, k = bf((b, t, 2048), seed), bf((b, t, 2048), seed + 1)
    wq = bf((2048,), seed + 2).to(DEV) if weights else None
    wk = bf((2048,), seed + 3).to(DEV) if weights else None
    got_q, got_k = q.to(DEV), k.to(DEV)
    ltxk.qk_norm_rope(got_q, got_k, 32, 64, wq, wk, compact, compact)
    c, s = full[0].cpu(), full[1].cpu()
    what = f"b={b} grid={grid} axes={axes} weights={weights}"
    assert_close_bf16(got_q.cpu(), O.qk_norm_rope(q, None if wq is None else wq.cpu(), c, s), what="q " + what)
    assert_close_bf16(got_k.cpu(), O.qk_norm_rope(k, None if wk is None else wk.cpu(), c, s), what="k " + what)
    if not weights:
        want_q, want_k = q.to(DEV), k.to(DEV)
        ltxk.qk_norm_rope(want_q, want_k, 32, 64, None, None, full, full)
        assert torch.equal(got_q.view(torch.int16), want_q.view(torch.int16)), what
        assert torch.equal(got_k.view(torch.int16), want_k.view(torch.int16)), what
