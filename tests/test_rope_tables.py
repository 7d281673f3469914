"""Compact RoPE tables (CPU): ltx_nn.precompute_freqs_cis_compact expanded back to
the full (B, H, T, Dh/2) form equals ltx_nn.precompute_freqs_cis bit for bit, for
the 3-axis video grid (with identity padding), the 1-axis audio/cross time axis,
and batches whose items have different positions."""

import pytest
import torch

from oracle import oracle as O


def _expand(cp):
    """Full tables from the compact form: sum over axes of the indexed rows."""
    b, h, t, hd = cp.shape
    rows_c = cp.cos.float()[cp.index.long()].sum(dim=2)   # (B, T, dim/2)
    rows_s = cp.sin.float()[cp.index.long()].sum(dim=2)
    def split(r):
        return r.to(cp.cos.dtype).reshape(b, t, h, hd).transpose(1, 2)
    return split(rows_c), split(rows_s)


def _video_pos(batch, f, hh, ww, fps):
    return O.video_positions(batch, f, hh, ww, fps)


@pytest.mark.parametrize("case", ["video", "video_two_fps", "audio", "cross", "fp32_grid"])
def test_compact_tables_expand_to_full_tables(case):
    import ltx_nn

    if case == "video":
        pos, dim, heads, mp = _video_pos(1, 4, 6, 5, 24.0), 4096, 32, [20, 2048, 2048]
    elif case == "video_two_fps":
        pos = torch.cat([_video_pos(1, 3, 2, 4, 24.0), _video_pos(1, 3, 2, 4, 25.0)])
        dim, heads, mp = 256, 2, [20, 2048, 2048]
    elif case == "audio":
        pos = torch.arange(126, dtype=torch.float32).view(1, 1, 126, 1).expand(1, 1, 126, 2).contiguous()
        dim, heads, mp = 2048, 32, [126]
    elif case == "cross":
        pos = _video_pos(2, 3, 2, 2, 24.0)[:, 0:1]
        dim, heads, mp = 2048, 32, [20]
    else:
        pos, dim, heads, mp = _video_pos(1, 2, 3, 3, 24.0), 384, 2, [20, 2048, 2048]
    dp = case != "fp32_grid"
    c, s = ltx_nn.precompute_freqs_cis(pos, dim, torch.bfloat16, max_pos=mp, num_attention_heads=heads,
                                       double_precision=dp)
    for merge in (False, True):
        cp = ltx_nn.precompute_freqs_cis_compact(pos, dim, torch.bfloat16, max_pos=mp, num_attention_heads=heads,
                                                 double_precision=dp, merge_slow_axes=merge)
        cols = 2 if merge and pos.shape[1] == 3 else pos.shape[1]
        assert cp.index.dtype == torch.int32 and cp.index.shape == (pos.shape[0], pos.shape[2], cols)
        assert cp.cos.shape[0] <= pos.shape[2] * pos.shape[1] * pos.shape[0]
        ec, es = _expand(cp)
        assert torch.equal(ec.view(torch.int16), c.view(torch.int16))
        assert torch.equal(es.view(torch.int16), s.view(torch.int16))


def test_compact_rows_are_few():
    """16x16x24 latent grid: 16+16+24 distinct coordinates, not 6144 tokens."""
    import ltx_nn

    pos = _video_pos(1, 16, 16, 24, 24.0)
    cp = ltx_nn.precompute_freqs_cis_compact(pos, 4096, max_pos=[20, 2048, 2048], num_attention_heads=32,
                                             merge_slow_axes=False)
    assert cp.cos.shape == (16 + 16 + 24, 2048)
    assert int(cp.index.max()) == 16 + 16 + 24 - 1
    # time and height merged: one row per (time, height) pair, then the width rows
    cp = ltx_nn.precompute_freqs_cis_compact(pos, 4096, max_pos=[20, 2048, 2048], num_attention_heads=32)
    assert cp.cos.shape == (16 * 16 + 24, 2048) and cp.n_axes == 2
    assert int(cp.index[..., 0].max()) == 16 * 16 - 1 and int(cp.index[..., 1].min()) == 16 * 16


def _grid_bounds(f, hh, ww):
    """Positions as integer grid bounds (i, i+1) per axis, (1, 3, f*hh*ww, 2)."""
    g = torch.stack(torch.meshgrid(torch.arange(float(f)), torch.arange(float(hh)), torch.arange(float(ww)),
                                   indexing="ij")).reshape(3, -1)
    return torch.stack([g, g + 1], dim=-1).unsqueeze(0).contiguous()


@pytest.mark.parametrize("double_precision", [True, False])
@pytest.mark.parametrize("case", ["model_positions", "grid_bounds", "audio"])
def test_host_tables_match_oracle(case, double_precision):
    """ltx_nn.precompute_freqs_cis built on the CPU equals the oracle's tables
    bit for bit, on both frequency-grid precisions and both position forms of
    the 16x16x24 video grid: the model's video_positions with max_pos
    (20, 2048, 2048), and grid bounds (i, i+1) normalised by max_pos (16, 16, 24)."""
    import ltx_nn

    if case == "model_positions":
        pos, dim, heads, mp = _video_pos(1, 16, 16, 24, 24.0), 4096, 32, [20, 2048, 2048]
    elif case == "grid_bounds":
        pos, dim, heads, mp = _grid_bounds(16, 16, 24), 4096, 32, [16, 16, 24]
    else:
        pos, dim, heads, mp = O.audio_positions(1, 126)[:, 0:1], 2048, 32, [20]
    c, s = ltx_nn.precompute_freqs_cis(pos, dim, torch.bfloat16, max_pos=mp, num_attention_heads=heads,
                                       double_precision=double_precision)
    oc, os_ = O.rope_tables(pos, dim, heads, mp, double_precision=double_precision)
    assert torch.equal(c.view(torch.int16), oc.view(torch.int16))
    assert torch.equal(s.view(torch.int16), os_.view(torch.int16))
