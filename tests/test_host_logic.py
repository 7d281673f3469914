"""Host-side logic of the model wrapper that needs no GPU: the de-duplicated
timesteps (one AdaLN row per distinct timestep value, ltx_dit.py:146-150 embeds
every token) and the binding's refusal of CPU tensors (no CPU fallback)."""

import pytest
import torch


def _ltx_dit():
    import ltx_dit

    return ltx_dit


def test_uniform_timesteps_give_one_row_per_item():
    ltx_dit = _ltx_dit()
    sig = torch.tensor([0.5, 0.25, 0.75])
    ts = sig.view(3, 1, 1).expand(3, 40, 1).contiguous()
    r = ltx_dit.timestep_rows(ts)
    assert r.per_item and r.index is None and r.rows == 3
    assert torch.equal(r.values, sig)
    # (B, 1, 1) timesteps need no read at all and give the same rows
    r1 = ltx_dit.timestep_rows(sig.view(3, 1, 1))
    assert r1.per_item and torch.equal(r1.values, sig)


@pytest.mark.parametrize("batch", [1, 4])
def test_keyframe_conditioned_timesteps_index_their_rows(batch):
    """denoise_mask 0 on the conditioning frame, 1 elsewhere, times each item's
    sigma (ltx_dit.py:578): the distinct values, and every token's index picks
    exactly its own value; scaling the rows equals scaling per token."""
    ltx_dit = _ltx_dit()
    t = 6 * 4 * 5
    mask = torch.ones(batch, t, 1)
    mask[:, : 4 * 5] = 0.0
    sig = torch.linspace(0.3, 0.9, batch)
    ts = mask * sig.view(batch, 1, 1)
    r = ltx_dit.timestep_rows(ts)
    assert not r.per_item and r.index.dtype == torch.int32 and r.index.numel() == batch * t
    assert torch.equal(r.values, torch.unique(ts.flatten()))
    assert torch.equal(r.values[r.index.long()], ts.flatten())
    # a loop scales the mask's rows by each step's sigma: the same fp32 products per token
    rm = ltx_dit.timestep_rows(mask)
    s = torch.tensor(0.6180339)
    assert torch.equal(rm.scaled(s).values[rm.index.long()], (mask * s).flatten())


def test_binding_refuses_cpu_tensors():
    import ltxk

    x = torch.zeros(2, 8, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm"):
        ltxk.modulate(x, None, None)
    with pytest.raises(RuntimeError, match="ROCm"):
        ltxk.modulate_layers(x, None, None, 3)
    with pytest.raises(RuntimeError, match="ROCm"):
        ltxk.norm_modulate(x)
