"""Host-side logic of the model wrapper that needs no GPU: the de-duplicated
timesteps (one AdaLN row per distinct timestep value, ltx_dit.py:146-150 embeds
every token), the binding's refusal of CPU tensors (no CPU fallback) and the
patchify/unpatchify token layouts."""

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


def _small_cfg(ltx_dit):
    return ltx_dit.DiTConfig(num_layers=2, video_heads=2, video_head_dim=64, video_in=128, video_out=128,
                             video_cross_dim=128, audio_heads=2, audio_head_dim=32, audio_in=128, audio_out=128,
                             audio_cross_dim=64)


def test_block_contexts_accept_inference_parameters():
    """A model built inside torch.inference_mode() (as the reference's pipeline
    loads its transformer) has inference-tensor parameters, which carry no
    in-place version counter: stacking every block's prompt table must not
    read one.  On the CPU the call gets as far as the binding, which refuses
    the CPU tensors."""
    ltx_dit = _ltx_dit()
    with torch.inference_mode():
        model = ltx_dit.LTXModel(_small_cfg(ltx_dit))
        for p in model.parameters():
            p.zero_()
        assert all(p.is_inference() for p in model.parameters())
        args = ltx_dit.TransformerArgs(
            x=torch.zeros(1, 4, 128), context=torch.zeros(1, 3, 128), context_mask=None, timesteps=None,
            embedded_timestep=None, pe=None, cross_pe=None, cross_scale_shift_timestep=None,
            cross_gate_timestep=None, enabled=True, prompt_timestep=torch.zeros(1, 1, 256))
        with pytest.raises(RuntimeError, match="ROCm device"):
            model._block_contexts(args, "prompt_scale_shift_table")


def test_block_contexts_fall_back_above_the_size_limit(monkeypatch):
    """Above BLOCK_CONTEXTS_MAX_BYTES each block modulates its own context."""
    ltx_dit = _ltx_dit()
    model = ltx_dit.LTXModel(_small_cfg(ltx_dit))
    args = ltx_dit.TransformerArgs(
        x=torch.zeros(1, 4, 128), context=torch.zeros(1, 3, 128), context_mask=None, timesteps=None,
        embedded_timestep=None, pe=None, cross_pe=None, cross_scale_shift_timestep=None,
        cross_gate_timestep=None, enabled=True, prompt_timestep=torch.zeros(1, 1, 256))
    monkeypatch.setattr(ltx_dit.LTXModel, "BLOCK_CONTEXTS_MAX_BYTES", 2 * 3 * 128 * 2 - 1)
    assert model._block_contexts(args, "prompt_scale_shift_table") is None


def test_perturbation_table_holds_its_host_copy():
    """PerturbationTable.of copies the keep-mask to the host once; the forward
    takes the copy from it, and makes a copy per call of a bare tensor."""
    ltx_dit = _ltx_dit()
    p = ltx_dit.build_perturbation_config(3, ["cond", "uncond", "ptb", "mod"], [1], [0], torch.device("cpu"),
                                          torch.bfloat16)
    t = ltx_dit.PerturbationTable.of(p)
    assert t.mask is p and t.host.dtype == torch.float32 and torch.equal(t.host, p.float())
    mask, host = ltx_dit.LTXModel._host_perturbations(t)
    assert mask is p and host is t.host
    mask, host = ltx_dit.LTXModel._host_perturbations(p)
    assert mask is p and torch.equal(host, p.float())
    assert ltx_dit.LTXModel._host_perturbations(None) == (None, None)


def test_connector_token_move_is_a_stable_partition():
    """ltx_te.kept_first: scattering by its destinations equals the reference's
    stable descending argsort of the keep flags (ltx_te.py:249-253), on masks
    with left, right, inner and no padding."""
    import ltx_te

    g = torch.Generator().manual_seed(3)
    masks = [torch.tensor([[0, 0, 1, 1, 0, 1], [1] * 6, [0] * 6, [1, 0, 1, 0, 1, 0]])]
    masks.append((torch.rand(5, 33, generator=g) > 0.4).to(torch.int64))
    for mask in masks:
        keep = mask >= 1
        dest, n_kept = ltx_te.kept_first(keep)
        f = torch.randn(*mask.shape, 3, generator=g)
        moved = torch.empty_like(f).scatter_(1, dest.unsqueeze(-1).expand_as(f), f)
        order = torch.argsort(keep.to(torch.int32), dim=-1, descending=True, stable=True)
        assert torch.equal(moved, torch.gather(f, 1, order.unsqueeze(-1).expand_as(f)))
        assert torch.equal(n_kept.view(-1), keep.sum(1))
        assert torch.equal(torch.sort(dest, dim=1).values, torch.arange(mask.shape[1]).expand_as(dest))


def test_connector_checkpoint_keys():
    """The connector and feature-projection key renames of the checkpoints
    (ltx_te.py:294-310)."""
    import ltx_te

    pre = "model.diffusion_model."
    assert ltx_te._connector_key(pre + "video_embeddings_connector.transformer_1d_blocks.3.attn1.to_out.0.weight") \
        == "video_connector.blocks.3.attn1.to_out.weight"
    assert ltx_te._connector_key(pre + "audio_embeddings_connector.transformer_1d_blocks.0.ff.net.0.proj.bias") \
        == "audio_connector.blocks.0.ff.proj_in.bias"
    assert ltx_te._connector_key(pre + "audio_embeddings_connector.learnable_registers") \
        == "audio_connector.learnable_registers"
    assert ltx_te._connector_key(pre + "transformer_blocks.0.attn1.to_q.weight") is None
    assert ltx_te._feature_key("text_embedding_projection.audio_aggregate_embed.bias") \
        == "feature_extractor.audio_aggregate_embed.bias"
    assert ltx_te._feature_key("model.layers.0.mlp.weight") is None
    kw = ltx_te._connector_kwargs({"connector_num_attention_heads": 16, "audio_connector_attention_head_dim": 64,
                                   "connector_num_learnable_registers": 64}, audio=True)
    assert kw["heads"] == 16 and kw["dim_head"] == 64 and kw["registers"] == 64 and kw["num_layers"] == 8
    assert ltx_te._connector_kwargs({"audio_connector_attention_head_dim": 64}, audio=False)["dim_head"] == 128


def test_patchify_layouts_and_round_trips():
    """patchify/unpatchify (ltx_dit.py:468-484): video latent (B, C, F, H, W) ->
    tokens (B, F*H*W, C) in (f, h, w) order with channels last; audio latent
    (B, C, T, M) -> (B, T, C*M) with the channel major in each token; each
    unpatchify inverts its patchify exactly."""
    from einops import rearrange

    ltx_dit = _ltx_dit()
    g = torch.Generator().manual_seed(11)
    v = torch.randn(2, 128, 3, 4, 5, generator=g).to(torch.bfloat16)
    tv = ltx_dit.patchify_video(v)
    assert tv.shape == (2, 60, 128)
    assert torch.equal(tv, rearrange(v, "b c f h w -> b (f h w) c"))
    assert torch.equal(tv[1, 2 * 20 + 3 * 5 + 4], v[1, :, 2, 3, 4])
    assert torch.equal(ltx_dit.unpatchify_video(tv, 3, 4, 5), v)
    a = torch.randn(2, 8, 7, 16, generator=g).to(torch.bfloat16)
    ta = ltx_dit.patchify_audio(a)
    assert ta.shape == (2, 7, 128)
    assert torch.equal(ta, rearrange(a, "b c t m -> b t (c m)"))
    assert torch.equal(ta[0, 6, 3 * 16 + 9], a[0, 3, 6, 9])
    assert torch.equal(ltx_dit.unpatchify_audio(ta, 8, 16), a)
