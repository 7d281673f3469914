"""Model-level parity (GPU): the fused LTXModel (ltx-nv_amd/ltx_dit.py) against the
reference's own LTXModel outputs stored in tests/golden/block_golden.npz (2 blocks,
video 12 tokens x 128 (2 heads x 64), audio 5 tokens x 64 (2 x 32), text 7 tokens;
B=1 plain and B=4 with the CFG/STG/modality perturbation masks), and in
tests/golden/block_golden_ltx2.npz for the configuration a checkpoint without its
optional metadata keys gets (no cross-attention AdaLN: 6-row tables and an ungated
text cross-attention; no per-head attention gates; biased video FFN projections; the
fp32 RoPE grid; no keyframe embedding).

GEMMs and attention run in bf16 on PyTorch-ROCm here and in fp32/bf16 on the CPU in
the reference, so the check is statistical: the fused bf16 result must be as close
to the reference's fp32 result as the reference's own bf16 run is (relative L2 within
1.5x of it, and cosine >= 0.999), which a wrong AdaLN row, a swapped shift/scale, a
missing residual or a wrong mask would break by orders of magnitude."""

import importlib.util

import numpy as np
import pytest
import torch

from conftest import GOLDEN, bf16_from_bits

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
G = np.load(GOLDEN / "block_golden.npz")
G_LTX2 = np.load(GOLDEN / "block_golden_ltx2.npz")


def _golden_module():
    spec = importlib.util.spec_from_file_location("make_block_golden", GOLDEN / "make_block_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _model(variant="default"):
    import ltx_dit

    mk = _golden_module()
    cfg = ltx_dit.DiTConfig(**mk.SMALL, **(mk.LTX2_FLAGS if variant == "ltx2" else {}))
    model = ltx_dit.LTXModel(cfg)
    golden = G_LTX2 if variant == "ltx2" else G
    assert sorted(n for n, _ in model.named_parameters()) == list(golden["param_names"])
    mk.init_weights(model)
    return cfg, model.to(DEV, torch.bfloat16).eval()


def _inputs(key, golden=G):
    out = {}
    for name in ("vlat", "alat", "vctx", "actx"):
        out[name] = bf16_from_bits(golden[f"{key}_{name}"]).to(DEV)
    for name in ("vpos", "apos", "kf", "sigma"):
        out[name] = torch.from_numpy(golden[f"{key}_{name}"]).to(DEV)
    return out


def _run(model, cfg, key, pert, uniform_ts=False, golden=G, disabled=None):
    import ltx_dit

    inp = _inputs(key, golden)
    b = inp["vlat"].shape[0]
    tv = 1 if uniform_ts else inp["vlat"].shape[1]
    ta = 1 if uniform_ts else inp["alat"].shape[1]
    v = ltx_dit.Modality(latent=inp["vlat"], sigma=inp["sigma"],
                         timesteps=torch.ones(b, tv, 1, device=DEV) * inp["sigma"].view(b, 1, 1),
                         positions=inp["vpos"], context=inp["vctx"], keyframes_mask=inp["kf"],
                         enabled=disabled != "video")
    a = ltx_dit.Modality(latent=inp["alat"], sigma=inp["sigma"],
                         timesteps=torch.ones(b, ta, 1, device=DEV) * inp["sigma"].view(b, 1, 1),
                         positions=inp["apos"], context=inp["actx"], enabled=disabled != "audio")
    p = None
    if pert:
        p = ltx_dit.build_perturbation_config(cfg.num_layers, ["cond", "uncond", "ptb", "mod"], [1], [0], DEV,
                                              torch.bfloat16)
    with torch.no_grad():
        vx, ax = model(v, a, p)
    torch.cuda.synchronize()
    return vx.float().cpu(), ax.float().cpu()


def _rel(a, b):
    return float((a - b).norm() / b.norm())


def _cos(a, b):
    return float(torch.nn.functional.cosine_similarity(a.flatten(), b.flatten(), dim=0))


@pytest.mark.parametrize("variant", ["default", "ltx2"])
@pytest.mark.parametrize("key,pert", [("b1", False), ("b4", True)])
def test_ltxmodel_matches_reference_outputs(variant, key, pert):
    golden = G_LTX2 if variant == "ltx2" else G
    cfg, model = _model(variant)
    vx, ax = _run(model, cfg, key, pert, golden=golden)
    for name, got in (("vx", vx), ("ax", ax)):
        ref32 = torch.from_numpy(golden[f"{key}_{name}_f32"])
        ref16 = torch.from_numpy(golden[f"{key}_{name}_bf16"])
        assert got.shape == ref32.shape
        e_ours, e_ref = _rel(got, ref32), _rel(ref16, ref32)
        assert _cos(got, ref32) >= 0.999, (name, _cos(got, ref32))
        assert e_ours <= 1.5 * e_ref + 2e-3, \
            f"{variant} {key} {name}: ours {e_ours:.4g} vs reference bf16 {e_ref:.4g}"


@pytest.mark.parametrize("variant", ["default", "ltx2"])
@pytest.mark.parametrize("dis", ["video", "audio"])
def test_ltxmodel_with_a_stream_disabled(variant, dis):
    """Modality.enabled False on one stream (ltx_dit.py:254-257): its rows pass
    through every block (the other stream's AV attention still reads them) and
    both outputs match the reference's, by the criteria above."""
    golden = G_LTX2 if variant == "ltx2" else G
    cfg, model = _model(variant)
    vx, ax = _run(model, cfg, "b1", False, golden=golden, disabled=dis)
    for name, got in (("vx", vx), ("ax", ax)):
        ref32 = torch.from_numpy(golden[f"b1_no{dis}_{name}_f32"])
        ref16 = torch.from_numpy(golden[f"b1_no{dis}_{name}_bf16"])
        assert got.shape == ref32.shape
        e_ours, e_ref = _rel(got, ref32), _rel(ref16, ref32)
        assert _cos(got, ref32) >= 0.999, (name, _cos(got, ref32))
        assert e_ours <= 1.5 * e_ref + 2e-3, \
            f"{variant} no{dis} {name}: ours {e_ours:.4g} vs reference bf16 {e_ref:.4g}"


def _checkpoint_name(name: str) -> str:
    """Our parameter name -> the checkpoint's (the inverse of load_transformer's
    renames, ltx_dit.py:418-425)."""
    k = "transformer_blocks." + name[len("blocks."):] if name.startswith("blocks.") else name
    for ours, theirs in (("to_out.", "to_out.0."), ("ff.proj_in.", "ff.net.0.proj."), ("ff.proj_out.", "ff.net.2.")):
        k = k.replace(ours, theirs)
    return "model.diffusion_model." + k


def test_load_transformer_reads_reference_checkpoint_names(tmp_path):
    """load_transformer on a checkpoint under the reference's key names (with a
    key outside the transformer, which it drops) gives the source model's
    parameters bit for bit and its outputs; a checkpoint missing a parameter
    (other than the keyframe embedding) is refused."""
    import ltx_dit
    from safetensors.torch import save_file

    cfg, src = _model()
    sd = {_checkpoint_name(n): p.detach().cpu().contiguous() for n, p in src.named_parameters()}
    assert "model.diffusion_model.transformer_blocks.0.ff.net.0.proj.weight" in sd
    assert "model.diffusion_model.transformer_blocks.1.audio_ff.net.2.bias" in sd
    assert "model.diffusion_model.transformer_blocks.0.attn1.to_out.0.weight" in sd
    sd["vae.decoder.conv_in.weight"] = torch.zeros(4)
    path = tmp_path / "transformer.safetensors"
    save_file(sd, str(path))
    model = ltx_dit.load_transformer(str(path), cfg)
    got = dict(model.named_parameters())
    assert set(got) == {n for n, _ in src.named_parameters()}
    for n, p in src.named_parameters():
        assert got[n].device.type == "cuda" and got[n].dtype == torch.bfloat16
        assert torch.equal(got[n], p), n
    assert all(torch.equal(a, b) for a, b in zip(_run(model, cfg, "b1", False), _run(src, cfg, "b1", False)))
    del sd["model.diffusion_model.transformer_blocks.1.attn2.to_q.weight"]
    save_file(sd, str(path))
    with pytest.raises(RuntimeError, match="missing keys"):
        ltx_dit.load_transformer(str(path), cfg)


def test_uniform_timesteps_equal_per_token():
    """(B,1,1) timesteps broadcast exactly like the per-token (B,T,1) form."""
    cfg, model = _model()
    vx1, ax1 = _run(model, cfg, "b1", False)
    vx2, ax2 = _run(model, cfg, "b1", False, uniform_ts=True)
    assert _rel(vx2, vx1) < 2e-3 and _rel(ax2, ax1) < 2e-3


def test_block_perturbation_flags_read_once():
    """apply_block_perturbations with the host copy gives the same masks/flags."""
    import ltx_dit

    cfg, _ = _model()
    p = ltx_dit.build_perturbation_config(cfg.num_layers, ["cond", "uncond", "ptb", "mod"], [1], [0], DEV,
                                          torch.bfloat16)
    args = ltx_dit.TransformerArgs(x=torch.zeros(4, 1, 8, device=DEV), context=None, context_mask=None,
                                   timesteps=None, embedded_timestep=None, pe=None, cross_pe=None,
                                   cross_scale_shift_timestep=None, cross_gate_timestep=None, enabled=True,
                                   prompt_timestep=None)
    host = p.cpu().float()
    for blk in range(cfg.num_layers):
        for st, ct in ((0, 2), (1, 3)):
            a1 = ltx_dit.apply_block_perturbations(args, p, blk, st, ct)
            a2 = ltx_dit.apply_block_perturbations(args, p, blk, st, ct, host)
            assert a1.self_attn_all_perturbed == a2.self_attn_all_perturbed
            assert a1.cross_attn_skip_all == a2.cross_attn_skip_all
            for m1, m2 in ((a1.self_attn_perturbation_mask, a2.self_attn_perturbation_mask),
                           (a1.cross_attn_perturbation_mask, a2.cross_attn_perturbation_mask)):
                assert (m1 is None) == (m2 is None)
                if m1 is not None:
                    assert torch.equal(m1, m2)


def test_create_noised_states_reproduces_reference_noise():
    """seed 10, 65 frames at 512x768 -> video [1,3456,128] then audio [1,68,128]
    with the reference GPU's thread policy: the golden noise of m1_philox."""
    import ltx_dit
    import torch_rng

    g = torch_rng.TorchRNG(10, DEV, *torch_rng.ADA_RTX6000)
    vs, as_ = ltx_dit.create_noised_states(1, 65, 512, 768, 24.0, 10, DEV, torch.bfloat16, generator=g)
    assert vs.latent.shape == (1, 3456, 128) and as_.latent.shape == (1, 68, 128)
    gv = np.fromfile(GOLDEN / "m1_philox" / "video_noise.bin", dtype=np.uint16)
    ga = np.fromfile(GOLDEN / "m1_philox" / "audio_noise.bin", dtype=np.uint16)
    v = vs.latent.view(torch.int16).cpu().numpy().view(np.uint16).ravel()
    a = as_.latent.view(torch.int16).cpu().numpy().view(np.uint16).ravel()
    assert (v == gv).mean() > 0.9997 and (a == ga).mean() > 0.999


@pytest.mark.parametrize("key,pert", [("b1", False), ("b4", True)])
def test_block_contexts_in_one_launch_equal_per_block(key, pert, monkeypatch):
    """LTXModel.forward modulates every block's text context in one launch
    (ltxk_modulate_layers); the same forward with each block modulating its own
    context (ltxk_modulate, the reference's placement) gives identical outputs."""
    import ltx_dit

    cfg, model = _model()
    vx1, ax1 = _run(model, cfg, key, pert)
    monkeypatch.setattr(ltx_dit.LTXModel, "_block_contexts", lambda self, args, table: None)
    vx2, ax2 = _run(model, cfg, key, pert)
    assert torch.equal(vx1, vx2) and torch.equal(ax1, ax2)


def test_block_contexts_follow_parameter_updates():
    """A block's prompt table changed in place between forwards is seen by the
    next forward, and that forward equals one of a model built with the new
    table from the start."""
    cfg, model = _model()
    vx1, _ = _run(model, cfg, "b1", False)
    with torch.no_grad():
        model.blocks[1].prompt_scale_shift_table.mul_(3.0)
    vx2, _ = _run(model, cfg, "b1", False)
    cfg2, fresh = _model()
    with torch.no_grad():
        fresh.blocks[1].prompt_scale_shift_table.mul_(3.0)
    vx3, _ = _run(fresh, cfg2, "b1", False)
    assert not torch.equal(vx1, vx2)
    assert torch.equal(vx2, vx3)


def _inference_model():
    """The small model built and cast inside torch.inference_mode(), as the
    reference's pipeline loads its transformer (every parameter an inference
    tensor, which has no in-place version counter)."""
    import ltx_dit

    mk = _golden_module()
    with torch.inference_mode():
        cfg = ltx_dit.DiTConfig(**mk.SMALL)
        model = ltx_dit.LTXModel(cfg)
        mk.init_weights(model)
        model = model.to(DEV, torch.bfloat16).eval()
    assert all(p.is_inference() for p in model.parameters())
    return cfg, model


def _run_inference(model, cfg, key, pert, positions=None, pcfg=None):
    import ltx_dit

    inp = _inputs(key)
    b = inp["vlat"].shape[0]
    with torch.inference_mode():
        vpos = inp["vpos"] if positions is None else positions
        v = ltx_dit.Modality(latent=inp["vlat"], sigma=inp["sigma"],
                             timesteps=torch.ones(b, inp["vlat"].shape[1], 1, device=DEV) * inp["sigma"].view(b, 1, 1),
                             positions=vpos, context=inp["vctx"], keyframes_mask=inp["kf"])
        a = ltx_dit.Modality(latent=inp["alat"], sigma=inp["sigma"],
                             timesteps=torch.ones(b, inp["alat"].shape[1], 1, device=DEV) * inp["sigma"].view(b, 1, 1),
                             positions=inp["apos"], context=inp["actx"])
        p = pcfg
        if pert and p is None:
            p = ltx_dit.build_perturbation_config(cfg.num_layers, ["cond", "uncond", "ptb", "mod"], [1], [0], DEV,
                                                  torch.bfloat16)
        vx, ax = model(v, a, p)
    torch.cuda.synchronize()
    return vx.float().cpu(), ax.float().cpu()


@pytest.mark.parametrize("key,pert", [("b1", False), ("b4", True)])
def test_model_built_under_inference_mode(key, pert):
    """A model whose parameters are inference tensors runs its forward, and
    gives the outputs of the same model built outside inference mode."""
    cfg, model = _model()
    want = _run(model, cfg, key, pert)
    cfg_i, model_i = _inference_model()
    got = _run_inference(model_i, cfg_i, key, pert)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])


def test_inference_tensors_changed_in_place_are_seen():
    """Positions and the perturbation table are inference tensors changed in
    place between two forwards: the second forward equals a forward on fresh
    tensors holding the new values (nothing derived from them is reused)."""
    import ltx_dit

    cfg, model = _inference_model()
    inp = _inputs("b4")
    with torch.inference_mode():
        pos = inp["vpos"].clone()
        pcfg = ltx_dit.build_perturbation_config(cfg.num_layers, ["cond", "uncond", "ptb", "mod"], [1], [0], DEV,
                                                 torch.bfloat16)
    first = _run_inference(model, cfg, "b4", True, positions=pos, pcfg=pcfg)
    with torch.inference_mode():
        pos.mul_(0.5)
        pcfg.fill_(1.0)  # every attention runs in every pass
    second = _run_inference(model, cfg, "b4", True, positions=pos, pcfg=pcfg)
    with torch.inference_mode():
        fresh_pos = (inp["vpos"] * 0.5).clone()
        fresh_p = torch.ones_like(pcfg)
    want = _run_inference(model, cfg, "b4", True, positions=fresh_pos, pcfg=fresh_p)
    assert not torch.equal(first[0], second[0])
    assert torch.equal(second[0], want[0]) and torch.equal(second[1], want[1])


def test_precomputed_tables_equal_per_forward_tables():
    """Modality.rope_tables and a PerturbationTable (what run_dit builds once per
    loop) give the outputs of the forward that derives them itself."""
    import ltx_dit

    cfg, model = _model()
    inp = _inputs("b4")
    b = 4
    p = ltx_dit.build_perturbation_config(cfg.num_layers, ["cond", "uncond", "ptb", "mod"], [1], [0], DEV,
                                          torch.bfloat16)

    def mods(pre):
        kw_v = {"rope_tables": model.video_pre.rope_tables(inp["vpos"])} if pre else {}
        kw_a = {"rope_tables": model.audio_pre.rope_tables(inp["apos"])} if pre else {}
        v = ltx_dit.Modality(latent=inp["vlat"], sigma=inp["sigma"],
                             timesteps=torch.ones(b, inp["vlat"].shape[1], 1, device=DEV) * inp["sigma"].view(b, 1, 1),
                             positions=inp["vpos"], context=inp["vctx"], keyframes_mask=inp["kf"], **kw_v)
        a = ltx_dit.Modality(latent=inp["alat"], sigma=inp["sigma"],
                             timesteps=torch.ones(b, inp["alat"].shape[1], 1, device=DEV) * inp["sigma"].view(b, 1, 1),
                             positions=inp["apos"], context=inp["actx"], **kw_a)
        return v, a

    with torch.no_grad():
        want = model(*mods(False), p)
        got = model(*mods(True), ltx_dit.PerturbationTable.of(p))
        v, a = mods(True)
        v.positions = v.positions.clone()  # tables of another tensor are refused
        with pytest.raises(ValueError, match="another positions tensor"):
            model(v, a, p)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])


def test_forwards_in_two_threads_equal_one_thread():
    """Two host threads running forwards at once (each on its own stream, sharing
    the audio side stream) give the outputs of one thread running them in turn:
    the cross-stream events are per thread."""
    import threading

    cfg, model = _model()
    want = [_run(model, cfg, "b1", False), _run(model, cfg, "b4", True)]
    got = [None, None]

    def work(i, key, pert):
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            for _ in range(3):
                got[i] = _run(model, cfg, key, pert)

    threads = [threading.Thread(target=work, args=(0, "b1", False)), threading.Thread(target=work, args=(1, "b4", True))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    for (wv, wa), (gv, ga) in zip(want, got):
        assert torch.equal(wv, gv) and torch.equal(wa, ga)
