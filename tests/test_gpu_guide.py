"""Parity of ltxk_guide (GPU): x0 of the four guidance passes, CFG/STG/modality
guidance with std rescale, and the Euler step (standalone/ltx_dit.py:551-562,
592-606) against the oracle on the same bf16 inputs.

Without rescale every fp32 operation matches the oracle's, so the outputs are
bit-exact.  With rescale the two standard deviations are fp64 sums in a
different order, so the factor may differ in its last fp32 bit: the outputs
must be bit-exact at >= 99.9% of elements and otherwise within one bf16 ulp."""

import pytest
import torch

from conftest import assert_close_bf16
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"

VIDEO = dict(cfg_scale=3.0, stg_scale=1.0, modality_scale=3.0, rescale_scale=0.7)   # run_all.py:43
AUDIO = dict(cfg_scale=7.0, stg_scale=1.0, modality_scale=3.0, rescale_scale=0.7)   # run_all.py:44
NO_RESCALE = dict(cfg_scale=3.0, stg_scale=1.0, modality_scale=3.0, rescale_scale=0.0)
NEUTRAL = dict(cfg_scale=1.0, stg_scale=0.0, modality_scale=1.0, rescale_scale=0.0)


def _inputs(b, t, c, seed, keyframe_tokens=0, per_token=True):
    g = torch.Generator().manual_seed(seed)
    lat = torch.randn(b, t, c, generator=g).to(torch.bfloat16)
    # velocities near the latent scale with pass-to-pass differences, as the model gives
    base = torch.randn(b, t, c, generator=g)
    vel = torch.cat([base + 0.3 * torch.randn(b, t, c, generator=g) for _ in range(4)]).to(torch.bfloat16)
    sigma = 0.8
    if per_token:
        mask = torch.ones(b, t, 1)
        mask[:, :keyframe_tokens] = 0.0        # conditioning tokens are not denoised
        ts = (mask.repeat(4, 1, 1) * sigma).contiguous()
    else:
        ts = torch.full((4, 1, 1), sigma)
    return lat, vel, ts


def _check(got, want, exact, what):
    got = got.cpu()
    if exact:
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), what
        return
    same = (got.view(torch.int16) == want.view(torch.int16)).float().mean().item()
    assert same >= 0.999, f"{what}: {same:.5f} bit-equal"
    diff = (got.float() - want.float()).abs()
    ulp = 2.0 ** (torch.floor(torch.log2(want.float().abs().clamp_min(2.0**-126))) - 7)
    assert bool((diff <= ulp).all()), f"{what}: max diff {diff.max().item()}"


@pytest.mark.parametrize("shape,kf", [((1, 6144, 128), 0), ((1, 126, 128), 0), ((1, 3456, 128), 384),
                                      ((2, 33, 64), 5), ((1, 1, 8), 0)])
@pytest.mark.parametrize("params", [VIDEO, AUDIO, NO_RESCALE, NEUTRAL], ids=["video", "audio", "plain", "neutral"])
def test_guide_matches_oracle(shape, kf, params):
    import ltxk

    b, t, c = shape
    lat, vel, ts = _inputs(b, t, c, 7 + t, kf)
    sigma, dt = 0.8, -0.0625
    want_den, want_next, want_x0 = O.guided_step(lat, vel, ts, **params, sigma=sigma, dt=dt)
    den, nxt, x0 = ltxk.guide(lat.to(DEV), vel.to(DEV), ts.to(DEV), **params, sigma=sigma, dt=dt, want_x0=True)
    torch.cuda.synchronize()
    exact = params["rescale_scale"] == 0
    assert torch.equal(x0.cpu().view(torch.int16), want_x0.view(torch.int16))
    _check(den, want_den, exact, "denoised")
    _check(nxt, want_next, exact, "next")


def test_guide_scalar_timesteps_and_in_place_step():
    import ltxk

    lat, vel, ts = _inputs(1, 300, 128, 3, per_token=False)
    want_den, want_next, _ = O.guided_step(lat, vel, ts, **NO_RESCALE, sigma=0.5, dt=-0.1)
    x = lat.to(DEV)
    den, nxt, x0 = ltxk.guide(x, vel.to(DEV), ts.to(DEV), **NO_RESCALE, sigma=0.5, dt=-0.1, next_out=x)
    assert x0 is None and nxt is x
    assert torch.equal(den.cpu(), want_den) and torch.equal(x.cpu(), want_next)


def test_guide_rescale_invariants_at_full_size():
    """r = 1 restores std(cond x0); r = 0.5 sits halfway between r = 0 and r = 1."""
    import ltxk

    lat, vel, ts = _inputs(1, 6144, 128, 11)
    lat, vel, ts = lat.to(DEV), vel.to(DEV), ts.to(DEV)
    p = dict(cfg_scale=3.0, stg_scale=1.0, modality_scale=3.0)
    d1, _, x0 = ltxk.guide(lat, vel, ts, **p, rescale_scale=1.0, want_x0=True)
    d0, _, _ = ltxk.guide(lat, vel, ts, **p, rescale_scale=0.0)
    dh, _, _ = ltxk.guide(lat, vel, ts, **p, rescale_scale=0.5)
    c = x0[:1].float()
    assert abs(float(d1.float().std() / c.std()) - 1) < 1e-3
    d0, d1, dh = d0.float(), d1.float(), dh.float()
    assert bool(((dh - (d0 + d1) / 2).abs() <= 2.0**-7 * (d0.abs() + d1.abs()) + 1e-6).all())


def test_guide_argument_errors():
    import ltxk

    lat, vel, ts = _inputs(1, 16, 64, 5)
    with pytest.raises(ValueError):
        ltxk.guide(lat.to(DEV), vel[:2].to(DEV), ts.to(DEV), **VIDEO)
    with pytest.raises(ValueError):
        ltxk.guide(lat.to(DEV), vel.to(DEV), ts[:2].to(DEV), **VIDEO)
    with pytest.raises(ValueError):
        ltxk.guide(lat.to(DEV), vel.to(DEV), ts.to(DEV), **VIDEO, sigma=0.5)


def test_guide_from_x0_matches_oracle():
    """ltx_dit.guide(cond, uncond, ptb, mod, params): the four x0 given directly."""
    import ltx_dit

    g = torch.Generator().manual_seed(21)
    parts = [torch.randn(1, 500, 128, generator=g).to(torch.bfloat16) for _ in range(4)]
    for params in (VIDEO, NO_RESCALE):
        gp = ltx_dit.GuiderParams(**params, stg_blocks=(28,))
        got = ltx_dit.guide(*[x.to(DEV) for x in parts], gp)
        want = O.guide(*parts, **params)
        _check(got, want, params["rescale_scale"] == 0, "guide")


class _NoTables:
    """Stands in for LTXModel's ArgsPreprocessor: run_dit asks it once per run
    for the RoPE tables of the positions; the fixed-velocity model needs none."""

    def rope_tables(self, positions, cross=True):
        return None


class _FixedVelocityModel:
    """Stands in for LTXModel: returns fixed per-pass velocities and records the
    modalities it was called with."""

    def __init__(self, vx, ax):
        self.vx, self.ax, self.calls = vx, ax, []
        self.video_pre = self.audio_pre = _NoTables()

    def __call__(self, video, audio, perturbations):
        self.calls.append((video, audio, perturbations))
        return self.vx, self.ax


def test_run_dit_steps_match_oracle():
    """run_dit's fused guidance + Euler step per modality against the oracle's
    x0 -> guide -> euler_step chain, two steps of the reference's scheduler."""
    import ltx_dit

    cfg = ltx_dit.DiTConfig(num_layers=2)
    g = torch.Generator().manual_seed(5)
    tv, ta, c = 96, 20, 128
    v0 = torch.randn(1, tv, c, generator=g).to(torch.bfloat16)
    a0 = torch.randn(1, ta, c, generator=g).to(torch.bfloat16)
    vmask = torch.ones(1, tv, 1)
    vmask[:, :8] = 0.0
    vx = torch.randn(4, tv, c, generator=g).to(torch.bfloat16)
    ax = torch.randn(4, ta, c, generator=g).to(torch.bfloat16)
    vs = ltx_dit.LatentState(latent=v0.to(DEV), denoise_mask=vmask.to(DEV), positions=torch.zeros(1, 3, tv, 2, device=DEV),
                             clean_latent=v0.to(DEV), keyframes_mask=torch.zeros(1, tv, 1, device=DEV))
    as_ = ltx_dit.LatentState(latent=a0.to(DEV), denoise_mask=torch.ones(1, ta, 1, device=DEV),
                              positions=torch.zeros(1, 1, ta, 2, device=DEV), clean_latent=a0.to(DEV))
    ctx = {k: torch.zeros(1, 4, 8, device=DEV, dtype=torch.bfloat16) for k in ("v_pos", "v_neg", "a_pos", "a_neg")}
    vp = ltx_dit.GuiderParams(**VIDEO, stg_blocks=(1,))
    ap = ltx_dit.GuiderParams(**AUDIO, stg_blocks=(1,))
    sigmas = ltx_dit.ltx2_scheduler_sigmas(4, tokens=tv).to(DEV)   # on the device, as run_all.py:74
    model = _FixedVelocityModel(vx.to(DEV), ax.to(DEV))
    seen = []
    got_v, got_a = ltx_dit.run_dit(model, cfg, ctx, vs, as_, sigmas[:3], vp, ap,
                                   on_step=lambda i, dt_, dv, da, r, v, a: seen.append(sorted(r)))
    assert seen == [sorted(["cond", "uncond", "ptb", "mod"])] * 2
    want_v, want_a = v0, a0
    for idx in range(2):
        hs = sigmas.cpu()
        sigma, dt = float(hs[idx]), float(hs[idx + 1] - hs[idx])
        video = model.calls[idx][0]
        assert tuple(video.timesteps.shape) == (4, tv, 1)
        ts_v = (vmask.repeat(4, 1, 1) * hs[idx]).float()
        ts_a = (torch.ones(4, ta, 1) * hs[idx]).float()
        _, want_v, _ = O.guided_step(want_v, vx, ts_v, **VIDEO, sigma=sigma, dt=dt)
        _, want_a, _ = O.guided_step(want_a, ax, ts_a, **AUDIO, sigma=sigma, dt=dt)
    _check(got_v, want_v, False, "video latent after 2 steps")
    _check(got_a, want_a, False, "audio latent after 2 steps")
