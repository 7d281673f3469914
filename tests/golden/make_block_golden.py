"""Writes model-level golden vectors with the reference's own LTXModel.

Block.forward's op order, its AdaLN row mapping (ltx_dit.py:192-206,237-317), the
A2V/V2A wiring, the perturbation masks (ltx_dit.py:381-411) and the output head
(ltx_dit.py:371-378) are not fixed by any closed form or library routine, so this
script runs the reference (standalone/ltx_dit.py, ltx_nn.py, imported from
/root/reference in the build container, CPU) on a small configuration with the
same structure and stores inputs and outputs in block_golden.npz (B=1 plain, B=4
with the perturbation masks, and B=1 with the video or the audio stream disabled).

Weights are not stored: every parameter, in sorted-name order, is drawn from one
CPU torch.Generator seeded WEIGHT_SEED as randn(shape) * 0.02 and rounded to bf16;
tests rebuild them the same way (init_weights below).

The same is written to block_golden_ltx2.npz for the configuration that
DiTConfig.from_checkpoint gives when a checkpoint's metadata leaves its optional
keys out (ltx_dit.py:68-72): no cross-attention AdaLN (6-row tables, the text
cross-attention added ungated, ltx_dit.py:237-248), no per-head attention gates,
biased video FFN projections, the fp32 RoPE frequency grid and no keyframe
embedding.

Run from the repository root: python tests/golden/make_block_golden.py
"""
import pathlib
import sys

import numpy as np
import torch

REF = pathlib.Path("/root/reference/standalone")
OUT = pathlib.Path(__file__).resolve().parent / "block_golden.npz"
OUT_LTX2 = pathlib.Path(__file__).resolve().parent / "block_golden_ltx2.npz"
WEIGHT_SEED = 2024
SMALL = dict(num_layers=2, video_heads=2, video_head_dim=64, video_in=128, video_out=128, video_cross_dim=128,
             audio_heads=2, audio_head_dim=32, audio_in=128, audio_out=128, audio_cross_dim=64)
LTX2_FLAGS = dict(cross_attention_adaln=False, gated_attention=False, ff_bias=True, double_rope=False,
                  use_keyframes=False)


def init_weights(model: torch.nn.Module) -> None:
    g = torch.Generator().manual_seed(WEIGHT_SEED)
    params = dict(model.named_parameters())
    with torch.no_grad():
        for name in sorted(params):
            p = params[name]
            p.copy_((torch.randn(p.shape, generator=g) * 0.02).to(torch.bfloat16).to(p.dtype))


def make_inputs(ltx_dit, batch: int, seed: int = 7):
    g = torch.Generator().manual_seed(seed)
    f, h, w, ta, s = 2, 2, 3, 5, 7
    tv = f * h * w
    sigma = torch.full((batch,), 0.5)
    r = lambda *shape: torch.randn(*shape, generator=g).to(torch.bfloat16)  # noqa: E731
    kf = torch.zeros(batch, tv, 1)
    kf[:, : h * w] = 1.0
    vlat, alat = r(batch, tv, 128), r(batch, ta, 128)
    vctx, actx = r(batch, s, 128), r(batch, s, 64)
    vpos = ltx_dit.video_positions(batch, f, h, w, 24.0, torch.device("cpu"))
    apos = ltx_dit.audio_positions(batch, ta, torch.device("cpu"))
    return dict(vlat=vlat, alat=alat, vctx=vctx, actx=actx, vpos=vpos, apos=apos, kf=kf, sigma=sigma)


def modalities(ltx_dit, inp, dtype, video_enabled=True, audio_enabled=True):
    b = inp["vlat"].shape[0]
    v = ltx_dit.Modality(latent=inp["vlat"].to(dtype), sigma=inp["sigma"],
                         timesteps=torch.ones(b, inp["vlat"].shape[1], 1) * inp["sigma"].view(b, 1, 1),
                         positions=inp["vpos"], context=inp["vctx"].to(dtype), keyframes_mask=inp["kf"],
                         enabled=video_enabled)
    a = ltx_dit.Modality(latent=inp["alat"].to(dtype), sigma=inp["sigma"],
                         timesteps=torch.ones(b, inp["alat"].shape[1], 1) * inp["sigma"].view(b, 1, 1),
                         positions=inp["apos"], context=inp["actx"].to(dtype), enabled=audio_enabled)
    return v, a


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main() -> None:
    sys.dont_write_bytecode = True  # the reference tree is read-only: no __pycache__ there
    sys.path.insert(0, str(REF))
    import ltx_dit  # noqa: E402  (reference module)

    for flags, out in (({}, OUT), (LTX2_FLAGS, OUT_LTX2)):
        write(ltx_dit, flags, out)


def write(ltx_dit, flags: dict, out: pathlib.Path) -> None:
    cfg = ltx_dit.DiTConfig(**SMALL, **flags)
    model = ltx_dit.LTXModel(cfg)
    init_weights(model)
    data = {"param_names": np.array(sorted(n for n, _ in model.named_parameters()))}
    for batch, pert in ((1, False), (4, True)):
        inp = make_inputs(ltx_dit, batch)
        key = f"b{batch}"
        for k, v in inp.items():
            data[f"{key}_{k}"] = bits(v) if v.dtype == torch.bfloat16 else v.numpy()
        for dtype, tag in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
            m = model.to(dtype)
            v, a = modalities(ltx_dit, inp, dtype)
            p = None
            if pert:
                p = ltx_dit.build_perturbation_config(cfg.num_layers, ["cond", "uncond", "ptb", "mod"], [1], [0],
                                                      torch.device("cpu"), dtype)
            with torch.no_grad():
                vx, ax = m(v, a, p)
            data[f"{key}_vx_{tag}"] = vx.float().numpy()
            data[f"{key}_ax_{tag}"] = ax.float().numpy()
    # one stream disabled (Modality.enabled False, ltx_dit.py:254-257): its rows
    # pass through the blocks (A2V or V2A still reads them), B=1 inputs
    inp = make_inputs(ltx_dit, 1)
    for dis in ("video", "audio"):
        for dtype, tag in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
            v, a = modalities(ltx_dit, inp, dtype, video_enabled=dis != "video", audio_enabled=dis != "audio")
            with torch.no_grad():
                vx, ax = model.to(dtype)(v, a, None)
            data[f"b1_no{dis}_vx_{tag}"] = vx.float().numpy()
            data[f"b1_no{dis}_ax_{tag}"] = ax.float().numpy()
    np.savez_compressed(out, **data)
    print(f"wrote {out} ({out.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
