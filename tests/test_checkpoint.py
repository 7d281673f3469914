"""Checkpoint boundary on the host (no GPU): DiTConfig.from_checkpoint's reading
of the safetensors metadata (ltx_dit.py:54-73: the required keys, the optional
keys' defaults, the fp64 RoPE grid only for frequencies_precision "float64")
and load_state_dict's filter, rename and float cast (common.py:40-65)."""

import json

import pytest
import torch

REQUIRED = dict(num_layers=48, num_attention_heads=32, attention_head_dim=128, in_channels=128, out_channels=128,
                cross_attention_dim=4096, audio_num_attention_heads=32, audio_attention_head_dim=64,
                audio_out_channels=128, audio_cross_attention_dim=2048, norm_eps=1e-6,
                positional_embedding_theta=10000.0, positional_embedding_max_pos=[20, 2048, 2048],
                audio_positional_embedding_max_pos=[20], timestep_scale_multiplier=1000,
                av_ca_timestep_scale_multiplier=1000.0)


def _write(tmp_path, tensors, transformer, name="ckpt.safetensors"):
    from safetensors.torch import save_file

    path = tmp_path / name
    save_file(tensors, str(path), metadata={"config": json.dumps({"transformer": transformer}), "note": "plain text"})
    return str(path)


def test_config_from_checkpoint_metadata(tmp_path):
    import common
    import ltx_dit

    path = _write(tmp_path, {"x": torch.zeros(1)}, REQUIRED)
    cfg = ltx_dit.DiTConfig.from_checkpoint(path)
    # the optional keys absent: LTX-2's defaults, not DiTConfig's
    assert cfg == ltx_dit.DiTConfig(num_layers=48, video_heads=32, video_head_dim=128, video_in=128, video_out=128,
                                    video_cross_dim=4096, audio_heads=32, audio_head_dim=64, audio_in=128,
                                    audio_out=128, audio_cross_dim=2048, norm_eps=1e-6, theta=10000.0,
                                    video_max_pos=(20, 2048, 2048), audio_max_pos=(20,),
                                    timestep_scale_multiplier=1000, av_ca_timestep_scale_multiplier=1000.0,
                                    double_rope=False, gated_attention=False, cross_attention_adaln=False,
                                    ff_bias=True, audio_ff_bias=True, use_keyframes=False)
    full = dict(REQUIRED, frequencies_precision="float64", apply_gated_attention=True, cross_attention_adaln=True,
                ff_bias=False, audio_ff_bias=False, use_keyframes_abs_pos_embedding=True, audio_in_channels=64,
                num_layers=2)
    cfg2 = ltx_dit.DiTConfig.from_checkpoint(_write(tmp_path, {"x": torch.zeros(1)}, full, "full.safetensors"))
    assert (cfg2.double_rope, cfg2.gated_attention, cfg2.cross_attention_adaln, cfg2.ff_bias, cfg2.audio_ff_bias,
            cfg2.use_keyframes, cfg2.audio_in, cfg2.num_layers) == (True, True, True, False, False, True, 64, 2)
    fp32 = dict(REQUIRED, frequencies_precision="float32")
    assert ltx_dit.DiTConfig.from_checkpoint(_write(tmp_path, {"x": torch.zeros(1)}, fp32, "f.safetensors")).double_rope is False
    meta = common.read_metadata(path)
    assert meta["note"] == "plain text" and meta["config"]["transformer"] == REQUIRED
    with pytest.raises(KeyError):
        ltx_dit.DiTConfig.from_checkpoint(_write(tmp_path, {"x": torch.zeros(1)},
                                                 {k: v for k, v in REQUIRED.items() if k != "norm_eps"}, "m.safetensors"))


def test_load_state_dict_filters_renames_and_casts(tmp_path):
    import common

    g = torch.Generator().manual_seed(3)
    src = {"a.w": torch.randn(3, 4, generator=g), "b.w": torch.randn(2, generator=g),
           "idx": torch.arange(5, dtype=torch.int64), "drop.me": torch.ones(1)}
    path = _write(tmp_path, src, REQUIRED)
    sd = common.load_state_dict(path, device="cpu", dtype=torch.bfloat16, keep=lambda k: k != "b.w",
                                rename=lambda k: None if k.startswith("drop.") else "m." + k)
    assert set(sd) == {"m.a.w", "m.idx"}
    assert sd["m.a.w"].dtype == torch.bfloat16 and torch.equal(sd["m.a.w"], src["a.w"].to(torch.bfloat16))
    assert sd["m.idx"].dtype == torch.int64 and torch.equal(sd["m.idx"], src["idx"])  # integers are not cast
    kept = common.load_state_dict(path, device="cpu", dtype=None)
    assert set(kept) == set(src) and all(torch.equal(kept[k], src[k]) and kept[k].dtype == src[k].dtype for k in src)
