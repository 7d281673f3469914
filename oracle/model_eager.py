"""Eager restatement of the reference's LTXModel forward, for model-level parity.

TEST INFRASTRUCTURE ONLY: tests/ import it to check the fused model
(ltx-nv_amd/ltx_dit.py); the product never imports it.

It follows the reference's op sequence with plain torch ops and none of the
fused model's shortcuts: per-token AdaLN embeddings (standalone/ltx_dit.py:
146-150), get_ada_values sums materialised (:192-206), full RoPE tables
(ltx_nn.py:63-96, through oracle.rope_tables), q/k RMSNorm then split RoPE
(ltx_nn.py:186-218), SDPA, head merge, perturbation blend and 2*sigmoid head
gate (:204-235), GELU-tanh FFN (:239-248), the block's residual order
(ltx_dit.py:250-317), the perturbation flags (:381-394) and the LayerNorm
output head (:371-378).  Every op runs in `dtype` (float32 for the target,
bfloat16 for the reference's own rounding after every op) on the device of
the inputs.

Parameters are read by name from a dict (the fused model's named_parameters:
the checkpoint layout both models share); `cfg` is any object with the
DiTConfig attributes.

Pinned by tests/golden/block_golden.npz: the reference's own LTXModel outputs
(2 blocks, B=1 plain and B=4 with the CFG/STG/modality masks); see
tests/test_oracle.py.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from oracle import oracle as O


def _linear(p, name, x):
    return F.linear(x, p[name + ".weight"], p.get(name + ".bias"))


def _timestep_proj(t: torch.Tensor, dim: int = 256, max_period: float = 10000.0) -> torch.Tensor:
    """Sinusoidal projection with cos first (common.py:138-148)."""
    half = dim // 2
    freqs = torch.exp(-math.log(max_period) * torch.arange(half, dtype=torch.float32, device=t.device) / half)
    a = t[:, None].float() * freqs[None]
    return torch.cat([torch.cos(a), torch.sin(a)], dim=-1)


def _adaln(p, name, t, dtype):
    """AdaLayerNormSingle (ltx_nn.py:133-158): (linear(silu(emb)), emb)."""
    h = _timestep_proj(t).to(dtype)
    h = _linear(p, name + ".emb.timestep_embedder.linear_1", h)
    emb = _linear(p, name + ".emb.timestep_embedder.linear_2", F.silu(h))
    return _linear(p, name + ".linear", F.silu(emb)), emb


def _rms(x, eps, weight=None):
    return F.rms_norm(x, (x.shape[-1],), weight=weight, eps=eps)


def _rope(x, pe):
    """Split rotation per head on token-major (B, T, H*Dh) (ltx_nn.py:99-115)."""
    cos, sin = pe
    b, t, d = x.shape
    h = cos.shape[1]
    xr = x.view(b, t, h, 2, d // (2 * h))
    x1, x2 = xr[..., 0, :], xr[..., 1, :]
    c, s = cos.transpose(1, 2), sin.transpose(1, 2)
    return torch.stack([x1 * c - x2 * s, x2 * c + x1 * s], dim=3).reshape(b, t, d)


def _tables(positions, dim, heads, max_pos, theta, dtype, double_precision):
    """The model's tables (ltx_dit.py:160-170): the frequency grid in fp64 or
    fp32 as DiTConfig.double_rope says."""
    cos, sin = O.rope_tables(positions.detach().float().cpu(), dim, heads, max_pos, theta, out_dtype=dtype,
                             double_precision=double_precision)
    return cos.to(positions.device), sin.to(positions.device)


def _sdpa(q, k, v):
    """softmax(q k^T / sqrt(D)) v.  fp32 on a GPU is evaluated explicitly, a few
    heads at a time (bounded memory at 6144 tokens; every product in fp32);
    otherwise torch's SDPA as the reference calls it (ltx_nn.py:22-26)."""
    if q.dtype != torch.float32 or not q.is_cuda:
        return F.scaled_dot_product_attention(q, k, v)
    out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(q.shape[-1])
    for b in range(q.shape[0]):
        for h in range(0, q.shape[1], 8):
            s = torch.matmul(q[b, h:h + 8], k[b, h:h + 8].transpose(-1, -2).contiguous()) * scale
            out[b, h:h + 8] = torch.matmul(torch.softmax(s, dim=-1), v[b, h:h + 8])
    return out


def _attention(p, name, x, ctx, heads, dim_head, eps, pe=None, k_pe=None, pmask=None, all_perturbed=False):
    """Attention.forward (ltx_nn.py:194-236)."""
    ctx = x if ctx is None else ctx
    b = x.shape[0]
    v = _linear(p, name + ".to_v", ctx)
    if all_perturbed:
        out = v
    else:
        q = _rms(_linear(p, name + ".to_q", x), eps, p[name + ".q_norm.weight"])
        k = _rms(_linear(p, name + ".to_k", ctx), eps, p[name + ".k_norm.weight"])
        if pe is not None:
            q = _rope(q, pe)
            k = _rope(k, pe if k_pe is None else k_pe)
        q4 = q.view(b, -1, heads, dim_head).transpose(1, 2)
        k4 = k.view(b, -1, heads, dim_head).transpose(1, 2)
        v4 = v.view(b, -1, heads, dim_head).transpose(1, 2)
        out = _sdpa(q4, k4, v4)
        out = out.transpose(1, 2).reshape(b, -1, heads * dim_head)
        if pmask is not None:
            out = out * pmask + v * (1 - pmask)
    if name + ".to_gate_logits.weight" in p:
        g = _linear(p, name + ".to_gate_logits", x)
        t = out.shape[1]
        out = (out.view(b, t, heads, dim_head) * (2.0 * torch.sigmoid(g)).unsqueeze(-1)).view(b, t, heads * dim_head)
    return _linear(p, name + ".to_out", out)


def _ada(table, ts, b, idx):
    """get_ada_values (ltx_dit.py:192-198): table[idx] + per-token rows, unbound."""
    n = table.shape[0]
    return (table[idx][None, None].to(ts.dtype) + ts.reshape(b, ts.shape[1], n, -1)[:, :, idx, :]).unbind(dim=2)


def _prepare(p, cfg, m, cross, audio: bool, dtype):
    """ArgsPreprocessor.prepare (ltx_dit.py:131-184), per-token AdaLN."""
    pre = "audio_" if audio else ""
    dim = cfg.audio_dim if audio else cfg.video_dim
    x = _linear(p, pre + "patchify_proj", m.latent.to(dtype))
    if not audio and m.keyframes_mask is not None and "keyframes_abs_pos_embedding" in p:
        x = x + (m.keyframes_mask > 0).to(dtype) * p["keyframes_abs_pos_embedding"]
    b = x.shape[0]
    ts = (m.timesteps * cfg.timestep_scale_multiplier).flatten()
    temb, emb = _adaln(p, pre + "adaln_single", ts, dtype)
    a = {"x": x, "timesteps": temb.view(b, -1, temb.shape[-1]), "embedded": emb.view(b, -1, emb.shape[-1]),
         "enabled": getattr(m, "enabled", True)}
    a["prompt"] = None  # no prompt AdaLN without cross-attention AdaLN (ltx_dit.py:334)
    if pre + "prompt_adaln_single.linear.weight" in p:
        pt, _ = _adaln(p, pre + "prompt_adaln_single", (m.sigma * cfg.timestep_scale_multiplier).flatten(), dtype)
        a["prompt"] = pt.view(b, -1, pt.shape[-1])
    a["context"] = m.context.to(dtype).view(b, -1, dim)
    heads = cfg.audio_heads if audio else cfg.video_heads
    max_pos = list(cfg.audio_max_pos) if audio else list(cfg.video_max_pos)
    a["pe"] = _tables(m.positions, dim, heads, max_pos, cfg.theta, dtype, cfg.double_rope)
    a["cross_pe"] = _tables(m.positions[:, 0:1], cfg.audio_cross_dim, heads,
                            [max(cfg.video_max_pos[0], cfg.audio_max_pos[0])], cfg.theta, dtype, cfg.double_rope)
    css, _ = _adaln(p, f"av_ca_{'audio' if audio else 'video'}_scale_shift_adaln_single", ts, dtype)
    a["css"] = css.view(b, -1, css.shape[-1])
    factor = cfg.av_ca_timestep_scale_multiplier / cfg.timestep_scale_multiplier
    cg, _ = _adaln(p, f"av_ca_{'v2a' if audio else 'a2v'}_gate_adaln_single",
                   (cross.sigma * cfg.timestep_scale_multiplier * factor).flatten(), dtype)
    a["cgate"] = cg.view(b, -1, cg.shape[-1])
    return a


def _flags(pcfg, blk, self_type, cross_type):
    """apply_block_perturbations (ltx_dit.py:381-394)."""
    zero = pcfg[self_type, blk] == 0
    all_self, any_self = bool(zero.all()), bool(zero.any())
    all_cross = bool((pcfg[cross_type, blk] == 0).all())
    return dict(smask=pcfg[self_type, blk].reshape(-1, 1, 1) if any_self and not all_self else None,
                sall=all_self, cmask=None if all_cross else pcfg[cross_type, blk].reshape(-1, 1, 1), cskip=all_cross)


def _block(p, cfg, i, va, aa, fv, fa):
    """Block.forward (ltx_dit.py:250-317) for the AV case.  A stream whose
    Modality.enabled is False (ltx_dit.py:254-257) skips its self/text
    attention, its side of the AV attentions and its FFN; the other side's AV
    attention still reads its rows."""
    pre = f"blocks.{i}."
    eps = cfg.norm_eps
    vx, ax = va["x"], aa["x"]

    def self_text(x, a, f, s, heads, dh):
        b = x.shape[0]
        sst = p[pre + s + "scale_shift_table"]
        shift, scale, gate = _ada(sst, a["timesteps"], b, slice(0, 3))
        attn1 = "audio_attn1" if s else "attn1"
        attn2 = "audio_attn2" if s else "attn2"
        out = _attention(p, pre + attn1, _rms(x, eps) * (1 + scale) + shift, None, heads, dh, eps, pe=a["pe"],
                         pmask=f["smask"], all_perturbed=f["sall"])
        x_fma = x + out * gate
        xn = _rms(x_fma, eps)
        if a["prompt"] is None:  # Block._text_cross without cross-attention AdaLN (ltx_dit.py:237-248)
            return x_fma + _attention(p, pre + attn2, xn, a["context"], heads, dh, eps)
        shq, scq, g2 = _ada(sst, a["timesteps"], b, slice(6, 9))
        kv = p[pre + s + "prompt_scale_shift_table"][None, None] + a["prompt"].reshape(b, a["prompt"].shape[1], 2, -1)
        shkv, sckv = kv.unbind(dim=2)
        out2 = _attention(p, pre + attn2, xn * (1 + scq) + shq, a["context"] * (1 + sckv) + shkv, heads, dh, eps)
        return x_fma + out2 * g2

    run_v, run_a = va["enabled"] and vx.numel() > 0, aa["enabled"] and ax.numel() > 0
    if run_v:
        vx = self_text(vx, va, fv, "", cfg.video_heads, cfg.video_head_dim)
    if run_a:
        ax = self_text(ax, aa, fa, "audio_", cfg.audio_heads, cfg.audio_head_dim)

    def av(table, a, idx, b):
        sc, sh = (u.squeeze(2) for u in _ada(table[:4], a["css"], b, idx))
        (g,) = (u.squeeze(2) for u in _ada(table[4:], a["cgate"], b, slice(None)))
        return sc, sh, g

    tv, ta = p[pre + "scale_shift_table_a2v_ca_video"], p[pre + "scale_shift_table_a2v_ca_audio"]
    vx_pre, ax_pre = vx, ax
    b = vx.shape[0]
    if run_v and ax.numel() > 0 and not fv["cskip"]:  # A2V (ltx_dit.py:282-296)
        s, sh, gate = av(tv, va, slice(0, 2), b)
        q_in = _rms(vx_pre, eps) * (1 + s) + sh
        s, sh, _ = av(ta, aa, slice(0, 2), b)
        kv_in = _rms(ax_pre, eps) * (1 + s) + sh
        out = _attention(p, pre + "audio_to_video_attn", q_in, kv_in, cfg.audio_heads, cfg.audio_head_dim, eps,
                         pe=va["cross_pe"], k_pe=aa["cross_pe"])
        vx = vx + out * gate * fv["cmask"]
    if run_a and vx.numel() > 0 and not fa["cskip"]:  # V2A (ltx_dit.py:297-307)
        s, sh, gate = av(ta, aa, slice(2, 4), b)
        q_in = _rms(ax_pre, eps) * (1 + s) + sh
        s, sh, _ = av(tv, va, slice(2, 4), b)
        kv_in = _rms(vx_pre, eps) * (1 + s) + sh
        out = _attention(p, pre + "video_to_audio_attn", q_in, kv_in, cfg.audio_heads, cfg.audio_head_dim, eps,
                         pe=aa["cross_pe"], k_pe=va["cross_pe"])
        ax = ax + out * gate * fa["cmask"]

    def ffn(x, a, s):
        sh, sc, gate = _ada(p[pre + s + "scale_shift_table"], a["timesteps"], x.shape[0], slice(3, 6))
        name = pre + ("audio_ff" if s else "ff")
        h = F.gelu(_linear(p, name + ".proj_in", _rms(x, eps) * (1 + sc) + sh), approximate="tanh")
        return x + _linear(p, name + ".proj_out", h) * gate

    va = dict(va, x=ffn(vx, va, "") if run_v else vx)
    aa = dict(aa, x=ffn(ax, aa, "audio_") if run_a else ax)
    return va, aa


def _output(p, cfg, a, pre):
    """LTXModel._output (ltx_dit.py:371-378): LayerNorm (no affine), modulate, project."""
    x = a["x"]
    ss = p[pre + "scale_shift_table"][None, None].to(x.dtype) + a["embedded"][:, :, None]
    shift, scale = ss[:, :, 0], ss[:, :, 1]
    x = F.layer_norm(x, (x.shape[-1],), eps=cfg.norm_eps) * (1 + scale) + shift
    return _linear(p, pre + "proj_out", x)


@torch.no_grad()
def forward(params: dict, cfg, video, audio, perturbations=None, dtype=torch.float32):
    """LTXModel.forward (ltx_dit.py:354-369) for both modalities.  `video`,
    `audio`: objects with the Modality fields (latent, sigma, timesteps,
    positions, context, keyframes_mask).  Returns (video out, audio out)."""
    p = {k: v.to(dtype) for k, v in params.items()}
    va = _prepare(p, cfg, video, audio, False, dtype)
    aa = _prepare(p, cfg, audio, video, True, dtype)
    b = va["x"].shape[0]
    pcfg = perturbations if perturbations is not None else torch.ones(4, cfg.num_layers, b, device=va["x"].device)
    pcfg = pcfg.to(dtype)
    for i in range(cfg.num_layers):
        va, aa = _block(p, cfg, i, va, aa, _flags(pcfg, i, 0, 2), _flags(pcfg, i, 1, 3))
    return _output(p, cfg, va, ""), _output(p, cfg, aa, "audio_")
