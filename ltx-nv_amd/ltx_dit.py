"""LTX-2.5 audio-video DiT with the reference's module API (standalone/ltx_dit.py),
its memory-bound chain running on the ltxk HIP kernels.

Public names and signatures follow the reference: DiTConfig, Modality,
TransformerArgs, ArgsPreprocessor, get_ada_values, get_av_ca_ada_values, Block,
LTXModel, apply_block_perturbations, build_perturbation_config,
load_transformer, video_positions, audio_positions, patchify/unpatchify,
LatentState, create_noised_states, ltx2_scheduler_sigmas, GuiderParams,
guide, guided_denoise_step, euler_step, run_dit.

What differs is how Block.forward executes the reference's op sequence
(ltx_dit.py:250-317).  AdaLN vectors (table row + timestep embedding) are
read by the kernels directly instead of being materialised, and neighbouring
elementwise ops share one pass over the activation:
  norm+modulate            one ltxk_norm_modulate per pre-attention norm
  residual+norm+modulate   `x + out*gate` fused with the following norm and
                           modulation (text-cross query, FFN input)
  A2V/V2A inputs           both modulations of vx_pre (and of ax_pre) from
                           one read
  q/k norm + RoPE          one in-place launch for q and k
  gate + head merge        one launch on the attention output
The flag reads of apply_block_perturbations use one host copy of the
perturbation table per model call instead of three device syncs per block.
"""

from __future__ import annotations

import math
import threading
import time
from dataclasses import dataclass, replace

import torch

import ltxk
from common import DEVICE, load_state_dict, read_metadata
from ltx_nn import AdaLayerNormSingle, Attention, FeedForward, precompute_freqs_cis, precompute_freqs_cis_compact
from torch_rng import TorchRNG

# ---------------------------------------------------------------------------
# Config
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class DiTConfig:
    num_layers: int = 48
    video_heads: int = 32
    video_head_dim: int = 128
    video_in: int = 128
    video_out: int = 128
    video_cross_dim: int = 4096
    audio_heads: int = 32
    audio_head_dim: int = 64
    audio_in: int = 128
    audio_out: int = 128
    audio_cross_dim: int = 2048
    norm_eps: float = 1e-6
    theta: float = 10000.0
    video_max_pos: tuple = (20, 2048, 2048)
    audio_max_pos: tuple = (20,)
    timestep_scale_multiplier: int = 1000
    av_ca_timestep_scale_multiplier: float = 1000.0
    double_rope: bool = True
    gated_attention: bool = True
    cross_attention_adaln: bool = True
    ff_bias: bool = False
    audio_ff_bias: bool = True
    use_keyframes: bool = True

    @staticmethod
    def from_checkpoint(transformer_path: str) -> "DiTConfig":
        """Config from the checkpoint's safetensors metadata (reference ltx_dit.py:54-73)."""
        c = read_metadata(transformer_path)["config"]["transformer"]
        return DiTConfig(
            num_layers=c["num_layers"], video_heads=c["num_attention_heads"],
            video_head_dim=c["attention_head_dim"], video_in=c["in_channels"], video_out=c["out_channels"],
            video_cross_dim=c["cross_attention_dim"], audio_heads=c["audio_num_attention_heads"],
            audio_head_dim=c["audio_attention_head_dim"], audio_in=c.get("audio_in_channels", 128),
            audio_out=c["audio_out_channels"], audio_cross_dim=c["audio_cross_attention_dim"],
            norm_eps=c["norm_eps"], theta=c["positional_embedding_theta"],
            video_max_pos=tuple(c["positional_embedding_max_pos"]),
            audio_max_pos=tuple(c["audio_positional_embedding_max_pos"]),
            timestep_scale_multiplier=c["timestep_scale_multiplier"],
            av_ca_timestep_scale_multiplier=c["av_ca_timestep_scale_multiplier"],
            double_rope=c.get("frequencies_precision", False) == "float64",
            gated_attention=c.get("apply_gated_attention", False),
            cross_attention_adaln=c.get("cross_attention_adaln", False),
            ff_bias=c.get("ff_bias", True), audio_ff_bias=c.get("audio_ff_bias", True),
            use_keyframes=c.get("use_keyframes_abs_pos_embedding", False),
        )

    @property
    def video_dim(self) -> int:
        return self.video_heads * self.video_head_dim

    @property
    def audio_dim(self) -> int:
        return self.audio_heads * self.audio_head_dim


# ---------------------------------------------------------------------------
# Transformer args
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class TimestepRows:
    """The distinct values of a (B, T, 1) timesteps tensor and each token's row
    among them, so the AdaLN MLPs run once per distinct value instead of once
    per token (the reference embeds every token, ltx_dit.py:146-150).

    per_item: every batch item has a single value; `values` is then (B,) and
    the embeddings broadcast over tokens (index None).  Otherwise `values` is
    (U,) and `index` (B*T,) int32 on the device names each token's row."""

    values: torch.Tensor
    index: torch.Tensor | None
    per_item: bool

    @property
    def rows(self) -> int:
        return self.values.shape[0]

    def scaled(self, factor: torch.Tensor | float) -> "TimestepRows":
        """The rows of timesteps * factor (the same fp32 multiply per value as per token)."""
        return TimestepRows(self.values * factor, self.index, self.per_item)


def timestep_rows(timesteps: torch.Tensor) -> TimestepRows:
    """De-duplicates (B, T, 1) (or (B, 1, 1)) timesteps: one device-to-host read
    of the values, the distinct ones found on the host, the index uploaded."""
    b, t = timesteps.shape[0], timesteps.shape[1]
    flat = timesteps.reshape(b, t)
    if t == 1:
        return TimestepRows(flat[:, 0].contiguous(), None, True)
    host = flat.detach().float().cpu().numpy()
    if bool((host == host[:, :1]).all()):
        return TimestepRows(flat[:, 0].contiguous(), None, True)
    import numpy as np

    vals, inverse = np.unique(host.reshape(-1), return_inverse=True)
    dev = timesteps.device
    return TimestepRows(torch.from_numpy(vals.astype(np.float32)).to(dev),
                        torch.from_numpy(inverse.astype(np.int32)).to(dev), False)


@dataclass(frozen=True)
class RopeTables:
    """A modality's compact RoPE tables, built once for one positions tensor
    (ArgsPreprocessor.rope_tables): `pe` for self-attention over every
    position axis, `cross_pe` for the A2V/V2A attentions over the time axis.
    Handing them to the forward through Modality.rope_tables is the caller's
    statement that `positions` has not changed since they were built."""

    positions: torch.Tensor
    pe: ltxk.CompactRope
    cross_pe: ltxk.CompactRope | None


@dataclass(frozen=True)
class PerturbationTable:
    """A (4, blocks, B) keep-mask (build_perturbation_config) with a host copy
    of it made once.  LTXModel.forward reads the per-block all/any flags from
    the copy instead of the device; passing this object instead of the tensor
    is the caller's statement that the mask has not changed since the copy."""

    mask: torch.Tensor
    host: torch.Tensor

    @staticmethod
    def of(mask: torch.Tensor) -> "PerturbationTable":
        return PerturbationTable(mask, mask.detach().to("cpu", torch.float32))


@dataclass
class Modality:
    latent: torch.Tensor            # (B, T, 128) patchified
    sigma: torch.Tensor             # (B,)
    timesteps: torch.Tensor         # (B, T, 1) = denoise_mask * sigma; (B, 1, 1) when uniform
    positions: torch.Tensor         # video (B, 3, T, 2) bounds; audio (B, 1, T, 2) seconds
    context: torch.Tensor           # (B, S, cross_dim)
    keyframes_mask: torch.Tensor | None = None
    enabled: bool = True
    # Not in the reference API (optional): `timesteps` de-duplicated in advance.
    # run_dit supplies it from the denoise mask it analysed once per run, so the
    # forward reads nothing back from the device; without it prepare() calls
    # timestep_rows (one device-to-host read).
    timestep_rows: TimestepRows | None = None
    # Not in the reference API (optional): RoPE tables built in advance for
    # `positions` (ArgsPreprocessor.rope_tables).  Without them every forward
    # builds the tables from `positions`, as the reference does.
    rope_tables: RopeTables | None = None


@dataclass
class TransformerArgs:
    x: torch.Tensor
    context: torch.Tensor
    context_mask: torch.Tensor | None
    timesteps: torch.Tensor         # (B, T or 1, n*D) embedded
    embedded_timestep: torch.Tensor  # (B, T or 1, D)
    pe: tuple | ltxk.CompactRope | None         # (cos, sin) (B, H, T, Dh/2) or the compact form
    cross_pe: tuple | ltxk.CompactRope | None   # time-axis tables, compact form
    cross_scale_shift_timestep: torch.Tensor | None
    cross_gate_timestep: torch.Tensor | None
    enabled: bool
    prompt_timestep: torch.Tensor | None
    self_attention_mask: torch.Tensor | None = None
    self_attn_perturbation_mask: torch.Tensor | None = None
    self_attn_all_perturbed: bool = False
    cross_attn_perturbation_mask: torch.Tensor | None = None
    cross_attn_skip_all: bool = False
    # A residual `x + f * gate` not yet added to x: (f, gate as ltxk.AdaRef);
    # f None means the gate operand is the addend itself (the keyframe position
    # embedding).  LTXModel.forward leaves each block's FFN residual (and the
    # keyframe add before block 0) pending so that the next block adds it in
    # the same pass as its first norm.
    pending: tuple | None = None
    # Rows of the de-duplicated per-token embeddings (timesteps,
    # embedded_timestep, cross_scale_shift_timestep): None when they broadcast
    # over tokens.
    timestep_index: ltxk.TimestepIndex | None = None
    # This block's text context already modulated by its prompt table (the
    # cross-AdaLN `context * (1 + scale_kv) + shift_kv`, ltx_dit.py:240-246):
    # LTXModel.forward makes every block's in one launch per step.
    block_context: torch.Tensor | None = None


class ArgsPreprocessor:
    """Per-modality input preparation (reference ltx_dit.py:120-184)."""

    def __init__(self, model: "LTXModel", stream: str):
        self.m = model
        self.stream = stream

    @property
    def cfg(self) -> DiTConfig:
        return self.m.cfg

    def rope_tables(self, positions: torch.Tensor, cross: bool = True) -> RopeTables:
        """This stream's RoPE tables for `positions` (ltx_dit.py:160-170) in the
        compact form: self-attention tables over every axis and, with `cross`,
        the A2V/V2A tables over the time axis.  Building them reads the count of
        distinct coordinates back from the device (one read per axis); a
        denoising loop builds them once and passes them on Modality.rope_tables."""
        cfg = self.cfg
        audio = self.stream == "audio"
        dim = cfg.audio_dim if audio else cfg.video_dim
        heads = cfg.audio_heads if audio else cfg.video_heads
        max_pos = list(cfg.audio_max_pos) if audio else list(cfg.video_max_pos)
        pe = self._rope(positions, slice(None), dim, max_pos, heads)
        cross_pe = None
        if cross:
            cross_pe = self._rope(positions, slice(0, 1), cfg.audio_cross_dim,
                                  [max(cfg.video_max_pos[0], cfg.audio_max_pos[0])], heads)
        return RopeTables(positions, pe, cross_pe)

    def _rope(self, positions: torch.Tensor, axes: slice, dim: int, max_pos: list, heads: int) -> ltxk.CompactRope:
        cfg = self.cfg
        return precompute_freqs_cis_compact(positions[:, axes], dim=dim, out_dtype=torch.bfloat16, theta=cfg.theta,
                                            max_pos=max_pos, use_middle_indices_grid=True, num_attention_heads=heads,
                                            double_precision=cfg.double_rope)

    def prepare(self, modality: Modality, cross: Modality | None) -> TransformerArgs:
        m, cfg = self.m, self.cfg
        audio = self.stream == "audio"
        patchify = m.audio_patchify_proj if audio else m.patchify_proj
        adaln = m.audio_adaln_single if audio else m.adaln_single
        prompt_adaln = m.audio_prompt_adaln_single if audio else m.prompt_adaln_single
        dim = cfg.audio_dim if audio else cfg.video_dim

        x = patchify(modality.latent)
        b = x.shape[0]
        pending = None
        if not audio and modality.keyframes_mask is not None and m.keyframes_abs_pos_embedding is not None:
            # x + (kf > 0) * keyframes_abs_pos_embedding (ltx_dit.py:142-144): the
            # addend is one of two rows (zeros, the embedding) per token, added by
            # block 0 in the pass of its first norm through an indexed operand.
            emb = m.keyframes_abs_pos_embedding.to(x.dtype).reshape(1, dim)
            rows = torch.cat([torch.zeros_like(emb), emb]).view(1, 2, dim)
            kidx = (modality.keyframes_mask.reshape(-1) > 0).to(torch.int32)
            pending = (None, ltxk.AdaRef(None, 0, rows, 0, dim=dim, index=ltxk.TimestepIndex(kidx, 2)))

        # AdaLN once per distinct timestep (ltx_dit.py:146-150 embeds every token).
        tsr = modality.timestep_rows if modality.timestep_rows is not None else timestep_rows(modality.timesteps)
        tsr = tsr.scaled(cfg.timestep_scale_multiplier)
        lead = (b, 1) if tsr.per_item else (1, tsr.rows)
        index = None if tsr.per_item else ltxk.TimestepIndex(tsr.index, tsr.rows)
        timestep, embedded = adaln(tsr.values, hidden_dtype=modality.latent.dtype)
        if tsr.per_item and tsr.rows != b:
            raise ValueError(f"per-item timestep rows {tsr.rows} != batch {b}")
        timestep = timestep.view(*lead, timestep.shape[-1])
        embedded = embedded.view(*lead, embedded.shape[-1])
        prompt_timestep = None
        if prompt_adaln is not None:
            pt, _ = prompt_adaln((modality.sigma * cfg.timestep_scale_multiplier).flatten(),
                                 hidden_dtype=modality.latent.dtype)
            prompt_timestep = pt.view(b, -1, pt.shape[-1])

        context = modality.context.view(b, -1, x.shape[-1])
        # RoPE tables (ltx_dit.py:160-170) in the compact form, bit-equal to the
        # full ones: one row per coordinate value of each axis plus a per-token
        # index, a few hundred KB that stay in cache, instead of a 50 MB (self)
        # or 25 MB (A2V/V2A) table streamed beside q/k on every launch.
        tables = modality.rope_tables
        if tables is None:
            tables = self.rope_tables(modality.positions, cross is not None)
        elif tables.positions is not modality.positions or (cross is not None and tables.cross_pe is None):
            raise ValueError("Modality.rope_tables were built for another positions tensor "
                             "(or without the A2V/V2A tables)")
        pe = tables.pe
        cross_pe = cross_ss = cross_gate = None
        if cross is not None:
            cross_pe = tables.cross_pe
            cross_adaln = m.av_ca_audio_scale_shift_adaln_single if audio else m.av_ca_video_scale_shift_adaln_single
            gate_adaln = m.av_ca_v2a_gate_adaln_single if audio else m.av_ca_a2v_gate_adaln_single
            cst, _ = cross_adaln(tsr.values, hidden_dtype=x.dtype)
            cross_ss = cst.view(*lead, cst.shape[-1])
            factor = cfg.av_ca_timestep_scale_multiplier / cfg.timestep_scale_multiplier
            cgt, _ = gate_adaln((cross.sigma * cfg.timestep_scale_multiplier * factor).flatten(), hidden_dtype=x.dtype)
            cross_gate = cgt.view(b, -1, cgt.shape[-1])
        return TransformerArgs(
            x=x, context=context, context_mask=None, timesteps=timestep, embedded_timestep=embedded,
            pe=pe, cross_pe=cross_pe, cross_scale_shift_timestep=cross_ss, cross_gate_timestep=cross_gate,
            enabled=modality.enabled, prompt_timestep=prompt_timestep, pending=pending, timestep_index=index,
        )


# ---------------------------------------------------------------------------
# AdaLN values
# ---------------------------------------------------------------------------


def get_ada_values(table: torch.Tensor, batch: int, timestep: torch.Tensor, indices: slice) -> tuple:
    """Materialised table[indices] + timestep rows (reference ltx_dit.py:192-198).

    Block.forward does not call this: its kernels read the same sums through
    ltxk.AdaRef without writing them out.  Kept for API users.
    """
    num = table.shape[0]
    rows = table[indices].unsqueeze(0).unsqueeze(0).to(device=timestep.device, dtype=timestep.dtype)
    return (rows + timestep.reshape(batch, timestep.shape[1], num, -1)[:, :, indices, :]).unbind(dim=2)


def get_av_ca_ada_values(table, batch, scale_shift_ts, gate_ts, ss_indices):
    """(scale, shift, gate) of an A2V/V2A table (reference ltx_dit.py:201-206)."""
    ss = get_ada_values(table[:4, :], batch, scale_shift_ts, ss_indices)
    g = get_ada_values(table[4:, :], batch, gate_ts, slice(None, None))
    scale, shift = (t.squeeze(2) for t in ss)
    (gate,) = (t.squeeze(2) for t in g)
    return scale, shift, gate


def _bf16(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.bfloat16 and t.is_contiguous() else t.to(torch.bfloat16).contiguous()


def _ada(table: torch.Tensor, row: int, emb, emb_row: int | None = None) -> ltxk.AdaRef:
    """table[row] + the matching row of a timestep embedding.  `emb` is a
    (B, T_e, n*D) tensor, or (tensor, TimestepIndex | None) for the
    per-token embeddings, which are de-duplicated to one row per distinct
    timestep when the index is set."""
    index = None
    if isinstance(emb, tuple):
        emb, index = emb
    return ltxk.AdaRef(_bf16(table), row, emb, emb_row, index=index)


def _apply_pending(x: torch.Tensor, pending: tuple) -> torch.Tensor:
    """x + f * gate (* mask) for a residual left pending; f None: x + gate."""
    f, g = pending[0], pending[1]
    mask = pending[2] if len(pending) > 2 else None
    if f is None:
        return ltxk.add_norm_modulate(x, None, gate=g, mask=mask, norm=False)
    return ltxk.gated_residual(x, f, gate=g, mask=mask)


def _mask_arg(mask: torch.Tensor | None) -> torch.Tensor | None:
    if mask is None:
        return None
    return _bf16(mask.reshape(-1))


# The audio stream's work inside a block is independent of the video stream's
# until the A2V/V2A exchange, and it is small (126 tokens): its kernels are
# launch-bound.  It runs on a second HIP stream of the same (default) priority
# so that it overlaps the video work instead of adding to it.
_SIDE_STREAMS: dict[int, torch.cuda.Stream] = {}
OVERLAP_AUDIO = True


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _SIDE_STREAMS:
        _SIDE_STREAMS[idx] = torch.cuda.Stream(device=idx)
    return _SIDE_STREAMS[idx]


_STREAM_EVENTS = threading.local()


def _events(device: torch.device) -> dict:
    """The cross-stream events of the two-stream block on `device` (fork, join,
    and the A2V/V2A hand-overs each way), made once per host thread and
    re-recorded: one thread runs its blocks one after another, and a wait takes
    the event's latest record.  Per thread, so that forwards running in two
    threads never record over each other's events."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    per_device = getattr(_STREAM_EVENTS, "by_device", None)
    if per_device is None:
        per_device = _STREAM_EVENTS.by_device = {}
    if idx not in per_device:
        with torch.cuda.device(idx):
            per_device[idx] = {k: ltxk.StreamEvent() for k in ("fork", "join", "main_ready", "side_ready")}
    return per_device[idx]


def _qk_pair(a2v: Attention, v2a: Attention, a: torch.Tensor | None, b: torch.Tensor | None, pe,
             k_first: bool = False) -> None:
    """q/k norm + RoPE of one stream's side of both AV attentions in one
    launch: on the video side A2V's queries (a) and V2A's keys (b), on the
    audio side (k_first) A2V's keys (a) and V2A's queries (b).  Both use that
    stream's time-axis tables; either may be absent."""
    if a2v.heads != v2a.heads or a2v.dim_head != v2a.dim_head:
        raise ValueError("A2V and V2A attentions must have the same head layout")
    wa = a2v.k_norm.weight if k_first else a2v.q_norm.weight
    wb = v2a.q_norm.weight if k_first else v2a.k_norm.weight
    if a is None and b is None:
        return
    if a is None:
        a, wa, b, wb = b, wb, None, None
    ltxk.qk_norm_rope(a, b, a2v.heads, a2v.dim_head, q_weight=wa, k_weight=wb, q_pe=pe,
                      k_pe=pe if b is not None else None, eps=a2v.eps)


def _hand_over(stream: torch.cuda.Stream, *tensors) -> None:
    """Tensors made on another stream and read on `stream`: keep their memory
    from being reused until `stream`'s work that reads them has run."""
    for t in tensors:
        if isinstance(t, torch.Tensor):
            t.record_stream(stream)


# ---------------------------------------------------------------------------
# Blocks
# ---------------------------------------------------------------------------


class Block(torch.nn.Module):
    """BasicAVTransformerBlock: video + audio streams with A<->V cross attention (ltx_dit.py:209-317)."""

    def __init__(self, cfg: DiTConfig):
        super().__init__()
        v, a = cfg.video_dim, cfg.audio_dim
        n_ca = 9 if cfg.cross_attention_adaln else 6
        self.norm_eps = cfg.norm_eps
        self.attn1 = Attention(v, None, cfg.video_heads, cfg.video_head_dim, cfg.norm_eps, cfg.gated_attention)
        self.attn2 = Attention(v, cfg.video_cross_dim, cfg.video_heads, cfg.video_head_dim, cfg.norm_eps,
                               cfg.gated_attention)
        self.ff = FeedForward(v, v, bias=cfg.ff_bias)
        self.scale_shift_table = torch.nn.Parameter(torch.empty(n_ca, v))
        self.audio_attn1 = Attention(a, None, cfg.audio_heads, cfg.audio_head_dim, cfg.norm_eps, cfg.gated_attention)
        self.audio_attn2 = Attention(a, cfg.audio_cross_dim, cfg.audio_heads, cfg.audio_head_dim, cfg.norm_eps,
                                     cfg.gated_attention)
        self.audio_ff = FeedForward(a, a, bias=cfg.audio_ff_bias)
        self.audio_scale_shift_table = torch.nn.Parameter(torch.empty(n_ca, a))
        self.audio_to_video_attn = Attention(v, a, cfg.audio_heads, cfg.audio_head_dim, cfg.norm_eps,
                                             cfg.gated_attention)
        self.video_to_audio_attn = Attention(a, v, cfg.audio_heads, cfg.audio_head_dim, cfg.norm_eps,
                                             cfg.gated_attention)
        self.scale_shift_table_a2v_ca_audio = torch.nn.Parameter(torch.empty(5, a))
        self.scale_shift_table_a2v_ca_video = torch.nn.Parameter(torch.empty(5, v))
        if cfg.cross_attention_adaln:
            self.prompt_scale_shift_table = torch.nn.Parameter(torch.empty(2, v))
            self.audio_prompt_scale_shift_table = torch.nn.Parameter(torch.empty(2, a))

    def _self_and_text(self, x: torch.Tensor, args: TransformerArgs, attn1: Attention, attn2: Attention,
                       sst: torch.Tensor, prompt_sst: torch.Tensor | None, cross_adaln: bool):
        """Self-attention + text cross-attention of one stream (ltx_dit.py:259-282, 237-248).

        Returns (x_fma, out2, gate): the text cross-attention residual
        `x_fma + out2 * gate` is left to the caller, which adds it in the same
        pass as the next norm."""
        eps = self.norm_eps
        ts = (args.timesteps, args.timestep_index)
        if args.pending is not None:  # previous block's FFN residual + this block's first norm
            f, g = args.pending
            x, norm_x = ltxk.add_norm_modulate(x, f, gate=g, shift=_ada(sst, 0, ts), scale=_ada(sst, 1, ts), eps=eps)
        else:
            norm_x = ltxk.norm_modulate(x, shift=_ada(sst, 0, ts), scale=_ada(sst, 1, ts), eps=eps)
        out = attn1(norm_x, pe=args.pe, mask=args.self_attention_mask,
                    perturbation_mask=args.self_attn_perturbation_mask, all_perturbed=args.self_attn_all_perturbed)
        if cross_adaln:
            x_fma, q_in = ltxk.add_norm_modulate(x, out, gate=_ada(sst, 2, ts), shift=_ada(sst, 6, ts),
                                                 scale=_ada(sst, 7, ts), eps=eps)
            enc = args.block_context
            if enc is None:
                kv_shift = _ada(prompt_sst, 0, args.prompt_timestep)
                kv_scale = _ada(prompt_sst, 1, args.prompt_timestep)
                enc = ltxk.modulate(_bf16(args.context), shift=kv_shift, scale=kv_scale)
            out2 = attn2(q_in, context=enc, mask=args.context_mask)
            return x_fma, out2, _ada(sst, 8, ts)
        x_fma, x_normed = ltxk.add_norm_modulate(x, out, gate=_ada(sst, 2, ts), eps=eps)
        return x_fma, attn2(x_normed, context=args.context, mask=args.context_mask), None

    @staticmethod
    def _settle(x: torch.Tensor, args: TransformerArgs) -> torch.Tensor:
        """x with a pending residual added (for a stream that does not run this block)."""
        if args is None or args.pending is None:
            return x
        return _apply_pending(x, args.pending)

    def forward(self, video: TransformerArgs | None, audio: TransformerArgs | None,
                defer_ffn_residual: bool = False, join: bool = True, fork: bool = True):
        """One AV block (ltx_dit.py:250-317).  With defer_ffn_residual the FFN
        residual is returned in `pending` instead of being added to x.

        When both streams run, the audio work runs on a side HIP stream.  The
        caller's stream waits for it once per block (for the A2V keys and
        values); the side stream waits at the block start (fork=True) and for
        the V2A keys and values.  With join=False the audio results are left on
        the side stream and the caller joins before reading them; with
        fork=False the side stream does not wait for the caller's stream at the
        block start, which is right when the previous block ran on the same two
        streams and the caller enqueued nothing since that the audio work reads
        (LTXModel.forward forks before its first block and joins after its
        last).  A cross-stream event record or wait costs the stream that makes
        it ~10 us on this part, so each block makes as few as possible."""
        vx = video.x if video is not None else None
        ax = audio.x if audio is not None else None
        run_vx = video is not None and video.enabled and vx.numel() > 0
        run_ax = audio is not None and audio.enabled and ax.numel() > 0
        main = torch.cuda.current_stream(vx.device if vx is not None else ax.device)
        if OVERLAP_AUDIO and run_vx and run_ax:
            return self._forward_two_streams(video, audio, main, _side_stream(main.device), defer_ffn_residual, join,
                                             fork)
        return self._forward_one_stream(video, audio, defer_ffn_residual)

    def _text_settle(self, x, text, table, ss, first, second):
        """Text cross-attention residual + norm/modulate with rows `first` [and
        `second`] of an AV table (the A2V/V2A inputs of ltx_dit.py:287-305)."""
        out2, g = text
        mods = {}
        if first is not None:
            mods.update(shift=_ada(table, first + 1, ss), scale=_ada(table, first, ss))
        if second is not None:
            key = ("shift2", "scale2") if first is not None else ("shift", "scale")
            mods.update({key[0]: _ada(table, second + 1, ss), key[1]: _ada(table, second, ss)})
        if not mods:
            return (ltxk.gated_residual(x, out2, gate=g, out=x),)
        return ltxk.add_norm_modulate(x, out2, gate=g, eps=self.norm_eps, x_out=x, **mods)

    def _forward_two_streams(self, video, audio, main, side, defer_ffn_residual, join, fork):
        cfg_ca = self.scale_shift_table.shape[0] == 9
        vx, ax = video.x, audio.x
        ev = _events(vx.device)
        if fork:
            ev["fork"].record(main)
            ev["fork"].wait(side)
        with torch.cuda.stream(side):
            ax, *atext = self._self_and_text(ax, audio, self.audio_attn1, self.audio_attn2,
                                             self.audio_scale_shift_table,
                                             getattr(self, "audio_prompt_scale_shift_table", None), cfg_ca)
        vx, *vtext = self._self_and_text(vx, video, self.attn1, self.attn2, self.scale_shift_table,
                                         getattr(self, "prompt_scale_shift_table", None), cfg_ca)

        # A2V / V2A (ltx_dit.py:284-307) read both streams after their text
        # cross-attention residual, which is added in the same pass as the two
        # AV modulations of the row.  Table rows: 0/1 = A2V (scale, shift),
        # 2/3 = V2A (scale, shift), 4 = gate.
        do_a2v = vx.numel() > 0 and ax.numel() > 0 and not video.cross_attn_skip_all
        do_v2a = vx.numel() > 0 and ax.numel() > 0 and not audio.cross_attn_skip_all
        tv, ta = self.scale_shift_table_a2v_ca_video, self.scale_shift_table_a2v_ca_audio
        vss = (video.cross_scale_shift_timestep, video.timestep_index)
        ass = (audio.cross_scale_shift_timestep, audio.timestep_index)
        A, V = self.audio_to_video_attn, self.video_to_audio_attn
        first, second = (0 if do_a2v else None), (2 if do_v2a else None)
        res = self._text_settle(vx, vtext, tv, vss, first, second)
        vx, a2v_v, v2a_v = res[0], res[1] if do_a2v else None, res[-1] if do_v2a else None
        # video-side projections of both attentions; A2V's queries and V2A's
        # keys share the video time-axis tables and rotate in one launch
        q_a2v = g_a2v = k_v2a = v_v2a = None
        if do_a2v:
            q_a2v = A.to_q(a2v_v)
            g_a2v = A.to_gate_logits(a2v_v).contiguous() if A.to_gate_logits is not None else None
        if do_v2a:
            k_v2a, v_v2a = V.to_k(v2a_v), V.to_v(v2a_v)
        _qk_pair(A, V, q_a2v, k_v2a, video.cross_pe)
        main_ready, side_ready = ev["main_ready"], ev["side_ready"]
        main_ready.record(main)

        pend_a = a_ffn = None
        k_a2v = v_a2v = None
        with torch.cuda.stream(side):
            res = self._text_settle(ax, atext, ta, ass, first, second)
            ax, a2v_a, v2a_a = res[0], res[1] if do_a2v else None, res[-1] if do_v2a else None
            q_v2a = g_v2a = None
            if do_a2v:
                k_a2v, v_a2v = A.to_k(a2v_a), A.to_v(a2v_a)
            if do_v2a:
                q_v2a = V.to_q(v2a_a)
                g_v2a = V.to_gate_logits(v2a_a).contiguous() if V.to_gate_logits is not None else None
            _qk_pair(A, V, k_a2v, q_v2a, audio.cross_pe, k_first=True)
            side_ready.record(side)
            if do_v2a:
                main_ready.wait(side)
                _hand_over(side, k_v2a, v_v2a)
                out = V.attend(q_v2a, k_v2a, v_v2a, g_v2a)
                pend_a = (out, _ada(ta, 4, audio.cross_gate_timestep, 0), _mask_arg(audio.cross_attn_perturbation_mask))
            ax, a_ffn = self._ffn(ax, pend_a, self.audio_scale_shift_table, (audio.timesteps, audio.timestep_index),
                                  self.audio_ff, defer_ffn_residual)
        pend_v = None
        if do_a2v:
            side_ready.wait(main)
            _hand_over(main, k_a2v, v_a2v)
            out = A.attend(q_a2v, k_a2v, v_a2v, g_a2v)
            pend_v = (out, _ada(tv, 4, video.cross_gate_timestep, 0), _mask_arg(video.cross_attn_perturbation_mask))
        vx, v_ffn = self._ffn(vx, pend_v, self.scale_shift_table, (video.timesteps, video.timestep_index), self.ff,
                              defer_ffn_residual)
        if join:  # audio results are ready for the caller's stream
            ev["join"].record(side)
            ev["join"].wait(main)
            _hand_over(main, ax, *(a_ffn[0:1] if a_ffn is not None else ()))
        return replace(video, x=vx, pending=v_ffn), replace(audio, x=ax, pending=a_ffn)

    def _forward_one_stream(self, video, audio, defer_ffn_residual):
        cfg_ca = self.scale_shift_table.shape[0] == 9
        eps = self.norm_eps
        vx = video.x if video is not None else None
        ax = audio.x if audio is not None else None
        run_vx = video is not None and video.enabled and vx.numel() > 0
        run_ax = audio is not None and audio.enabled and ax.numel() > 0
        run_a2v = run_vx and ax.numel() > 0
        run_v2a = run_ax and vx.numel() > 0
        if not run_vx:
            vx = self._settle(vx, video)
        if not run_ax:
            ax = self._settle(ax, audio)
        vtext = atext = None
        if run_vx:
            vx, *vtext = self._self_and_text(vx, video, self.attn1, self.attn2, self.scale_shift_table,
                                             getattr(self, "prompt_scale_shift_table", None), cfg_ca)
        if run_ax:
            ax, *atext = self._self_and_text(ax, audio, self.audio_attn1, self.audio_attn2,
                                             self.audio_scale_shift_table,
                                             getattr(self, "audio_prompt_scale_shift_table", None), cfg_ca)
        do_a2v = run_a2v and not video.cross_attn_skip_all
        do_v2a = run_v2a and not audio.cross_attn_skip_all
        tv = self.scale_shift_table_a2v_ca_video
        ta = self.scale_shift_table_a2v_ca_audio
        vss = (video.cross_scale_shift_timestep, video.timestep_index) if video is not None else None
        ass = (audio.cross_scale_shift_timestep, audio.timestep_index) if audio is not None else None
        a2v_v = v2a_v = a2v_a = v2a_a = None
        if run_vx:
            res = self._text_settle(vx, vtext, tv, vss, 0 if do_a2v else None, 2 if do_v2a else None)
            vx = res[0]
            a2v_v = res[1] if do_a2v else None
            v2a_v = res[-1] if do_v2a else None
        elif do_v2a:
            v2a_v = ltxk.norm_modulate(vx, shift=_ada(tv, 3, vss), scale=_ada(tv, 2, vss), eps=eps)
        if run_ax:
            res = self._text_settle(ax, atext, ta, ass, 0 if do_a2v else None, 2 if do_v2a else None)
            ax = res[0]
            a2v_a = res[1] if do_a2v else None
            v2a_a = res[-1] if do_v2a else None
        elif do_a2v:
            a2v_a = ltxk.norm_modulate(ax, shift=_ada(ta, 1, ass), scale=_ada(ta, 0, ass), eps=eps)

        pend_v = pend_a = None
        if do_a2v:
            out = self.audio_to_video_attn(a2v_v, context=a2v_a, pe=video.cross_pe, k_pe=audio.cross_pe)
            pend_v = (out, _ada(tv, 4, video.cross_gate_timestep, 0), _mask_arg(video.cross_attn_perturbation_mask))
        if do_v2a:
            out = self.video_to_audio_attn(v2a_a, context=v2a_v, pe=audio.cross_pe, k_pe=video.cross_pe)
            pend_a = (out, _ada(ta, 4, audio.cross_gate_timestep, 0), _mask_arg(audio.cross_attn_perturbation_mask))

        v_ffn = a_ffn = None
        if run_vx:
            vx, v_ffn = self._ffn(vx, pend_v, self.scale_shift_table, (video.timesteps, video.timestep_index),
                                  self.ff, defer_ffn_residual)
        elif pend_v is not None:
            vx = _apply_pending(vx, pend_v)
        if run_ax:
            ax, a_ffn = self._ffn(ax, pend_a, self.audio_scale_shift_table, (audio.timesteps, audio.timestep_index),
                                  self.audio_ff, defer_ffn_residual)
        elif pend_a is not None:
            ax = _apply_pending(ax, pend_a)
        return (replace(video, x=vx, pending=v_ffn) if video is not None else None,
                replace(audio, x=ax, pending=a_ffn) if audio is not None else None)

    def _ffn(self, x, pending, sst, ts, ff: FeedForward, defer: bool):
        """[pending A2V/V2A residual +] norm + modulate -> FFN -> gated residual (ltx_dit.py:309-314).

        Returns (x, None), or (x without the FFN residual, (ffn_out, gate)) when deferring."""
        eps = self.norm_eps
        shift, scale, gate = _ada(sst, 3, ts), _ada(sst, 4, ts), _ada(sst, 5, ts)
        if pending is not None:
            out, cgate, mask = pending
            x, h = ltxk.add_norm_modulate(x, out, gate=cgate, mask=mask, shift=shift, scale=scale, eps=eps)
        else:
            h = ltxk.norm_modulate(x, shift=shift, scale=scale, eps=eps)
        f = ff(h)
        if defer:
            return x, (f, gate)
        return ltxk.gated_residual(x, f, gate=gate), None


# ---------------------------------------------------------------------------
# Model
# ---------------------------------------------------------------------------


class LTXModel(torch.nn.Module):
    def __init__(self, cfg: DiTConfig):
        super().__init__()
        self.cfg = cfg
        v, a = cfg.video_dim, cfg.audio_dim
        n_adaln = 9 if cfg.cross_attention_adaln else 6
        self.patchify_proj = torch.nn.Linear(cfg.video_in, v, bias=True)
        self.keyframes_abs_pos_embedding = torch.nn.Parameter(torch.zeros(1, v)) if cfg.use_keyframes else None
        self.adaln_single = AdaLayerNormSingle(v, n_adaln)
        self.prompt_adaln_single = AdaLayerNormSingle(v, 2) if cfg.cross_attention_adaln else None
        self.scale_shift_table = torch.nn.Parameter(torch.empty(2, v))
        self.norm_out = torch.nn.LayerNorm(v, elementwise_affine=False, eps=cfg.norm_eps)
        self.proj_out = torch.nn.Linear(v, cfg.video_out)
        self.audio_patchify_proj = torch.nn.Linear(cfg.audio_in, a, bias=True)
        self.audio_adaln_single = AdaLayerNormSingle(a, n_adaln)
        self.audio_prompt_adaln_single = AdaLayerNormSingle(a, 2) if cfg.cross_attention_adaln else None
        self.audio_scale_shift_table = torch.nn.Parameter(torch.empty(2, a))
        self.audio_norm_out = torch.nn.LayerNorm(a, elementwise_affine=False, eps=cfg.norm_eps)
        self.audio_proj_out = torch.nn.Linear(a, cfg.audio_out)
        self.av_ca_video_scale_shift_adaln_single = AdaLayerNormSingle(v, 4)
        self.av_ca_audio_scale_shift_adaln_single = AdaLayerNormSingle(a, 4)
        self.av_ca_a2v_gate_adaln_single = AdaLayerNormSingle(v, 1)
        self.av_ca_v2a_gate_adaln_single = AdaLayerNormSingle(a, 1)
        self.blocks = torch.nn.ModuleList([Block(cfg) for _ in range(cfg.num_layers)])
        self.video_pre = ArgsPreprocessor(self, "video")
        self.audio_pre = ArgsPreprocessor(self, "audio")

    def forward(self, video: Modality | None, audio: Modality | None, perturbations) -> tuple:
        """perturbations: the (4, blocks, B) keep-mask tensor, None (every
        attention runs), or a PerturbationTable holding the mask with its host
        copy (what a denoising loop passes: the copy is made once per loop)."""
        va = self.video_pre.prepare(video, audio) if video is not None else None
        aa = self.audio_pre.prepare(audio, video) if audio is not None else None
        # One host copy of the keep-mask table per forward replaces the
        # reference's three device syncs per stream and block.
        perturbations, host = self._host_perturbations(perturbations)
        # The context, the blocks' prompt tables and the prompt timestep are the
        # same for every block of the step: their text-context modulations
        # (ltx_dit.py:240-246, once per block there) are made in one launch.
        v_ctx = self._block_contexts(va, "prompt_scale_shift_table")
        a_ctx = self._block_contexts(aa, "audio_prompt_scale_shift_table")
        for idx, block in enumerate(self.blocks):
            if va is not None:
                va = apply_block_perturbations(va, perturbations, idx, 0, 2, host)
                if v_ctx is not None:
                    va = replace(va, block_context=v_ctx[idx])
            if aa is not None:
                aa = apply_block_perturbations(aa, perturbations, idx, 1, 3, host)
                if a_ctx is not None:
                    aa = replace(aa, block_context=a_ctx[idx])
            # the audio side stream forks from this stream before the first
            # block and is joined once, after the last (every block runs the
            # same streams: which ones run is fixed by the modalities)
            va, aa = block(va, aa, defer_ffn_residual=True, join=idx == len(self.blocks) - 1, fork=idx == 0)
        if va is not None:
            va = replace(va, x=Block._settle(va.x, va), pending=None)
        if aa is not None:
            aa = replace(aa, x=Block._settle(aa.x, aa), pending=None)
        vx = self._output(self.scale_shift_table, self.norm_out, self.proj_out, va) if va is not None else None
        ax = self._output(self.audio_scale_shift_table, self.audio_norm_out, self.audio_proj_out, aa) \
            if aa is not None else None
        return vx, ax

    # Above this size LTXModel.forward does not hold every block's modulated
    # context at once; each block modulates its own (ltx_dit.py:240-246).
    BLOCK_CONTEXTS_MAX_BYTES = 8 << 30

    def _block_contexts(self, args: TransformerArgs | None, table: str) -> torch.Tensor | None:
        """Every block's modulated text context, (blocks, B, S, D), or None when
        the blocks have no cross-attention AdaLN or the result would exceed
        BLOCK_CONTEXTS_MAX_BYTES.  The blocks' prompt tables are stacked afresh
        on every forward (one launch), so an update of a table between forwards
        is always seen."""
        if args is None or not self.blocks or not hasattr(self.blocks[0], table) or \
                self.blocks[0].scale_shift_table.shape[0] != 9:
            return None
        if len(self.blocks) * args.context.numel() * 2 > self.BLOCK_CONTEXTS_MAX_BYTES:
            return None
        with torch.no_grad():
            stacked = torch.stack([getattr(b, table).detach() for b in self.blocks]).to(torch.bfloat16).contiguous()
        pt = args.prompt_timestep
        return ltxk.modulate_layers(_bf16(args.context), ltxk.AdaRef(stacked, 0, pt), ltxk.AdaRef(stacked, 1, pt),
                                    len(self.blocks))

    @staticmethod
    def _host_perturbations(pcfg) -> tuple:
        """(keep-mask tensor, its CPU copy): the copy a PerturbationTable holds,
        or one made now."""
        if pcfg is None:
            return None, None
        if isinstance(pcfg, PerturbationTable):
            return pcfg.mask, pcfg.host
        return pcfg, pcfg.detach().to("cpu", torch.float32)

    @staticmethod
    def _output(sst, norm_out, proj_out, args) -> torch.Tensor:
        """LayerNorm(no affine) + (shift, scale) = sst + embedded_timestep, fused; then proj_out (ltx_dit.py:371-378)."""
        emb = (args.embedded_timestep, args.timestep_index)
        x = ltxk.norm_modulate(args.x, shift=_ada(sst, 0, emb, 0), scale=_ada(sst, 1, emb, 0),
                               eps=norm_out.eps, layer=True)
        return proj_out(x)


def apply_block_perturbations(args: TransformerArgs, pcfg, block_idx: int, self_type: int, cross_type: int,
                              host_pcfg: torch.Tensor | None = None):
    """Attach this block's keep-masks (reference ltx_dit.py:381-394).

    pcfg None means every attention runs (no masks).  The all/any flags are
    read from `host_pcfg` (a CPU copy of pcfg) when given, so the loop over
    blocks never waits on the device.
    """
    if pcfg is None:
        return args
    src = host_pcfg if host_pcfg is not None else pcfg
    self_zero = src[self_type, block_idx] == 0
    all_self = bool(self_zero.all())
    any_self = bool(self_zero.any())
    all_cross = bool((src[cross_type, block_idx] == 0).all())
    return replace(
        args,
        self_attn_perturbation_mask=pcfg[self_type, block_idx].reshape(-1, 1, 1) if any_self and not all_self else None,
        self_attn_all_perturbed=all_self,
        cross_attn_perturbation_mask=None if all_cross else pcfg[cross_type, block_idx].reshape(-1, 1, 1),
        cross_attn_skip_all=all_cross,
    )


def build_perturbation_config(num_blocks: int, passes: list[str], v_stg_blocks: list[int], a_stg_blocks: list[int],
                              device: torch.device, dtype: torch.dtype) -> torch.Tensor:
    """(4, num_blocks, B) keep-mask: 0 skip-video-self, 1 skip-audio-self, 2 skip-A2V, 3 skip-V2A (ltx_dit.py:397-411)."""
    keep = torch.ones(4, num_blocks, len(passes), dtype=dtype)
    for i, name in enumerate(passes):
        if name == "ptb":
            for blk in v_stg_blocks:
                keep[0, blk, i] = 0
            for blk in a_stg_blocks:
                keep[1, blk, i] = 0
        elif name == "mod":
            keep[2, :, i] = 0
            keep[3, :, i] = 0
    return keep.to(device)


def load_transformer(path: str, cfg: DiTConfig) -> LTXModel:
    """Checkpoint load with the reference's key renames (ltx_dit.py:414-432)."""
    with torch.device("meta"):
        model = LTXModel(cfg)

    def rename(key: str) -> str | None:
        if not key.startswith("model.diffusion_model."):
            return None
        k = key.removeprefix("model.diffusion_model.").replace("transformer_blocks.", "blocks.")
        for old, new in (("to_out.0.", "to_out."), ("ff.net.0.proj.", "ff.proj_in."), ("ff.net.2.", "ff.proj_out.")):
            k = k.replace(old, new)
        return k

    sd = load_state_dict(path, rename=rename)
    res = model.load_state_dict(sd, strict=False, assign=True)
    missing = [k for k in res.missing_keys if k != "keyframes_abs_pos_embedding"]
    if missing:
        raise RuntimeError(f"transformer missing keys: {missing[:10]} ({len(missing)} total)")
    return model.to(DEVICE).eval()


# ---------------------------------------------------------------------------
# Latent state construction
# ---------------------------------------------------------------------------

SCALE_T, SCALE_H, SCALE_W = 8, 32, 32


def video_positions(batch: int, f: int, h: int, w: int, fps: float, device) -> torch.Tensor:
    """(B, 3, T, 2) pixel-space [start, end) bounds, time axis causal-shifted and divided by fps (ltx_dit.py:442-456)."""
    grid = torch.meshgrid(torch.arange(f, device=device), torch.arange(h, device=device),
                          torch.arange(w, device=device), indexing="ij")
    start = torch.stack(grid, dim=0).reshape(3, -1).float()
    bounds = torch.stack([start, start + 1], dim=-1)                              # (3, T, 2)
    bounds = bounds * torch.tensor([SCALE_T, SCALE_H, SCALE_W], device=device, dtype=torch.float32).view(3, 1, 1)
    bounds[0] = (bounds[0] + 1 - SCALE_T).clamp(min=0) / fps
    return bounds.unsqueeze(0).expand(batch, -1, -1, -1).contiguous()


def audio_positions(batch: int, frames: int, device) -> torch.Tensor:
    """(B, 1, T, 2) latent-frame bounds in seconds of the causal mel timing (ltx_dit.py:459-465)."""
    i = torch.arange(frames, dtype=torch.float32, device=device)
    start = (i * 4 + 1 - 4).clamp(min=0) * 160 / 16000
    end = ((i + 1) * 4 + 1 - 4).clamp(min=0) * 160 / 16000
    return torch.stack([start, end], dim=-1)[None, None].expand(batch, 1, -1, -1).contiguous()


def patchify_video(latent: torch.Tensor) -> torch.Tensor:
    return latent.permute(0, 2, 3, 4, 1).reshape(latent.shape[0], -1, latent.shape[1])


def unpatchify_video(tokens: torch.Tensor, f: int, h: int, w: int) -> torch.Tensor:
    b, _, c = tokens.shape
    return tokens.view(b, f, h, w, c).permute(0, 4, 1, 2, 3)


def patchify_audio(latent: torch.Tensor) -> torch.Tensor:
    return latent.permute(0, 2, 1, 3).reshape(latent.shape[0], latent.shape[2], -1)


def unpatchify_audio(tokens: torch.Tensor, channels: int, mel_bins: int) -> torch.Tensor:
    b, t, _ = tokens.shape
    return tokens.view(b, t, channels, mel_bins).permute(0, 2, 1, 3)


@dataclass
class LatentState:
    latent: torch.Tensor
    denoise_mask: torch.Tensor
    positions: torch.Tensor
    clean_latent: torch.Tensor
    keyframes_mask: torch.Tensor | None = None


def create_noised_states(batch: int, num_video_frames: int, height: int, width: int, fps: float, seed: int,
                         device: torch.device, dtype: torch.dtype,
                         generator: TorchRNG | None = None) -> tuple[LatentState, LatentState]:
    """Noised t2v states (reference ltx_dit.py:495-520): video noise then audio noise
    from one Philox generator seeded `seed` (ltxk_philox_normal).  Pass
    `generator` to draw with another device's thread policy (e.g.
    TorchRNG(seed, device, *torch_rng.ADA_RTX6000) for the reference's stream)."""
    gen = generator if generator is not None else TorchRNG(seed, device)
    f = (num_video_frames - 1) // SCALE_T + 1
    h, w = height // SCALE_H, width // SCALE_W
    v_tokens = f * h * w
    video_noise = gen.randn(batch, v_tokens, 128, dtype=dtype)
    keyframes_mask = torch.zeros(batch, v_tokens, 1, device=device, dtype=torch.float32)
    keyframes_mask[:, : h * w] = 1.0
    video_state = LatentState(
        latent=video_noise,
        denoise_mask=torch.ones(batch, v_tokens, 1, device=device, dtype=torch.float32),
        positions=video_positions(batch, f, h, w, fps, device),
        clean_latent=torch.zeros_like(video_noise),
        keyframes_mask=keyframes_mask,
    )
    audio_frames = round(num_video_frames / fps * 25.0)
    audio_noise = gen.randn(batch, audio_frames, 128, dtype=dtype)
    audio_state = LatentState(
        latent=audio_noise,
        denoise_mask=torch.ones(batch, audio_frames, 1, device=device, dtype=torch.float32),
        positions=audio_positions(batch, audio_frames, device),
        clean_latent=torch.zeros_like(audio_noise),
    )
    return video_state, audio_state


# ---------------------------------------------------------------------------
# Scheduler + guidance + sampling loop
# ---------------------------------------------------------------------------


def ltx2_scheduler_sigmas(steps: int, tokens: int = 4096, max_shift: float = 2.05, base_shift: float = 0.95,
                          terminal: float = 0.1) -> torch.Tensor:
    """Shifted, terminal-stretched flow-matching sigmas (reference ltx_dit.py:528-539)."""
    sigmas = torch.linspace(1.0, 0.0, steps + 1)
    slope = (max_shift - base_shift) / (4096 - 1024)
    e = math.exp(tokens * slope + (base_shift - slope * 1024))
    sigmas = torch.where(sigmas != 0, e / (e + (1 / sigmas - 1)), sigmas)
    nz = sigmas != 0
    one_minus = 1.0 - sigmas[nz]
    sigmas[nz] = 1.0 - one_minus / (one_minus[-1] / (1.0 - terminal))
    return sigmas.to(torch.float32)


@dataclass(frozen=True)
class GuiderParams:
    cfg_scale: float
    stg_scale: float
    rescale_scale: float
    modality_scale: float
    stg_blocks: tuple[int, ...]


def guide(cond, uncond, ptb, mod, p: GuiderParams) -> torch.Tensor:
    """CFG + STG + modality guidance with std rescale (reference ltx_dit.py:551-562) on ltxk_guide."""
    x0 = torch.cat([cond, uncond, ptb, mod]).contiguous()
    den, _, _ = ltxk.guide(None, x0, None, p.cfg_scale, p.stg_scale, p.modality_scale, p.rescale_scale)
    return den


PASSES = ("cond", "uncond", "ptb", "mod")


@dataclass(frozen=True)
class _StepInputs:
    """What the B=4 guidance call reuses unchanged from step to step: the
    stacked contexts, positions, masks and perturbation table, and the distinct
    levels of the denoise masks, with what the model derives from them: the
    RoPE tables, the perturbation table's host copy and the distinct timestep
    rows.  Built once per denoising run and handed to each step's forward
    (Modality.rope_tables / timestep_rows, PerturbationTable), so a step reads
    nothing back from the device."""

    v_ctx: torch.Tensor
    a_ctx: torch.Tensor
    v_pos: torch.Tensor
    a_pos: torch.Tensor
    v_mask: torch.Tensor
    a_mask: torch.Tensor
    v_keyframes: torch.Tensor | None
    v_rows: TimestepRows
    a_rows: TimestepRows
    v_rope: RopeTables
    a_rope: RopeTables
    perturbations: PerturbationTable


def _step_inputs(model: LTXModel, video_state: LatentState, audio_state: LatentState, contexts: dict,
                 v_params: GuiderParams, a_params: GuiderParams, cfg: DiTConfig) -> _StepInputs:
    n = len(PASSES)
    v_mask = video_state.denoise_mask.repeat(n, 1, 1)
    a_mask = audio_state.denoise_mask.repeat(n, 1, 1)
    kf = video_state.keyframes_mask.repeat(n, 1, 1) if video_state.keyframes_mask is not None else None
    v_pos = video_state.positions.repeat(n, 1, 1, 1)
    a_pos = audio_state.positions.repeat(n, 1, 1, 1)
    return _StepInputs(
        v_ctx=torch.cat([contexts["v_pos"], contexts["v_neg"], contexts["v_pos"], contexts["v_pos"]], dim=0),
        a_ctx=torch.cat([contexts["a_pos"], contexts["a_neg"], contexts["a_pos"], contexts["a_pos"]], dim=0),
        v_pos=v_pos, a_pos=a_pos, v_mask=v_mask, a_mask=a_mask, v_keyframes=kf,
        v_rows=timestep_rows(v_mask), a_rows=timestep_rows(a_mask),
        v_rope=model.video_pre.rope_tables(v_pos), a_rope=model.audio_pre.rope_tables(a_pos),
        perturbations=PerturbationTable.of(build_perturbation_config(
            cfg.num_layers, list(PASSES), list(v_params.stg_blocks), list(a_params.stg_blocks),
            video_state.latent.device, video_state.latent.dtype)),
    )


def _denoise(model: LTXModel, video_state: LatentState, audio_state: LatentState, contexts: dict,
             sigma: torch.Tensor, v_params: GuiderParams, a_params: GuiderParams, cfg: DiTConfig,
             step: tuple[float, float] | None, want_x0: bool, inputs: _StepInputs | None = None):
    """The B=4 guidance call (ltx_dit.py:565-599) with its tail (x0 of every
    pass, guide, and with `step` = (sigma, dt) the Euler update) on ltxk_guide:
    one pass over the latent-sized tensors per modality."""
    n = len(PASSES)
    c = inputs if inputs is not None else _step_inputs(model, video_state, audio_state, contexts, v_params,
                                                       a_params, cfg)
    sigma_b = sigma.expand(n)
    # timesteps = denoise_mask * sigma per token (ltx_dit.py:578,584); the
    # distinct levels times sigma are the same fp32 products
    video = Modality(latent=video_state.latent.repeat(n, 1, 1), sigma=sigma_b,
                     timesteps=c.v_mask * sigma_b.view(n, 1, 1), positions=c.v_pos, context=c.v_ctx,
                     keyframes_mask=c.v_keyframes, timestep_rows=c.v_rows.scaled(sigma), rope_tables=c.v_rope)
    audio = Modality(latent=audio_state.latent.repeat(n, 1, 1), sigma=sigma_b,
                     timesteps=c.a_mask * sigma_b.view(n, 1, 1), positions=c.a_pos, context=c.a_ctx,
                     timestep_rows=c.a_rows.scaled(sigma), rope_tables=c.a_rope)
    vx, ax = model(video, audio, c.perturbations)
    kw = {} if step is None else {"sigma": step[0], "dt": step[1]}
    out = []
    for state, vel, mod, p in ((video_state, vx, video, v_params), (audio_state, ax, audio, a_params)):
        out.append(ltxk.guide(state.latent.contiguous(), vel.contiguous(), mod.timesteps.float().contiguous(),
                              p.cfg_scale, p.stg_scale, p.modality_scale, p.rescale_scale, want_x0=want_x0, **kw))
    (dv, nv, x0_v), (da, na, x0_a) = out
    r = dict(zip(PASSES, zip(x0_v.chunk(n), x0_a.chunk(n), strict=True), strict=True)) if want_x0 else None
    return dv, da, r, nv, na


def guided_denoise_step(model: LTXModel, video_state: LatentState, audio_state: LatentState, contexts: dict,
                        sigma: torch.Tensor, step_idx: int, v_params: GuiderParams, a_params: GuiderParams,
                        cfg: DiTConfig) -> tuple:
    """One B=4 transformer call (cond | uncond | ptb | mod) -> guided x0 per modality (ltx_dit.py:565-599)."""
    dv, da, r, _, _ = _denoise(model, video_state, audio_state, contexts, sigma, v_params, a_params, cfg, None, True)
    return dv, da, r


def euler_step(sample: torch.Tensor, denoised: torch.Tensor, sigmas: torch.Tensor, idx: int) -> torch.Tensor:
    """vel = ((x - x0)/sigma).to(dtype); x' = (x + vel*dt).to(dtype) on ltxk_euler_step (ltx_dit.py:602-606)."""
    sigma, dt = _step_scalars(sigmas, idx)
    return ltxk.euler_step(sample.contiguous(), denoised.contiguous(), sigma, dt)


def _step_scalars(sigmas: torch.Tensor, idx: int) -> tuple[float, float]:
    """sigma and dt as the reference's fp32 values (ltx_dit.py:603-604)."""
    return float(sigmas[idx].float()), float((sigmas[idx + 1] - sigmas[idx]).float())


@torch.inference_mode()
def run_dit(model: LTXModel, cfg: DiTConfig, contexts: dict, video_state: LatentState, audio_state: LatentState,
            sigmas: torch.Tensor, v_params: GuiderParams, a_params: GuiderParams,
            on_step=None) -> tuple[torch.Tensor, torch.Tensor]:
    """Denoising loop (reference ltx_dit.py:609-621)."""
    host_sigmas = sigmas.detach().float().cpu()  # one read for every step's sigma and dt
    # contexts, positions, masks and the perturbation table are the same every
    # step: built (and their host-side analyses cached) once
    inputs = _step_inputs(model, video_state, audio_state, contexts, v_params, a_params, cfg)
    for idx in range(len(sigmas) - 1):
        t0 = time.perf_counter()
        # guidance and the Euler update in one ltxk_guide pass per modality;
        # the per-pass x0 only when a callback will look at them
        dv, da, passes, nv, na = _denoise(model, video_state, audio_state, contexts, sigmas[idx], v_params,
                                          a_params, cfg, _step_scalars(host_sigmas, idx), on_step is not None,
                                          inputs)
        video_state = replace(video_state, latent=nv)
        audio_state = replace(audio_state, latent=na)
        if on_step:
            on_step(idx, time.perf_counter() - t0, dv, da, passes, video_state, audio_state)
    return video_state.latent, audio_state.latent
