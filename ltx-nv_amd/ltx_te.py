"""Text-encoder connector path of LTX-2.5 with the reference's module API
(standalone/ltx_te.py:159-310): the multi-layer feature extractor, the 1D
connector transformers and their weight loading.

Kept as in the reference (names, signatures, shapes): FeatureExtractorV2,
ConnectorBlock, Embeddings1DConnector, EmbeddingsProcessor,
build_embeddings_processor.  The Gemma language model, the tokenizer and the
prompt-encoding driver that feed it (ltx_te.py:37-146, 313-) are not part of
this module; it takes the language model's hidden states as input.

Memory-bound work runs on ltxk kernels: the feature extractor's per-layer RMS
norm + layer interleave + token mask + projection scales is one
ltxk_feature_norm pass; in the connector blocks every residual add is fused
with the RMSNorm that follows it (the FFN residual with the next block's first
norm, the last one with the output norm), q/k norm + RoPE, the attention head
gate and GELU are the DiT's kernels.  Linear layers and attention are
PyTorch-ROCm.
"""

from __future__ import annotations

import math

import torch

import ltxk
from common import DEVICE, load_state_dict, read_metadata
from ltx_nn import Attention, FeedForward, precompute_freqs_cis


class FeatureExtractorV2(torch.nn.Module):
    """Per-token RMS over the hidden dim of every language-model layer, the
    layers interleaved into one (B, T, D*L) feature, masked, then two
    projections (ltx_te.py:159-184)."""

    def __init__(self, gemma_hidden: int, num_layers: int, video_dim: int, audio_dim: int):
        super().__init__()
        flat = gemma_hidden * (num_layers + 1)
        self.video_aggregate_embed = torch.nn.Linear(flat, video_dim, bias=True)
        self.audio_aggregate_embed = torch.nn.Linear(flat, audio_dim, bias=True)
        self.embedding_dim = gemma_hidden

    def forward(self, hidden_states: tuple[torch.Tensor, ...], attention_mask: torch.Tensor):
        vd = self.video_aggregate_embed.out_features
        ad = self.audio_aggregate_embed.out_features
        layers = [h.contiguous() for h in hidden_states]
        v_in, a_in = ltxk.feature_norm(layers, attention_mask, math.sqrt(vd / self.embedding_dim),
                                       math.sqrt(ad / self.embedding_dim), eps=1e-6)
        return self.video_aggregate_embed(v_in), self.audio_aggregate_embed(a_in)


class ConnectorBlock(torch.nn.Module):
    """x += attn1(rms(x)); x += ff(rms(x)) (ltx_te.py:187-196)."""

    def __init__(self, dim: int, heads: int, dim_head: int, gated: bool, ff_bias: bool, norm_eps: float = 1e-6):
        super().__init__()
        self.attn1 = Attention(dim, None, heads, dim_head, norm_eps, apply_gated_attention=gated)
        self.ff = FeedForward(dim, dim, bias=ff_bias)

    def forward(self, x, additive_mask=None, pe=None):
        x, _ = self._run(x, None, additive_mask, pe)
        return x

    def _run(self, x: torch.Tensor, pending: torch.Tensor | None, additive_mask, pe, defer: bool = False):
        """One block on x (+ a residual branch `pending` not yet added).  The
        residual adds are fused with the norms after them; with `defer` the FF
        branch is returned unadded, for the next norm to take in."""
        x = x.contiguous()
        if pending is None:
            y = ltxk.rms_norm(x, None, 1e-6)
        else:
            x, y = ltxk.add_norm_modulate(x, pending, eps=1e-6)
        a = self.attn1(y, mask=additive_mask, pe=pe)
        x, y = ltxk.add_norm_modulate(x, a.contiguous(), eps=1e-6)
        f = self.ff(y).contiguous()
        if defer:
            return x, f
        return ltxk.gated_residual(x, f), None


class Embeddings1DConnector(torch.nn.Module):
    """Bidirectional 1D transformer with learnable registers (ltx_te.py:199-233)."""

    def __init__(self, heads: int, dim_head: int, num_layers: int, max_pos: list[int],
                 registers: int, gated: bool, ff_bias: bool):
        super().__init__()
        self.inner_dim = heads * dim_head
        self.positional_max_pos = list(max_pos)
        self.blocks = torch.nn.ModuleList(
            [ConnectorBlock(self.inner_dim, heads, dim_head, gated, ff_bias) for _ in range(num_layers)]
        )
        self.num_registers = registers
        if registers:
            self.learnable_registers = torch.nn.Parameter(torch.empty(registers, self.inner_dim))

    def _with_registers(self, x: torch.Tensor, open_tokens: torch.Tensor) -> torch.Tensor:
        """Every token the mask closes takes register (its position mod R); the
        open tokens keep their features (ltx_te.py:216-221).  The sequence must
        hold a whole number of register sets."""
        s = x.shape[1]
        if s % self.num_registers:
            raise ValueError(f"sequence of {s} tokens is not a multiple of {self.num_registers} registers")
        slot = torch.arange(s, device=x.device) % self.num_registers
        regs = self.learnable_registers.to(x.dtype)[slot]                       # (S, D)
        return torch.where(open_tokens.unsqueeze(-1), x, regs.unsqueeze(0))

    def _rope(self, batch: int, s: int, device, dtype) -> ltxk.CompactRope:
        """Rotation tables of the 1D positions 0..S-1 (ltx_te.py:222-226): the
        position of token t is t in every batch item, so the tables are one row
        per position, shared by the batch, in ltxk's compact form."""
        heads = self.blocks[0].attn1.heads if len(self.blocks) else 1
        grid = torch.arange(s, dtype=torch.float32, device=device).view(1, 1, s)
        cos, sin = precompute_freqs_cis(grid, dim=self.inner_dim, out_dtype=dtype, theta=10000.0,
                                        max_pos=list(self.positional_max_pos), use_middle_indices_grid=False,
                                        num_attention_heads=heads, double_precision=True)
        half = self.inner_dim // 2
        rows = [t.transpose(1, 2).reshape(s, half).contiguous() for t in (cos, sin)]
        index = torch.arange(s, dtype=torch.int32, device=device).view(1, s, 1).expand(batch, s, 1).contiguous()
        return ltxk.CompactRope(rows[0], rows[1], index, (batch, heads, s, half // heads), checked=True)

    def forward(self, hidden_states: torch.Tensor, additive_mask: torch.Tensor):
        b, s, _ = hidden_states.shape
        if self.num_registers:
            # every token is open once the registers fill the closed ones
            hidden_states = self._with_registers(hidden_states, additive_mask[:, 0, 0, :] >= 0)
            additive_mask = torch.zeros_like(additive_mask)
        pe = self._rope(b, s, hidden_states.device, hidden_states.dtype)
        x, pending = hidden_states.contiguous(), None
        for block in self.blocks:
            x, pending = block._run(x, pending, additive_mask, pe, defer=True)
        if pending is None:
            return ltxk.rms_norm(x, None, 1e-6), additive_mask
        _, out = ltxk.add_norm_modulate(x, pending, eps=1e-6)  # last residual + the output norm
        return out, additive_mask


def kept_first(keep: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Destination of each token when the kept tokens (keep (B, S) bool) move in
    front of the others, each group in its own order: a kept token goes to the
    count of kept tokens before it, any other to the batch item's kept count
    plus the count of other tokens before it.  Returns (dest (B, S) int64,
    kept count (B, 1))."""
    n_kept = keep.sum(dim=1, keepdim=True)
    kept_before = torch.cumsum(keep, dim=1) - 1
    other_before = torch.cumsum(~keep, dim=1) - 1
    return torch.where(keep, kept_before, n_kept + other_before), n_kept


class EmbeddingsProcessor(torch.nn.Module):
    """Feature extractor + video/audio connectors (ltx_te.py:236-263)."""

    def __init__(self, feature_extractor: FeatureExtractorV2, video_connector: Embeddings1DConnector,
                 audio_connector: Embeddings1DConnector):
        super().__init__()
        self.feature_extractor = feature_extractor
        self.video_connector = video_connector
        self.audio_connector = audio_connector

    def process_hidden_states(self, hidden_states, attention_mask):
        """Features of the prompt's tokens, the tokens the attention mask keeps
        moved in front of the padded ones (each group in its own order), then
        the two connectors over them with the moved mask (ltx_te.py:244-262).

        Returns (video encoding, audio encoding, video token mask).  The
        reference's mask test `(connector mask < 1e-6)` holds for both values
        its additive masks take (0 and -max), so the video mask is all ones and
        the video encoding is returned as the connector made it."""
        video_feats, audio_feats = self.feature_extractor(hidden_states, attention_mask)
        keep = attention_mask.reshape(attention_mask.shape[0], -1).to(torch.int64) >= 1   # (B, S)
        b, s = keep.shape
        dest, n_kept = kept_first(keep)

        def moved(f: torch.Tensor) -> torch.Tensor:
            return torch.empty_like(f).scatter_(1, dest.unsqueeze(-1).expand_as(f), f)

        dtype = video_feats.dtype
        closed = torch.arange(s, device=keep.device).unsqueeze(0) >= n_kept      # (B, S) after the move
        moved_mask = torch.zeros(b, 1, 1, s, dtype=dtype, device=keep.device).masked_fill_(
            closed.view(b, 1, 1, s), -torch.finfo(dtype).max)
        video_enc, _ = self.video_connector(moved(video_feats), moved_mask)
        audio_enc, _ = self.audio_connector(moved(audio_feats), moved_mask)
        return video_enc, audio_enc, torch.ones(b, s, dtype=torch.int64, device=keep.device)


# ---------------------------------------------------------------------------
# Assembly + weight loading
# ---------------------------------------------------------------------------

# Checkpoint module names -> this module tree's (the same renames as
# ltx_dit.load_transformer: the Sequential wrappers of the checkpoint's
# to_out and ff have no counterpart here).
_LEAF_RENAMES = (("transformer_1d_blocks", "blocks"), ("to_out.0.", "to_out."), ("ff.net.0.proj.", "ff.proj_in."),
                 ("ff.net.2.", "ff.proj_out."))
_CONNECTOR_PREFIX = "model.diffusion_model."


def _connector_key(key: str) -> str | None:
    """A DiT checkpoint key of the video or audio embeddings connector ->
    its EmbeddingsProcessor key; anything else -> None (ltx_te.py:294-310)."""
    if not key.startswith(_CONNECTOR_PREFIX) or "_embeddings_connector." not in key:
        return None
    owner, leaf = key.split("_embeddings_connector.", 1)
    for old, new in _LEAF_RENAMES:
        leaf = leaf.replace(old, new)
    return ("video_connector." if owner.endswith("video") else "audio_connector.") + leaf


def _feature_key(key: str) -> str | None:
    """A text-encoder checkpoint key of the feature projections -> its key."""
    head = "text_embedding_projection."
    return "feature_extractor." + key[len(head):] if key.startswith(head) else None


def _connector_kwargs(tr: dict, audio: bool) -> dict:
    """Embeddings1DConnector arguments from the DiT's config metadata: the
    audio connector's shape keys carry an `audio_` prefix and fall back to the
    shared ones; registers, positions, gating and bias are shared (defaults:
    32 heads x 128, 8 layers, 128 registers, positions up to 4096)."""
    def shape(key: str, default: int) -> int:
        shared = tr.get("connector_" + key, default)
        return tr.get("audio_connector_" + key, shared) if audio else shared

    return dict(heads=shape("num_attention_heads", 32), dim_head=shape("attention_head_dim", 128),
                num_layers=shape("num_layers", 8),
                max_pos=tr.get("connector_positional_embedding_max_pos", [4096]),
                registers=tr.get("connector_num_learnable_registers", 128),
                gated=tr.get("connector_apply_gated_attention", False), ff_bias=tr.get("connector_ff_bias", True))


def build_embeddings_processor(te_path: str, transformer_path: str) -> EmbeddingsProcessor:
    """The connector path with its weights: the feature projections from the
    text-encoder checkpoint, both connectors from the DiT checkpoint
    (ltx_te.py:270-301)."""
    gemma = read_metadata(te_path)["gemma_config"]
    text = gemma.get("text_config", gemma)
    tr = read_metadata(transformer_path)["config"]["transformer"]
    with torch.device("meta"):
        proc = EmbeddingsProcessor(
            FeatureExtractorV2(text["hidden_size"], text["num_hidden_layers"],
                               tr["num_attention_heads"] * tr["attention_head_dim"],
                               tr["audio_num_attention_heads"] * tr["audio_attention_head_dim"]),
            Embeddings1DConnector(**_connector_kwargs(tr, audio=False)),
            Embeddings1DConnector(**_connector_kwargs(tr, audio=True)))
    weights = {**load_state_dict(te_path, rename=_feature_key), **load_state_dict(transformer_path,
                                                                                   rename=_connector_key)}
    proc.load_state_dict(weights, strict=False, assign=True)
    return proc.to(DEVICE).eval()
