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

    def forward(self, hidden_states: torch.Tensor, additive_mask: torch.Tensor):
        b, s, _ = hidden_states.shape
        if self.num_registers:
            # padded positions take the learnable registers (ltx_te.py:216-221)
            regs = self.learnable_registers.repeat(s // self.num_registers, 1).to(hidden_states.dtype)
            regs = regs.unsqueeze(0).expand(b, -1, -1)
            binary = (additive_mask[:, 0, 0, :] >= 0).to(hidden_states.dtype).unsqueeze(-1)
            hidden_states = binary * hidden_states + (1 - binary) * regs
            additive_mask = torch.zeros_like(additive_mask)
        grid = torch.arange(s, dtype=torch.float32, device=hidden_states.device)[None, None, :].expand(b, -1, -1)
        pe = precompute_freqs_cis(
            grid, dim=self.inner_dim, out_dtype=hidden_states.dtype, theta=10000.0,
            max_pos=list(self.positional_max_pos), use_middle_indices_grid=False,
            num_attention_heads=self.blocks[0].attn1.heads if len(self.blocks) else 1, double_precision=True,
        )
        x, pending = hidden_states.contiguous(), None
        for block in self.blocks:
            x, pending = block._run(x, pending, additive_mask, pe, defer=True)
        if pending is None:
            return ltxk.rms_norm(x, None, 1e-6), additive_mask
        _, out = ltxk.add_norm_modulate(x, pending, eps=1e-6)  # last residual + the output norm
        return out, additive_mask


class EmbeddingsProcessor(torch.nn.Module):
    """Feature extractor + video/audio connectors (ltx_te.py:236-263)."""

    def __init__(self, feature_extractor: FeatureExtractorV2, video_connector: Embeddings1DConnector,
                 audio_connector: Embeddings1DConnector):
        super().__init__()
        self.feature_extractor = feature_extractor
        self.video_connector = video_connector
        self.audio_connector = audio_connector

    def process_hidden_states(self, hidden_states, attention_mask):
        video_feats, audio_feats = self.feature_extractor(hidden_states, attention_mask)
        additive = (attention_mask.to(torch.int64) - 1).to(video_feats.dtype).reshape(
            attention_mask.shape[0], 1, -1, attention_mask.shape[-1]
        ) * torch.finfo(video_feats.dtype).max
        # kept tokens first, in order (ltx_te.py:249-253)
        binary = (additive[:, 0, 0, :] >= 0).to(torch.int32)
        sort_idx = torch.argsort(binary, dim=-1, descending=True, stable=True)
        new_binary = torch.gather(binary, 1, sort_idx)
        reordered = (new_binary.to(additive.dtype) - 1) * torch.finfo(additive.dtype).max
        reordered = reordered[:, None, None, :]

        def gather_feats(f):
            return torch.gather(f, 1, sort_idx.unsqueeze(-1).expand_as(f))

        video_enc, video_mask = self.video_connector(gather_feats(video_feats), reordered)
        video_bin = (video_mask < 1e-6).to(torch.int64).reshape(*video_enc.shape[:2], 1)
        video_enc = video_enc * video_bin
        audio_enc, _ = self.audio_connector(gather_feats(audio_feats), reordered)
        return video_enc, audio_enc, video_bin.squeeze(-1)


def build_embeddings_processor(te_path: str, transformer_path: str) -> EmbeddingsProcessor:
    """Instantiate and load the connector path from the text-encoder and DiT
    checkpoints (ltx_te.py:270-301)."""
    te_cfg = read_metadata(te_path)["gemma_config"]
    text_cfg = te_cfg["text_config"] if "text_config" in te_cfg else te_cfg
    hidden, n_layers = text_cfg["hidden_size"], text_cfg["num_hidden_layers"]
    tr_cfg = read_metadata(transformer_path)["config"]["transformer"]

    def conn(heads_key: str, head_dim_key: str, layers_key: str):
        return Embeddings1DConnector(
            tr_cfg.get(heads_key, tr_cfg.get("connector_num_attention_heads", 32)),
            tr_cfg.get(head_dim_key, tr_cfg.get("connector_attention_head_dim", 128)),
            tr_cfg.get(layers_key, tr_cfg.get("connector_num_layers", 8)),
            tr_cfg.get("connector_positional_embedding_max_pos", [4096]),
            tr_cfg.get("connector_num_learnable_registers", 128),
            tr_cfg.get("connector_apply_gated_attention", False), tr_cfg.get("connector_ff_bias", True))

    with torch.device("meta"):
        fe = FeatureExtractorV2(hidden, n_layers,
                                tr_cfg["num_attention_heads"] * tr_cfg["attention_head_dim"],
                                tr_cfg["audio_num_attention_heads"] * tr_cfg["audio_attention_head_dim"])
        video_conn = conn("connector_num_attention_heads", "connector_attention_head_dim", "connector_num_layers")
        audio_conn = conn("audio_connector_num_attention_heads", "audio_connector_attention_head_dim",
                          "audio_connector_num_layers")
        proc = EmbeddingsProcessor(fe, video_conn, audio_conn)
    sd = {}
    sd.update(load_state_dict(te_path, rename=lambda k: (
        "feature_extractor." + k.removeprefix("text_embedding_projection.")
        if k.startswith("text_embedding_projection.") else None)))
    sd.update(load_state_dict(transformer_path, rename=lambda k: (
        ("video_connector." if "video_embeddings" in k else "audio_connector.") + _conn_leaf(k)
        if k.startswith("model.diffusion_model.") and "_embeddings_connector." in k else None)))
    proc.load_state_dict(sd, strict=False, assign=True)
    return proc.to(DEVICE).eval()


def _conn_leaf(key: str) -> str:
    """Checkpoint key -> module key inside a connector (ltx_te.py:304-310)."""
    leaf = key.split("_embeddings_connector.", 1)[1]
    return (leaf.replace("transformer_1d_blocks", "blocks")
                .replace("to_out.0.", "to_out.")
                .replace("ff.net.0.proj.", "ff.proj_in.")
                .replace("ff.net.2.", "ff.proj_out."))
