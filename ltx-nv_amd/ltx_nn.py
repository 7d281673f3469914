"""Neural building blocks of the LTX-2.5 DiT with the reference's module API
(standalone/ltx_nn.py), the memory-bound parts running on the ltxk HIP kernels.

Kept as in the reference (names, signatures, shapes): rms_norm, sdpa,
generate_freq_grid_np/_pytorch, precompute_freqs_cis, apply_split_rotary_emb,
TimestepEmbedder, CombinedTimestepEmbeddings, AdaLayerNormSingle, Attention,
FeedForward.  Linear layers and scaled-dot-product attention stay on
PyTorch-ROCm; RMSNorm, q/k norm + split RoPE, the per-head gate and
GELU-tanh are ltxk kernels, with fp32 arithmetic and one bf16 rounding per
output.
"""

import functools
import math

import numpy
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

import ltxk

SDPA_PRIORITY = [SDPBackend.CUDNN_ATTENTION, SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION,
                 SDPBackend.MATH]


def rms_norm(x: torch.Tensor, eps: float = 1e-6, weight: torch.Tensor | None = None) -> torch.Tensor:
    """RMSNorm over the last dim (reference ltx_nn.py:18-19) on ltxk_rms_norm."""
    return ltxk.rms_norm(x.contiguous(), weight, eps)


def sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: torch.Tensor | None = None) -> torch.Tensor:
    """q,k,v: (B, H, T, D); PyTorch-ROCm attention with the reference's backend order (ltx_nn.py:22-26).

    Few queries over many keys (the V2A attention: 126 audio tokens over 6144
    video tokens) leave the flash kernel a handful of query tiles, so it runs
    on a few CUs; that shape is split over the keys instead (key_split_applies,
    key_split_partials) and merged by ltxk_attn_combine."""
    if key_split_applies(q, k, mask):
        b, h, tq, d = q.shape
        merged = ltxk.attn_combine(*key_split_partials(q, k, v, KEY_SPLIT_PARTS), KEY_SPLIT_PARTS)
        return merged.view(b, tq, h, d).transpose(1, 2)
    with sdpa_kernel(SDPA_PRIORITY, set_priority=True):
        return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, dropout_p=0.0, is_causal=False)


KEY_SPLIT_MAX_Q = 256
KEY_SPLIT_MIN_K = 2048
KEY_SPLIT_PARTS = 8


def key_split_applies(q: torch.Tensor, k: torch.Tensor, mask: torch.Tensor | None) -> bool:
    """Whether attention of q over k runs split over the keys: no mask, at most
    KEY_SPLIT_MAX_Q queries over at least KEY_SPLIT_MIN_K keys, in whole chunks."""
    return mask is None and q.is_cuda and q.shape[-2] <= KEY_SPLIT_MAX_Q and k.shape[-2] >= KEY_SPLIT_MIN_K \
        and k.shape[-2] % KEY_SPLIT_PARTS == 0


def key_split_partials(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, parts: int) -> tuple:
    """softmax(q k^T / sqrt(D)) v over `parts` equal chunks of the keys: one
    flash-attention launch with the chunks as extra batch items.  Returns the
    chunk outputs (B*parts, H, Tq, D) bf16 and their log-sum-exps
    (B*parts, H, Tq) fp32, which ltxk.attn_combine merges: out = sum_c
    exp(lse_c - lse) out_c with lse = logsumexp_c lse_c, the same softmax
    evaluated in a different order (each chunk's output is rounded to bf16 by
    the flash kernel before the merge)."""
    b, h, tq, d = q.shape
    tk = k.shape[-2]

    def chunks(x):  # (B, H, T, D) -> (B*parts, H, T/parts, D); a view for token-major storage
        return x.transpose(1, 2).reshape(b * parts, tk // parts, h, d).transpose(1, 2)

    qc = q.unsqueeze(1).expand(b, parts, h, tq, d).reshape(b * parts, h, tq, d)
    out, lse = torch.ops.aten._scaled_dot_product_flash_attention(qc, chunks(k), chunks(v))[:2]
    return out, lse


# ---------------------------------------------------------------------------
# RoPE (LTXRopeType.SPLIT)
# ---------------------------------------------------------------------------


@functools.lru_cache(maxsize=8)
def generate_freq_grid_np(theta: float, n_axes: int, inner_dim: int) -> torch.Tensor:
    """theta ** linspace(0, 1, inner_dim // (2 n_axes)) * pi/2 in fp64, cast to fp32 (ltx_nn.py:34-46)."""
    count = inner_dim // (2 * n_axes)
    exps = numpy.linspace(numpy.log(1.0) / numpy.log(theta), numpy.log(theta) / numpy.log(theta), count,
                          dtype=numpy.float64)
    return torch.as_tensor(numpy.power(theta, exps) * math.pi / 2, dtype=torch.float32)


@functools.lru_cache(maxsize=8)
def generate_freq_grid_pytorch(theta: float, n_axes: int, inner_dim: int) -> torch.Tensor:
    """fp32 variant of the frequency grid (ltx_nn.py:49-60)."""
    count = inner_dim // (2 * n_axes)
    exps = torch.linspace(math.log(1.0, theta), math.log(theta, theta), count, dtype=torch.float32)
    return (theta ** exps).to(torch.float32) * math.pi / 2


def precompute_freqs_cis(
    indices_grid: torch.Tensor,
    dim: int,
    out_dtype: torch.dtype,
    theta: float = 10000.0,
    max_pos: list[int] | None = None,
    use_middle_indices_grid: bool = True,
    num_attention_heads: int = 32,
    double_precision: bool = True,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin) tables (B, H, T, D_head/2) for split RoPE (ltx_nn.py:63-96).

    Frequency p = f*n_axes + a (axis fastest) is ind[f] * (2*pos_a/max_pos[a] - 1);
    dim/2 - n_axes*F identity entries are padded in front; the flat table is
    then split per head.  Built once per model call; consumed by
    ltxk_qk_norm_rope.
    """
    if max_pos is None:
        max_pos = [20, 2048, 2048]
    n_axes = indices_grid.shape[1]
    grid_fn = generate_freq_grid_np if double_precision else generate_freq_grid_pytorch
    ind = grid_fn(theta, n_axes, dim).to(indices_grid.device)
    pos = indices_grid
    if pos.ndim == 4:
        pos = (pos[..., 0] + pos[..., 1]) / 2.0 if use_middle_indices_grid else pos[..., 0]
    frac = torch.stack([pos[:, a] / max_pos[a] for a in range(n_axes)], dim=-1)      # (B, T, A)
    ang = (ind * (frac.unsqueeze(-1) * 2 - 1)).transpose(-1, -2).flatten(2)          # (B, T, F*A)
    pad = dim // 2 - ang.shape[-1]
    cos, sin = ang.cos(), ang.sin()
    if pad:
        cos = torch.cat([torch.ones_like(cos[:, :, :pad]), cos], dim=-1)
        sin = torch.cat([torch.zeros_like(sin[:, :, :pad]), sin], dim=-1)
    b, t = cos.shape[0], cos.shape[1]
    cos = cos.reshape(b, t, num_attention_heads, -1).swapaxes(1, 2)
    sin = sin.reshape(b, t, num_attention_heads, -1).swapaxes(1, 2)
    return cos.to(out_dtype).contiguous(), sin.to(out_dtype).contiguous()


def precompute_freqs_cis_compact(
    indices_grid: torch.Tensor,
    dim: int,
    out_dtype: torch.dtype = torch.bfloat16,
    theta: float = 10000.0,
    max_pos: list[int] | None = None,
    use_middle_indices_grid: bool = True,
    num_attention_heads: int = 32,
    double_precision: bool = True,
    merge_slow_axes: bool = True,
) -> ltxk.CompactRope:
    """The tables of precompute_freqs_cis in ltxk's compact form.

    A pair's angle depends on one position axis only, so the table row of a
    token is assembled from one row per axis, keyed by that axis' coordinate:
    for each axis the distinct coordinates (16, 16 and 24 for a 16x16x24 latent
    grid, 16 for the A2V/V2A time axis) get a row holding cos/sin at that
    axis' pairs and 0 elsewhere.  Each distinct angle is computed with the same
    fp32 operations as the full tables, so every combined entry equals the
    full table's bit for bit, while the rows (a few hundred KB) stay in cache.
    With three axes and merge_slow_axes the time and height rows are merged
    into one row per distinct (time, height) pair (256 for the 16x16x24 grid,
    2 MB), so the index has two columns.  One device-to-host read per axis
    (the count of distinct coordinates).
    """
    if max_pos is None:
        max_pos = [20, 2048, 2048]
    b, n_axes, t = indices_grid.shape[0], indices_grid.shape[1], indices_grid.shape[2]
    grid_fn = generate_freq_grid_np if double_precision else generate_freq_grid_pytorch
    ind = grid_fn(theta, n_axes, dim).to(indices_grid.device)
    pos = indices_grid
    if pos.ndim == 4:
        pos = (pos[..., 0] + pos[..., 1]) / 2.0 if use_middle_indices_grid else pos[..., 0]
    nf = ind.numel()
    half = dim // 2
    pad = half - nf * n_axes
    axis_rows = []
    for a in range(n_axes):
        coords, inverse = torch.unique(pos[:, a], return_inverse=True)
        frac = coords / max_pos[a]
        ang = ind * (frac.unsqueeze(-1) * 2 - 1)                        # (U, F)
        cols = pad + torch.arange(nf, device=ang.device) * n_axes + a
        c = torch.zeros(coords.numel(), half, device=ang.device, dtype=torch.float32)
        s = torch.zeros_like(c)
        c[:, cols] = ang.cos()
        s[:, cols] = ang.sin()
        if a == 0 and pad:
            c[:, :pad] = 1.0
        axis_rows.append((c, s, inverse))
    if n_axes == 3 and merge_slow_axes:
        # The two slower axes (time, height) change every w tokens only: one
        # row per distinct (time, height) pair holding both axes' entries
        # (their pairs are disjoint, so the sum is exact) leaves the kernel two
        # table rows per token instead of three.
        (c0, s0, i0), (c1, s1, i1) = axis_rows[0], axis_rows[1]
        pairs, inverse = torch.unique(i0 * c1.shape[0] + i1, return_inverse=True)
        p0, p1 = pairs // c1.shape[0], pairs % c1.shape[0]
        axis_rows = [(c0[p0] + c1[p1], s0[p0] + s1[p1], inverse), axis_rows[2]]
    cos_rows, sin_rows, index = [], [], []
    first = 0
    for c, s, inverse in axis_rows:
        cos_rows.append(c)
        sin_rows.append(s)
        index.append(inverse + first)
        first += c.shape[0]
    cos = torch.cat(cos_rows).to(out_dtype).contiguous()
    sin = torch.cat(sin_rows).to(out_dtype).contiguous()
    idx = torch.stack(index, dim=-1).to(torch.int32).contiguous()  # (B, T, A)
    return ltxk.CompactRope(cos, sin, idx, (b, num_attention_heads, t, half // num_attention_heads), checked=True)


def apply_split_rotary_emb(x: torch.Tensor, freqs_cis) -> torch.Tensor:
    """Split-half rotation per head (ltx_nn.py:99-115) on ltxk_qk_norm_rope.

    x: (B, T, H*D) token-major or (B, H, T, D); freqs: (cos, sin) (B, H, T, D/2)
    or the compact form of precompute_freqs_cis_compact.  Returns a new tensor
    of x's shape.
    """
    if isinstance(freqs_cis, ltxk.CompactRope):
        pe, h = freqs_cis, freqs_cis.shape[1]
    else:
        cos, sin = freqs_cis
        pe, h = (cos.contiguous(), sin.contiguous()), cos.shape[1]
    if x.ndim == 4:
        b, _, t, d = x.shape
        tok = x.transpose(1, 2).reshape(b, t, h * d).contiguous()
        ltxk.qk_norm_rope(tok, None, h, d, q_pe=pe)
        return tok.view(b, t, h, d).transpose(1, 2)
    out = x.contiguous().clone()
    ltxk.qk_norm_rope(out, None, h, x.shape[-1] // h, q_pe=pe)
    return out


# ---------------------------------------------------------------------------
# Timestep embedding (PixArt-alpha style)
# ---------------------------------------------------------------------------


class TimestepEmbedder(torch.nn.Module):
    def __init__(self, in_channels: int, time_embed_dim: int):
        super().__init__()
        self.linear_1 = torch.nn.Linear(in_channels, time_embed_dim)
        self.linear_2 = torch.nn.Linear(time_embed_dim, time_embed_dim)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.linear_2(F.silu(self.linear_1(x)))


class CombinedTimestepEmbeddings(torch.nn.Module):
    """256-wide sinusoidal projection then TimestepEmbedder (ltx_nn.py:133-145)."""

    def __init__(self, embedding_dim: int):
        super().__init__()
        self.timestep_embedder = TimestepEmbedder(256, embedding_dim)

    def forward(self, timestep: torch.Tensor, hidden_dtype: torch.dtype) -> torch.Tensor:
        from common import get_timestep_embedding

        proj = get_timestep_embedding(timestep, 256, max_period=10000)
        return self.timestep_embedder(proj.to(hidden_dtype))


class AdaLayerNormSingle(torch.nn.Module):
    """SiLU -> Linear(embedding_dim -> coefficient*embedding_dim) (ltx_nn.py:148-158)."""

    def __init__(self, embedding_dim: int, embedding_coefficient: int = 6):
        super().__init__()
        self.emb = CombinedTimestepEmbeddings(embedding_dim)
        self.linear = torch.nn.Linear(embedding_dim, embedding_coefficient * embedding_dim, bias=True)

    def forward(self, timestep: torch.Tensor, hidden_dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
        embedded = self.emb(timestep, hidden_dtype=hidden_dtype)
        return self.linear(F.silu(embedded)), embedded


# ---------------------------------------------------------------------------
# Attention + FFN
# ---------------------------------------------------------------------------


class Attention(torch.nn.Module):
    """Multi-head attention with RMS q/k-norm, split RoPE and per-head gating (ltx_nn.py:166-236).

    q/k/v projections and SDPA are PyTorch-ROCm.  q_norm/k_norm + RoPE run as
    one in-place ltxk_qk_norm_rope launch on the fresh projections; the head
    merge, the perturbation blend (B=4 guidance batch) and the per-head
    2*sigmoid gate are one ltxk_head_gate pass over the attention output.
    """

    def __init__(self, query_dim: int, context_dim: int | None = None, heads: int = 8, dim_head: int = 64,
                 norm_eps: float = 1e-6, apply_gated_attention: bool = False):
        super().__init__()
        self.heads = heads
        self.dim_head = dim_head
        inner_dim = heads * dim_head
        context_dim = query_dim if context_dim is None else context_dim
        self.q_norm = torch.nn.RMSNorm(inner_dim, eps=norm_eps)
        self.k_norm = torch.nn.RMSNorm(inner_dim, eps=norm_eps)
        self.to_q = torch.nn.Linear(query_dim, inner_dim, bias=True)
        self.to_k = torch.nn.Linear(context_dim, inner_dim, bias=True)
        self.to_v = torch.nn.Linear(context_dim, inner_dim, bias=True)
        self.to_gate_logits = torch.nn.Linear(query_dim, heads, bias=True) if apply_gated_attention else None
        self.to_out = torch.nn.Linear(inner_dim, query_dim, bias=True)

    def forward(self, x: torch.Tensor, context: torch.Tensor | None = None, mask: torch.Tensor | None = None,
                pe: tuple[torch.Tensor, torch.Tensor] | None = None,
                k_pe: tuple[torch.Tensor, torch.Tensor] | None = None,
                perturbation_mask: torch.Tensor | None = None, all_perturbed: bool = False) -> torch.Tensor:
        context = x if context is None else context
        b = x.shape[0]
        h, dh = self.heads, self.dim_head
        v = self.to_v(context)
        gates = self.to_gate_logits(x).contiguous() if self.to_gate_logits is not None else None
        if all_perturbed:
            out = v if gates is None else ltxk.head_gate(v, gates)
            return self.to_out(out)
        q = self.to_q(x)
        k = self.to_k(context)
        ltxk.qk_norm_rope(q, k, h, dh, q_weight=self.q_norm.weight, k_weight=self.k_norm.weight,
                          q_pe=pe, k_pe=pe if k_pe is None else k_pe, eps=self.eps)
        return self.attend(q, k, v, gates, mask, perturbation_mask)

    @property
    def eps(self) -> float:
        return self.q_norm.eps if self.q_norm.eps is not None else 1e-6

    def attend(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gates: torch.Tensor | None,
               mask: torch.Tensor | None = None, perturbation_mask: torch.Tensor | None = None) -> torch.Tensor:
        """The part of forward after q/k norm + RoPE (ltx_nn.py:219-236): SDPA on
        token-major q, k, v (B, T, H*Dh), the head merge [+ perturbation blend]
        [+ per-head gate] in one ltxk_head_gate pass, then to_out.  Lets a caller
        prepare the q/k of two attentions in one launch (Block's A2V/V2A)."""
        b = q.shape[0]
        h, dh = self.heads, self.dim_head
        q4 = q.view(b, -1, h, dh).transpose(1, 2)
        k4 = k.view(b, -1, h, dh).transpose(1, 2)
        v4 = v.view(b, -1, h, dh).transpose(1, 2)
        if mask is not None:
            if mask.ndim == 2:
                mask = mask.unsqueeze(0)
            if mask.ndim == 3:
                mask = mask.unsqueeze(1)
        if perturbation_mask is None and key_split_applies(q4, k4, mask):
            # key-split attention: its merge, the head merge and the gate in one pass
            part, lse = key_split_partials(q4, k4, v4, KEY_SPLIT_PARTS)
            return self.to_out(ltxk.attn_combine(part, lse, KEY_SPLIT_PARTS, gates))
        attn = sdpa(q4, k4, v4, mask)  # (B, H, T, D) view
        if perturbation_mask is None and gates is None:
            out = attn.transpose(1, 2).reshape(b, -1, h * dh)
        else:
            # head merge [+ perturbation blend] [+ per-head gate] in one pass
            pm = None
            if perturbation_mask is not None:
                pm = perturbation_mask.reshape(-1).to(torch.bfloat16).contiguous()
            out = ltxk.head_gate(attn, gates, v=v.contiguous() if pm is not None else None, mask=pm)
        return self.to_out(out)


class FeedForward(torch.nn.Module):
    """proj_in -> GELU-tanh (ltxk, in place) -> proj_out (ltx_nn.py:239-248)."""

    def __init__(self, dim: int, dim_out: int | None = None, mult: int = 4, bias: bool = True):
        super().__init__()
        dim_out = dim if dim_out is None else dim_out
        inner = int(dim * mult)
        self.proj_in = torch.nn.Linear(dim, inner, bias=bias)
        self.proj_out = torch.nn.Linear(inner, dim_out, bias=bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        hdn = self.proj_in(x)
        ltxk.gelu_tanh(hdn, out=hdn)
        return self.proj_out(hdn)
