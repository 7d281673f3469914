"""Attention on PyTorch-ROCm as ltx_nn.sdpa runs it (GPU): the key-split form
used for few queries over many keys (the V2A attention, 126 audio tokens over
6144 video tokens) equals the softmax attention within the bf16 rounding of its
result, on the token-major views the model passes and on contiguous inputs,
against an fp32 evaluation of the formula and against PyTorch's own bf16
attention."""

import math

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _fp32_attention(q, k, v):
    s = torch.matmul(q.float(), k.float().transpose(-1, -2).contiguous()) / math.sqrt(q.shape[-1])
    return torch.matmul(torch.softmax(s, dim=-1), v.float())


@pytest.mark.parametrize("b,tq,tk,h,d,views", [(1, 126, 6144, 32, 64, True), (2, 126, 6144, 32, 64, False),
                                               (1, 7, 2048, 4, 64, True), (4, 256, 4096, 2, 128, True)])
def test_key_split_attention_matches_softmax_attention(b, tq, tk, h, d, views):
    import ltx_nn

    g = torch.Generator(device=DEV).manual_seed(tq + tk)
    if views:  # token-major projections viewed as (B, H, T, D), as Attention.forward passes them
        q, k, v = (torch.randn(b, t, h * d, device=DEV, generator=g).to(torch.bfloat16).view(b, t, h, d)
                   .transpose(1, 2) for t in (tq, tk, tk))
    else:
        q, k, v = (torch.randn(b, h, t, d, device=DEV, generator=g).to(torch.bfloat16) for t in (tq, tk, tk))
    assert tq <= ltx_nn.KEY_SPLIT_MAX_Q and tk >= ltx_nn.KEY_SPLIT_MIN_K  # the split path is the one taken
    got = ltx_nn.sdpa(q, k, v)
    assert got.shape == (b, h, tq, d) and got.dtype == torch.bfloat16
    want = _fp32_attention(q, k, v)
    err = (got.float() - want).abs()
    # at the bf16 rounding level of the result's scale
    assert err.max().item() <= 2.0**-7 * want.abs().max().item(), f"max err {err.max().item():.3e}"
    # and as close to the formula as PyTorch's own bf16 attention is (its chunk outputs are rounded once more)
    lib_err = (torch.nn.functional.scaled_dot_product_attention(q, k, v).float() - want).abs()
    assert err.max().item() <= 2.0 * lib_err.max().item() + 1e-5
    assert err.mean().item() <= 2.0 * lib_err.mean().item() + 1e-6


def test_masked_or_many_query_attention_keeps_the_library_path():
    import ltx_nn

    g = torch.Generator(device=DEV).manual_seed(3)
    q, k, v = (torch.randn(1, 2, t, 64, device=DEV, generator=g).to(torch.bfloat16) for t in (300, 2048, 2048))
    torch.testing.assert_close(ltx_nn.sdpa(q, k, v), torch.nn.functional.scaled_dot_product_attention(q, k, v),
                               rtol=0, atol=0)
    mask = torch.zeros(1, 1, 100, 2048, device=DEV, dtype=torch.bfloat16)
    q2 = q[:, :, :100]
    torch.testing.assert_close(ltx_nn.sdpa(q2, k, v, mask),
                               torch.nn.functional.scaled_dot_product_attention(q2, k, v, attn_mask=mask),
                               rtol=0, atol=0)


def test_key_split_attention_with_the_gate_in_the_combine():
    """Attention.attend on the V2A shape (126 audio queries over 6144 video keys,
    32 heads x 64, gated): the key-split merge, head merge and per-head gate in
    one ltxk_attn_combine pass equal the unfused sequence (merge, then
    ltxk_head_gate) bit for bit, and 2*sigmoid(logit) * softmax attention in
    fp32 within the bf16 rounding of the result."""
    import ltx_nn
    import ltxk

    b, tq, tk, h, d = 1, 126, 6144, 32, 64
    g = torch.Generator(device=DEV).manual_seed(11)
    q, k, v = (torch.randn(b, t, h * d, device=DEV, generator=g).to(torch.bfloat16) for t in (tq, tk, tk))
    logits = torch.randn(b, tq, h, device=DEV, generator=g).to(torch.bfloat16)
    q4, k4, v4 = (x.view(b, -1, h, d).transpose(1, 2) for x in (q, k, v))
    assert ltx_nn.key_split_applies(q4, k4, None)
    part, lse = ltx_nn.key_split_partials(q4, k4, v4, ltx_nn.KEY_SPLIT_PARTS)
    fused = ltxk.attn_combine(part, lse, ltx_nn.KEY_SPLIT_PARTS, logits)
    merged = ltxk.attn_combine(part, lse, ltx_nn.KEY_SPLIT_PARTS)
    unfused = ltxk.head_gate(merged.view(b, tq, h, d).transpose(1, 2), logits)
    assert torch.equal(fused.view(torch.int16), unfused.view(torch.int16))
    gate = 2.0 * torch.sigmoid(logits.float())                                  # (B, T, H)
    want = (_fp32_attention(q4, k4, v4) * gate.transpose(1, 2).unsqueeze(-1)).transpose(1, 2).reshape(b, tq, h * d)
    err = (fused.float() - want).abs()
    assert err.max().item() <= 2.0**-7 * want.abs().max().item(), f"max err {err.max().item():.3e}"


@pytest.mark.parametrize("b,parts,t,h,d", [(4, 8, 126, 32, 64), (1, 16, 5, 2, 128), (2, 4, 33, 3, 64),
                                           (1, 1, 9, 2, 64)])
def test_attn_combine_on_given_partials(b, parts, t, h, d):
    """ltxk_attn_combine on partials and log-sum-exps given directly (strided
    views, lse rows longer than the token count): the log-sum-exp softmax over
    the chunks and the weighted sum in fp32 (torch), to the bf16 rounding of the
    result; with one chunk the partial itself, bit for bit."""
    import ltxk

    g = torch.Generator(device=DEV).manual_seed(b * 100 + parts)
    part = torch.randn(b * parts, t, h, d, device=DEV, generator=g).to(torch.bfloat16).transpose(1, 2)  # BTHD memory
    lse_full = torch.randn(b * parts, h, t + 7, device=DEV, generator=g) * 3.0
    lse = lse_full[:, :, :t]
    got = ltxk.attn_combine(part, lse, parts)
    w = torch.softmax(lse.reshape(b, parts, h, t), dim=1).unsqueeze(-1)
    want = (part.float().reshape(b, parts, h, t, d) * w).sum(dim=1).transpose(1, 2).reshape(b, t, h * d)
    err = (got.float() - want).abs()
    assert err.max().item() <= 2.0**-8 * want.abs().max().item() + 1e-6
    if parts == 1:
        assert torch.equal(got.view(torch.int16), part.transpose(1, 2).reshape(b, t, h * d).view(torch.int16))
