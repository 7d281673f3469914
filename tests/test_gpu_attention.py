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
