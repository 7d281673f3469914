"""The entry points under HIP graph capture (GPU): a miniature denoise step
(noise, norm + modulation, q/k norm + compact RoPE, head gate, residual + norm
with two modulations, GELU, gated residual, guidance with rescale and its
workspace, Euler) captured once and replayed; every replay must equal the
eager run bit for bit.  Between replays the outputs are overwritten and the
eager step runs again, with device synchronisations, so a replay cannot pass
on values left behind by an earlier run."""

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bf(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16).to(DEV)


def _inputs():
    import ltx_dit
    import ltx_nn

    f, h, w = 6, 10, 10  # 600 video tokens, one batch item, full 4096-wide rows
    t, d, heads = f * h * w, 4096, 32
    pos = ltx_dit.video_positions(1, f, h, w, 24.0, torch.device(DEV))
    pe = ltx_nn.precompute_freqs_cis_compact(pos, d, torch.bfloat16, max_pos=[20, 2048, 2048],
                                             num_attention_heads=heads)
    c = 128
    return {
        "t": t, "d": d, "heads": heads, "pe": pe,
        "x": bf((1, t, d), 1), "f": bf((1, t, d), 2), "q0": bf((1, t, d), 3), "k0": bf((1, t, d), 4),
        "wq": bf((d,), 5), "wk": bf((d,), 6), "logits": bf((1, t, heads), 7),
        "h": bf((1, t, 4 * d), 8), "table": bf((9, d), 9, 0.05), "emb": bf((1, 1, 9 * d), 10, 0.05),
        "lat": bf((1, t, c), 11), "vel": bf((4, t, c), 12),
        "ts": torch.full((4, 1, 1), 0.5, dtype=torch.float32, device=DEV),
        "e0": torch.randn(t * c, generator=torch.Generator().manual_seed(13)).to(DEV),
        "noise": torch.empty(t * c, dtype=torch.float32, device=DEV),
        "q": torch.empty(1, t, d, dtype=torch.bfloat16, device=DEV),
        "k": torch.empty(1, t, d, dtype=torch.bfloat16, device=DEV),
        "e": torch.empty(t * c, dtype=torch.float32, device=DEV),
    }


def _step(b):
    """One pass over the entry points; returns every output tensor."""
    import ltxk

    A = lambda r: ltxk.AdaRef(b["table"], r, b["emb"])  # noqa: E731
    n = b["noise"].numel()
    ltxk.philox_normal(b["noise"], 42, 0, ltxk.device_policy_threads(n))
    y = ltxk.norm_modulate(b["x"], shift=A(0), scale=A(1))
    b["q"].copy_(b["q0"])
    b["k"].copy_(b["k0"])
    ltxk.qk_norm_rope(b["q"], b["k"], b["heads"], b["d"] // b["heads"], q_weight=b["wq"], k_weight=b["wk"],
                      q_pe=b["pe"], k_pe=b["pe"])
    hg = ltxk.head_gate(b["q"], b["logits"])
    xo, y1, y2 = ltxk.add_norm_modulate(b["x"], hg, gate=A(2), shift=A(3), scale=A(4), shift2=A(5), scale2=A(6))
    g = ltxk.gelu_tanh(b["h"])
    r = ltxk.gated_residual(xo, b["f"], gate=A(7))
    den, nxt, _ = ltxk.guide(b["lat"], b["vel"], b["ts"], 3.0, 1.0, 3.0, 0.7, sigma=0.5, dt=-0.125)
    b["e"].copy_(b["e0"])
    ltxk.euler_update(b["e"], b["noise"], -0.125)
    return [b["noise"], y, b["q"], b["k"], hg, xo, y1, y2, g, r, den, nxt, b["e"]]


def test_graph_replays_equal_eager():
    b = _inputs()
    want = [o.clone() for o in _step(b)]  # eager (also warms the launch-shape caches)
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        got = _step(b)
    torch.cuda.synchronize()

    for replay in range(3):
        for o in got:
            o.fill_(float("nan") if o.is_floating_point() else 0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (o, w) in enumerate(zip(got, want)):
            assert torch.equal(o, w), f"replay {replay}: output {i} differs from the eager run"
        # the program's own eager work between replays
        again = _step(b)
        torch.cuda.synchronize()
        for i, (o, w) in enumerate(zip(again, want)):
            assert torch.equal(o, w), f"eager run after replay {replay}: output {i} differs"
