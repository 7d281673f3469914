"""The 48-block chain bench times what it claims: bench.fused_block (the ltxk
kernels as LTXModel runs them, on one HIP stream and on two) computes what
its comparator bench.eager_block (the reference's non-GEMM op sequence of a
block, ltx_dit.py:250-317 and ltx_nn.py:204-248, in bf16 eager) computes, at
the full LTX-2.5 shape (video 6144 x 4096, audio 126 x 2048, text 1024): every
launch's output against the eager op's, by relative L2 error and cosine.  The
fused kernels round once where the eager ops round after every op, so the two
differ by bf16 rounding (relative L2 ~ 2^-8); a wrong operand, row or table
gives errors of order 1."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _copy(t):
    return {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in t.items()}


@pytest.mark.parametrize("two_streams", [False, True])
def test_fused_chain_block_matches_eager_comparator(two_streams):
    import bench

    dev = torch.device("cuda")
    t = bench.make_chain_inputs(dev)
    for p in ("v", "a"):
        # the fused block's first norm adds the previous block's FFN residual
        # (x + off * gate); with off = 0 both start from the same x
        t[f"{p}_off"].zero_()
    tf, te = _copy(t), _copy(t)
    for p in ("v", "a"):  # the step's context modulation with this block's prompt table
        tf[f"{p}_psst_all"] = t[f"{p}_psst"][None].contiguous()
    bench.chain_prologue(tf, 1)
    got = {}
    side = torch.cuda.Stream() if two_streams else None
    bench.fused_block(tf, side, fork=True, join=True, collect=got)
    torch.cuda.synchronize()
    for k in ("a2v_q", "v2a_k", "a2v_k", "v2a_q"):  # rotated in place
        got[k] = tf[k]
    for p in ("v", "a"):
        got[f"{p}_ctx"] = tf[f"{p}_ctx_all"][0]
    want = {}
    bench.eager_block(te, collect=want)
    torch.cuda.synchronize()
    assert set(want) <= set(got), sorted(set(want) - set(got))
    bad, worst = [], (0.0, 1.0)
    for name, w in sorted(want.items()):
        g = got[name].float().reshape(-1)
        w = w.float().reshape(-1)
        assert g.numel() == w.numel(), (name, g.numel(), w.numel())
        rel = float((g - w).norm() / w.norm())
        cos = float(torch.nn.functional.cosine_similarity(g, w, dim=0))
        worst = (max(worst[0], rel), min(worst[1], cos))
        if not (rel < 2e-2 and cos > 0.9998):
            bad.append(f"{name}: rel-L2 {rel:.3g} cos {cos:.6f}")
    print(f"{len(want)} outputs, largest rel-L2 {worst[0]:.3g}, smallest cosine {worst[1]:.6f}")
    assert not bad, bad
