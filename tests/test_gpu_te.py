"""Text-encoder connector path (GPU): ltxk_feature_norm against the oracle, and
the connector modules (ltx-nv_amd/ltx_te.py) against the reference's own
outputs in tests/golden/te_golden.npz (FeatureExtractorV2 and
EmbeddingsProcessor.process_hidden_states on a small configuration: 4 layers of
64, video connector 2x64 gated, audio 2x32, 2 blocks, 4 registers, B=2 with
left padding).

Projections and attention run in bf16 on PyTorch-ROCm here and in fp32/bf16 on
the CPU in the reference, so the module check is statistical, as for LTXModel:
relative L2 to the fp32 reference within 1.5x of the reference's own bf16 run,
cosine >= 0.999."""

import importlib.util

import numpy as np
import pytest
import torch

from conftest import GOLDEN, assert_close_bf16, bf16_from_bits
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
G = np.load(GOLDEN / "te_golden.npz")


def _golden_module():
    spec = importlib.util.spec_from_file_location("make_te_golden", GOLDEN / "make_te_golden.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _bf(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def _normed_neighbours(layers, eps=1e-6):
    """The oracle's interleaved bf16 normed values (ltx_te.py:167-184 before the
    scales) and their bf16 neighbours one ulp down and up."""
    normed = torch.stack([O.rnd(O._rms(O.f32(x), eps)) for x in layers], dim=-1)
    b, t, d, n = normed.shape
    bits = normed.reshape(b, t, d * n).view(torch.int16)
    return [(bits + k).view(torch.bfloat16) for k in (-1, 0, 1)]


@pytest.mark.parametrize("b,t,d,n", [(1, 64, 3840, 9), (2, 7, 72, 5), (1, 3, 8, 1), (1, 5, 64, 64), (2, 1100, 64, 3),
                                     (1, 40, 3840, 49), (1, 300, 3840, 49), (1, 5, 520, 7), (1, 9, 4096, 30),
                                     (1, 3, 8192, 25), (1, 3, 256, 64), (2, 300, 4096, 30), (1, 520, 8192, 1),
                                     (1, 700, 3840, 9), (1, 290, 4000, 40)])
def test_feature_norm_matches_oracle(b, t, d, n):
    """Rows held in registers (d >= 512 and n * d / 8 <= 24576 chunks: one,
    two and three tiles of columns, more rows than workgroups so a workgroup
    carries its next row's loads and statistics across tiles, a last tile
    narrower than the others, d not a multiple of 64, one layer of 8192) and
    rows streamed twice (smaller d, 64 layers of 256, or 25 x 8192)."""
    import ltxk

    layers = [_bf((b, t, d), 60 + i, scale=0.5 + i) for i in range(n)]
    keep = torch.ones(b, t, dtype=torch.int64)
    keep[0, : t // 3] = 0
    scales = (1.0327956, 0.7302967)
    w0, w1 = O.feature_norm(layers, keep, *scales)
    g0, g1 = ltxk.feature_norm([x.to(DEV) for x in layers], keep.to(DEV), *scales)
    normed = _normed_neighbours(layers)
    kept = keep.reshape(b, t, 1) != 0
    for got, want, sc, nm in ((g0, w0, scales[0], "out0"), (g1, w1, scales[1], "out1")):
        got = got.cpu()
        assert got.shape == (b, t, d * n)
        same = (got.view(torch.int16) == want.view(torch.int16)).float().mean().item()
        assert same > 0.999, f"{nm}: {same:.5f} bit-equal"
        # every element is round(n' * scale) for n' the oracle's bf16 normed
        # value or one of its bf16 neighbours: the sum of squares is
        # accumulated in another order than torch's, which can move a normed
        # value across a bf16 rounding boundary (one ulp), and the scaled
        # rounding can make that two ulps of the output
        ok = torch.zeros_like(got, dtype=torch.bool)
        for nb in normed:
            ok |= got.view(torch.int16) == O.rnd(O.f32(nb) * sc).view(torch.int16)
        ok |= ~kept.expand_as(got) & (got.view(torch.int16) == 0)
        assert bool(ok.all()), f"{nm}: {int((~ok).sum())} elements off by more than one normed ulp"
        # masked tokens are exactly +0
        assert int(got[0, : t // 3].view(torch.int16).abs().sum()) == 0


@pytest.mark.parametrize("b,t,d,n", [(1, 600, 3840, 49), (1, 37, 3840, 9), (1, 40, 8192, 25)])
def test_feature_norm_masked_tokens_ignore_their_hidden_states(b, t, d, n):
    """A masked token's outputs are +0 whatever its hidden states hold (NaN,
    inf, huge values; the register-resident form does not read them, the
    streamed form reads them), and the kept tokens' outputs equal those of
    the same call with finite values there: bit for bit, so the workgroups
    that pass over masked rows hand correct statistics to their next rows."""
    import ltxk

    layers = [_bf((b, t, d), 300 + i, scale=0.5 + i) for i in range(n)]
    keep = torch.ones(b, t, dtype=torch.int64)
    keep[0, 1::3] = 0
    keep[0, -5:] = 0
    dirty = [x.clone() for x in layers]
    for i, x in enumerate(dirty):
        x[0, 1::3] = [float("nan"), float("inf"), -1e30][i % 3]
        x[0, -5:] = float("nan")
    scales = (1.0327956, 0.7302967)
    clean = ltxk.feature_norm([x.to(DEV) for x in layers], keep.to(DEV), *scales)
    got = ltxk.feature_norm([x.to(DEV) for x in dirty], keep.to(DEV), *scales)
    masked = keep.reshape(b, t) == 0
    for g, c in zip(got, clean):
        g, c = g.cpu().view(torch.int16), c.cpu().view(torch.int16)
        assert torch.equal(g, c)
        assert int(g[masked].abs().sum()) == 0


def test_feature_norm_single_output_and_no_mask():
    import ltxk

    layers = [_bf((1, 10, 128), 70 + i) for i in range(3)]
    g0, g1 = ltxk.feature_norm([x.to(DEV) for x in layers], None, 2.0)
    w0, _ = O.feature_norm(layers, None, 2.0, 1.0)
    assert g1 is None
    assert_close_bf16(g0.cpu(), w0, what="out0")


def _processor():
    import ltx_te

    mk = _golden_module()
    proc = mk.build(ltx_te)
    assert sorted(n for n, _ in proc.named_parameters()) == list(G["param_names"])
    mk.init_weights(proc)
    return mk, proc.to(DEV, torch.bfloat16).eval()


def _layers():
    n = sum(1 for k in G.files if k.startswith("layer"))
    return tuple(bf16_from_bits(G[f"layer{i}"]).to(DEV) for i in range(n))


def _rel(a, b):
    return float((a - b).norm() / b.norm())


def _cos(a, b):
    return float(torch.nn.functional.cosine_similarity(a.flatten(), b.flatten(), dim=0))


def _check(got, key):
    ref32 = torch.from_numpy(G[f"{key}_f32"])
    ref16 = torch.from_numpy(G[f"{key}_bf16"])
    got = got.float().cpu()
    assert got.shape == ref32.shape
    e_ours, e_ref = _rel(got, ref32), _rel(ref16, ref32)
    assert _cos(got, ref32) >= 0.999, (key, _cos(got, ref32))
    assert e_ours <= 1.5 * e_ref + 2e-3, f"{key}: ours {e_ours:.4g} vs reference bf16 {e_ref:.4g}"


def test_feature_extractor_matches_reference_outputs():
    _, proc = _processor()
    mask = torch.from_numpy(G["mask"]).to(DEV)
    with torch.no_grad():
        v, a = proc.feature_extractor(_layers(), mask)
    _check(v, "vfeat")
    _check(a, "afeat")


def test_embeddings_processor_matches_reference_outputs():
    _, proc = _processor()
    mask = torch.from_numpy(G["mask"]).to(DEV)
    with torch.no_grad():
        venc, aenc, vbin = proc.process_hidden_states(_layers(), mask)
    _check(venc, "venc")
    _check(aenc, "aenc")
    assert np.array_equal(vbin.cpu().numpy(), G["vbin_f32"])


def test_connector_block_forward_equals_fused_chain():
    """ConnectorBlock.forward (residuals added per block) and the connector's
    fused chain (FF residual taken in by the next norm) give the same bits."""
    import ltxk
    import ltx_nn

    _, proc = _processor()
    conn = proc.video_connector
    x = _bf((2, 16, 128), 80).to(DEV)
    mask = torch.zeros(2, 1, 1, 16, device=DEV, dtype=torch.bfloat16)
    grid = torch.arange(16, dtype=torch.float32, device=DEV)[None, None, :].expand(2, -1, -1)
    pe = ltx_nn.precompute_freqs_cis(grid, dim=128, out_dtype=torch.bfloat16, max_pos=[4096],
                                     use_middle_indices_grid=False, num_attention_heads=2)
    with torch.no_grad():
        ref = x
        for blk in conn.blocks:
            ref = blk(ref, mask, pe)
        ref = ltxk.rms_norm(ref, None, 1e-6)
        fused = x
        pending = None
        for blk in conn.blocks:
            fused, pending = blk._run(fused, pending, mask, pe, defer=True)
        _, fused = ltxk.add_norm_modulate(fused, pending, eps=1e-6)
    assert torch.equal(ref, fused)


def _te_checkpoint_name(name: str) -> tuple[str, str]:
    """Our EmbeddingsProcessor parameter name -> (checkpoint, key): the text
    encoder's feature projections or the DiT's connectors, under the
    reference's names (the inverse of build_embeddings_processor's renames,
    ltx_te.py:289-310)."""
    if name.startswith("feature_extractor."):
        return "te", "text_embedding_projection." + name[len("feature_extractor."):]
    owner, leaf = name.split(".", 1)
    for ours, theirs in (("blocks.", "transformer_1d_blocks."), ("to_out.", "to_out.0."),
                         ("ff.proj_in.", "ff.net.0.proj."), ("ff.proj_out.", "ff.net.2.")):
        leaf = leaf.replace(ours, theirs)
    side = "video" if owner == "video_connector" else "audio"
    return "dit", f"model.diffusion_model.{side}_embeddings_connector.{leaf}"


@pytest.mark.parametrize("gated", [False, True])
def test_build_embeddings_processor_reads_reference_checkpoints(tmp_path, gated):
    """build_embeddings_processor on a text-encoder checkpoint (gemma_config
    metadata, text_embedding_projection.* keys) and a DiT checkpoint (connector
    config keys, *_embeddings_connector.* keys, the audio connector's own head
    width) gives the source processor's parameters bit for bit and its
    outputs; keys of other modules in either file are dropped."""
    import json

    import ltx_te
    from safetensors.torch import save_file

    mk = _golden_module()
    vconn = dict(mk.VCONN, gated=gated)
    aconn = dict(mk.ACONN, gated=gated)
    src = ltx_te.EmbeddingsProcessor(ltx_te.FeatureExtractorV2(**mk.FE), ltx_te.Embeddings1DConnector(**vconn),
                                     ltx_te.Embeddings1DConnector(**aconn))
    mk.init_weights(src)
    src = src.to(DEV, torch.bfloat16).eval()
    files = {"te": {"model.language_model.embed_tokens.weight": torch.zeros(4)},
             "dit": {"model.diffusion_model.patchify_proj.weight": torch.zeros(4)}}
    for n, p in src.named_parameters():
        which, key = _te_checkpoint_name(n)
        files[which][key] = p.detach().cpu().contiguous()
    gemma = {"text_config": {"hidden_size": mk.FE["gemma_hidden"], "num_hidden_layers": mk.FE["num_layers"]}}
    transformer = {"num_attention_heads": 2, "attention_head_dim": mk.FE["video_dim"] // 2,
                   "audio_num_attention_heads": 2, "audio_attention_head_dim": mk.FE["audio_dim"] // 2,
                   "connector_num_attention_heads": vconn["heads"], "connector_attention_head_dim": vconn["dim_head"],
                   "audio_connector_attention_head_dim": aconn["dim_head"], "connector_num_layers": vconn["num_layers"],
                   "connector_num_learnable_registers": vconn["registers"],
                   "connector_positional_embedding_max_pos": vconn["max_pos"],
                   "connector_apply_gated_attention": gated, "connector_ff_bias": vconn["ff_bias"]}
    te_path, dit_path = tmp_path / "te.safetensors", tmp_path / "dit.safetensors"
    save_file(files["te"], str(te_path), metadata={"gemma_config": json.dumps(gemma)})
    save_file(files["dit"], str(dit_path), metadata={"config": json.dumps({"transformer": transformer})})
    proc = ltx_te.build_embeddings_processor(str(te_path), str(dit_path))
    got = dict(proc.named_parameters())
    assert set(got) == {n for n, _ in src.named_parameters()}
    for n, p in src.named_parameters():
        assert got[n].device.type == "cuda" and got[n].dtype == torch.bfloat16
        assert torch.equal(got[n], p), n
    mask = torch.from_numpy(G["mask"]).to(DEV)
    with torch.no_grad():
        want = src.process_hidden_states(_layers(), mask)
        have = proc.process_hidden_states(_layers(), mask)
    assert all(torch.equal(a, b) for a, b in zip(have, want))
