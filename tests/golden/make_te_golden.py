"""Writes golden vectors of the text-encoder connector path with the reference's
own modules (standalone/ltx_te.py: FeatureExtractorV2, Embeddings1DConnector,
EmbeddingsProcessor.process_hidden_states), imported from /root/reference in
the build container and run on the CPU.

Nothing but the reference pins the connector's op order (register mixing,
token reordering, residual/norm placement, output masking), so a small
configuration of the same structure is run in fp32 and in bf16 and its inputs
and outputs are stored in te_golden.npz.  Weights are not stored: every
parameter, in sorted-name order, is randn(shape) * 0.02 from one CPU generator
seeded WEIGHT_SEED, rounded to bf16 (init_weights below; the tests rebuild them
the same way).

Run from the repository root: python tests/golden/make_te_golden.py
"""
import pathlib
import sys

import numpy as np
import torch

REF = pathlib.Path("/root/reference/standalone")
OUT = pathlib.Path(__file__).resolve().parent / "te_golden.npz"
WEIGHT_SEED = 77
# gemma hidden 64 with 3+1 layers; video connector 2 heads x 64, audio 2 x 32; 2 blocks; 4 registers
FE = dict(gemma_hidden=64, num_layers=3, video_dim=128, audio_dim=64)
VCONN = dict(heads=2, dim_head=64, num_layers=2, max_pos=[4096], registers=4, gated=True, ff_bias=True)
ACONN = dict(heads=2, dim_head=32, num_layers=2, max_pos=[4096], registers=4, gated=False, ff_bias=True)
BATCH, TOKENS, PADS = 2, 16, (5, 0)   # left padding per batch item, as the reference's tokenizer pads


def build(mod):
    fe = mod.FeatureExtractorV2(**FE)
    return mod.EmbeddingsProcessor(fe, mod.Embeddings1DConnector(**VCONN), mod.Embeddings1DConnector(**ACONN))


def init_weights(model: torch.nn.Module) -> None:
    g = torch.Generator().manual_seed(WEIGHT_SEED)
    params = dict(model.named_parameters())
    with torch.no_grad():
        for name in sorted(params):
            p = params[name]
            scale = 1.0 if name.endswith("learnable_registers") else 0.02
            p.copy_((torch.randn(p.shape, generator=g) * scale).to(torch.bfloat16).to(p.dtype))


def make_inputs(seed: int = 5):
    g = torch.Generator().manual_seed(seed)
    layers = [(torch.randn(BATCH, TOKENS, FE["gemma_hidden"], generator=g) * (1.0 + i)).to(torch.bfloat16)
              for i in range(FE["num_layers"] + 1)]
    mask = torch.ones(BATCH, TOKENS, dtype=torch.int64)
    for b, p in enumerate(PADS):
        mask[b, :p] = 0
    return layers, mask


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main() -> None:
    sys.dont_write_bytecode = True  # the reference tree is read-only: no __pycache__ there
    sys.path.insert(0, str(REF))
    import ltx_te  # noqa: E402  (reference module)

    proc = build(ltx_te)
    init_weights(proc)
    layers, mask = make_inputs()
    data = {"param_names": np.array(sorted(n for n, _ in proc.named_parameters())), "mask": mask.numpy()}
    for i, x in enumerate(layers):
        data[f"layer{i}"] = bits(x)
    for dtype, tag in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
        m = proc.to(dtype)
        with torch.no_grad():
            feats = m.feature_extractor(tuple(x.to(dtype) for x in layers), mask)
            venc, aenc, vbin = m.process_hidden_states(tuple(x.to(dtype) for x in layers), mask)
        data[f"vfeat_{tag}"] = feats[0].float().numpy()
        data[f"afeat_{tag}"] = feats[1].float().numpy()
        data[f"venc_{tag}"] = venc.float().numpy()
        data[f"aenc_{tag}"] = aenc.float().numpy()
        data[f"vbin_{tag}"] = vbin.numpy()
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
