"""Writes RoPE golden vectors with the reference's own functions.

The table layout of precompute_freqs_cis (axis-fastest interleave, identity
padding in front, per-head split) and video_positions / audio_positions are
not fixed by any closed form or library routine, so their input/output pairs
come from the reference itself: standalone/ltx_nn.py:34-115 and
standalone/ltx_dit.py:442-465, imported from /root/reference in this
container (CPU).  Output: rope_golden.npz (bf16 as uint16 bit patterns).

Run from the repository root: python tests/golden/make_rope_golden.py
"""
import pathlib
import sys

import numpy as np
import torch

REF = pathlib.Path("/root/reference/standalone")
OUT = pathlib.Path(__file__).resolve().parent / "rope_golden.npz"


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main() -> None:
    sys.dont_write_bytecode = True  # the reference tree is read-only: no __pycache__ there
    sys.path.insert(0, str(REF))
    import ltx_nn  # noqa: E402  (reference module)
    import ltx_dit  # noqa: E402  (reference module)

    cpu = torch.device("cpu")
    g = torch.Generator().manual_seed(1234)
    data = {}
    cases = {
        # name: (positions, dim, heads, max_pos)
        "video": (ltx_dit.video_positions(1, 2, 3, 4, 24.0, cpu), 4096, 32, [20, 2048, 2048]),
        "video_small": (ltx_dit.video_positions(2, 3, 2, 2, 25.0, cpu), 256, 2, [20, 2048, 2048]),
        "audio": (ltx_dit.audio_positions(1, 10, cpu), 2048, 32, [20]),
        "cross": (ltx_dit.video_positions(1, 2, 2, 2, 24.0, cpu)[:, 0:1], 2048, 32, [20]),
    }
    for name, (pos, dim, heads, max_pos) in cases.items():
        cos, sin = ltx_nn.precompute_freqs_cis(pos, dim=dim, out_dtype=torch.bfloat16, theta=10000.0,
                                               max_pos=max_pos, use_middle_indices_grid=True,
                                               num_attention_heads=heads, double_precision=True)
        b, t = pos.shape[0], pos.shape[2]
        x = torch.randn(b, t, dim, generator=g).to(torch.bfloat16)
        y = ltx_nn.apply_split_rotary_emb(x, (cos, sin))
        data[f"{name}_positions"] = pos.float().numpy()
        data[f"{name}_meta"] = np.array([dim, heads] + list(max_pos), dtype=np.float64)
        data[f"{name}_cos"] = bits(cos)
        data[f"{name}_sin"] = bits(sin)
        data[f"{name}_x"] = bits(x)
        data[f"{name}_rot"] = bits(y)
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes): {sorted(data)}")


if __name__ == "__main__":
    main()
