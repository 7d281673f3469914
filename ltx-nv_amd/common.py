"""Shared helpers of the LTX-2.5 DiT path (module API of the reference's
standalone/common.py that the DiT path uses).

gelu_tanh and rms_norm run on the ltxk HIP kernels; the safetensors helpers
and the sinusoidal timestep embedding are host/torch code as in the reference.
"""

import json
import math

import torch

import ltxk

DEVICE = torch.device("cuda")
DTYPE = torch.bfloat16


def read_metadata(path: str) -> dict:
    """JSON-decoded safetensors metadata (reference standalone/common.py:28-37)."""
    from safetensors import safe_open

    with safe_open(path, framework="pt") as f:
        meta = f.metadata() or {}
    out = {}
    for k, v in meta.items():
        try:
            out[k] = json.loads(v)
        except (json.JSONDecodeError, TypeError):
            out[k] = v
    return out


def load_state_dict(path: str, *, device: torch.device = DEVICE, dtype: torch.dtype | None = DTYPE, rename=None,
                    keep=None) -> dict:
    """Tensors of a safetensors file with optional key filter/rename and float cast
    (reference standalone/common.py:40-65)."""
    from safetensors import safe_open

    sd = {}
    with safe_open(path, framework="pt", device=str(device)) as f:
        for name in f.keys():  # noqa: SIM118
            if keep is not None and not keep(name):
                continue
            new = name if rename is None else rename(name)
            if new is None:
                continue
            t = f.get_tensor(name)
            if dtype is not None and t.is_floating_point():
                t = t.to(dtype)
            sd[new] = t
    return sd


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """GELU with the tanh approximation (reference common.py:130-131) on ltxk."""
    return ltxk.gelu_tanh(x.contiguous())


def rms_norm(x: torch.Tensor, eps: float = 1e-6, weight: torch.Tensor | None = None) -> torch.Tensor:
    """RMSNorm over the last dim (reference common.py:134-135) on ltxk."""
    return ltxk.rms_norm(x.contiguous(), weight, eps)


def get_timestep_embedding(timesteps: torch.Tensor, dim: int, max_period: int = 10000) -> torch.Tensor:
    """Sinusoidal [cos, sin] embedding (flip_sin_to_cos=True, shift 0), reference common.py:138-148."""
    half = dim // 2
    freqs = torch.exp(-math.log(max_period) * torch.arange(0, half, dtype=torch.float32,
                                                            device=timesteps.device) / half)
    args = timesteps[:, None].float() * freqs[None, :]
    emb = torch.cat([torch.cos(args), torch.sin(args)], dim=-1)
    if dim % 2:
        emb = torch.nn.functional.pad(emb, (0, 1))
    return emb
