"""Counter-based Gaussian noise with torch's Philox layout, on ltxk_philox_normal.

TorchRNG keeps the interface of the reference's native generator
(cuda_c_standalone/common/philox.h:6-18): a seed, a per-thread offset counted
in 32-bit draws, manual_seed(), randn_bf16(out) and randn_fp32(out); each
draw advances the offset by 4*ceil(n/(4T)) (philox.cu:47-61).

T, the thread count of torch's grid-stride launch, depends on the device the
stream was drawn on (philox.cu:6-17).  By default it follows this device's
properties, as torch.randn does here: the same Philox words reach the same
elements and the generator offsets advance alike.  The values are not
identical to torch-ROCm's: it evaluates Box-Muller with rocRAND's
single-precision device log/sin/cos (measured on the MI355X: up to 1.7e-6 from
the exact formula, 0.02 % of bf16 values one bf16 ulp apart), while
ltxk_philox_normal stays within 1 fp32 ulp of it.  Pass multiprocessors /
max_threads_per_mp to reproduce another device's stream (the reference's
golden noise came from an RTX 6000 Ada: 142 SMs x 1536 threads).
"""

from __future__ import annotations

import torch

import ltxk

# RTX 6000 Ada (SM 8.9), the device the reference's golden noise was drawn on.
ADA_RTX6000 = (142, 1536)


class TorchRNG:
    def __init__(self, seed: int = 0, device: torch.device | str | int | None = None,
                 multiprocessors: int | None = None, max_threads_per_mp: int | None = None):
        self.device = torch.device(device if device is not None else "cuda")
        if self.device.type != "cuda":
            raise RuntimeError("TorchRNG draws on the ROCm device only")
        if (multiprocessors is None) != (max_threads_per_mp is None):
            raise ValueError("give both multiprocessors and max_threads_per_mp, or neither")
        self.multiprocessors = multiprocessors
        self.max_threads_per_mp = max_threads_per_mp
        self.seed = 0
        self.offset = 0
        self.manual_seed(seed)

    def manual_seed(self, seed: int) -> "TorchRNG":
        self.seed = int(seed) & (2**64 - 1)
        self.offset = 0
        return self

    def total_threads(self, n: int) -> int:
        if self.multiprocessors is None:
            return ltxk.device_policy_threads(n, self.device)
        return ltxk.policy_threads(n, self.multiprocessors, self.max_threads_per_mp)

    def fill_(self, out: torch.Tensor) -> torch.Tensor:
        """normal(0, 1) into `out` (fp32 or bf16, contiguous); advances the offset."""
        n = out.numel()
        if n == 0:
            return out
        adv = ltxk.philox_normal(out, self.seed, self.offset, self.total_threads(n))
        self.offset += adv
        return out

    def randn_bf16(self, out: torch.Tensor) -> torch.Tensor:
        if out.dtype != torch.bfloat16:
            raise ValueError("randn_bf16 needs a bf16 tensor")
        return self.fill_(out)

    def randn_fp32(self, out: torch.Tensor) -> torch.Tensor:
        if out.dtype != torch.float32:
            raise ValueError("randn_fp32 needs an fp32 tensor")
        return self.fill_(out)

    def randn(self, *shape: int, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """torch.randn(*shape, dtype, generator) equivalent on this generator."""
        out = torch.empty(shape, device=self.device, dtype=dtype)
        return self.fill_(out)
