"""CPU oracle for the LTX-2.5 DiT memory-bound path.

TEST INFRASTRUCTURE ONLY.  tests/, the smoke check and bench.py's CPU-baseline
leg import this module to check and time the HIP kernels; the product package
(ltx-nv_amd/) never imports it and has no CPU fallback.

Integer work (Philox) is plain C in philox_oracle.c (built into
libltx_oracle.so by oracle/Makefile).  Floating-point work is restated here
with fp32 torch-CPU arithmetic on the stored (bf16) inputs, rounding each
output once, which is the "fp32-accumulated" formulation of the reference's
eager bf16 chain.  Each function cites the reference lines it restates.

Pins (tests/test_oracle.py):
  philox_*        Random123 known-answer vectors, rocRAND's host Philox engine
                  (tests/golden/rocrand_philox.json), the reference's bf16
                  golden noise (tests/golden/m1_philox/).
  box-muller      golden noise (bf16), moments, fp64 closed form.
  rms_norm        torch.nn.functional.rms_norm (library routine).
  layer_norm_mod  torch.nn.functional.layer_norm (library routine).
  gelu_tanh       torch.nn.functional.gelu(approximate="tanh") and erf-GELU.
  modulate/residual/head_gate/euler/x0
                  special cases that reduce to library ops (scale=-1, gate=0,
                  logit=0, dt=0, ...) and linearity checks.
  feature_norm    F.rms_norm per layer (library routine), the interleave checked
                  element by element on a tiny case, masked rows exactly +0.
  guide           neutral scales, single-term offsets that fix each term's
                  sign and weight, rescale cases with an exact std ratio (1/2),
                  std(out) = std(cond) at r = 1, linearity in r.
  rope tables     vectors written by the reference's own precompute_freqs_cis
                  (tests/golden/rope_*.npz), plus rotation invariants.
  freq_grid fp32  (no reference vectors) the fp64 closed form within 16 ulp,
                  the exact first entry pi/2, the count, monotonicity, and a
                  different rounding path from the fp64 grid.
  model_eager     outputs of the reference's own LTXModel on a small config
                  (tests/golden/block_golden.npz) to 1e-6.
"""

from __future__ import annotations

import ctypes
import math
import pathlib

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "libltx_oracle.so"

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing; run `make -C oracle`")
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i64, u64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64
        L.oracle_philox4x32_10.argtypes = [vp, vp, vp]
        L.oracle_offset_advance.argtypes = [i64, i64]
        L.oracle_offset_advance.restype = i64
        L.oracle_policy_threads.argtypes = [i64, i64, i64]
        L.oracle_policy_threads.restype = i64
        L.oracle_philox_u32.argtypes = [vp, i64, i64, u64, u64, i64]
        L.oracle_philox_normal.argtypes = [vp, i64, i64, u64, u64, i64]
        L.oracle_philox_normal_full.argtypes = [vp, i64, u64, u64, i64]
        L.oracle_box_muller_uv.argtypes = [ctypes.c_uint32, ctypes.c_uint32, vp, vp]
        L.oracle_f32_to_bf16.argtypes = [vp, vp, i64]
        L.oracle_euler_update_f32.argtypes = [vp, vp, i64, ctypes.c_float]
        _lib = L
    return _lib


# ---------------------------------------------------------------------------
# bf16 helpers
# ---------------------------------------------------------------------------


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16(a.ctypes.data, out.ctypes.data, a.size)
    return out


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def rnd(x: torch.Tensor) -> torch.Tensor:
    """Round fp32 to bf16 (RNE) and return the bf16 tensor."""
    return x.to(torch.bfloat16)


def f32(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.float32)


# ---------------------------------------------------------------------------
# Philox noise (cuda_c_standalone/common/philox.cu:6-61)
# ---------------------------------------------------------------------------


def philox_block(ctr, key) -> list[int]:
    c = (ctypes.c_uint32 * 4)(*ctr)
    k = (ctypes.c_uint32 * 2)(*key)
    o = (ctypes.c_uint32 * 4)()
    lib().oracle_philox4x32_10(c, k, o)
    return list(o)


def policy_threads(n: int, multiprocessors: int, max_threads_per_mp: int) -> int:
    """philox.cu:6-17 (calc_policy): 256*min(ceil(n/256), SMs*floor(maxThreads/256))."""
    return lib().oracle_policy_threads(n, multiprocessors, max_threads_per_mp)


def offset_advance(n: int, total_threads: int) -> int:
    """philox.cu:16,47-61: 4*ceil(n/(4T))."""
    return lib().oracle_offset_advance(n, total_threads)


def philox_u32(n: int, seed: int, offset: int, total_threads: int, first: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    lib().oracle_philox_u32(out.ctypes.data, first, n, seed, offset, total_threads)
    return out


def philox_normal(n: int, seed: int, offset: int, total_threads: int) -> np.ndarray:
    """fp32 N(0,1) of the whole tensor (philox.cu:19-35 + Box-Muller)."""
    out = np.empty(n, dtype=np.float32)
    lib().oracle_philox_normal_full(out.ctypes.data, n, seed, offset, total_threads)
    return out


def philox_normal_at(idx: np.ndarray, seed: int, offset: int, total_threads: int) -> np.ndarray:
    """fp32 values at selected element indices (for sampled checks of big tensors)."""
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    out = np.empty(idx.size, dtype=np.float32)
    one = np.empty(1, dtype=np.float32)
    L = lib()
    for i, e in enumerate(idx):
        L.oracle_philox_normal(one.ctypes.data, int(e), 1, seed, offset, total_threads)
        out[i] = one[0]
    return out


def box_muller_uv(x: int, y: int) -> tuple[float, float]:
    u = ctypes.c_float()
    v = ctypes.c_float()
    lib().oracle_box_muller_uv(x, y, ctypes.byref(u), ctypes.byref(v))
    return u.value, v.value


def euler_update_f32(x: np.ndarray, v: np.ndarray, dt: float) -> np.ndarray:
    """x + v*dt in fp32, product rounded before the add (ltx_dit.py:606 op order)."""
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    v = np.ascontiguousarray(v, dtype=np.float32)
    lib().oracle_euler_update_f32(x.ctypes.data, v.ctypes.data, x.size, dt)
    return x


# ---------------------------------------------------------------------------
# AdaLN values (ltx_dit.py:192-206)
# ---------------------------------------------------------------------------


def ada_value(table: torch.Tensor, row: int, emb: torch.Tensor | None, batch: int, tokens: int) -> torch.Tensor:
    """get_ada_values row: table[row] + emb.reshape(B, T_e, n, D)[:, :, row], bf16 add.
    Returns a (B or 1, T_e, D) bf16 tensor that broadcasts over (B, T, D)."""
    d = table.shape[-1]
    tab = table[row].to(torch.bfloat16).reshape(1, 1, d)
    if emb is None:
        return tab
    n = emb.shape[-1] // d
    e = emb.reshape(emb.shape[0], emb.shape[1], n, d)[:, :, row]
    return rnd(f32(tab) + f32(e))


# ---------------------------------------------------------------------------
# Norms / modulation (ltx_nn.py:18-19, ltx_dit.py:245-246,261,265-267,311,371-378)
# ---------------------------------------------------------------------------


def _rms(x32: torch.Tensor, eps: float) -> torch.Tensor:
    return x32 * torch.rsqrt((x32 * x32).mean(dim=-1, keepdim=True) + eps)


def rms_norm(x: torch.Tensor, weight: torch.Tensor | None = None, eps: float = 1e-6) -> torch.Tensor:
    """ltx_nn.py:18-19: F.rms_norm(x, weight, eps) = x*rsqrt(mean(x^2)+eps)*w, fp32, one rounding."""
    y = _rms(f32(x), eps)
    if weight is not None:
        y = y * f32(weight)
    return rnd(y)


def norm_modulate(x, shift=None, scale=None, eps=1e-6, layer=False) -> torch.Tensor:
    """rms_norm(x)*(1+scale)+shift (ltx_dit.py:261); layer=True: LayerNorm(no affine)
    then the same modulation (ltx_dit.py:371-378).  shift/scale are bf16 tensors
    broadcasting over x (None = 0)."""
    x32 = f32(x)
    if layer:
        mu = x32.mean(dim=-1, keepdim=True)
        c = x32 - mu
        n = c * torch.rsqrt((c * c).mean(dim=-1, keepdim=True) + eps)
    else:
        n = _rms(x32, eps)
    sc = f32(scale) if scale is not None else 0.0
    sh = f32(shift) if shift is not None else 0.0
    return rnd(n * (1.0 + sc) + sh)


def modulate(x, shift=None, scale=None) -> torch.Tensor:
    """ltx_dit.py:246: context*(1+scale_kv)+shift_kv."""
    sc = f32(scale) if scale is not None else 0.0
    sh = f32(shift) if shift is not None else 0.0
    return rnd(f32(x) * (1.0 + sc) + sh)


def gated_residual(x, f, gate=None, mask=None) -> torch.Tensor:
    """ltx_dit.py:265,311 (x + f*gate) and 295-296,306-307 (x + f*gate*mask)."""
    g = f32(gate) if gate is not None else 1.0
    m = f32(mask).reshape(-1, 1, 1) if mask is not None else 1.0
    return rnd(f32(x) + (f32(f) * g) * m)


def add_norm_modulate(x, f, gate=None, mask=None, shift=None, scale=None, eps=1e-6):
    """ltx_dit.py:265-266 + 245: x' = x + f*gate (rounded); y = rms(x')*(1+scale)+shift."""
    xo = gated_residual(x, f, gate, mask)
    return xo, norm_modulate(xo, shift, scale, eps)


def head_gate(out, logits, heads) -> torch.Tensor:
    """ltx_nn.py:231-235: out.view(b,t,h,dh) * 2*sigmoid(logits)."""
    b, t, d = out.shape
    o = f32(out).view(b, t, heads, d // heads) * (2.0 * torch.sigmoid(f32(logits))).unsqueeze(-1)
    return rnd(o.view(b, t, d))


def gelu_tanh(x) -> torch.Tensor:
    """ltx_nn.py:248 / common.py:130-131: 0.5x(1+tanh(sqrt(2/pi)(x+0.044715x^3)))."""
    x32 = f32(x)
    inner = math.sqrt(2.0 / math.pi) * (x32 + 0.044715 * x32 * x32 * x32)
    return rnd(0.5 * x32 * (1.0 + torch.tanh(inner)))


def euler_step(sample, denoised, sigma: float, dt: float) -> torch.Tensor:
    """ltx_dit.py:602-606: vel = ((x - x0)/sigma).to(dtype); (x + vel*dt).to(dtype)."""
    s32 = f32(sample)
    vel = ((s32 - f32(denoised)) / torch.tensor(sigma, dtype=torch.float32)).to(sample.dtype)
    return (s32 + f32(vel) * torch.tensor(dt, dtype=torch.float32)).to(sample.dtype)


def x0(latent, velocity, timesteps) -> torch.Tensor:
    """ltx_dit.py:592-593: (latent - v*timesteps) in fp32, cast back."""
    return (f32(latent) - f32(velocity) * f32(timesteps)).to(latent.dtype)


def guide(cond, uncond, ptb, mod, cfg_scale: float, stg_scale: float, modality_scale: float,
          rescale_scale: float) -> torch.Tensor:
    """ltx_dit.py:551-562: CFG + STG + modality guidance in fp32, std rescale, cast back.

    Python scalars meet the fp32 tensors as fp32 values (torch's scalar rule),
    the terms are added left to right, and torch.std is the unbiased standard
    deviation over all elements (evaluated here in fp64, then as fp32)."""
    c = f32(cond)
    pred = c + (cfg_scale - 1) * (c - f32(uncond)) + stg_scale * (c - f32(ptb)) \
        + (modality_scale - 1) * (c - f32(mod))
    if rescale_scale != 0:
        factor = c.double().std().float() / pred.double().std().float()
        factor = rescale_scale * factor + (1 - rescale_scale)
        pred = pred * factor
    return pred.to(cond.dtype)


def guided_step(latent, velocity, timesteps, cfg_scale, stg_scale, modality_scale, rescale_scale,
                sigma: float | None = None, dt: float | None = None):
    """x0 of the 4 passes (ltx_dit.py:592-598), guide (:551-562), euler_step (:602-606).

    latent (B, T, C); velocity (4B, T, C) passes cond|uncond|ptb|mod along the
    batch; timesteps (4B, T or 1, 1).  Returns (denoised, next or None, x0)."""
    n = 4
    lat = latent.repeat(n, 1, 1)
    x0s = x0(lat, velocity, timesteps)
    parts = x0s.chunk(n)
    den = guide(*parts, cfg_scale, stg_scale, modality_scale, rescale_scale)
    nxt = euler_step(latent, den, sigma, dt) if sigma is not None else None
    return den, nxt, x0s


def feature_norm(layers, keep, scale0: float, scale1: float, eps: float = 1e-6):
    """ltx_te.py:167-184 up to the projections: per-layer RMS over the hidden dim
    (fp32 statistics, the normalised value materialised in bf16 as the reference
    does), layers stacked on a new last axis and flattened, masked tokens +0,
    then each projection input scaled (fp32 product, one rounding)."""
    normed = torch.stack([rnd(_rms(f32(x), eps)) for x in layers], dim=-1)
    b, t, d, n = normed.shape
    flat = f32(normed.reshape(b, t, d * n))
    k = torch.ones(b, t, 1) if keep is None else (keep != 0).reshape(b, t, 1).float()
    out = []
    for s in (scale0, scale1):
        out.append(rnd(torch.where(k > 0, flat * s, torch.zeros_like(flat))))
    return out[0], out[1]


# ---------------------------------------------------------------------------
# RoPE (LTXRopeType.SPLIT), ltx_nn.py:34-115
# ---------------------------------------------------------------------------


def freq_grid(theta: float, n_axes: int, inner_dim: int, double_precision: bool = True) -> torch.Tensor:
    """theta**linspace(0, 1, inner_dim//(2 n_axes)) * pi/2 as fp32.

    double_precision: powers in fp64, cast once (ltx_nn.py:34-46); otherwise
    the exponents and powers are fp32 (torch on the CPU) and the pi/2 product
    rounds in fp32 as well (ltx_nn.py:49-60, the `frequencies_precision` !=
    "float64" checkpoints of ltx_dit.py:68).
    """
    n = inner_dim // (2 * n_axes)
    if not double_precision:
        e = torch.linspace(math.log(1.0, theta), math.log(theta, theta), n, dtype=torch.float32)
        return (theta ** e).to(torch.float32) * math.pi / 2
    lo = np.log(1.0) / np.log(theta)
    hi = np.log(theta) / np.log(theta)
    p = np.power(theta, np.linspace(lo, hi, n, dtype=np.float64))
    return torch.as_tensor(p * math.pi / 2, dtype=torch.float32)


def rope_tables(positions: torch.Tensor, dim: int, heads: int, max_pos, theta: float = 10000.0,
                out_dtype=torch.bfloat16, double_precision: bool = True):
    """ltx_nn.py:63-96 with use_middle_indices_grid (grid precision as freq_grid).

    positions (B, n_axes, T, 2) fp32 [start, end) bounds.  Returns (cos, sin)
    (B, heads, T, dim/(2 heads)).  Frequency index p = f*n_axes + a (axis
    fastest), identity entries (cos 1, sin 0) padded in front.
    """
    b, n_axes, t, _ = positions.shape
    ind = freq_grid(theta, n_axes, dim, double_precision)     # (F,)
    mid = (positions[..., 0] + positions[..., 1]) / 2.0       # (B, A, T) fp32
    frac = torch.stack([mid[:, a] / max_pos[a] for a in range(n_axes)], dim=-1)  # (B, T, A)
    ang = ind.view(1, 1, 1, -1) * (frac.unsqueeze(-1) * 2 - 1)  # (B, T, A, F)
    ang = ang.transpose(-1, -2).reshape(b, t, -1)              # (B, T, F*A), axis fastest
    pad = dim // 2 - ang.shape[-1]
    c, s = torch.cos(ang), torch.sin(ang)
    if pad:
        c = torch.cat([torch.ones(b, t, pad), c], dim=-1)
        s = torch.cat([torch.zeros(b, t, pad), s], dim=-1)
    c = c.reshape(b, t, heads, -1).transpose(1, 2)
    s = s.reshape(b, t, heads, -1).transpose(1, 2)
    return c.to(out_dtype).contiguous(), s.to(out_dtype).contiguous()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """ltx_nn.py:99-115 on token-major x (B, T, H*Dh): per head halves (x1, x2) ->
    (x1 c - x2 s, x2 c + x1 s) in fp32, one rounding."""
    b, t, d = x.shape
    h = cos.shape[1]
    dh = d // h
    xr = f32(x).view(b, t, h, 2, dh // 2)
    x1, x2 = xr[..., 0, :], xr[..., 1, :]
    c = f32(cos).transpose(1, 2)  # (B, T, H, Dh/2)
    s = f32(sin).transpose(1, 2)
    o1 = x1 * c - x2 * s
    o2 = x2 * c + x1 * s
    return rnd(torch.stack([o1, o2], dim=3).reshape(b, t, d))


def qk_norm_rope(x, weight, cos, sin, eps=1e-6) -> torch.Tensor:
    """ltx_nn.py:214-218 fused: rope(rms_norm(x)*weight) in fp32, one rounding."""
    y = f32(x)
    if weight is not None:
        y = _rms(y, eps) * f32(weight)
    if cos is None:
        return rnd(y)
    b, t, d = x.shape
    h = cos.shape[1]
    dh = d // h
    yr = y.view(b, t, h, 2, dh // 2)
    x1, x2 = yr[..., 0, :], yr[..., 1, :]
    c = f32(cos).transpose(1, 2)
    s = f32(sin).transpose(1, 2)
    return rnd(torch.stack([x1 * c - x2 * s, x2 * c + x1 * s], dim=3).reshape(b, t, d))


# ---------------------------------------------------------------------------
# Positions (ltx_dit.py:439-465)
# ---------------------------------------------------------------------------


def video_positions(batch: int, f: int, h: int, w: int, fps: float) -> torch.Tensor:
    """(B, 3, T, 2) [start, end) bounds: time (8t-7 clamped at 0, 8t+1)/fps, h/w x32."""
    ft, hh, ww = torch.meshgrid(torch.arange(f), torch.arange(h), torch.arange(w), indexing="ij")
    starts = torch.stack([ft, hh, ww]).reshape(3, -1).float()
    scale = torch.tensor([8.0, 32.0, 32.0]).view(3, 1)
    s = starts * scale
    e = (starts + 1) * scale
    s[0] = (s[0] + 1 - 8).clamp(min=0) / fps
    e[0] = (e[0] + 1 - 8).clamp(min=0) / fps
    return torch.stack([s, e], dim=-1).unsqueeze(0).expand(batch, -1, -1, -1).contiguous()


def audio_positions(batch: int, frames: int) -> torch.Tensor:
    """(B, 1, T, 2) mel-frame bounds in seconds: [max(0, 4i-3), max(0, 4i+1)] * 160/16000."""
    i = torch.arange(frames, dtype=torch.float32)
    s = (i * 4 + 1 - 4).clamp(min=0) * 160 / 16000
    e = ((i + 1) * 4 + 1 - 4).clamp(min=0) * 160 / 16000
    return torch.stack([s, e], dim=-1)[None, None].expand(batch, 1, -1, -1).contiguous()
