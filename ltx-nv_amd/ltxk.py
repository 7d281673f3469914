"""ctypes binding of libltxk.so (the gfx950 HIP kernels declared in include/ltxk.h).

Every function takes torch tensors that live on a ROCm device, enqueues one
kernel on the current HIP stream of that device and returns without a host
synchronisation.  There is no CPU fallback: a missing library, a CPU tensor,
a wrong dtype or a non-contiguous operand raises RuntimeError/ValueError.
"""

from __future__ import annotations

import ctypes
import pathlib
import sys
import threading

import torch

LIB_PATH = pathlib.Path(__file__).resolve().with_name("libltxk.so")

# LTXK_VERSION of include/ltxk.h: the layout of the structs below
ABI_VERSION = 200

E_ARG, E_ALIGN, E_DTYPE, E_HIP = 1, 2, 3, 4
DTYPE_F32, DTYPE_BF16 = 0, 1
NORM_RMS, NORM_LAYER = 0, 1

_c_i64 = ctypes.c_int64
_c_u64 = ctypes.c_uint64
_c_int = ctypes.c_int
_c_float = ctypes.c_float
_c_vp = ctypes.c_void_p


class Ada(ctypes.Structure):
    """ltxk_ada: one AdaLN vector = round(tab[d] + emb[b*bs + t*ts + d]), or with
    an index round(tab[d] + emb[index[row]*ts + d])."""

    _fields_ = [("tab", _c_vp), ("emb", _c_vp), ("emb_bstride", _c_i64), ("emb_tstride", _c_i64),
                ("emb_index", _c_vp), ("emb_rows", _c_i64)]


class QK(ctypes.Structure):
    """ltxk_qk: one q or k operand of ltxk_qk_norm_rope."""

    _fields_ = [
        ("x", _c_vp),
        ("weight", _c_vp),
        ("cos", _c_vp),
        ("sin", _c_vp),
        ("batch", _c_i64),
        ("tokens", _c_i64),
        ("table_bstride", _c_i64),
        ("pos_index", _c_vp),
        ("n_axes", _c_i64),
        ("table_rows", _c_i64),
    ]


class Guidance(ctypes.Structure):
    """ltxk_guidance: GuiderParams' scales (cfg, stg, modality, rescale)."""

    _fields_ = [("cfg_scale", ctypes.c_double), ("stg_scale", ctypes.c_double),
                ("modality_scale", ctypes.c_double), ("rescale_scale", ctypes.c_double)]


_ADA_P = ctypes.POINTER(Ada)
_QK_P = ctypes.POINTER(QK)
_GUIDE_P = ctypes.POINTER(Guidance)

# name -> (restype, argtypes); the complete exported surface of include/ltxk.h
SIGNATURES = {
    "ltxk_version": (_c_int, []),
    "ltxk_last_error": (ctypes.c_char_p, []),
    "ltxk_philox_policy_threads": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "ltxk_philox_offset_advance": (_c_i64, [_c_i64, _c_i64]),
    "ltxk_philox_normal": (_c_int, [_c_vp, _c_int, _c_i64, _c_u64, _c_u64, _c_i64, _c_vp]),
    "ltxk_philox_u32": (_c_int, [_c_vp, _c_i64, _c_u64, _c_u64, _c_i64, _c_vp]),
    "ltxk_euler_update": (_c_int, [_c_vp, _c_vp, _c_i64, _c_int, _c_float, _c_vp]),
    "ltxk_euler_step": (_c_int, [_c_vp, _c_vp, _c_vp, _c_i64, _c_int, _c_float, _c_float, _c_vp]),
    "ltxk_x0": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]),
    "ltxk_feature_norm": (
        _c_int, [_c_vp, _c_vp, ctypes.POINTER(_c_vp), _c_i64, _c_vp, _c_i64, _c_i64, _c_float, _c_float, _c_float,
                 _c_vp],
    ),
    "ltxk_guide_workspace_bytes": (_c_i64, [_c_i64]),
    "ltxk_guide": (
        _c_int,
        [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _GUIDE_P, _c_float, _c_float,
         _c_vp, _c_i64, _c_vp],
    ),
    "ltxk_guide_noalloc": (
        _c_int,
        [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _GUIDE_P, _c_float, _c_float,
         _c_vp],
    ),
    "ltxk_rms_norm": (_c_int, [_c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_float, _c_vp]),
    "ltxk_norm_modulate": (
        _c_int,
        [_c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_float, _ADA_P, _ADA_P, _ADA_P, _ADA_P, _c_vp],
    ),
    "ltxk_add_norm_modulate": (
        _c_int,
        [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _ADA_P, _c_vp, _c_i64, _c_i64, _c_i64, _c_float, _ADA_P, _ADA_P,
         _ADA_P, _ADA_P, _c_vp],
    ),
    "ltxk_modulate": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _ADA_P, _ADA_P, _c_vp]),
    "ltxk_modulate_layers": (
        _c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _ADA_P, _ADA_P, _c_i64, _c_i64, _c_vp],
    ),
    "ltxk_qk_norm_rope": (_c_int, [_QK_P, _QK_P, _c_i64, _c_i64, _c_float, _c_vp]),
    "ltxk_gelu_tanh": (_c_int, [_c_vp, _c_vp, _c_i64, _c_vp]),
    "ltxk_gated_residual": (_c_int, [_c_vp, _c_vp, _c_vp, _ADA_P, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp]),
    "ltxk_head_gate": (
        _c_int,
        [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp],
    ),
    "ltxk_attn_combine": (
        _c_int,
        [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_vp],
    ),
}

_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Loads libltxk.so once (after torch, so it binds to torch's HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python ltx-nv_amd/build_lib.py` "
                    "(the ltxk kernels have no fallback)"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            built = lib.ltxk_version()
            if built != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH} has ABI version {built}, this binding's structs are version "
                                   f"{ABI_VERSION}; rebuild the library")
            _lib = lib
    return _lib


def last_error() -> str:
    return load().ltxk_last_error().decode()


# ---------------------------------------------------------------------------
# Ordering between HIP streams
# ---------------------------------------------------------------------------

_EVENT_FLAGS = 0x2 | 0x20000000  # hipEventDisableTiming | hipEventDisableSystemFence
_hip = None


def _hip_runtime() -> ctypes.CDLL:
    """The HIP runtime libltxk.so is bound to (torch's), for its event calls."""
    global _hip
    if _hip is None:
        lib = load()
        lib.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(_c_vp), ctypes.c_uint]
        lib.hipEventRecord.argtypes = [_c_vp, _c_vp]
        lib.hipStreamWaitEvent.argtypes = [_c_vp, _c_vp, ctypes.c_uint]
        lib.hipEventDestroy.argtypes = [_c_vp]
        for name in ("hipEventCreateWithFlags", "hipEventRecord", "hipStreamWaitEvent", "hipEventDestroy"):
            getattr(lib, name).restype = _c_int
        _hip = lib
    return _hip


class StreamEvent:
    """Orders one HIP stream's later work after another stream's earlier work
    on the same GPU (record on the producer, wait on the consumer), like
    torch.cuda.Event without timing, and without the system-scope memory fence
    on record and wait: every kernel already releases its writes to the whole
    device when it ends, and nothing on the host or on another device reads
    what these events order.  Created on the current device; its streams must
    be on that device."""

    def __init__(self):
        hip = _hip_runtime()
        handle = _c_vp()
        rc = hip.hipEventCreateWithFlags(ctypes.byref(handle), _EVENT_FLAGS)
        if rc:
            raise RuntimeError(f"hipEventCreateWithFlags failed (hipError {rc})")
        self._hip, self._h = hip, handle

    def record(self, stream: torch.cuda.Stream) -> None:
        rc = self._hip.hipEventRecord(self._h, _c_vp(stream.cuda_stream))
        if rc:
            raise RuntimeError(f"hipEventRecord failed (hipError {rc})")

    def wait(self, stream: torch.cuda.Stream) -> None:
        """`stream`'s work enqueued from now on runs after the recorded work."""
        rc = self._hip.hipStreamWaitEvent(_c_vp(stream.cuda_stream), self._h, 0)
        if rc:
            raise RuntimeError(f"hipStreamWaitEvent failed (hipError {rc})")

    def __del__(self, _finalizing=sys.is_finalizing):
        # at interpreter shutdown the HIP runtime may already be torn down (and
        # this module's globals cleared): the process frees the event
        if _finalizing():
            return
        try:
            self._hip.hipEventDestroy(self._h)
        except Exception:
            pass


def _check_rc(rc: int, what: str) -> None:
    if rc != 0:
        kind = {E_ARG: "bad argument", E_ALIGN: "misaligned buffer", E_DTYPE: "bad dtype", E_HIP: "HIP error"}.get(
            rc, f"error {rc}"
        )
        raise RuntimeError(f"ltxk {what}: {kind}: {last_error()}")


def _dev(t: torch.Tensor, name: str, dtype: torch.dtype | tuple = torch.bfloat16) -> None:
    # the common case in three attribute reads (every kernel call checks several tensors)
    if type(t) is torch.Tensor and t.is_cuda and t.dtype == dtype and t.is_contiguous():
        return
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} is on {t.device}; ltxk kernels run on the ROCm device only")
    dts = dtype if isinstance(dtype, tuple) else (dtype,)
    if t.dtype not in dts:
        raise ValueError(f"{name} has dtype {t.dtype}, expected {' or '.join(map(str, dts))}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _out_like(out: torch.Tensor | None, like: torch.Tensor, name: str = "out") -> torch.Tensor:
    """A fresh tensor like `like`, or the caller's `out` after checking it matches."""
    if out is None:
        return torch.empty_like(like, memory_format=torch.contiguous_format)
    _dev(out, name, like.dtype)
    if out.shape != like.shape or out.get_device() != like.get_device():
        raise ValueError(f"{name} {tuple(out.shape)} on {out.device} does not match {tuple(like.shape)} on {like.device}")
    return out


# the current stream's handle without building a torch.cuda.Stream object per
# call (the accessor torch's own generated kernels use); the public route otherwise
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return DTYPE_F32
    if t.dtype == torch.bfloat16:
        return DTYPE_BF16
    raise ValueError(f"unsupported dtype {t.dtype}")


# --------------------------------------------------------------------------
# AdaLN operands
# --------------------------------------------------------------------------


class TimestepIndex:
    """Per-token rows of a de-duplicated timestep embedding: the AdaLN MLP ran on
    the U distinct timestep values, and `index` (int32, one entry per token,
    B*T) names each token's row among them.  `index` must lie in [0, rows);
    the kernels clamp it, so a bad entry reads a wrong row, never outside."""

    __slots__ = ("index", "rows")

    def __init__(self, index: torch.Tensor, rows: int):
        _dev(index, "timestep index", torch.int32)
        if rows <= 0:
            raise ValueError("a timestep index needs at least one embedding row")
        self.index = index
        self.rows = int(rows)


class AdaRef:
    """One modulation vector of get_ada_values without materialising it.

    value[b, t, :] = round(table[row] + emb[b, t', emb_row*D:(emb_row+1)*D]),
    where emb is the (B, T_e, n*D) timestep embedding (T_e == 1: the same row
    for every token), t' = t (or 0) and emb_row defaults to row.  table or emb
    may be None.  With `index` (a TimestepIndex) emb is (1, U, n*D), one row
    per distinct timestep, and token (b, t) reads row index[b*T + t].
    """

    __slots__ = ("table", "row", "emb", "emb_row", "dim", "index")

    def __init__(self, table: torch.Tensor | None, row: int, emb: torch.Tensor | None = None,
                 emb_row: int | None = None, dim: int | None = None, index: TimestepIndex | None = None):
        self.table = table
        self.row = row
        self.emb = emb
        self.emb_row = row if emb_row is None else emb_row
        self.dim = dim if dim is not None else (table.shape[-1] if table is not None else emb.shape[-1])
        self.index = index if emb is not None else None

    def struct(self, batch: int, tokens: int) -> Ada:
        d = self.dim
        tab = None
        if self.table is not None:
            _dev(self.table, "ada table")
            if self.table.shape[-1] != d:
                raise ValueError(f"ada table width {self.table.shape[-1]} != {d}")
            if not 0 <= self.row < self.table.numel() // d:
                raise ValueError(f"ada table row {self.row} out of range")
            tab = self.table.data_ptr() + self.row * d * 2
        emb = None
        bs = ts = 0
        idx, n_idx = None, 0
        if self.emb is not None:
            e = self.emb
            _dev(e, "ada timestep embedding")
            if e.ndim != 3:
                raise ValueError(f"timestep embedding must be (B, T, n*D), got {tuple(e.shape)}")
            eb, et, ew = e.shape
            if ew % d or not 0 <= self.emb_row < ew // d:
                raise ValueError(f"timestep embedding width {ew} has no row {self.emb_row} of width {d}")
            emb = e.data_ptr() + self.emb_row * d * 2
            if self.index is not None:
                if eb != 1 or et != self.index.rows:
                    raise ValueError(f"indexed timestep embedding must be (1, {self.index.rows}, n*D), "
                                     f"got {tuple(e.shape)}")
                if self.index.index.numel() != batch * tokens:
                    raise ValueError(f"timestep index has {self.index.index.numel()} entries, activation has "
                                     f"{batch * tokens} rows")
                return Ada(tab, emb, 0, ew, self.index.index.data_ptr(), self.index.rows)
            if et not in (1, tokens):
                raise ValueError(f"timestep embedding has {et} tokens, activation has {tokens}")
            if eb not in (1, batch):
                raise ValueError(f"timestep embedding batch {eb} vs activation batch {batch}")
            bs = et * ew if eb > 1 else 0
            ts = ew if et > 1 else 0
        return Ada(tab, emb, bs, ts, idx, n_idx)


def _ada_arg(a: AdaRef | None, batch: int, tokens: int, dim: int):
    if a is None:
        return None
    if a.dim != dim:
        raise ValueError(f"modulation width {a.dim} != activation width {dim}")
    return ctypes.byref(a.struct(batch, tokens))


def _btd(x: torch.Tensor, name: str) -> tuple[int, int, int]:
    """(batch, tokens, dim) of a token-major activation (B, T, D) or (T, D)."""
    _dev(x, name)
    if x.ndim == 3:
        return x.shape[0], x.shape[1], x.shape[2]
    if x.ndim == 2:
        return 1, x.shape[0], x.shape[1]
    raise ValueError(f"{name} must be (B, T, D) or (T, D), got {tuple(x.shape)}")


# --------------------------------------------------------------------------
# Philox noise
# --------------------------------------------------------------------------


def policy_threads(n: int, multiprocessors: int, max_threads_per_mp: int) -> int:
    return load().ltxk_philox_policy_threads(n, multiprocessors, max_threads_per_mp)


def device_policy_threads(n: int, device: torch.device | int | None = None) -> int:
    """T that torch's grid-stride launch policy picks for n values on `device`."""
    props = torch.cuda.get_device_properties(device if device is not None else torch.cuda.current_device())
    return policy_threads(n, props.multi_processor_count, props.max_threads_per_multi_processor)


def offset_advance(n: int, total_threads: int) -> int:
    return load().ltxk_philox_offset_advance(n, total_threads)


def philox_normal(out: torch.Tensor, seed: int, offset: int, total_threads: int) -> int:
    """Fills `out` (fp32 or bf16) with N(0,1); returns the generator offset advance."""
    _dev(out, "out", (torch.float32, torch.bfloat16))
    n = out.numel()
    rc = load().ltxk_philox_normal(
        _ptr(out), _dtype_code(out), n, seed & (2**64 - 1), offset, total_threads, _stream(out)
    )
    _check_rc(rc, "philox_normal")
    return offset_advance(n, total_threads)


def philox_u32(out: torch.Tensor, seed: int, offset: int, total_threads: int) -> int:
    """Raw uint32 words of the same stream, stored in an int32 tensor."""
    _dev(out, "out", torch.int32)
    n = out.numel()
    rc = load().ltxk_philox_u32(_ptr(out), n, seed & (2**64 - 1), offset, total_threads, _stream(out))
    _check_rc(rc, "philox_u32")
    return offset_advance(n, total_threads)


# --------------------------------------------------------------------------
# Euler / x0
# --------------------------------------------------------------------------


def euler_update(x: torch.Tensor, v: torch.Tensor, dt: float) -> torch.Tensor:
    """x <- x + dt*v in place (fp32 or bf16)."""
    _dev(x, "x", (torch.float32, torch.bfloat16))
    _dev(v, "v", x.dtype)
    if v.shape != x.shape:
        raise ValueError(f"shape mismatch {tuple(x.shape)} vs {tuple(v.shape)}")
    _check_rc(load().ltxk_euler_update(_ptr(x), _ptr(v), x.numel(), _dtype_code(x), dt, _stream(x)), "euler_update")
    return x


def euler_step(sample: torch.Tensor, denoised: torch.Tensor, sigma: float, dt: float,
               out: torch.Tensor | None = None) -> torch.Tensor:
    _dev(sample, "sample", (torch.float32, torch.bfloat16))
    _dev(denoised, "denoised", sample.dtype)
    if denoised.shape != sample.shape:
        raise ValueError("sample/denoised shape mismatch")
    out = _out_like(out, sample)
    rc = load().ltxk_euler_step(_ptr(out), _ptr(sample), _ptr(denoised), sample.numel(), _dtype_code(sample),
                                sigma, dt, _stream(sample))
    _check_rc(rc, "euler_step")
    return out


def x0(latent: torch.Tensor, velocity: torch.Tensor, timesteps: torch.Tensor) -> torch.Tensor:
    """x0 = round(latent - velocity * timesteps) with timesteps (B, T or 1, 1) fp32."""
    b, t, d = _btd(latent, "latent")
    _dev(velocity, "velocity")
    if velocity.shape != latent.shape:
        raise ValueError("latent/velocity shape mismatch")
    ts = timesteps
    _dev(ts, "timesteps", torch.float32)
    if ts.ndim != 3 or ts.shape[-1] != 1 or ts.shape[1] not in (1, t) or ts.shape[0] not in (1, b):
        raise ValueError(f"timesteps must be (B, T or 1, 1), got {tuple(ts.shape)}")
    bs = ts.shape[1] if ts.shape[0] > 1 else 0
    tstride = 1 if ts.shape[1] > 1 else 0
    out = torch.empty_like(latent)
    rc = load().ltxk_x0(_ptr(out), _ptr(latent), _ptr(velocity), _ptr(ts), bs, tstride, b * t, t, d,
                        _stream(latent))
    _check_rc(rc, "x0")
    return out


def guide(latent: torch.Tensor | None, velocity: torch.Tensor, timesteps: torch.Tensor | None, cfg_scale: float,
          stg_scale: float, modality_scale: float, rescale_scale: float, sigma: float | None = None,
          dt: float | None = None, want_denoised: bool = True, want_x0: bool = False,
          next_out: torch.Tensor | None = None, no_alloc: bool = False):
    """x0 of the four guidance passes, guide() and (with sigma, dt) euler_step.

    latent (B, T, C) bf16; velocity (4B, T, C) bf16, passes cond, uncond, ptb,
    mod stacked along the batch as the model returns them; timesteps fp32
    (4B, T, 1) (per token) or, for B == 1, (4, 1, 1).  With timesteps None,
    `velocity` holds the four x0 and latent is needed only for the Euler
    step.  Returns (denoised or None, next latent or None, x0 (4B, T, C) or
    None).  next_out may be the latent itself (in-place step).
    """
    _dev(velocity, "velocity")
    if velocity.ndim != 3 or velocity.shape[0] % 4 or not velocity.is_contiguous():
        raise ValueError(f"velocity must be contiguous (4B, T, C), got {tuple(velocity.shape)}")
    b, t, d = velocity.shape[0] // 4, velocity.shape[1], velocity.shape[2]
    if latent is not None:
        if tuple(_btd(latent, "latent")) != (b, t, d):
            raise ValueError(f"latent {tuple(latent.shape)} does not match velocity {tuple(velocity.shape)}")
    elif timesteps is not None or sigma is not None:
        raise ValueError("the latent is required with timesteps or an Euler step")
    ps = rs = 0
    ts = timesteps
    if ts is not None:
        _dev(ts, "timesteps", torch.float32)
        if ts.ndim != 3 or ts.shape[-1] != 1 or ts.shape[0] != 4 * b or ts.shape[1] not in (1, t) \
                or not ts.is_contiguous():
            raise ValueError(f"timesteps must be contiguous (4B, T or 1, 1), got {tuple(ts.shape)}")
        if ts.shape[1] == t:
            ps, rs = b * t, 1
        elif b == 1:
            ps, rs = 1, 0
        else:
            raise ValueError("per-pass scalar timesteps need B == 1; pass (4B, T, 1)")
    if (sigma is None) != (dt is None):
        raise ValueError("sigma and dt go together")
    like = velocity[:b]
    den = torch.empty_like(like) if want_denoised else None
    xo = torch.empty_like(velocity) if want_x0 else None
    nxt = _out_like(next_out, latent, "next_out") if sigma is not None else None
    n = b * t * d
    g = Guidance(cfg_scale, stg_scale, modality_scale, rescale_scale)
    sig = 0.0 if sigma is None else sigma
    dtv = 0.0 if dt is None else dt
    if no_alloc:  # the rescale's partial sums in the library's own device array
        rc = load().ltxk_guide_noalloc(_ptr(den), _ptr(xo), _ptr(nxt), _ptr(latent), _ptr(velocity), _ptr(ts), ps,
                                       rs, b * t, d, ctypes.byref(g), sig, dtv, _stream(velocity))
        _check_rc(rc, "guide_noalloc")
        return den, nxt, xo
    ws = None
    nbytes = 0
    if rescale_scale != 0:
        nbytes = int(load().ltxk_guide_workspace_bytes(n))
        ws = torch.empty(max(nbytes, 8), dtype=torch.uint8, device=velocity.device)
    rc = load().ltxk_guide(_ptr(den), _ptr(xo), _ptr(nxt), _ptr(latent), _ptr(velocity), _ptr(ts), ps, rs, b * t,
                           d, ctypes.byref(g), sig, dtv, _ptr(ws), nbytes, _stream(velocity))
    _check_rc(rc, "guide")
    return den, nxt, xo


def feature_norm(layers, keep: torch.Tensor | None, scale0: float, scale1: float | None = None,
                 eps: float = 1e-6):
    """FeatureExtractorV2's per-layer RMS norm, layer interleave, token mask and
    the two projection-input scales in one pass.  layers: L tensors (B, T, D)
    bf16; keep: (B, T) mask (non-zero = keep) or None.  Returns (out0, out1 or
    None), each (B, T, D*L) bf16."""
    layers = list(layers)
    if not layers:
        raise ValueError("no layers")
    b, t, d = _btd(layers[0], "layer 0")
    for i, x in enumerate(layers):
        _dev(x, f"layer {i}")
        if tuple(x.shape) != (b, t, d) or not x.is_contiguous():
            raise ValueError(f"layer {i} must be contiguous {(b, t, d)}, got {tuple(x.shape)}")
    n = len(layers)
    out0 = torch.empty(b, t, d * n, device=layers[0].device, dtype=torch.bfloat16)
    out1 = torch.empty_like(out0) if scale1 is not None else None
    k = None
    if keep is not None:
        if tuple(keep.shape) != (b, t):
            raise ValueError(f"keep mask must be {(b, t)}, got {tuple(keep.shape)}")
        _dev(keep, "keep", (torch.bool, torch.uint8, torch.int32, torch.int64, torch.bfloat16, torch.float32))
        k = (keep != 0).to(torch.uint8).contiguous()
    ptrs = (_c_vp * n)(*[x.data_ptr() for x in layers])
    rc = load().ltxk_feature_norm(_ptr(out0), _ptr(out1), ptrs, n, _ptr(k), b * t, d, eps, scale0,
                                  0.0 if scale1 is None else scale1, _stream(layers[0]))
    _check_rc(rc, "feature_norm")
    return out0, out1


# --------------------------------------------------------------------------
# Norms and modulation
# --------------------------------------------------------------------------


def rms_norm(x: torch.Tensor, weight: torch.Tensor | None = None, eps: float = 1e-6,
             out: torch.Tensor | None = None) -> torch.Tensor:
    _dev(x, "x")
    d = x.shape[-1]
    if weight is not None:
        _dev(weight, "weight")
        if weight.numel() != d:
            raise ValueError("weight size != last dim")
    out = _out_like(out, x)
    if x.numel() == 0:
        return out
    rc = load().ltxk_rms_norm(_ptr(out), _ptr(x), _ptr(weight), x.numel() // d, d, eps, _stream(x))
    _check_rc(rc, "rms_norm")
    return out


def norm_modulate(x: torch.Tensor, shift: AdaRef | None = None, scale: AdaRef | None = None,
                  shift2: AdaRef | None = None, scale2: AdaRef | None = None, eps: float = 1e-6,
                  layer: bool = False, out: torch.Tensor | None = None, out2: torch.Tensor | None = None):
    """y = norm(x)*(1+scale)+shift (and y2 with shift2/scale2 if either is given)."""
    b, t, d = _btd(x, "x")
    two = shift2 is not None or scale2 is not None
    out = _out_like(out, x)
    if two:
        out2 = _out_like(out2, x, "out2")
    if x.numel() == 0:
        return (out, out2) if two else out
    rc = load().ltxk_norm_modulate(
        _ptr(out), _ptr(out2) if two else None, _ptr(x), b * t, t, d, NORM_LAYER if layer else NORM_RMS, eps,
        _ada_arg(shift, b, t, d), _ada_arg(scale, b, t, d), _ada_arg(shift2, b, t, d), _ada_arg(scale2, b, t, d), _stream(x),
    )
    _check_rc(rc, "norm_modulate")
    return (out, out2) if two else out


def add_norm_modulate(x: torch.Tensor, f: torch.Tensor, gate: AdaRef | None = None,
                      mask: torch.Tensor | None = None, shift: AdaRef | None = None,
                      scale: AdaRef | None = None, eps: float = 1e-6, norm: bool = True,
                      x_out: torch.Tensor | None = None, shift2: AdaRef | None = None,
                      scale2: AdaRef | None = None):
    """x' = x + f*gate*mask; returns (x', rms(x')*(1+scale)+shift[, rms(x')*(1+scale2)+shift2])
    or x' alone if norm=False.  mask: one 0/1 value per batch item.  f None: the
    gate operand is the addend itself, x' = x + gate*mask (the keyframe
    position embedding added per token through an indexed operand)."""
    b, t, d = _btd(x, "x")
    if f is None:
        if gate is None:
            raise ValueError("add_norm_modulate without f needs the gate operand as the addend")
    else:
        _dev(f, "f")
        if f.shape != x.shape:
            raise ValueError(f"x {tuple(x.shape)} and f {tuple(f.shape)} differ")
    two = norm and (shift2 is not None or scale2 is not None)
    x_out = _out_like(x_out, x, "x_out")
    y = torch.empty_like(x) if norm else None
    y2 = torch.empty_like(x) if two else None
    if x.numel() == 0:
        return ((x_out, y, y2) if two else (x_out, y)) if norm else x_out
    if mask is not None:
        _dev(mask, "mask")
        if mask.numel() != b:
            raise ValueError(f"mask must hold one value per batch item ({b}), got {mask.numel()}")
    rc = load().ltxk_add_norm_modulate(
        _ptr(x_out), _ptr(y), _ptr(y2), _ptr(x), _ptr(f), _ada_arg(gate, b, t, d), _ptr(mask), b * t, t, d, eps,
        _ada_arg(shift, b, t, d), _ada_arg(scale, b, t, d), _ada_arg(shift2, b, t, d), _ada_arg(scale2, b, t, d),
        _stream(x),
    )
    _check_rc(rc, "add_norm_modulate")
    if not norm:
        return x_out
    return (x_out, y, y2) if two else (x_out, y)


def modulate(x: torch.Tensor, shift: AdaRef | None, scale: AdaRef | None,
             out: torch.Tensor | None = None) -> torch.Tensor:
    b, t, d = _btd(x, "x")
    out = _out_like(out, x)
    if x.numel() == 0:
        return out
    rc = load().ltxk_modulate(_ptr(out), _ptr(x), b * t, t, d, _ada_arg(shift, b, t, d), _ada_arg(scale, b, t, d),
                              _stream(x))
    _check_rc(rc, "modulate")
    return out


def modulate_layers(x: torch.Tensor, shift: AdaRef | None, scale: AdaRef | None, layers: int,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """`layers` context modulations of x (B, T, D) from one read of it:
    out[l] = round(x * (1 + scale_l) + shift_l), out (layers, B, T, D).

    shift / scale take their table from a stacked (layers, n, D) tensor (layer
    l reads table[l, row]) and one timestep embedding row shared by all
    layers; out[l] equals modulate(x, shift_l, scale_l).  The text
    cross-attention of every block modulates the same context with its own
    prompt table and the step's prompt timestep (ltx_dit.py:240-246), so a step
    can make all of them in one launch."""
    b, t, d = _btd(x, "x")
    strides = []
    for name, a in (("shift", shift), ("scale", scale)):
        if a is None or a.table is None:
            strides.append(0)
            continue
        if a.table.ndim != 3 or a.table.shape[0] != layers:
            raise ValueError(f"{name} table must be (layers={layers}, n, D), got {tuple(a.table.shape)}")
        strides.append(a.table[0].numel())
    if strides[0] and strides[1] and strides[0] != strides[1]:
        raise ValueError("shift and scale tables must have the same layer stride")
    tab_ls = max(strides)
    want = (layers, b, t, d)
    if out is None:
        out = torch.empty(want, device=x.device, dtype=x.dtype)
    else:
        _dev(out, "out")
        if tuple(out.shape) != want:
            raise ValueError(f"out {tuple(out.shape)} must be {want}")
    if x.numel() == 0 or layers == 0:
        return out
    rc = load().ltxk_modulate_layers(_ptr(out), _ptr(x), layers, b * t, t, d, _ada_arg(shift, b, t, d),
                                     _ada_arg(scale, b, t, d), tab_ls, 0, _stream(x))
    _check_rc(rc, "modulate_layers")
    return out


def gated_residual(x: torch.Tensor, f: torch.Tensor, gate: AdaRef | None = None,
                   mask: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    b, t, d = _btd(x, "x")
    _dev(f, "f")
    if f.shape != x.shape:
        raise ValueError(f"x {tuple(x.shape)} and f {tuple(f.shape)} differ")
    if mask is not None:
        _dev(mask, "mask")
        if mask.numel() != b:
            raise ValueError(f"mask must hold one value per batch item ({b}), got {mask.numel()}")
    out = _out_like(out, x)
    if x.numel() == 0:
        return out
    rc = load().ltxk_gated_residual(_ptr(out), _ptr(x), _ptr(f), _ada_arg(gate, b, t, d), _ptr(mask), b * t, t, d,
                                    _stream(x))
    _check_rc(rc, "gated_residual")
    return out


def head_gate(attn: torch.Tensor, logits: torch.Tensor | None, out: torch.Tensor | None = None,
              v: torch.Tensor | None = None, mask: torch.Tensor | None = None, heads: int | None = None) -> torch.Tensor:
    """attn (B, H, T, Dh) (any strides, Dh contiguous) or (B, T, H*Dh) token-major;
    logits (B, T, H) or None (gate 1).  With v (B, T, H*Dh) and a per-batch 0/1
    keep mask, attn is first blended with v: attn*m + v*(1-m).
    Returns (B, T, H*Dh) = blended attn * 2*sigmoid(logits) per head."""
    if not isinstance(attn, torch.Tensor) or attn.device.type != "cuda" or attn.dtype != torch.bfloat16:
        raise RuntimeError("attn must be a bf16 tensor on the ROCm device")
    if attn.ndim == 4:
        b, h, t, dh = attn.shape
        if attn.stride(3) != 1:
            raise ValueError("attn head_dim axis must be contiguous")
        sb, sh, st = attn.stride(0), attn.stride(1), attn.stride(2)
    else:
        _dev(attn, "attn")
        b, t = attn.shape[0], attn.shape[1]
        h = logits.shape[2] if logits is not None else heads
        if h is None or attn.shape[2] % h:
            raise ValueError("token-major attn needs logits or heads dividing its width")
        dh = attn.shape[2] // h
        sb, st, sh = attn.stride(0), attn.stride(1), dh
    if logits is not None:
        _dev(logits, "logits")
        if tuple(logits.shape) != (b, t, h):
            raise ValueError(f"logits {tuple(logits.shape)} != {(b, t, h)}")
    if v is not None:
        _dev(v, "v")
        if tuple(v.shape) != (b, t, h * dh):
            raise ValueError(f"v {tuple(v.shape)} != {(b, t, h * dh)}")
        if mask is None or mask.numel() != b:
            raise ValueError("a value blend needs one keep-mask value per batch item")
        _dev(mask, "mask")
    want_shape = (b, t, h * dh)
    if out is None:
        out = torch.empty(want_shape, device=attn.device, dtype=attn.dtype)
    else:
        _dev(out, "out")
        if tuple(out.shape) != want_shape:
            raise ValueError(f"out {tuple(out.shape)} != {want_shape}")
    if out.numel() == 0:
        return out
    rc = load().ltxk_head_gate(_ptr(out), _ptr(attn), sb, st, sh, _ptr(logits), _ptr(v),
                               _ptr(mask) if v is not None else None, b, t, h, dh, _stream(attn))
    _check_rc(rc, "head_gate")
    return out


def attn_combine(part: torch.Tensor, lse: torch.Tensor, parts: int, logits: torch.Tensor | None = None,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """Merges key-split attention: part (B*parts, H, T, Dh) bf16 (any strides,
    Dh contiguous) and lse (B*parts, H, >=T) fp32 from the flash kernel over
    `parts` key chunks -> (B, T, H*Dh) token-major, gated per head by
    2*sigmoid(logits (B, T, H)) when logits is given."""
    if not isinstance(part, torch.Tensor) or part.device.type != "cuda" or part.dtype != torch.bfloat16:
        raise RuntimeError("part must be a bf16 tensor on the ROCm device")
    if part.ndim != 4 or part.stride(3) != 1:
        raise ValueError("part must be (B*parts, H, T, Dh) with Dh contiguous")
    bp, h, t, dh = part.shape
    if parts < 1 or bp % parts:
        raise ValueError(f"leading dim {bp} is not a multiple of parts={parts}")
    b = bp // parts
    if not isinstance(lse, torch.Tensor) or lse.device != part.device or lse.dtype != torch.float32:
        raise ValueError("lse must be an fp32 tensor on part's device")
    if lse.ndim != 3 or lse.shape[0] != bp or lse.shape[1] != h or lse.shape[2] < t:
        raise ValueError(f"lse {tuple(lse.shape)} does not cover {(bp, h, t)}")
    if logits is not None:
        _dev(logits, "logits")
        if tuple(logits.shape) != (b, t, h):
            raise ValueError(f"logits {tuple(logits.shape)} != {(b, t, h)}")
    want_shape = (b, t, h * dh)
    if out is None:
        out = torch.empty(want_shape, device=part.device, dtype=torch.bfloat16)
    else:
        _dev(out, "out")
        if tuple(out.shape) != want_shape:
            raise ValueError(f"out {tuple(out.shape)} != {want_shape}")
    ps, ls = part.stride(), lse.stride()
    rc = load().ltxk_attn_combine(_ptr(out), _ptr(part), parts * ps[0], ps[0], ps[1], ps[2], _ptr(lse),
                                  parts * ls[0], ls[0], ls[1], ls[2], _ptr(logits), b, parts, t, h, dh, _stream(part))
    _check_rc(rc, "attn_combine")
    return out


def gelu_tanh(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    _dev(x, "x")
    out = _out_like(out, x)
    _check_rc(load().ltxk_gelu_tanh(_ptr(out), _ptr(x), x.numel(), _stream(x)), "gelu_tanh")
    return out


# --------------------------------------------------------------------------
# q/k norm + RoPE
# --------------------------------------------------------------------------


class CompactRope:
    """Rotation tables in the compact form of ltxk_qk: `cos`, `sin` bf16 rows
    [R, heads*head_dim/2] (one per coordinate value per position axis, zero
    outside that axis' pairs), `index` int32 [B, T, n_axes] of each token's row
    per axis, and the (B, H, T, head_dim/2) shape of the equivalent full
    tables.  Built by ltx_nn.precompute_freqs_cis_compact.

    The index is range-checked once here (one device-to-host read) unless the
    builder vouches for it (`checked=True`: precompute_freqs_cis_compact makes
    it from torch.unique's inverse, in range by construction).  The kernel
    clamps every index into [0, R) as well, so no index reads outside the
    tables."""

    __slots__ = ("cos", "sin", "index", "n_axes", "shape")

    def __init__(self, cos, sin, index, shape, checked: bool = False):
        self.cos, self.sin, self.index = cos, sin, index
        self.n_axes = index.shape[-1]
        self.shape = tuple(shape)
        if not checked and index.numel():
            lo, hi = int(index.min()), int(index.max())
            if lo < 0 or hi >= cos.shape[0]:
                raise ValueError(f"compact RoPE index spans [{lo}, {hi}], tables have {cos.shape[0]} rows")

    @property
    def rows(self) -> int:
        return self.cos.shape[0]


def _qk_struct(x: torch.Tensor, weight: torch.Tensor | None, pe, heads: int, head_dim: int, name: str) -> QK:
    b, t, d = _btd(x, name)
    if d != heads * head_dim:
        raise ValueError(f"{name} width {d} != heads*head_dim {heads * head_dim}")
    if weight is not None:
        _dev(weight, f"{name} norm weight")
        if weight.numel() != d:
            raise ValueError(f"{name} norm weight has {weight.numel()} entries, expected {d}")
    if pe is None:
        return QK(x.data_ptr(), _ptr(weight), None, None, b, t, 0, None, 0, 0)
    if isinstance(pe, CompactRope):
        _dev(pe.cos, f"{name} compact cos")
        _dev(pe.sin, f"{name} compact sin")
        _dev(pe.index, f"{name} position index", torch.int32)
        if pe.cos.shape != pe.sin.shape or pe.cos.ndim != 2 or pe.cos.shape[1] != d // 2:
            raise ValueError(f"{name} compact tables {tuple(pe.cos.shape)} != (R, {d // 2})")
        if tuple(pe.index.shape) != (b, t, pe.n_axes) or not 1 <= pe.n_axes <= 3:
            raise ValueError(f"{name} position index {tuple(pe.index.shape)} != ({b}, {t}, 1..3)")
        if pe.shape[1] != heads or pe.shape[3] != head_dim // 2:
            raise ValueError(f"{name} tables are for {pe.shape[1]} heads of {2 * pe.shape[3]}")
        return QK(x.data_ptr(), _ptr(weight), pe.cos.data_ptr(), pe.sin.data_ptr(), b, t, 0, pe.index.data_ptr(),
                  pe.n_axes, pe.rows)
    cos, sin = pe
    for tab, nm in ((cos, "cos"), (sin, "sin")):
        _dev(tab, f"{name} {nm}")
        if tab.ndim != 4 or tab.shape[1] != heads or tab.shape[2] != t or tab.shape[3] != head_dim // 2:
            raise ValueError(f"{name} {nm} table {tuple(tab.shape)} != (B, {heads}, {t}, {head_dim // 2})")
        if tab.shape[0] not in (1, b):
            raise ValueError(f"{name} {nm} table batch {tab.shape[0]} vs {b}")
    if cos.shape != sin.shape:
        raise ValueError("cos/sin shapes differ")
    tbs = cos.stride(0) if cos.shape[0] > 1 else 0
    return QK(x.data_ptr(), _ptr(weight), cos.data_ptr(), sin.data_ptr(), b, t, tbs, None, 0, 0)


def qk_norm_rope(q: torch.Tensor, k: torch.Tensor | None, heads: int, head_dim: int,
                 q_weight: torch.Tensor | None = None, k_weight: torch.Tensor | None = None,
                 q_pe=None, k_pe=None, eps: float = 1e-6) -> None:
    """In place: q = rope(rmsnorm(q)*q_weight, q_pe), same for k (weights/pe may be None)."""
    qs = _qk_struct(q, q_weight, q_pe, heads, head_dim, "q")
    ks = _qk_struct(k, k_weight, k_pe, heads, head_dim, "k") if k is not None else None
    rc = load().ltxk_qk_norm_rope(ctypes.byref(qs), ctypes.byref(ks) if ks is not None else None, heads, head_dim,
                                  eps, _stream(q))
    _check_rc(rc, "qk_norm_rope")
