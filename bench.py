"""Benchmark of the LTX-2.5 DiT memory-bound path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-chain] [--no-full-step]

Prints ONE JSON line.  The headline (`value`) is the achieved HBM bandwidth of
the fused RMSNorm + AdaLN-modulate kernel on x [6144, 4096] bf16 with
broadcast shift/scale [4096] (one "step" = one kernel call over that
activation; K calls are timed).  `kernels` holds the same figures for every
kernel of the path at its workload; `chain` holds the non-GEMM microseconds of
one full 48-block audio-video denoise step (fused kernels vs the reference's
unfused eager PyTorch op sequence on the same GPU, with the GEMM/attention
outputs supplied as pre-made tensors) and the host time to enqueue it;
`full_step` and `guided_step` time whole denoise steps of the 48-block model
(GEMMs and attention on PyTorch-ROCm).  `cpu_baseline` times the oracle's CPU
restatement of every config on the host.

Timing: before the first kernel the GPU runs the headline kernel back to back
for a fixed settling time (so that short warm-ups measure the steady clock);
each kernel then runs W warm-up calls and K timed calls back to back between
two HIP events on the stream the kernels run on, behind a device-side head
start so the host never starves the queue (`us`), and 20 batches of 25 calls
(`us_median`, the median batch mean).  Launch-bound workloads (microseconds)
are timed from replays of a HIP graph of 20 calls (median over 25 replays).
Every kernel
rotates >= 3 buffer sets so no call finds its inputs in the 256 MB last-level
cache.  Algorithmic bytes count each tensor the op must read or write once
(bf16 = 2 bytes); RoPE tables and AdaLN rows are not counted.
"""

from __future__ import annotations

import argparse
import ctypes
import hashlib
import json
import os
import pathlib
import platform
import statistics
import sys
import time

REPO = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "ltx-nv_amd"))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s
CONFIG1 = "rmsnorm+adaln modulate, x [6144,4096] bf16, shift/scale [4096] bf16"
HEADLINE_KERNEL = ("norm_modulate_wave_kernel<8, false>", "1024")
SETTLE_S = 0.5  # device seconds of the headline kernel before anything is timed
RAMP_US = 40000.0  # device us of untimed calls between a head start and the timed calls
PLAIN = False  # --plain: each kernel runs warmup + steps calls only (counter passes)
ROTATE_BYTES = 4 * 256 * 2**20  # each line's buffer sets together span >= this: 4x the 256 MiB MALL
# philox_normal_vec<float> on 256 Mi values, per normal: executed VALU instructions (per
# lane) and fp64 flops (FMA = 2), from rocprofv3's SQ_INSTS_VALU / SQ_INSTS_VALU_FMA_F64 /
# SQ_INSTS_VALU_MUL_F64 (profiles/philox_normal_256M_valu_counters.md)
PHILOX_VALU_PER_NORMAL = 41.92
PHILOX_FP64_FLOPS_PER_NORMAL = 23.0


def nsets(per_set_bytes: int, least: int = 2) -> int:
    """How many input/output sets a line rotates so that no call finds its
    operands in the last-level (MALL) cache: ROTATE_BYTES over the bytes one
    call touches."""
    return max(least, -(-int(ROTATE_BYTES) // int(per_set_bytes)))


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--no-chain", action="store_true", help="skip the 48-block non-GEMM chain")
    ap.add_argument("--chain-steps", type=int, default=3)
    ap.add_argument("--only", default="",
                    help="comma list of kernel names to run (profiling); 'chain', 'full_step' and 'guided_step' "
                         "add those")
    ap.add_argument("--no-full-step", action="store_true",
                    help="skip the 48-block denoise steps with GEMMs and attention (B=1 and the B=4 guided step)")
    ap.add_argument("--full-steps", type=int, default=2)
    ap.add_argument("--plain", action="store_true",
                    help="each kernel line runs only warmup + steps calls, no head start or batches "
                         "(counter passes, where every dispatch is serialised)")
    ap.add_argument("--settle", type=float, default=SETTLE_S,
                    help="device seconds of the headline kernel before timing (0 for counter passes)")
    ap.add_argument("--summarize-trace", nargs="+", metavar=("CSV", "PATTERN"),
                    help="print a markdown summary of a rocprofv3 kernel-trace CSV and exit (no GPU)")
    ap.add_argument("--summarize-steps", nargs="+", metavar=("CSV", "BOUNDARY"),  # [STEPS]
                    help="print where traced full/guided denoise steps spend their time and exit (no GPU)")
    ap.add_argument("--summarize-counters", nargs="+", metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print a markdown summary of FETCH_SIZE and WRITE_SIZE counter CSVs and exit (no GPU)")
    ap.add_argument("--summarize-pmc", nargs="+", metavar="CSV",
                    help="print the mean of every counter per dispatch, per kernel, from rocprofv3 --pmc CSVs "
                         "and exit (no GPU); --pmc-pattern selects the kernels")
    ap.add_argument("--pmc-pattern", default="", help="regular expression over kernel names for --summarize-pmc")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# timing helpers
# ---------------------------------------------------------------------------


def head_start(us: float = 20000.0) -> None:
    """A device-side sleep on the current stream, so that the calls enqueued
    behind it are all queued before the GPU reaches them."""
    import torch

    torch.cuda._sleep(int(us * 2100))  # ~2.1 GHz cycles


def settle(call, seconds: float = SETTLE_S) -> float:
    """Runs `call` back to back for about `seconds` of device time (the GPU
    reaches its steady clocks); returns the device seconds spent."""
    import torch

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    spent, batch = 0.0, 50
    while spent < seconds:
        e0.record()
        for _ in range(batch):
            call()
        e1.record()
        e1.synchronize()
        dt = e0.elapsed_time(e1) * 1e-3
        spent += dt
        batch = max(50, min(20000, int(batch * (seconds - spent) / max(dt, 1e-6)) + 1))
    return spent


def time_calls(calls, steps: int, warmup: int, batches: int = 20, per_batch: int = 25) -> dict:
    """Device time per call of `calls[i % len(calls)]()`.

    `us`: the `steps` timed calls back to back between two HIP events (after
    `warmup` calls), behind a device-side head start so the host never starves
    the queue.  After the head start's near-idle 20 ms the clocks go through a
    transient once the load returns (measured per 25 calls: the headline 17.5
    us, then up to 18.7 us 2-6 ms in, back to 17.4-17.5 us after ~10 ms;
    Philox 256 Mi 379 us, up to 522 us 3 ms in, 366-377 us after ~30 ms), so
    about 40 ms of untimed calls run between the head start and the first
    event, and the timed calls see the steady state.
    `us_median`: the median over `batches` batch means of `per_batch`
    back-to-back calls (events only between batches: an event between every
    two calls costs ~3 us of queue time on this part, more than the spread it
    would resolve), after the same untimed calls."""
    import torch

    n = len(calls)
    w0, w1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0.record()
    for i in range(warmup):
        calls[i % n]()
    w1.record()
    torch.cuda.synchronize()
    per_call = w0.elapsed_time(w1) * 1e3 / max(warmup, 1)
    if PLAIN:
        w0.record()
        for i in range(steps):
            calls[i % n]()
        w1.record()
        w1.synchronize()
        us = w0.elapsed_time(w1) * 1e3 / max(steps, 1)
        return {"us": us, "us_median": us, "calls": steps, "timing": f"--plain: {warmup} + {steps} calls"}
    ramp = min(5000, max(2, int(RAMP_US / max(per_call, 1e-3)) + 1))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    head_start()
    for i in range(ramp):
        calls[i % n]()
    e0.record()
    for i in range(steps):
        calls[i % n]()
    e1.record()
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(batches + 1)]
    head_start()
    for i in range(ramp):
        calls[i % n]()
    ev[0].record()
    for b in range(batches):
        for i in range(per_batch):
            calls[(b * per_batch + i) % n]()
        ev[b + 1].record()
    ev[-1].synchronize()
    per = [ev[b].elapsed_time(ev[b + 1]) * 1e3 / per_batch for b in range(batches)]
    return {"us": us, "us_median": statistics.median(per), "calls": steps,
            "timing": f"{steps} calls back to back; median of {batches} batches of {per_batch}; "
                      f"{ramp} untimed calls before each"}


def time_graph(make_call, samples: int = 25, reps: int = 20) -> dict:
    """Per-call device time with the host's launch cost removed: `reps` calls
    captured into one HIP graph (on a side stream) and replayed `samples`
    times, each replay between two events; median and mean per call.
    `make_call(stream)` builds a zero-argument call that enqueues on that
    stream."""
    import torch

    side = torch.cuda.Stream()
    call = make_call(side.cuda_stream)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            call()
    side.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        for _ in range(reps):
            call()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(samples + 1)]
    head_start()
    ev[0].record()
    for i in range(samples):
        g.replay()
        ev[i + 1].record()
    ev[-1].synchronize()
    per = [ev[i].elapsed_time(ev[i + 1]) * 1e3 / reps for i in range(samples)]
    return {"us": statistics.median(per), "us_median": statistics.median(per), "calls": samples * reps,
            "timing": f"HIP graph of {reps} calls, median of {samples} replays"}


def bound_call(fn, *args):
    """A zero-argument raw C call with its ctypes arguments built once; raises on a nonzero status."""
    import ltxk

    def call():
        rc = fn(*args)
        if rc != 0:
            raise RuntimeError(f"{fn.__name__}: {ltxk.last_error()}")
    return call


def line(name, t: dict, nbytes, extra=None):
    us = t["us"]
    gbs = nbytes / (us * 1e-6) / 1e9
    d = {"us": round(us, 3), "us_median": round(t["us_median"], 3), "calls": t["calls"], "bytes": int(nbytes),
         "GB_s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
    if "timing" in t:
        d["timing"] = t["timing"]
    if extra:
        d.update(extra)
    return name, d


# ---------------------------------------------------------------------------
# per-kernel workloads
# ---------------------------------------------------------------------------


def bench_kernels(steps: int, warmup: int, only: set[str], settle_s: float = SETTLE_S):
    import torch

    import ltxk

    lib = ltxk.load()
    dev = torch.device("cuda")
    stream = torch.cuda.current_stream().cuda_stream
    out = {}
    g = torch.Generator(device=dev).manual_seed(0)

    def randn(*shape, scale=1.0):
        return (torch.randn(*shape, device=dev, generator=g) * scale).to(torch.bfloat16)

    def want(name):
        return not only or name in only

    meta = {}
    # config 1: fused RMSNorm + AdaLN modulate (headline); the clock settling runs on it first
    if want("norm_modulate"):
        sets = [(randn(6144, 4096), torch.empty(6144, 4096, device=dev, dtype=torch.bfloat16))
                for _ in range(nsets(2 * 6144 * 4096 * 2))]
        shift, scale = randn(4096, scale=0.02), randn(4096, scale=0.02)
        a_sh = ltxk.Ada(shift.data_ptr(), None, 0, 0)
        a_sc = ltxk.Ada(scale.data_ptr(), None, 0, 0)
        calls = [bound_call(lib.ltxk_norm_modulate, y.data_ptr(), None, x.data_ptr(), 6144, 6144, 4096, 0, 1e-6,
                            ctypes.byref(a_sh), ctypes.byref(a_sc), None, None, stream) for x, y in sets]
        k = [0]

        def rotating():
            calls[k[0] % len(calls)]()
            k[0] += 1
        meta["clock_settle_s"] = round(settle(rotating, settle_s), 3)
        t = time_calls(calls, steps, warmup)
        out.update([line("norm_modulate", t, 2 * 6144 * 4096 * 2 + 2 * 4096 * 2, {"config": CONFIG1})])
        del sets

    # a plain device copy of the config-1 activation: the bandwidth a streaming
    # read+write achieves here, and the calibration kernel for HBM byte counters
    if want("copy"):
        sets = [(randn(6144, 4096), torch.empty(6144, 4096, device=dev, dtype=torch.bfloat16))
                for _ in range(nsets(2 * 6144 * 4096 * 2))]
        calls = [lambda x=x, y=y: y.copy_(x) for x, y in sets]
        t = time_calls(calls, steps, warmup)
        out.update([line("copy", t, 2 * 6144 * 4096 * 2, {"config": "torch copy_ of [6144,4096] bf16"})])
        del sets

    # config 3: GELU-tanh on h [6144, 16384]
    if want("gelu_tanh"):
        n = 6144 * 16384
        sets = [(randn(n), torch.empty(n, device=dev, dtype=torch.bfloat16)) for _ in range(nsets(4 * n))]
        calls = [bound_call(lib.ltxk_gelu_tanh, y.data_ptr(), x.data_ptr(), n, stream) for x, y in sets]
        t = time_calls(calls, steps, warmup)
        out.update([line("gelu_tanh", t, 2 * n * 2, {"config": "h [6144,16384] bf16"})])
        del sets

    # every block's text-context modulation of a step in one launch: context
    # [1024,4096] read once, 48 modulated copies written
    if want("modulate_layers"):
        ctx = randn(1, 1024, 4096)
        tabs, pts = randn(48, 2, 4096, scale=0.02), randn(1, 1, 2 * 4096, scale=0.02)
        outs = [torch.empty(48, 1, 1024, 4096, device=dev, dtype=torch.bfloat16) for _ in range(2)]
        sh, sc = ltxk.AdaRef(tabs, 0, pts).struct(1, 1024), ltxk.AdaRef(tabs, 1, pts).struct(1, 1024)
        calls = [bound_call(lib.ltxk_modulate_layers, o.data_ptr(), ctx.data_ptr(), 48, 1024, 1024, 4096,
                            ctypes.byref(sh), ctypes.byref(sc), 2 * 4096, 0, stream) for o in outs]
        t = time_calls(calls, max(steps // 2, 20), warmup)
        out.update([line("modulate_layers", t, 1024 * 4096 * 2 * 49,
                         {"config": "context [1024,4096] bf16 x 48 blocks' prompt tables -> [48,1024,4096]"})])
        del outs

    # config 3: gated residual x + gate*f
    if want("gated_residual"):
        gate = randn(4096, scale=0.02)
        a_g = ltxk.Ada(gate.data_ptr(), None, 0, 0)
        sets = [(randn(6144, 4096), randn(6144, 4096), torch.empty(6144, 4096, device=dev, dtype=torch.bfloat16))
                for _ in range(nsets(3 * 6144 * 4096 * 2))]
        calls = [bound_call(lib.ltxk_gated_residual, o.data_ptr(), x.data_ptr(), f.data_ptr(), ctypes.byref(a_g),
                            None, 6144, 6144, 4096, stream) for x, f, o in sets]
        t = time_calls(calls, steps, warmup)
        out.update([line("gated_residual", t, 3 * 6144 * 4096 * 2 + 4096 * 2,
                         {"config": "x,f [6144,4096], gate [4096] bf16"})])
        del sets

    # the chain's video row kernels at the same shape: residual + norm + modulate (three broadcast
    # AdaLN rows), its two-output form (the A2V/V2A inputs), and the attention epilogue (per-head gate
    # + head merge) on SDPA's output layout
    if want("add_norm_modulate"):
        rows9 = randn(5, 4096, scale=0.02)
        a_gate, a_shift, a_scale, a_sh2, a_sc2 = (ltxk.Ada(rows9[i].data_ptr(), None, 0, 0) for i in range(5))
        sets = [tuple(randn(6144, 4096) for _ in range(2)) + tuple(
            torch.empty(6144, 4096, device=dev, dtype=torch.bfloat16) for _ in range(3))
                for _ in range(nsets(5 * 6144 * 4096 * 2))]
        calls = [bound_call(lib.ltxk_add_norm_modulate, xo.data_ptr(), y.data_ptr(), None, x.data_ptr(), f.data_ptr(),
                            ctypes.byref(a_gate), None, 6144, 6144, 4096, ctypes.c_float(1e-6),
                            ctypes.byref(a_shift), ctypes.byref(a_scale), None, None, stream)
                 for x, f, xo, y, _ in sets]
        t = time_calls(calls, steps, warmup)
        out.update([line("add_norm_modulate", t, 4 * 6144 * 4096 * 2 + 3 * 4096 * 2,
                         {"config": "x,f [6144,4096] -> x+f*gate, norm(.)*(1+scale)+shift; gate/shift/scale [4096]"})])
        calls = [bound_call(lib.ltxk_add_norm_modulate, xo.data_ptr(), y.data_ptr(), y2.data_ptr(), x.data_ptr(),
                            f.data_ptr(), ctypes.byref(a_gate), None, 6144, 6144, 4096, ctypes.c_float(1e-6),
                            ctypes.byref(a_shift), ctypes.byref(a_scale), ctypes.byref(a_sh2), ctypes.byref(a_sc2),
                            stream) for x, f, xo, y, y2 in sets]
        t = time_calls(calls, steps, warmup)
        out.update([line("add_norm_modulate_dual", t, 5 * 6144 * 4096 * 2 + 5 * 4096 * 2,
                         {"config": "the same with a second modulation of the normed row (two outputs)"})])
        del sets
    if want("head_gate"):
        sets = [(randn(6144, 32, 128), randn(6144, 32), torch.empty(6144, 4096, device=dev, dtype=torch.bfloat16))
                for _ in range(nsets(2 * 6144 * 4096 * 2))]
        calls = [bound_call(lib.ltxk_head_gate, o.data_ptr(), a.data_ptr(), 6144 * 4096, 4096, 128, lg.data_ptr(),
                            None, None, 1, 6144, 32, 128, stream) for a, lg, o in sets]
        t = time_calls(calls, steps, warmup)
        out.update([line("head_gate", t, 2 * 6144 * 4096 * 2 + 6144 * 32 * 2,
                         {"config": "attention out [6144,32,128] -> out * 2*sigmoid(logits [6144,32]), merged heads"})])
        del sets

    # config 2: RoPE on video q and k [1,32,6144,128] (token-major [6144,4096]), shared tables
    if want("rope_video"):
        import ltx_dit
        import ltx_nn

        pos = ltx_dit.video_positions(1, 16, 16, 24, 24.0, dev)
        cos, sin = ltx_nn.precompute_freqs_cis(pos, 4096, torch.bfloat16, max_pos=[20, 2048, 2048],
                                               num_attention_heads=32)
        sets = [(randn(6144, 4096), randn(6144, 4096)) for _ in range(nsets(2 * 6144 * 4096 * 2))]
        structs = [(ltxk.QK(q.data_ptr(), None, cos.data_ptr(), sin.data_ptr(), 1, 6144, 0),
                    ltxk.QK(k.data_ptr(), None, cos.data_ptr(), sin.data_ptr(), 1, 6144, 0)) for q, k in sets]
        calls = [bound_call(lib.ltxk_qk_norm_rope, ctypes.byref(sq), ctypes.byref(sk), 32, 128, 1e-6, stream)
                 for sq, sk in structs]
        t = time_calls(calls, steps, warmup)
        out.update([line("rope_video_qk", t, 4 * 6144 * 4096 * 2,
                         {"config": "q,k [1,32,6144,128] bf16, 16x16x24 grid, model positions (max_pos 20,2048,2048)",
                          "table_bytes": 2 * 6144 * 2048 * 2})])
        # the same launch with the q/k RMSNorm (weights) fused in, as the model runs it
        wq, wk = randn(4096), randn(4096)
        structs = [(ltxk.QK(q.data_ptr(), wq.data_ptr(), cos.data_ptr(), sin.data_ptr(), 1, 6144, 0),
                    ltxk.QK(k.data_ptr(), wk.data_ptr(), cos.data_ptr(), sin.data_ptr(), 1, 6144, 0))
                   for q, k in sets]
        calls = [bound_call(lib.ltxk_qk_norm_rope, ctypes.byref(sq), ctypes.byref(sk), 32, 128, 1e-6, stream)
                 for sq, sk in structs]
        t = time_calls(calls, steps, warmup)
        out.update([line("qk_norm_rope_video", t, 4 * 6144 * 4096 * 2,
                         {"config": "q,k [6144,4096] bf16 + RMSNorm weights + RoPE"})])
        # compact per-axis tables (56 rows of 2048 pairs + a [6144,3] index), as LTXModel runs it
        cp = ltx_nn.precompute_freqs_cis_compact(pos, 4096, torch.bfloat16, max_pos=[20, 2048, 2048],
                                                 num_attention_heads=32)
        structs = [(ltxk.QK(q.data_ptr(), wq.data_ptr(), cp.cos.data_ptr(), cp.sin.data_ptr(), 1, 6144, 0,
                            cp.index.data_ptr(), 3, cp.rows),
                    ltxk.QK(k.data_ptr(), wk.data_ptr(), cp.cos.data_ptr(), cp.sin.data_ptr(), 1, 6144, 0,
                            cp.index.data_ptr(), 3, cp.rows))
                   for q, k in sets]
        calls = [bound_call(lib.ltxk_qk_norm_rope, ctypes.byref(sq), ctypes.byref(sk), 32, 128, 1e-6, stream)
                 for sq, sk in structs]
        t = time_calls(calls, steps, warmup)
        out.update([line("qk_norm_rope_video_compact", t, 4 * 6144 * 4096 * 2,
                         {"config": "q,k [6144,4096] bf16 + RMSNorm weights + RoPE, compact tables"})])
        # config 2 itself (RoPE only) on the compact tables, for both position forms the config names:
        # the model's video_positions, and grid-normalised bounds (i, i+1) with max_pos (16, 16, 24)
        grid = torch.stack(torch.meshgrid(torch.arange(16.0), torch.arange(16.0), torch.arange(24.0),
                                          indexing="ij")).reshape(3, -1).to(dev)
        gpos = torch.stack([grid, grid + 1], dim=-1).unsqueeze(0).contiguous()
        for form, p_, mp in (("", pos, [20, 2048, 2048]), ("_grid", gpos, [16, 16, 24])):
            cp = ltx_nn.precompute_freqs_cis_compact(p_, 4096, torch.bfloat16, max_pos=mp, num_attention_heads=32)
            structs = [(ltxk.QK(q.data_ptr(), None, cp.cos.data_ptr(), cp.sin.data_ptr(), 1, 6144, 0,
                                cp.index.data_ptr(), 3, cp.rows),
                        ltxk.QK(k.data_ptr(), None, cp.cos.data_ptr(), cp.sin.data_ptr(), 1, 6144, 0,
                                cp.index.data_ptr(), 3, cp.rows))
                       for q, k in sets]
            calls = [bound_call(lib.ltxk_qk_norm_rope, ctypes.byref(sq), ctypes.byref(sk), 32, 128, 1e-6, stream)
                     for sq, sk in structs]
            t = time_calls(calls, steps, warmup)
            out.update([line(f"rope_video_qk_compact{form}", t, 4 * 6144 * 4096 * 2,
                             {"config": f"q,k [1,32,6144,128] bf16, 16x16x24 grid, max_pos {mp}, compact tables "
                                        f"({cp.rows} rows + index)"})])
        del sets, structs

    # A2V cross-attention q/k: video q [6144,2048] and audio k [126,2048] (32x64), time axis only
    if want("rope_cross"):
        import ltx_dit
        import ltx_nn

        vpos = ltx_dit.video_positions(1, 16, 16, 24, 24.0, dev)[:, 0:1]
        apos = ltx_dit.audio_positions(1, 126, dev)[:, 0:1]
        w = randn(2048)
        sets = [(randn(6144, 2048), randn(126, 2048)) for _ in range(nsets((6144 + 126) * 2048 * 2))]
        for form, build in (("full", ltx_nn.precompute_freqs_cis), ("compact", ltx_nn.precompute_freqs_cis_compact)):
            qt = build(vpos, 2048, torch.bfloat16, max_pos=[20], num_attention_heads=32)
            kt = build(apos, 2048, torch.bfloat16, max_pos=[20], num_attention_heads=32)
            if form == "full":
                qs = [ltxk.QK(q.data_ptr(), w.data_ptr(), qt[0].data_ptr(), qt[1].data_ptr(), 1, 6144, 0)
                      for q, _ in sets]
                ks = [ltxk.QK(k.data_ptr(), w.data_ptr(), kt[0].data_ptr(), kt[1].data_ptr(), 1, 126, 0)
                      for _, k in sets]
            else:
                qs = [ltxk.QK(q.data_ptr(), w.data_ptr(), qt.cos.data_ptr(), qt.sin.data_ptr(), 1, 6144, 0,
                              qt.index.data_ptr(), 1, qt.rows) for q, _ in sets]
                ks = [ltxk.QK(k.data_ptr(), w.data_ptr(), kt.cos.data_ptr(), kt.sin.data_ptr(), 1, 126, 0,
                              kt.index.data_ptr(), 1, kt.rows) for _, k in sets]
            calls = [bound_call(lib.ltxk_qk_norm_rope, ctypes.byref(sq), ctypes.byref(sk), 32, 64, 1e-6, stream)
                     for sq, sk in zip(qs, ks)]
            t = time_calls(calls, steps, warmup)
            out.update([line(f"qk_norm_rope_a2v_{form}", t, 2 * (6144 + 126) * 2048 * 2,
                             {"config": f"q [6144,2048] + k [126,2048] bf16, weights, 1-axis RoPE, {form} tables"})])
        # the model's form: A2V's video-side q and V2A's video-side k share the video time-axis tables, so
        # one paired launch rotates both (weights of their own), the audio sides in a second small launch
        qt = ltx_nn.precompute_freqs_cis_compact(vpos, 2048, torch.bfloat16, max_pos=[20], num_attention_heads=32)
        w2 = randn(2048)
        pairs = [(randn(6144, 2048), randn(6144, 2048)) for _ in range(nsets(2 * 6144 * 2048 * 2))]
        structs = [(ltxk.QK(a.data_ptr(), w.data_ptr(), qt.cos.data_ptr(), qt.sin.data_ptr(), 1, 6144, 0,
                            qt.index.data_ptr(), 1, qt.rows),
                    ltxk.QK(b.data_ptr(), w2.data_ptr(), qt.cos.data_ptr(), qt.sin.data_ptr(), 1, 6144, 0,
                            qt.index.data_ptr(), 1, qt.rows)) for a, b in pairs]
        calls = [bound_call(lib.ltxk_qk_norm_rope, ctypes.byref(sq), ctypes.byref(sk), 32, 64, 1e-6, stream)
                 for sq, sk in structs]
        t = time_calls(calls, steps, warmup)
        out.update([line("qk_norm_rope_av_video_pair", t, 4 * 6144 * 2048 * 2,
                         {"config": "A2V q + V2A k [6144,2048] each, own weights, shared time-axis compact tables"})])
        del sets, pairs

    # the text cross-attention's q/k norm (no RoPE): video q [6144,4096] and this block's context keys
    # [1024,4096], each with its own weight, one launch
    if want("text_qk"):
        w1, w2 = randn(4096), randn(4096)
        sets = [(randn(6144, 4096), randn(1024, 4096)) for _ in range(nsets((6144 + 1024) * 4096 * 2 * 2))]
        structs = [(ltxk.QK(q.data_ptr(), w1.data_ptr(), None, None, 1, 6144, 0),
                    ltxk.QK(k.data_ptr(), w2.data_ptr(), None, None, 1, 1024, 0)) for q, k in sets]
        calls = [bound_call(lib.ltxk_qk_norm_rope, ctypes.byref(a), ctypes.byref(b), 32, 128, 1e-6, stream)
                 for a, b in structs]
        t = time_calls(calls, steps, warmup)
        out.update([line("qk_norm_text_video", t, (6144 + 1024) * 4096 * 2 * 2,
                         {"config": "q [6144,4096] + context k [1024,4096] bf16, RMSNorm with weights, no RoPE"})])
        del sets, structs

    # config 2: audio RoPE q,k [1,32,126,64], positions 0..125 (launch-bound: graph replay)
    if want("rope_audio"):
        import ltx_nn

        pos = torch.arange(126, device=dev, dtype=torch.float32).view(1, 1, 126, 1).expand(1, 1, 126, 2).contiguous()
        cos, sin = ltx_nn.precompute_freqs_cis(pos, 2048, torch.bfloat16, max_pos=[126], num_attention_heads=32)
        q, k = randn(126, 2048), randn(126, 2048)
        sq = ltxk.QK(q.data_ptr(), None, cos.data_ptr(), sin.data_ptr(), 1, 126, 0)
        sk = ltxk.QK(k.data_ptr(), None, cos.data_ptr(), sin.data_ptr(), 1, 126, 0)
        t = time_graph(lambda st: bound_call(lib.ltxk_qk_norm_rope, ctypes.byref(sq), ctypes.byref(sk), 32, 64,
                                             1e-6, st))
        out.update([line("rope_audio_qk", t, 4 * 126 * 2048 * 2, {"config": "q,k [1,32,126,64] bf16"})])

    # guidance tail of a B=4 denoise step on the video latent [1,6144,128]: x0 of the
    # four passes + CFG/STG/modality guidance + std rescale + Euler (ltx_dit.py:551-606)
    if want("guide"):
        t_, c_ = 6144, 128
        n = t_ * c_
        lat = randn(1, t_, c_)
        vel = randn(4, t_, c_)
        ts = torch.full((4, t_, 1), 0.8, device=dev)
        nxt = torch.empty_like(lat)
        den = torch.empty_like(lat)
        ws = torch.empty(int(lib.ltxk_guide_workspace_bytes(n)), dtype=torch.uint8, device=dev)
        gp = ltxk.Guidance(3.0, 1.0, 3.0, 0.7)

        def make(st):
            return bound_call(lib.ltxk_guide, den.data_ptr(), None, nxt.data_ptr(), lat.data_ptr(), vel.data_ptr(),
                              ts.data_ptr(), t_, 1, t_, c_, ctypes.byref(gp), ctypes.c_float(0.8),
                              ctypes.c_float(-0.0625), ws.data_ptr(), ws.numel(), st)
        t = time_graph(make)
        # one pass of algorithmic traffic: latent + 4 velocities + timesteps in, denoised + next out
        nbytes = 2 * n + 4 * 2 * n + 4 * t_ * 4 + 2 * 2 * n
        out.update([line("guide_step_video", t, nbytes, {
            "config": "latent [1,6144,128] bf16, 4 passes, cfg 3 stg 1 mod 3 rescale 0.7, two launches"})])

        def eager():  # the reference's ops (ltx_dit.py:592-593, 551-562, 602-606) in bf16 eager
            v_latent = lat.repeat(4, 1, 1)
            x0 = (v_latent.float() - vel.float() * ts.float()).to(torch.bfloat16)
            c, u, p, m = (t.float() for t in x0.chunk(4))
            pred = c + 2.0 * (c - u) + 1.0 * (c - p) + 2.0 * (c - m)
            factor = 0.7 * (c.std() / pred.std()) + 0.3
            d = (pred * factor).to(torch.bfloat16)
            v = ((lat.float() - d.float()) / 0.8).to(torch.bfloat16)
            return (lat.float() + v.float() * -0.0625).to(torch.bfloat16)
        t = time_calls([eager], max(steps // 4, 10), max(warmup // 4, 3))
        out.update([line("guide_step_video_eager", t, nbytes, {"config": "same, PyTorch-ROCm eager ops"})])
        del lat, vel, ts, nxt, den

    # the V2A attention's key-split merge + head merge + per-head gate (ltx_nn.py:22-26,227-235): 8 chunk
    # outputs of 126 audio queries x 32 heads x 64 and their log-sum-exps -> the gated token-major output
    if want("attn_combine"):
        parts, h_, t_, d_ = 8, 32, 126, 64
        for b_ in (1, 4):
            part = randn(b_ * parts, t_, h_, d_).transpose(1, 2)  # the flash kernel's BTHD memory
            lse = torch.randn(b_ * parts, h_, t_, device=dev, generator=g)
            logits = randn(b_, t_, h_)
            o = torch.empty(b_, t_, h_ * d_, device=dev, dtype=torch.bfloat16)
            ps, ls = part.stride(), lse.stride()

            def make(st, part=part, lse=lse, logits=logits, o=o, ps=ps, ls=ls, b_=b_):
                return bound_call(lib.ltxk_attn_combine, o.data_ptr(), part.data_ptr(), parts * ps[0], ps[0], ps[1],
                                  ps[2], lse.data_ptr(), parts * ls[0], ls[0], ls[1], ls[2], logits.data_ptr(), b_,
                                  parts, t_, h_, d_, st)
            t = time_graph(make)
            nbytes = part.numel() * 2 + lse.numel() * 4 + logits.numel() * 2 + o.numel() * 2
            out.update([line(f"attn_combine_v2a_b{b_}", t, nbytes, {
                "config": f"{parts} key chunks x [{b_},32 heads,126,64] bf16 + lse -> [{b_},126,2048] gated"})])
            del part, lse, logits, o

    # text-encoder connector input: FeatureExtractorV2's per-layer RMS + interleave + mask + the two
    # projection scales over 49 language-model layers of [1024, 3840] (ltx_te.py:167-184)
    if want("feature_norm"):
        import math

        n_l, t_, d_ = 49, 1024, 3840
        layers = [randn(1, t_, d_) for _ in range(n_l)]
        keep = torch.ones(1, t_, dtype=torch.uint8, device=dev)
        keep[:, :300] = 0
        o0 = torch.empty(1, t_, d_ * n_l, device=dev, dtype=torch.bfloat16)
        o1 = torch.empty_like(o0)
        ptrs = (ctypes.c_void_p * n_l)(*[x.data_ptr() for x in layers])
        s0, s1 = math.sqrt(4096 / d_), math.sqrt(2048 / d_)
        keep_all = torch.ones_like(keep)
        nbytes = 3 * n_l * t_ * d_ * 2
        calls = [bound_call(lib.ltxk_feature_norm, o0.data_ptr(), o1.data_ptr(), ptrs, n_l, keep_all.data_ptr(), t_,
                            d_, ctypes.c_float(1e-6), ctypes.c_float(s0), ctypes.c_float(s1), stream)]
        t = time_calls(calls, max(steps // 4, 50), max(warmup // 4, 5))
        out.update([line("feature_norm_te", t, nbytes, {
            "config": "49 layers x [1024,3840] bf16 -> 2 x [1024,188160], scales, every token kept"})])
        # with 300 masked tokens: their outputs are +0 and their hidden states are not read, so the
        # algorithmic bytes are the kept tokens' reads and every output
        n_kept = int(keep.sum().item())
        calls = [bound_call(lib.ltxk_feature_norm, o0.data_ptr(), o1.data_ptr(), ptrs, n_l, keep.data_ptr(), t_, d_,
                            ctypes.c_float(1e-6), ctypes.c_float(s0), ctypes.c_float(s1), stream)]
        t = time_calls(calls, max(steps // 4, 50), max(warmup // 4, 5))
        out.update([line("feature_norm_te_masked", t, (n_kept + 2 * t_) * n_l * d_ * 2, {
            "config": f"same, {t_ - n_kept} of {t_} tokens masked (their rows not read)"})])
        mask3 = keep.bool().unsqueeze(-1)

        def eager():  # the reference's ops (ltx_te.py:167-179)
            enc = torch.stack(layers, dim=-1)
            var = torch.mean(enc ** 2, dim=2, keepdim=True)
            nrm = (enc * torch.rsqrt(var + 1e-6)).reshape(1, t_, d_ * n_l)
            nrm = torch.where(mask3, nrm, torch.zeros_like(nrm))
            return nrm * s0, nrm * s1
        t = time_calls([eager], 10, 3)
        out.update([line("feature_norm_te_eager", t, nbytes, {"config": "same, PyTorch-ROCm eager ops"})])
        del layers, o0, o1

    # config 0: Philox normal [1,128,16,16,24] fp32 and the Euler update (launch-bound: graph replay)
    if want("philox"):
        n = 128 * 16 * 16 * 24
        T = ltxk.device_policy_threads(n)
        x = torch.empty(n, device=dev)
        v = torch.empty(n, device=dev)
        t = time_graph(lambda st: bound_call(lib.ltxk_philox_normal, x.data_ptr(), 0, n, 42, 0, T, st))
        out.update([line("philox_normal_cfg0", t, 4 * n, {"config": "[1,128,16,16,24] fp32 seed 42", "T": T})])
        # the same draw under the reference run's thread policy (RTX 6000 Ada: 852 x 256 threads), the
        # T its golden noise pins
        T_ada = 852 * 256
        t = time_graph(lambda st: bound_call(lib.ltxk_philox_normal, x.data_ptr(), 0, n, 42, 0, T_ada, st))
        out.update([line("philox_normal_cfg0_ada_T", t, 4 * n,
                         {"config": "[1,128,16,16,24] fp32 seed 42, reference-Ada thread count", "T": T_ada})])
        t = time_graph(lambda st: bound_call(lib.ltxk_euler_update, x.data_ptr(), v.data_ptr(), n, 0,
                                             ctypes.c_float(-0.125), st))
        out.update([line("euler_update_cfg0", t, 12 * n, {"config": "[1,128,16,16,24] fp32, dt -0.125"})])
        # size sweep point: 256 Mi values, fp32 and bf16
        big = 1 << 28
        for dt_code, tdt, esz, nm in ((0, torch.float32, 4, "philox_normal_256M_f32"),
                                      (1, torch.bfloat16, 2, "philox_normal_256M_bf16")):
            buf = torch.empty(big, device=dev, dtype=tdt)
            Tb = ltxk.device_policy_threads(big)
            calls = [bound_call(lib.ltxk_philox_normal, buf.data_ptr(), dt_code, big, 7, 0, Tb, stream)]
            t = time_calls(calls, max(20, steps // 10), 2)
            extra = {"T": Tb, "normals_per_s": round(big / (t["us"] * 1e-6) / 1e9, 2)}
            if dt_code == 0:
                # ALU side: the executed VALU instructions per normal (rocprofv3 counters) against the
                # VALU issue peak, one wave64 instruction per CU per clock: CUs x 64 lanes x 2.4 GHz
                # lane-instructions per second at MI355X's nominal peak engine clock
                cus = torch.cuda.get_device_properties(0).multi_processor_count
                nps = big / (t["us"] * 1e-6)
                valu = nps * PHILOX_VALU_PER_NORMAL
                peak = cus * 64 * 2.4e9
                tf = nps * PHILOX_FP64_FLOPS_PER_NORMAL / 1e12
                extra["alu"] = {"valu_instructions_per_normal": PHILOX_VALU_PER_NORMAL,
                                "achieved_valu_lane_ops_per_s": round(valu / 1e12, 2),
                                "peak_valu_lane_ops_per_s": round(peak / 1e12, 2), "unit": "T/s",
                                "frac": round(valu / peak, 4),
                                "fp64_flops_per_normal": PHILOX_FP64_FLOPS_PER_NORMAL,
                                "achieved_tflops_fp64": round(tf, 2), "peak_tflops_fp64": 78.6,
                                "fp64_frac": round(tf / 78.6, 4)}
            out.update([line(nm, t, esz * big, extra)])
            del buf
        big_x = torch.empty(1 << 28, device=dev)
        big_v = torch.empty(1 << 28, device=dev)
        calls = [bound_call(lib.ltxk_euler_update, big_x.data_ptr(), big_v.data_ptr(), 1 << 28, 0,
                            ctypes.c_float(-0.125), stream)]
        t = time_calls(calls, max(20, steps // 10), 2)
        out.update([line("euler_update_256M_f32", t, 12 * (1 << 28))])
        del big_x, big_v
    torch.cuda.synchronize()
    return out, meta


# ---------------------------------------------------------------------------
# 48-block non-GEMM chain: fused kernels vs the reference's eager ops
# ---------------------------------------------------------------------------


def make_chain_inputs(dev, seed=123):
    """Activations and pre-made GEMM/attention outputs of one LTX-2.5 AV block at
    B=1: video 6144 x 4096 (32x128), audio 126 x 2048 (32x64), text 1024 tokens
    (video context 4096-d, audio context 2048-d), FFN 4x."""
    import torch

    import ltx_dit
    import ltx_nn

    g = torch.Generator(device=dev).manual_seed(seed)

    def r(*shape, s=1.0):
        return (torch.randn(*shape, device=dev, generator=g) * s).to(torch.bfloat16)

    V, A, C, D, DA = 6144, 126, 1024, 4096, 2048
    t = {}
    t["vx"], t["ax"] = r(1, V, D), r(1, A, DA)
    t["vctx"], t["actx"] = r(1, C, D), r(1, C, DA)
    for p, T_, d, h, dh in (("v", V, D, 32, 128), ("a", A, DA, 32, 64)):
        t[f"{p}_sst"] = r(9, d, s=0.02)
        t[f"{p}_psst"] = r(2, d, s=0.02)
        t[f"{p}_ts"] = r(1, 1, 9 * d, s=0.02)     # (B, 1, 9D): one timestep for all tokens
        t[f"{p}_pts"] = r(1, 1, 2 * d, s=0.02)
        t[f"{p}_css"] = r(1, 1, 4 * d, s=0.02)
        t[f"{p}_cgt"] = r(1, 1, d, s=0.02)
        t[f"{p}_avsst"] = r(5, d, s=0.02)
        t[f"{p}_q1"], t[f"{p}_k1"] = r(1, T_, d), r(1, T_, d)
        # attention outputs in the layout PyTorch-ROCm's SDPA returns: a
        # (B, T, H, D)-contiguous buffer viewed as (B, H, T, D)
        t[f"{p}_attn1"] = r(1, T_, h, dh).transpose(1, 2)
        t[f"{p}_logit1"] = r(1, T_, h)
        t[f"{p}_o1"] = r(1, T_, d)
        t[f"{p}_q2"], t[f"{p}_k2"] = r(1, T_, d), r(1, C, d)
        t[f"{p}_attn2"] = r(1, T_, h, dh).transpose(1, 2)
        t[f"{p}_logit2"] = r(1, T_, h)
        t[f"{p}_o2"] = r(1, T_, d)
        t[f"{p}_wq"], t[f"{p}_wk"] = r(d), r(d)
        t[f"{p}_h"] = r(1, T_, 4 * d)
        t[f"{p}_off"] = r(1, T_, d)
    # A2V: q from video (6144 x 2048), k from audio (126 x 2048); V2A the reverse
    t["a2v_q"], t["a2v_k"] = r(1, V, DA), r(1, A, DA)
    t["v2a_q"], t["v2a_k"] = r(1, A, DA), r(1, V, DA)
    t["a2v_attn"], t["a2v_logit"], t["a2v_o"] = r(1, V, 32, 64).transpose(1, 2), r(1, V, 32), r(1, V, D)
    t["v2a_attn"], t["v2a_logit"], t["v2a_o"] = r(1, A, 32, 64).transpose(1, 2), r(1, A, 32), r(1, A, DA)
    # the 48 blocks' prompt tables, stacked as LTXModel stacks them
    t["v_psst_all"], t["a_psst_all"] = r(48, 2, D, s=0.02), r(48, 2, DA, s=0.02)
    # the same timestep embeddings materialised per token, as the reference's
    # denoise step feeds them (timesteps = denoise_mask * sigma, (B, T, 1):
    # ltx_dit.py:578,584 -> adaln on B*T tokens, ltx_dit.py:146-150)
    for p, T_, d in (("v", V, D), ("a", A, DA)):
        t[f"{p}_ts_tok"] = t[f"{p}_ts"].expand(1, T_, 9 * d).contiguous()
        t[f"{p}_css_tok"] = t[f"{p}_css"].expand(1, T_, 4 * d).contiguous()
        t[f"{p}_cgt_tok"] = t[f"{p}_cgt"].expand(1, T_, d).contiguous()
    t["cw"] = r(DA)
    t["mask"] = torch.ones(1, device=dev, dtype=torch.bfloat16)
    vpos = ltx_dit.video_positions(1, 16, 16, 24, 24.0, dev)
    apos = ltx_dit.audio_positions(1, A, dev)
    t["vpe"] = ltx_nn.precompute_freqs_cis(vpos, D, torch.bfloat16, max_pos=[20, 2048, 2048], num_attention_heads=32)
    t["ape"] = ltx_nn.precompute_freqs_cis(apos, DA, torch.bfloat16, max_pos=[20], num_attention_heads=32)
    t["vcpe"] = ltx_nn.precompute_freqs_cis(vpos[:, 0:1], DA, torch.bfloat16, max_pos=[20], num_attention_heads=32)
    t["acpe"] = ltx_nn.precompute_freqs_cis(apos[:, 0:1], DA, torch.bfloat16, max_pos=[20], num_attention_heads=32)
    # the fused path takes the tables in the compact form, as LTXModel builds them
    for key, pos_, d_, mp in (("vpe", vpos, D, [20, 2048, 2048]), ("ape", apos, DA, [20]),
                              ("vcpe", vpos[:, 0:1], DA, [20]), ("acpe", apos[:, 0:1], DA, [20])):
        t[key + "_c"] = ltx_nn.precompute_freqs_cis_compact(pos_, d_, torch.bfloat16, max_pos=mp,
                                                            num_attention_heads=32)
    return t


def chain_bytes(blocks: int = 48) -> int:
    """Algorithmic HBM bytes of one step of the fused chain: every tensor each
    launch must read or write, once (bf16, 2 B), summed over the kernel list
    of fused_block and chain_prologue (AdaLN rows, RoPE tables and gate logits
    of a few KB aside: the logits are counted, the rest is not)."""
    V, A, C, D, DA = 6144, 126, 1024, 4096, 2048
    e = 2
    per_block = 0
    for T_, d, h in ((V, D, 32), (A, DA, 32)):
        per_block += 4 * T_ * d * e                    # residual + norm + modulate: x, f in; x, y out
        per_block += 4 * T_ * d * e                    # self-attention q/k norm + RoPE, in place
        per_block += 2 * T_ * d * e + T_ * h * e       # head gate: attention out in, merged out, logits
        per_block += 4 * T_ * d * e                    # residual + norm for the text cross-attention
        per_block += 2 * T_ * d * e + 2 * C * d * e    # text q norm and context k norm, in place
        per_block += 2 * T_ * d * e + T_ * h * e       # head gate
        per_block += 5 * T_ * d * e                    # residual + both AV modulations: x, f in; x, y, y2 out
        per_block += 4 * T_ * DA * e                   # A2V/V2A q/k on this side: two tensors in place
        per_block += 2 * T_ * DA * e + T_ * h * e      # AV head gate
        per_block += 4 * T_ * d * e                    # residual + FFN norm
        per_block += 2 * T_ * 4 * d * e                # GELU in place
    prologue = sum(C * d * e + blocks * C * d * e for d in (D, DA))  # context modulation of every block
    return blocks * per_block + prologue


_EVENTS: dict = {}
_EVENTS: dict = {}


def chain_prologue(t, blocks: int = 48):
    """Once per step, as LTXModel.forward: every block's text-context
    modulation (video and audio) in one launch each."""
    import ltxk

    for p in ("v", "a"):
        tabs, pts = t[f"{p}_psst_all"][:blocks], t[f"{p}_pts"]
        t[f"{p}_ctx_all"] = ltxk.modulate_layers(t[f"{p}ctx"], ltxk.AdaRef(tabs, 0, pts), ltxk.AdaRef(tabs, 1, pts),
                                                 tabs.shape[0])


def _chain_events() -> dict:
    import ltxk

    if not _EVENTS:
        _EVENTS.update({k: ltxk.StreamEvent() for k in ("fork", "join", "main_ready", "side_ready")})
    return _EVENTS


def fused_block(t, side=None, fork=True, join=False, collect=None):
    """The non-GEMM ops of one block as ltx_dit.Block runs them inside LTXModel:
    ltxk kernels; each residual is added in the same pass as the norm that
    follows it (the FFN residual in the next block's first norm, so a steady
    block starts with one); the audio stream's self/text and FFN work on a
    second HIP stream, forked from the main stream before a step's first block
    (fork) and joined after its last (join).  The block's modulated text
    context comes from chain_prologue, once per step.  `collect` (a dict)
    receives every launch's output by name (tests compare them with
    eager_block's)."""
    import torch

    import ltxk

    A_ = ltxk.AdaRef
    main = torch.cuda.current_stream()
    outs = {}
    keep = collect.__setitem__ if collect is not None else (lambda k, v: None)

    def self_text(p, heads, dh):
        x = t[f"{p}x"]
        sst, ts = t[f"{p}_sst"], t[f"{p}_ts"]
        x, y1 = ltxk.add_norm_modulate(x, t[f"{p}_off"], gate=A_(sst, 5, ts), shift=A_(sst, 0, ts),
                                       scale=A_(sst, 1, ts))
        ltxk.qk_norm_rope(t[f"{p}_q1"], t[f"{p}_k1"], heads, dh, t[f"{p}_wq"], t[f"{p}_wk"], t[f"{p}pe_c"],
                          t[f"{p}pe_c"])
        g1 = ltxk.head_gate(t[f"{p}_attn1"], t[f"{p}_logit1"])
        xf, q_in = ltxk.add_norm_modulate(x, t[f"{p}_o1"], gate=A_(sst, 2, ts), shift=A_(sst, 6, ts),
                                          scale=A_(sst, 7, ts))
        # (the block's modulated text context comes from chain_prologue)
        ltxk.qk_norm_rope(t[f"{p}_q2"], t[f"{p}_k2"], heads, dh, t[f"{p}_wq"], t[f"{p}_wk"])
        g2 = ltxk.head_gate(t[f"{p}_attn2"], t[f"{p}_logit2"])
        outs[p] = xf
        for k, v in (("norm1", y1), ("q1", t[f"{p}_q1"]), ("k1", t[f"{p}_k1"]), ("gate1", g1),
                     ("norm2", q_in), ("q2", t[f"{p}_q2"]), ("k2", t[f"{p}_k2"]), ("gate2", g2)):
            keep(f"{p}_{k}", v)

    def ffn(p, x, o, tab, cgt):
        sst, ts = t[f"{p}_sst"], t[f"{p}_ts"]
        x, h_in = ltxk.add_norm_modulate(x, o, gate=A_(tab, 4, cgt, 0), mask=t["mask"], shift=A_(sst, 3, ts),
                                         scale=A_(sst, 4, ts))
        ltxk.gelu_tanh(t[f"{p}_h"], out=t[f"{p}_h"])
        # the FFN residual is added by the next block's first norm
        for k, v in (("x3", x), ("norm4", h_in), ("gelu", t[f"{p}_h"])):
            keep(f"{p}_{k}", v)

    tv, vss = t["v_avsst"], t["v_css"]
    ta, ass = t["a_avsst"], t["a_css"]

    def av_inputs(p, x, tab, ss):
        # text cross-attention residual + both AV modulations of the row, one pass
        x, ya, yb = ltxk.add_norm_modulate(x, t[f"{p}_o2"], gate=A_(t[f"{p}_sst"], 8, t[f"{p}_ts"]), x_out=x,
                                           shift=A_(tab, 1, ss), scale=A_(tab, 0, ss), shift2=A_(tab, 3, ss),
                                           scale2=A_(tab, 2, ss))
        for k, v in (("x2", x), ("norm3a", ya), ("norm3b", yb)):
            keep(f"{p}_{k}", v)
        return x

    if side is None:  # one stream: the ops in the reference's order
        self_text("v", 32, 128)
        self_text("a", 32, 64)
        vx = av_inputs("v", outs["v"], tv, vss)
        ax = av_inputs("a", outs["a"], ta, ass)
        ltxk.qk_norm_rope(t["a2v_q"], t["v2a_k"], 32, 64, t["cw"], t["cw"], t["vcpe_c"], t["vcpe_c"])
        ltxk.qk_norm_rope(t["a2v_k"], t["v2a_q"], 32, 64, t["cw"], t["cw"], t["acpe_c"], t["acpe_c"])
        keep("a_gate3", ltxk.head_gate(t["v2a_attn"], t["v2a_logit"]))
        ffn("a", ax, t["v2a_o"], ta, t["a_cgt"])
        keep("v_gate3", ltxk.head_gate(t["a2v_attn"], t["a2v_logit"]))
        ffn("v", vx, t["a2v_o"], tv, t["v_cgt"])
        return
    # two streams, as Block._forward_two_streams: the main stream waits for the
    # side stream once (A2V keys), the side stream for the main once (V2A keys);
    # the same event kind (no timing, no system-scope fence), made once
    ev = _chain_events()
    if fork:
        ev["fork"].record(main)
        ev["fork"].wait(side)
    with torch.cuda.stream(side):
        self_text("a", 32, 64)
    self_text("v", 32, 128)
    vx = av_inputs("v", outs["v"], tv, vss)
    # A2V's queries and V2A's keys: both video-side, shared time-axis tables, one launch
    ltxk.qk_norm_rope(t["a2v_q"], t["v2a_k"], 32, 64, t["cw"], t["cw"], t["vcpe_c"], t["vcpe_c"])
    main_ready, side_ready = ev["main_ready"], ev["side_ready"]
    main_ready.record(main)
    with torch.cuda.stream(side):
        ax = av_inputs("a", outs["a"], ta, ass)
        ltxk.qk_norm_rope(t["a2v_k"], t["v2a_q"], 32, 64, t["cw"], t["cw"], t["acpe_c"], t["acpe_c"])
        side_ready.record(side)
        main_ready.wait(side)
        keep("a_gate3", ltxk.head_gate(t["v2a_attn"], t["v2a_logit"]))
        ffn("a", ax, t["v2a_o"], ta, t["a_cgt"])
    side_ready.wait(main)
    keep("v_gate3", ltxk.head_gate(t["a2v_attn"], t["a2v_logit"]))
    ffn("v", vx, t["a2v_o"], tv, t["v_cgt"])
    if join:
        ev["join"].record(side)
        ev["join"].wait(main)


def eager_block(t, per_token=False, collect=None):
    """The same ops as the reference writes them (ltx_dit.py:250-317, ltx_nn.py:204-248),
    unfused PyTorch eager in bf16, GEMM/attention outputs taken from `t`.
    per_token: timestep embeddings (B, T, n*D) as the reference's denoise step
    builds them; otherwise (B, 1, n*D), broadcast over tokens.  `collect`
    receives each op's result under fused_block's names (the FFN residual of
    the block's start, which fused_block takes from `{p}_off`, is the last op
    here)."""
    import torch
    import torch.nn.functional as F

    suffix = "_tok" if per_token else ""

    def ada(table, ts, idx):
        num = table.shape[0]
        rows = table[idx].unsqueeze(0).unsqueeze(0).to(dtype=ts.dtype)
        return (rows + ts.reshape(1, ts.shape[1], num, -1)[:, :, idx, :]).unbind(dim=2)

    def rms(x, w=None):
        return F.rms_norm(x, (x.shape[-1],), weight=w, eps=1e-6)

    def rope(x, pe):  # ltx_nn.py:99-115
        cos, sin = pe
        h = cos.shape[1]
        x = x.unflatten(-1, (h, -1)).transpose(1, 2)
        split = x.reshape(*x.shape[:-1], 2, x.shape[-1] // 2)
        first, second = split[..., :1, :], split[..., 1:, :]
        c, s = cos.unsqueeze(-2), sin.unsqueeze(-2)
        out = torch.cat([first * c - second * s, second * c + first * s], dim=-2).reshape(*x.shape)
        return out.transpose(1, 2).flatten(-2)

    def attn_tail(attn, logits, h, dh):  # ltx_nn.py:228,231-235
        b, _, tq, _ = attn.shape
        out = attn.transpose(1, 2).reshape(b, -1, h * dh)
        return (out.view(b, tq, h, dh) * (2.0 * torch.sigmoid(logits)).unsqueeze(-1)).view(b, tq, h * dh)

    keep = collect.__setitem__ if collect is not None else (lambda k, v: None)
    res = {}
    for p, heads, dh in (("v", 32, 128), ("a", 32, 64)):
        x = t[f"{p}x"]
        sst, ts = t[f"{p}_sst"], t[f"{p}_ts" + suffix]
        shift, scale, gate = ada(sst, ts, slice(0, 3))
        keep(f"{p}_norm1", rms(x) * (1 + scale) + shift)
        keep(f"{p}_q1", rope(rms(t[f"{p}_q1"], t[f"{p}_wq"]), t[f"{p}pe"]))
        keep(f"{p}_k1", rope(rms(t[f"{p}_k1"], t[f"{p}_wk"]), t[f"{p}pe"]))
        keep(f"{p}_gate1", attn_tail(t[f"{p}_attn1"], t[f"{p}_logit1"], heads, dh))
        xf = x + t[f"{p}_o1"] * gate
        xn = rms(xf)
        shq, scq, g2 = ada(sst, ts, slice(6, 9))
        kv = t[f"{p}_psst"][None, None] + t[f"{p}_pts"].reshape(1, 1, 2, -1)
        shkv, sckv = kv.unbind(dim=2)
        keep(f"{p}_norm2", xn * (1 + scq) + shq)
        keep(f"{p}_ctx", t[f"{p}ctx"] * (1 + sckv) + shkv)
        keep(f"{p}_q2", rms(t[f"{p}_q2"], t[f"{p}_wq"]))
        keep(f"{p}_k2", rms(t[f"{p}_k2"], t[f"{p}_wk"]))
        keep(f"{p}_gate2", attn_tail(t[f"{p}_attn2"], t[f"{p}_logit2"], heads, dh))
        res[p] = xf + t[f"{p}_o2"] * g2
    vx, ax = res["v"], res["a"]
    keep("v_x2", vx)
    keep("a_x2", ax)

    def av(table, ss, gt, idx):
        sc, sh = (u.squeeze(2) for u in ada(table[:4], ss, idx))
        (g,) = (u.squeeze(2) for u in ada(table[4:], gt, slice(None)))
        return sc, sh, g

    vcss, vcgt = t["v_css" + suffix], t["v_cgt" + suffix]
    acss, acgt = t["a_css" + suffix], t["a_cgt" + suffix]
    s, sh, gv = av(t["v_avsst"], vcss, vcgt, slice(0, 2))
    keep("v_norm3a", rms(vx) * (1 + s) + sh)
    s, sh, _g = av(t["a_avsst"], acss, acgt, slice(0, 2))
    keep("a_norm3a", rms(ax) * (1 + s) + sh)
    keep("a2v_q", rope(rms(t["a2v_q"], t["cw"]), t["vcpe"]))
    keep("a2v_k", rope(rms(t["a2v_k"], t["cw"]), t["acpe"]))
    keep("v_gate3", attn_tail(t["a2v_attn"], t["a2v_logit"], 32, 64))
    mask = t["mask"].reshape(-1, 1, 1)
    vx = vx + t["a2v_o"] * gv * mask
    s, sh, ga = av(t["a_avsst"], acss, acgt, slice(2, 4))
    keep("a_norm3b", rms(ax) * (1 + s) + sh)
    s, sh, _g = av(t["v_avsst"], vcss, vcgt, slice(2, 4))
    keep("v_norm3b", rms(res["v"]) * (1 + s) + sh)
    keep("v2a_q", rope(rms(t["v2a_q"], t["cw"]), t["acpe"]))
    keep("v2a_k", rope(rms(t["v2a_k"], t["cw"]), t["vcpe"]))
    keep("a_gate3", attn_tail(t["v2a_attn"], t["v2a_logit"], 32, 64))
    ax = ax + t["v2a_o"] * ga * mask
    for p, x in (("v", vx), ("a", ax)):
        sh, sc, g = ada(t[f"{p}_sst"], t[f"{p}_ts" + suffix], slice(3, 6))
        keep(f"{p}_x3", x)
        keep(f"{p}_norm4", rms(x) * (1 + sc) + sh)
        keep(f"{p}_gelu", F.gelu(t[f"{p}_h"], approximate="tanh"))
        _ = x + t[f"{p}_off"] * g


def bench_chain(steps: int, blocks: int = 48):
    """Device time per 48-block step of the fused chain and of the two eager
    comparators (a device-side head start keeps the host ahead of the GPU),
    and the host time the fused chain takes to enqueue one step."""
    import torch

    dev = torch.device("cuda")
    t = make_chain_inputs(dev)
    res = {}
    host = {}
    side = torch.cuda.Stream()

    def fused(t, i):
        if i % blocks == 0:
            chain_prologue(t, blocks)
        fused_block(t, side, fork=i % blocks == 0, join=i % blocks == blocks - 1)

    for name, fn in (("fused", fused),
                     ("eager", lambda t, i: eager_block(t)),
                     ("eager_tok", lambda t, i: eager_block(t, per_token=True))):
        fn(t, 0)  # warm-up (allocator, kernels): a first block, then a last one
        fn(t, blocks - 1)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        head_start(1_000_000)  # 1 s: the host enqueues every block before the GPU starts on them
        e0.record()
        h0 = time.perf_counter()
        for i in range(steps * blocks):
            fn(t, i)
        host[name] = (time.perf_counter() - h0) * 1e6 / steps
        torch.cuda.current_stream().wait_stream(side)  # the side stream's last work is inside the timing
        e1.record()
        e1.synchronize()
        res[name] = e0.elapsed_time(e1) * 1e3 / steps
    # the fused chain as one HIP graph (the forward has no host syncs, so a
    # step can be captured): device time per replay, host time per launch
    graph = None
    try:
        g = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cap):
            fused(t, 0)
            cap.wait_stream(side)
        cap.synchronize()
        with torch.cuda.graph(g, stream=cap):
            for i in range(blocks):
                # the last block's join brings every forked stream back before the capture ends
                fused(t, i)
        g.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        h0 = time.perf_counter()
        for _ in range(steps):
            g.replay()
        h1 = time.perf_counter()
        e1.record()
        e1.synchronize()
        graph = {"us_per_step_fused": round(e0.elapsed_time(e1) * 1e3 / steps, 1),
                 "host_us_per_step": round((h1 - h0) * 1e6 / steps, 1)}
        del g
    except RuntimeError as exc:  # capture is a measurement here, not a requirement of the chain
        graph = {"error": str(exc)[:200]}
    del t
    torch.cuda.empty_cache()
    return {
        "workload": "48 AV blocks, B=1: video 6144x4096 (32x128), audio 126x2048 (32x64), text 1024, FFN 4x; "
                    "GEMM/attention outputs pre-made",
        "us_per_step_fused": round(res["fused"], 1),
        "us_per_step_eager": round(res["eager"], 1),
        "speedup": round(res["eager"] / res["fused"], 2),
        "algorithmic_bytes_per_step": chain_bytes(blocks),
        "GB_s": round(chain_bytes(blocks) / (res["fused"] * 1e-6) / 1e9, 1),
        "frac": round(chain_bytes(blocks) / (res["fused"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "host_enqueue_us_per_step_fused": round(host["fused"], 1),
        "host_enqueue_us_per_step_eager": round(host["eager"], 1),
        "graph": graph,
        "timing": "device time of `steps` steps enqueued behind a 1 s device sleep, so the host's enqueue cost "
                  "(reported separately, host_enqueue_us_*) does not appear as GPU time",
        "eager_comparator": "reference Block ops in bf16 eager with one timestep embedding row per batch item "
                            "(broadcast over tokens), the same inputs the fused chain reads",
        "us_per_step_eager_per_token_timesteps": round(res["eager_tok"], 1),
        "speedup_vs_per_token_timesteps": round(res["eager_tok"] / res["fused"], 2),
        "per_token_comparator": "the same eager ops fed per-token timestep embeddings (B, T, n*D), as the "
                                "reference's denoise step builds them (ltx_dit.py:146-150,578,584); the fused "
                                "model de-duplicates them to one row per distinct timestep",
    }


# ---------------------------------------------------------------------------
# One full denoise step of the LTX-2.5-shape model (GEMMs and attention included)
# ---------------------------------------------------------------------------


def bench_guided_step(steps: int, warmup: int = 1):
    """The reference's denoising loop step at the 48-block model shape
    (ltx_dit.py:565-621): B=4 guidance batch (cond, uncond, STG-perturbed at
    block 28, modality-isolated), x0 + CFG/STG/modality guidance + std rescale +
    Euler per modality, on noise drawn by create_noised_states (121 frames at
    512x768: video 16x16x24 = 6144 tokens, audio 126); random bf16 weights
    (seed 123), random text contexts; sigmas of the 30-step schedule."""
    import dataclasses

    import torch

    import ltx_dit

    dev = torch.device("cuda")
    cfg = ltx_dit.DiTConfig()
    with torch.device("meta"):
        model = ltx_dit.LTXModel(cfg)
    model = model.to_empty(device=dev).to(torch.bfloat16).eval()
    g = torch.Generator(device=dev).manual_seed(123)
    with torch.no_grad():
        for p in model.parameters():
            p.normal_(0.0, 0.02, generator=g)
    vs, as_ = ltx_dit.create_noised_states(1, 121, 512, 768, 24.0, 10, dev, torch.bfloat16)
    r = lambda *shape: (torch.randn(*shape, device=dev, generator=g)).to(torch.bfloat16)  # noqa: E731
    contexts = {"v_pos": r(1, 1024, 4096), "v_neg": r(1, 1024, 4096), "a_pos": r(1, 1024, 2048),
                "a_neg": r(1, 1024, 2048)}
    vp = ltx_dit.GuiderParams(3.0, 1.0, 0.7, 3.0, (28,))
    ap = ltx_dit.GuiderParams(7.0, 1.0, 0.7, 3.0, (28,))
    sigmas = ltx_dit.ltx2_scheduler_sigmas(30, tokens=vs.latent.shape[1]).to(dev)
    state = {"v": vs, "a": as_, "i": 0}
    steps = min(steps, 28)

    def run(n):
        # n consecutive steps of the schedule in one run_dit call, as a denoising
        # loop runs them (its per-loop set-up is made once per call)
        i = state["i"]
        v, a = ltx_dit.run_dit(model, cfg, contexts, state["v"], state["a"], sigmas[i:i + n + 1], vp, ap)
        state["v"] = dataclasses.replace(state["v"], latent=v)
        state["a"] = dataclasses.replace(state["a"], latent=a)
        state["i"] += n

    for _ in range(warmup):
        run(1)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    run(steps)
    e1.record()
    e1.synchronize()
    ms = e0.elapsed_time(e1) / steps
    finite = bool(torch.isfinite(state["v"].latent.float()).all() and torch.isfinite(state["a"].latent.float()).all())
    del model
    torch.cuda.empty_cache()
    return {"workload": "LTX-2.5-shape AV DiT denoising step, 48 blocks, B=4 guidance batch (CFG 3/7, STG block 28, "
                        "modality 3, rescale 0.7), video 6144x4096, audio 126x2048, text 1024, random bf16 weights",
            "ms_per_step": round(ms, 2), "steps": steps, "latents_finite": finite}


def bench_full_step(steps: int, warmup: int = 1):
    """48-block AV model, random N(0, 0.02^2) bf16 weights (seed 123): video
    16x16x24 latent grid = 6144 tokens x 4096 (32 heads x 128), audio 126 tokens x
    2048 (32 x 64), text context 1024 tokens (4096-d video, 2048-d audio), FFN 4x,
    sigma 0.5, Euler dt -0.125.  One step = LTXModel.forward + x0 + Euler update."""
    import torch

    import ltx_dit
    import ltxk
    from torch_rng import TorchRNG

    dev = torch.device("cuda")
    cfg = ltx_dit.DiTConfig()
    with torch.device("meta"):
        model = ltx_dit.LTXModel(cfg)
    model = model.to_empty(device=dev).to(torch.bfloat16).eval()
    g = torch.Generator(device=dev).manual_seed(123)
    with torch.no_grad():
        for p in model.parameters():
            p.normal_(0.0, 0.02, generator=g)
    n_params = sum(p.numel() for p in model.parameters())
    rng = TorchRNG(123, dev)
    f, h, w, ta = 16, 16, 24, 126
    v_lat = rng.randn(1, f * h * w, 128, dtype=torch.bfloat16)
    a_lat = rng.randn(1, ta, 128, dtype=torch.bfloat16)
    v_ctx = rng.randn(1, 1024, 4096, dtype=torch.bfloat16)
    a_ctx = rng.randn(1, 1024, 2048, dtype=torch.bfloat16)
    sigma = torch.full((1,), 0.5, device=dev)
    v_ts = torch.full((1, f * h * w, 1), 0.5, device=dev)
    a_ts = torch.full((1, ta, 1), 0.5, device=dev)
    kf = torch.zeros(1, f * h * w, 1, device=dev)
    kf[:, : h * w] = 1.0
    # the distinct timesteps and the RoPE tables are made once, as a denoising
    # loop does (run_dit: from the denoise masks and positions of the run), not
    # read back from the device inside every step
    v_pos = ltx_dit.video_positions(1, f, h, w, 24.0, dev)
    a_pos = ltx_dit.audio_positions(1, ta, dev)
    video = ltx_dit.Modality(latent=v_lat, sigma=sigma, timesteps=v_ts, positions=v_pos, context=v_ctx,
                             keyframes_mask=kf, timestep_rows=ltx_dit.timestep_rows(v_ts),
                             rope_tables=model.video_pre.rope_tables(v_pos))
    audio = ltx_dit.Modality(latent=a_lat, sigma=sigma, timesteps=a_ts, positions=a_pos, context=a_ctx,
                             timestep_rows=ltx_dit.timestep_rows(a_ts),
                             rope_tables=model.audio_pre.rope_tables(a_pos))

    def step():
        with torch.no_grad():
            vx, ax = model(video, audio, None)
            x0v = ltxk.x0(v_lat, vx, v_ts)
            x0a = ltxk.x0(a_lat, ax, a_ts)
            ltxk.euler_step(v_lat, x0v, 0.5, -0.125)
            ltxk.euler_step(a_lat, x0a, 0.5, -0.125)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    e1.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # the same step as one HIP graph (the forward has no host sync once its
    # host-side caches are warm): device time per replay
    graph = None
    try:
        g = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(torch.cuda.current_stream())
        with torch.cuda.graph(g, stream=cap):
            step()
        g.replay()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            g.replay()
        e1.record()
        e1.synchronize()
        graph = {"ms_per_step": round(e0.elapsed_time(e1) / steps, 2)}
        del g
    except RuntimeError as exc:  # capture is a measurement here, not a requirement of the step
        graph = {"error": str(exc)[:200]}
    del model
    torch.cuda.empty_cache()
    return {"workload": "LTX-2.5-shape AV DiT, 48 blocks, B=1, video 6144x4096, audio 126x2048, text 1024, "
                        "random bf16 weights", "params": n_params, "ms_per_step": round(ms, 2), "steps": steps,
            "graph": graph}


# ---------------------------------------------------------------------------
# Measured HBM traffic of the headline kernel (committed counter summary)
# ---------------------------------------------------------------------------

COUNTER_SUMMARY = REPO / "profiles" / "hbm_traffic_counters.md"
COUNTER_SOURCES = ("ltx-nv_amd/csrc/rows.hip", "ltx-nv_amd/csrc/ltxk_common.h")


def source_digest() -> str:
    """sha256 (16 hex digits) over the sources the headline kernel is built from."""
    h = hashlib.sha256()
    for rel in COUNTER_SOURCES:
        h.update((REPO / rel).read_bytes())
    return h.hexdigest()[:16]


def counter_traffic(kernel: str, workgroups: str):
    """(bytes, note): HBM bytes per dispatch of `kernel` from the committed
    rocprofv3 counter summary (its calibrated traffic column: FETCH_SIZE and
    WRITE_SIZE scaled by what they read for a device copy of known size), or
    (None, why) when the summary has no row or was measured on other kernel
    sources than the ones built now (its `sources sha256` line)."""
    if not COUNTER_SUMMARY.exists():
        return None, "no counter summary"
    text = COUNTER_SUMMARY.read_text()
    digest = None
    for row in text.splitlines():
        if row.startswith("sources sha256:"):
            digest = row.split(":", 1)[1].strip().strip("`")
    if digest != source_digest():
        return None, f"counter summary measured on kernel sources {digest}, built now {source_digest()}"
    for row in text.splitlines():
        cells = [c.strip().strip("`") for c in row.strip().strip("|").split("|")]
        if len(cells) >= 6 and cells[0] == kernel and cells[1] == workgroups:
            return int(round(float(cells[5]) * 1e6)), "rocprofv3 FETCH_SIZE/WRITE_SIZE, calibrated on a device copy"
    return None, f"no row for {kernel} ({workgroups} workgroups)"


# ---------------------------------------------------------------------------
# rocprofv3 CSV summaries (the tables committed under profiles/)
# ---------------------------------------------------------------------------


def short_kernel_name(name: str) -> str:
    """A kernel's template name without namespaces and argument list."""
    import re

    name = re.sub(r"ltxk::\(anonymous namespace\)::", "", name)
    name = name.replace("(anonymous namespace)::", "").replace("at::native::", "")
    name = re.sub(r"^void ", "", name)
    if "(" in name:
        name = name[:name.index("(")] if not name.startswith("(") else name
    return name[:90]


def summarize_trace(path: str, pattern: str = "") -> str:
    """Markdown table of a rocprofv3 --kernel-trace CSV: one row per kernel and
    grid, with dispatches, mean and median duration."""
    import csv
    import re

    groups: dict = {}
    for r in csv.DictReader(open(path)):
        name = short_kernel_name(r["Kernel_Name"])
        if pattern and not re.search(pattern, name):
            continue
        key = (name, int(r["Grid_Size_X"]) // int(r["Workgroup_Size_X"]), int(r["Workgroup_Size_X"]),
               r.get("VGPR_Count", r.get("Arch_VGPR_Count", "")))
        groups.setdefault(key, []).append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    out = ["| kernel | workgroups | wg size | VGPRs | dispatches | mean us | median us |",
           "|---|---|---|---|---|---|---|"]
    for (name, wgs, wg, vgpr), v in groups.items():
        out.append(f"| `{name}` | {wgs} | {wg} | {vgpr} | {len(v)} | {sum(v) / len(v) / 1e3:.2f} | "
                   f"{statistics.median(v) / 1e3:.2f} |")
    return "\n".join(out)


def summarize_steps(path: str, boundary: str = "flat_kernel<2", steps: int | None = None) -> str:
    """Where a traced bench_full_step / bench_guided_step run spends its time:
    kernels that start inside the first `steps` timed steps (all when None; a
    step ends with its second Euler launch, the kernel named by `boundary`; the
    first such step is the warm-up), per HIP stream and class
    (GEMM = hipBLASLt/rocBLAS kernels, attention = SDPA's kernels, ltxk = this
    library's kernels, other = remaining torch ops), the union of busy
    intervals, and the ltxk kernels per stream."""
    import collections
    import csv
    import re

    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    ends = sorted(int(r["End_Timestamp"]) for r in rows if boundary in r["Kernel_Name"])[1::2]
    if steps is not None:
        ends = ends[:steps + 1]
    t0, t1, n = ends[0], ends[-1], len(ends) - 1

    def cls(name):
        low = name.lower()
        if re.search(r"cijk|gemm|hipblaslt|rocblas|matmul|xdl|gemv", low):
            return "GEMM"
        if re.search(r"attn_fwd|flash|fmha|aotriton|sdpa|softmax", low):
            return "attention"
        return "ltxk" if "ltxk::" in name else "other"

    by, cnt = collections.defaultdict(collections.Counter), collections.defaultdict(collections.Counter)
    per = collections.defaultdict(lambda: collections.defaultdict(list))
    busy = []
    for r in rows:
        st, en = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
        if st < t0 or st >= t1:
            continue
        c, sid = cls(r["Kernel_Name"]), r["Stream_Id"]
        by[sid][c] += en - st
        cnt[sid][c] += 1
        busy.append((st, en))
        if c == "ltxk":
            wgs = int(r["Grid_Size_X"]) // int(r["Workgroup_Size_X"])
            per[sid][(short_kernel_name(r["Kernel_Name"]), wgs)].append(en - st)
    busy.sort()
    union, (cs, ce) = 0, busy[0]
    for st, en in busy[1:]:
        if st > ce:
            union, cs, ce = union + ce - cs, st, en
        else:
            ce = max(ce, en)
    union += ce - cs
    out = [f"timed steps: {n}, window {(t1 - t0) / 1e6 / n:.2f} ms/step, GPU busy (union) {union / 1e6 / n:.2f} "
           f"ms/step", "", "| stream | class | dispatches/step | kernel ms/step |", "|---|---|---|---|"]
    for sid in sorted(by):
        for c, v in by[sid].most_common():
            out.append(f"| {sid} | {c} | {cnt[sid][c] // n} | {v / 1e6 / n:.2f} |")
    for sid in sorted(per):
        out += ["", f"ltxk kernels on stream {sid}:", "",
                "| kernel | workgroups | dispatches/step | mean us | ms/step |", "|---|---|---|---|---|"]
        for (name, wgs), v in sorted(per[sid].items(), key=lambda kv: -sum(kv[1])):
            out.append(f"| `{name}` | {wgs} | {len(v) // n} | {sum(v) / len(v) / 1e3:.2f} | {sum(v) / 1e6 / n:.3f} |")
    return "\n".join(out)


def summarize_counters(fetch_csv: str, write_csv: str, pattern: str = "",
                       copy_bytes: int = 6144 * 4096 * 2) -> str:
    """Markdown table of two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE; KiB
    per dispatch).  The device copy of `copy_bytes` (bench line `copy`, a
    torch copy_ of the config-1 activation) calibrates each counter: traffic =
    FETCH_SIZE * (copy_bytes / copy's FETCH_SIZE) + WRITE_SIZE * (copy_bytes /
    copy's WRITE_SIZE).  The `sources sha256` line names the kernel sources
    the counters were measured on (counter_traffic compares it)."""
    import csv
    import re

    def load(path):
        g: dict = {}
        for r in csv.DictReader(open(path)):
            name = short_kernel_name(r["Kernel_Name"])
            key = (name, int(r["Grid_Size"]) // int(r["Workgroup_Size"]))
            g.setdefault(key, []).append(float(r["Counter_Value"]))
        return {k: sum(v) / len(v) for k, v in g.items()}, {k: len(v) for k, v in g.items()}

    f, nf = load(fetch_csv)
    w, _ = load(write_csv)
    kib = copy_bytes / 1024
    copies = [k for k in f if "copyBuffer" in k[0] and k in w and abs(w[k] - kib) < 0.02 * kib]
    if not copies:
        raise SystemExit("no device-copy dispatch of the calibration size in the counter CSVs")
    cf, cw = kib / f[copies[0]], kib / w[copies[0]]
    out = [f"sources sha256: `{source_digest()}`", "",
           f"Calibration: `{copies[0][0]}` ({copies[0][1]} workgroups) copies {kib:.0f} KiB and reads "
           f"FETCH_SIZE {f[copies[0]]:.1f}, WRITE_SIZE {w[copies[0]]:.1f} KiB: fetch factor {cf:.3f}, "
           f"write factor {cw:.3f}.", "",
           "| kernel | workgroups | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | traffic MB |",
           "|---|---|---|---|---|---|"]
    for k in f:
        if pattern and not re.search(pattern, k[0]) and k not in copies:
            continue
        wv = w.get(k, float("nan"))
        out.append(f"| `{k[0]}` | {k[1]} | {nf[k]} | {f[k]:.1f} | {wv:.1f} | "
                   f"{(cf * f[k] + cw * wv) * 1024 / 1e6:.2f} |")
    return "\n".join(out)


def summarize_pmc(paths: list, pattern: str = "") -> str:
    """Markdown table: for each kernel (name, workgroups) matching `pattern`,
    the mean value per dispatch of every counter in the rocprofv3 --pmc CSVs
    (one pass per CSV; a counter's rows of one dispatch are summed first),
    plus the two ratios the memory-pipeline comparisons use: reads
    outstanding at the L2's memory interface (TCC_EA0_RDREQ_LEVEL /
    GRBM_GUI_ACTIVE) and vector-memory instructions in flight per busy SQ
    cycle (SQ_INST_LEVEL_VMEM / SQ_BUSY_CYCLES)."""
    import csv
    import re

    per: dict = {}  # (kernel, workgroups) -> counter -> dispatch -> value
    for path in paths:
        for r in csv.DictReader(open(path)):
            name = short_kernel_name(r["Kernel_Name"])
            if pattern and not re.search(pattern, name):
                continue
            key = (name, int(r["Grid_Size"]) // int(r["Workgroup_Size"]))
            d = per.setdefault(key, {}).setdefault(r["Counter_Name"], {})
            disp = r.get("Dispatch_Id") or r.get("Correlation_Id") or str(len(d))
            d[disp] = d.get(disp, 0.0) + float(r["Counter_Value"])
    kernels = sorted(per)
    counters = sorted({c for k in kernels for c in per[k]})
    mean = {k: {c: (sum(per[k][c].values()) / len(per[k][c])) for c in per[k]} for k in kernels}
    out = ["| counter | " + " | ".join(f"`{k[0]}` ({k[1]})" for k in kernels) + " |",
           "|---|" + "---:|" * len(kernels)]
    for c in counters:
        out.append(f"| {c} | " + " | ".join(f"{mean[k][c]:,.0f}" if c in mean[k] else "" for k in kernels) + " |")
    for label, num, den, fmt in (("reads outstanding (RDREQ_LEVEL / GUI_ACTIVE)", "TCC_EA0_RDREQ_LEVEL",
                                  "GRBM_GUI_ACTIVE", "{:,.0f}"),
                                 ("SQ_INST_LEVEL_VMEM / SQ_BUSY_CYCLES", "SQ_INST_LEVEL_VMEM", "SQ_BUSY_CYCLES",
                                  "{:.2f}")):
        if all(num in mean[k] and den in mean[k] and mean[k][den] for k in kernels):
            out.append(f"| {label} | " + " | ".join(fmt.format(mean[k][num] / mean[k][den]) for k in kernels) + " |")
    dispatches = {k: max(len(v) for v in per[k].values()) for k in kernels}
    out.append("")
    out.append("dispatches: " + ", ".join(f"`{k[0]}` {dispatches[k]}" for k in kernels))
    return "\n".join(out)


# ---------------------------------------------------------------------------
# CPU baselines: the oracle's restatement of every config on the host
# ---------------------------------------------------------------------------


def cpu_model() -> dict:
    name = platform.processor() or "unknown"
    try:
        for row in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
            if row.startswith("model name"):
                name = row.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"model": name, "logical_cpus": os.cpu_count(), "usable_cpus": usable}


def _median_time(fn, budget_s: float, max_runs: int = 5) -> tuple[float, int]:
    fn()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < max_runs and (not times or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baselines(budget_s: float = 6.0) -> dict:
    """Each config's op(s) on the host, timed with the oracle (fp32 torch-CPU on
    the stored bf16 inputs, one rounding per output; Philox in the oracle's
    scalar C).  Median of up to 5 runs after one warm-up."""
    import numpy as np
    import torch

    sys.path.insert(0, str(REPO))
    from oracle import oracle as O

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    out = {}

    # config 0: Philox noise (2 x 786,432 fp32, seeds 42 and 7) + Euler x + dt*v, the oracle's scalar C
    n = 128 * 16 * 16 * 24
    T = O.policy_threads(n, 142, 1536)

    def cfg0():
        x = O.philox_normal(n, 42, 0, T)
        v = O.philox_normal(n, 7, 0, T)
        return O.euler_update_f32(x, v, -0.125)
    s, runs = _median_time(cfg0, budget_s)
    out["config0"] = {"value": round(3 * 4 * n / s / 1e9, 3), "unit": "GB/s", "ms_per_call": round(s * 1e3, 2),
                      "cores": 1, "kind": "port", "runs": runs,
                      "sample": "oracle C Philox4x32-10 + Box-Muller (fp64) for x (seed 42) and v (seed 7), "
                                "[1,128,16,16,24] fp32 each, then x + dt*v; bytes = the three tensors written/read"}

    # config 1: RMSNorm + AdaLN modulate on the full input (the headline's CPU twin)
    x = torch.randn(6144, 4096, generator=g).to(torch.bfloat16)
    shift = (torch.randn(4096, generator=g) * 0.02).to(torch.bfloat16)
    scale = (torch.randn(4096, generator=g) * 0.02).to(torch.bfloat16)
    s, runs = _median_time(lambda: O.norm_modulate(x, shift, scale), budget_s)
    nb = 2 * 6144 * 4096 * 2 + 2 * 4096 * 2
    out["config1"] = {"value": round(nb / s / 1e9, 3), "unit": "GB/s", "ms_per_call": round(s * 1e3, 2),
                      "cores": threads, "kind": "port", "runs": runs,
                      "sample": "oracle fp32 torch-CPU norm_modulate on the full [6144,4096] bf16 input"}
    del x

    # config 2: split RoPE on q and k [1,32,6144,128] (token-major) with the model's video tables
    pos = O.video_positions(1, 16, 16, 24, 24.0)
    cos, sin = O.rope_tables(pos, 4096, 32, [20, 2048, 2048])
    q = torch.randn(1, 6144, 4096, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 6144, 4096, generator=g).to(torch.bfloat16)
    s, runs = _median_time(lambda: (O.apply_rope(q, cos, sin), O.apply_rope(k, cos, sin)), budget_s)
    nb = 4 * 6144 * 4096 * 2
    out["config2"] = {"value": round(nb / s / 1e9, 3), "unit": "GB/s", "ms_per_call": round(s * 1e3, 2),
                      "cores": threads, "kind": "port", "runs": runs,
                      "sample": "oracle fp32 torch-CPU apply_rope on q and k [1,6144,4096] bf16, full tables"}
    del q, k, cos, sin

    # config 3: GELU-tanh on [6144,16384] and the gated residual on [6144,4096]
    h = torch.randn(6144, 16384, generator=g).to(torch.bfloat16)
    xr = torch.randn(6144, 4096, generator=g).to(torch.bfloat16)
    fr = torch.randn(6144, 4096, generator=g).to(torch.bfloat16)
    gate = (torch.randn(4096, generator=g) * 0.02).to(torch.bfloat16)
    s, runs = _median_time(lambda: (O.gelu_tanh(h), O.gated_residual(xr, fr, gate)), budget_s)
    nb = 2 * 6144 * 16384 * 2 + 3 * 6144 * 4096 * 2
    out["config3"] = {"value": round(nb / s / 1e9, 3), "unit": "GB/s", "ms_per_call": round(s * 1e3, 2),
                      "cores": threads, "kind": "port", "runs": runs,
                      "sample": "oracle fp32 torch-CPU gelu_tanh [6144,16384] + gated_residual [6144,4096] bf16"}
    del h, xr, fr

    # config 4: one block's non-GEMM ops at the real shapes, x48 blocks
    t = make_chain_inputs(torch.device("cpu"))
    s, runs = _median_time(lambda: eager_block(t), budget_s, max_runs=3)
    out["config4"] = {"value": round(s * 48 * 1e3, 1), "unit": "ms non-GEMM per 48-block step",
                      "ms_per_block": round(s * 1e3, 1), "cores": threads, "kind": "port", "runs": runs,
                      "sample": "the reference's non-GEMM op sequence of one AV block (ltx_dit.py:250-317, "
                                "ltx_nn.py:204-248) in bf16 torch-CPU eager on pre-made GEMM/attention outputs, "
                                "timed once per block and multiplied by the 48 identical blocks of a step"}
    del t
    head = dict(out["config1"])
    head["configs"] = out
    head["cpu"] = cpu_model()
    head["torch_threads"] = threads
    return head


def main() -> int:
    args = parse()
    if args.summarize_pmc:
        print(summarize_pmc(args.summarize_pmc, args.pmc_pattern))
        return 0
    if args.summarize_trace:
        print(summarize_trace(*args.summarize_trace[:2]))
        return 0
    if args.summarize_steps:
        a = args.summarize_steps
        print(summarize_steps(a[0], a[1] if len(a) > 1 else "flat_kernel<2", int(a[2]) if len(a) > 2 else None))
        return 0
    if args.summarize_counters:
        print(summarize_counters(*args.summarize_counters[:3]))
        return 0
    if os.environ.get("ROCPROF_COUNTER_COLLECTION") and not args.plain:
        # counter passes serialise every dispatch: the head starts (a device
        # sleep), the clock settling and the graph replays measure nothing there
        print(json.dumps({"error": "under rocprofv3 counter collection run bench.py with --plain"}))
        return 2
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU; --gpus must be 1 (the kernels shard by token "
                                   "rows; only the guidance rescale's partial sums would be all-reduced)"}))
        return 2
    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm GPU visible"}))
        return 1
    only = set(filter(None, args.only.split(",")))
    global PLAIN
    PLAIN = args.plain
    print(f"[bench] kernels: steps={args.steps} warmup={args.warmup}", file=sys.stderr, flush=True)
    kern, meta = bench_kernels(args.steps, args.warmup, only, args.settle)
    head = kern.get("norm_modulate")
    chain = None
    if not args.no_chain and (not only or "chain" in only):
        print("[bench] 48-block non-GEMM chain", file=sys.stderr, flush=True)
        chain = bench_chain(args.chain_steps)
    full = guided = None
    if not args.no_full_step and (not only or "full_step" in only):
        print("[bench] full denoise step (B=1)", file=sys.stderr, flush=True)
        full = bench_full_step(args.full_steps)
    if not args.no_full_step and (not only or "guided_step" in only):
        print("[bench] guided denoising step (B=4)", file=sys.stderr, flush=True)
        guided = bench_guided_step(args.full_steps)
    cpu = None
    if not args.no_cpu and not only:
        print("[bench] cpu baselines", file=sys.stderr, flush=True)
        cpu = cpu_baselines()
    traffic, traffic_note = counter_traffic(*HEADLINE_KERNEL)
    rec = {
        "metric": "achieved HBM GB/s (% of peak) per fused kernel; us non-GEMM per DiT denoise step",
        "value": head["GB_s"] if head else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us"] / 1e3, 5) if head else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": CONFIG1, "rows": 6144, "dim": 4096, "eps": 1e-6},
        "gpu": torch.cuda.get_device_name(0),
        "clock_settle_s": meta.get("clock_settle_s"),
        "roofline": None,
        "cpu_baseline": cpu,
        "kernels": kern,
        "chain": chain,
        "full_step": full,
        "guided_step": guided,
    }
    if head:
        rec["roofline"] = {"bound": "hbm", "achieved": head["GB_s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": head["frac"], "traffic": traffic, "traffic_source": traffic_note,
                           "kernel": HEADLINE_KERNEL[0]}
    print(json.dumps(rec))
    return 0


if __name__ == "__main__":
    sys.exit(main())
