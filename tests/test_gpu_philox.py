"""Parity of ltxk_philox_u32 / ltxk_philox_normal / ltxk_euler_update with the
oracle and with the reference's golden noise (GPU)."""

import json

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ADA_T_VIDEO = 852 * 256
DEV = "cuda"


def _u32(n, seed, off, T):
    import ltxk

    out = torch.empty(n, device=DEV, dtype=torch.int32)
    ltxk.philox_u32(out, seed, off, T)
    return out.cpu().numpy().view(np.uint32)


def _normal(n, seed, off, T, dtype=torch.float32):
    import ltxk

    out = torch.empty(n, device=DEV, dtype=dtype)
    adv = ltxk.philox_normal(out, seed, off, T)
    assert adv == O.offset_advance(n, T)
    return out


@pytest.mark.parametrize("n,seed,off,T", [
    (442368, 10, 0, ADA_T_VIDEO),
    (8704, 10, 4, 8704),
    (786432, 42, 0, ADA_T_VIDEO),
    (786432, 7, 0, 524288),
    (1000, 3, 8, 256),
    (77, 0xFFFFFFFFFFFF, 12, 6),      # tiny T: general (non-vector) path
    (1, 5, 0, 256),
    (4 * 256 * 3 + 1, 2**63 + 11, 4 * 2**33, 256),  # counter and key high words in use
])
def test_u32_stream_bit_exact(n, seed, off, T):
    assert np.array_equal(_u32(n, seed, off, T), O.philox_u32(n, seed, off, T))


def test_u32_stream_large_sampled():
    """64 Mi values (64 iterations per thread at T = 2^18): sampled indices."""
    n, seed, T = 1 << 26, 123, 1 << 18
    got = _u32(n, seed, 0, T)
    rng = np.random.default_rng(0)
    idx = np.concatenate([np.arange(4096), rng.integers(0, n, 4096), np.arange(n - 4096, n)])
    for e in idx[::7]:
        assert got[e] == O.philox_u32(1, seed, 0, T, first=int(e))[0]
    # a checksum over the whole stream against the oracle's (in 4 Mi chunks)
    total = np.uint64(0)
    for s in range(0, n, 1 << 22):
        total += O.philox_u32(1 << 22, seed, 0, T, first=s).astype(np.uint64).sum()
    assert got.astype(np.uint64).sum() == total


def _ulp_dist(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


@pytest.mark.parametrize("n,seed,T", [(786432, 42, ADA_T_VIDEO), (786432, 7, ADA_T_VIDEO), (1 << 20, 9, 524288),
                                      (999, 1, 6)])
def test_normal_fp32_within_2ulp(n, seed, T):
    got = _normal(n, seed, 0, T).cpu().numpy()
    want = O.philox_normal(n, seed, 0, T)
    d = _ulp_dist(got, want)
    print(f"n={n} seed={seed} T={T}: max ulp {d.max()}, {(d > 0).mean():.5%} differ, {(d > 1).sum()} by more than 1",
          flush=True)
    assert d.max() <= 2, f"max ulp {d.max()} ({(d > 0).mean():.4%} differ)"  # the parity bar
    # the kernel's own accuracy (fp64 Box-Muller rounded once): within 1 ulp of
    # the oracle's fp64 formula, and equal to it for all but a few in 10^5
    # (measured 0.002-0.0036 %)
    assert d.max() <= 1 and (d > 0).mean() <= 1e-4, f"max ulp {d.max()} ({(d > 0).mean():.5%} differ)"


def _golden(name):
    meta = json.loads((GOLDEN / "m1_philox" / "manifest.json").read_text())[name]
    return meta, np.fromfile(GOLDEN / "m1_philox" / name, dtype=np.uint16)


def test_reference_golden_noise_via_torch_rng():
    """TorchRNG seeded 10 with the Ada thread policy: video then audio, as
    create_noised_states / m1_philox.cu draw them."""
    from torch_rng import ADA_RTX6000, TorchRNG

    g = TorchRNG(10, DEV, *ADA_RTX6000)
    v = g.randn(1, 3456, 128, dtype=torch.bfloat16)
    assert g.offset == 4
    a = g.randn(1, 68, 128, dtype=torch.bfloat16)
    mv, gv = _golden("video_noise.bin")
    ma, ga = _golden("audio_noise.bin")
    vb = v.view(torch.int16).cpu().numpy().view(np.uint16).ravel()
    ab = a.view(torch.int16).cpu().numpy().view(np.uint16).ravel()
    dv = np.abs(O.bf16_bits_to_f32(vb) - O.bf16_bits_to_f32(gv))
    assert (vb == gv).mean() > 0.9997 and dv.max() <= 2.0**-7
    assert (ab == ga).mean() > 0.999 and np.abs(O.bf16_bits_to_f32(ab) - O.bf16_bits_to_f32(ga)).max() <= 2.0**-7
    # and the bf16 kernel output is the RNE rounding of the fp32 one
    v32 = _normal(3456 * 128, 10, 0, ADA_T_VIDEO).cpu().numpy()
    assert np.array_equal(vb, O.f32_to_bf16_bits(v32))


def test_bf16_odd_sizes_and_offsets():
    for n, off, T in ((13, 0, 256), (1031, 4, 512), (8 * 256 + 3, 8, 256), (5000, 0, 40)):
        got = _normal(n, 77, off, T, torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
        want = O.f32_to_bf16_bits(O.philox_normal(n, 77, off, T))
        assert (got == want).mean() > 0.999
        assert np.abs(O.bf16_bits_to_f32(got) - O.bf16_bits_to_f32(want)).max() <= 2.0**-7


def test_config0_noise_then_euler():
    """[1,128,16,16,24] fp32: x = N(seed 42), v = N(seed 7), x += -0.125 v."""
    import ltxk

    n = 128 * 16 * 16 * 24
    T = ltxk.device_policy_threads(n)
    x = _normal(n, 42, 0, T)
    v = _normal(n, 7, 0, T)
    x_before, v_host = x.cpu().numpy(), v.cpu().numpy()
    ltxk.euler_update(x, v, -0.125)
    # Euler is bit-exact given the same inputs (mul rounded, then add).
    assert np.array_equal(x.cpu().numpy(), O.euler_update_f32(x_before, v_host, -0.125))
    assert _ulp_dist(x_before, O.philox_normal(n, 42, 0, T)).max() <= 2


def test_empty_and_errors():
    import ltxk

    out = torch.empty(0, device=DEV)
    assert ltxk.philox_normal(out, 1, 0, 256) == 0
    with pytest.raises(RuntimeError, match="offset"):
        ltxk.philox_normal(torch.empty(8, device=DEV), 1, 2, 256)


def _sweep(n_cases=24, seed=5):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n_cases):
        n = int(rng.choice([1, 3, 4, 7, 63, 256, 1000, 4097, 65536 + 5, 300001]))
        T = int(rng.choice([1, 2, 3, 4, 6, 8, 12, 256, 1000, 4096, 65536, 218112]))
        out.append((n, int(rng.integers(0, 2**63)), 4 * int(rng.integers(0, 1 << 40)), T,
                    str(rng.choice(["f32", "bf16"]))))
    return out


@pytest.mark.parametrize("n,seed,off,T,dt", _sweep())
def test_stream_layout_sweep(n, seed, off, T, dt):
    """Seeded sweep of sizes, thread counts (multiples of 4 and 8 take the
    vector kernels, others the general one), offsets and seeds: the u32 stream
    bit-exact, fp32 normals within 2 ulp, bf16 normals the rounding of a value
    within 2 fp32 ulp of the oracle's, the offset advance as the oracle's."""
    assert np.array_equal(_u32(n, seed, off, T), O.philox_u32(n, seed, off, T))
    want = O.philox_normal(n, seed, off, T)
    if dt == "f32":
        got = _normal(n, seed, off, T).cpu().numpy()
        assert _ulp_dist(got, want).max() <= 2
    else:
        got = _normal(n, seed, off, T, torch.bfloat16).float().cpu().numpy()
        lo = np.nextafter(np.nextafter(want, -np.inf), -np.inf)
        hi = np.nextafter(np.nextafter(want, np.inf), np.inf)
        r = lambda a: torch.from_numpy(a).to(torch.bfloat16).float().numpy()  # noqa: E731
        assert bool(((got == r(lo)) | (got == r(want)) | (got == r(hi))).all())



# torch-ROCm's randn evaluates Box-Muller with rocRAND's single-precision device
# log/sin/cos: measured on the MI355X up to 1.67e-6 from the exact formula (config
# 0, seed 42; ltxk's normals are within 1 fp32 ulp of it).  A different thread
# count, offset or lane order changes the values by O(1).
TORCH_ROCM_ABS = 8e-6


def test_default_policy_matches_torch_randn_on_this_device():
    """TorchRNG's default (this device's thread policy) against torch.randn with a
    seeded generator of this device, the source create_noised_states draws from in
    the reference (ltx_dit.py:495-520): video [1,6144,128] bf16 then audio
    [1,126,128] bf16 from one generator (seed 10), and config 0's fp32 draw (seed
    42).  The generator offsets agree after every draw; >= 99.9 % of the bf16
    values are bit-equal and every other value is within one bf16 ulp (or
    TORCH_ROCM_ABS); every fp32 value is within TORCH_ROCM_ABS, the error of
    torch-ROCm's device transcendentals (ltxk's are within 1 ulp of the exact
    formula, which the oracle tests check)."""
    import torch_rng

    report = {}
    g = torch.Generator(device=DEV).manual_seed(10)
    ours = torch_rng.TorchRNG(10, DEV)
    for name, shape in (("video", (1, 6144, 128)), ("audio", (1, 126, 128))):
        want = torch.randn(*shape, generator=g, device=DEV, dtype=torch.bfloat16)
        got = ours.randn(*shape, dtype=torch.bfloat16)
        assert ours.offset == g.get_offset(), (name, ours.offset, g.get_offset())
        a, b = got.float().cpu().numpy().ravel(), want.float().cpu().numpy().ravel()
        eq = float((a == b).mean())
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.maximum(np.abs(a), np.abs(b)), 1e-30))) - 7)
        report[name] = eq
        assert eq >= 0.999, report
        assert bool((np.abs(a - b) <= np.maximum(ulp, TORCH_ROCM_ABS)).all()), name
    g = torch.Generator(device=DEV).manual_seed(42)
    ours = torch_rng.TorchRNG(42, DEV)
    want = torch.randn(1, 128, 16, 16, 24, generator=g, device=DEV, dtype=torch.float32)
    got = ours.randn(1, 128, 16, 16, 24, dtype=torch.float32)
    assert ours.offset == g.get_offset()
    d = np.abs(got.cpu().numpy() - want.cpu().numpy()).ravel()
    report["cfg0_f32_bit_equal"] = float((d == 0).mean())
    report["cfg0_f32_max_abs"] = float(d.max())
    print("torch.randn vs TorchRNG:", report, flush=True)
    assert float(d.max()) <= TORCH_ROCM_ABS and float(np.median(d)) <= 3e-7, report
