"""Pins the CPU oracle (oracle/) before it is trusted to check the HIP kernels.

Each oracle function is checked against something it does not restate:
published known-answer vectors, an independent library implementation,
the reference's own golden outputs, or a special case that reduces to a
library routine.  Runs on the CPU.
"""

import json
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import GOLDEN, bf16_from_bits
from oracle import oracle as O

# ---------------------------------------------------------------------------
# Philox4x32-10
# ---------------------------------------------------------------------------

# Random123 known-answer vectors for philox4x32 with 10 rounds (kat_vectors of
# the Random123 distribution): (counter, key) -> output.
R123_KAT = [
    ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
]


@pytest.mark.parametrize("ctr,key,want", R123_KAT)
def test_philox_known_answers(ctr, key, want):
    assert O.philox_block(ctr, key) == want


def test_philox_matches_rocrand_engine():
    """rocRAND's host philox4x32_10_engine(seed, subsequence, offset): subsequence
    = the counter's high 64 bits (thread id), offset/4 = the low 64 bits."""
    cases = json.loads((GOLDEN / "rocrand_philox.json").read_text())
    assert len(cases) >= 8
    for c in cases:
        seed, sub, off = c["seed"], c["subsequence"], c["offset"]
        for i, blk in enumerate(c["blocks"]):
            b = (off // 4 + i) & (2**64 - 1)
            ctr = [b & 0xFFFFFFFF, b >> 32, sub & 0xFFFFFFFF, sub >> 32]
            assert O.philox_block(ctr, [seed & 0xFFFFFFFF, seed >> 32]) == blk, c


def test_stream_layout_element_order():
    """Element e of a T-thread draw is word (e/T)%4 of thread e%T's block e/(4T)."""
    T, seed, off = 6, 99, 8
    n = 4 * T * 3 - 5
    s = O.philox_u32(n, seed, off, T)
    for e in range(n):
        it, r = divmod(e, 4 * T)
        lane, tid = divmod(r, T)
        blk = off // 4 + it
        assert s[e] == O.philox_block([blk, 0, tid, 0], [seed, 0])[lane]


def test_policy_and_offset_advance():
    # Ada RTX 6000: 142 SMs x 1536 threads -> grid capped at 852 blocks.
    assert O.policy_threads(442368, 142, 1536) == 852 * 256
    assert O.policy_threads(8704, 142, 1536) == 34 * 256
    assert O.offset_advance(442368, 852 * 256) == 4
    assert O.offset_advance(852 * 256 * 4 + 1, 852 * 256) == 8
    assert O.offset_advance(0, 256) == 0


def _golden(name):
    meta = json.loads((GOLDEN / "m1_philox" / "manifest.json").read_text())[name]
    bits = np.fromfile(GOLDEN / "m1_philox" / name, dtype=np.uint16)
    return meta, bits


def test_golden_fixture_integrity():
    import hashlib

    for name in ("video_noise.bin", "audio_noise.bin"):
        meta, bits = _golden(name)
        assert hashlib.sha256(bits.tobytes()).hexdigest() == meta["sha256"]
        assert bits.size == int(np.prod(meta["shape"]))


def test_oracle_reproduces_reference_audio_noise():
    """seed 10, offset 4 (after the video draw), T = 8704: bit-exact in bf16."""
    meta, gold = _golden("audio_noise.bin")
    mine = O.f32_to_bf16_bits(O.philox_normal(gold.size, meta["seed"], meta["offset"], meta["total_threads"]))
    assert np.array_equal(mine, gold)


def test_oracle_reproduces_reference_video_noise():
    """seed 10, offset 0, T = 852*256.  The reference's device transcendentals
    (not reproducible here) flip ~0.03% of bf16 roundings; all by <= 2^-7."""
    meta, gold = _golden("video_noise.bin")
    mine = O.f32_to_bf16_bits(O.philox_normal(gold.size, meta["seed"], meta["offset"], meta["total_threads"]))
    diff = np.abs(O.bf16_bits_to_f32(mine) - O.bf16_bits_to_f32(gold))
    assert (mine == gold).mean() > 0.9997
    assert diff.max() <= 2.0**-7
    # Another thread count gives another stream: the layout is what is pinned.
    other = O.f32_to_bf16_bits(O.philox_normal(gold.size, 10, 0, 2048 * 256))
    assert (other == gold).mean() < 0.6


def test_box_muller_closed_form_and_moments():
    # (u, v) from the published formula: u in (0, 1], v in (0, 2pi].
    u, v = O.box_muller_uv(0, 0)
    assert u == np.float32(2.0**-32) and v == np.float32(2 * math.pi * 2.0**-32)
    u, v = O.box_muller_uv(0xFFFFFFFF, 0xFFFFFFFF)
    assert u == 1.0 and abs(v - 2 * math.pi) < 1e-6
    # Lane order of a pair: (s sin v, s cos v).
    blk = O.philox_block([0, 0, 0, 0], [5, 0])
    u, v = O.box_muller_uv(blk[0], blk[1])
    s = math.sqrt(-2 * math.log(u))
    z = O.philox_normal(4, 5, 0, 1)
    assert abs(z[0] - s * math.sin(v)) < 1e-6 * max(1, abs(z[0]))
    assert abs(z[1] - s * math.cos(v)) < 1e-6 * max(1, abs(z[1]))
    big = O.philox_normal(1 << 20, 123, 0, 2048 * 256)
    assert abs(big.mean()) < 5e-3 and abs(big.std() - 1) < 5e-3
    # P(|z| > 3) = 0.0027
    assert abs((np.abs(big) > 3).mean() - 0.0027) < 3e-4


def test_euler_update_f32_rounding_order():
    x = np.array([1.0, 3.0, -2.5], dtype=np.float32)
    v = np.array([0.1, -7.0, 1e-8], dtype=np.float32)
    got = O.euler_update_f32(x, v, -0.125)
    want = x + (v * np.float32(-0.125)).astype(np.float32)
    assert np.array_equal(got, want)
    assert np.array_equal(O.euler_update_f32(x, v, 0.0), x)


# ---------------------------------------------------------------------------
# Floating-point restatements vs library routines / special cases
# ---------------------------------------------------------------------------


def _bf(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def test_rms_norm_matches_torch():
    x = _bf((37, 256), 1)
    w = _bf((256,), 2)
    assert torch.equal(O.rms_norm(x), F.rms_norm(x, (256,), eps=1e-6))
    assert torch.equal(O.rms_norm(x, w), F.rms_norm(x, (256,), weight=w, eps=1e-6))


def test_norm_modulate_special_cases():
    x = _bf((2, 11, 128), 3)
    zero = torch.zeros(128, dtype=torch.bfloat16)
    # scale 0, shift 0 -> plain RMSNorm (library routine)
    assert torch.equal(O.norm_modulate(x, zero, zero), F.rms_norm(x, (128,), eps=1e-6))
    # scale -1 -> output is exactly the shift
    sh = _bf((128,), 4)
    out = O.norm_modulate(x, sh, -torch.ones(128, dtype=torch.bfloat16))
    assert torch.equal(out, sh.expand_as(out))
    # layer=True, no modulation -> F.layer_norm without affine
    ln = F.layer_norm(x.float(), (128,), eps=1e-6).to(torch.bfloat16)
    d = (O.norm_modulate(x, layer=True).float() - ln.float()).abs()
    assert d.max() <= 2.0**-7 * max(1.0, ln.float().abs().max().item())
    # scale 1 doubles the normalised value (exact in binary)
    two = O.norm_modulate(x, zero, torch.ones(128, dtype=torch.bfloat16))
    assert torch.equal(two, (2 * F.rms_norm(x.float(), (128,), eps=1e-6)).to(torch.bfloat16))


def test_gated_residual_and_modulate_special_cases():
    x, f = _bf((3, 5, 64), 5), _bf((3, 5, 64), 6)
    assert torch.equal(O.gated_residual(x, f, torch.zeros(64, dtype=torch.bfloat16)), x)
    assert torch.equal(O.gated_residual(x, f), torch.add(x.float(), f.float()).to(torch.bfloat16))
    mask = torch.tensor([1.0, 0.0, 1.0], dtype=torch.bfloat16)
    g = _bf((64,), 7)
    r = O.gated_residual(x, f, g, mask)
    assert torch.equal(r[1], x[1])
    assert torch.equal(r[0], O.gated_residual(x[0:1], f[0:1], g)[0])
    # modulate with scale 0 adds the shift; with scale -1 returns the shift
    sh = _bf((64,), 8)
    assert torch.equal(O.modulate(x, sh, torch.zeros(64, dtype=torch.bfloat16)),
                       torch.add(x.float(), sh.float()).to(torch.bfloat16))
    assert torch.equal(O.modulate(x, sh, -torch.ones(64, dtype=torch.bfloat16)), sh.expand_as(x))


def test_add_norm_modulate_composes():
    x, f, g = _bf((2, 7, 96), 9), _bf((2, 7, 96), 10), _bf((96,), 11, 0.1)
    xo, y = O.add_norm_modulate(x, f, g)
    assert torch.equal(xo, O.gated_residual(x, f, g))
    assert torch.equal(y, F.rms_norm(xo, (96,), eps=1e-6))


def test_head_gate_special_cases():
    out = _bf((2, 3, 4 * 16), 12)
    zero = torch.zeros(2, 3, 4, dtype=torch.bfloat16)
    assert torch.equal(O.head_gate(out, zero, 4), out)       # 2*sigmoid(0) = 1
    big = torch.full((2, 3, 4), 100.0, dtype=torch.bfloat16)
    assert torch.equal(O.head_gate(out, big, 4), (2 * out.float()).to(torch.bfloat16))
    lg = _bf((2, 3, 4), 13, 3.0)
    # head h scales only its own slice
    lg2 = lg.clone()
    lg2[..., 1] = 0
    a, b = O.head_gate(out, lg, 4), O.head_gate(out, lg2, 4)
    assert torch.equal(b[..., 16:32], out[..., 16:32])
    assert torch.equal(a[..., :16], b[..., :16])


def test_gelu_tanh_matches_torch():
    x = _bf((1 << 16,), 14, 3.0)
    a, b = O.gelu_tanh(x), F.gelu(x, approximate="tanh")
    # Identical except deep in the negative tail (x < -5), where 1 + tanh
    # cancels and torch's vectorised tanh saturates to -1 one step earlier.
    same = a == b
    assert bool(same[x.float() > -5].all())
    assert (a.float() - b.float()).abs().max() < 1e-6
    # tanh approximation stays within 1e-3 of the exact (erf) GELU
    assert (O.gelu_tanh(x).float() - F.gelu(x.float())).abs().max() < 1e-2


def test_euler_step_and_x0_special_cases():
    s, d = _bf((2, 9, 128), 15), _bf((2, 9, 128), 16)
    # dt = 0 leaves the sample unchanged; denoised == sample gives zero velocity
    assert torch.equal(O.euler_step(s, d, 0.7, 0.0), s)
    assert torch.equal(O.euler_step(s, s, 0.7, -0.1), s)
    # sigma = 1, dt = -1: x + (d - x) = d up to the velocity rounding
    assert (O.euler_step(s, d, 1.0, -1.0).float() - d.float()).abs().max() <= 2.0**-5 * 4
    ts = torch.full((2, 1, 1), 0.0)
    assert torch.equal(O.x0(s, d, ts), s)
    ts1 = torch.ones(2, 1, 1)
    assert torch.equal(O.x0(s, d, ts1), torch.sub(s.float(), d.float()).to(torch.bfloat16))


def test_feature_norm_layout_and_norm():
    layers = [_bf((2, 3, 16), 40 + i) for i in range(3)]
    keep = torch.tensor([[1, 1, 0], [0, 1, 1]])
    o0, o1 = O.feature_norm(layers, keep, 1.0, 0.5)
    assert o0.shape == (2, 3, 48)
    # each layer's norm is the library RMSNorm, rounded once
    want = [F.rms_norm(x.float(), (16,), eps=1e-6).to(torch.bfloat16) for x in layers]
    for b in range(2):
        for t in range(3):
            for d in range(16):
                for l in range(3):
                    got0, got1 = o0[b, t, d * 3 + l], o1[b, t, d * 3 + l]
                    if keep[b, t]:
                        assert got0 == want[l][b, t, d]                        # scale 1: the normed value
                        assert got1 == (want[l][b, t, d].float() * 0.5).to(torch.bfloat16)
                    else:
                        assert got0.view(torch.int16) == 0 and got1.view(torch.int16) == 0  # +0


def test_guide_special_cases():
    c, u, p, m = (_bf((1, 40, 128), 20 + i) for i in range(4))
    # neutral scales give the cond prediction; passes equal to cond add nothing
    assert torch.equal(O.guide(c, u, p, m, 1.0, 0.0, 1.0, 0.0), c)
    assert torch.equal(O.guide(c, c, c, c, 3.0, 1.0, 3.0, 0.0), c)
    # direction and weight of each term, on exactly representable offsets
    z = torch.zeros(1, 4, 8, dtype=torch.bfloat16)
    def off(v):
        return torch.full_like(z, v)
    assert torch.equal(O.guide(z, off(-0.25), z, z, 3.0, 0.0, 1.0, 0.0), off(0.5))    # (cfg-1)(c-u)
    assert torch.equal(O.guide(z, z, off(-1.0), z, 1.0, 1.0, 1.0, 0.0), off(1.0))     # stg (c-p)
    assert torch.equal(O.guide(z, z, z, off(0.5), 1.0, 0.0, 2.0, 0.0), off(-0.5))     # (mod-1)(c-m)
    # rescale 1 with pred = 2c: std ratio exactly 1/2, so the output is c again
    assert torch.equal(O.guide(c, torch.zeros_like(c), c, c, 2.0, 0.0, 1.0, 1.0), c)
    # rescale 1 matches std(out) to std(c); the factor is linear in r
    d0 = O.guide(c, u, p, m, 3.0, 1.0, 3.0, 0.0).float()
    d1 = O.guide(c, u, p, m, 3.0, 1.0, 3.0, 1.0).float()
    dh = O.guide(c, u, p, m, 3.0, 1.0, 3.0, 0.5).float()
    assert abs(float(d1.std() / c.float().std()) - 1) < 5e-3
    assert ((dh - (d0 + d1) / 2).abs() <= 2.0**-7 * (d0.abs() + d1.abs()) + 1e-6).all()


def test_guided_step_composes():
    lat = _bf((1, 24, 64), 30)
    vel = _bf((4, 24, 64), 31)
    ts = torch.rand(4, 24, 1, generator=torch.Generator().manual_seed(32))
    den, nxt, x0s = O.guided_step(lat, vel, ts, 1.0, 0.0, 1.0, 0.0, 0.6, -0.05)
    assert torch.equal(x0s, O.x0(lat.repeat(4, 1, 1), vel, ts))
    assert torch.equal(den, x0s[:1])
    assert torch.equal(nxt, O.euler_step(lat, den, 0.6, -0.05))


# ---------------------------------------------------------------------------
# RoPE against the reference's own vectors
# ---------------------------------------------------------------------------

ROPE = np.load(GOLDEN / "rope_golden.npz")
ROPE_CASES = ["video", "video_small", "audio", "cross"]


@pytest.mark.parametrize("name", ROPE_CASES)
def test_rope_tables_match_reference(name):
    meta = ROPE[f"{name}_meta"]
    dim, heads = int(meta[0]), int(meta[1])
    max_pos = [int(m) for m in meta[2:]]
    pos = torch.from_numpy(ROPE[f"{name}_positions"])
    c, s = O.rope_tables(pos, dim, heads, max_pos)
    assert torch.equal(c.view(torch.int16), bf16_from_bits(ROPE[f"{name}_cos"]).view(torch.int16))
    assert torch.equal(s.view(torch.int16), bf16_from_bits(ROPE[f"{name}_sin"]).view(torch.int16))


@pytest.mark.parametrize("name", ROPE_CASES)
def test_rope_rotation_against_reference(name):
    """The reference rotates in eager bf16 (rounding after every op); the
    oracle rotates in fp32 and rounds once.  Same layout => small, bounded
    differences; a wrong half/sign/head mapping would be O(1)."""
    x = bf16_from_bits(ROPE[f"{name}_x"])
    want = bf16_from_bits(ROPE[f"{name}_rot"]).float()
    c, s = bf16_from_bits(ROPE[f"{name}_cos"]), bf16_from_bits(ROPE[f"{name}_sin"])
    got = O.apply_rope(x, c, s).float()
    # bound: two bf16 product roundings + one difference rounding in the reference
    b, t, d = x.shape
    h = c.shape[1]
    xr = x.float().view(b, t, h, 2, d // h // 2)
    mag = (xr[..., 0, :].abs() + xr[..., 1, :].abs()).unsqueeze(3).expand_as(xr).reshape(b, t, d)
    # unit roundoff 2^-8: two products, the difference, and the oracle's own rounding
    bound = 2.0**-8 * (mag + 2 * want.abs()) + 1e-6
    assert bool(((got - want).abs() <= bound).all())
    # most elements round identically (the rest differ by the eager roundings)
    assert (got == want).float().mean() > 0.5


def test_rope_invariants():
    pos = O.video_positions(1, 2, 2, 3, 24.0)
    c, s = O.rope_tables(pos, 256, 2, [20, 2048, 2048], out_dtype=torch.float32)
    # cos^2 + sin^2 = 1
    assert (c * c + s * s - 1).abs().max() < 1e-5
    # 256/6 -> 42 freqs per axis, 2 identity entries in front of head 0
    assert torch.all(c[:, 0, :, :2] == 1) and torch.all(s[:, 0, :, :2] == 0)
    # rotation preserves the norm of every (x1, x2) pair
    x = _bf((1, pos.shape[2], 256), 17)
    y = O.apply_rope(x, c.to(torch.bfloat16), s.to(torch.bfloat16))
    xr, yr = x.float().view(1, -1, 2, 2, 64), y.float().view(1, -1, 2, 2, 64)
    nx = xr[..., 0, :] ** 2 + xr[..., 1, :] ** 2
    ny = yr[..., 0, :] ** 2 + yr[..., 1, :] ** 2
    assert ((nx - ny).abs() <= 0.03 * nx + 1e-3).all()
    # a position at max_pos/2 has angle 0 on that axis: identity for those pairs
    mid = torch.tensor([[[[10.0, 10.0]]]])
    c1, s1 = O.rope_tables(mid, 64, 1, [20], out_dtype=torch.float32)
    assert torch.all(c1 == 1) and torch.all(s1 == 0)


@pytest.mark.parametrize("dim,n_axes", [(4096, 3), (2048, 1), (384, 3)])
def test_fp32_freq_grid_pins(dim, n_axes):
    """The fp32 frequency grid (checkpoints without float64 frequencies) has no
    reference vectors: pin it on the closed form.  theta**e for e = i/(n-1)
    rounds the exponent and the power in fp32, so every entry lies within a
    few ulp of the fp64 grid; the first entry is fp32(pi/2) exactly (theta**0
    = 1) and there are inner_dim // (2 n_axes) entries.  A wrong count, a
    missing pi/2, a reversed or fp64-cast exponent ramp all fail here."""
    g32 = O.freq_grid(1e4, n_axes, dim, double_precision=False)
    g64 = O.freq_grid(1e4, n_axes, dim)
    n = dim // (2 * n_axes)
    assert g32.dtype == torch.float32 and g32.shape == (n,)
    assert g32[0].item() == np.float32(math.pi / 2)
    want = np.pi / 2 * np.power(1e4, np.arange(n, dtype=np.float64) / (n - 1))
    rel = np.abs(g32.double().numpy() - want) / want
    # exponent rounding (<= 2^-24 * ln 1e4 relative) + power + product roundings
    assert rel.max() <= 16 * 2.0**-24
    # increasing, and a different rounding path from the fp64 grid
    assert bool((g32[1:] > g32[:-1]).all())
    if n > 100:
        assert not torch.equal(g32, g64)
    # a plausible slip: exponents computed in fp64 and cast gives the fp64 grid
    slip = torch.as_tensor(np.power(1e4, np.linspace(0, 1, n)) * np.pi / 2, dtype=torch.float32)
    assert n <= 100 or not torch.equal(slip, g32)


def test_fp32_grid_tables_stay_rotations():
    """Tables on the fp32 grid: cos^2 + sin^2 = 1, the identity padding, and
    within bf16 rounding of the fp64-grid tables (the grids differ by ulps)."""
    pos = O.video_positions(1, 3, 4, 5, 24.0)
    c32, s32 = O.rope_tables(pos, 4096, 32, [20, 2048, 2048], out_dtype=torch.float32, double_precision=False)
    c64, s64 = O.rope_tables(pos, 4096, 32, [20, 2048, 2048], out_dtype=torch.float32)
    assert (c32 * c32 + s32 * s32 - 1).abs().max() < 1e-5
    assert torch.all(c32[:, 0, :, :2] == 1) and torch.all(s32[:, 0, :, :2] == 0)
    # angles are at most |ind| <= 1e4*pi/2; a few-ulp grid change moves them by < 1e-2
    assert (c32 - c64).abs().max() < 2e-2 and (s32 - s64).abs().max() < 2e-2
    assert not torch.equal(c32, c64)


def test_positions_match_reference_vectors():
    for name, pos in (("video_small", O.video_positions(2, 3, 2, 2, 25.0)),
                      ("video", O.video_positions(1, 2, 3, 4, 24.0)),
                      ("audio", O.audio_positions(1, 10)),
                      ("cross", O.video_positions(1, 2, 2, 2, 24.0)[:, 0:1])):
        assert torch.equal(pos, torch.from_numpy(ROPE[f"{name}_positions"])), name


def test_qk_norm_rope_composes():
    x = _bf((1, 6, 256), 18)
    w = _bf((256,), 19)
    pos = O.video_positions(1, 1, 2, 3, 24.0)
    c, s = O.rope_tables(pos, 256, 2, [20, 2048, 2048])
    # no tables: exactly the weighted RMSNorm (library routine)
    assert torch.equal(O.qk_norm_rope(x, w, None, None), F.rms_norm(x, (256,), weight=w, eps=1e-6))
    # identity tables: same
    one, zero = torch.ones_like(c), torch.zeros_like(s)
    assert torch.equal(O.qk_norm_rope(x, w, one, zero), F.rms_norm(x, (256,), weight=w, eps=1e-6))
    # no weight: pure rotation of x
    assert torch.equal(O.qk_norm_rope(x, None, c, s), O.apply_rope(x, c, s))


# ---------------------------------------------------------------------------
# Model-level eager restatement (oracle/model_eager.py) against the outputs the
# reference's own LTXModel wrote (tests/golden/block_golden.npz)
# ---------------------------------------------------------------------------

BLOCKS = {"default": np.load(GOLDEN / "block_golden.npz"), "ltx2": np.load(GOLDEN / "block_golden_ltx2.npz")}
BLOCK = BLOCKS["default"]


def _golden_model_params(variant="default"):
    """The small model of the fixture: the DiTConfig defaults, or ("ltx2") the
    flags a checkpoint without them in its metadata gets (no cross-attention
    AdaLN, no attention gates)."""
    import importlib.util

    import ltx_dit

    spec = importlib.util.spec_from_file_location("make_block_golden", GOLDEN / "make_block_golden.py")
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    cfg = ltx_dit.DiTConfig(**mk.SMALL, **(mk.LTX2_FLAGS if variant == "ltx2" else {}))
    model = ltx_dit.LTXModel(cfg)
    assert sorted(n for n, _ in model.named_parameters()) == list(BLOCKS[variant]["param_names"])
    mk.init_weights(model)
    return cfg, {n: p.detach() for n, p in model.named_parameters()}


def _golden_modalities(key, variant="default"):
    from types import SimpleNamespace

    blk = BLOCKS[variant]
    g = {n: bf16_from_bits(blk[f"{key}_{n}"]) for n in ("vlat", "alat", "vctx", "actx")}
    g.update({n: torch.from_numpy(blk[f"{key}_{n}"]) for n in ("vpos", "apos", "kf", "sigma")})
    b = g["vlat"].shape[0]
    sig = g["sigma"].view(b, 1, 1)
    video = SimpleNamespace(latent=g["vlat"], sigma=g["sigma"], timesteps=torch.ones(b, g["vlat"].shape[1], 1) * sig,
                            positions=g["vpos"], context=g["vctx"], keyframes_mask=g["kf"])
    audio = SimpleNamespace(latent=g["alat"], sigma=g["sigma"], timesteps=torch.ones(b, g["alat"].shape[1], 1) * sig,
                            positions=g["apos"], context=g["actx"], keyframes_mask=None)
    return video, audio


@pytest.mark.parametrize("variant", ["default", "ltx2"])
@pytest.mark.parametrize("key,pert", [("b1", False), ("b4", True)])
@pytest.mark.parametrize("dtype,tag", [(torch.float32, "f32"), (torch.bfloat16, "bf16")])
def test_model_eager_matches_reference_outputs(variant, key, pert, dtype, tag):
    """On the CPU the restatement reproduces the reference's outputs to within
    1e-6 relative in both precisions (bit for bit with this torch): the same
    ops in the same order with the same roundings, with and without the
    cross-attention AdaLN and the attention gates."""
    tol = 1e-6
    import ltx_dit
    from oracle import model_eager

    cfg, params = _golden_model_params(variant)
    video, audio = _golden_modalities(key, variant)
    p = None
    if pert:
        p = ltx_dit.build_perturbation_config(cfg.num_layers, ["cond", "uncond", "ptb", "mod"], [1], [0],
                                              torch.device("cpu"), dtype)
    vx, ax = model_eager.forward(params, cfg, video, audio, p, dtype=dtype)
    for name, got in (("vx", vx), ("ax", ax)):
        want = torch.from_numpy(BLOCKS[variant][f"{key}_{name}_{tag}"])
        rel = float((got.float() - want).norm() / want.norm())
        assert rel < tol, f"{key} {name} {tag}: relative L2 {rel:.3g}"


@pytest.mark.parametrize("variant", ["default", "ltx2"])
@pytest.mark.parametrize("dis", ["video", "audio"])
@pytest.mark.parametrize("dtype,tag", [(torch.float32, "f32"), (torch.bfloat16, "bf16")])
def test_model_eager_disabled_stream(variant, dis, dtype, tag):
    """One stream disabled (Modality.enabled False): the restatement matches the
    reference's outputs for both streams to 1e-6, and the disabled case differs
    from the enabled one (the flag is not ignored)."""
    from oracle import model_eager

    cfg, params = _golden_model_params(variant)
    video, audio = _golden_modalities("b1", variant)
    (video if dis == "video" else audio).enabled = False
    vx, ax = model_eager.forward(params, cfg, video, audio, None, dtype=dtype)
    blk = BLOCKS[variant]
    for name, got in (("vx", vx), ("ax", ax)):
        want = torch.from_numpy(blk[f"b1_no{dis}_{name}_{tag}"])
        rel = float((got.float() - want).norm() / want.norm())
        assert rel < 1e-6, f"{variant} no{dis} {name} {tag}: relative L2 {rel:.3g}"
    moved = torch.from_numpy(blk[f"b1_no{dis}_{'vx' if dis == 'video' else 'ax'}_{tag}"])
    both = torch.from_numpy(blk[f"b1_{'vx' if dis == 'video' else 'ax'}_{tag}"])
    assert float((moved - both).norm() / both.norm()) > 1e-3


def test_model_eager_catches_a_swapped_modulation():
    """A plausible mistake (shift and scale of the first norm swapped) moves the
    output by ~2e-4 relative: far outside the 1e-6 bound above."""
    from oracle import model_eager

    cfg, params = _golden_model_params()
    video, audio = _golden_modalities("b1")
    want = torch.from_numpy(BLOCK["b1_vx_f32"])
    bad = dict(params)
    sst = params["blocks.0.scale_shift_table"].clone()
    bad["blocks.0.scale_shift_table"] = sst[[1, 0, 2, 3, 4, 5, 6, 7, 8]]
    vx, _ = model_eager.forward(bad, cfg, video, audio, None)
    assert float((vx - want).norm() / want.norm()) > 1e-5


def test_model_eager_ltx2_text_cross_is_live():
    """The ltx2 fixture exercises the ungated text cross-attention
    (ltx_dit.py:237-248): its model has 6-row tables and no prompt AdaLN or
    gate parameters, and zeroing that attention's output projection moves the
    output far beyond the 1e-6 bound above, so a dropped or mis-scaled text
    term fails the fixture check."""
    from oracle import model_eager

    cfg, params = _golden_model_params("ltx2")
    assert params["blocks.0.scale_shift_table"].shape[0] == 6
    assert not any("prompt" in n or "to_gate_logits" in n for n in params)
    video, audio = _golden_modalities("b1", "ltx2")
    want = torch.from_numpy(BLOCKS["ltx2"]["b1_vx_f32"])
    cut = dict(params)
    for i in range(cfg.num_layers):
        for leaf in ("weight", "bias"):
            name = f"blocks.{i}.attn2.to_out.{leaf}"
            cut[name] = params[name] * 0
    vx, _ = model_eager.forward(cut, cfg, video, audio, None)
    assert float((vx - want).norm() / want.norm()) > 1e-4


def test_model_tables_follow_double_rope():
    """The small fixtures cannot tell the RoPE grids apart (at 64-wide heads
    the fp32 and fp64 grids round to the same bf16 tables), so the grid
    precision is checked on the model's own tables at the video width: with
    double_rope False (the from_checkpoint default, ltx_dit.py:68) and True,
    the tables LTXModel builds (ltx_dit.py:160-170) expand to the oracle's
    tables of that grid precision bit for bit, and the two differ."""
    import dataclasses

    import ltx_dit

    pos = O.video_positions(1, 4, 6, 5, 24.0)
    got = {}
    for dp in (False, True):
        cfg = dataclasses.replace(ltx_dit.DiTConfig(), num_layers=1, double_rope=dp)
        with torch.device("meta"):
            model = ltx_dit.LTXModel(cfg)
        cp = model.video_pre.rope_tables(pos, cross=False).pe
        idx = cp.index.long()
        cos = torch.zeros_like(cp.cos[idx[..., 0]])
        sin = torch.zeros_like(cos)
        for a in range(cp.n_axes):  # OR of the axis rows: the full table's entries
            cos = (cos.view(torch.int16) | cp.cos[idx[..., a]].view(torch.int16)).view(torch.bfloat16)
            sin = (sin.view(torch.int16) | cp.sin[idx[..., a]].view(torch.int16)).view(torch.bfloat16)
        c, s_ = O.rope_tables(pos, 4096, 32, [20, 2048, 2048], double_precision=dp)
        c = c.transpose(1, 2).reshape(cos.shape)
        s_ = s_.transpose(1, 2).reshape(sin.shape)
        assert torch.equal(cos.view(torch.int16), c.view(torch.int16)), dp
        assert torch.equal(sin.view(torch.int16), s_.view(torch.int16)), dp
        got[dp] = cos
    assert not torch.equal(got[False].view(torch.int16), got[True].view(torch.int16))
