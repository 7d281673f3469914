"""C-ABI surface checks that need no GPU: the library loads, exports every
function include/ltxk.h declares, the host-side helpers agree with the
oracle, argument errors come back as codes (never an exit), and the Python
binding refuses CPU tensors instead of computing anything on the host."""

import ctypes
import re

import pytest
import torch

from conftest import REPO
from oracle import oracle as O

HEADER = (REPO / "include" / "ltxk.h").read_text()


def declared_functions():
    body = re.sub(r"/\*.*?\*/", "", HEADER, flags=re.S)
    return sorted(set(re.findall(r"\b(ltxk_[a-z0-9_]+)\s*\(", body)))


def test_header_declares_the_path():
    names = declared_functions()
    for required in ("ltxk_philox_normal", "ltxk_philox_u32", "ltxk_euler_update", "ltxk_norm_modulate",
                     "ltxk_add_norm_modulate", "ltxk_qk_norm_rope", "ltxk_gelu_tanh", "ltxk_gated_residual",
                     "ltxk_head_gate", "ltxk_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    import ltxk

    lib = ltxk.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # the binding's signature table covers the header exactly
    assert sorted(ltxk.SIGNATURES) == declared_functions()


def test_version_and_error_string():
    import ltxk

    lib = ltxk.load()
    want = int(re.search(r"#define LTXK_VERSION (\d+)", HEADER).group(1))
    assert lib.ltxk_version() == want == ltxk.ABI_VERSION
    assert isinstance(ltxk.last_error(), str)


def test_host_policy_helpers_match_oracle():
    import ltxk

    for n in (1, 255, 256, 8704, 442368, 786432, 1 << 28):
        for sms, thr in ((142, 1536), (256, 2048), (304, 2048)):
            assert ltxk.policy_threads(n, sms, thr) == O.policy_threads(n, sms, thr)
    for n, t in ((442368, 218112), (8704, 8704), (786432, 524288), (1, 256), (0, 256)):
        assert ltxk.offset_advance(n, t) == O.offset_advance(n, t)


def test_argument_errors_return_codes_without_touching_the_device():
    import ltxk

    lib = ltxk.load()
    # null output with n > 0
    assert lib.ltxk_philox_normal(None, 0, 16, 1, 0, 256, None) == ltxk.E_ARG
    assert "null" in ltxk.last_error()
    # offset not a multiple of 4
    assert lib.ltxk_philox_u32(ctypes.c_void_p(16), 16, 1, 2, 256, None) == ltxk.E_ARG
    assert "offset" in ltxk.last_error()
    # bad dtype code
    assert lib.ltxk_philox_normal(ctypes.c_void_p(16), 7, 16, 1, 0, 256, None) == ltxk.E_DTYPE
    # dim not a multiple of 8
    assert lib.ltxk_norm_modulate(ctypes.c_void_p(16), None, ctypes.c_void_p(16), 4, 4, 12, 0, 1e-6,
                                  None, None, None, None, None) == ltxk.E_ARG
    # misaligned buffer
    assert lib.ltxk_gelu_tanh(ctypes.c_void_p(18), ctypes.c_void_p(16), 64, None) == ltxk.E_ALIGN
    # head_dim not a multiple of 16 for RoPE
    q = ltxk.QK(16, None, None, None, 1, 4, 0)
    assert lib.ltxk_qk_norm_rope(ctypes.byref(q), None, 4, 24, 1e-6, None) == ltxk.E_ARG
    # compact tables: 1..3 position axes, and an index needs tables
    q = ltxk.QK(16, None, 16, 16, 1, 4, 0, 16, 4, 8)
    assert lib.ltxk_qk_norm_rope(ctypes.byref(q), None, 4, 32, 1e-6, None) == ltxk.E_ARG
    q = ltxk.QK(16, None, None, None, 1, 4, 0, 16, 1, 8)
    assert lib.ltxk_qk_norm_rope(ctypes.byref(q), None, 4, 32, 1e-6, None) == ltxk.E_ARG
    # compact tables need their row count (the kernel clamps indexes into it)
    q = ltxk.QK(16, None, 16, 16, 1, 4, 0, 16, 1, 0)
    assert lib.ltxk_qk_norm_rope(ctypes.byref(q), None, 4, 32, 1e-6, None) == ltxk.E_ARG
    assert "table_rows" in ltxk.last_error()
    # one-wave-per-row launches (rows of 2048, 64-wide heads, one-axis tables; the
    # text q/k norm) count rows in int with a few wave strides of headroom: a count
    # within 2^20 of 2^31 is refused before any launch
    near = 0x7FFFFFFF - (1 << 20) + 1
    q = ltxk.QK(16, 16, 16, 16, 1, near, 0, 16, 1, 8)
    assert lib.ltxk_qk_norm_rope(ctypes.byref(q), None, 32, 64, 1e-6, None) == ltxk.E_ARG
    assert "too many rows" in ltxk.last_error()
    q = ltxk.QK(16, 16, None, None, 1, near, 0)
    assert lib.ltxk_qk_norm_rope(ctypes.byref(q), None, 32, 128, 1e-6, None) == ltxk.E_ARG
    assert "too many rows" in ltxk.last_error()
    # feature_norm: layer count 1..64, dim a multiple of 8, aligned layers
    ptrs = (ctypes.c_void_p * 1)(16)
    assert lib.ltxk_feature_norm(ctypes.c_void_p(16), None, ptrs, 0, None, 4, 64, 1e-6, 1.0, 1.0, None) == ltxk.E_ARG
    ptrs65 = (ctypes.c_void_p * 65)(*([16] * 65))
    assert lib.ltxk_feature_norm(ctypes.c_void_p(16), None, ptrs65, 65, None, 4, 64, 1e-6, 1.0, 1.0,
                                 None) == ltxk.E_ARG
    assert lib.ltxk_feature_norm(ctypes.c_void_p(16), None, ptrs, 1, None, 4, 60, 1e-6, 1.0, 1.0, None) == ltxk.E_ARG
    bad = (ctypes.c_void_p * 1)(24)
    assert lib.ltxk_feature_norm(ctypes.c_void_p(16), None, bad, 1, None, 4, 64, 1e-6, 1.0, 1.0, None) == ltxk.E_ALIGN
    # guide: rescale needs the workspace ltxk_guide_workspace_bytes states
    g = ltxk.Guidance(3.0, 1.0, 3.0, 0.7)
    assert lib.ltxk_guide(ctypes.c_void_p(16), None, None, ctypes.c_void_p(16), ctypes.c_void_p(16),
                          ctypes.c_void_p(16), 64, 1, 64, 128, ctypes.byref(g), 0.5, -0.1, None, 0,
                          None) == ltxk.E_ARG
    assert 32 <= lib.ltxk_guide_workspace_bytes(64 * 128) <= 8192
    # attn_combine: parts a power of two up to 16, aligned partials
    p16 = ctypes.c_void_p(16)
    assert lib.ltxk_attn_combine(p16, p16, 64, 64, 64, 64, p16, 1, 1, 1, 1, None, 1, 3, 4, 2, 64, None) == ltxk.E_ARG
    assert "power of two" in ltxk.last_error()
    assert lib.ltxk_attn_combine(p16, p16, 64, 64, 64, 64, p16, 1, 1, 1, 1, None, 1, 32, 4, 2, 64, None) == ltxk.E_ARG
    assert lib.ltxk_attn_combine(p16, ctypes.c_void_p(24), 64, 64, 64, 64, p16, 1, 1, 1, 1, None, 1, 8, 4, 2, 64,
                                 None) == ltxk.E_ALIGN
    assert lib.ltxk_attn_combine(p16, p16, 64, 60, 64, 64, p16, 1, 1, 1, 1, None, 1, 8, 4, 2, 64, None) == ltxk.E_ALIGN
    assert lib.ltxk_attn_combine(p16, p16, 64, 64, 64, 64, p16, 1, 1, 1, 1, None, 1, 8, 4, 2, 60, None) == ltxk.E_ARG
    # empty work is a no-op success
    assert lib.ltxk_gelu_tanh(None, None, 0, None) == 0
    assert lib.ltxk_attn_combine(None, None, 0, 0, 0, 0, None, 0, 0, 0, 0, None, 1, 8, 0, 2, 64, None) == 0


def test_binding_refuses_cpu_tensors():
    import ltxk

    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm device"):
        ltxk.gelu_tanh(x)
    with pytest.raises(RuntimeError, match="ROCm device"):
        ltxk.norm_modulate(x)
    with pytest.raises(RuntimeError, match="ROCm device"):
        ltxk.philox_normal(torch.zeros(16), 1, 0, 256)


def test_product_modules_import_without_a_gpu():
    import ltx_dit
    import ltx_nn

    cfg = ltx_dit.DiTConfig()
    assert cfg.video_dim == 4096 and cfg.audio_dim == 2048
    assert hasattr(ltx_nn, "apply_split_rotary_emb") and hasattr(ltx_dit, "create_noised_states")
    s = ltx_dit.ltx2_scheduler_sigmas(8)
    assert abs(float(s[0]) - 1.0) < 1e-6 and s[-1] == 0.0 and bool((s[1:] <= s[:-1]).all())


def test_empty_work_returns_ok_without_touching_the_device():
    """Zero rows / elements is a successful no-op for every entry point (no HIP
    call is made, so this runs on a host without a GPU)."""
    import ltxk

    lib = ltxk.load()
    p = ctypes.c_void_p(16)
    assert lib.ltxk_philox_normal(p, 0, 0, 1, 0, 256, None) == 0
    assert lib.ltxk_philox_u32(p, 0, 1, 0, 256, None) == 0
    assert lib.ltxk_euler_update(p, p, 0, 0, ctypes.c_float(0.1), None) == 0
    assert lib.ltxk_euler_step(p, p, p, 0, 1, 0.5, -0.1, None) == 0
    assert lib.ltxk_x0(p, p, p, p, 0, 1, 0, 1, 64, None) == 0
    assert lib.ltxk_rms_norm(p, p, None, 0, 64, 1e-6, None) == 0
    assert lib.ltxk_norm_modulate(p, None, p, 0, 1, 64, 0, 1e-6, None, None, None, None, None) == 0
    assert lib.ltxk_add_norm_modulate(p, p, None, p, p, None, None, 0, 1, 64, 1e-6, None, None, None, None,
                                      None) == 0
    assert lib.ltxk_modulate(p, p, 0, 1, 64, None, None, None) == 0
    assert lib.ltxk_gated_residual(p, p, p, None, None, 0, 1, 64, None) == 0
    assert lib.ltxk_head_gate(p, p, 0, 0, 0, p, None, None, 0, 1, 2, 32, None) == 0
    q = ltxk.QK(16, None, None, None, 0, 4, 0)
    assert lib.ltxk_qk_norm_rope(ctypes.byref(q), None, 2, 32, 1e-6, None) == 0
    g = ltxk.Guidance(3.0, 1.0, 3.0, 0.7)
    assert lib.ltxk_guide(p, None, None, p, p, p, 0, 1, 0, 128, ctypes.byref(g), 0.5, -0.1, None, 0, None) == 0
    ptrs = (ctypes.c_void_p * 1)(16)
    assert lib.ltxk_feature_norm(p, None, ptrs, 1, None, 0, 64, 1e-6, 1.0, 1.0, None) == 0


def test_noalloc_guide_rejects_oversize_before_any_device_call():
    """ltxk_guide_noalloc checks the size against its array before it looks up
    the array's address, so the refusal needs no device (the pointers are never
    dereferenced)."""
    import ltxk

    lib = ltxk.load()
    gp = ltxk.Guidance(3.0, 1.0, 3.0, 0.7)
    p = ctypes.c_void_p(256)
    rc = lib.ltxk_guide_noalloc(p, None, None, p, p, None, 0, 0, (1 << 28) // 64 + 1, 64, ctypes.byref(gp), 0.5,
                                -0.1, None)
    assert rc == ltxk.E_ARG and "2^28" in ltxk.last_error()
