"""The C-ABI library builds, loads without a GPU and exports what the header declares.

No kernel is launched here: only entry points that reject their arguments
before touching the HIP runtime are called.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "techjam_attn.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tj_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_path_entry_points():
    names = declared_functions()
    for required in ("tj_attn_fwd", "tj_score_guard", "tj_poly_attn_fwd",
                     "tj_poly_workspace_bytes", "tj_error_string", "tj_abi_version"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from techjam_amd.kernels import _lib

    handle = _lib.lib()
    for name in declared_functions():
        assert hasattr(handle, name), name
    # and the binding describes each one
    assert set(declared_functions()) == set(_lib.SIGNATURES)


def test_error_strings_are_distinct_and_never_null():
    from techjam_amd.kernels import _lib

    texts = {_lib.error_text(c) for c in range(0, 8)}
    assert len(texts) == 8
    assert _lib.error_text(12345) == "unknown error"


def test_abi_version():
    from techjam_amd.kernels import _lib

    assert _lib.lib().tj_abi_version() == _lib.ABI_VERSION == 3


def _strides(*s):
    return (ctypes.c_int64 * 4)(*s)


def test_attn_proj_bias_rejects_bad_arguments_before_launching():
    from techjam_amd.kernels import _lib

    L = _lib.lib()
    st = _strides(64 * 128 * 4, 64, 64 * 4, 1)
    args = [16, 16, 16, 16]  # fake aligned pointers: never dereferenced on these paths
    f = L.tj_attn_fwd_proj_bias
    assert f(*args, 7, 1, 4, 128, 64, st, st, st, st, 0.125, 1, None, 16, 16, None) == _lib.TJ_ERR_DTYPE
    assert f(*args, _lib.TJ_F32, 1, 4, 128, 48, st, st, st, st, 0.125, 1, None, 16, 16, None) == _lib.TJ_ERR_UNSUPPORTED
    # bias pointers must be 16-byte aligned
    assert f(*args, _lib.TJ_F32, 1, 4, 128, 64, st, st, st, st, 0.125, 1, None, 20, 16, None) == _lib.TJ_ERR_ALIGN
    assert f(*args, _lib.TJ_F32, 1, 4, 128, 64, st, st, st, st, 0.125, 1, None, 16, 24, None) == _lib.TJ_ERR_ALIGN
    assert f(*args, _lib.TJ_F32, 0, 4, 128, 64, st, st, st, st, 0.125, 1, None, 16, 16, None) == _lib.TJ_OK


def test_attn_rejects_bad_arguments_before_launching():
    from techjam_amd.kernels import _lib

    L = _lib.lib()
    st = _strides(64 * 128 * 4, 64, 64 * 4, 1)
    args = [16, 16, 16, 16]  # fake aligned pointers: never dereferenced on these paths
    # unsupported dtype
    assert L.tj_attn_fwd(*args, 7, 1, 4, 128, 64, st, st, st, st, 0.125, 1, None, None, None, None) == _lib.TJ_ERR_DTYPE
    # unsupported head dim
    assert L.tj_attn_fwd(*args, _lib.TJ_F32, 1, 4, 128, 48, st, st, st, st, 0.125, 1, None, None, None, None) == _lib.TJ_ERR_UNSUPPORTED
    # negative sizes
    assert L.tj_attn_fwd(*args, _lib.TJ_F32, -1, 4, 128, 64, st, st, st, st, 0.125, 1, None, None, None, None) == _lib.TJ_ERR_SHAPE
    # grids beyond the 32-bit dispatch size: 2**20 (b, h) x 128 tiles x 256 threads >= 2**32
    assert L.tj_attn_fwd(*args, _lib.TJ_F16, 65536, 16, 32768, 32, st, st, st, st, 0.125, 1, None, None, None, None) == _lib.TJ_ERR_SHAPE
    # innermost stride != 1
    bad = _strides(64 * 128 * 4, 64, 64 * 4, 2)
    assert L.tj_attn_fwd(*args, _lib.TJ_F32, 1, 4, 128, 64, bad, st, st, st, 0.125, 1, None, None, None, None) == _lib.TJ_ERR_ALIGN
    # misaligned base pointer
    assert L.tj_attn_fwd(4, 16, 16, 16, _lib.TJ_F32, 1, 4, 128, 64, st, st, st, st, 0.125, 1, None, None, None, None) == _lib.TJ_ERR_ALIGN
    # row stride not a multiple of 16 bytes
    odd = _strides(64 * 128 * 4, 64, 66, 1)
    assert L.tj_attn_fwd(*args, _lib.TJ_F32, 1, 4, 128, 64, st, odd, st, st, 0.125, 1, None, None, None, None) == _lib.TJ_ERR_ALIGN
    # empty problems are a successful no-op
    assert L.tj_attn_fwd(*args, _lib.TJ_F32, 0, 4, 128, 64, st, st, st, st, 0.125, 1, None, None, None, None) == _lib.TJ_OK
    # K/V rows of one (b, h) must span less than 2 GiB (31-bit buffer offsets)...
    huge = _strides(64 * 128 * 4, 64, 1 << 23, 1)
    assert L.tj_attn_fwd(*args, _lib.TJ_F32, 1, 4, 128, 64, st, huge, st, st, 0.125, 1, None, None, None, None) == _lib.TJ_ERR_UNSUPPORTED
    assert L.tj_attn_fwd(*args, _lib.TJ_F32, 1, 4, 128, 64, st, st, huge, st, 0.125, 1, None, None, None, None) == _lib.TJ_ERR_UNSUPPORTED
    # ... and run forward in memory
    back = _strides(64 * 128 * 4, 64, -64 * 4, 1)
    assert L.tj_attn_fwd(*args, _lib.TJ_F32, 1, 4, 128, 64, st, back, st, st, 0.125, 1, None, None, None, None) == _lib.TJ_ERR_UNSUPPORTED


def test_guard_rejects_bad_arguments_before_launching():
    from techjam_amd.kernels import _lib

    L = _lib.lib()
    st = _strides(64 * 128 * 4, 64, 64 * 4, 1)
    # more samples than rows
    assert L.tj_score_guard(16, 16, _lib.TJ_F32, 1, 4, 128, 64, st, st, 0.125, 16, 256, 0.4, 64,
                            None, None, None, 16, None, None, None, 16, 1 << 20, None) == _lib.TJ_ERR_SHAPE
    # missing flags output
    assert L.tj_score_guard(16, 16, _lib.TJ_F32, 1, 4, 128, 64, st, st, 0.125, 16, 64, 0.4, 64,
                            None, None, None, None, None, None, None, 16, 1 << 20, None) == _lib.TJ_ERR_SHAPE
    assert L.tj_score_guard(16, 16, _lib.TJ_F32, 1, 4, 128, 256, st, st, 0.125, 16, 64, 0.4, 64,
                            None, None, None, 16, None, None, None, 16, 1 << 20, None) == _lib.TJ_ERR_UNSUPPORTED
    # workspace: missing, too small, misaligned
    need = L.tj_score_guard_workspace_bytes(1, 4, 64)
    assert need == 1 * 4 * 1 * 3 * 8
    assert L.tj_score_guard_workspace_bytes(1, 4, 512) == 4 * 8 * 3 * 8
    assert L.tj_score_guard_workspace_bytes(0, 4, 512) == 0
    for ws, nbytes in ((None, need), (16, need - 8), (24, need)):
        assert L.tj_score_guard(16, 16, _lib.TJ_F32, 1, 4, 128, 64, st, st, 0.125, 16, 64, 0.4, 64,
                                None, None, None, 16, None, None, None, ws, nbytes, None) == _lib.TJ_ERR_WORKSPACE
    # rows must be 4-element aligned for the gathers
    odd = _strides(64 * 128 * 4, 64, 66, 1)
    assert L.tj_score_guard(16, 16, _lib.TJ_F32, 1, 4, 128, 64, odd, st, 0.125, 16, 64, 0.4, 64,
                            None, None, None, 16, None, None, None, 16, need, None) == _lib.TJ_ERR_ALIGN


def test_check_maps_codes_to_reference_exceptions():
    from techjam_amd.errors import UnsupportedCaseError
    from techjam_amd.kernels import _lib

    _lib.check(_lib.TJ_OK, "x")
    for code in (_lib.TJ_ERR_SHAPE, _lib.TJ_ERR_DTYPE, _lib.TJ_ERR_ALIGN, _lib.TJ_ERR_WORKSPACE):
        with pytest.raises(ValueError):
            _lib.check(code, "x")
    with pytest.raises(UnsupportedCaseError):
        _lib.check(_lib.TJ_ERR_UNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.TJ_ERR_LAUNCH, "x")


def test_cpu_tensors_are_refused_not_computed():
    import torch

    from techjam_amd.errors import UnsupportedCaseError
    from techjam_amd.kernels import scaled_dot_product_attention

    q = torch.randn(1, 2, 16, 64)
    with pytest.raises(UnsupportedCaseError):
        scaled_dot_product_attention(q, q, q, is_causal=True)


def _s3(*s):
    return (ctypes.c_int64 * 3)(*s)


def test_poly_parts_reject_bad_arguments_before_launching():
    from techjam_amd.kernels import _lib

    L = _lib.lib()
    st = _s3(128 * 64, 64, 1)
    ss = _s3(4096 * 64, 64, 1)
    # the kernels are written for D = V = 64
    assert L.tj_quad_apply(16, 16, 16, _lib.TJ_F32, 2, 128, 32, 64, st, ss, st, None) == _lib.TJ_ERR_UNSUPPORTED
    assert L.tj_quad_apply(16, 16, 16, 9, 2, 128, 64, 64, st, ss, st, None) == _lib.TJ_ERR_DTYPE
    assert L.tj_quad_apply(16, 16, 16, _lib.TJ_F32, -1, 128, 64, 64, st, ss, st, None) == _lib.TJ_ERR_SHAPE
    assert L.tj_quad_apply(16, 16, 16, _lib.TJ_F32, 0, 128, 64, 64, st, ss, st, None) == _lib.TJ_OK
    assert L.tj_quad_apply(8, 16, 16, _lib.TJ_F32, 2, 128, 64, 64, st, ss, st, None) == _lib.TJ_ERR_ALIGN
    assert L.tj_quad_apply(16, 16, 16, _lib.TJ_F32, 2, 128, 64, 64, _s3(128 * 64, 65, 1), ss, st, None) == _lib.TJ_ERR_ALIGN
    assert L.tj_quad_update(16, 16, 16, None, 2, 128, 64, 32, st, st, ss, None, None) == _lib.TJ_ERR_UNSUPPORTED
    assert L.tj_quad_update(16, 16, 16, None, 2, 128, 64, 64, st, st, _s3(4096 * 64, 64, 2), None, None) == _lib.TJ_ERR_ALIGN
    assert L.tj_quad_update(16, 16, 16, 24, 2, 128, 64, 64, st, st, ss, ss, None) == _lib.TJ_ERR_ALIGN
    assert L.tj_causal_diag(16, 16, 16, 16, 16, 2, 128, 64, 64, st, st, st, st, 127, None) == _lib.TJ_ERR_SHAPE
    assert L.tj_causal_diag(16, 16, 16, 16, None, 2, 128, 64, 64, st, st, st, st, 128, None) == _lib.TJ_ERR_ALIGN
    assert L.tj_causal_diag(16, 16, 16, 16, 16, 2, 128, 48, 64, st, st, st, st, 128, None) == _lib.TJ_ERR_UNSUPPORTED


def test_poly_parts_refuse_cpu_tensors():
    import torch

    from techjam_amd.errors import UnsupportedCaseError
    from techjam_amd.kernels.poly_parts import causal_diag, quad_apply, quad_update

    a = torch.zeros(2, 128, 64, dtype=torch.float16)
    with pytest.raises(UnsupportedCaseError):
        quad_apply(a, torch.zeros(2, 4096, 64))
    with pytest.raises(UnsupportedCaseError):
        quad_update(a, a, torch.zeros(2, 4096, 64))
    with pytest.raises(UnsupportedCaseError):
        causal_diag(a, a, a)


def test_block_tails_reject_bad_arguments_before_launching():
    from techjam_amd.kernels import _lib

    L = _lib.lib()
    assert L.tj_bias_residual(16, 16, 16, 16, 4, 6, 2, None, 0, None) == _lib.TJ_ERR_UNSUPPORTED
    assert L.tj_bias_residual(16, 16, 16, 16, 4, 8, 2, None, 3, None) == _lib.TJ_ERR_SHAPE
    assert L.tj_bias_residual(16, 16, 16, 16, 5, 8, 2, 16, 1, None) == _lib.TJ_ERR_SHAPE
    assert L.tj_bias_residual(16, 24, 16, 16, 4, 8, 2, None, 0, None) == _lib.TJ_ERR_ALIGN
    assert L.tj_bias_residual(16, 16, 16, 16, 0, 8, 2, None, 0, None) == _lib.TJ_OK
    assert L.tj_bias_gelu(16, 16, 4, 6, None, None) == _lib.TJ_ERR_UNSUPPORTED
    assert L.tj_bias_gelu(8, 16, 4, 8, None, None) == _lib.TJ_ERR_ALIGN
    assert L.tj_bias_gelu(16, 16, -1, 8, None, None) == _lib.TJ_ERR_SHAPE
    assert L.tj_bias_gelu(16, 16, 4, 8, 20, None) == _lib.TJ_ERR_ALIGN       # fp16 output 8-byte aligned
    assert L.tj_bias_gelu(16, 16, 4, 8, 64, None) == _lib.TJ_ERR_SHAPE       # overlaps y
    assert L.tj_bias_relu(16, 16, 4, 6, None, None) == _lib.TJ_ERR_UNSUPPORTED
    assert L.tj_bias_relu(8, 16, 4, 8, None, None) == _lib.TJ_ERR_ALIGN
    assert L.tj_bias_relu(16, 16, 4, 8, 64, None) == _lib.TJ_ERR_SHAPE       # overlaps y
    assert L.tj_bias_relu(16, 16, 0, 8, None, None) == _lib.TJ_OK
    # tj_bias_residual_layernorm(out, ln_out, ln_dtype, x, y, bias, gamma, beta, rows, cols, seq_len,
    # valid_len, mode, eps, zero_ln_padded, stream) on 4 x 256 fp32 rows (4 KiB): out may be null,
    # the norm output may overlap nothing else
    ln = L.tj_bias_residual_layernorm
    x, y, g = 1 << 20, 1 << 21, 1 << 22
    assert ln(None, None, _lib.TJ_F32, x, y, g, g, g, 4, 256, 4, None, 0, 1e-5, 0, None) == _lib.TJ_ERR_SHAPE
    assert ln(None, x + 2048, _lib.TJ_F32, x, y, g, g, g, 4, 256, 4, None, 0, 1e-5, 0, None) == _lib.TJ_ERR_SHAPE
    assert ln(None, y, _lib.TJ_F16, x, y, g, g, g, 4, 256, 4, None, 0, 1e-5, 0, None) == _lib.TJ_ERR_SHAPE
    o = 1 << 23
    assert ln(o, o + 2048, _lib.TJ_F32, x, y, g, g, g, 4, 256, 4, None, 0, 1e-5, 0, None) == _lib.TJ_ERR_SHAPE
    assert ln(None, g, _lib.TJ_F32, x, y, g, g, g, 4, 384, 4, None, 0, 1e-5, 0, None) == _lib.TJ_ERR_UNSUPPORTED
    assert ln(None, g + 8, _lib.TJ_F32, x, y, g, g, g, 4, 256, 4, None, 0, 1e-5, 0, None) == _lib.TJ_ERR_ALIGN


def test_noalloc_guard_rejects_requests_beyond_its_scratch_before_launching():
    """tj_score_guard_noalloc checks its arguments, then the size of its fixed
    scratch, before any HIP call (so these run without a GPU)."""
    from techjam_amd.kernels import _lib

    L = _lib.lib()
    f = L.tj_score_guard_noalloc
    st = _strides(16 * 4096 * 64, 4096 * 64, 64, 1)
    outs = [16] * 7
    # 6000 (b, h) x 8 row blocks x 24 bytes = 1.15 MB > 1 MiB
    assert f(16, 16, _lib.TJ_F32, 375, 16, 4096, 64, st, st, 0.125, 16, 512, 0.4, 4096, *outs, None) == \
        _lib.TJ_ERR_SCRATCH
    assert f(16, 16, 9, 1, 16, 4096, 64, st, st, 0.125, 16, 512, 0.4, 4096, *outs, None) == _lib.TJ_ERR_DTYPE
    assert f(16, 16, _lib.TJ_F32, 1, 16, 100, 64, st, st, 0.125, 16, 512, 0.4, 4096, *outs, None) == \
        _lib.TJ_ERR_SHAPE  # more samples than rows
    assert f(16, 16, _lib.TJ_F32, 1, 16, 4096, 66, st, st, 0.125, 16, 512, 0.4, 4096, *outs, None) == \
        _lib.TJ_ERR_UNSUPPORTED
    # the same request through the workspace entry point is limited only by its workspace
    g = L.tj_score_guard
    assert g(16, 16, _lib.TJ_F32, 375, 16, 4096, 64, st, st, 0.125, 16, 512, 0.4, 4096, *outs, None, 0, None) == \
        _lib.TJ_ERR_WORKSPACE
    assert L.tj_score_guard_workspace_bytes(5461, 1, 512) <= 1 << 20 < L.tj_score_guard_workspace_bytes(5462, 1, 512)
