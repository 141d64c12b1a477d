"""ctypes binding of ``libtechjam_attn.so`` (the C ABI of ``include/techjam_attn.h``).

The library is loaded lazily from ``techjam_amd/lib``. A missing library is an
error, never a reason to compute something else: every caller of ``lib()``
fails loudly with instructions to build it.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

from ..errors import UnsupportedCaseError

LIB_PATH = Path(__file__).resolve().parents[1] / "lib" / "libtechjam_attn.so"

TJ_OK = 0
TJ_ERR_SHAPE = 1
TJ_ERR_DTYPE = 2
TJ_ERR_ALIGN = 3
TJ_ERR_UNSUPPORTED = 4
TJ_ERR_LAUNCH = 5
TJ_ERR_WORKSPACE = 6
TJ_ERR_SCRATCH = 7

TJ_F32 = 0
TJ_F16 = 1

#: The C ABI these bindings describe (tj_abi_version); a library built from
#: other sources is refused at load time.
ABI_VERSION = 3

_i64 = ctypes.c_int64
_i64p = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p
_f32 = ctypes.c_float
_int = ctypes.c_int

# name -> (restype, argtypes); one entry per declaration of the header.
SIGNATURES = {
    "tj_abi_version": (_int, []),
    "tj_error_string": (ctypes.c_char_p, [_int]),
    "tj_attn_fwd": (
        _int,
        [_vp, _vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _i64p, _i64p, _i64p, _i64p,
         _f32, _int, _vp, _vp, _vp, _vp],
    ),
    "tj_attn_fwd_proj_bias": (
        _int,
        [_vp, _vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _i64p, _i64p, _i64p, _i64p,
         _f32, _int, _vp, _vp, _vp, _vp],
    ),
    "tj_score_guard": (
        _int,
        [_vp, _vp, _int, _i64, _i64, _i64, _i64, _i64p, _i64p, _f32, _vp, _i64, _f32, _i64,
         _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp],
    ),
    "tj_score_guard_noalloc": (
        _int,
        [_vp, _vp, _int, _i64, _i64, _i64, _i64, _i64p, _i64p, _f32, _vp, _i64, _f32, _i64,
         _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    ),
    "tj_score_guard_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64]),
    "tj_poly_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64, _i64, _i64]),
    "tj_poly_attn_fwd": (
        _int,
        [_vp, _vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _i64p, _i64p, _i64p, _i64p,
         _f32, _i64, _i64, _vp, _vp, _vp, ctypes.c_size_t, _vp],
    ),
    "tj_bias_residual": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _int, _vp]),
    "tj_bias_gelu": (_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "tj_bias_relu": (_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "tj_bias_residual_layernorm": (
        _int,
        [_vp, _vp, _int, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _int, _f32, _int, _vp],
    ),
    "tj_quad_apply": (
        _int,
        [_vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _i64p, _i64p, _i64p, _vp],
    ),
    "tj_quad_update": (
        _int,
        [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64p, _i64p, _i64p, _i64p, _vp],
    ),
    "tj_causal_diag": (
        _int,
        [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64p, _i64p, _i64p, _i64p, _i64, _vp],
    ),
}

_lock = threading.Lock()
_lib = None


class LibraryMissingError(RuntimeError):
    """The HIP library has not been built, or a symbol is missing from it."""


def lib() -> ctypes.CDLL:
    """The loaded library with argument types set; raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise LibraryMissingError(
                    f"{LIB_PATH} is missing: build it with `python -m techjam_amd.build` "
                    "(the attention hot path has no non-HIP implementation)"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                try:
                    fn = getattr(handle, name)
                except AttributeError as err:
                    raise LibraryMissingError(f"{LIB_PATH} does not export {name}") from err
                fn.restype = res
                fn.argtypes = args
            version = handle.tj_abi_version()
            if version != ABI_VERSION:
                raise LibraryMissingError(
                    f"{LIB_PATH} has C ABI version {version}, these bindings expect {ABI_VERSION}: "
                    "rebuild it with `python -m techjam_amd.build`")
            _lib = handle
    return _lib


def error_text(code: int) -> str:
    return lib().tj_error_string(code).decode()


def check(code: int, what: str) -> None:
    """Map a C-ABI return code onto the reference's exception conventions.

    Shape, dtype, alignment and workspace problems are ``ValueError``
    (``poly_attention_triton.py:433-436``); unimplemented configurations are
    ``UnsupportedCaseError``; a rejected launch is ``RuntimeError``.
    """
    if code == TJ_OK:
        return
    msg = f"{what}: {error_text(code)} (code {code})"
    if code in (TJ_ERR_SHAPE, TJ_ERR_DTYPE, TJ_ERR_ALIGN, TJ_ERR_WORKSPACE, TJ_ERR_SCRATCH):
        raise ValueError(msg)
    if code == TJ_ERR_UNSUPPORTED:
        raise UnsupportedCaseError(msg)
    raise RuntimeError(msg)


def strides4(t) -> ctypes.Array:
    return (ctypes.c_int64 * 4)(*t.stride())
