"""The reference's kernel-level polynomial API on the stand-alone HIP kernels.

Same names, arguments, results and errors as ``quad_apply``, ``quad_update``
and ``causal_diag`` in ``src/kernels/poly_attention_triton.py:420-591``:

* ``quad_apply(a, s)``: ``phi2(a) @ s`` for ``a`` ``[M, C, D]`` and ``s``
  ``[M, D*D, V]`` (fp32 master or fp16 shadow; the state is rounded to fp16
  before the products either way), returned in ``a``'s dtype;
* ``quad_update(b, v, out, shadow=None)``: ``out += phi2(b)^T @ v`` in place on
  an fp32 ``[M, D*D, V]`` master (``ValueError`` for any other dtype), with the
  optional fp16 ``shadow`` set to the updated master rounded;
* ``causal_diag(a, b, v)``: ``w = tril(exp(a @ b^T))`` (no max subtraction),
  returning ``(w @ v, w.sum(-1, keepdim=True))`` in fp32.

The kernels are written for ``D = V = 64`` (the extreme-length
configuration); narrower heads and value widths are zero-padded to 64 here,
which leaves every product unchanged. The fused ``poly_rows`` path does not go
through these functions.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from ..errors import UnsupportedCaseError
from . import _lib
from .attention import _require_device, _stream_ptr

_W = 64  # head dim and value width of the kernels


def _strides3(t: torch.Tensor) -> ctypes.Array:
    return (ctypes.c_int64 * 3)(*t.stride())


def _half_rows(t: torch.Tensor) -> torch.Tensor:
    """fp16, unit innermost stride, 16-byte aligned rows (copies only when needed)."""
    t = t.to(torch.float16)
    if t.stride(-1) != 1 or any(st % 8 for st in t.stride()[:-1]) or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def _pad_last(t: torch.Tensor, width: int, dtype: torch.dtype) -> torch.Tensor:
    if t.shape[-1] == width:
        return _half_rows(t) if dtype == torch.float16 else t
    out = torch.zeros(*t.shape[:-1], width, dtype=dtype, device=t.device)
    out[..., : t.shape[-1]] = t
    return out


def _check_dims(d: int, vw: int) -> None:
    if d > _W or vw > _W or d < 1 or vw < 1:
        raise UnsupportedCaseError(f"head dim {d} / value width {vw}: the kernels handle up to {_W}")


def _pad_state(s: torch.Tensor, d: int, vw: int, dtype: torch.dtype) -> torch.Tensor:
    """[M, d*d, vw] -> [M, 64*64, 64] with feature (i, j) at row 64 i + j."""
    m = s.shape[0]
    out = torch.zeros(m, _W, _W, _W, dtype=dtype, device=s.device)
    out[:, :d, :d, :vw] = s.reshape(m, d, d, vw)
    return out.reshape(m, _W * _W, _W)


def quad_apply(a: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """``phi2(a) @ s`` without materialising ``phi2(a)``."""
    dev = _require_device(a, s)
    if a.dim() != 3 or s.dim() != 3:
        raise ValueError(f"a must be [M, C, D] and s [M, D*D, V]; got {tuple(a.shape)}, {tuple(s.shape)}")
    m, c, d = a.shape
    if s.shape[0] != m or s.shape[1] != d * d:
        raise ValueError(f"state shape {tuple(s.shape)} does not match a {tuple(a.shape)}")
    if s.dtype not in (torch.float32, torch.float16):
        raise ValueError(f"state dtype must be float32 or float16, got {s.dtype}")
    vw = s.shape[2]
    _check_dims(d, vw)
    a16 = _pad_last(a, _W, torch.float16)
    if d == _W and vw == _W and s.stride(-1) == 1 and s.stride(1) % 8 == 0 and s.stride(0) % 8 == 0 \
            and s.data_ptr() % 16 == 0:
        sp = s
    else:
        sp = _pad_state(s, d, vw, s.dtype)
    y = torch.empty(m, c, _W, dtype=torch.float16, device=dev)
    code = _lib.lib().tj_quad_apply(
        a16.data_ptr(), sp.data_ptr(), y.data_ptr(),
        _lib.TJ_F32 if sp.dtype == torch.float32 else _lib.TJ_F16,
        m, c, _W, _W, _strides3(a16), _strides3(sp), _strides3(y), _stream_ptr(dev),
    )
    _lib.check(code, "tj_quad_apply")
    return y[..., :vw].to(a.dtype)


def quad_update(
    b: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    shadow: Optional[torch.Tensor] = None,
) -> None:
    """Accumulate ``phi2(b)^T @ v`` into the fp32 master ``out`` in place."""
    dev = _require_device(b, v, out)
    if b.dim() != 3 or v.dim() != 3 or b.shape[:2] != v.shape[:2]:
        raise ValueError(f"b must be [M, C, D] and v [M, C, V]; got {tuple(b.shape)}, {tuple(v.shape)}")
    m, c, d = b.shape
    vw = v.shape[2]
    if tuple(out.shape) != (m, d * d, vw):
        raise ValueError(f"out shape {tuple(out.shape)} != {(m, d * d, vw)}")
    if out.dtype != torch.float32:
        # A float16 accumulator loses the chunked sums at long sequence lengths;
        # fail loudly rather than compute something plausible.
        raise ValueError("the master state must be float32")
    if shadow is not None and (tuple(shadow.shape) != tuple(out.shape) or shadow.dtype != torch.float16):
        raise ValueError(f"shadow must be float16 shaped {tuple(out.shape)}, got {shadow.dtype} {tuple(shadow.shape)}")
    if shadow is not None and shadow.device != dev:
        raise ValueError(f"shadow is on {shadow.device}, the other tensors on {dev}")
    _check_dims(d, vw)
    b16 = _pad_last(b, _W, torch.float16)
    v16 = _pad_last(v, _W, torch.float16)
    direct = (d == _W and vw == _W and out.stride(-1) == 1 and out.stride(0) % 4 == 0
              and out.stride(1) % 4 == 0 and out.data_ptr() % 16 == 0)
    if direct and (shadow is None or (shadow.stride(-1) == 1 and shadow.stride(0) % 8 == 0
                                      and shadow.stride(1) % 8 == 0 and shadow.data_ptr() % 16 == 0)):
        code = _lib.lib().tj_quad_update(
            b16.data_ptr(), v16.data_ptr(), out.data_ptr(), None if shadow is None else shadow.data_ptr(),
            m, c, _W, _W, _strides3(b16), _strides3(v16), _strides3(out),
            None if shadow is None else _strides3(shadow), _stream_ptr(dev),
        )
        _lib.check(code, "tj_quad_update")
        return
    delta = torch.zeros(m, _W * _W, _W, dtype=torch.float32, device=dev)
    code = _lib.lib().tj_quad_update(
        b16.data_ptr(), v16.data_ptr(), delta.data_ptr(), None,
        m, c, _W, _W, _strides3(b16), _strides3(v16), _strides3(delta), None, _stream_ptr(dev),
    )
    _lib.check(code, "tj_quad_update")
    out += delta.reshape(m, _W, _W, _W)[:, :d, :d, :vw].reshape(m, d * d, vw)
    if shadow is not None:
        shadow.copy_(out.to(torch.float16))


def causal_diag(a: torch.Tensor, b: torch.Tensor, v: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """``w = tril(exp(a @ b.T))``, then ``(w @ v, w.sum(-1))``, fused."""
    dev = _require_device(a, b, v)
    if a.dim() != 3 or b.shape != a.shape:
        raise ValueError(f"b shape {tuple(b.shape)} != a shape {tuple(a.shape)}")
    m, c, d = a.shape
    if v.dim() != 3 or v.shape[0] != m or v.shape[1] != c:
        raise ValueError(f"v shape {tuple(v.shape)} does not match a {tuple(a.shape)}")
    vw = v.shape[2]
    _check_dims(d, vw)
    a16 = _pad_last(a, _W, torch.float16)
    b16 = _pad_last(b, _W, torch.float16)
    v16 = _pad_last(v, _W, torch.float16)
    num = torch.empty(m, c, _W, dtype=torch.float32, device=dev)
    den = torch.empty(m, c, dtype=torch.float32, device=dev)
    code = _lib.lib().tj_causal_diag(
        a16.data_ptr(), b16.data_ptr(), v16.data_ptr(), num.data_ptr(), den.data_ptr(),
        m, c, _W, _W, _strides3(a16), _strides3(b16), _strides3(v16), _strides3(num), den.stride(0),
        _stream_ptr(dev),
    )
    _lib.check(code, "tj_causal_diag")
    return num[..., :vw], den.unsqueeze(-1)
