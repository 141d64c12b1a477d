"""Fused elementwise tails of the encoder block on the HIP kernels.

``bias_residual`` and ``bias_gelu`` replace the bias add / residual add /
``masked_fill`` and bias add / exact GELU pairs that follow the block's
projection GEMMs (``torch_transformer_benchmark.py:116-121``, ``:140-145``)
with one pass each; ``bias_residual_layernorm`` also produces the LayerNorm of
the residual stream that the next step reads. ``bias_relu`` serves the
optional post-norm / ReLU block. They return ``None`` for
layouts the kernels do not take (non-fp32, a last dimension that is not a
multiple of 4 -- one of ``NORM_WIDTHS`` for the norm --, unaligned or
non-contiguous tensors), and the caller then uses the plain tensor ops.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from .attention import _stream_ptr

#: Row widths the fused residual + LayerNorm kernel takes.
NORM_WIDTHS = (32, 64, 128, 256, 512, 1024, 2048)

MODE_PLAIN = 0       # out = x + y + b
MODE_ZERO_Y = 1      # out = x + (row valid ? y + b : 0)
MODE_ZERO_OUT = 2    # out = row valid ? x + y + b : 0


def _check_out(out: Optional[torch.Tensor], x: torch.Tensor) -> None:
    """A caller-supplied ``out`` must have ``x``'s shape, dtype and device: the
    kernels write ``x.numel()`` elements through it."""
    if out is not None and (out.shape != x.shape or out.dtype != x.dtype or out.device != x.device):
        raise ValueError(f"out must match x ({tuple(x.shape)}, {x.dtype}, {x.device}); "
                         f"got ({tuple(out.shape)}, {out.dtype}, {out.device})")


def _ok(*ts: torch.Tensor) -> bool:
    return all(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous() and t.data_ptr() % 16 == 0
               and t.shape[-1] % 4 == 0 for t in ts)


def bias_residual(x: torch.Tensor, y: torch.Tensor, bias: torch.Tensor, valid_len: Optional[torch.Tensor],
                  mode: int, out: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
    """One pass of ``x + y + bias`` with padded rows handled per ``mode``; ``x``, ``y`` ``[B, S, C]``."""
    if x.ndim != 3 or y.shape != x.shape or bias.shape != (x.shape[-1],):
        return None
    if valid_len is not None and (valid_len.dtype != torch.int32 or valid_len.shape != (x.shape[0],)
                                  or valid_len.device != x.device):
        return None
    _check_out(out, x)
    out = torch.empty_like(x) if out is None else out
    if not _ok(x, y, bias, out):
        return None
    b, s, c = x.shape
    code = _lib.lib().tj_bias_residual(
        out.data_ptr(), x.data_ptr(), y.data_ptr(), bias.data_ptr(), b * s, c, s,
        None if valid_len is None else valid_len.data_ptr(), mode, _stream_ptr(x.device))
    _lib.check(code, "tj_bias_residual")
    return out


def _bias_act(name: str, y: torch.Tensor, bias: torch.Tensor, out_f16: bool) -> Optional[torch.Tensor]:
    if bias.ndim != 1 or y.shape[-1] != bias.shape[0] or not _ok(y, bias):
        return None
    out = torch.empty(y.shape, dtype=torch.float16, device=y.device) if out_f16 else None
    code = getattr(_lib.lib(), name)(y.data_ptr(), bias.data_ptr(), y.numel() // y.shape[-1], y.shape[-1],
                                     None if out is None else out.data_ptr(), _stream_ptr(y.device))
    _lib.check(code, name)
    return y if out is None else out


def bias_gelu(y: torch.Tensor, bias: torch.Tensor, out_f16: bool = False) -> Optional[torch.Tensor]:
    """``gelu(y + bias)`` (exact form); ``y`` ``[..., C]``. In place, or with
    ``out_f16`` into a new fp16 tensor (``y`` unchanged) -- the operand of an
    fp16 GEMM."""
    return _bias_act("tj_bias_gelu", y, bias, out_f16)


def bias_relu(y: torch.Tensor, bias: torch.Tensor, out_f16: bool = False) -> Optional[torch.Tensor]:
    """``relu(y + bias)``, in place or into a new fp16 tensor, as :func:`bias_gelu`."""
    return _bias_act("tj_bias_relu", y, bias, out_f16)


def bias_residual_layernorm(x: torch.Tensor, y: torch.Tensor, bias: torch.Tensor,
                            valid_len: Optional[torch.Tensor], mode: int, norm: torch.nn.LayerNorm,
                            out: Optional[torch.Tensor] = None, zero_padded_norm: bool = False,
                            norm_dtype: torch.dtype = torch.float32, keep_sum: bool = True):
    """``bias_residual`` and ``norm`` of its result in one pass: ``(out, norm(out))``.

    With ``zero_padded_norm`` the norm output of padded rows is zero (the final
    ``masked_fill``); ``norm_dtype`` float16 stores the norm as the operand of
    an fp16 GEMM. Without ``keep_sum`` the sum is not stored and ``(None,
    norm)`` comes back (a post-norm block keeps only the norm). ``None`` when
    the shapes or the norm are not covered.
    """
    c = x.shape[-1] if x.ndim == 3 else 0
    if (x.ndim != 3 or y.shape != x.shape or bias.shape != (c,) or c not in NORM_WIDTHS
            or not isinstance(norm, torch.nn.LayerNorm) or tuple(norm.normalized_shape) != (c,)
            or norm.weight is None or norm.bias is None):
        return None
    if valid_len is not None and (valid_len.dtype != torch.int32 or valid_len.shape != (x.shape[0],)
                                  or valid_len.device != x.device):
        return None
    if norm_dtype not in (torch.float32, torch.float16):
        raise ValueError(f"norm_dtype must be float32 or float16, not {norm_dtype}")
    if not keep_sum and out is not None:
        raise ValueError("out is not written when keep_sum is False")
    _check_out(out, x)
    if keep_sum and out is None:
        out = torch.empty_like(x)
    if not _ok(x, y, bias, norm.weight, norm.bias, *([out] if keep_sum else [])):
        return None
    ln = torch.empty(x.shape, dtype=norm_dtype, device=x.device)
    b, s, _ = x.shape
    code = _lib.lib().tj_bias_residual_layernorm(
        None if out is None else out.data_ptr(), ln.data_ptr(), _lib.TJ_F16 if norm_dtype == torch.float16 else _lib.TJ_F32, x.data_ptr(),
        y.data_ptr(), bias.data_ptr(), norm.weight.data_ptr(), norm.bias.data_ptr(), b * s, c, s, None if valid_len is None else valid_len.data_ptr(), mode,
        float(norm.eps), int(bool(zero_padded_norm)), _stream_ptr(x.device))
    _lib.check(code, "tj_bias_residual_layernorm")
    return out, ln
