"""Python entry point of the HIP polynomial-attention kernels.

``poly_rows`` stands where the reference runs its chunk scan
(``src/implementations/poly_reference.py:162-249``) with the three Triton
kernels (``src/kernels/poly_attention_triton.py:420-591``): it fills rows
``>= exact_prefix`` of every flagged head. The fp32 states, their fp16
shadows and the per-chunk scratch live in one workspace allocated here from
torch's caching allocator.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from .attention import _DTYPES, _check_qkv, _kernel_view, _require_device, _stream_ptr, empty_like_heads


def workspace_bytes(b: int, h: int, s: int, d: int, chunk: int) -> int:
    return int(_lib.lib().tj_poly_workspace_bytes(b, h, s, d, chunk))


def poly_rows(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    coeffs: torch.Tensor,
    *,
    flags: Optional[torch.Tensor] = None,
    chunk: int = 512,
    exact_prefix: int = 4096,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Rows ``>= exact_prefix`` of the chunked polynomial attention of each flagged head.

    ``coeffs``: float32 ``[B*H, 3]`` device tensor of ``(c0, c1, c2)`` per head.
    ``flags``: int32 ``[B*H]`` device tensor (``0`` skips the head) or ``None``.
    Rows ``< exact_prefix`` of ``out`` are not written.
    """
    _check_qkv(q, k, v)
    # The kernel writes B*H*S*D elements of q's type through out's strides.
    if out is not None and (out.shape != q.shape or out.dtype != q.dtype or out.device != q.device):
        raise ValueError("out must match q in shape, dtype and device")
    dev = _require_device(q, k, v)
    b, h, s, d = q.shape
    q, k, v = _kernel_view(q), _kernel_view(k, keys=True), _kernel_view(v, keys=True)
    if out is None:
        out = empty_like_heads(q)
    m = b * h
    if coeffs.dtype != torch.float32 or coeffs.device != dev or coeffs.numel() != 3 * m or not coeffs.is_contiguous():
        raise ValueError(f"coeffs must be a contiguous float32 [B*H, 3] tensor on {dev}")
    if flags is not None and (flags.dtype != torch.int32 or flags.device != dev or flags.numel() != m
                              or not flags.is_contiguous()):
        raise ValueError(f"flags must be a contiguous int32 [B*H] tensor on {dev}")
    nbytes = workspace_bytes(b, h, s, d, chunk)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    code = _lib.lib().tj_poly_attn_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), _DTYPES[q.dtype],
        b, h, s, d,
        _lib.strides4(q), _lib.strides4(k), _lib.strides4(v), _lib.strides4(out),
        float(scale), int(chunk), int(exact_prefix),
        coeffs.data_ptr(), None if flags is None else flags.data_ptr(),
        ws.data_ptr(), nbytes, _stream_ptr(dev),
    )
    _lib.check(code, "tj_poly_attn_fwd")
    return out
