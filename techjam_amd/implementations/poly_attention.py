"""Guarded degree-2 polynomial attention on the HIP kernels.

Mirrors ``src/implementations/poly_attention.py:17-83``. ``CHUNK`` and
``EXACT_PREFIX`` keep the reference's values; the master states are fp32
unconditionally (an fp16 master passes at N=16384 and fails at N=65536 in the
reference's measurements), and the final state update is always skipped.

``poly_attention_forward`` evaluates one coefficient set for every head (the
reference's one-sigma-per-module semantics); ``guarded_attention`` is the
device-side route: the guard kernel measures each head, the polynomial kernel
fills rows ``>= EXACT_PREFIX`` of the safe heads, and one exact-attention launch
fills the exact prefix of those heads and every row of the others (with split
fp16 scores, since their score range is wide). Nothing synchronises the host.
"""

from __future__ import annotations

from typing import Optional

import torch

from ..kernels.attention import empty_like_heads, scaled_dot_product_attention
from ..kernels.poly import poly_rows
from .poly_guard import ATTENTION_SIGMA_CEILING, guard, hermite_coefficients

CHUNK = 512
EXACT_PREFIX = 4096


def _prefix(n: int) -> int:
    return min(EXACT_PREFIX, n)


def poly_attention_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    *,
    sigma: Optional[float],
    disable: frozenset = frozenset(),
) -> torch.Tensor:
    """Causal polynomial attention over ``[B, H, N, D]`` with one sigma for all heads.

    ``disable`` accepts ``"poly"`` (run every row exactly, for A/B runs in one
    session); the reference's Triton-specific names have no counterpart.
    """
    b, h, n, _ = q.shape
    out = empty_like_heads(q)
    if "poly" in disable:
        return scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale, out=out)
    c = torch.tensor(hermite_coefficients(sigma), dtype=torch.float32, device=q.device)
    coeffs = c.repeat(b * h, 1).contiguous()
    poly_rows(q, k, v, scale, coeffs, chunk=CHUNK, exact_prefix=_prefix(n), out=out)
    if _prefix(n) > 0:
        limit = torch.full((b * h,), _prefix(n), dtype=torch.int32, device=q.device)
        scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale, row_limit=limit, out=out)
    return out


def guarded_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    *,
    enabled: bool = True,
    ceiling: float = ATTENTION_SIGMA_CEILING,
    out: Optional[torch.Tensor] = None,
):
    """Per-head guarded causal attention; returns ``(out, guard_result)``.

    A head takes the polynomial route when its sampled score sigma is in
    ``(0, ceiling]``. The default keeps the attention output itself within
    the OR rule (``ATTENTION_SIGMA_CEILING``); the dispatcher's model module
    passes the reference's model-level ``SIGMA_CEILING``. With
    ``enabled=False`` every head takes the exact kernel (the guard still
    runs, to select split scores for wide-range heads).
    """
    g = guard(q, k, scale, ceiling=ceiling, exact_prefix=_prefix(q.shape[2]))
    if out is None:
        out = empty_like_heads(q)
    if not enabled:
        scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale, qk_split=g.split, out=out)
        return out, g
    # The exact launch (prefix rows of the polynomial heads, every row of the
    # fallback heads) writes rows disjoint from the polynomial kernel's, so it
    # runs on a side stream, overlapping the chunk launches, which leave most
    # of the GPU idle.
    main = torch.cuda.current_stream(q.device)
    side = _side_stream(q.device)
    side.wait_stream(main)
    with torch.cuda.stream(side):
        scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale, row_limit=g.row_limit,
                                     qk_split=g.split, out=out)
    for t in (q, k, v, out, g.row_limit, g.split):
        t.record_stream(side)
    poly_rows(q, k, v, scale, g.coeffs, flags=g.flags, chunk=CHUNK, exact_prefix=_prefix(q.shape[2]), out=out)
    main.wait_stream(side)
    return out, g


_SIDE_STREAMS: dict = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """One default-priority side stream per device, created on first use."""
    key = torch.device(device).index
    if key not in _SIDE_STREAMS:
        _SIDE_STREAMS[key] = torch.cuda.Stream(device=device)
    return _SIDE_STREAMS[key]
