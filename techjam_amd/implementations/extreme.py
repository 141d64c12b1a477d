"""Memory-bounded execution for extreme shapes and the guarded polynomial module.

Mirrors ``src/implementations/extreme.py:18-319``:

* The reference's batch-chunk estimator (``:40-117``: a power-of-two chunk
  from SDPA score-copy counts) has no counterpart here: chunk sizes come from
  ``planner.plan_batch_chunk``, which budgets the HIP kernels' real working
  set (they never materialise scores).
* ``right_padded_lengths`` (``:120-133``), ``forward_batch_chunks`` with OOM
  halving (``:136-164``) and ``forward_prefix_chunks`` with trimmed equal-length
  groups (``:167-204``).
* ``ExactOnlySelfAttention`` -- the forced exact fallback (the reference's
  ``FlashOnlySDPASelfAttention``, ``:207-238``): mask-free, padding trimmed by
  the caller, FP32 or FP16 interface.
* ``PolyOrExactSelfAttention`` -- the guarded route (``PolyOrFlashSelfAttention``,
  ``:249-319``) with the guard evaluated per head on the device instead of one
  cached host-side sigma.
"""

from __future__ import annotations

from collections.abc import Callable
from typing import Optional

import torch
import torch.nn.functional as F

from ..kernels.attention import scaled_dot_product_attention
from ..model import fp16_weight
from .poly_attention import guarded_attention
from .poly_guard import SIGMA_CEILING, poly_is_safe
from .sdpa import StridedSDPASelfAttention

CASE_6_CONFIG = (10000, 128, 128, 4, 128, True, 4)
CASE_14_CONFIG = (32, 100000, 1024, 16, 1024, True, 2)

ChunkForward = Callable[[torch.Tensor, Optional[torch.Tensor]], torch.Tensor]

# One switch returns the guarded modules to exact attention on every head.
POLY_ATTENTION_ENABLED = True


def right_padded_lengths(valid_token_mask: torch.Tensor) -> list:
    """Per-sample prefix lengths as a host list; rejects masks with interior holes."""
    if valid_token_mask.ndim != 2 or valid_token_mask.dtype != torch.bool:
        raise ValueError("valid_token_mask must be a two-dimensional bool tensor")
    lengths = valid_token_mask.sum(dim=1, dtype=torch.int64)
    pos = torch.arange(valid_token_mask.shape[1], device=valid_token_mask.device)
    if not bool(torch.equal(valid_token_mask, pos[None, :] < lengths[:, None])):
        raise ValueError("extreme route requires right-padded prefix masks")
    return [int(n) for n in lengths.cpu().tolist()]


def forward_batch_chunks(forward_chunk: ChunkForward, x: torch.Tensor,
                         valid_token_mask: Optional[torch.Tensor], chunk_size: int) -> torch.Tensor:
    """Independent batch slices into one output; an OOM halves the chunk and retries."""
    if chunk_size <= 0:
        raise ValueError("chunk_size must be positive")
    out = torch.empty_like(x)
    start = 0
    active = min(chunk_size, x.shape[0])
    while start < x.shape[0]:
        end = min(start + active, x.shape[0])
        mask = None if valid_token_mask is None else valid_token_mask[start:end]
        try:
            res = forward_chunk(x[start:end], mask)
            out[start:end].copy_(res)
            del res
            start = end
        except torch.OutOfMemoryError:
            if active == 1:
                raise
            active = max(1, active // 2)
            torch.cuda.empty_cache()
    return out


def forward_prefix_chunks(forward_chunk: ChunkForward, x: torch.Tensor,
                          valid_token_mask: Optional[torch.Tensor], chunk_size: int) -> torch.Tensor:
    """Equal-length prefix groups, padding trimmed, no mask passed; padded rows stay zero."""
    lengths = [x.shape[1]] * x.shape[0] if valid_token_mask is None else right_padded_lengths(valid_token_mask)
    out = torch.zeros_like(x)
    start = 0
    active = min(chunk_size, x.shape[0])
    while start < x.shape[0]:
        n = lengths[start]
        end = start + 1
        while end < x.shape[0] and end - start < active and lengths[end] == n:
            end += 1
        if n:
            try:
                res = forward_chunk(x[start:end, :n], None)
                out[start:end, :n].copy_(res)
                del res
            except torch.OutOfMemoryError:
                if active == 1:
                    raise
                active = max(1, active // 2)
                torch.cuda.empty_cache()
                continue
        start = end
    return out


class ExactOnlySelfAttention(StridedSDPASelfAttention):
    """Exact causal attention for trimmed, mask-free extreme-length inputs."""

    def _check(self, x, valid_token_mask):
        if x.device.type != "cuda":
            raise RuntimeError("extreme attention requires a ROCm device")
        if x.dtype not in (torch.float16, torch.float32):
            raise RuntimeError("extreme attention requires float16 or float32")
        if valid_token_mask is not None:
            raise ValueError("trim padding before calling extreme attention")

    def qkv(self, x):
        """q, k, v head views. An fp16 ``x`` (the fp16-operand layer stack)
        runs each projection as one fp16 GEMM with its bias in the epilogue
        (the parameters' cached fp16 copies, fp32 accumulation) and returns
        fp16 q, k, v -- the reference's fp16 case-14 contract."""
        if x.dtype != torch.float16:
            return self.project_qkv(x)
        out = []
        for lin in (self.q_proj, self.k_proj, self.v_proj):
            bias = None if lin.bias is None else fp16_weight(lin, "bias", lin.bias)
            out.append(self.heads_view(F.linear(x, fp16_weight(lin, "weight", lin.weight), bias)))
        return tuple(out)

    def context(self, x, valid_token_mask=None, causal=False, valid_len=None):
        self._check(x, valid_token_mask)
        b, s, _ = x.shape
        q, k, v = self.qkv(x)
        ctx = scaled_dot_product_attention(q, k, v, is_causal=causal, scale=self.scale)
        return ctx.transpose(1, 2).reshape(b, s, self.d_model)


class PolyOrExactSelfAttention(ExactOnlySelfAttention):
    """Extreme-length attention: guarded polynomial route with exact fallback, per head.

    ``route_name(sigma)`` keeps the reference's pure routing predicate for
    tests; at run time the decision is made per ``(b, h)`` on the device, and
    ``last_guard`` holds the most recent per-head guard tensors.
    """

    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__(d_model, num_heads)
        self.poly_enabled = POLY_ATTENTION_ENABLED
        # The model-level ceiling: this module's output feeds the residual
        # stream, and the reference calibrates the guard on the model's output.
        self.sigma_ceiling = SIGMA_CEILING
        self.last_guard = None

    def route_name(self, sigma: Optional[float]) -> str:
        return "poly" if self.poly_enabled and poly_is_safe(sigma) and sigma <= self.sigma_ceiling else "exact"

    def context(self, x, valid_token_mask=None, causal=False, valid_len=None):
        self._check(x, valid_token_mask)
        if not causal:
            raise ValueError("the polynomial route is causal attention")
        b, s, _ = x.shape
        q, k, v = self.qkv(x)
        ctx, self.last_guard = guarded_attention(q, k, v, self.scale, enabled=self.poly_enabled,
                                                 ceiling=self.sigma_ceiling)
        return ctx.transpose(1, 2).reshape(b, s, self.d_model)
