"""Exact attention oracles: fp64 brute force and a linear-memory blockwise form.

Restates the arithmetic of the reference's exact path:

* ``F.scaled_dot_product_attention`` as called at ``src/implementations/sdpa.py:65-73``
  (``softmax(q k^T * scale + causal) v``, key mask dropped under causal +
  right padding -- ``src/implementations/attention_routing.py:76-98``);
* ``LinearMemoryFP32SelfAttention`` / ``LinearMemoryFP32Reference``
  (``src/implementations/fp32_reference.py:70-142``): the dense model with only
  the score materialisation replaced by an algebraically equal linear-memory
  evaluation;
* ``compare_outputs_streamed`` (``src/implementations/fp32_reference.py:157-204``).

The blockwise form is an online softmax over key blocks (running max ``m``,
running sum ``l``, rescaled accumulator); it never holds more than one
``[B, H, block_q, block_k]`` score tile, so it runs at S = 65536 on a GPU and at
S <= 8192 on the CPU.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from .model import DenseSelfAttention, DenseTransformer, TransformerConfig


def brute_force_attention(q, k, v, scale: float, causal: bool, valid_len=None) -> np.ndarray:
    """Definition-level exact attention in float64 numpy.

    ``q, k, v``: ``[B, H, S, D]`` arrays or tensors. ``valid_len``: per-batch
    key counts or ``None``. Keys ``j >= valid_len[b]`` and (under ``causal``)
    keys ``j > i`` are excluded; query rows with no admissible key -- and, when
    ``valid_len`` is given, every row ``i >= valid_len[b]`` -- are zero.
    """
    q, k, v = (np.asarray(t.detach().cpu().double() if torch.is_tensor(t) else t, dtype=np.float64)
               for t in (q, k, v))
    b_, h_, s_, _ = q.shape
    out = np.zeros((b_, h_, s_, v.shape[-1]))
    for b in range(b_):
        n_valid = s_ if valid_len is None else int(valid_len[b])
        for h in range(h_):
            scores = (q[b, h] @ k[b, h].T) * scale
            allowed = np.zeros((s_, s_), dtype=bool)
            allowed[:, :n_valid] = True
            if causal:
                allowed &= np.tril(np.ones((s_, s_), dtype=bool))
            if valid_len is not None:
                allowed[n_valid:, :] = False
            for i in range(s_):
                cols = np.nonzero(allowed[i])[0]
                if cols.size == 0:
                    continue
                row = scores[i, cols]
                w = np.exp(row - row.max())
                out[b, h, i] = (w / w.sum()) @ v[b, h, cols]
    return out


def blockwise_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    causal: bool,
    valid_len: Optional[torch.Tensor] = None,
    block_q: int = 1024,
    block_k: int = 1024,
    acc_dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Linear-memory exact attention by online softmax, ``[B, H, S, D]`` in and out.

    Works on any device. The accumulation dtype defaults to fp32 (the
    reference's "FP32 oracle"); fp64 is used by the tests that pin it. The
    masking convention is the one of ``brute_force_attention``.
    """
    b_, h_, s_, d_ = q.shape
    dv = v.shape[-1]
    out = torch.zeros(b_, h_, s_, dv, dtype=q.dtype, device=q.device)
    if valid_len is not None:
        valid_len = valid_len.to(device=q.device, dtype=torch.int64)
        key_pos = torch.arange(s_, device=q.device)
    for q0 in range(0, s_, block_q):
        q1 = min(q0 + block_q, s_)
        qb = q[:, :, q0:q1].to(acc_dtype) * scale
        m = torch.full((b_, h_, q1 - q0, 1), float("-inf"), dtype=acc_dtype, device=q.device)
        l = torch.zeros((b_, h_, q1 - q0, 1), dtype=acc_dtype, device=q.device)
        acc = torch.zeros((b_, h_, q1 - q0, dv), dtype=acc_dtype, device=q.device)
        k_end = q1 if causal else s_
        rows = torch.arange(q0, q1, device=q.device)
        for k0 in range(0, k_end, block_k):
            k1 = min(k0 + block_k, k_end)
            s = qb @ k[:, :, k0:k1].to(acc_dtype).transpose(-2, -1)
            cols = torch.arange(k0, k1, device=q.device)
            if causal:
                s = s.masked_fill(cols[None, :] > rows[:, None], float("-inf"))
            if valid_len is not None:
                dead = key_pos[k0:k1][None, :] >= valid_len[:, None]          # [B, K]
                s = s.masked_fill(dead[:, None, None, :], float("-inf"))
            m_new = torch.maximum(m, s.amax(dim=-1, keepdim=True))
            safe = torch.where(torch.isfinite(m_new), m_new, torch.zeros_like(m_new))
            p = torch.exp(s - safe)
            alpha = torch.exp(torch.where(torch.isfinite(m), m - safe, torch.full_like(m, float("-inf"))))
            l = l * alpha + p.sum(dim=-1, keepdim=True)
            acc = acc * alpha + p @ v[:, :, k0:k1].to(acc_dtype)
            m = m_new
        blk = torch.where(l > 0, acc / l.clamp_min(torch.finfo(acc_dtype).tiny), torch.zeros_like(acc))
        if valid_len is not None:
            dead_rows = rows[None, :] >= valid_len[:, None]                    # [B, Q]
            blk = blk.masked_fill(dead_rows[:, None, :, None], 0)
        out[:, :, q0:q1] = blk.to(q.dtype)
    return out


class LinearMemorySelfAttention(DenseSelfAttention):
    """Dense attention module with the score tensor replaced by ``blockwise_attention``.

    Restates ``LinearMemoryFP32SelfAttention`` (``fp32_reference.py:70-127``):
    FP32 only; the key mask is dropped under causal attention (exact for
    right-padded masks, whose padded query rows are zeroed afterwards) and
    applied as per-batch valid lengths otherwise.
    """

    block = 1024

    def attend(self, q, k, v, valid_token_mask, causal):
        if q.dtype != torch.float32:
            raise RuntimeError("the linear-memory oracle requires float32 input")
        valid_len = None
        if valid_token_mask is not None:
            lengths = valid_token_mask.sum(dim=1)
            expected = torch.arange(valid_token_mask.shape[1], device=q.device)[None, :] < lengths[:, None]
            if not bool(torch.equal(valid_token_mask, expected)):
                raise ValueError("the linear-memory oracle requires right-padded masks")
            if not causal:
                valid_len = lengths
        return blockwise_attention(q, k, v, self.scale, causal, valid_len, self.block, self.block)


class LinearMemoryReference(DenseTransformer):
    """``DenseTransformer`` with every attention evaluated blockwise (``fp32_reference.py:130-142``)."""

    def __init__(self, config: TransformerConfig) -> None:
        super().__init__(config)
        for layer in self.layers:
            replacement = LinearMemorySelfAttention(config.d_model, config.num_heads)
            replacement.load_state_dict(layer.attention.state_dict())
            layer.attention = replacement


@dataclass(frozen=True)
class StreamedAccuracy:
    passed: bool
    total_elements: int
    failed_elements: int
    max_abs_error: float
    max_relative_error: float
    mean_abs_error: float


def compare_outputs_streamed(reference, candidate, *, rtol=0.02, atol=0.002, token_chunk=2048) -> StreamedAccuracy:
    """The OR rule over ``[B, N, D]`` tensors in bounded token chunks (``fp32_reference.py:157-204``)."""
    if reference.shape != candidate.shape:
        raise AssertionError(
            f"shape mismatch: reference={tuple(reference.shape)}, candidate={tuple(candidate.shape)}"
        )
    if reference.ndim != 3:
        raise ValueError("reference and candidate must be [B, N, D]")
    if token_chunk <= 0:
        raise ValueError("token_chunk must be positive")
    failed, abs_sum, max_abs, max_rel = 0, 0.0, 0.0, 0.0
    for t0 in range(0, reference.shape[1], token_chunk):
        ref = reference[:, t0:t0 + token_chunk].detach().float()
        got = candidate[:, t0:t0 + token_chunk].detach().to(ref.device).float()
        err = (got - ref).abs()
        ok = torch.isfinite(ref) & torch.isfinite(got) & ((err <= atol) | (err <= rtol * ref.abs()))
        failed += int((~ok).sum().item())
        abs_sum += float(err.sum(dtype=torch.float64).item())
        max_abs = max(max_abs, float(err.max().item()))
        max_rel = max(max_rel, float((err / ref.abs().clamp_min(1e-12)).max().item()))
    total = reference.numel()
    return StreamedAccuracy(failed == 0, total, failed, max_abs, max_rel, abs_sum / total)


def exact_attention_flops(valid_lengths, num_heads: int, head_dim: int) -> float:
    """Algorithmic FLOPs of causal attention: ``2*d*H*sum_b L_b(L_b+1)``.

    QK^T and PV at 2 FLOP per multiply-add over the lower triangle including
    the diagonal.
    """
    return float(2 * head_dim * num_heads * sum(int(n) * (int(n) + 1) for n in valid_lengths))
