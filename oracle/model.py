"""Dense FP32 Transformer encoder: the semantic definition of the hot path.

Restates ``torch_transformer_benchmark.py:29-356`` of the reference:

* ``TransformerConfig``               -- ``:29-56``
* ``DenseSelfAttention``              -- ``BaselineSelfAttention`` ``:59-122``
* ``DenseBlock`` / ``DenseTransformer`` -- ``:125-172`` (pre-norm, exact GELU)
* ``copy_model_weights``              -- ``:203-213``
* ``generate_random_case``            -- ``:234-272``
* ``compare_outputs``                 -- ``:289-356`` (exact OR rule)

Parameter names and the order in which the ``nn.Linear`` layers are created
match the reference, so ``torch.manual_seed(s)`` followed by construction gives
bit-identical weights and the state dicts are interchangeable.
"""

from __future__ import annotations

import copy
from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass(frozen=True)
class TransformerConfig:
    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    num_layers: int
    causal: bool

    def validate(self) -> None:
        for name in ("batch_size", "seq_len", "d_model", "num_heads", "ffn_dim", "num_layers"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive")
        if self.d_model % self.num_heads:
            raise ValueError(
                f"d_model ({self.d_model}) must be divisible by num_heads ({self.num_heads})"
            )


class DenseSelfAttention(nn.Module):
    """Explicit-score multi-head attention (reference ``:59-122``).

    Scores are materialised as ``[B, H, S, S]``; the causal mask fills the
    strict upper triangle and the key mask fills invalid keys with ``-inf``;
    softmax runs in fp32; padded query rows are zeroed after the output
    projection.
    """

    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__()
        if d_model % num_heads:
            raise ValueError("d_model must be divisible by num_heads")
        self.d_model = d_model
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.scale = self.head_dim ** -0.5
        # Creation order fixes the seeded initialisation: q, k, v, out.
        self.q_proj = nn.Linear(d_model, d_model)
        self.k_proj = nn.Linear(d_model, d_model)
        self.v_proj = nn.Linear(d_model, d_model)
        self.out_proj = nn.Linear(d_model, d_model)

    def heads(self, t: torch.Tensor) -> torch.Tensor:
        b, s, _ = t.shape
        return t.view(b, s, self.num_heads, self.head_dim).transpose(1, 2).contiguous()

    def attend(self, q, k, v, valid_token_mask, causal):
        s = q.shape[2]
        scores = torch.matmul(q, k.transpose(-2, -1)) * self.scale
        if causal:
            upper = torch.ones(s, s, dtype=torch.bool, device=q.device).triu(1)
            scores = scores.masked_fill(upper, float("-inf"))
        if valid_token_mask is not None:
            scores = scores.masked_fill(~valid_token_mask[:, None, None, :], float("-inf"))
        probs = torch.softmax(scores.float(), dim=-1).to(q.dtype)
        return torch.matmul(probs, v)

    def forward(self, x, valid_token_mask=None, causal=False):
        b, s, _ = x.shape
        q = self.heads(self.q_proj(x))
        k = self.heads(self.k_proj(x))
        v = self.heads(self.v_proj(x))
        ctx = self.attend(q, k, v, valid_token_mask, causal)
        ctx = ctx.transpose(1, 2).contiguous().view(b, s, self.d_model)
        out = self.out_proj(ctx)
        if valid_token_mask is not None:
            out = out.masked_fill(~valid_token_mask[..., None], 0)
        return out


class DenseBlock(nn.Module):
    """Pre-norm residual block with exact GELU (reference ``:125-145``)."""

    def __init__(self, d_model: int, num_heads: int, ffn_dim: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)
        self.attention = DenseSelfAttention(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model)
        self.ffn_in = nn.Linear(d_model, ffn_dim)
        self.ffn_out = nn.Linear(ffn_dim, d_model)

    def forward(self, x, valid_token_mask, causal):
        x = x + self.attention(self.norm1(x), valid_token_mask, causal)
        x = x + self.ffn_out(F.gelu(self.ffn_in(self.norm2(x)), approximate="none"))
        if valid_token_mask is not None:
            x = x.masked_fill(~valid_token_mask[..., None], 0)
        return x


class DenseTransformer(nn.Module):
    """Layer stack plus final LayerNorm (reference ``:148-172``)."""

    def __init__(self, config: TransformerConfig) -> None:
        super().__init__()
        self.config = config
        self.layers = nn.ModuleList(
            DenseBlock(config.d_model, config.num_heads, config.ffn_dim)
            for _ in range(config.num_layers)
        )
        self.final_norm = nn.LayerNorm(config.d_model)

    def forward(self, x, valid_token_mask=None):
        for layer in self.layers:
            x = layer(x, valid_token_mask, self.config.causal)
        x = self.final_norm(x)
        if valid_token_mask is not None:
            x = x.masked_fill(~valid_token_mask[..., None], 0)
        return x


def copy_model_weights(src: nn.Module, dst: nn.Module, strict: bool = True) -> None:
    """Load ``src``'s state dict into ``dst`` (reference ``:203-213``)."""
    dst.load_state_dict(copy.deepcopy(src.state_dict()), strict=strict)


def generate_random_case(
    config: TransformerConfig,
    device: torch.device,
    dtype: torch.dtype,
    seed: int,
    padding_ratio: float,
    input_scale: float,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Seeded input and right-padded valid-token mask (reference ``:234-272``).

    One generator draws ``x`` first and then the per-sample lengths, uniform in
    ``[round(S * (1 - padding_ratio)), S]``; padded rows of ``x`` are zeroed.
    """
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    b, s = config.batch_size, config.seq_len
    x = torch.randn(b, s, config.d_model, generator=gen, device=device, dtype=dtype) * input_scale
    if padding_ratio <= 0:
        return x, torch.ones(b, s, dtype=torch.bool, device=device)
    low = max(1, int(round(s * (1.0 - padding_ratio))))
    lengths = torch.randint(low, s + 1, (b,), generator=gen, device=device)
    mask = torch.arange(s, device=device)[None, :] < lengths[:, None]
    return x.masked_fill(~mask[..., None], 0), mask


@dataclass
class AccuracyResult:
    passed: bool
    total_elements: int
    failed_elements: int
    max_abs_error: float
    max_relative_error: float
    mean_abs_error: float
    failed_feature_dims: List[int]
    worst_index: Tuple[int, ...]
    reference_at_worst: float
    optimized_at_worst: float


def compare_outputs(reference: torch.Tensor, optimized: torch.Tensor, rtol: float, atol: float) -> AccuracyResult:
    """Per-element ``|d| <= atol OR |d| <= rtol*|ref|``, both finite (reference ``:289-356``).

    The OR rule is applied literally; it is slightly stricter than
    ``torch.isclose``'s ``atol + rtol*|ref|``.
    """
    if reference.shape != optimized.shape:
        raise AssertionError(
            f"shape mismatch: baseline={tuple(reference.shape)}, optimized={tuple(optimized.shape)}"
        )
    ref = reference.detach().float()
    got = optimized.detach().float()
    err = (got - ref).abs()
    ok = torch.isfinite(ref) & torch.isfinite(got) & ((err <= atol) | (err <= rtol * ref.abs()))
    failed = ~ok
    n_failed = int(failed.sum().item())
    flat = int(err.reshape(-1).argmax().item())
    worst = tuple(int(i) for i in torch.unravel_index(torch.tensor(flat), reference.shape))
    rel = err / ref.abs().clamp_min(1e-12)
    if reference.ndim == 0:
        dims = [0] if n_failed else []
    elif reference.ndim == 1:
        dims = torch.nonzero(failed).flatten().tolist()
    else:
        dims = torch.nonzero(failed.any(dim=tuple(range(reference.ndim - 1)))).flatten().tolist()
    return AccuracyResult(
        passed=n_failed == 0,
        total_elements=reference.numel(),
        failed_elements=n_failed,
        max_abs_error=float(err.max().item()),
        max_relative_error=float(rel.max().item()),
        mean_abs_error=float(err.mean().item()),
        failed_feature_dims=dims,
        worst_index=worst,
        reference_at_worst=float(ref[worst].item()),
        optimized_at_worst=float(got[worst].item()),
    )
