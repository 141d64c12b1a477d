"""Algorithmic work of the hot path and the harness's seeded inputs.

The FLOP and byte counts are what a roofline fraction is priced on: the work
the algorithm must do, not what a kernel happens to issue.

* exact causal attention: ``2*d*H*sum_b L_b(L_b+1)`` -- QK^T and PV at two
  FLOP per multiply-add over the lower triangle including the diagonal;
* the guarded polynomial path per (b, h): the exact prefix ``2*d*W(W+1)``;
  per emitted token ``2d^2 dv + 2d dv + 2d^2 + 4d`` (the quadratic, linear
  and constant terms of numerator and denominator); per token of every chunk
  but the last ``2d^2 dv + 2d dv + 2d^2`` (the state update, skipped after
  the final chunk as in ``src/implementations/poly_reference.py:232-249``);
  the exact diagonal block ``2d*C(C+1)`` per emitted chunk;
* bytes: fp32 (or fp16) q, k, v read once and o written once.

``random_case`` draws the benchmark harness's inputs
(``torch_transformer_benchmark.py:234-272``): one generator draws ``x`` and then
the per-sample valid lengths, uniform in ``[round(S*(1-padding_ratio)), S]``;
the mask is right-padded and padded rows of ``x`` are zero.
"""

from __future__ import annotations

from typing import Iterable, Tuple

import torch


def exact_attention_flops(valid_lengths: Iterable[int], num_heads: int, head_dim: int) -> float:
    return float(2 * head_dim * num_heads * sum(int(n) * (int(n) + 1) for n in valid_lengths))


def poly_flops(n: int, d: int, dv: int, chunk: int, exact_prefix: int) -> float:
    """FLOPs of one (b, h) of the polynomial path over ``n`` tokens."""
    w = min(exact_prefix, n)
    total = 2.0 * d * w * (w + 1)
    for t0 in range(0, n, chunk):
        t1 = min(t0 + chunk, n)
        c = t1 - t0
        if t1 > w:  # a chunk with rows past the exact prefix is emitted
            total += c * (2 * d * d * dv + 2 * d * dv + 2 * d * d + 4 * d) + 2.0 * d * c * (c + 1)
        if t1 != n:  # every chunk but the last folds into the state
            total += c * (2 * d * d * dv + 2 * d * dv + 2 * d * d)
    return total


def attention_bytes(batch: int, seq_len: int, heads: int, head_dim: int, element_size: int = 4) -> float:
    return float(4 * element_size * batch * seq_len * heads * head_dim)


def random_case(batch: int, seq_len: int, d_model: int, seed: int, padding_ratio: float,
                input_scale: float = 1.0, device: torch.device = torch.device("cpu"),
                dtype: torch.dtype = torch.float32) -> Tuple[torch.Tensor, torch.Tensor]:
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    x = torch.randn(batch, seq_len, d_model, generator=gen, device=device, dtype=dtype) * input_scale
    if padding_ratio <= 0:
        return x, torch.ones(batch, seq_len, dtype=torch.bool, device=device)
    low = max(1, int(round(seq_len * (1.0 - padding_ratio))))
    lengths = torch.randint(low, seq_len + 1, (batch,), generator=gen, device=device)
    mask = torch.arange(seq_len, device=device)[None, :] < lengths[:, None]
    return x.masked_fill(~mask[..., None], 0), mask
