"""Streaming planner: batch chunks sized from the HIP path's own working set.

The reference picks the batch chunk of its streamed routes from a guess of
PyTorch's SDPA allocations -- ``activation_copies * S*D + score_copies * S^2*H``
elements per item (``src/implementations/extreme.py:40-117``, called with 12
score copies for case 6 and none for case 14, ``src/dispatcher.py:452-465``,
``:525-538``). No kernel here materialises scores, so that formula plans for
memory that is never used. This planner counts what the encoder forward on the
HIP kernels actually holds per batch item at its peak:

* attention phase of a layer: the residual stream, the normed input, q/k/v
  (one packed ``[S, 3D]`` projection or three ``[S, D]`` ones, at the GEMM's
  output type) and the attention output -- six ``[S, D]`` float32 activations;
  on the guarded polynomial route also the per-head polynomial workspace
  (``tj_poly_workspace_bytes``: fp32 states, fp16 shadow ring, token images),
  the guard's partial sums (``tj_score_guard_workspace_bytes``) and its seven
  per-head outputs;
* FFN phase: the residual, one normed copy and the ``[S, F]`` hidden
  activation, then the residual, the hidden activation and the output
  projection (``TransformerEncoder._forward_layers_fused`` releases every
  intermediate at its last use, which is what makes these counts an upper
  bound); the unfused float16 path can hold the residual and two hidden
  activations (before and after GELU), so the larger of the two is counted.

The caller's output buffer for the whole batch is reserved first, as in the
reference, and a fixed allowance covers the GEMM libraries' workspaces. The
chunk is the largest power of two whose items fit what is left -- powers of
two keep the out-of-memory halving of ``forward_batch_chunks`` on the same
sizes.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Optional

import torch

from ..kernels import _lib

DEFAULT_MEMORY_FRACTION = 0.85
#: Allowance for workspaces the GEMM libraries take from torch's allocator
#: on first use (hipBLASLt / rocBLAS) and for the small per-call tensors
#: (valid lengths, the guard's cached row sample).
LIBRARY_ALLOWANCE_BYTES = 256 << 20
GUARD_OUTPUT_BYTES_PER_HEAD = 4 * (1 + 1 + 1 + 1 + 3 + 1 + 1)  # sigma, mean, smax, flag, 3 coeffs, limit, split
GUARD_SAMPLES = 512
POLY_HEAD_DIM = 64
POLY_CHUNK = 512


@dataclass(frozen=True)
class Footprint:
    """Peak device bytes one batch item adds, and its parts."""

    per_item_bytes: int
    output_per_item_bytes: int
    parts: Dict[str, int] = field(default_factory=dict)


def poly_workspace_bytes_per_head() -> int:
    """Bytes of polynomial workspace per (b, h), as the library reports them."""
    n = int(_lib.lib().tj_poly_workspace_bytes(1, 1, POLY_CHUNK, POLY_HEAD_DIM, POLY_CHUNK))
    if n <= 0:
        raise RuntimeError("tj_poly_workspace_bytes returned no size")
    return n


def guard_workspace_bytes_per_head() -> int:
    return int(_lib.lib().tj_score_guard_workspace_bytes(1, 1, GUARD_SAMPLES))


def encoder_item_footprint(seq_len: int, d_model: int, num_heads: int, ffn_dim: int, *,
                           poly: bool = False, element_size: int = 4) -> Footprint:
    """Peak bytes of one batch item of the fused encoder forward."""
    if min(seq_len, d_model, num_heads, ffn_dim, element_size) <= 0:
        raise ValueError("sizes must be positive")
    act = seq_len * d_model * element_size
    hidden = seq_len * ffn_dim * element_size
    parts = {
        "residual": act,
        "normed_input": act,
        "qkv": 3 * act,
        "attention_output": act,
    }
    if poly:
        parts["poly_workspace"] = num_heads * poly_workspace_bytes_per_head()
        parts["guard"] = num_heads * (guard_workspace_bytes_per_head() + GUARD_OUTPUT_BYTES_PER_HEAD)
    attention_phase = sum(parts.values())
    ffn_phase = act + hidden + max(act, hidden)
    parts["ffn_phase"] = ffn_phase
    return Footprint(max(attention_phase, ffn_phase), act, parts)


def attention_core_bytes(batch: int, num_heads: int, seq_len: int, head_dim: int, *, poly: bool,
                         element_size: int = 4) -> int:
    """Bytes ``guarded_attention`` (``poly``) or the exact kernel allocates for
    resident q, k, v: the output, plus on the guarded route the polynomial
    workspace and the guard's workspace and outputs."""
    heads = batch * num_heads
    total = heads * seq_len * head_dim * element_size
    if poly:
        total += heads * (poly_workspace_bytes_per_head() + guard_workspace_bytes_per_head()
                          + GUARD_OUTPUT_BYTES_PER_HEAD)
    return total


def available_bytes(device: torch.device, memory_fraction: float = DEFAULT_MEMORY_FRACTION) -> int:
    """Device bytes a forward may still take: the fraction of the device not
    yet allocated, bounded by what is free plus what torch's cache holds
    unused (the reference's rule, ``src/implementations/extreme.py:57-69``)."""
    if not 0.0 < memory_fraction <= 1.0:
        raise ValueError("memory_fraction must be in (0, 1]")
    free, total = torch.cuda.mem_get_info(device)
    allocated = torch.cuda.memory_allocated(device)
    reusable = max(0, torch.cuda.memory_reserved(device) - allocated)
    return max(0, min(int(total * memory_fraction) - allocated, free + reusable))


@dataclass(frozen=True)
class ChunkPlan:
    chunk: int
    budget_bytes: int
    reserved_bytes: int          # output buffer + library allowance
    per_item_bytes: int
    planned_peak_bytes: int      # reserved + chunk * per_item


def plan_batch_chunk(batch_size: int, footprint: Footprint, budget_bytes: int) -> ChunkPlan:
    """Largest power-of-two chunk (at least 1) whose working set fits the budget."""
    if batch_size <= 0:
        raise ValueError("batch_size must be positive")
    if budget_bytes < 0:
        raise ValueError("budget must be non-negative")
    reserved = batch_size * footprint.output_per_item_bytes + LIBRARY_ALLOWANCE_BYTES
    room = max(0, budget_bytes - reserved)
    n = max(1, min(batch_size, room // footprint.per_item_bytes))
    chunk = 1 << (int(n).bit_length() - 1)
    return ChunkPlan(chunk, budget_bytes, reserved, footprint.per_item_bytes,
                     reserved + chunk * footprint.per_item_bytes)


def plan_for_input(x: torch.Tensor, num_heads: int, ffn_dim: int, *, poly: bool,
                   budget_bytes: Optional[int] = None,
                   memory_fraction: float = DEFAULT_MEMORY_FRACTION) -> ChunkPlan:
    """Plan the chunk of a ``[B, S, D]`` input on its device (budget from the
    device unless given)."""
    fp = encoder_item_footprint(x.shape[1], x.shape[2], num_heads, ffn_dim, poly=poly,
                                element_size=x.element_size())
    if budget_bytes is None:
        budget_bytes = available_bytes(x.device, memory_fraction) if x.device.type == "cuda" else 0
    return plan_batch_chunk(x.shape[0], fp, budget_bytes)
