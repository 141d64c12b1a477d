"""Mask classification and the per-forward attention route.

Restates ``src/implementations/attention_routing.py:15-98`` for the HIP
kernels. ``classify_mask`` keeps the reference's semantics exactly: one host
synchronisation, ``PREFIX`` iff the mask never rises along the sequence.
``select_route`` is a pure function, testable without a GPU; its routes are
the kernel's masking modes rather than SDPA backends:

* no mask                      -> ``KERNEL`` (plain or causal attention);
* right-padded (prefix) mask   -> ``KERNEL_VALID_LENGTHS``: the mask becomes a
  per-sample length. Keys past it are excluded and padded rows are skipped
  (written as zeros). Under causal attention excluding the keys is redundant
  -- every valid row i only sees keys j <= i < L, the property the reference
  pins bitwise in ``test_padding_mask_redundancy.py`` -- so the length only
  saves the padded query tiles;
* any other mask               -> ``REFUSE``: the kernels take lengths, not
  arbitrary masks, and there is no fallback.
"""

from __future__ import annotations

import enum
from typing import Any, Optional


class MaskKind(enum.Enum):
    """How much structure a ``valid_token_mask`` has."""

    ABSENT = "absent"
    PREFIX = "prefix"
    GENERAL = "general"


class Route(enum.Enum):
    """Masking mode of the HIP exact-attention kernel for one forward."""

    KERNEL = "kernel"
    KERNEL_VALID_LENGTHS = "kernel_valid_lengths"
    REFUSE = "refuse"


def select_route(dtype_supported: bool, causal: bool, mask_kind: MaskKind) -> Route:
    """The kernel mode for one forward; ``causal`` does not change it (see module docstring)."""
    del causal
    if not dtype_supported or mask_kind is MaskKind.GENERAL:
        return Route.REFUSE
    if mask_kind is MaskKind.ABSENT:
        return Route.KERNEL
    return Route.KERNEL_VALID_LENGTHS


def classify_mask(valid_token_mask: Optional[Any]) -> MaskKind:
    """Classify a ``[B, N]`` bool mask with ONE host synchronisation.

    ``PREFIX`` when no row rises along the sequence axis (right padding, the
    shape ``generate_random_case`` produces); a length-1 axis is trivially
    prefix. Call it once per forward, above the layer loop, never inside a
    captured or replayed region.
    """
    if valid_token_mask is None:
        return MaskKind.ABSENT
    if valid_token_mask.shape[-1] <= 1:
        return MaskKind.PREFIX
    non_increasing = bool((valid_token_mask[:, :-1] >= valid_token_mask[:, 1:]).all())
    return MaskKind.PREFIX if non_increasing else MaskKind.GENERAL
