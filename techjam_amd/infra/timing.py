"""Interleaved timing with an A/A control, and the noise floor it yields.

Mirrors the reference's paired-timing statistics (``src/bench_poly.py:30-127``):
variants are timed by alternating them, every sample is kept, and the floor a
difference must clear is the gap between the minima of two arms that run the
*same* callable. Field names of the summary match the reference's so records
from either harness read the same way.
"""

from __future__ import annotations

import time
from typing import Callable, Dict, Iterable, List, Mapping, Sequence, Tuple


def _default_sync() -> Callable[[], None]:
    import torch

    if torch.cuda.is_available():
        return torch.cuda.synchronize
    return lambda: None


def time_interleaved(variants: Mapping[str, Callable[[], object]], reps: int = 5,
                     sync: Callable[[], None] | None = None) -> Dict[str, List[float]]:
    """Milliseconds per call of each variant, ``reps`` samples each.

    Every variant runs once untimed, then the variants take turns, one call
    per turn, so clock drift over the session lands on all of them alike
    (``bench_poly.py:30-56``). Each sample is the wall time between a device
    synchronisation before and after the call.
    """
    if reps < 1:
        raise ValueError("reps must be >= 1")
    sync = sync or _default_sync()
    for fn in variants.values():
        fn()
    sync()
    samples: Dict[str, List[float]] = {name: [] for name in variants}
    for _ in range(reps):
        for name, fn in variants.items():
            sync()
            t0 = time.perf_counter()
            fn()
            sync()
            samples[name].append((time.perf_counter() - t0) * 1e3)
    return samples


def _median(ordered: Sequence[float]) -> float:
    n = len(ordered)
    half = n // 2
    return ordered[half] if n % 2 else 0.5 * (ordered[half - 1] + ordered[half])


def summarise_timings(samples: Mapping[str, Sequence[float]],
                      control_pairs: Iterable[Tuple[str, str]] = ()) -> dict:
    """Per-variant min / median / max / spread and the A/A noise floor.

    ``control_pairs`` names pairs of variants that ran the same code. The
    floor is the largest relative gap between the minima of such a pair --
    the statistic an A/B compares -- and, only without any pair, the largest
    within-variant spread ``(max - min) / min`` (``bench_poly.py:59-122``).
    ``minimum_detectable_effect`` is ``1 + floor``: ratios inside
    ``[1/mde, mde]`` are not distinguishable from noise.
    """
    stats = {}
    for name, values in samples.items():
        if not values:
            raise ValueError(f"variant {name!r} has no samples")
        ordered = sorted(values)
        low = ordered[0]
        stats[name] = {
            "min_ms": low,
            "median_ms": _median(ordered),
            "max_ms": ordered[-1],
            "spread": (ordered[-1] - low) / low if low else 0.0,
            "reps": len(ordered),
        }

    discrepancy = None
    paired = None
    for left, right in control_pairs:
        lo_a, lo_b = stats[left]["min_ms"], stats[right]["min_ms"]
        gap = abs(lo_a - lo_b) / min(lo_a, lo_b)
        discrepancy = gap if discrepancy is None else max(discrepancy, gap)
        for x, y in zip(samples[left], samples[right]):
            one = abs(x - y) / min(x, y)
            paired = one if paired is None else max(paired, one)

    spread = max((s["spread"] for s in stats.values()), default=0.0)
    floor = discrepancy if discrepancy is not None else spread
    return {
        "variants": stats,
        "noise": {
            "aa_discrepancy": discrepancy,
            "worst_paired_aa_discrepancy": paired,
            "worst_within_variant_spread": spread,
            "minimum_detectable_effect": 1.0 + floor,
        },
    }


def is_resolvable(ratio: float, minimum_detectable_effect: float) -> bool:
    """True when ``ratio`` (either direction) lies outside the noise floor
    (``bench_poly.py:125-129``)."""
    if ratio <= 0:
        return False
    return max(ratio, 1.0 / ratio) >= minimum_detectable_effect
