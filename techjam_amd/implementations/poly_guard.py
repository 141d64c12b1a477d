"""Validity guard of the polynomial attention route.

Mirrors ``src/implementations/poly_guard.py:65-102`` and
``poly_reference.py:35-58``. The degree-2 fit of ``exp`` is accurate only while
the scaled scores stay small -- a property of randomly initialised weights,
not of attention -- so the route is gated on a measured score spread. The
measurement runs in the HIP guard kernel, per ``(b, h)`` and on the device:

* ``guard(q, k, scale)`` returns per-head sigma, flags, coefficients and exact
  row limits as device tensors -- no host synchronisation (the dispatcher's
  path);
* ``estimate_sigma`` keeps the reference's interface (one pooled sigma as a
  Python float, one synchronisation), derived exactly from the per-head
  moments.

Two ceilings, for the two things a caller can require to stay within the
benchmark's OR rule (|d| <= 2e-3 or 2 %):

* ``SIGMA_CEILING`` = 0.40, the reference's calibration, for the model's
  output (``src/implementations/poly_guard.py:22-65``: q/k projection weights
  scaled in both models, the case-14 model's output against the dense
  oracle). Re-measured with this build's kernels the same way: zero failing
  elements through a per-head sigma of 0.489 at N = 8192 and 16384, first
  failures at 0.52 -- 0.40 keeps its margin. The dispatcher's model route
  uses it.
* ``ATTENTION_SIGMA_CEILING`` = 0.29, for the attention output itself (every
  head's output against exact fp32 attention, v ~ N(0, 1)), the default of
  ``guarded_attention``. Largest clean pass 0.30 at N = 8192 .. 131072;
  0.334 fails at N = 16384 (3 of 16.8 M elements) and 0.36 at 8192 -- and the
  reference's scan restated in fp32 fails on the same elements, so that
  boundary is the degree-2 fit's, not the kernel's. Attention feeding a
  residual stream (the case above) tolerates more.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from ..kernels.attention import GuardResult, score_guard

SIGMA_CEILING = 0.40
ATTENTION_SIGMA_CEILING = 0.29


def guard(q: torch.Tensor, k: torch.Tensor, scale: float, *, samples: int = 512, seed: int = 0,
          ceiling: float = SIGMA_CEILING, exact_prefix: int = 4096) -> GuardResult:
    """Per-(b,h) device-side guard; see ``tj_score_guard`` in ``include/techjam_attn.h``."""
    return score_guard(q, k, scale, samples=samples, seed=seed, ceiling=ceiling, exact_prefix=exact_prefix)


def estimate_sigma(q: torch.Tensor, k: torch.Tensor, scale: float, samples: int = 512, seed: int = 0) -> float:
    """Pooled std of the scaled scores of a row sample, all heads together (one host sync)."""
    if q.ndim != 4 or k.ndim != 4:
        raise ValueError("q and k must be [B, H, N, D]")
    res = score_guard(q, k, scale, samples=samples, seed=seed)
    n = min(samples, q.shape[2])
    cnt = float(n * n)
    sig = res.sigma.double().cpu()
    mu = res.mean.double().cpu()
    s1 = mu * cnt
    s2 = sig.pow(2) * (cnt - 1.0) + mu.pow(2) * cnt
    total = cnt * sig.numel()
    mean = float(s1.sum()) / total
    var = (float(s2.sum()) - total * mean * mean) / max(total - 1.0, 1.0)
    return math.sqrt(max(var, 0.0))


def poly_is_safe(sigma: Optional[float]) -> bool:
    """True when the measured spread is inside the validated range (0, SIGMA_CEILING]."""
    if sigma is None or math.isnan(sigma) or math.isinf(sigma):
        return False
    return 0.0 < sigma <= SIGMA_CEILING


def hermite_coefficients(sigma: Optional[float]) -> Tuple[float, float, float]:
    """``(c0, c1, c2)``: ``exp(s) ~ exp(sigma^2/2)*[max(1 - sigma^2/2, 1e-3) + s + s^2/2]``; ``None`` is Taylor."""
    if sigma is None:
        return 1.0, 1.0, 0.5
    g = math.exp(0.5 * sigma * sigma)
    return g * max(1.0 - 0.5 * sigma * sigma, 1e-3), g, 0.5 * g
