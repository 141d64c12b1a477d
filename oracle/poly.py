"""Degree-2 polynomial linear attention and its sigma guard -- CPU restatement.

Restates, from the reference:

* ``phi2`` and ``hermite_coefficients`` (``src/implementations/poly_reference.py:30-58``);
* ``poly_linear_attention`` (``src/implementations/poly_reference.py:61-265``): the
  chunked causal scan with fp32 state ``(S_const, S_lin, z_lin, G, S_quad)``,
  an exact ``exp`` diagonal block per chunk with no max subtraction, the
  skipped prefix chunks and the exact softmax over the first ``exact_prefix``
  tokens;
* ``estimate_sigma``, ``poly_is_safe`` and ``SIGMA_CEILING``
  (``src/implementations/poly_guard.py:65-102``).

``compute_dtype`` rounds every operand of a contraction to that dtype, as the
reference does by casting ``a, b, v`` and the state shadows before each
matmul. The scan keeps its states in ``state_dtype`` (fp32 by default).
Per-(b,h) coefficients are accepted as a ``[B, H, 3]`` tensor, which is how the
build's device-side guard hands them over; a scalar ``sigma`` reproduces the
reference's one-sigma-per-module behaviour.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple, Union

import torch

from .attention import blockwise_attention

SIGMA_CEILING = 0.40


def phi2(x: torch.Tensor) -> torch.Tensor:
    """``[..., C, D] -> [..., C, D*D]`` with feature ``i*D + j = x_i * x_j``."""
    return (x.unsqueeze(-1) * x.unsqueeze(-2)).flatten(-2)


def hermite_coefficients(sigma: Optional[float]) -> Tuple[float, float, float]:
    """``(c0, c1, c2)`` of the L2-optimal quadratic fit to ``exp(s)``, ``s ~ N(0, sigma^2)``.

    ``exp(s) ~= g * [max(1 - sigma^2/2, 1e-3) + s + s^2/2]`` with
    ``g = exp(sigma^2/2)``; ``None`` is the plain Taylor expansion ``(1, 1, 1/2)``.
    """
    if sigma is None:
        return 1.0, 1.0, 0.5
    g = math.exp(0.5 * sigma * sigma)
    return g * max(1.0 - 0.5 * sigma * sigma, 1e-3), g, 0.5 * g


def coefficient_table(sigmas: torch.Tensor) -> torch.Tensor:
    """Per-head ``[..., 3]`` coefficient tensor from per-head sigmas (fp64)."""
    s2 = sigmas.double() ** 2
    g = torch.exp(0.5 * s2)
    return torch.stack((g * torch.clamp(1.0 - 0.5 * s2, min=1e-3), g, 0.5 * g), dim=-1)


Coeffs = Union[None, float, torch.Tensor]


def _coeff_views(sigma: Coeffs, coeffs: Optional[torch.Tensor], b: int, h: int):
    if coeffs is None:
        c = torch.tensor(hermite_coefficients(sigma), dtype=torch.float64).expand(b, h, 3)
    else:
        c = coeffs.to(torch.float64).expand(b, h, 3)
    return c[..., 0].reshape(b * h, 1, 1), c[..., 1].reshape(b * h, 1, 1), c[..., 2].reshape(b * h, 1, 1)


def poly_linear_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    *,
    chunk: int = 512,
    exact_prefix: int = 4096,
    sigma: Optional[float] = None,
    coeffs: Optional[torch.Tensor] = None,
    state_dtype: torch.dtype = torch.float32,
    compute_dtype: torch.dtype = torch.float32,
    skip_final_state_update: bool = False,
    diag_hook=None,
    update_hook=None,
) -> torch.Tensor:
    """Chunked causal polynomial attention over ``[B, H, N, D]`` tensors.

    With ``a = q*sqrt(scale)`` and ``b = k*sqrt(scale)`` (so ``a.b`` is the
    scaled score), chunk ``[t0, t1)`` emits

        num = c0*S_const + c1*a@S_lin + c2*phi2(a)@S_quad + sum_{j<=i in chunk} exp(a_i.b_j) v_j
        den = c0*t0      + c1*a@z_lin + c2*sum((a@G)*a)   + sum_{j<=i in chunk} exp(a_i.b_j)

    and then folds the chunk into the states. Chunks that end inside the exact
    prefix are not emitted (their rows are overwritten); the final state update
    may be skipped (nothing reads it). Rows ``< exact_prefix`` are exact causal
    softmax attention. ``diag_hook(a, b, v) -> (num, den)`` and
    ``update_hook(b, v)`` exist so the tests can count calls.
    """
    if q.ndim != 4:
        raise ValueError("q, k, v must be [B, H, N, D]")
    b_, h_, n_, d_ = q.shape
    dv = v.shape[-1]
    m_ = b_ * h_
    cdt = compute_dtype
    sdt = state_dtype
    dev = q.device
    rs = math.sqrt(scale)
    c0, c1, c2 = _coeff_views(sigma, coeffs, b_, h_)
    c0, c1, c2 = c0.to(sdt), c1.to(sdt), c2.to(sdt)

    out = torch.empty(b_, h_, n_, dv, dtype=q.dtype, device=dev)
    s_const = torch.zeros(m_, 1, dv, dtype=sdt, device=dev)
    s_lin = torch.zeros(m_, d_, dv, dtype=sdt, device=dev)
    z_lin = torch.zeros(m_, d_, 1, dtype=sdt, device=dev)
    gram = torch.zeros(m_, d_, d_, dtype=sdt, device=dev)
    s_quad = torch.zeros(m_, d_ * d_, dv, dtype=sdt, device=dev)
    prefix_end = min(exact_prefix, n_) if exact_prefix > 0 else 0

    for t0 in range(0, n_, chunk):
        t1 = min(t0 + chunk, n_)
        c = t1 - t0
        a = (q[:, :, t0:t1] * rs).reshape(m_, c, d_).to(cdt)
        b = (k[:, :, t0:t1] * rs).reshape(m_, c, d_).to(cdt)
        vc = v[:, :, t0:t1].reshape(m_, c, dv).to(cdt)

        if t1 > prefix_end:
            if t0 == 0:
                num = torch.zeros(m_, c, dv, dtype=sdt, device=dev)
                den = torch.zeros(m_, c, 1, dtype=sdt, device=dev)
            else:
                num = c0 * s_const + c1 * (a @ s_lin.to(cdt)).to(sdt)
                num = num + c2 * (phi2(a) @ s_quad.to(cdt)).to(sdt)
                den = c0 * float(t0) + c1 * (a @ z_lin.to(cdt)).to(sdt)
                den = den + c2 * ((a @ gram.to(cdt)) * a).sum(-1, keepdim=True).to(sdt)
            if diag_hook is None:
                # exp and the row sum run in at least fp32 (in fp64 for an fp64 scan); the
                # weights are rounded to the compute dtype before the PV product, and the
                # denominator sums the same rounded weights.
                wide = torch.promote_types(cdt, torch.float32)
                upper = torch.ones(c, c, dtype=torch.bool, device=dev).triu(1)
                w = torch.exp((a @ b.transpose(-2, -1)).to(wide)).masked_fill(upper, 0.0).to(cdt)
                d_num = w @ vc
                d_den = w.to(wide).sum(-1, keepdim=True)
            else:
                d_num, d_den = diag_hook(a, b, vc)
            num = num + d_num.to(sdt)
            den = den + d_den.to(sdt)
            out[:, :, t0:t1] = (num / den).to(q.dtype).reshape(b_, h_, c, dv)

        if skip_final_state_update and t1 == n_:
            continue
        if update_hook is not None:
            update_hook(b, vc)
        s_const += vc.sum(1, keepdim=True).to(sdt)
        s_lin += (b.transpose(-2, -1) @ vc).to(sdt)
        z_lin += b.sum(1).unsqueeze(-1).to(sdt)
        gram += (b.transpose(-2, -1) @ b).to(sdt)
        s_quad += (phi2(b).transpose(-2, -1) @ vc).to(sdt)

    if prefix_end > 0:
        w0 = prefix_end
        out[:, :, :w0] = blockwise_attention(
            q[:, :, :w0], k[:, :, :w0], v[:, :, :w0], scale, True, None, 1024, 1024,
            torch.float64 if sdt == torch.float64 else torch.float32,
        ).to(q.dtype)
    return out


def sample_rows(n: int, samples: int = 512, seed: int = 0) -> torch.Tensor:
    """The row sample of ``estimate_sigma``: the first ``min(samples, n)`` of a seeded permutation."""
    gen = torch.Generator().manual_seed(seed)
    return torch.randperm(n, generator=gen)[: min(samples, n)]


def estimate_sigma(q, k, scale: float, samples: int = 512, seed: int = 0, index=None) -> float:
    """Std of the scaled scores over all pairs of a row sample, all heads pooled (``poly_guard.py:68-93``).

    ``torch.std`` semantics (Bessel-corrected). The reference draws the sample
    on the input's device; this restatement draws it on the CPU so that the
    device-side guard and the oracle can share one index set.
    """
    if q.ndim != 4 or k.ndim != 4:
        raise ValueError("q and k must be [B, H, N, D]")
    idx = sample_rows(q.shape[2], samples, seed) if index is None else index
    idx = idx.to(q.device)
    qs = q[:, :, idx].double()
    ks = k[:, :, idx].double()
    return float(((qs @ ks.transpose(-2, -1)) * scale).std().item())


def estimate_sigma_per_head(q, k, scale: float, samples: int = 512, seed: int = 0, index=None) -> torch.Tensor:
    """Per-(b,h) version of ``estimate_sigma``: ``[B, H]`` fp64 stds."""
    idx = sample_rows(q.shape[2], samples, seed) if index is None else index
    idx = idx.to(q.device)
    s = (q[:, :, idx].double() @ k[:, :, idx].double().transpose(-2, -1)) * scale
    return s.flatten(-2).std(dim=-1)


def poly_is_safe(sigma: Optional[float]) -> bool:
    """Validated range of the approximation: ``0 < sigma <= SIGMA_CEILING`` and finite."""
    if sigma is None or math.isnan(sigma) or math.isinf(sigma):
        return False
    return 0.0 < sigma <= SIGMA_CEILING


def guarded_attention(q, k, v, scale: float, *, chunk: int = 512, exact_prefix: int = 4096,
                      samples: int = 512, seed: int = 0, ceiling: float = SIGMA_CEILING,
                      state_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Per-head guarded polynomial attention: the build's semantics, restated on the CPU.

    Heads whose sampled sigma is unsafe get exact causal attention over all
    rows; the others get ``poly_linear_attention`` with their own coefficients.
    """
    sig = estimate_sigma_per_head(q, k, scale, samples, seed)
    safe = torch.isfinite(sig) & (sig > 0) & (sig <= ceiling)
    coeffs = coefficient_table(sig)
    out = poly_linear_attention(q, k, v, scale, chunk=chunk, exact_prefix=exact_prefix,
                                coeffs=coeffs, state_dtype=state_dtype)
    if (~safe).any():
        exact = blockwise_attention(q, k, v, scale, True)
        out = torch.where(safe[:, :, None, None], out, exact)
    return out


def poly_flops(n: int, d: int, dv: int, chunk: int, exact_prefix: int) -> float:
    """Algorithmic FLOPs of one (b,h) of the guarded polynomial path.

    Exact prefix ``2*d*W(W+1)``; per emitted token ``2d^2 dv + 2d dv + 2d^2 + 4d``;
    per non-final-chunk token ``2d^2 dv + 2d dv + 2d^2``; the diagonal
    ``2d*C(C+1)`` per emitted chunk (QK^T and PV over the lower triangle).
    """
    w = min(exact_prefix, n)
    total = 2.0 * d * w * (w + 1)
    prefix_end = w if exact_prefix > 0 else 0
    for t0 in range(0, n, chunk):
        t1 = min(t0 + chunk, n)
        c = t1 - t0
        if t1 > prefix_end:
            total += c * (2 * d * d * dv + 2 * d * dv + 2 * d * d + 4 * d)
            total += 2.0 * d * c * (c + 1)
        if t1 != n:
            total += c * (2 * d * d * dv + 2 * d * dv + 2 * d * d)
    return total
