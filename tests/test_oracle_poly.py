"""Pins the polynomial-attention oracle and the sigma guard (CPU).

Besides the reference's own known answers (``src/tests/test_poly_reference.py``,
``src/tests/test_poly_guard.py``), the chunked scan is checked against a
definitional O(N^2) form: token i sees earlier chunks through the quadratic
``c0 + c1*s + c2*s^2`` and its own chunk through ``exp(s)``, so a dropped
term, a wrong chunk boundary or a swapped operand fails it.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle.attention import blockwise_attention
from oracle.poly import (
    SIGMA_CEILING,
    coefficient_table,
    estimate_sigma,
    estimate_sigma_per_head,
    guarded_attention,
    hermite_coefficients,
    phi2,
    poly_flops,
    poly_is_safe,
    poly_linear_attention,
    sample_rows,
)

F64 = dict(state_dtype=torch.float64, compute_dtype=torch.float64)
F32 = dict(state_dtype=torch.float32, compute_dtype=torch.float32)


def _qkv(b=1, h=2, n=1024, d=64, seed=0, std=0.577, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return tuple((torch.randn(b, h, n, d, generator=g) * std).to(dtype) for _ in range(3)) + (d ** -0.5,)


def definitional(q, k, v, scale, chunk, exact_prefix, coeffs):
    """O(N^2) statement of the chunked polynomial attention, in float64."""
    q, k, v = q.double(), k.double(), v.double()
    b_, h_, n, _ = q.shape
    s = (q @ k.transpose(-2, -1)) * scale                         # [B, H, N, N]
    c = coeffs.double().view(b_, h_, 1, 1, 3)
    poly = c[..., 0] + c[..., 1] * s + c[..., 2] * s * s
    i = torch.arange(n)
    same_chunk = (i[:, None] // chunk) == (i[None, :] // chunk)
    causal = i[None, :] <= i[:, None]
    w = torch.where(same_chunk, torch.exp(s), poly) * causal
    out = (w @ v) / w.sum(-1, keepdim=True)
    w0 = min(exact_prefix, n)
    if w0:
        out[:, :, :w0] = F.scaled_dot_product_attention(q[:, :, :w0], k[:, :, :w0], v[:, :, :w0],
                                                        is_causal=True, scale=scale)
    return out


@pytest.mark.parametrize("n,chunk,prefix", [(256, 64, 0), (300, 64, 100), (512, 128, 128), (200, 512, 0)])
def test_scan_equals_definitional_form(n, chunk, prefix):
    q, k, v, scale = _qkv(b=2, h=2, n=n, d=16, std=0.7, dtype=torch.float64)
    coeffs = coefficient_table(torch.tensor([[0.2, 0.3], [0.334, 0.5]], dtype=torch.float64))
    got = poly_linear_attention(q, k, v, scale, chunk=chunk, exact_prefix=prefix, coeffs=coeffs, **F64)
    ref = definitional(q, k, v, scale, chunk, prefix, coeffs)
    assert torch.allclose(got, ref, atol=1e-10, rtol=1e-10)


def test_scalar_sigma_equals_broadcast_coefficients():
    q, k, v, scale = _qkv(n=256, d=16)
    a = poly_linear_attention(q, k, v, scale, chunk=64, exact_prefix=0, sigma=0.3, **F32)
    c = torch.tensor(hermite_coefficients(0.3)).expand(1, 2, 3)
    b = poly_linear_attention(q, k, v, scale, chunk=64, exact_prefix=0, coeffs=c, **F32)
    assert torch.equal(a, b)


def test_prefix_region_is_exact():
    q, k, v, scale = _qkv(n=512)
    got = poly_linear_attention(q, k, v, scale, chunk=128, exact_prefix=512, sigma=0.334, **F32)
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale)
    assert (got - ref).abs().max().item() < 1e-5


def test_exact_prefix_covering_everything_is_exact_attention():
    q, k, v, scale = _qkv(n=300)
    got = poly_linear_attention(q, k, v, scale, chunk=64, exact_prefix=4096, sigma=0.334, **F32)
    ref = blockwise_attention(q, k, v, scale, True)
    assert (got - ref).abs().max().item() < 1e-5


def test_approximation_is_close_to_softmax_attention():
    q, k, v, scale = _qkv(n=2048)
    got = poly_linear_attention(q, k, v, scale, chunk=512, exact_prefix=512, sigma=0.334, **F32)
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale)
    rel = ((got - ref).pow(2).mean().sqrt() / ref.pow(2).mean().sqrt()).item()
    assert rel < 0.02


def test_hermite_constant_beats_plain_taylor():
    q, k, v, scale = _qkv(n=2048)
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale)
    kw = dict(chunk=512, exact_prefix=512, **F32)
    taylor = poly_linear_attention(q, k, v, scale, sigma=None, **kw)
    hermite = poly_linear_attention(q, k, v, scale, sigma=0.334, **kw)
    assert (hermite - ref).pow(2).mean() < (taylor - ref).pow(2).mean()


@pytest.mark.parametrize("sigma", [0.2, 0.334, 0.5])
def test_coefficients_match_the_mean_of_exp(sigma):
    """E[c0 + c1 s + c2 s^2] = exp(sigma^2/2) = E[exp(s)] for s ~ N(0, sigma^2)."""
    c0, _, c2 = hermite_coefficients(sigma)
    assert math.isclose(c0 + c2 * sigma * sigma, math.exp(0.5 * sigma * sigma), rel_tol=1e-12)


def test_coefficient_fit_is_the_gauss_hermite_projection():
    """The fit is the L2 projection of exp onto {1, s, s^2} under N(0, sigma^2) (numerical quadrature)."""
    import numpy as np

    sigma = 0.3
    x, w = np.polynomial.hermite_e.hermegauss(60)
    s = sigma * x
    basis = np.stack([np.ones_like(s), s, s * s], axis=1)
    gram = basis.T @ (w[:, None] * basis)
    rhs = basis.T @ (w * np.exp(s))
    fit = np.linalg.solve(gram, rhs)
    assert np.allclose(fit, hermite_coefficients(sigma), rtol=1e-9)


def test_taylor_coefficients_are_unscaled():
    assert hermite_coefficients(None) == (1.0, 1.0, 0.5)


def test_coefficient_table_matches_scalar_form():
    sig = torch.tensor([0.1, 0.25, 0.4, 2.0])
    tab = coefficient_table(sig)
    for i, s in enumerate(sig.tolist()):
        assert torch.allclose(tab[i], torch.tensor(hermite_coefficients(s), dtype=torch.float64))


def test_phi2_inner_product_is_the_squared_score():
    g = torch.Generator().manual_seed(1)
    a, b = torch.randn(5, 16, generator=g, dtype=torch.float64), torch.randn(5, 16, generator=g, dtype=torch.float64)
    assert torch.allclose((phi2(a) * phi2(b)).sum(-1), (a * b).sum(-1) ** 2)


def test_batch_and_head_dims_are_independent():
    q, k, v, scale = _qkv(b=2, h=3, n=512)
    kw = dict(chunk=128, exact_prefix=128, sigma=0.334, **F32)
    full = poly_linear_attention(q, k, v, scale, **kw)
    one = poly_linear_attention(q[1:2, 2:3], k[1:2, 2:3], v[1:2, 2:3], scale, **kw)
    assert torch.allclose(full[1:2, 2:3], one, atol=1e-6)


def _dense_diag(a, b, vc):
    blocked = torch.ones(a.shape[1], b.shape[1], dtype=torch.bool).triu(1)
    w = torch.exp(a @ b.transpose(-2, -1)).masked_fill_(blocked, 0.0)
    return (w @ vc).float(), w.sum(-1, keepdim=True, dtype=torch.float32)


def test_chunks_inside_the_exact_prefix_are_not_computed():
    q, k, v, scale = _qkv(n=1024)
    calls = []

    def counting(a, b, vc):
        calls.append(a.shape[1])
        return _dense_diag(a, b, vc)

    poly_linear_attention(q, k, v, scale, chunk=256, exact_prefix=512, sigma=0.334, diag_hook=counting, **F32)
    assert len(calls) == 2


def test_final_state_update_can_be_skipped_bitwise():
    q, k, v, scale = _qkv(n=1024)
    calls = []
    kw = dict(chunk=256, exact_prefix=0, sigma=0.334, update_hook=lambda b, v: calls.append(1), **F32)
    full = poly_linear_attention(q, k, v, scale, **kw)
    assert len(calls) == 4
    calls.clear()
    skipped = poly_linear_attention(q, k, v, scale, skip_final_state_update=True, **kw)
    assert len(calls) == 3
    assert torch.equal(full, skipped)


def test_ragged_final_chunk_is_finite_and_close():
    q, k, v, scale = _qkv(n=1536 + 77)
    got = poly_linear_attention(q, k, v, scale, chunk=512, exact_prefix=0, sigma=0.334, **F32)
    ref = definitional(q, k, v, scale, 512, 0, torch.tensor(hermite_coefficients(0.334)).expand(1, 2, 3))
    assert torch.isfinite(got).all()
    assert (got.double() - ref).abs().max() < 1e-4


# -- guard ---------------------------------------------------------------------

def _qk(d=64, n=4096, scaleup=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(1, 2, n, d, generator=g) * 0.577 * scaleup,
            torch.randn(1, 2, n, d, generator=g) * 0.577 * scaleup, d ** -0.5)


def test_guard_recovers_the_benchmark_sigma():
    q, k, scale = _qk()
    assert abs(estimate_sigma(q, k, scale) - 0.334) < 0.02


def test_sigma_scales_with_input_magnitude():
    q1, k1, scale = _qk()
    q2, k2, _ = _qk(scaleup=2.0)
    assert abs(estimate_sigma(q2, k2, scale) / estimate_sigma(q1, k1, scale) - 4.0) < 0.5


def test_estimate_is_stable_across_sample_draws():
    q, k, scale = _qk()
    assert abs(estimate_sigma(q, k, scale, seed=1) - estimate_sigma(q, k, scale, seed=2)) < 0.01


def test_full_sample_equals_population_std():
    q, k, scale = _qk(n=64)
    got = estimate_sigma(q, k, scale, samples=512)
    direct = ((q.double() @ k.double().transpose(-2, -1)) * scale).std().item()
    assert math.isclose(got, direct, rel_tol=1e-12)


def test_pooled_and_per_head_sigmas_agree_when_heads_match():
    q, k, scale = _qk()
    per = estimate_sigma_per_head(q, k, scale)
    assert per.shape == (1, 2)
    assert abs(float(per.mean()) - estimate_sigma(q, k, scale)) < 0.01


def test_sample_rows_clamped_and_distinct():
    idx = sample_rows(64, 512, 0)
    assert idx.numel() == 64 and len(set(idx.tolist())) == 64
    assert sample_rows(10000, 512, 0).numel() == 512


def test_safety_thresholds():
    assert poly_is_safe(0.334)
    assert not poly_is_safe(SIGMA_CEILING + 0.01)
    for bad in (float("nan"), float("inf"), None, 0.0, 0.5217, 0.5642, 0.6544, 0.7512):
        assert not poly_is_safe(bad)
    for ok in (0.3327, 0.3339, 0.3343):
        assert poly_is_safe(ok)
    assert 0.334 < SIGMA_CEILING <= 0.4188


def test_guard_rejects_wrongly_shaped_inputs():
    q, k, scale = _qk()
    with pytest.raises(ValueError):
        estimate_sigma(q[0], k[0], scale)


def test_guarded_attention_routes_wide_heads_to_exact():
    g = torch.Generator().manual_seed(4)
    b, h, n, d = 1, 3, 1024, 64
    std = torch.tensor([0.5, 2.0, 0.5]).view(1, 3, 1, 1)
    q, k = torch.randn(b, h, n, d, generator=g) * std, torch.randn(b, h, n, d, generator=g) * std
    v = torch.randn(b, h, n, d, generator=g)
    out = guarded_attention(q, k, v, d ** -0.5, chunk=256, exact_prefix=256)
    exact = blockwise_attention(q, k, v, d ** -0.5, True)
    assert torch.allclose(out[:, 1], exact[:, 1], atol=1e-6)          # fallback head is exact
    assert not torch.allclose(out[:, 0], exact[:, 0], atol=1e-7)      # poly head approximates...
    err = out[:, 0] - exact[:, 0]
    assert (err.pow(2).mean().sqrt() / exact[:, 0].pow(2).mean().sqrt()) < 0.02  # ...closely


def test_poly_flops_closed_form_for_the_extreme_workload():
    d = dv = 64
    n, c, w = 65536, 512, 4096
    emitted, updated = (n - w) // c, n // c - 1
    expect = (2 * d * w * (w + 1) + emitted * c * (2 * d * d * dv + 2 * d * dv + 2 * d * d + 4 * d)
              + emitted * 2 * d * c * (c + 1) + updated * c * (2 * d * d * dv + 2 * d * dv + 2 * d * d))
    assert poly_flops(n, d, dv, c, w) == expect
