"""The stand-alone polynomial kernels against fp32 truth (GPU).

Mirrors the reference's kernel tests (``src/tests/test_poly_kernel.py``,
``src/tests/test_poly_diag.py``): the kernels compute the same sums as dense
fp16 PyTorch in a different order, so each is judged against fp32 truth and
must be no worse than three times the dense fp16 path's error. Plus the
contract properties: accumulate-not-overwrite, the fp16 shadow is exactly the
rounded master, an fp16 master is refused, and the diagonal block is strictly
causal.
"""

from __future__ import annotations

import pytest
import torch

from oracle.poly import phi2

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator(device="cuda").manual_seed(seed)


def _apply_case(M=2, C=128, D=64, V=64, seed=0):
    g = _gen(seed)
    a = torch.randn(M, C, D, generator=g, device="cuda", dtype=torch.float16) * 0.2
    s = torch.randn(M, D * D, V, generator=g, device="cuda", dtype=torch.float32)
    return a, s


def _no_worse(kernel, dense, truth, what):
    k_err = (kernel.float() - truth).abs().max().item()
    d_err = (dense.float() - truth).abs().max().item()
    assert k_err <= max(3.0 * d_err, 1e-6), f"{what}: kernel err {k_err:.3e} vs dense err {d_err:.3e}"


@pytest.mark.parametrize("D,C,V", [(64, 128, 64), (64, 512, 64), (32, 128, 32), (16, 512, 64),
                                   (32, 512, 64), (64, 100, 64), (64, 128, 1)])
def test_quad_apply_matches_dense(cuda, D, C, V):
    from techjam_amd.kernels.poly_parts import quad_apply

    a, s = _apply_case(C=C, D=D, V=V)
    truth = phi2(a.float()) @ s
    dense = phi2(a) @ s.to(a.dtype)
    y = quad_apply(a, s)
    assert y.dtype == torch.float16 and y.shape == (2, C, V)
    _no_worse(y, dense, truth, f"quad_apply D={D} C={C} V={V}")


def test_quad_apply_error_is_rounding_not_bias(cuda):
    from techjam_amd.kernels.poly_parts import quad_apply

    a, s = _apply_case(C=512)
    truth = phi2(a.float()) @ s
    diff = quad_apply(a, s).float() - truth
    assert abs(diff.mean().item()) / truth.abs().mean().item() < 1e-3


@pytest.mark.parametrize("D,C", [(64, 128), (64, 512), (16, 128), (32, 512), (64, 100)])
def test_quad_update_matches_dense(cuda, D, C):
    from techjam_amd.kernels.poly_parts import quad_update

    g = _gen(0)
    b = torch.randn(2, C, D, generator=g, device="cuda", dtype=torch.float16) * 0.2
    v = torch.randn(2, C, 64, generator=g, device="cuda", dtype=torch.float16) * 0.2
    out = torch.zeros(2, D * D, 64, device="cuda", dtype=torch.float32)
    quad_update(b, v, out)
    truth = phi2(b.float()).transpose(-2, -1).contiguous() @ v.float()
    dense = phi2(b).transpose(-2, -1).contiguous() @ v
    _no_worse(out, dense, truth, f"quad_update D={D} C={C}")


def test_quad_update_accumulates_rather_than_overwrites(cuda):
    from techjam_amd.kernels.poly_parts import quad_update

    g = _gen(1)
    b = torch.randn(2, 128, 64, generator=g, device="cuda", dtype=torch.float16) * 0.2
    v = torch.randn(2, 128, 64, generator=g, device="cuda", dtype=torch.float16) * 0.2
    once = torch.zeros(2, 64 * 64, 64, device="cuda", dtype=torch.float32)
    quad_update(b, v, once)
    twice = torch.zeros_like(once)
    quad_update(b, v, twice)
    quad_update(b, v, twice)
    assert (twice - 2 * once).abs().max().item() < 1e-3
    # and a non-zero starting state is added to, not replaced
    start = torch.randn(2, 64 * 64, 64, generator=g, device="cuda")
    acc = start.clone()
    quad_update(b, v, acc)
    assert (acc - start - once).abs().max().item() < 1e-5


def test_quad_update_single_value_column(cuda):
    from techjam_amd.kernels.poly_parts import quad_update

    g = _gen(2)
    b = torch.randn(2, 128, 64, generator=g, device="cuda", dtype=torch.float16) * 0.2
    ones = torch.ones(2, 128, 1, device="cuda", dtype=torch.float16)
    out = torch.zeros(2, 64 * 64, 1, device="cuda", dtype=torch.float32)
    quad_update(b, ones, out)
    truth = phi2(b.float()).transpose(-2, -1).contiguous() @ ones.float()
    assert (out - truth).abs().max().item() < 1e-2


def test_quad_update_refuses_a_float16_master(cuda):
    from techjam_amd.kernels.poly_parts import quad_update

    b = torch.zeros(2, 128, 64, device="cuda", dtype=torch.float16)
    bad = torch.zeros(2, 64 * 64, 64, device="cuda", dtype=torch.float16)
    with pytest.raises(ValueError):
        quad_update(b, b, bad)


@pytest.mark.parametrize("D", [64, 32])
def test_shadow_is_the_float16_rounding_of_the_master(cuda, D):
    from techjam_amd.kernels.poly_parts import quad_apply, quad_update

    g = _gen(3)
    b = torch.randn(2, 128, D, generator=g, device="cuda", dtype=torch.float16) * 0.2
    v = torch.randn(2, 128, 64, generator=g, device="cuda", dtype=torch.float16) * 0.2
    state = torch.zeros(2, D * D, 64, device="cuda", dtype=torch.float32)
    shadow = torch.zeros_like(state, dtype=torch.float16)
    for _ in range(4):
        quad_update(b, v, state, shadow=shadow)
        assert torch.equal(shadow, state.to(torch.float16))
    a = torch.randn(2, 128, D, generator=_gen(7), device="cuda", dtype=torch.float16) * 0.2
    # the apply kernel rounds the master to fp16 itself: bitwise identical
    assert torch.equal(quad_apply(a, state), quad_apply(a, shadow))


def _diag_case(M=2, C=512, D=64, seed=0):
    g = _gen(seed)
    kw = dict(generator=g, device="cuda", dtype=torch.float16)
    return (torch.randn(M, C, D, **kw) * 0.2, torch.randn(M, C, D, **kw) * 0.2, torch.randn(M, C, D, **kw) * 0.2)


# 192 and 64 tokens give row blocks with an odd number of key tiles and a
# single tile (the key sweep is split between two wave groups).
@pytest.mark.parametrize("M,C,D", [(2, 512, 64), (3, 128, 64), (2, 256, 32), (2, 352, 64), (2, 192, 64),
                                   (1, 64, 64), (2, 1000, 64)])
def test_causal_diag_matches_dense(cuda, M, C, D):
    from techjam_amd.kernels.poly_parts import causal_diag

    a, b, v = _diag_case(M, C, D)
    blocked = torch.ones(C, C, device="cuda", dtype=torch.bool).triu(1)
    w = torch.exp(a.float() @ b.float().transpose(-2, -1).contiguous()).masked_fill(blocked, 0.0)
    t_num, t_den = w @ v.float(), w.sum(-1, keepdim=True)
    wd = torch.exp(a @ b.transpose(-2, -1).contiguous()).masked_fill_(blocked, 0.0)
    d_num, d_den = (wd @ v).float(), wd.sum(-1, keepdim=True, dtype=torch.float32)
    num, den = causal_diag(a, b, v)
    assert num.dtype == torch.float32 and den.shape == (M, C, 1)
    _no_worse(num, d_num, t_num, "num")
    _no_worse(den, d_den, t_den, "den")


def test_causal_diag_is_strictly_causal(cuda):
    from techjam_amd.kernels.poly_parts import causal_diag

    a, b, v = _diag_case(M=1, C=128)
    n0, d0 = causal_diag(a, b, v)
    b2, v2 = b.clone(), v.clone()
    b2[:, 64:] *= 7.0
    v2[:, 64:] *= 7.0
    n1, d1 = causal_diag(a, b2, v2)
    assert torch.equal(n0[:, :64], n1[:, :64]) and torch.equal(d0[:, :64], d1[:, :64])


def test_shape_errors_are_value_errors(cuda):
    from techjam_amd.kernels.poly_parts import causal_diag, quad_apply, quad_update

    a = torch.zeros(2, 128, 64, device="cuda", dtype=torch.float16)
    with pytest.raises(ValueError):
        quad_apply(a, torch.zeros(2, 63 * 64, 64, device="cuda"))
    with pytest.raises(ValueError):
        quad_update(a, a, torch.zeros(2, 64 * 64, 32, device="cuda"))
    with pytest.raises(ValueError):
        causal_diag(a, a[:, :64], a)
