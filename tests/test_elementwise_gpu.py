"""Fused block tails (bias + residual + row zeroing, bias + exact GELU) against
the plain tensor ops they replace (GPU)."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _case(cuda, b=3, s=37, c=64, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(b, s, c, generator=g, device="cuda")
    y = torch.randn(b, s, c, generator=g, device="cuda")
    bias = torch.randn(c, generator=g, device="cuda")
    lens = torch.tensor([s, 1, s // 2][:b], dtype=torch.int32, device="cuda")
    mask = torch.arange(s, device="cuda")[None, :] < lens[:, None]
    return x, y, bias, lens, mask


@pytest.mark.parametrize("masked", [False, True])
def test_bias_residual_modes_match_tensor_ops(cuda, masked):
    from techjam_amd.kernels.elementwise import MODE_PLAIN, MODE_ZERO_OUT, MODE_ZERO_Y, bias_residual

    x, y, bias, lens, mask = _case(cuda)
    vl = lens if masked else None
    m = mask[..., None] if masked else torch.ones_like(mask)[..., None]
    want0 = x + (y + bias)
    want1 = x + (y + bias).masked_fill(~m, 0)
    want2 = (x + (y + bias)).masked_fill(~m, 0)
    assert torch.equal(bias_residual(x, y, bias, None, MODE_PLAIN), want0)
    assert torch.equal(bias_residual(x, y, bias, vl, MODE_ZERO_Y), want1)
    assert torch.equal(bias_residual(x, y, bias, vl, MODE_ZERO_OUT), want2)


def test_bias_residual_may_write_over_its_input(cuda):
    from techjam_amd.kernels.elementwise import MODE_ZERO_OUT, bias_residual

    x, y, bias, lens, mask = _case(cuda, seed=1)
    want = (x + (y + bias)).masked_fill(~mask[..., None], 0)
    out = bias_residual(x, y, bias, lens, MODE_ZERO_OUT, out=y)
    assert out.data_ptr() == y.data_ptr() and torch.equal(out, want)


def test_bias_residual_zeroes_non_finite_padded_rows(cuda):
    from techjam_amd.kernels.elementwise import MODE_ZERO_OUT, MODE_ZERO_Y, bias_residual

    x, y, bias, lens, mask = _case(cuda, seed=2)
    y[1, 5:] = float("inf")  # padded rows of sample 1 (length 1)
    assert torch.isfinite(bias_residual(x, y, bias, lens, MODE_ZERO_Y)).all()
    out = bias_residual(x, y, bias, lens, MODE_ZERO_OUT)
    assert float(out[~mask].abs().max()) == 0.0


def test_bias_gelu_matches_exact_gelu(cuda):
    from techjam_amd.kernels.elementwise import bias_gelu

    x, y, bias, _, _ = _case(cuda, c=256, seed=3)
    want = F.gelu(y * 3 + bias, approximate="none")
    got = bias_gelu((y * 3).contiguous(), bias)
    assert (got - want).abs().max().item() < 1e-6


def test_unsupported_layouts_are_declined(cuda):
    from techjam_amd.kernels.elementwise import MODE_PLAIN, bias_gelu, bias_residual

    x, y, bias, _, _ = _case(cuda, c=66)
    assert bias_residual(x, y, bias, None, MODE_PLAIN) is None        # width not a multiple of 4
    x, y, bias, _, _ = _case(cuda)
    assert bias_residual(x.transpose(0, 1), y.transpose(0, 1), bias, None, MODE_PLAIN) is None
    assert bias_gelu(y.half(), bias.half()) is None                     # fp32 only


@pytest.mark.parametrize("c", [32, 64, 128, 256, 512, 1024, 2048])
@pytest.mark.parametrize("masked", [False, True])
def test_bias_residual_layernorm_matches_tensor_ops(cuda, c, masked):
    """The residual pass is bitwise the tensor ops; the fused LayerNorm is
    within fp32 rounding of torch's (two exact passes vs torch's reduction)."""
    from techjam_amd.kernels.elementwise import MODE_ZERO_OUT, MODE_ZERO_Y, bias_residual_layernorm

    x, y, bias, lens, mask = _case(cuda, c=c, seed=10 + c)
    norm = torch.nn.LayerNorm(c).to(cuda)
    with torch.no_grad():
        norm.weight.normal_(1.0, 0.2)
        norm.bias.normal_(0.0, 0.2)
    vl = lens if masked else None
    m = mask[..., None] if masked else torch.ones_like(mask)[..., None]
    for mode, want in ((MODE_ZERO_Y, x + (y + bias).masked_fill(~m, 0)),
                       (MODE_ZERO_OUT, (x + (y + bias)).masked_fill(~m, 0))):
        for zero in (False, True):
            out, ln = bias_residual_layernorm(x, y, bias, vl, mode, norm, zero_padded_norm=zero)
            assert torch.equal(out, want)
            want_ln = F.layer_norm(want, (c,), norm.weight, norm.bias, norm.eps)
            if zero and masked:
                want_ln = want_ln.masked_fill(~m, 0)
            err = (ln - want_ln).abs().max().item()
            assert err < 2e-5, f"mode {mode} zero {zero}: {err:.2e}"


def test_bias_residual_layernorm_in_place_and_unsupported_widths(cuda):
    from techjam_amd.kernels.elementwise import MODE_ZERO_OUT, bias_residual_layernorm

    x, y, bias, lens, mask = _case(cuda, c=512, seed=21)
    norm = torch.nn.LayerNorm(512).to(cuda)
    want = (x + (y + bias)).masked_fill(~mask[..., None], 0)
    out, ln = bias_residual_layernorm(x, y, bias, lens, MODE_ZERO_OUT, norm, out=y)
    assert out.data_ptr() == y.data_ptr() and torch.equal(out, want)
    assert (ln - F.layer_norm(want, (512,), norm.weight, norm.bias, norm.eps)).abs().max().item() < 2e-5
    for c in (16, 96, 768, 4096):  # none of 32, 64, 128 or a power-of-two multiple of 256 up to 2048
        x, y, bias, lens, _ = _case(cuda, c=c, seed=22)
        assert bias_residual_layernorm(x, y, bias, lens, MODE_ZERO_OUT, torch.nn.LayerNorm(c).to(cuda)) is None


def test_fp16_outputs_are_the_fp32_results_rounded(cuda):
    """With fp16 GEMM operands the GELU and LayerNorm kernels write the fp16
    operand directly: the fp32 result rounded to fp16 (the cast pass it
    replaces) -- bitwise for GELU; for the norm within one fp16 ulp (the
    affine step may contract into an fma differently in the two instances)
    -- with the fp32 residual stream unchanged."""
    from techjam_amd.kernels.elementwise import MODE_ZERO_Y, bias_gelu, bias_residual_layernorm

    x, y, bias, lens, _ = _case(cuda, c=1024, seed=31)
    h = (y * 3).contiguous()
    want = bias_gelu(h.clone(), bias)
    got = bias_gelu(h, bias, out_f16=True)
    assert got.dtype == torch.float16 and torch.equal(got, want.half())
    assert torch.equal(h, (y * 3))  # the fp32 input is left as it was
    norm = torch.nn.LayerNorm(1024).to(cuda)
    with torch.no_grad():
        norm.weight.normal_(1.0, 0.2)
        norm.bias.normal_(0.0, 0.2)
    out32, ln32 = bias_residual_layernorm(x, y, bias, lens, MODE_ZERO_Y, norm)
    out16, ln16 = bias_residual_layernorm(x, y, bias, lens, MODE_ZERO_Y, norm, norm_dtype=torch.float16)
    assert ln16.dtype == torch.float16 and torch.equal(out16, out32)
    ulp = torch.where(ln32.abs() < 2 ** -14, torch.full_like(ln32, 2 ** -24),
                      torch.exp2(torch.floor(torch.log2(ln32.abs())) - 10))
    assert bool(((ln16.float() - ln32).abs() <= ulp).all())
    assert (ln16 != ln32.half()).float().mean().item() < 1e-3


def test_bias_relu_matches_relu(cuda):
    from techjam_amd.kernels.elementwise import bias_relu

    x, y, bias, _, _ = _case(cuda, c=256, seed=7)
    want = F.relu(y + bias)
    h16 = bias_relu(y.clone(), bias, out_f16=True)
    assert h16.dtype == torch.float16 and torch.equal(h16, want.half())
    got = bias_relu(y, bias)
    assert got.data_ptr() == y.data_ptr() and torch.equal(got, want)


@pytest.mark.parametrize("masked", [False, True])
@torch.no_grad()
def test_layernorm_only_pass_matches_the_full_pass(cuda, masked):
    """Without ``keep_sum`` (the post-norm block) the norm is bitwise the one
    the pass computes when it also stores the sum."""
    from techjam_amd.kernels.elementwise import MODE_PLAIN, MODE_ZERO_Y, bias_residual_layernorm

    x, y, bias, lens, mask = _case(cuda, c=512, seed=8)
    norm = torch.nn.LayerNorm(512).to(cuda)
    norm.weight.uniform_(0.5, 1.5)
    norm.bias.uniform_(-0.5, 0.5)
    vl = lens if masked else None
    for mode in (MODE_PLAIN, MODE_ZERO_Y):
        s_full, ln_full = bias_residual_layernorm(x, y, bias, vl, mode, norm, zero_padded_norm=masked)
        s_none, ln_only = bias_residual_layernorm(x, y, bias, vl, mode, norm, zero_padded_norm=masked,
                                                  keep_sum=False)
        assert s_none is None and torch.equal(ln_only, ln_full)
        want = F.layer_norm(s_full, (512,), norm.weight, norm.bias, norm.eps)
        if masked:
            want = want.masked_fill(~mask[..., None], 0)
        assert float((ln_only - want).abs().max()) < 1e-5
