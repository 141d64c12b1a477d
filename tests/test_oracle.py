"""Pins the oracle against definitions, closed forms and the reference's known answers (CPU).

Each oracle function is checked against something independent of its own
formula: float64 brute force, torch's SDPA math path, bitwise properties the
reference pins, or the known answers of the reference's tests.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.attention import (
    LinearMemoryReference,
    blockwise_attention,
    brute_force_attention,
    compare_outputs_streamed,
    exact_attention_flops,
)
from oracle.model import (
    DenseTransformer,
    TransformerConfig,
    compare_outputs,
    copy_model_weights,
    generate_random_case,
)


def _qkv(b=2, h=3, s=40, d=16, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(b, h, s, d, generator=g, dtype=torch.float64) * scale for _ in range(3))


# -- exact attention ---------------------------------------------------------

@pytest.mark.parametrize("causal", [True, False])
def test_brute_force_matches_torch_sdpa_math(causal):
    q, k, v = _qkv()
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=causal, scale=0.25)
    np.testing.assert_allclose(brute_force_attention(q, k, v, 0.25, causal), ref.numpy(), atol=1e-12)


def test_brute_force_first_causal_row_is_the_first_value():
    q, k, v = _qkv()
    out = brute_force_attention(q, k, v, 0.3, True)
    np.testing.assert_allclose(out[:, :, 0], v[:, :, 0].numpy(), atol=1e-14)


def test_brute_force_valid_lengths_match_sdpa_with_key_mask():
    q, k, v = _qkv(b=3)
    lengths = [40, 17, 1]
    mask = torch.arange(40)[None, :] < torch.tensor(lengths)[:, None]
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=mask[:, None, None, :], scale=0.25)
    ref = ref.masked_fill(~mask[:, None, :, None], 0)  # padded rows are zero by contract
    np.testing.assert_allclose(brute_force_attention(q, k, v, 0.25, False, valid_len=lengths), ref.numpy(),
                               atol=1e-12)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("blocks", [(7, 5), (16, 64), (64, 3)])
def test_blockwise_equals_brute_force(causal, blocks):
    q, k, v = _qkv(s=61)
    lengths = torch.tensor([61, 30])
    for vl in (None, lengths):
        got = blockwise_attention(q, k, v, 0.25, causal, vl, *blocks, acc_dtype=torch.float64)
        ref = brute_force_attention(q, k, v, 0.25, causal, None if vl is None else vl.tolist())
        np.testing.assert_allclose(got.numpy(), ref, atol=1e-12)


def test_blockwise_handles_wide_score_ranges():
    q, k, v = _qkv(s=64, scale=6.0)
    got = blockwise_attention(q, k, v, 0.125, True, None, 16, 16, acc_dtype=torch.float64)
    np.testing.assert_allclose(got.numpy(), brute_force_attention(q, k, v, 0.125, True), atol=1e-10)


def test_exact_attention_flops_closed_form():
    # L(L+1) summed per sample: the lower triangle including the diagonal, QK^T and PV.
    assert exact_attention_flops([4096] * 64, 16, 64) == 2 * 64 * 16 * 64 * 4096 * 4097
    assert exact_attention_flops([1], 1, 64) == 2 * 64 * 2


# -- dense model, inputs and checker ---------------------------------------------

def test_checker_or_rule_known_answer():
    """Reference test_fp32_reference.py:83-91: exactly one failure."""
    ref = torch.tensor([[[0.0, 1.0, 100.0]]])
    got = torch.tensor([[[0.0019, 1.019, 102.001]]])
    assert compare_outputs_streamed(ref, got, atol=0.002, rtol=0.02, token_chunk=1).failed_elements == 1
    assert compare_outputs(ref, got, rtol=0.02, atol=0.002).failed_elements == 1


def test_checker_rejects_non_finite():
    ref = torch.zeros(1, 1, 3)
    got = torch.tensor([[[0.0, float("nan"), float("inf")]]])
    assert compare_outputs(ref, got, rtol=0.02, atol=0.002).failed_elements == 2


def test_generated_masks_are_right_padded_and_in_range():
    cfg = TransformerConfig(16, 32, 8, 2, 8, 1, True)
    for ratio in (0.1, 0.5, 0.9):
        x, mask = generate_random_case(cfg, torch.device("cpu"), torch.float32, 3, ratio, 1.0)
        assert not bool((mask[:, :-1] < mask[:, 1:]).any())
        lengths = mask.sum(1)
        assert int(lengths.min()) >= max(1, round(32 * (1 - ratio))) and int(lengths.max()) <= 32
        assert float(x[~mask].abs().sum()) == 0.0


def test_unpadded_case_has_full_mask():
    cfg = TransformerConfig(2, 8, 4, 1, 4, 1, True)
    _, mask = generate_random_case(cfg, torch.device("cpu"), torch.float32, 1, 0.0, 1.0)
    assert bool(mask.all())


def _reference_style_attention(block, x, mask, causal):
    """Independent restatement with einsum (different contraction order)."""
    a = block.attention
    b, s, d = x.shape
    def heads(t):
        return t.view(b, s, a.num_heads, a.head_dim)
    q, k, v = heads(a.q_proj(x)), heads(a.k_proj(x)), heads(a.v_proj(x))
    scores = torch.einsum("bshd,bthd->bhst", q, k) * a.scale
    if causal:
        scores = scores.masked_fill(torch.ones(s, s, dtype=torch.bool).triu(1), float("-inf"))
    if mask is not None:
        scores = scores.masked_fill(~mask[:, None, None, :], float("-inf"))
    p = torch.softmax(scores, -1)
    ctx = torch.einsum("bhst,bthd->bshd", p, v).reshape(b, s, d)
    out = a.out_proj(ctx)
    return out.masked_fill(~mask[..., None], 0) if mask is not None else out


def test_dense_model_matches_an_einsum_restatement():
    cfg = TransformerConfig(3, 24, 32, 4, 48, 2, True)
    torch.manual_seed(7)
    model = DenseTransformer(cfg).double().eval()
    x, mask = generate_random_case(cfg, torch.device("cpu"), torch.float64, 11, 0.5, 1.0)
    with torch.inference_mode():
        got = model(x, mask)
        h = x
        for layer in model.layers:
            h = h + _reference_style_attention(layer, layer.norm1(h), mask, True)
            h = h + layer.ffn_out(F.gelu(layer.ffn_in(layer.norm2(h)), approximate="none"))
            h = h.masked_fill(~mask[..., None], 0)
        ref = model.final_norm(h).masked_fill(~mask[..., None], 0)
    assert torch.allclose(got, ref, atol=1e-12)


def test_seeded_construction_order_and_state_dict_names():
    cfg = TransformerConfig(1, 4, 8, 2, 16, 2, True)
    torch.manual_seed(123)
    a = DenseTransformer(cfg)
    torch.manual_seed(123)
    q0 = torch.nn.Linear(8, 8).weight.detach().clone()  # first Linear created after the seed
    assert torch.equal(a.layers[0].attention.q_proj.weight, q0)
    names = list(a.state_dict())
    assert names[:4] == ["layers.0.norm1.weight", "layers.0.norm1.bias",
                         "layers.0.attention.q_proj.weight", "layers.0.attention.q_proj.bias"]
    assert names[-2:] == ["final_norm.weight", "final_norm.bias"]


def test_key_mask_is_redundant_under_causal_right_padding():
    """Reference test_padding_mask_redundancy.py:59-82 -- dropping the key mask is bitwise exact."""
    cfg = TransformerConfig(4, 16, 16, 4, 16, 2, True)
    torch.manual_seed(19)
    model = DenseTransformer(cfg).eval()

    def no_key_mask(self, q, k, v, mask, causal):
        return type(self).attend(self, q, k, v, None, causal)

    variant = DenseTransformer(cfg).eval()
    copy_model_weights(model, variant)
    for layer in variant.layers:
        layer.attention.attend = no_key_mask.__get__(layer.attention)
    for ratio in (0.0, 0.3, 0.5, 0.9):
        for seed in (101, 202):
            x, mask = generate_random_case(cfg, torch.device("cpu"), torch.float32, seed, ratio, 1.0)
            with torch.inference_mode():
                assert float((model(x, mask) - variant(x, mask)).abs().max()) == 0.0


def test_linear_memory_oracle_matches_dense_model():
    """Reference test_fp32_reference.py:24-69: padded and unpadded, within 1e-4."""
    for s, lengths in ((32, None), (24, [17, 9])):
        cfg = TransformerConfig(2, s, 32, 4, 32, 2, True)
        torch.manual_seed(1234)
        dense = DenseTransformer(cfg).eval()
        oracle = LinearMemoryReference(cfg).eval()
        copy_model_weights(dense, oracle)
        x = torch.randn(2, s, 32)
        mask = torch.ones(2, s, dtype=torch.bool) if lengths is None else \
            torch.arange(s)[None, :] < torch.tensor(lengths)[:, None]
        x = x.masked_fill(~mask[..., None], 0)
        LinearMemoryReference.block = 5
        with torch.inference_mode():
            res = compare_outputs_streamed(dense(x, mask), oracle(x, mask), token_chunk=7)
        assert res.passed and res.max_abs_error < 1e-4


def test_linear_memory_oracle_validated_against_dense_at_4096():
    """The extreme-length oracle is validated against the dense model at S = 4096."""
    cfg = TransformerConfig(1, 4096, 64, 1, 64, 1, True)
    torch.manual_seed(5)
    dense = DenseTransformer(cfg).eval()
    oracle = LinearMemoryReference(cfg).eval()
    copy_model_weights(dense, oracle)
    LinearMemoryReference.block = 1024
    x = torch.randn(1, 4096, 64)
    mask = torch.ones(1, 4096, dtype=torch.bool)
    with torch.inference_mode():
        res = compare_outputs_streamed(dense(x, mask), oracle(x, mask))
    assert res.passed and res.max_abs_error < 1e-4


def test_linear_memory_oracle_rejects_non_prefix_masks_and_fp16():
    from oracle.attention import LinearMemorySelfAttention

    attn = LinearMemorySelfAttention(32, 4).eval()
    mask = torch.tensor([[True, True, False, True, False, False, False, False]])
    with pytest.raises(ValueError, match="right-padded"):
        attn(torch.randn(1, 8, 32), mask, causal=True)
    with pytest.raises(RuntimeError, match="float32"):
        attn.half()(torch.randn(1, 8, 32).half(), causal=True)


def test_flops_constant_for_the_attention_core_workload():
    assert math.isclose(exact_attention_flops([4096] * 64, 16, 64), 2.19956e12, rel_tol=1e-5)


def _torch_encoder_with_oracle_weights(model, cfg):
    """``torch.nn.TransformerEncoder`` with pre-norm layers, exact GELU and a
    final LayerNorm, carrying ``model``'s weights (q/k/v stacked into the
    packed in-projection)."""
    layer = torch.nn.TransformerEncoderLayer(cfg.d_model, cfg.num_heads, dim_feedforward=cfg.ffn_dim, dropout=0.0,
                                             activation="gelu", batch_first=True, norm_first=True)
    enc = torch.nn.TransformerEncoder(layer, cfg.num_layers, norm=torch.nn.LayerNorm(cfg.d_model),
                                      enable_nested_tensor=False).double().eval()
    with torch.no_grad():
        for mine, theirs in zip(model.layers, enc.layers):
            a = mine.attention
            theirs.self_attn.in_proj_weight.copy_(torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]))
            theirs.self_attn.in_proj_bias.copy_(torch.cat([a.q_proj.bias, a.k_proj.bias, a.v_proj.bias]))
            theirs.self_attn.out_proj.weight.copy_(a.out_proj.weight)
            theirs.self_attn.out_proj.bias.copy_(a.out_proj.bias)
            theirs.linear1.load_state_dict(mine.ffn_in.state_dict())
            theirs.linear2.load_state_dict(mine.ffn_out.state_dict())
            theirs.norm1.load_state_dict(mine.norm1.state_dict())
            theirs.norm2.load_state_dict(mine.norm2.state_dict())
        enc.norm.load_state_dict(model.final_norm.state_dict())
    return enc


@pytest.mark.parametrize("layers", [1, 3])
def test_dense_model_block_wiring_matches_torch_transformer_encoder(layers):
    """The oracle's block wiring against a library routine, not a second
    restatement: torch's pre-norm encoder (norm_first, exact GELU, no dropout,
    final LayerNorm) with the same weights, causal mask, fp64. A slip in norm
    placement, residual order, activation or the final norm moves outputs by
    O(0.1); what remains here (~5e-8) is the reference's fp32 softmax
    (``torch_transformer_benchmark.py:111``), kept in the oracle's fp64 mode."""
    cfg = TransformerConfig(batch_size=2, seq_len=48, d_model=64, num_heads=4, ffn_dim=96, num_layers=layers,
                            causal=True)
    torch.manual_seed(3)
    model = DenseTransformer(cfg).double().eval()
    enc = _torch_encoder_with_oracle_weights(model, cfg)
    x = torch.randn(2, 48, 64, dtype=torch.float64)
    causal = torch.nn.Transformer.generate_square_subsequent_mask(48, dtype=torch.float64)
    with torch.no_grad():
        ref = enc(x, mask=causal, is_causal=True)
        got = model(x)
    assert torch.allclose(got, ref, atol=1e-6, rtol=0), float((got - ref).abs().max())


def test_dense_model_padding_matches_torch_encoder_on_valid_rows():
    """With right padding the oracle zeroes padded rows after every block
    (reference ``torch_transformer_benchmark.py:120-121``, ``:145``, ``:170-171``);
    under a causal mask those rows never reach a valid one, so the valid rows
    equal torch's encoder with a key-padding mask, and the padded rows are 0."""
    cfg = TransformerConfig(batch_size=3, seq_len=40, d_model=64, num_heads=4, ffn_dim=96, num_layers=2, causal=True)
    torch.manual_seed(4)
    model = DenseTransformer(cfg).double().eval()
    enc = _torch_encoder_with_oracle_weights(model, cfg)
    lengths = torch.tensor([40, 17, 1])
    mask = torch.arange(40)[None, :] < lengths[:, None]
    x = torch.randn(3, 40, 64, dtype=torch.float64).masked_fill(~mask[..., None], 0)
    causal = torch.nn.Transformer.generate_square_subsequent_mask(40, dtype=torch.float64)
    with torch.no_grad():
        pad = torch.zeros(3, 40, dtype=torch.float64).masked_fill(~mask, float("-inf"))  # same type as `causal`
        ref = enc(x, mask=causal, src_key_padding_mask=pad, is_causal=True)
        got = model(x, mask)
    assert torch.allclose(got[mask], ref[mask], atol=1e-6, rtol=0), float((got[mask] - ref[mask]).abs().max())
    assert bool((got[~mask] == 0).all())
