"""The official case-14 route end to end on the GPU (GPU).

Case 14 is the 2-layer, d_model 1024, 16-head encoder at 100 000 tokens whose
attention runs the guarded polynomial module (``src/dispatcher.py:488-563``,
``src/implementations/extreme.py:249-319``). Here the dispatcher's own case-14
entry points run at 8192 tokens -- past the 4096-token exact prefix, so every
head's rows 4096.. come from the polynomial kernel -- and their output is
compared with the linear-memory FP32 oracle (``oracle.attention.
LinearMemoryReference``, the reference's ``fp32_reference.py:130-142``) on
the GPU, through the streamed OR-rule checker (``fp32_reference.py:157-204``),
with zero failing elements required. This is how the reference validates
case 14 (``src/case14_fp32_reference.py:168-245``).

Weights: ``torch.manual_seed(1234)`` and the oracle's default initialisation,
copied strictly into the dispatcher. Inputs: N(0, 1) (case 14's default input
scale), drawn on the CPU and copied to the GPU.
"""

from __future__ import annotations

import contextlib

import pytest
import torch

from oracle.attention import LinearMemoryReference, compare_outputs_streamed
from oracle.model import TransformerConfig as OracleConfig

pytestmark = pytest.mark.gpu

CASE_14 = OracleConfig(batch_size=32, seq_len=100000, d_model=1024, num_heads=16, ffn_dim=1024, num_layers=2,
                       causal=True)


@contextlib.contextmanager
def _fp32_matmuls():
    old = (torch.get_float32_matmul_precision(), torch.backends.cuda.matmul.allow_tf32)
    torch.set_float32_matmul_precision("highest")
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        yield
    finally:
        torch.set_float32_matmul_precision(old[0])
        torch.backends.cuda.matmul.allow_tf32 = old[1]


@pytest.fixture(scope="module")
def case14_models(cuda):
    from techjam_amd.dispatcher import DispatchingTransformer

    torch.manual_seed(1234)
    oracle = LinearMemoryReference(CASE_14).eval()
    cand = DispatchingTransformer(CASE_14).eval()
    cand.load_state_dict(oracle.state_dict())
    return oracle.to(cuda), cand.to(cuda)


def _input(b, n, lengths, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(b, n, CASE_14.d_model, generator=g)
    mask = torch.arange(n)[None, :] < torch.tensor(lengths)[:, None]
    return x.masked_fill(~mask[..., None], 0), mask


def _poly_heads(cand) -> int:
    """Heads the last forward sent to the polynomial kernel, summed over layers."""
    return sum(int(layer.attention.last_guard.flags.sum()) for layer in cand.layers)


@pytest.mark.parametrize("operands", ["fp16", "fp32"])
def test_streamed_sample_route_matches_linear_memory_oracle(cuda, case14_models, operands, monkeypatch):
    """Both GEMM-operand contracts of the route: fp16 operands (the default,
    the reference's fp16 case-14 compute) and fp32."""
    from techjam_amd.implementations.extreme import PolyOrExactSelfAttention

    oracle, cand = case14_models
    monkeypatch.setattr(cand, "case14_gemm_operands", operands)
    assert all(type(layer.attention) is PolyOrExactSelfAttention for layer in cand.layers)
    x, mask = _input(1, 8192, [8192], 1234)
    x, mask = x.to(cuda), mask.to(cuda)
    with torch.inference_mode(), _fp32_matmuls():
        got = cand.forward_case14_streamed_sample(x, mask)
        ref = oracle(x, mask)
        torch.cuda.synchronize()
    n_poly = _poly_heads(cand)
    res = compare_outputs_streamed(ref, got)
    print(f"case 14 streamed sample ({operands} GEMM operands), 8192 tokens: {n_poly}/32 heads polynomial, "
          f"max_abs={res.max_abs_error:.3e} "
          f"failed={res.failed_elements}/{res.total_elements}")
    assert n_poly > 0, "no head took the polynomial route"
    assert res.passed, f"{res.failed_elements} failing elements, max_abs {res.max_abs_error:.3e}"


def test_prefix_chunked_batch_with_padding_matches_linear_memory_oracle(cuda, case14_models):
    """Three samples of valid lengths 8192, 5000 and 0: equal-length prefix
    groups, padding trimmed, a ragged last chunk (5000 = 9 chunks + 392) and
    an empty sample whose rows must stay zero."""
    oracle, cand = case14_models
    x, mask = _input(3, 8192, [8192, 5000, 0], 1235)
    x, mask = x.to(cuda), mask.to(cuda)
    with torch.inference_mode(), _fp32_matmuls():
        got = cand._forward_case_14(x, mask)
        ref = oracle(x, mask)
        torch.cuda.synchronize()
    assert cand.last_extreme_chunk_size is not None and cand.last_extreme_chunk_size >= 1
    assert bool((got[1, 5000:] == 0).all()) and bool((got[2] == 0).all())
    res = compare_outputs_streamed(ref, got)
    print(f"case 14 prefix chunks (8192, 5000, 0): max_abs={res.max_abs_error:.3e} "
          f"failed={res.failed_elements}/{res.total_elements}")
    assert res.passed, f"{res.failed_elements} failing elements, max_abs {res.max_abs_error:.3e}"


def test_prefix_group_of_equal_lengths_is_served(cuda, case14_models):
    """Two padded samples of the same valid length form one prefix group,
    whose trimmed slice x[0:2, :5000] is a strided view: the route copies it
    to contiguous rows for the fused layer stack instead of refusing it."""
    oracle, cand = case14_models
    x, mask = _input(3, 8192, [5000, 5000, 8192], 1236)
    x, mask = x.to(cuda), mask.to(cuda)
    with torch.inference_mode(), _fp32_matmuls():
        got = cand._forward_case_14(x, mask)
        ref = oracle(x, mask)
        torch.cuda.synchronize()
    assert bool((got[:2, 5000:] == 0).all())
    res = compare_outputs_streamed(ref, got)
    print(f"case 14 prefix chunks (5000, 5000, 8192): max_abs={res.max_abs_error:.3e} "
          f"failed={res.failed_elements}/{res.total_elements}")
    assert res.passed, f"{res.failed_elements} failing elements, max_abs {res.max_abs_error:.3e}"


def test_fp16_input_runs_the_fp16_model(cuda, case14_models):
    """Case 14 also declares float16 input (an fp16 model, as the harness
    builds it for that dtype; the reference routes it through its SDPA
    module in fp16). The route serves it on the layer loop in fp16 -- fp16
    operands, fp32 accumulation inside the GEMMs and the attention kernels --
    and the result stays within the OR rule of the FP32 oracle."""
    import copy

    oracle, cand = case14_models
    half = copy.deepcopy(cand).half()
    x, mask = _input(2, 8192, [8192, 6000], 1237)
    x, mask = x.to(cuda), mask.to(cuda)
    with torch.inference_mode(), _fp32_matmuls():
        got = half._forward_case_14(x.half(), mask)
        ref = oracle(x.half().float(), mask)
        torch.cuda.synchronize()
    assert got.dtype == torch.float16
    assert bool((got[1, 6000:] == 0).all())
    res = compare_outputs_streamed(ref, got.float())
    print(f"case 14 fp16 model, (8192, 6000): max_abs={res.max_abs_error:.3e} "
          f"failed={res.failed_elements}/{res.total_elements}")
    assert res.passed, f"{res.failed_elements} failing elements, max_abs {res.max_abs_error:.3e}"
