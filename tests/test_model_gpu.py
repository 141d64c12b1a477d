"""Whole-model parity: the dispatcher on the GPU against the dense FP32 oracle (GPU).

Weights: ``torch.manual_seed(seed)`` then the oracle's default initialisation,
copied into the dispatcher with a strict ``load_state_dict``. Inputs:
``generate_random_case`` on the CPU (seeds 1234+i), copied to the GPU. The
oracle runs on the CPU where a dense forward takes seconds, and as the
linear-memory oracle on the GPU (torch FP32 ops, TF32 off) for the 8192-token
configuration. Pass bar: the benchmark's OR rule (2e-3 abs or 2% rel) with
zero failing elements.
"""

from __future__ import annotations

import contextlib

import pytest
import torch

from oracle.attention import LinearMemoryReference
from oracle.model import DenseTransformer, compare_outputs, generate_random_case
from oracle.model import TransformerConfig as OracleConfig

pytestmark = pytest.mark.gpu


def _pair(cfg: OracleConfig, seed: int, device):
    from techjam_amd.dispatcher import DispatchingTransformer

    torch.manual_seed(seed)
    base = DenseTransformer(cfg).eval()
    cand = DispatchingTransformer(cfg).eval()
    cand.load_state_dict(base.state_dict())
    return base, cand.to(device)


@contextlib.contextmanager
def _matmul_flags(precision: str, allow_tf32: bool):
    """Scoped float32-matmul flags (they are process-global in torch)."""
    old = (torch.get_float32_matmul_precision(), torch.backends.cuda.matmul.allow_tf32)
    torch.set_float32_matmul_precision(precision)
    torch.backends.cuda.matmul.allow_tf32 = allow_tf32
    try:
        yield
    finally:
        torch.set_float32_matmul_precision(old[0])
        torch.backends.cuda.matmul.allow_tf32 = old[1]


def _check(cfg, seeds, padding, cuda, oracle_on_gpu=False, oracle_cls=DenseTransformer, harness_flags=False,
           gemm_operands="fp32"):
    """``harness_flags``: run the candidate under the reference harness's
    validated numerics flags (matmul precision "high", TF32 allowed;
    src/benchmark.py:133-141, src/dispatcher.py:69-70) while the oracle keeps
    full fp32 GEMMs. ``gemm_operands="fp16"``: the candidate's GEMMs take
    fp16-rounded operands (TF32's mantissa) with fp32 accumulation."""
    from techjam_amd import dispatcher as D

    torch.backends.cuda.matmul.allow_tf32 = False
    cand_flags = ("high", True) if harness_flags else ("highest", False)
    base, cand = _pair(cfg, 4321, cuda)
    cand.gemm_operands = gemm_operands
    if oracle_cls is not DenseTransformer:
        lm = oracle_cls(cfg).eval()
        lm.load_state_dict(base.state_dict())
        base = lm
    if oracle_on_gpu:
        base = base.to(cuda)
    for seed in seeds:
        x, mask = generate_random_case(cfg, torch.device("cpu"), torch.float32, seed, padding, 1.0)
        with torch.inference_mode():
            with _matmul_flags("highest", False):
                ref = base(x.to(cuda), mask.to(cuda)).cpu() if oracle_on_gpu else base(x, mask)
            with _matmul_flags(*cand_flags):
                got = cand(x.to(cuda), mask.to(cuda))
                torch.cuda.synchronize()
        res = compare_outputs(ref, got.cpu(), rtol=0.02, atol=0.002)
        print(f"seed {seed}: max_abs={res.max_abs_error:.3e} failed={res.failed_elements}/{res.total_elements}")
        assert res.passed, f"seed {seed}: {res.failed_elements} failed, max_abs {res.max_abs_error:.3e}"
        assert cand.last_route.backend in (D.HIP_EXACT_BACKEND, D.EXTREME_MEMORY_BACKEND)


def test_config_1_one_layer_encoder(cuda):
    cfg = OracleConfig(2, 128, 256, 4, 1024, 1, True)
    _check(cfg, range(1234, 1239), 0.5, cuda)


def test_config_2_packed_qkv_four_layers(cuda):
    """The harness's five accuracy trials (seeds 1234+i, src/benchmark.py:80, :185-192)."""
    cfg = OracleConfig(8, 1024, 512, 8, 2048, 4, True)
    _check(cfg, range(1234, 1239), 0.5, cuda)


@pytest.mark.parametrize("case_id", list(range(1, 14)))
def test_official_cases(cuda, case_id):
    """Official cases 1-13 at their own sizes (case 6: 10000 samples through
    the batch-streamed route, oracle on the GPU)."""
    from techjam_amd.infra import load_official_cases

    c = load_official_cases()[case_id]
    cfg = OracleConfig(c.batch_size, c.seq_len, c.qkv_dim, c.heads, c.ffn_dim, c.layers, c.causal)
    _check(cfg, (1234,), 0.3, cuda, oracle_on_gpu=case_id == 6)


def test_config_2_under_the_reference_harness_matmul_flags(cuda):
    cfg = OracleConfig(8, 1024, 512, 8, 2048, 4, True)
    _check(cfg, (1234,), 0.5, cuda, harness_flags=True)


def test_config_4_under_the_reference_harness_matmul_flags(cuda):
    cfg = OracleConfig(2, 8192, 1024, 16, 4096, 4, True)
    _check(cfg, (1234,), 0.5, cuda, oracle_on_gpu=True, oracle_cls=LinearMemoryReference, harness_flags=True)


def test_config_1_with_fp16_gemm_operands(cuda):
    cfg = OracleConfig(2, 128, 256, 4, 1024, 1, True)
    _check(cfg, range(1234, 1239), 0.5, cuda, gemm_operands="fp16")


def test_config_2_with_fp16_gemm_operands(cuda):
    cfg = OracleConfig(8, 1024, 512, 8, 2048, 4, True)
    _check(cfg, range(1234, 1239), 0.5, cuda, gemm_operands="fp16")


def test_config_4_with_fp16_gemm_operands(cuda):
    cfg = OracleConfig(2, 8192, 1024, 16, 4096, 4, True)
    _check(cfg, range(1234, 1239), 0.5, cuda, oracle_on_gpu=True, oracle_cls=LinearMemoryReference,
           gemm_operands="fp16")


def test_fp16_gemm_operands_refuse_the_unfused_path(cuda):
    from techjam_amd.errors import UnsupportedCaseError

    cfg = OracleConfig(2, 64, 384, 6, 256, 1, True)   # d_model 384: no fused LayerNorm width
    _, cand = _pair(cfg, 3, cuda)
    x = torch.randn(2, 64, 384, device=cuda)
    with torch.inference_mode():
        cand(x, None)
        cand.gemm_operands = "fp16"
        with pytest.raises(UnsupportedCaseError):
            cand(x, None)
        cand.gemm_operands = "bf16"
        with pytest.raises(ValueError):
            cand(x, None)


def test_non_causal_right_padded_model(cuda):
    cfg = OracleConfig(3, 200, 256, 4, 256, 2, False)
    _check(cfg, (1234, 1235), 0.5, cuda)


def test_config_4_long_sequence_on_the_linear_memory_oracle(cuda):
    """The harness's five accuracy trials (seeds 1234+i)."""
    cfg = OracleConfig(2, 8192, 1024, 16, 4096, 4, True)
    _check(cfg, range(1234, 1239), 0.5, cuda, oracle_on_gpu=True, oracle_cls=LinearMemoryReference)


@pytest.mark.parametrize("causal", [True, False])
def test_unmasked_encoder_forward(cuda, causal):
    """No mask at all: the fused tails and norms run with every row valid."""
    cfg = OracleConfig(2, 300, 512, 8, 1024, 2, causal)
    base, cand = _pair(cfg, 77, cuda)
    x = torch.randn(2, 300, 512, generator=torch.Generator().manual_seed(5))
    with torch.inference_mode():
        with _matmul_flags("highest", False):
            ref = base(x, None)
            got = cand(x.to(cuda), None)
            torch.cuda.synchronize()
    res = compare_outputs(ref, got.cpu(), rtol=0.02, atol=0.002)
    assert res.passed, f"{res.failed_elements} failed, max_abs {res.max_abs_error:.3e}"


def test_padded_rows_are_zero_and_route_is_cached(cuda):
    cfg = OracleConfig(2, 128, 256, 4, 1024, 1, True)
    _, cand = _pair(cfg, 1, cuda)
    x, mask = generate_random_case(cfg, torch.device("cpu"), torch.float32, 1234, 0.5, 1.0)
    x, mask = x.to(cuda), mask.to(cuda)
    with torch.inference_mode():
        a = cand(x, mask)
        b = cand(x, mask)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert float(a[~mask].abs().max()) == 0.0
    assert len(cand._compiled_forwards) == 1


def test_hip_library_is_the_one_loaded(cuda):
    from techjam_amd.kernels import _lib

    handle = _lib.lib()
    assert str(_lib.LIB_PATH).endswith("techjam_amd/lib/libtechjam_attn.so")
    with open("/proc/self/maps") as f:
        assert any("libtechjam_attn.so" in line for line in f)
    assert handle.tj_abi_version() == _lib.ABI_VERSION
