"""Dispatcher policy, streaming helpers and candidate contract (CPU).

Mirrors the policy halves of the reference's ``test_dispatcher.py``,
``test_extreme.py``, ``test_attention_routing.py`` and
``test_candidate_contract.py``; GPU execution is covered by
``test_model_gpu.py``.
"""

from __future__ import annotations

from unittest import mock

import pytest
import torch

from oracle.model import DenseTransformer
from techjam_amd import dispatcher as D
from techjam_amd.errors import UnsupportedCaseError
from techjam_amd.implementations.attention_routing import MaskKind, Route, classify_mask, select_route
from techjam_amd.infra import BENCHMARK_CONFIGS, load_official_cases
from techjam_amd.model import TransformerConfig

GPU = dict(device_type="cuda", device_name="AMD Instinct MI355X", device_capability=(9, 5),
           torch_version=torch.__version__, matmul_precision="highest", allow_tf32=False,
           device_arch="gfx950")


def official(case_id):
    c = load_official_cases()[case_id]
    return TransformerConfig(c.batch_size, c.seq_len, c.qkv_dim, c.heads, c.ffn_dim, c.layers, c.causal)


def bench_cfg(name):
    c = BENCHMARK_CONFIGS[name]
    return TransformerConfig(c.batch_size, c.seq_len, c.d_model, c.num_heads, c.ffn_dim, c.num_layers, c.causal)


def test_routes_every_supported_official_case_to_the_hip_kernels():
    for cid in (1, 2, 3, 4, 5, 9, 10, 12, 13):
        r = D.select_route(official(cid), dtype=torch.float32, **GPU)
        assert (r.case_id, r.backend, r.compile_mode) == (cid, D.HIP_EXACT_BACKEND, None)


def test_routes_extreme_cases_to_the_memory_bounded_backend():
    assert D.select_route(official(6), dtype=torch.float32, **GPU).backend == D.EXTREME_MEMORY_BACKEND
    for dt in (torch.float16, torch.float32):
        assert D.select_route(official(14), dtype=dt, **GPU).backend == D.EXTREME_MEMORY_BACKEND


def test_routes_benchmark_model_configurations():
    for name in ("C1", "C2", "C4"):
        r = D.select_route(bench_cfg(name), dtype=torch.float32, **GPU)
        assert (r.case_id, r.backend) == (name, D.HIP_EXACT_BACKEND)


def test_refuses_what_the_kernels_do_not_implement():
    cases = [
        (official(1), dict(GPU, device_type="cpu")),
        (official(1), dict(GPU, device_arch="gfx942")),
        (official(1), dict(GPU)),          # bfloat16 below
        (official(6), dict(GPU)),          # case 6 in float16
        (TransformerConfig(2, 64, 1024, 2, 64, 1, True), dict(GPU)),   # head_dim 512
    ]
    dtypes = [torch.float32, torch.float32, torch.bfloat16, torch.float16, torch.float32]
    for (cfg, contract), dt in zip(cases, dtypes):
        assert D.select_route(cfg, dtype=dt, **contract).backend == D.UNSUPPORTED_BACKEND


def test_small_head_dims_take_the_exact_route_padded():
    from techjam_amd.kernels.attention import kernel_head_dim

    for case_id in (7, 8, 11):             # head_dim 8, 256, 8
        r = D.select_route(official(case_id), dtype=torch.float32, **GPU)
        assert r.backend == D.HIP_EXACT_BACKEND
    assert [kernel_head_dim(d) for d in (1, 8, 32, 33, 64, 65, 100, 128, 129, 256, 257)] == \
        [32, 32, 32, 64, 64, 128, 128, 128, 256, 256, None]


def test_generic_shapes_take_the_exact_route():
    cfg = TransformerConfig(3, 77, 192, 3, 64, 2, False)
    r = D.select_route(cfg, dtype=torch.float16, **GPU)
    assert r.backend == D.HIP_EXACT_BACKEND and r.case_id is None


def test_the_dense_fallback_name_is_never_selected():
    for cid in range(1, 15):
        for dt in (torch.float32, torch.float16, torch.bfloat16):
            for dev in ("cuda", "cpu"):
                r = D.select_route(official(cid), dtype=dt, **dict(GPU, device_type=dev))
                assert r.backend != D.REFERENCE_BACKEND


def _models(cfg):
    base = DenseTransformer(cfg).eval()
    cand = D.DispatchingTransformer(cfg).eval()
    cand.load_state_dict(base.state_dict())
    return base, cand


def test_state_dict_contract_matches_the_dense_model():
    base, cand = _models(TransformerConfig(2, 8, 16, 4, 16, 2, True))
    assert list(base.state_dict()) == list(cand.state_dict())


def test_attention_module_types_per_case():
    from techjam_amd.implementations.extreme import PolyOrExactSelfAttention
    from techjam_amd.implementations.sdpa import PackedQKVSDPASelfAttention, StridedSDPASelfAttention

    expect = {1: StridedSDPASelfAttention, 2: PackedQKVSDPASelfAttention, 3: PackedQKVSDPASelfAttention,
              14: PolyOrExactSelfAttention}
    for cid, typ in expect.items():
        m = D.DispatchingTransformer(official(cid))
        assert all(type(layer.attention) is typ for layer in m.layers)
    m = D.DispatchingTransformer(bench_cfg("C2"))
    assert all(type(layer.attention) is PackedQKVSDPASelfAttention for layer in m.layers)


def _gpu_key(shape, kind=MaskKind.PREFIX):
    return D.RuntimeKey(tuple(shape), "cuda", 0, torch.float32, "AMD Instinct MI355X", (9, 5), kind,
                        True, False, "highest", False, "gfx950")


def test_extreme_shape_mismatch_is_refused():
    cand = D.DispatchingTransformer(official(14))
    assert cand._resolve_route(_gpu_key((1, 1024, 1024))).backend == D.UNSUPPORTED_BACKEND


def test_general_masks_are_refused():
    cand = D.DispatchingTransformer(official(1))
    key = _gpu_key((64, 128, 128), MaskKind.GENERAL)
    assert cand._resolve_route(key).backend == D.UNSUPPORTED_BACKEND


def test_cpu_forward_raises_instead_of_computing():
    _, cand = _models(TransformerConfig(2, 8, 64, 1, 16, 1, True))
    with pytest.raises(UnsupportedCaseError):
        with torch.inference_mode():
            cand(torch.randn(2, 8, 64), torch.ones(2, 8, dtype=torch.bool))
    assert cand.last_route.backend == D.UNSUPPORTED_BACKEND


def test_routes_are_cached_per_runtime_key_and_failures_reraise():
    _, cand = _models(official(2))
    key = _gpu_key((1, 128, 128), MaskKind.ABSENT)
    calls = []

    def fake(x, mask=None):
        calls.append(1)
        if len(calls) == 2:
            raise RuntimeError("synthetic kernel failure")
        return x

    with mock.patch.object(cand, "_runtime_key", return_value=key), \
            mock.patch.object(cand, "_forward_hip", side_effect=fake):
        x = torch.randn(1, 128, 128)
        assert cand(x) is x
        with pytest.raises(RuntimeError, match="synthetic"):
            cand(x)
    assert len(cand._compiled_forwards) == 1
    assert "synthetic" in next(iter(cand.compile_failures.values()))
    assert cand.last_route.case_id == 2


def test_parameter_conversion_clears_runtime_cache():
    _, cand = _models(TransformerConfig(2, 8, 16, 4, 16, 2, True))
    key = _gpu_key((2, 8, 16))
    cand._compiled_forwards[key] = D.CachedForward(cand._forward_hip, compiled=False, case_id=None)
    cand._compile_failures[key] = "synthetic"
    cand.to(dtype=torch.float64)
    assert not cand._compiled_forwards and not cand.compile_failures


def test_case14_streamed_entrypoint_requires_the_official_model():
    _, cand = _models(TransformerConfig(2, 8, 16, 4, 16, 2, True))
    with torch.inference_mode(), pytest.raises(UnsupportedCaseError):
        cand.forward_case14_streamed_sample(torch.randn(1, 8, 16), torch.ones(1, 8, dtype=torch.bool))


def test_packed_weights_follow_loads_and_conversions():
    from techjam_amd.implementations.sdpa import PackedQKVSDPASelfAttention

    m = PackedQKVSDPASelfAttention(32, 4)
    other = PackedQKVSDPASelfAttention(32, 4)
    m.load_state_dict(other.state_dict())
    assert torch.equal(m._packed_qkv_weight[:32], other.q_proj.weight)
    assert torch.equal(m._packed_qkv_bias[64:], other.v_proj.bias)
    m.double()
    assert m._packed_qkv_weight.dtype == torch.float64
    assert "_packed_qkv_weight" not in m.state_dict()


# -- mask routing ----------------------------------------------------------------

def test_classify_mask_known_answers():
    assert classify_mask(None) is MaskKind.ABSENT
    assert classify_mask(torch.ones(3, 5, dtype=torch.bool)) is MaskKind.PREFIX
    assert classify_mask(torch.tensor([[True, True, False, False], [True, True, True, False]])) is MaskKind.PREFIX
    assert classify_mask(torch.tensor([[False, True, True, True]])) is MaskKind.GENERAL
    assert classify_mask(torch.tensor([[True, False, True, False]])) is MaskKind.GENERAL
    assert classify_mask(torch.zeros(2, 1, dtype=torch.bool)) is MaskKind.PREFIX


def test_kernel_routes():
    for causal in (True, False):
        assert select_route(True, causal, MaskKind.ABSENT) is Route.KERNEL
        assert select_route(True, causal, MaskKind.PREFIX) is Route.KERNEL_VALID_LENGTHS
        assert select_route(True, causal, MaskKind.GENERAL) is Route.REFUSE
        for kind in MaskKind:
            assert select_route(False, causal, kind) is Route.REFUSE


def test_prefix_lengths_rejects_general_masks():
    from techjam_amd.model import prefix_lengths

    assert prefix_lengths(torch.tensor([[True, True, False], [True, False, False]])).tolist() == [2, 1]
    with pytest.raises(UnsupportedCaseError):
        prefix_lengths(torch.tensor([[False, True, True]]))


# -- streaming helpers (reference test_extreme.py known answers) -------------------

def test_right_padded_lengths():
    from techjam_amd.implementations.extreme import right_padded_lengths

    mask = torch.tensor([[True] * 4, [True, True, False, False], [False] * 4])
    assert right_padded_lengths(mask) == [4, 2, 0]
    with pytest.raises(ValueError, match="right-padded"):
        right_padded_lengths(torch.tensor([[True, False, True]]))


def test_batch_chunks_preserve_order_and_masks():
    from techjam_amd.implementations.extreme import forward_batch_chunks

    x = torch.arange(30, dtype=torch.float32).view(5, 3, 2)
    mask = torch.tensor([[1, 1, 1], [1, 1, 0], [1, 0, 0], [1, 1, 1], [1, 1, 0]], dtype=torch.bool)
    got = forward_batch_chunks(lambda c, m: (c + 1).masked_fill(~m[..., None], 0), x, mask, 2)
    assert torch.equal(got, (x + 1).masked_fill(~mask[..., None], 0))


def test_batch_chunks_halve_after_oom():
    from techjam_amd.implementations.extreme import forward_batch_chunks

    x = torch.arange(24, dtype=torch.float32).view(4, 3, 2)
    tried = []

    def fwd(c, m):
        tried.append(c.shape[0])
        if c.shape[0] > 1:
            raise torch.OutOfMemoryError("synthetic")
        return c + 1

    with mock.patch("techjam_amd.implementations.extreme.torch.cuda.empty_cache"):
        got = forward_batch_chunks(fwd, x, None, 4)
    assert torch.equal(got, x + 1) and tried == [4, 2, 1, 1, 1, 1]


def test_prefix_chunks_trim_padding_and_restore_shape():
    from techjam_amd.implementations.extreme import forward_prefix_chunks

    x = torch.arange(32, dtype=torch.float32).view(4, 4, 2)
    mask = torch.tensor([[1, 1, 1, 1], [1, 1, 1, 1], [1, 1, 0, 0], [1, 0, 0, 0]], dtype=torch.bool)
    calls = []

    def fwd(c, m):
        calls.append((tuple(c.shape), m))
        return c + 1

    got = forward_prefix_chunks(fwd, x, mask, 2)
    assert torch.equal(got, (x + 1).masked_fill(~mask[..., None], 0))
    assert calls == [((2, 4, 2), None), ((1, 2, 2), None), ((1, 1, 2), None)]


def test_guarded_module_route_predicate():
    from techjam_amd.implementations import extreme

    m = extreme.PolyOrExactSelfAttention(1024, 16)
    assert m.poly_enabled == extreme.POLY_ATTENTION_ENABLED
    assert m.route_name(0.334) == "poly"
    assert m.route_name(0.5217) == "exact" and m.route_name(5.0) == "exact"
    m.poly_enabled = False
    assert m.route_name(0.334) == "exact"
    assert issubclass(extreme.PolyOrExactSelfAttention, extreme.ExactOnlySelfAttention)


# -- candidate contract ------------------------------------------------------------

def test_candidate_loads_and_validates():
    from techjam_amd.infra import load_candidate

    spec = load_candidate("techjam_amd.dispatcher")
    assert spec is D.CANDIDATE and spec.model_factory is D.DispatchingTransformer


def test_candidate_refuses_before_allocation():
    from techjam_amd.infra import CandidateSpec, validate_candidate_execution

    spec = D.CANDIDATE
    with pytest.raises(ValueError, match="compiles itself"):
        validate_candidate_execution(spec, 1, compile_user=True)
    refusing = CandidateSpec("r", D.DispatchingTransformer, "o", "d", self_compiling=True,
                             unsupported_official_cases=(8,))
    with pytest.raises(ValueError, match="does not support"):
        validate_candidate_execution(refusing, 8, compile_user=False, device_type="cuda")
    with pytest.raises(ValueError, match="only with"):
        validate_candidate_execution(spec, 6, compile_user=False, dtype_name="float16", device_type="cuda")
    with pytest.raises(ValueError, match="dense baseline"):
        validate_candidate_execution(spec, 14, compile_user=False, dtype_name="float32", device_type="cuda")
    with pytest.raises(ValueError, match="GPU"):
        validate_candidate_execution(spec, 1, compile_user=False, dtype_name="float32", device_type="cpu")
    validate_candidate_execution(spec, 1, compile_user=False, dtype_name="float32", device_type="cuda")
    for case_id in (7, 8, 11):
        validate_candidate_execution(spec, case_id, compile_user=False, dtype_name="float32", device_type="cuda")


def test_candidate_spec_validation_rules():
    from techjam_amd.infra import CandidateSpec

    with pytest.raises(ValueError):
        CandidateSpec("Bad Name", D.DispatchingTransformer, "o", "d").validate()
    with pytest.raises(ValueError):
        CandidateSpec("ok", D.DispatchingTransformer, "o", "d", unsupported_official_cases=(15,)).validate()
    with pytest.raises(ValueError):
        CandidateSpec("ok", D.DispatchingTransformer, "o", "d", official_case_dtypes=((1, ("int8",)),)).validate()


# The reference's CandidateSpec field list (src/infra/candidate.py:15-39), in
# declaration order, restated as the interface a harness binds to.
REFERENCE_CANDIDATE_FIELDS = (
    "name", "model_factory", "owner", "description", "weight_loader", "strict_weight_copy",
    "self_compiling", "unsupported_official_cases", "official_case_dtypes", "candidate_only_official_cases",
    "default_input_scale_only_cases", "cuda_only_official_cases", "official_case_min_cuda_capability",
    "official_case_torch_versions",
)


def test_candidate_fields_are_the_reference_contract():
    import dataclasses

    assert tuple(f.name for f in dataclasses.fields(D.CANDIDATE)) == REFERENCE_CANDIDATE_FIELDS


def test_candidate_converts_to_a_foreign_spec_class():
    """What the reference-side module does: build the reference's own class
    (here a stand-in with the same field list and defaults) from CANDIDATE,
    both through ``as_spec`` and through ``dataclasses.asdict``."""
    import dataclasses

    from techjam_amd.infra import as_spec

    defaults = {f.name: f for f in dataclasses.fields(D.CANDIDATE)}
    Foreign = dataclasses.make_dataclass(
        "CandidateSpec",
        [(n, object) if defaults[n].default is dataclasses.MISSING else (n, object, dataclasses.field(
            default=defaults[n].default)) for n in REFERENCE_CANDIDATE_FIELDS],
        frozen=True)
    for spec in (as_spec(Foreign, D.CANDIDATE), Foreign(**dataclasses.asdict(D.CANDIDATE))):
        assert type(spec) is Foreign
        for name in REFERENCE_CANDIDATE_FIELDS:
            assert getattr(spec, name) == getattr(D.CANDIDATE, name), name
        assert spec.model_factory is D.DispatchingTransformer
    Short = dataclasses.make_dataclass("Short", [("name", str)], frozen=True)
    with pytest.raises(TypeError, match="fields differ"):
        as_spec(Short, D.CANDIDATE)
