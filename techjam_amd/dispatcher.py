"""Shape-aware dispatcher: the drop-in model of the attention hot path.

Keeps the public interface of the reference's ``src/dispatcher.py:39-818`` --
``DispatchingTransformer``, ``select_route``, ``RouteDecision``, ``RuntimeKey``,
``CachedForward``, ``UnsupportedCaseError``, the backend constants,
``last_route``, ``compile_failures``, ``last_extreme_chunk_size``,
``clear_runtime_cache``, ``forward_case14_streamed_sample`` and ``CANDIDATE``
-- with a different engine underneath:

* every attention call runs the gfx950 HIP kernels through the C ABI; there is
  no ``torch.compile`` route and no dense fallback. Requests the kernels do not
  implement (CPU tensors, other GPUs, head sizes above 256,
  bfloat16, non-prefix masks) raise ``UnsupportedCaseError`` before any
  allocation, and a failing kernel call is recorded in ``compile_failures``
  and re-raised;
* routes are keyed by the reference's 7-tuple ``(B, S, d_model, H, ffn, causal,
  layers)``: the fourteen disclosed cases plus the five benchmark model
  configurations (C1-C5); shapes outside the table take the generic exact route
  (the kernels are shape-generic);
* a right-padded mask is classified once per tensor and version (one host
  synchronisation, ``src/dispatcher.py:393-423``) and turned into device-side
  per-sample lengths that the kernel uses to skip padded rows;
* official case 6 streams batch slices (``:452-465``); official case 14 streams
  trimmed prefixes through the guarded polynomial module (``:488-538``), with
  its FP32 interface computed in FP32 around fp16-MFMA attention instead of
  casting the model to FP16. Their chunk sizes come from the streaming
  planner (``implementations.planner``), which budgets the HIP path's real
  working set instead of the reference's SDPA score-copy estimate.
"""

from __future__ import annotations

import os
import weakref
from dataclasses import dataclass
from typing import Callable, Dict, Optional, Tuple, Union

import torch

from .errors import UnsupportedCaseError
from .implementations.attention_routing import MaskKind, classify_mask
from .implementations.extreme import (
    CASE_14_CONFIG,
    PolyOrExactSelfAttention,
    forward_batch_chunks,
    forward_prefix_chunks,
)
from .implementations.planner import ChunkPlan, plan_for_input
from .implementations.sdpa import PackedQKVSDPASelfAttention, StridedSDPASelfAttention
from .infra import BENCHMARK_CONFIGS, CandidateSpec, OfficialCase, load_official_cases
from .kernels.attention import SUPPORTED_HEAD_DIMS, kernel_head_dim
from .graphs import GraphedForward, graph_key, weights_signature
from .model import TransformerConfig, TransformerEncoder, config_key

ConfigKey = Tuple[int, int, int, int, int, bool, int]
CaseId = Union[int, str]
ForwardCallable = Callable[[torch.Tensor, Optional[torch.Tensor]], torch.Tensor]

HIP_EXACT_BACKEND = "hip-exact"
EXTREME_MEMORY_BACKEND = "extreme-memory"
UNSUPPORTED_BACKEND = "unsupported"
# The reference's names for its compiled-SDPA and dense-eager routes. The
# compiled route's role is played by the HIP exact route; the dense route has
# no counterpart and is never selected.
COMPILED_SDPA_BACKEND = HIP_EXACT_BACKEND
REFERENCE_BACKEND = "reference"

REQUIRED_GPU_ARCH = "gfx950"
SUPPORTED_DTYPES = (torch.float32, torch.float16)


def _official_key(case: OfficialCase) -> ConfigKey:
    return (case.batch_size, case.seq_len, case.qkv_dim, case.heads, case.ffn_dim, case.causal, case.layers)


OFFICIAL_CASE_BY_CONFIG: Dict[ConfigKey, int] = {
    _official_key(c): cid for cid, c in load_official_cases().items()
}
BENCHMARK_CASE_BY_CONFIG: Dict[ConfigKey, str] = {
    cfg.model_key(): name for name, cfg in BENCHMARK_CONFIGS.items() if cfg.model_key() is not None
}
PACKED_QKV_CASES = frozenset((2, 3, "C2", "C4"))
EXTREME_CASES = (6, 14)
# Launch-bound sizes replayed as HIP graphs, by input elements (tokens x
# d_model): C1 (256 x 256) and the official cases of 128-token sequences up to
# 128 x 128 x 128 are launch-bound; C2 (8192 x 512), C4 and cases 8 and 13
# (8192 x 1024, 65536 x 128) are kernel-bound and gain nothing. Captures are
# kept per model.
GRAPH_MAX_ELEMENTS = 1 << 21
GRAPH_CACHE_SIZE = 8


def case_for(config) -> Optional[CaseId]:
    key = config_key(config)
    return OFFICIAL_CASE_BY_CONFIG.get(key, BENCHMARK_CASE_BY_CONFIG.get(key))


@dataclass(frozen=True)
class RouteDecision:
    """Resolved backend for one static model and runtime contract."""

    case_id: Optional[CaseId]
    backend: str
    compile_mode: Optional[str]
    reason: str


@dataclass(frozen=True)
class RuntimeKey:
    """Inputs that can change the selected route or its numerics."""

    input_shape: Tuple[int, ...]
    device_type: str
    device_index: Optional[int]
    dtype: torch.dtype
    device_name: Optional[str]
    device_capability: Optional[Tuple[int, int]]
    mask_kind: MaskKind
    inference_mode: bool
    grad_enabled: bool
    matmul_precision: str
    allow_tf32: bool
    device_arch: Optional[str] = None


@dataclass(frozen=True)
class CachedForward:
    """One runtime-key callable. ``compiled`` is always False: nothing is traced."""

    function: ForwardCallable
    compiled: bool
    case_id: Optional[CaseId]
    drop_key_mask: bool = False


def select_route(
    config,
    *,
    device_type: str,
    dtype: torch.dtype,
    device_name: Optional[str],
    device_capability: Optional[Tuple[int, int]],
    torch_version: str,
    matmul_precision: str,
    allow_tf32: bool,
    device_arch: Optional[str] = None,
) -> RouteDecision:
    """Route one static configuration under one runtime contract (pure; no GPU needed)."""
    del device_name, device_capability, torch_version, matmul_precision, allow_tf32
    case_id = case_for(config)
    if device_type != "cuda":
        return RouteDecision(case_id, UNSUPPORTED_BACKEND, None,
                             "the attention kernels need a ROCm GPU; there is no CPU implementation")
    if device_arch is not None and not device_arch.startswith(REQUIRED_GPU_ARCH):
        return RouteDecision(case_id, UNSUPPORTED_BACKEND, None,
                             f"the HIP library is built for {REQUIRED_GPU_ARCH} only, not {device_arch}")
    if dtype not in SUPPORTED_DTYPES:
        return RouteDecision(case_id, UNSUPPORTED_BACKEND, None, f"dtype {dtype} is not supported")
    head_dim = config.d_model // config.num_heads
    if kernel_head_dim(head_dim) is None:
        return RouteDecision(case_id, UNSUPPORTED_BACKEND, None,
                             f"head_dim {head_dim} is not implemented (at most {SUPPORTED_HEAD_DIMS[-1]})")
    if case_id in EXTREME_CASES:
        if case_id == 6 and dtype != torch.float32:
            return RouteDecision(case_id, UNSUPPORTED_BACKEND, None, "case 6 is validated in float32")
        return RouteDecision(case_id, EXTREME_MEMORY_BACKEND, None, "memory-bounded extreme route")
    return RouteDecision(case_id, HIP_EXACT_BACKEND, None,
                         "HIP exact attention" + ("" if case_id is not None else " (generic shape)"))


def _device_arch(device: torch.device) -> Optional[str]:
    if device.type != "cuda" or not torch.cuda.is_available():
        return None
    name = getattr(torch.cuda.get_device_properties(device), "gcnArchName", None)
    return None if name is None else name.split(":")[0]


class DispatchingTransformer(TransformerEncoder):
    """Lazy per-instance dispatcher whose attention always runs the HIP kernels."""

    #: Replay the exact-attention forward as a HIP graph for inputs of at most
    #: ``GRAPH_MAX_ELEMENTS`` input elements (inference only); ``TECHJAM_AMD_GRAPHS=0``
    #: in the environment turns it off.
    use_graphs = True
    #: Device bytes the streamed routes (cases 6 and 14) may plan for; None
    #: takes 85 % of the device less what is already allocated.
    memory_budget_bytes: Optional[int] = None
    #: GEMM operands of the case-14 route. The reference computes that case in
    #: fp16 behind its fp32 interface (src/dispatcher.py:488-518: fp16
    #: residual stream, autocast fp16 GEMMs); "fp16" here rounds the GEMM
    #: operands only, with fp32 accumulation, residual stream and norms.
    case14_gemm_operands = "fp16"

    def __init__(self, config: TransformerConfig) -> None:
        super().__init__(config)
        if not self.norm_first or self.activation != "gelu":
            raise UnsupportedCaseError(
                "the dispatcher serves the reference model (pre-norm, exact GELU); run other block "
                "variants on TransformerEncoder directly")
        case_id = case_for(config)
        if config_key(config) == CASE_14_CONFIG:
            attention_type = PolyOrExactSelfAttention
        elif case_id in PACKED_QKV_CASES:
            attention_type = PackedQKVSDPASelfAttention
        else:
            attention_type = StridedSDPASelfAttention
        for layer in self.layers:
            layer.attention = attention_type(config.d_model, config.num_heads)
        self._compiled_forwards: Dict[RuntimeKey, CachedForward] = {}
        self._compile_failures: Dict[RuntimeKey, str] = {}
        self._device_contracts: Dict[tuple, tuple] = {}
        self._last_route: Optional[RouteDecision] = None
        self._last_extreme_chunk_size: Optional[int] = None
        self._last_chunk_plan: Optional[ChunkPlan] = None
        self._mask_ref = None
        self._mask_version = None
        self._mask_kind: Optional[MaskKind] = None
        self._graphs: Dict[tuple, GraphedForward] = {}
        self._graph_failures: Dict[tuple, str] = {}

    # -- diagnostics -------------------------------------------------------
    @property
    def last_route(self) -> Optional[RouteDecision]:
        return self._last_route

    @property
    def compile_failures(self) -> Dict[RuntimeKey, str]:
        """Kernel-call failures seen per runtime key (each was re-raised)."""
        return dict(self._compile_failures)

    @property
    def last_extreme_chunk_size(self) -> Optional[int]:
        return self._last_extreme_chunk_size

    @property
    def last_chunk_plan(self) -> Optional[ChunkPlan]:
        """The streaming planner's decision for the last streamed forward."""
        return self._last_chunk_plan

    def clear_runtime_cache(self) -> None:
        self._graphs.clear()
        self._graph_failures.clear()
        self._compiled_forwards.clear()
        self._compile_failures.clear()
        self._device_contracts.clear()
        self._last_route = None
        self._last_extreme_chunk_size = None
        self._last_chunk_plan = None
        self._mask_ref = None
        self._mask_version = None
        self._mask_kind = None

    def _apply(self, fn, recurse: bool = True):
        result = super()._apply(fn, recurse=recurse)
        if hasattr(self, "_compiled_forwards"):
            self.clear_runtime_cache()
        return result

    def load_state_dict(self, state_dict, strict: bool = True, assign: bool = False):
        result = super().load_state_dict(state_dict, strict=strict, assign=assign)
        self.clear_runtime_cache()
        return result

    def _set_drop_key_mask(self, enabled: bool) -> None:
        for layer in self.layers:
            layer.attention.drop_key_mask = enabled

    # -- mask handling -----------------------------------------------------
    @staticmethod
    def _version(mask: torch.Tensor) -> Optional[int]:
        try:
            return mask._version
        except RuntimeError:  # inference tensors do not track versions
            return None

    def _mask_kind_cached(self, mask: torch.Tensor) -> MaskKind:
        """Kind of a mask, classified once per tensor identity and version
        (``src/dispatcher.py:393-423``): the classification synchronises the
        host, so a timed loop over one mask pays it once. Inference tensors
        carry no version counter and are treated as immutable, as there."""
        version = self._version(mask)
        cached = None if self._mask_ref is None else self._mask_ref()
        if cached is mask and version == self._mask_version and self._mask_kind is not None:
            return self._mask_kind
        kind = classify_mask(mask)
        self._mask_ref = weakref.ref(mask)
        self._mask_version = version
        self._mask_kind = kind
        return kind

    def _mask_info(self, mask: Optional[torch.Tensor]) -> Tuple[MaskKind, Optional[torch.Tensor]]:
        """Kind (cached) and device int32 valid lengths of a mask.

        The lengths are recomputed from the live mask on every call -- one
        asynchronous device reduction, no host synchronisation -- so a mask
        buffer refilled in place (which an inference tensor's missing version
        counter cannot reveal) never feeds stale lengths to the kernels."""
        if mask is None:
            return MaskKind.ABSENT, None
        kind = self._mask_kind_cached(mask)
        lengths = mask.sum(dim=1, dtype=torch.int32) if kind is MaskKind.PREFIX else None
        return kind, lengths

    # -- routes ------------------------------------------------------------
    def _forward_hip(self, x, valid_token_mask=None):
        _, lengths = self._mask_info(valid_token_mask)
        if self._graphable(x):
            return self._forward_graphed(x, valid_token_mask, lengths)
        return self.forward_layers(x, valid_token_mask, lengths)

    # -- graph replay (the counterpart of the reference's "reduce-overhead" routes)
    def _graphable(self, x) -> bool:
        return (self.use_graphs and os.environ.get("TECHJAM_AMD_GRAPHS", "1") != "0"
                and x.is_cuda and x.device.index == torch.cuda.current_device()
                and x.ndim == 3 and x.is_contiguous() and not torch.is_grad_enabled()
                and x.numel() <= GRAPH_MAX_ELEMENTS
                and not torch.cuda.is_current_stream_capturing())

    def _forward_graphed(self, x, mask, lengths):
        key = graph_key(x, mask, lengths, (self.gemm_operands, torch.get_float32_matmul_precision(),
                                           bool(torch.backends.cuda.matmul.allow_tf32),
                                           str(torch.backends.cuda.preferred_blas_library())))
        if key in self._graph_failures:
            return self.forward_layers(x, mask, lengths)
        signature = weights_signature(self)
        graphed = self._graphs.get(key)
        if graphed is None or graphed.signature != signature or not graphed.matches(x, mask, lengths):
            self._graphs.pop(key, None)
            if len(self._graphs) >= GRAPH_CACHE_SIZE:
                self._graphs.pop(next(iter(self._graphs)))
            try:
                graphed = GraphedForward(self.forward_layers, x, mask, lengths, signature)
            except UnsupportedCaseError:
                raise
            except Exception as err:  # capture refused: this signature runs eagerly from now on
                self._graph_failures[key] = f"{type(err).__name__}: {err}"
                return self.forward_layers(x, mask, lengths)
            self._graphs[key] = graphed
        return graphed(x, mask, lengths)

    def _plan_chunk(self, x, poly: bool) -> int:
        plan = plan_for_input(x, self.config.num_heads, self.config.ffn_dim, poly=poly,
                              budget_bytes=self.memory_budget_bytes)
        self._last_chunk_plan = plan
        self._last_extreme_chunk_size = plan.chunk
        return plan.chunk

    def _forward_case_6(self, x, valid_token_mask=None):
        chunk = self._plan_chunk(x, poly=False)
        return forward_batch_chunks(self._forward_hip_chunk, x, valid_token_mask, chunk)

    def _forward_hip_chunk(self, x, valid_token_mask=None):
        lengths = None
        if valid_token_mask is not None:
            lengths = valid_token_mask.sum(dim=1, dtype=torch.int32)
        return self.forward_layers(x, valid_token_mask, lengths)

    def _forward_case_14_chunk(self, x, valid_token_mask=None):
        if x.device.type != "cuda" or x.dtype not in SUPPORTED_DTYPES:
            raise UnsupportedCaseError("case 14 chunks require float16 or float32 GPU input")
        if valid_token_mask is not None:
            raise ValueError("trim padding before the case 14 chunk")
        # A trimmed group of two or more samples (x[start:end, :n]) is a
        # strided view; the fused layer stack reads contiguous rows.
        x = x.contiguous()
        # fp16 GEMM operands are the fused fp32-interface path; fp16 input
        # (an fp16 model, the reference's _forward_sdpa branch for case 14)
        # runs the layer loop in its own dtype.
        operands = self.case14_gemm_operands if x.dtype == torch.float32 else "fp32"
        return self.forward_layers(x, None, None, gemm_operands=operands)

    def _forward_case_14(self, x, valid_token_mask=None):
        chunk = self._plan_chunk(x, poly=True)
        return forward_prefix_chunks(self._forward_case_14_chunk, x, valid_token_mask, chunk)

    def forward_case14_streamed_sample(self, x, valid_token_mask=None):
        """One sample of the official case-14 model, for oracle harnesses that stream samples."""
        if config_key(self.config) != CASE_14_CONFIG:
            raise UnsupportedCaseError("streamed sample entrypoint is only valid for case 14")
        if x.ndim != 3 or x.shape[0] != 1 or x.shape[2] != self.config.d_model:
            raise ValueError("case 14 streamed input must be [1, N, 1024]")
        if x.shape[1] > self.config.seq_len:
            raise ValueError("streamed sequence exceeds case 14's sequence length")
        if not torch.is_inference_mode_enabled() or torch.is_grad_enabled():
            raise UnsupportedCaseError("case 14 streamed route is inference-only")
        return self._forward_case_14(x, valid_token_mask)

    def _extreme_entrypoint(self, case_id: int) -> ForwardCallable:
        return {6: self._forward_case_6, 14: self._forward_case_14}[case_id]

    def _device_contract(self, device: torch.device):
        key = (device.type, device.index)
        hit = self._device_contracts.get(key)
        if hit is not None:
            return hit
        if device.type != "cuda" or not torch.cuda.is_available():
            contract = (None, None, None)
        else:
            contract = (torch.cuda.get_device_name(device), torch.cuda.get_device_capability(device),
                        _device_arch(device))
        self._device_contracts[key] = contract
        return contract

    def _runtime_key(self, x, valid_token_mask) -> RuntimeKey:
        name, capability, arch = self._device_contract(x.device)
        if valid_token_mask is None:
            kind = MaskKind.ABSENT
        elif x.device.type == "cuda":
            kind = self._mask_kind_cached(valid_token_mask)
        else:
            kind = classify_mask(valid_token_mask)
        return RuntimeKey(
            input_shape=tuple(x.shape), device_type=x.device.type, device_index=x.device.index,
            dtype=x.dtype, device_name=name, device_capability=capability, mask_kind=kind,
            inference_mode=torch.is_inference_mode_enabled(), grad_enabled=torch.is_grad_enabled(),
            matmul_precision=torch.get_float32_matmul_precision(),
            allow_tf32=bool(torch.backends.cuda.matmul.allow_tf32) if x.device.type == "cuda" else False,
            device_arch=arch,
        )

    def _resolve_route(self, key: RuntimeKey) -> RouteDecision:
        case_id = case_for(self.config)
        expected = (self.config.batch_size, self.config.seq_len, self.config.d_model)
        if key.input_shape != expected and case_id in EXTREME_CASES:
            return RouteDecision(case_id, UNSUPPORTED_BACKEND, None,
                                 "runtime input shape does not match the static extreme configuration")
        if key.mask_kind is MaskKind.GENERAL:
            return RouteDecision(case_id, UNSUPPORTED_BACKEND, None,
                                 "the kernels take right-padded masks only (left padding or gaps given)")
        return select_route(
            self.config, device_type=key.device_type, dtype=key.dtype, device_name=key.device_name,
            device_capability=key.device_capability, torch_version=torch.__version__,
            matmul_precision=key.matmul_precision, allow_tf32=key.allow_tf32, device_arch=key.device_arch,
        )

    def _call(self, key: RuntimeKey, cached: CachedForward, x, valid_token_mask):
        try:
            return cached.function(x, valid_token_mask)
        except UnsupportedCaseError:
            raise
        except Exception as err:  # recorded for diagnostics, never swallowed
            self._compile_failures[key] = f"{type(err).__name__}: {err}"
            raise

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        key = self._runtime_key(x, valid_token_mask)
        cached = self._compiled_forwards.get(key)
        if cached is not None:
            self._set_drop_key_mask(cached.drop_key_mask)
            return self._call(key, cached, x, valid_token_mask)
        route = self._resolve_route(key)
        self._last_route = route
        if route.backend == UNSUPPORTED_BACKEND:
            raise UnsupportedCaseError(f"case {route.case_id} is unsupported: {route.reason}")
        drop = bool(self.config.causal and key.mask_kind is MaskKind.PREFIX)
        self._set_drop_key_mask(drop)
        if route.backend == EXTREME_MEMORY_BACKEND:
            if not key.inference_mode or key.grad_enabled:
                raise UnsupportedCaseError(f"case {route.case_id} extreme route is inference-only")
            function = self._extreme_entrypoint(route.case_id)
        else:
            function = self._forward_hip
        cached = CachedForward(function, compiled=False, case_id=route.case_id, drop_key_mask=drop)
        self._compiled_forwards[key] = cached
        return self._call(key, cached, x, valid_token_mask)


CANDIDATE = CandidateSpec(
    name="dispatcher",
    model_factory=DispatchingTransformer,
    owner="techjam-amd",
    description=(
        "gfx950 HIP attention dispatcher: exact fused attention for every supported shape, "
        "packed QKV for cases 2/3 and C2, batch streaming for case 6, and guarded polynomial "
        "attention with per-head exact fallback for case 14."
    ),
    self_compiling=True,
    unsupported_official_cases=(),
    official_case_dtypes=((6, ("float32",)), (14, ("float16", "float32"))),
    candidate_only_official_cases=(14,),
    default_input_scale_only_cases=(14,),
    cuda_only_official_cases=tuple(range(1, 15)),
)
