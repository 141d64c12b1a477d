"""Candidate contract consumed by a benchmark harness.

Same fields and refusal rules as the reference's ``src/infra/candidate.py:15-232``;
the only generalisation is that device constraints are phrased for any GPU
runtime torch exposes as ``"cuda"`` -- ROCm here.

The reference's ``load_candidate`` accepts only instances of *its own*
``CandidateSpec`` class (``src/infra/candidate.py:156``), so this package's
``CANDIDATE`` reaches a reference harness through ``as_spec``: a module on the
reference side builds the reference's class from this one's fields.
"""

from __future__ import annotations

import dataclasses
import importlib
import re
from dataclasses import dataclass
from typing import Any, Callable, Optional, Tuple

ModelFactory = Callable[[Any], Any]
WeightLoader = Callable[[Any, Any, bool], None]

_DTYPE_NAMES = ("float32", "float16", "bfloat16")


def _case_ids_ok(ids) -> bool:
    return all(isinstance(c, int) and 1 <= c <= 14 for c in ids)


@dataclass(frozen=True)
class CandidateSpec:
    """Description and construction hooks of one full-model candidate."""

    name: str
    model_factory: ModelFactory
    owner: str
    description: str
    weight_loader: Optional[WeightLoader] = None
    strict_weight_copy: bool = True
    self_compiling: bool = False
    unsupported_official_cases: Tuple[int, ...] = ()
    official_case_dtypes: Tuple[Tuple[int, Tuple[str, ...]], ...] = ()
    candidate_only_official_cases: Tuple[int, ...] = ()
    default_input_scale_only_cases: Tuple[int, ...] = ()
    cuda_only_official_cases: Tuple[int, ...] = ()
    official_case_min_cuda_capability: Tuple[Tuple[int, Tuple[int, int]], ...] = ()
    official_case_torch_versions: Tuple[Tuple[int, Tuple[str, ...]], ...] = ()

    def validate(self) -> None:
        if not re.fullmatch(r"[a-z0-9][a-z0-9_-]*", self.name):
            raise ValueError("candidate name must contain only lowercase letters, numbers, "
                             "underscores, and hyphens")
        if not callable(self.model_factory):
            raise TypeError("candidate model_factory must be callable")
        if self.weight_loader is not None and not callable(self.weight_loader):
            raise TypeError("candidate weight_loader must be callable")
        if not isinstance(self.self_compiling, bool):
            raise TypeError("candidate self_compiling must be a bool")
        for label, ids in (("unsupported_official_cases", self.unsupported_official_cases),
                           ("candidate_only_official_cases", self.candidate_only_official_cases),
                           ("default_input_scale_only_cases", self.default_input_scale_only_cases),
                           ("cuda_only_official_cases", self.cuda_only_official_cases)):
            if not isinstance(ids, tuple):
                raise TypeError(f"candidate {label} must be a tuple")
            if not _case_ids_ok(ids):
                raise ValueError(f"{label} must contain only ids 1 through 14")
        if len(set(self.unsupported_official_cases)) != len(self.unsupported_official_cases):
            raise ValueError("unsupported official cases must not contain duplicates")
        seen = set()
        for case_id, dtypes in self.official_case_dtypes:
            if not _case_ids_ok((case_id,)):
                raise ValueError("dtype contracts require official case ids 1 through 14")
            if case_id in seen:
                raise ValueError("dtype contracts must not repeat an official case")
            if not isinstance(dtypes, tuple) or not dtypes:
                raise TypeError("dtype contracts must contain a non-empty dtype tuple")
            if any(d not in _DTYPE_NAMES for d in dtypes):
                raise ValueError("dtype contracts contain an unsupported dtype name")
            seen.add(case_id)
        seen = set()
        for case_id, cap in self.official_case_min_cuda_capability:
            if not _case_ids_ok((case_id,)):
                raise ValueError("capability contracts require case ids 1 through 14")
            if case_id in seen:
                raise ValueError("capability contracts must not repeat a case")
            if not (isinstance(cap, tuple) and len(cap) == 2
                    and all(isinstance(x, int) and x >= 0 for x in cap)):
                raise TypeError("device capabilities must be non-negative integer pairs")
            seen.add(case_id)
        seen = set()
        for case_id, versions in self.official_case_torch_versions:
            if not _case_ids_ok((case_id,)):
                raise ValueError("version contracts require case ids 1 through 14")
            if case_id in seen:
                raise ValueError("version contracts must not repeat a case")
            if not (isinstance(versions, tuple) and versions
                    and all(isinstance(v, str) and v for v in versions)):
                raise TypeError("version contracts require non-empty version strings")
            seen.add(case_id)


def as_spec(spec_class, candidate: CandidateSpec):
    """``candidate`` rebuilt as an instance of another ``CandidateSpec`` class
    with the same fields -- the reference's, so that its ``load_candidate``
    type check passes. Values are passed as they are (the model factory stays
    this package's ``DispatchingTransformer``); a field the target class lacks,
    or one it requires that this class does not have, is an error."""
    ours = {f.name for f in dataclasses.fields(CandidateSpec)}
    theirs = {f.name for f in dataclasses.fields(spec_class)}
    if ours != theirs:
        raise TypeError(f"{spec_class.__qualname__} fields differ from the candidate contract: "
                        f"missing {sorted(ours - theirs)}, extra {sorted(theirs - ours)}")
    return spec_class(**{name: getattr(candidate, name) for name in sorted(ours)})


def load_candidate(selector: str) -> CandidateSpec:
    """Load ``module[:attribute]``; a bare name resolves under ``techjam_amd.implementations``."""
    module_name, sep, attr = selector.partition(":")
    if not module_name:
        raise ValueError("candidate selector must not be empty")
    if "." not in module_name:
        module_name = f"techjam_amd.implementations.{module_name}"
    attr = attr if sep else "CANDIDATE"
    if not attr:
        raise ValueError("candidate attribute must not be empty")
    module = importlib.import_module(module_name)
    try:
        cand = getattr(module, attr)
    except AttributeError as err:
        raise AttributeError(f"candidate module {module_name!r} has no {attr!r} attribute") from err
    if not isinstance(cand, CandidateSpec):
        raise TypeError(f"{module_name}:{attr} must be a CandidateSpec, got {type(cand).__name__}")
    cand.validate()
    return cand


def validate_candidate_execution(spec: CandidateSpec, official_case_id: Optional[int], *, compile_user: bool,
                                 dtype_name: Optional[str] = None, candidate_only: bool = False,
                                 input_scale: float = 1.0, device_type: Optional[str] = None,
                                 cuda_capability: Optional[Tuple[int, int]] = None,
                                 torch_version: Optional[str] = None) -> None:
    """Refuse harness options that violate the candidate's contract, before any allocation."""
    if spec.self_compiling and compile_user:
        raise ValueError(f"candidate {spec.name!r} compiles itself; remove --compile-user "
                         "to avoid nested compilation")
    if official_case_id in spec.unsupported_official_cases:
        raise ValueError(f"candidate {spec.name!r} explicitly does not support official case "
                         f"{official_case_id}; refusing before model/input allocation")
    allowed = dict(spec.official_case_dtypes).get(official_case_id)
    if allowed is not None and dtype_name not in allowed:
        raise ValueError(f"candidate {spec.name!r} supports official case {official_case_id} only with "
                         f"{', '.join(allowed)}; received {dtype_name}; refusing before model/input allocation")
    if official_case_id in spec.candidate_only_official_cases and not candidate_only:
        raise ValueError(f"official case {official_case_id} has no runnable dense baseline; "
                         "use the candidate-only runner")
    if official_case_id in spec.default_input_scale_only_cases and input_scale != 1.0:
        raise ValueError(f"official case {official_case_id} is validated only at the default input scale 1.0")
    if official_case_id in spec.cuda_only_official_cases and device_type != "cuda":
        raise ValueError(f"official case {official_case_id} requires a GPU device; "
                         "refusing before model/input allocation")
    minimum = dict(spec.official_case_min_cuda_capability).get(official_case_id)
    if minimum is not None and (cuda_capability is None or cuda_capability < minimum):
        raise ValueError(f"official case {official_case_id} requires device capability {minimum} or newer; "
                         "refusing before model/input allocation")
    versions = dict(spec.official_case_torch_versions).get(official_case_id)
    if versions is not None and torch_version not in versions:
        raise ValueError(f"official case {official_case_id} requires PyTorch {', '.join(versions)}; "
                         "refusing before model/input allocation")
