"""Candidate contract and case tables (mirrors ``src/infra`` of the reference)."""

from .candidate import CandidateSpec, as_spec, load_candidate, validate_candidate_execution
from .cases import BENCHMARK_CONFIGS, OfficialCase, load_official_cases

__all__ = [
    "BENCHMARK_CONFIGS",
    "CandidateSpec",
    "as_spec",
    "OfficialCase",
    "load_candidate",
    "load_official_cases",
    "validate_candidate_execution",
]
