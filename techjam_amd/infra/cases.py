"""Case tables: the reference's fourteen disclosed shapes and the five benchmark workloads.

``OFFICIAL_CASES`` holds the organiser's shape table that the reference keeps
in ``src/cases/task_shapes.json`` (loaded by ``src/infra/cases.py:54-71``); the
values are data the route table must key on, so they are the same.
``BENCHMARK_CONFIGS`` are the five benchmark configurations (C1-C5) the kernels are measured on.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional


@dataclass(frozen=True)
class OfficialCase:
    id: int
    batch_size: int
    qkv_dim: int
    heads: int
    seq_len: int
    layers: int
    causal: bool
    ffn_dim: int

    def validate(self) -> None:
        if min(self.id, self.batch_size, self.qkv_dim, self.heads, self.seq_len, self.layers, self.ffn_dim) <= 0:
            raise ValueError(f"case {self.id} contains a non-positive value")
        if self.qkv_dim % self.heads:
            raise ValueError(f"case {self.id}: qkv_dim must be divisible by heads")

    def benchmark_config(self) -> Dict[str, object]:
        return {"batch_size": self.batch_size, "d_model": self.qkv_dim, "heads": self.heads,
                "seq_len": self.seq_len, "layers": self.layers, "causal": self.causal,
                "ffn_dim": self.ffn_dim}


# id: (batch, qkv_dim, heads, seq_len, layers, causal, ffn_dim)
_OFFICIAL = {
    1: (64, 128, 4, 128, 4, True, 128),
    2: (1, 128, 4, 128, 4, True, 128),
    3: (4, 128, 4, 128, 4, True, 128),
    4: (16, 128, 4, 128, 4, True, 128),
    5: (128, 128, 4, 128, 4, True, 128),
    6: (10000, 128, 4, 128, 4, True, 128),
    7: (64, 32, 4, 128, 4, True, 32),
    8: (64, 1024, 4, 128, 4, True, 1024),
    9: (64, 128, 1, 128, 4, True, 128),
    10: (64, 128, 2, 128, 4, True, 128),
    11: (64, 128, 16, 128, 4, True, 128),
    12: (64, 128, 4, 32, 4, True, 128),
    13: (64, 128, 4, 1024, 4, True, 128),
    14: (32, 1024, 16, 100000, 2, True, 1024),
}


def load_official_cases() -> Dict[int, OfficialCase]:
    cases = {}
    for cid, (b, d, h, s, layers, causal, ffn) in _OFFICIAL.items():
        case = OfficialCase(cid, b, d, h, s, layers, causal, ffn)
        case.validate()
        cases[cid] = case
    return cases


@dataclass(frozen=True)
class BenchmarkConfig:
    """One of the five measured workloads. ``layers == 0`` marks an attention-core workload."""

    name: str
    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    num_layers: int
    causal: bool
    padding_ratio: float
    description: str

    @property
    def head_dim(self) -> int:
        return self.d_model // self.num_heads

    def model_key(self) -> Optional[tuple]:
        if self.num_layers == 0:
            return None
        return (self.batch_size, self.seq_len, self.d_model, self.num_heads, self.ffn_dim,
                self.causal, self.num_layers)


BENCHMARK_CONFIGS = {
    "C1": BenchmarkConfig("C1", 2, 128, 256, 4, 1024, 1, True, 0.5,
                          "1-layer pre-norm encoder, fp32, causal + right padding (valid length in [64, 128])"),
    "C2": BenchmarkConfig("C2", 8, 1024, 512, 8, 2048, 4, True, 0.5,
                          "4-layer encoder, packed QKV projection, causal + right padding ([512, 1024])"),
    "C3": BenchmarkConfig("C3", 64, 4096, 1024, 16, 0, 0, True, 0.0,
                          "attention core, q/k/v ~ N(0, 1), causal, no padding"),
    "C4": BenchmarkConfig("C4", 2, 8192, 1024, 16, 4096, 4, True, 0.5,
                          "4-layer encoder, causal + right padding ([4096, 8192])"),
    "C5": BenchmarkConfig("C5", 4, 65536, 1024, 16, 0, 0, True, 0.0,
                          "extreme-length attention core, q/k ~ N(0, 0.5^2), head 0 of every sample "
                          "~ N(0, 2^2) (exact fallback), guarded polynomial attention"),
}
