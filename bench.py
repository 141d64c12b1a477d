#!/usr/bin/env python3
"""Benchmark of the attention hot path on one MI355X.

Default workload (the attention-core configuration the MFMA target is quoted
on): exact causal attention, batch 64, seq 4096, 16 heads, head_dim 64, fp32
q/k/v ~ N(0, 1) resident in HBM as [B, S, H, D] tensors viewed as [B, H, S, D].
One step = one forward of the attention layer core over the whole batch.

Prints ONE JSON line with the driver's fields plus
  roofline     : algorithmic FLOPs of one launch / its average duration,
                 timed with HIP events on the launch stream, against the
                 dense fp16 MFMA peak; `traffic` is the HBM bytes per launch
                 from rocprofv3 FETCH_SIZE/WRITE_SIZE (profiles/), or null;
  cpu_baseline : the dense FP32 oracle on this host's cores over a bounded
                 sample of the same workload (one batch element);
  samples_ms   : median / p90 / min / mean of the per-step HIP-event times
                 inside the timed region;
  memory       : peak HBM allocated during one step (inputs included);
  accuracy     : the timed output checked on sampled heads against exact
                 softmax attention evaluated in fp32 by torch on the GPU,
                 with the benchmark's rule (|d| <= 2e-3 or <= 2% of |ref|);
  extreme      : the same measurements for the extreme-length workload
                 (guarded polynomial attention, B=4 S=65536 H=16 D=64 with
                 one exact-fallback head per sample), timed in the same run
                 (``--no-extreme`` skips it);
  git, source_digest, seeds : what was measured.

Also in the line: ``environment`` (host, software, device), ``gpu_state``
(rocm-smi clocks/power/temperature sampled after the timed region) and, with
``--aa-reps N``, ``noise``: the step timed against itself N times, interleaved,
giving the A/A floor below which two measurements are not distinguishable.

Other workloads (``--workload``) exist for manual measurement; the driver
runs the default.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import re
import statistics
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable, List, Optional

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from techjam_amd.infra.environment import collect_environment, collect_git, collect_gpu_state  # noqa: E402
from techjam_amd.infra.timing import summarise_timings, time_interleaved  # noqa: E402
from techjam_amd.infra.workload import attention_bytes, exact_attention_flops, poly_flops, random_case  # noqa: E402

PEAK_MFMA_F16_TFLOPS = 2500.0   # MI355X dense fp16/bf16
PEAK_HBM_GBS = 8000.0           # MI355X HBM3E

METRIC = "attention-layer forward latency (ms) and tokens/s; % MFMA peak / % HBM BW"
TIMING_SEED = 1234 + 100000      # the reference harness's timing-input seed (src/benchmark.py:379)
ATOL, RTOL = 2e-3, 0.02          # torch_transformer_benchmark.py:309-319


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--workload", default="attn-core",
                   choices=["attn-core", "extreme", "model-c1", "model-c2", "model-c4", "copy-1gib",
                            "quad-apply", "quad-update", "causal-diag", "core-100k-exact", "core-100k-poly"]
                   + [f"case-{i}" for i in range(1, 15)])
    p.add_argument("--no-extreme", action="store_true",
                   help="with the default workload, skip the extreme-length measurement")
    p.add_argument("--no-accuracy", action="store_true", help="skip the sampled-heads accuracy check")
    p.add_argument("--no-models", action="store_true",
                   help="with the default workload, skip the C2/C4 encoder timings on both GEMM-operand paths")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-repeats", type=int, default=3)
    p.add_argument("--aa-reps", type=int, default=0,
                   help="after the timed region, time the step against itself (A/A control, "
                        "interleaved) this many times and report the noise floor")
    # Float32 GEMM flags of the model workloads; the defaults are the reference
    # harness's validated contract (src/benchmark.py:133-141, src/dispatcher.py:69-70).
    p.add_argument("--matmul-precision", choices=("highest", "high", "medium"), default="high")
    p.add_argument("--allow-tf32", action=argparse.BooleanOptionalAction, default=True)
    # Opt-in: encoder GEMM operands rounded to fp16 (TF32's mantissa), fp32 accumulation.
    p.add_argument("--gemm-operands", choices=("fp32", "fp16"), default="fp32")
    return p.parse_args()


@dataclass
class Workload:
    step: Callable[[], object]
    tokens: int
    flops: float
    bytes_alg: float
    config: dict
    profile: str
    data: str = "synthetic: q, k, v ~ N(0, 1) generated on the GPU (seed 101234)"
    bound: Optional[str] = None
    accuracy: Optional[Callable[[], dict]] = None
    seeds: dict = field(default_factory=lambda: {"timing_input": TIMING_SEED})


def traffic_from_profiles(name: str):
    """HBM bytes per launch recorded by the rocprofv3 counter runs, if committed.

    `name` is a file under profiles/, optionally `file#kernel` for a summary
    that records several kernels (`traffic_bytes_per_launch[kernel]: ...`).
    """
    name, _, kernel = name.partition("#")
    path = ROOT / "profiles" / name
    if not path.exists():
        return None
    key = r"traffic_bytes_per_launch" + (r"\[" + re.escape(kernel) + r"\]" if kernel else "")
    m = re.search(r"^" + key + r":\s*([0-9.eE+]+)", path.read_text(), re.M)
    return float(m.group(1)) if m else None


# -- accuracy: exact softmax attention in fp32 on the GPU ----------------------------

def exact_rows(q, k, v, b: int, h: int, rows: torch.Tensor, scale: float) -> torch.Tensor:
    """Causal softmax attention of query ``rows`` of head (b, h), fp32 on the device.

    Plain tensor ops under matmul precision "highest": scores of the rows
    against every key up to the last row, ``-inf`` above the diagonal, fp32
    softmax, product with v.
    """
    kmax = int(rows.max()) + 1
    qr = q[b, h].index_select(0, rows).float()
    kk = k[b, h, :kmax].float().contiguous()
    scores = (qr @ kk.t()) * scale
    cols = torch.arange(kmax, device=q.device)
    scores.masked_fill_(cols[None, :] > rows[:, None], float("-inf"))
    return torch.softmax(scores, dim=-1) @ v[b, h, :kmax].float().contiguous()


def check_heads(out, q, k, v, scale: float, heads, rows: torch.Tensor, what: str) -> dict:
    """The benchmark's per-element rule on ``rows`` of each (b, h) in ``heads``."""
    prev = torch.get_float32_matmul_precision()
    torch.set_float32_matmul_precision("highest")
    failed, total, max_abs = 0, 0, 0.0
    try:
        for b, h in heads:
            for r0 in range(0, rows.numel(), 1024):
                rr = rows[r0:r0 + 1024]
                ref = exact_rows(q, k, v, b, h, rr, scale)
                got = out[b, h].index_select(0, rr).float()
                err = (got - ref).abs()
                ok = torch.isfinite(got) & ((err <= ATOL) | (err <= RTOL * ref.abs()))
                failed += int((~ok).sum())
                total += ok.numel()
                max_abs = max(max_abs, float(torch.nan_to_num(err, nan=float("inf")).max()))
    finally:
        torch.set_float32_matmul_precision(prev)
    return {"passed": failed == 0, "failed_elements": failed, "total_elements": total, "max_abs_error": max_abs,
            "heads_checked": [list(x) for x in heads], "rows_per_head": int(rows.numel()),
            "tolerance": f"|d| <= {ATOL} or |d| <= {RTOL} * |ref|, finite",
            "reference": f"exact causal softmax attention in fp32 (torch on the GPU, matmul precision "
                         f"'highest') of the timed inputs; {what}"}


# -- workloads -------------------------------------------------------------------------

def attn_core(args, dev) -> Workload:
    from techjam_amd.kernels import scaled_dot_product_attention

    b, s, h, d = 64, 4096, 16, 64
    g = torch.Generator(device=dev).manual_seed(TIMING_SEED)
    q, k, v = (torch.randn(b, s, h, d, generator=g, device=dev).transpose(1, 2) for _ in range(3))
    out = torch.empty(b, s, h, d, device=dev).transpose(1, 2)
    scale = d ** -0.5

    def step():
        scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale, out=out)

    def accuracy():
        heads = [(0, 0), (63, 15), (17, 9)] + [((37 * i) % b, (5 * i + 3) % h) for i in range(13)]
        return check_heads(out, q, k, v, scale, heads, torch.arange(s, device=dev),
                           "16 of the 1024 (b, h) heads, every row")

    config = {
        "workload": "attention core: exact causal SDPA, B=64 S=4096 H=16 D=64, fp32 io",
        "batch": b, "seq_len": s, "heads": h, "head_dim": d, "causal": True,
        "layout": "[B,S,H,D] storage viewed as [B,H,S,D]",
        "mfma": "fp16 operands, fp32 accumulation",
    }
    return Workload(step, b * s, exact_attention_flops([s] * b, h, d), attention_bytes(b, s, h, d), config,
                    "attn_fwd_b64_s4096_h16_d64_causal.md", accuracy=accuracy)


def extreme(args, dev) -> Workload:
    """Guarded polynomial attention, B=4 S=65536 H=16 D=64; head 0 of each sample at sigma 4."""
    from techjam_amd.implementations.poly_attention import guarded_attention

    b, s, h, d = 4, 65536, 16, 64
    g = torch.Generator(device=dev).manual_seed(TIMING_SEED)
    q = torch.randn(b, s, h, d, generator=g, device=dev) * 0.5
    k = torch.randn(b, s, h, d, generator=g, device=dev) * 0.5
    v = torch.randn(b, s, h, d, generator=g, device=dev)
    q[:, :, 0] = torch.randn(b, s, d, generator=g, device=dev) * 2.0
    k[:, :, 0] = torch.randn(b, s, d, generator=g, device=dev) * 2.0
    qh, kh, vh = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    out = torch.empty(b, s, h, d, device=dev).transpose(1, 2)
    scale = d ** -0.5
    guards = []

    def step():
        guards[:] = [guarded_attention(qh, kh, vh, scale, out=out)[1]]

    def accuracy():
        flags = guards[0].flags.view(b, h).cpu()
        routes = {"polynomial_heads": int(flags.sum()), "exact_fallback_heads": int((flags == 0).sum())}
        # rows at the start, across the end of the exact prefix, and at the end
        rows = torch.cat([torch.arange(0, 512), torch.arange(3584, 4608), torch.arange(s - 512, s)]).to(dev)
        res = check_heads(out, qh, kh, vh, scale, [(0, 0), (3, 0), (0, 5), (1, 11), (2, 1), (3, 15)], rows,
                          "heads (b, 0) take the exact fallback, the others the polynomial route")
        res.update(routes)
        res["passed"] = res["passed"] and routes == {"polynomial_heads": 60, "exact_fallback_heads": 4}
        return res

    n_poly, n_exact = b * (h - 1), b
    flops = n_poly * poly_flops(s, d, d, 512, 4096) + exact_attention_flops([s] * n_exact, 1, d)
    config = {
        "workload": "extreme-length attention core: guarded degree-2 polynomial attention, "
                    "B=4 S=65536 H=16 D=64, fp32 io, 60 polynomial heads + 4 exact fallback heads",
        "batch": b, "seq_len": s, "heads": h, "head_dim": d, "chunk": 512, "exact_prefix": 4096,
    }
    return Workload(step, b * s, flops, attention_bytes(b, s, h, d), config, "poly_extreme_b4_s65536_h16_d64.md",
                    data="synthetic: q, k ~ N(0, 0.5^2), v ~ N(0, 1), head 0 of each sample q, k ~ N(0, 2^2), "
                         "generated on the GPU (seed 101234)", accuracy=accuracy)


def copy_1gib(args, dev) -> Workload:
    """Plain device copy of 1 GiB: calibrates the FETCH_SIZE / WRITE_SIZE counters."""
    n = 1 << 28
    src = torch.ones(n, device=dev)
    dst = torch.empty(n, device=dev)

    def step():
        dst.copy_(src)

    config = {"workload": "calibration: torch device copy of 2^28 fp32 (1 GiB read + 1 GiB write)"}
    return Workload(step, n, 0.0, 2.0 * 4 * n, config, "copy_1gib_calibration.md", bound="hbm")


def poly_part(name):
    """One stand-alone polynomial kernel at the reference's quoted shape
    (M=32 (b, h) pairs, C=512 tokens, D=V=64, the shape its timings for
    src/kernels/poly_attention_triton.py are quoted at)."""
    def build(args, dev) -> Workload:
        from techjam_amd.kernels.poly_parts import causal_diag, quad_apply, quad_update

        m, c, d = 32, 512, 64
        kernel = name.replace("-", "_")
        g = torch.Generator(device=dev).manual_seed(TIMING_SEED)
        a, b, v = (torch.randn(m, c, d, generator=g, device=dev, dtype=torch.float16) * 0.2 for _ in range(3))
        state = torch.randn(m, d * d, d, generator=g, device=dev)
        shadow = torch.zeros(m, d * d, d, device=dev, dtype=torch.float16)
        if name == "quad-apply":
            def step():
                quad_apply(a, state)
            flops, nbytes = 2.0 * m * c * d ** 3, m * d ** 3 * 4 + 2 * m * c * d * 2
        elif name == "quad-update":
            def step():
                quad_update(b, v, state, shadow=shadow)
            flops, nbytes = 2.0 * m * c * d ** 3, 2 * m * d ** 3 * 4 + m * d ** 3 * 2 + 2 * m * c * d * 2
        else:
            def step():
                causal_diag(a, b, v)
            flops, nbytes = 2.0 * m * d * c * (c + 1), 3 * m * c * d * 2 + m * c * (d + 1) * 4
        config = {"workload": f"stand-alone {kernel}: M={m} (b, h) pairs, C={c} tokens, D=V={d}, "
                              "fp16 operands, fp32 state", "m": m, "chunk": c, "head_dim": d}
        # the update reads and writes the fp32 state once per call: HBM sets its floor
        return Workload(step, m * c, flops, float(nbytes), config, "poly_parts_m32_c512_d64.md#" + kernel,
                        data="synthetic: a, b, v ~ N(0, 0.2^2) fp16, state ~ N(0, 1) fp32, generated on the GPU "
                             "(seed 101234)", bound="hbm" if name == "quad-update" else "mfma")
    return build


def model(name):
    def build(args, dev) -> Workload:
        from techjam_amd.dispatcher import DispatchingTransformer
        from techjam_amd.infra import BENCHMARK_CONFIGS
        from techjam_amd.model import TransformerConfig

        c = BENCHMARK_CONFIGS[name]
        cfg = TransformerConfig(c.batch_size, c.seq_len, c.d_model, c.num_heads, c.ffn_dim, c.num_layers, c.causal)
        torch.manual_seed(1234)  # default initialisation in the reference model's construction order
        cand = DispatchingTransformer(cfg).eval().to(dev)
        cand.gemm_operands = args.gemm_operands
        x, mask = random_case(c.batch_size, c.seq_len, c.d_model, TIMING_SEED, c.padding_ratio, 1.0)
        x, mask = x.to(dev), mask.to(dev)
        lengths = mask.sum(1).tolist()
        torch.set_float32_matmul_precision(args.matmul_precision)
        torch.backends.cuda.matmul.allow_tf32 = args.allow_tf32

        def step():
            with torch.inference_mode():
                cand(x, mask)

        def outputs():
            with torch.inference_mode():
                return cand(x, mask)

        hd = c.d_model // c.num_heads
        config = {"workload": f"{c.num_layers}-layer encoder {name}: {c.description}",
                  "batch": c.batch_size, "seq_len": c.seq_len, "d_model": c.d_model,
                  "heads": c.num_heads, "ffn_dim": c.ffn_dim, "layers": c.num_layers,
                  "roofline_scope": "attention FLOPs over the whole forward (GEMMs not counted)",
                  "gemm": f"hipBLASLt, fp32 tensors, matmul precision {args.matmul_precision!r}, "
                          f"allow_tf32={args.allow_tf32}"
                          if args.gemm_operands == "fp32" else
                          "hipBLASLt, fp16-rounded operands (TF32 mantissa), fp32 accumulation"}
        w = Workload(step, c.batch_size * c.seq_len, c.num_layers * exact_attention_flops(lengths, c.num_heads, hd),
                     0.0, config, f"model_{name.lower()}.md",
                     data="synthetic: x ~ N(0, 1) with right-padded masks (seed 101234), "
                          "default-initialised weights (seed 1234)",
                     seeds={"timing_input": TIMING_SEED, "weights": 1234})
        w.outputs = outputs
        return w
    build.__doc__ = BENCHMARK_CONFIG_TEXT.get(name)
    return build


# The reference's published candidate latencies on an RTX 5080, for context
# beside the same shapes here (research/benchmarks/2026-08-31-rtx5080-775c820/
# README.md:22-34 for cases 1-13; latest-dispatcher-case14.json: 67.095 s over
# five full forwards of case 14; research/benchmarks/2026-08-30-rtx5080-b9506f3/
# attention-core.json:37-39 for the attention core at N = 100 000).
REFERENCE_RTX5080_MS = {
    "case-1": 0.6975, "case-2": 0.1609, "case-3": 0.1643, "case-4": 0.2678, "case-5": 1.2513,
    "case-6": 210.5723, "case-7": 0.4060, "case-8": 15.5889, "case-9": 0.6881, "case-10": 0.6464,
    "case-11": 1.3724, "case-12": 0.2335, "case-13": 13.6078, "case-14": 67094.5 / 5,
    "core-100k-exact": 200.006, "core-100k-poly": 128.104,
}


def official_case(case_id: int):
    """Whole-model forward of one of the fourteen official cases: the
    dispatcher at the case's shape, default-initialised weights, the harness's
    inputs without padding (its default), float32 GEMMs under its flags."""
    def build(args, dev) -> Workload:
        from techjam_amd.dispatcher import DispatchingTransformer
        from techjam_amd.infra import load_official_cases
        from techjam_amd.model import TransformerConfig

        c = load_official_cases()[case_id]
        cfg = TransformerConfig(c.batch_size, c.seq_len, c.qkv_dim, c.heads, c.ffn_dim, c.layers, c.causal)
        torch.manual_seed(1234)
        cand = DispatchingTransformer(cfg).eval().to(dev)
        x, mask = random_case(c.batch_size, c.seq_len, c.qkv_dim, TIMING_SEED, 0.0, 1.0, device=dev)
        torch.set_float32_matmul_precision(args.matmul_precision)
        torch.backends.cuda.matmul.allow_tf32 = args.allow_tf32

        def step():
            with torch.inference_mode():
                cand(x, mask)

        hd = c.qkv_dim // c.heads
        config = {"workload": f"official case {case_id}: {c.layers}-layer encoder, B={c.batch_size} "
                              f"S={c.seq_len} d_model={c.qkv_dim} H={c.heads} FFN={c.ffn_dim}, causal",
                  "batch": c.batch_size, "seq_len": c.seq_len, "d_model": c.qkv_dim, "heads": c.heads,
                  "ffn_dim": c.ffn_dim, "layers": c.layers,
                  "reference_rtx5080_ms": REFERENCE_RTX5080_MS[f"case-{case_id}"],
                  "roofline_scope": "exact attention FLOPs over the whole forward (GEMMs not counted)",
                  "gemm": f"fp32 tensors, matmul precision {args.matmul_precision!r}, allow_tf32={args.allow_tf32}"}
        return Workload(step, c.batch_size * c.seq_len,
                        c.layers * exact_attention_flops([c.seq_len] * c.batch_size, c.heads, hd), 0.0, config,
                        f"case_{case_id}.md", data="synthetic: x ~ N(0, 1), no padding (seed 101234, generated on "
                        "the GPU), default-initialised weights (seed 1234)",
                        seeds={"timing_input": TIMING_SEED, "weights": 1234})
    return build


def core_100k(route: str):
    """The reference's attention-core benchmark shape (src/bench_poly.py:194-233):
    B=1, N=100 000, H=16, d=64, fp16 q, k, v ~ N(0, 0.577^2) as strided
    [B, N, H, D] views, causal; ``exact`` is exact attention, ``poly`` the
    polynomial path at the reference's fixed sigma 0.3338 (no guard)."""
    def build(args, dev) -> Workload:
        from techjam_amd.implementations.poly_attention import poly_attention_forward
        from techjam_amd.kernels import scaled_dot_product_attention

        b, n, h, d = 1, 100_000, 16, 64
        g = torch.Generator(device=dev).manual_seed(0)
        packed = [(torch.randn(b, n, h * d, generator=g, device=dev) * 0.577).half() for _ in range(3)]
        q, k, v = (t.view(b, n, h, d).transpose(1, 2) for t in packed)
        scale = d ** -0.5

        def step():
            with torch.inference_mode():
                if route == "exact":
                    scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale)
                else:
                    poly_attention_forward(q, k, v, scale, sigma=0.3338)

        flops = (exact_attention_flops([n], h, d) if route == "exact" else h * poly_flops(n, d, d, 512, 4096))
        config = {"workload": f"attention core at the reference's benchmark shape, {route}: B=1 N=100000 H=16 "
                              "d=64, fp16, causal",
                  "batch": b, "seq_len": n, "heads": h, "head_dim": d,
                  "reference_rtx5080_ms": REFERENCE_RTX5080_MS[f"core-100k-{route}"]}
        return Workload(step, b * n, flops, attention_bytes(b, n, h, d, 2), config, f"core_100k_{route}.md",
                        data="synthetic: q, k, v ~ N(0, 0.577^2) fp16 (seed 0, generated on the GPU)")
    return build


BENCHMARK_CONFIG_TEXT = {
    "C2": "4-layer encoder, B=8 S=1024 d_model=512 H=8 FFN=2048, packed QKV, causal, right padding",
    "C4": "4-layer encoder, B=2 S=8192 d_model=1024 H=16 FFN=4096, causal, right padding",
}


# -- measurement -----------------------------------------------------------------------

def timed(step, steps: int, warmup: int, dev):
    """``steps`` launches bracketed by device synchronisations, one HIP event
    per step boundary on the launch stream; returns (ms per step, per-step
    ms, wall seconds of the timed region)."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)  # the stream the kernels are launched on
    events = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    events[0].record(stream)
    for i in range(steps):
        step()
        events[i + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_step = [events[i].elapsed_time(events[i + 1]) for i in range(steps)]
    return events[0].elapsed_time(events[-1]) / steps, per_step, wall


def sample_stats(values: List[float]) -> dict:
    ordered = sorted(values)
    p90 = ordered[min(len(ordered) - 1, int(round(0.9 * (len(ordered) - 1))))]
    return {"median": round(statistics.median(ordered), 4), "p90": round(p90, 4), "min": round(ordered[0], 4),
            "mean": round(statistics.fmean(ordered), 4), "n": len(ordered)}


def step_memory(step, dev) -> dict:
    """Peak HBM allocated by torch's allocator during one step, resident inputs included."""
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    before = torch.cuda.memory_allocated(dev)
    step()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated(dev)
    return {"peak_allocated_bytes": peak, "before_step_allocated_bytes": before,
            "step_increment_bytes": peak - before}


def roofline_block(w: Workload, ms: float) -> dict:
    sec = ms / 1e3
    tflops = w.flops / sec / 1e12
    hbm_gbs = w.bytes_alg / sec / 1e9
    bound = w.bound or ("mfma" if w.flops else "hbm")
    block = {
        "bound": "mfma",
        "achieved": round(tflops, 2),
        "peak": PEAK_MFMA_F16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(tflops / PEAK_MFMA_F16_TFLOPS, 4),
    } if bound == "mfma" else {
        "bound": "hbm",
        "achieved": round(hbm_gbs, 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(hbm_gbs / PEAK_HBM_GBS, 4),
    }
    block.update({
        "traffic": traffic_from_profiles(w.profile),
        "algorithmic_flops_per_launch": w.flops,
        "algorithmic_bytes_per_launch": w.bytes_alg,
        "mfma_frac_algorithmic": round(tflops / PEAK_MFMA_F16_TFLOPS, 4),
        "hbm_frac_algorithmic": round(hbm_gbs / PEAK_HBM_GBS, 4),
    })
    return block


def measure(w: Workload, args, dev) -> dict:
    ms, per_step, wall = timed(w.step, args.steps, args.warmup, dev)
    rec = {
        "ms_per_step": round(ms, 4),
        "tokens_per_s": round(w.tokens / (ms / 1e3), 1),
        "samples_ms": sample_stats(per_step),
        "wall_s_timed_region": round(wall, 4),
        "roofline": roofline_block(w, ms),
        "memory": step_memory(w.step, dev),
    }
    if w.accuracy is not None and not args.no_accuracy:
        rec["accuracy"] = w.accuracy()
    return rec


def encoder_operand_paths(name: str, args, dev) -> dict:
    """One encoder (C2 or C4) timed on both GEMM-operand paths, same weights
    and inputs: float32 GEMMs under the harness flags, and fp16 operands with
    fp32 accumulation. ``max_abs_between_paths`` is how far the fp16 path's
    output moves from the float32 path's (the oracle comparison itself is in
    the tests)."""
    rec = {}
    outs = {}
    for operands in ("fp32", "fp16"):
        args.gemm_operands = operands
        w = model(name)(args, dev)
        ms, per_step, _ = timed(w.step, args.steps, args.warmup, dev)
        rec[operands] = {"ms_per_step": round(ms, 4), "tokens_per_s": round(w.tokens / (ms / 1e3), 1),
                         "samples_ms": sample_stats(per_step), "gemm": w.config["gemm"]}
        outs[operands] = w.outputs()
        del w
    rec["max_abs_between_paths"] = float((outs["fp16"] - outs["fp32"]).abs().max())
    rec["workload"] = f"{name}: {model(name).__doc__ or ''}".strip()
    args.gemm_operands = "fp32"
    torch.set_float32_matmul_precision("highest")  # the model builder set the harness flags
    torch.backends.cuda.matmul.allow_tf32 = False
    return rec


def cpu_baseline_attn_core(repeats: int):
    """Dense FP32 oracle attention on the host: one batch element (16 heads x 4096)."""
    from oracle.model import DenseSelfAttention

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    h, s, d = 16, 4096, 64
    g = torch.Generator().manual_seed(TIMING_SEED)
    q, k, v = (torch.randn(1, h, s, d, generator=g) for _ in range(3))
    attn = DenseSelfAttention(h * d, h)
    with torch.inference_mode():
        attn.attend(q, k, v, None, True)  # warm-up
        times = []
        for _ in range(repeats):
            t0 = time.perf_counter_ns()
            attn.attend(q, k, v, None, True)
            times.append((time.perf_counter_ns() - t0) / 1e9)
    med = statistics.median(times)
    return {
        "value": s / med,
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"oracle dense fp32 causal attention, 1 of 64 batch elements (16 heads x 4096 x 64), "
                  f"median of {repeats} after 1 warm-up: {med * 1e3:.1f} ms",
    }


def git_record() -> dict:
    """The repository's commit when it has one here; otherwise (a copy of the
    tree without history) the commit the in-tree library was built at, with
    whether the kernel sources still match that build."""
    rec = collect_git(ROOT)
    if rec.get("commit"):
        return rec
    from techjam_amd import build as tj_build

    try:
        info = json.loads(tj_build.BUILD_INFO.read_text())
    except (OSError, ValueError):
        return rec
    return {"commit": info.get("commit"), "dirty": info.get("library_sources_dirty"), "status": "",
            "source": "library build record",
            "library_sources_match": info.get("library_source_digest") == tj_build.library_source_digest()}


def source_digest() -> str:
    """sha256 (16 hex digits) of the kernel sources, the C header and this file."""
    h = hashlib.sha256()
    files = sorted((ROOT / "techjam_amd" / "csrc").glob("*")) + sorted((ROOT / "include").glob("*.h"))
    for f in files + [Path(__file__).resolve()]:
        h.update(f.name.encode())
        h.update(f.read_bytes())
    return h.hexdigest()[:16]


BUILDERS = {"attn-core": attn_core, "extreme": extreme, "copy-1gib": copy_1gib,
            "quad-apply": poly_part("quad-apply"), "quad-update": poly_part("quad-update"),
            "causal-diag": poly_part("causal-diag"),
            "model-c1": model("C1"), "model-c2": model("C2"), "model-c4": model("C4"),
            "core-100k-exact": core_100k("exact"), "core-100k-poly": core_100k("poly"),
            **{f"case-{i}": official_case(i) for i in range(1, 15)}}


def main():
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the library has no multi-GPU path "
              "(each (b, h) is independent; see the sharding notes)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False

    w = BUILDERS[args.workload](args, dev)
    head = measure(w, args, dev)
    gpu_state = collect_gpu_state(dev)
    noise = None
    if args.aa_reps > 0:
        samples = time_interleaved({"step_ms": w.step, "step_control_ms": w.step}, args.aa_reps)
        stats = summarise_timings(samples, [("step_ms", "step_control_ms")])
        noise = {"samples_ms": samples, "variants": stats["variants"], **stats["noise"]}

    extreme_rec = None
    if args.workload == "attn-core" and not args.no_extreme:
        del w.step, w.accuracy  # free the attention-core tensors before allocating the next workload
        torch.cuda.empty_cache()
        wx = extreme(args, dev)
        extreme_rec = {"metric": METRIC, "config": wx.config, "data": wx.data, **measure(wx, args, dev)}
        del wx
        torch.cuda.empty_cache()

    models_rec = None
    if args.workload == "attn-core" and not args.no_models:
        models_rec = {name: encoder_operand_paths(name, args, dev) for name in ("C2", "C4")}
        torch.cuda.empty_cache()

    cpu = None
    if args.workload == "attn-core" and not args.no_cpu_baseline:
        cpu = cpu_baseline_attn_core(args.cpu_repeats)

    line = {
        "metric": METRIC,
        "value": head["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": w.data,
        "config": w.config,
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "samples_ms": head["samples_ms"],
        "memory": head["memory"],
        "accuracy": head.get("accuracy"),
        "extreme": extreme_rec,
        "encoders": models_rec,
        "wall_s_timed_region": head["wall_s_timed_region"],
        "seeds": w.seeds,
        "git": git_record(),
        "source_digest": source_digest(),
        "environment": collect_environment(torch, dev),
        "gpu_state": gpu_state,
    }
    if noise is not None:
        line["noise"] = noise
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
