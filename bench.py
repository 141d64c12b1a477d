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
                 sample of the same workload (one batch element).

Other workloads (``--workload``) exist for manual measurement; the driver
runs the default.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_MFMA_F16_TFLOPS = 2500.0   # MI355X dense fp16/bf16
PEAK_HBM_GBS = 8000.0           # MI355X HBM3E

METRIC = "attention-layer forward latency (ms) and tokens/s; % MFMA peak / % HBM BW"


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--workload", default="attn-core", choices=["attn-core", "copy-1gib"])
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-repeats", type=int, default=3)
    return p.parse_args()


def traffic_from_profiles(name: str):
    """HBM bytes per launch recorded by the rocprofv3 counter runs, if committed."""
    path = ROOT / "profiles" / name
    if not path.exists():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", path.read_text(), re.M)
    return float(m.group(1)) if m else None


def attn_core(args, dev):
    from techjam_amd.kernels import scaled_dot_product_attention

    b, s, h, d = 64, 4096, 16, 64
    g = torch.Generator(device=dev).manual_seed(1234 + 100000)
    q, k, v = (torch.randn(b, s, h, d, generator=g, device=dev).transpose(1, 2) for _ in range(3))
    out = torch.empty(b, s, h, d, device=dev).transpose(1, 2)
    scale = d ** -0.5

    def step():
        scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale, out=out)

    flops = 2.0 * d * h * b * s * (s + 1)        # QK^T + PV, lower triangle incl. diagonal
    bytes_alg = 16.0 * b * s * h * d             # fp32 q, k, v read once, o written once
    config = {
        "workload": "attention core: exact causal SDPA, B=64 S=4096 H=16 D=64, fp32 io",
        "batch": b, "seq_len": s, "heads": h, "head_dim": d, "causal": True,
        "layout": "[B,S,H,D] storage viewed as [B,H,S,D]",
        "mfma": "fp16 operands, fp32 accumulation",
    }
    return step, b * s, flops, bytes_alg, config, "attn_fwd_b64_s4096_h16_d64_causal.md"


def copy_1gib(args, dev):
    """Plain device copy of 1 GiB: calibrates the FETCH_SIZE / WRITE_SIZE counters."""
    n = 1 << 28
    src = torch.ones(n, device=dev)
    dst = torch.empty(n, device=dev)

    def step():
        dst.copy_(src)

    config = {"workload": "calibration: torch device copy of 2^28 fp32 (1 GiB read + 1 GiB write)"}
    return step, n, 0.0, 2.0 * 4 * n, config, "copy_1gib_calibration.md"


def cpu_baseline_attn_core(repeats: int):
    """Dense FP32 oracle attention on the host: one batch element (16 heads x 4096)."""
    from oracle.model import DenseSelfAttention

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    h, s, d = 16, 4096, 64
    g = torch.Generator().manual_seed(1234 + 100000)
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


def main():
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(each (b, h) is independent; see the sharding notes)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False

    if args.workload == "copy-1gib":
        step, tokens, flops, bytes_alg, config, prof_name = copy_1gib(args, dev)
        args.no_cpu_baseline = True
    else:
        step, tokens, flops, bytes_alg, config, prof_name = attn_core(args, dev)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream(dev)  # the stream the kernels are launched on
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = e0.elapsed_time(e1) / args.steps

    sec = ms_per_step / 1e3
    tflops = flops / sec / 1e12
    hbm_gbs = bytes_alg / sec / 1e9
    roofline = {
        "bound": "mfma",
        "achieved": round(tflops, 2),
        "peak": PEAK_MFMA_F16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(tflops / PEAK_MFMA_F16_TFLOPS, 4),
    } if flops else {
        "bound": "hbm",
        "achieved": round(hbm_gbs, 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(hbm_gbs / PEAK_HBM_GBS, 4),
    }
    roofline.update({
        "traffic": traffic_from_profiles(prof_name),
        "algorithmic_flops_per_launch": flops,
        "algorithmic_bytes_per_launch": bytes_alg,
        "hbm_frac_algorithmic": round(hbm_gbs / PEAK_HBM_GBS, 4),
    })
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_attn_core(args.cpu_repeats)
    line = {
        "metric": METRIC,
        "value": round(tokens / sec, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: q, k, v ~ N(0, 1) generated on the GPU (seed 101234)",
        "config": config,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "wall_s_timed_region": round(wall, 4),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
