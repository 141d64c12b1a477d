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

Also in the line: ``environment`` (host, software, device), ``gpu_state``
(rocm-smi clocks/power/temperature sampled after the timed region) and, with
``--aa-reps N``, ``noise``: the step timed against itself N times, interleaved,
giving the A/A floor below which two measurements are not distinguishable.

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

from techjam_amd.infra.environment import collect_environment, collect_gpu_state  # noqa: E402
from techjam_amd.infra.timing import summarise_timings, time_interleaved  # noqa: E402

PEAK_MFMA_F16_TFLOPS = 2500.0   # MI355X dense fp16/bf16
PEAK_HBM_GBS = 8000.0           # MI355X HBM3E

METRIC = "attention-layer forward latency (ms) and tokens/s; % MFMA peak / % HBM BW"


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--workload", default="attn-core",
                   choices=["attn-core", "extreme", "model-c1", "model-c2", "model-c4", "copy-1gib",
                            "quad-apply", "quad-update", "causal-diag"])
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


def poly_part(name):
    """One stand-alone polynomial kernel at the reference's quoted shape
    (M=32 (b, h) pairs, C=512 tokens, D=V=64, the shape its timings for
    src/kernels/poly_attention_triton.py are quoted at)."""
    def build(args, dev):
        from techjam_amd.kernels.poly_parts import causal_diag, quad_apply, quad_update

        m, c, d = 32, 512, 64
        kernel = name.replace("-", "_")
        g = torch.Generator(device=dev).manual_seed(1234 + 100000)
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
                              "fp16 operands, fp32 state", "m": m, "chunk": c, "head_dim": d,
                  # the update reads and writes the fp32 state once per call: HBM sets its floor
                  "bound": "hbm" if name == "quad-update" else "mfma",
                  "data": "synthetic: a, b, v ~ N(0, 0.2^2) fp16, state ~ N(0, 1) fp32, generated on the GPU "
                          "(seed 101234)"}
        return step, m * c, flops, float(nbytes), config, "poly_parts_m32_c512_d64.md#" + kernel
    return build


def extreme(args, dev):
    """Guarded polynomial attention, B=4 S=65536 H=16 D=64; head 0 of each sample at sigma 4."""
    from oracle.poly import poly_flops
    from techjam_amd.implementations.poly_attention import guarded_attention

    b, s, h, d = 4, 65536, 16, 64
    g = torch.Generator(device=dev).manual_seed(1234 + 100000)
    q = torch.randn(b, s, h, d, generator=g, device=dev) * 0.5
    k = torch.randn(b, s, h, d, generator=g, device=dev) * 0.5
    v = torch.randn(b, s, h, d, generator=g, device=dev)
    q[:, :, 0] = torch.randn(b, s, d, generator=g, device=dev) * 2.0
    k[:, :, 0] = torch.randn(b, s, d, generator=g, device=dev) * 2.0
    qh, kh, vh = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    out = torch.empty(b, s, h, d, device=dev).transpose(1, 2)
    scale = d ** -0.5

    def step():
        guarded_attention(qh, kh, vh, scale, out=out)

    n_poly, n_exact = b * (h - 1), b
    flops = n_poly * poly_flops(s, d, d, 512, 4096) + n_exact * 2.0 * d * s * (s + 1)
    bytes_alg = 16.0 * b * s * h * d
    config = {
        "workload": "extreme-length attention core: guarded degree-2 polynomial attention, "
                    "B=4 S=65536 H=16 D=64, fp32 io, 60 polynomial heads + 4 exact fallback heads",
        "batch": b, "seq_len": s, "heads": h, "head_dim": d, "chunk": 512, "exact_prefix": 4096,
        "data": "synthetic: q, k ~ N(0, 0.5^2), v ~ N(0, 1), head 0 of each sample q, k ~ N(0, 2^2), "
                "generated on the GPU (seed 101234)",
    }
    return step, b * s, flops, bytes_alg, config, "poly_extreme_b4_s65536_h16_d64.md"


def model(name):
    def build(args, dev):
        from oracle.model import DenseTransformer, generate_random_case
        from oracle.model import TransformerConfig as OracleConfig
        from techjam_amd.dispatcher import DispatchingTransformer
        from techjam_amd.infra import BENCHMARK_CONFIGS

        c = BENCHMARK_CONFIGS[name]
        cfg = OracleConfig(c.batch_size, c.seq_len, c.d_model, c.num_heads, c.ffn_dim, c.num_layers, c.causal)
        torch.manual_seed(1234)
        base = DenseTransformer(cfg).eval()
        cand = DispatchingTransformer(cfg).eval()
        cand.load_state_dict(base.state_dict())
        cand = cand.to(dev)
        cand.gemm_operands = args.gemm_operands
        x, mask = generate_random_case(cfg, torch.device("cpu"), torch.float32, 1234 + 100000,
                                       c.padding_ratio, 1.0)
        x, mask = x.to(dev), mask.to(dev)
        lengths = mask.sum(1).tolist()
        torch.set_float32_matmul_precision(args.matmul_precision)
        torch.backends.cuda.matmul.allow_tf32 = args.allow_tf32

        def step():
            with torch.inference_mode():
                cand(x, mask)

        hd = c.d_model // c.num_heads
        flops = c.num_layers * 2.0 * hd * c.num_heads * sum(n * (n + 1) for n in lengths)
        config = {"workload": f"{c.num_layers}-layer encoder {name}: {c.description}",
                  "batch": c.batch_size, "seq_len": c.seq_len, "d_model": c.d_model,
                  "heads": c.num_heads, "ffn_dim": c.ffn_dim, "layers": c.num_layers,
                  "roofline_scope": "attention FLOPs over the whole forward (GEMMs not counted)",
                  "gemm": f"hipBLASLt, fp32 tensors, matmul precision {args.matmul_precision!r}, "
                          f"allow_tf32={args.allow_tf32}"
                          if args.gemm_operands == "fp32" else
                          "hipBLASLt, fp16-rounded operands (TF32 mantissa), fp32 accumulation"}
        return step, c.batch_size * c.seq_len, flops, 0.0, config, f"model_{name.lower()}.md"
    return build


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

    builders = {"attn-core": attn_core, "extreme": extreme, "copy-1gib": copy_1gib,
                "quad-apply": poly_part("quad-apply"), "quad-update": poly_part("quad-update"),
                "causal-diag": poly_part("causal-diag"),
                "model-c1": model("C1"), "model-c2": model("C2"), "model-c4": model("C4")}
    step, tokens, flops, bytes_alg, config, prof_name = builders[args.workload](args, dev)
    if args.workload != "attn-core":
        args.no_cpu_baseline = True

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
    gpu_state = collect_gpu_state(dev)
    noise = None
    if args.aa_reps > 0:
        samples = time_interleaved({"step_ms": step, "step_control_ms": step}, args.aa_reps)
        stats = summarise_timings(samples, [("step_ms", "step_control_ms")])
        noise = {"samples_ms": samples, "variants": stats["variants"], **stats["noise"]}

    sec = ms_per_step / 1e3
    tflops = flops / sec / 1e12
    hbm_gbs = bytes_alg / sec / 1e9
    bound = config.pop("bound", "mfma" if flops else "hbm")
    roofline = {
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
        "data": config.pop("data", "synthetic: q, k, v ~ N(0, 1) generated on the GPU (seed 101234)"),
        "config": config,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "wall_s_timed_region": round(wall, 4),
        "environment": collect_environment(torch, dev),
        "gpu_state": gpu_state,
    }
    if noise is not None:
        line["noise"] = noise
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
