"""The streaming planner's budget holds on the GPU (GPU).

For official case 6 (B=10000, 4 layers, batch-streamed) and one streamed
sample of the case-14 model, the peak memory torch's allocator records
during the forward stays within what the planner reserved for it: the whole
batch's output, the library allowance and chunk x per-item working set.
"""

from __future__ import annotations

import pytest
import torch

from oracle.model import TransformerConfig, generate_random_case

pytestmark = pytest.mark.gpu


def _peak_during(fn):
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    out = fn()
    torch.cuda.synchronize()
    return out, torch.cuda.max_memory_allocated() - base


@pytest.mark.parametrize("budget", [None, 1 << 30])
def test_case_6_peak_within_plan(cuda, budget):
    from techjam_amd.dispatcher import DispatchingTransformer

    cfg = TransformerConfig(10000, 128, 128, 4, 128, 4, True)
    torch.manual_seed(1234)
    cand = DispatchingTransformer(cfg).eval().to(cuda)
    cand.memory_budget_bytes = budget
    x, mask = generate_random_case(cfg, torch.device("cpu"), torch.float32, 1234, 0.0, 1.0)
    x, mask = x.to(cuda), mask.to(cuda)
    with torch.inference_mode():
        # library workspaces come up outside the measurement (the extreme
        # route accepts only the full batch, so warm up on its chunk forward)
        cand._forward_hip_chunk(x[:64].contiguous(), mask[:64].contiguous())
        out, peak = _peak_during(lambda: cand(x, mask))
    plan = cand.last_chunk_plan
    print(f"case 6 budget={budget}: chunk={plan.chunk} planned={plan.planned_peak_bytes / 2**20:.0f} MiB "
          f"measured={peak / 2**20:.0f} MiB")
    assert cand.last_route.backend == "extreme-memory"
    if budget is not None:
        assert plan.chunk == 256 and plan.planned_peak_bytes <= budget
    assert peak <= plan.planned_peak_bytes
    assert bool(torch.isfinite(out).all())


def test_case_14_streamed_sample_peak_within_plan(cuda):
    from techjam_amd.dispatcher import DispatchingTransformer

    cfg = TransformerConfig(32, 100000, 1024, 16, 1024, 2, True)
    torch.manual_seed(1234)
    cand = DispatchingTransformer(cfg).eval().to(cuda)
    g = torch.Generator().manual_seed(7)
    x = torch.randn(1, 8192, 1024, generator=g).to(cuda)
    with torch.inference_mode():
        cand.forward_case14_streamed_sample(x[:, :1024].contiguous())  # warm-up
        out, peak = _peak_during(lambda: cand.forward_case14_streamed_sample(x))
    plan = cand.last_chunk_plan
    print(f"case 14 sample: planned={plan.planned_peak_bytes / 2**20:.0f} MiB measured={peak / 2**20:.0f} MiB")
    assert plan.chunk == 1 and peak <= plan.planned_peak_bytes
    assert bool(torch.isfinite(out).all())
