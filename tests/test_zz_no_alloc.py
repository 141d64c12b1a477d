"""tj_score_guard_noalloc against tj_score_guard through the C ABI (GPU).

The allocation-free entry point runs the same kernels with the partial sums
in the library's fixed device scratch instead of a caller's workspace, so its
outputs must be bitwise those of the workspace entry point. Two calls in a
row, the second on a smaller input, check that a call never depends on what
an earlier one left in the shared scratch; a third, on fp16 inputs, and the
refusal of a request larger than the scratch complete it.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

FIELDS = ("sigma", "mean", "smax", "flags", "coeffs", "row_limit", "split")


def _outputs(m, dev, fill):
    f32 = dict(dtype=torch.float32, device=dev)
    i32 = dict(dtype=torch.int32, device=dev)
    return {"sigma": torch.full((m,), fill, **f32), "mean": torch.full((m,), fill, **f32),
            "smax": torch.full((m,), fill, **f32), "flags": torch.full((m,), 7, **i32),
            "coeffs": torch.full((m, 3), fill, **f32), "row_limit": torch.full((m,), -5, **i32),
            "split": torch.full((m,), 9, **i32)}


def _call(q, k, idx, outs, workspace=None):
    from techjam_amd.kernels import _lib
    from techjam_amd.kernels.attention import _DTYPES, _stream_ptr

    b, h, s, d = q.shape
    common = (q.data_ptr(), k.data_ptr(), _DTYPES[q.dtype], b, h, s, d, _lib.strides4(q), _lib.strides4(k),
              d ** -0.5, idx.data_ptr(), idx.numel(), 0.40, 4096,
              *(outs[f].data_ptr() for f in FIELDS))
    L = _lib.lib()
    if workspace is None:
        return L.tj_score_guard_noalloc(*common, _stream_ptr(q.device))
    return L.tj_score_guard(*common, workspace.data_ptr(), workspace.numel(), _stream_ptr(q.device))


def _inputs(b, h, s, seed, dev, dtype=torch.float32):
    g = torch.Generator(device=dev).manual_seed(seed)
    std = torch.full((1, h, 1, 1), 0.5, device=dev)
    std[0, 0] = 2.0  # one wide head per sample: flag 0, split 1
    q = (torch.randn(b, h, s, 64, generator=g, device=dev) * std).to(dtype)
    k = (torch.randn(b, h, s, 64, generator=g, device=dev) * std).to(dtype)
    return q, k


@pytest.mark.parametrize("calls", [[(4, 16, 4096, torch.float32), (1, 3, 1000, torch.float32),
                                    (2, 5, 700, torch.float16)]])
def test_noalloc_guard_matches_the_workspace_guard(cuda, calls):
    from techjam_amd.kernels import _lib
    from techjam_amd.kernels.attention import sample_index

    for i, (b, h, s, dtype) in enumerate(calls):
        q, k = _inputs(b, h, s, 100 + i, cuda, dtype)
        idx = sample_index(s, 512, 0, cuda)
        ws = torch.full((_lib.lib().tj_score_guard_workspace_bytes(b, h, idx.numel()),), 0xFF,
                        dtype=torch.uint8, device=cuda)
        want, got = _outputs(b * h, cuda, -1.0), _outputs(b * h, cuda, -2.0)
        assert _call(q, k, idx, want, ws) == _lib.TJ_OK
        assert _call(q, k, idx, got) == _lib.TJ_OK
        torch.cuda.synchronize()
        for f in FIELDS:
            assert torch.equal(want[f], got[f]), f"call {i} ({b}x{h}x{s}): {f} differs"
        flags = got["flags"].view(b, h)
        assert bool((flags[:, 0] == 0).all()) and bool((flags[:, 1:] == 1).all()), f"call {i}: flags {flags}"


def test_noalloc_guard_refuses_more_than_its_scratch(cuda):
    from techjam_amd.kernels import _lib
    from techjam_amd.kernels.attention import sample_index

    b, h, s = 375, 16, 512  # 6000 (b, h) x 8 blocks x 24 bytes > 1 MiB
    q = torch.zeros(1, 1, s, 64, device=cuda).expand(b, h, s, 64)
    idx = sample_index(s, 512, 0, cuda)
    outs = _outputs(b * h, cuda, 0.0)
    assert _call(q, q, idx, outs) == _lib.TJ_ERR_SCRATCH
    assert bool((outs["flags"] == 7).all())  # nothing was launched
