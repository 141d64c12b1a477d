"""Captured forwards replayed as HIP graphs, for launch-bound shapes.

The reference runs its small and medium cases through
``torch.compile(mode="reduce-overhead")`` (``src/dispatcher.py:47-61``,
``:765-790``), i.e. CUDA-graph replay of an Inductor-generated forward. Here
the forward is already a handful of hand-written kernels and library GEMMs,
so it is captured directly: one ``torch.cuda.CUDAGraph`` per input signature,
recorded on static input buffers and replayed after copying each call's
inputs into them. The kernels read their stream from torch, so they record
into the capture stream like any torch op; none of them issues a memset
(workspaces are cleared by a kernel).

A replay writes the same static output buffer every time; each call returns
a fresh copy, so earlier results stay valid. A capture is keyed on the
addresses and versions of every parameter and buffer, so replacing or
modifying weights (``load_state_dict``, ``.to()``, in-place updates) triggers
a new capture instead of replaying stale addresses.
"""

from __future__ import annotations

from typing import Callable, Optional, Tuple

import torch


def weights_signature(module: torch.nn.Module) -> tuple:
    """Addresses and in-place versions of every parameter and buffer."""
    sig = []
    for t in list(module.parameters()) + list(module.buffers()):
        try:
            version = t._version
        except RuntimeError:  # inference tensors carry no version counter
            version = None
        sig.append((t.data_ptr(), version, tuple(t.shape), t.dtype))
    return tuple(sig)


class GraphedForward:
    """``fn(x, mask, lengths)`` captured once on static copies of its inputs."""

    def __init__(self, fn: Callable, x: torch.Tensor, mask: Optional[torch.Tensor],
                 lengths: Optional[torch.Tensor], signature: tuple, warmup: int = 2) -> None:
        self.signature = signature
        self.static_x = x.clone()
        self.static_mask = None if mask is None else mask.clone()
        self.static_lengths = None if lengths is None else lengths.clone()
        dev = x.device
        # Warm-up on a side stream (default priority): first-call library
        # set-up and the caching allocator must not happen during capture.
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(warmup):
                fn(self.static_x, self.static_mask, self.static_lengths)
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.static_out = fn(self.static_x, self.static_mask, self.static_lengths)

    def matches(self, x: torch.Tensor, mask: Optional[torch.Tensor], lengths: Optional[torch.Tensor]) -> bool:
        def same(a, b):
            if a is None or b is None:
                return a is None and b is None
            return a.shape == b.shape and a.dtype == b.dtype and a.device == b.device
        return same(self.static_x, x) and same(self.static_mask, mask) and same(self.static_lengths, lengths)

    def __call__(self, x: torch.Tensor, mask: Optional[torch.Tensor],
                 lengths: Optional[torch.Tensor]) -> torch.Tensor:
        self.static_x.copy_(x)
        if self.static_mask is not None:
            self.static_mask.copy_(mask)
        if self.static_lengths is not None:
            self.static_lengths.copy_(lengths)
        self.graph.replay()
        return self.static_out.clone()


def graph_key(x: torch.Tensor, mask: Optional[torch.Tensor], lengths: Optional[torch.Tensor],
              extra: Tuple = ()) -> tuple:
    """Input signature a capture is valid for."""
    def desc(t):
        return None if t is None else (tuple(t.shape), t.dtype, t.device)
    return (desc(x), desc(mask), desc(lengths)) + tuple(extra)
