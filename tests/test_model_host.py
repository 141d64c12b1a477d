"""Host-side helpers of the encoder model (no GPU): the fp16 weight cache and
the GEMM dispatch on the input's dtype."""

from __future__ import annotations

import torch
import torch.nn.functional as F

from techjam_amd.model import fp16_weight, project


def test_fp16_weight_cache_follows_the_weight():
    lin = torch.nn.Linear(8, 4)
    w16 = fp16_weight(lin, "weight", lin.weight)
    assert w16.dtype == torch.float16 and torch.equal(w16, lin.weight.detach().half())
    assert fp16_weight(lin, "weight", lin.weight) is w16            # cached
    with torch.no_grad():
        lin.weight.mul_(2.0)                                         # in place: new version
    w16b = fp16_weight(lin, "weight", lin.weight)
    assert w16b is not w16 and torch.equal(w16b, lin.weight.detach().half())
    lin.weight = torch.nn.Parameter(torch.ones(4, 8))                # replaced
    assert torch.equal(fp16_weight(lin, "weight", lin.weight), torch.ones(4, 8, dtype=torch.float16))
    assert fp16_weight(lin, "other", lin.bias).shape == (4,)          # keys are separate entries


def test_fp16_weight_of_an_inference_tensor_follows_an_in_place_refill():
    """Weights created under inference mode have no version counter, so an
    in-place refill (same storage) cannot be detected: such weights are
    converted on every call, never served from a stale cache."""
    with torch.inference_mode():
        lin = torch.nn.Linear(8, 4)
        w16 = fp16_weight(lin, "weight", lin.weight)
        assert torch.equal(w16, lin.weight.detach().half())
        lin.weight.data.copy_(torch.full((4, 8), 3.0))          # same data_ptr
        assert torch.equal(fp16_weight(lin, "weight", lin.weight), torch.full((4, 8), 3.0, dtype=torch.float16))
    assert "_fp16_weights" not in lin.__dict__


def test_project_keeps_fp32_inputs_on_the_fp32_gemm():
    lin = torch.nn.Linear(8, 4, bias=False)
    x = torch.randn(2, 3, 8)
    assert torch.equal(project(x, lin.weight, lin, "weight"), F.linear(x, lin.weight))
    assert "_fp16_weights" not in lin.__dict__


def test_project_rounds_operands_for_fp16_inputs():
    lin = torch.nn.Linear(8, 4, bias=False)
    x = torch.randn(2, 3, 8)
    y = project(x.half(), lin.weight, lin, "weight")
    assert y.dtype == torch.float16 and y.shape == (2, 3, 4)
    ref = x.half().double() @ lin.weight.detach().half().double().t()
    assert torch.allclose(y.double(), ref, atol=2e-3, rtol=2e-3)


def test_weights_signature_tracks_in_place_edits_and_replacement():
    from techjam_amd.graphs import weights_signature

    net = torch.nn.Sequential(torch.nn.Linear(4, 4), torch.nn.LayerNorm(4))
    net.register_buffer("cache", torch.zeros(3))
    sig = weights_signature(net)
    assert weights_signature(net) == sig
    with torch.no_grad():
        net[0].weight.add_(1.0)
    edited = weights_signature(net)
    assert edited != sig
    net[1].bias = torch.nn.Parameter(torch.ones(4))
    assert weights_signature(net) != edited
    net.cache = torch.ones(3)                       # a replaced buffer counts too
    assert len(weights_signature(net)) == len(sig)


def test_graph_key_separates_shapes_dtypes_and_flags():
    from techjam_amd.graphs import graph_key

    x = torch.zeros(2, 8, 4)
    m = torch.ones(2, 8, dtype=torch.bool)
    lens = torch.full((2,), 8, dtype=torch.int32)
    base = graph_key(x, m, lens, ("fp32",))
    assert base == graph_key(x.clone(), m.clone(), lens.clone(), ("fp32",))
    assert base != graph_key(x, None, None, ("fp32",))
    assert base != graph_key(x.half(), m, lens, ("fp32",))
    assert base != graph_key(torch.zeros(2, 9, 4), m, lens, ("fp32",))
    assert base != graph_key(x, m, lens, ("fp16",))
