"""Parity of the HIP polynomial-attention path with the oracle (GPU).

Three levels:

* the fused chunk kernels against the oracle's chunked scan
  (``oracle.poly.poly_linear_attention`` in fp32) -- same algorithm, so any
  indexing or state bug shows as an O(output) error while fp16 operand
  rounding stays near 1e-3 relative;
* the guarded route (device guard + polynomial + exact fallback with split
  scores) against exact softmax attention, the way the reference validates
  its polynomial route (``src/validate_poly.py``);
* the extreme-length workload (B=4, S=65536, H=16, D=64; q,k ~ N(0, 0.5^2),
  head 0 of every sample ~ N(0, 2^2)) against the linear-memory FP32 oracle,
  with the benchmark's OR rule and zero failing elements.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.attention import blockwise_attention
from oracle.poly import coefficient_table, hermite_coefficients, poly_linear_attention

pytestmark = pytest.mark.gpu


def _draw(b, h, n, d=64, std=0.577, seed=0, vstd=None):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, h, n, d, generator=g) * std
    k = torch.randn(b, h, n, d, generator=g) * std
    v = torch.randn(b, h, n, d, generator=g) * (std if vstd is None else vstd)
    return q, k, v


def _or_failures(got, ref, atol=2e-3, rtol=0.02):
    err = (got.double() - ref.double()).abs()
    ok = torch.isfinite(got) & ((err <= atol) | (err <= rtol * ref.double().abs()))
    return int((~ok).sum()), float(err.max())


def _rel_rms(got, ref):
    return float((got.double() - ref.double()).pow(2).mean().sqrt() / ref.double().pow(2).mean().sqrt())


# The kernel keeps a 32-slot ring of fp16 state shadows (state c in slot
# c % 32, sixteen chunks per launch): 16461 tokens (33 chunks, ragged tail of
# 77) and 24876 tokens (49 chunks, ragged tail of 300) reuse slots, the second
# one every slot at least once, and both cross launch boundaries mid-ring;
# 10240 tokens (20 chunks) crosses one launch boundary.
@pytest.mark.parametrize("n,prefix", [(2048, 512), (2000, 700), (1536, 0), (300, 0), (4096, 4000),
                                      (10240, 4096), (16384 + 77, 0), (24576 + 300, 1000)])
def test_fused_scan_matches_oracle_scan(cuda, n, prefix):
    from techjam_amd.kernels.poly import poly_rows

    b, h = 1, 3
    q, k, v = _draw(b, h, n)
    scale = 64 ** -0.5
    sig = torch.tensor([[0.334, 0.25, 0.2]])
    coeffs = coefficient_table(sig)
    ref = poly_linear_attention(q, k, v, scale, chunk=512, exact_prefix=prefix, coeffs=coeffs,
                                skip_final_state_update=True)
    out = torch.full((b, h, n, 64), 777.0, device=cuda)
    poly_rows(q.to(cuda), k.to(cuda), v.to(cuda), scale, coeffs.float().reshape(-1, 3).to(cuda),
              chunk=512, exact_prefix=prefix, out=out)
    torch.cuda.synchronize()
    got = out.cpu()
    if prefix:
        assert bool((got[:, :, :prefix] == 777.0).all()), "rows inside the exact prefix were written"
    tail = slice(prefix, n)
    rel = _rel_rms(got[:, :, tail], ref[:, :, tail])
    bad, mx = _or_failures(got[:, :, tail], ref[:, :, tail])
    print(f"n={n} prefix={prefix}: rel_rms={rel:.2e} max_abs={mx:.2e} failed={bad}")
    assert rel < 5e-3 and bad == 0


def _scan_cases(n_cases, seed):
    """Random shapes for the fused scan: lengths from one token to 24 chunks,
    exact prefixes anywhere (also inside a chunk), fp32 and fp16 inputs."""
    import random

    rng = random.Random(seed)
    cases = []
    for i in range(n_cases):
        n = rng.choice([rng.randint(1, 600), rng.randint(500, 5000), rng.randint(4000, 12000)])
        cases.append(dict(seed=seed + i, b=rng.randint(1, 2), h=rng.randint(1, 3), n=n,
                          prefix=rng.choice([0, 0, rng.randint(0, n - 1)]), f16=rng.random() < 0.3))
    return cases


@pytest.mark.parametrize("case", _scan_cases(16, 31), ids=lambda c: "b{b}h{h}n{n}p{prefix}{}".format("h" if c["f16"] else "", **c))
def test_fused_scan_random_shapes(cuda, case):
    from techjam_amd.kernels.poly import poly_rows

    b, h, n, prefix = case["b"], case["h"], case["n"], case["prefix"]
    g = torch.Generator().manual_seed(case["seed"])
    q, k, v = (torch.randn(b, h, n, 64, generator=g) * 0.577 for _ in range(3))
    dt = torch.float16 if case["f16"] else torch.float32
    q, k, v = (t.to(dt).float() for t in (q, k, v))
    coeffs = coefficient_table(torch.rand(b, h, generator=g) * 0.3 + 0.1)
    ref = poly_linear_attention(q, k, v, 64 ** -0.5, chunk=512, exact_prefix=prefix, coeffs=coeffs,
                                skip_final_state_update=True)
    out = torch.full((b, h, n, 64), 777.0, device=cuda, dtype=dt)
    poly_rows(q.to(cuda, dt), k.to(cuda, dt), v.to(cuda, dt), 64 ** -0.5, coeffs.float().reshape(-1, 3).to(cuda),
              chunk=512, exact_prefix=prefix, out=out)
    torch.cuda.synchronize()
    got = out.float().cpu()
    if prefix:
        assert bool((got[:, :, :prefix] == 777.0).all()), "rows inside the exact prefix were written"
    tail = slice(prefix, n)
    bad, mx = _or_failures(got[:, :, tail], ref[:, :, tail])
    rel = _rel_rms(got[:, :, tail], ref[:, :, tail])
    assert bad == 0 and rel < 5e-3, f"{case}: rel_rms={rel:.2e} max_abs={mx:.2e} failed={bad}"


def test_rows_past_the_sequence_end_read_as_zeros(cuda):
    """Token tiles of 64 reach past S = 1000 + 37: K and V views whose memory
    continues with NaN after row S - 1 must give the same output as compact
    tensors (the kernel's bounds-checked loads read those rows as zeros)."""
    from techjam_amd.kernels.poly import poly_rows

    b, h, n, pad = 1, 2, 1037, 64
    q, k, v = _draw(b, h, n, seed=9)
    scale = 64 ** -0.5
    coeffs = coefficient_table(torch.tensor([[0.334, 0.25]])).float().reshape(-1, 3).to(cuda)
    views = []
    for t in (k, v):
        full = torch.full((b, h, n + pad, 64), float("nan"), device=cuda)
        full[:, :, :n] = t.to(cuda)
        views.append(full[:, :, :n])
    got = poly_rows(q.to(cuda), *views, scale, coeffs, chunk=512, exact_prefix=0)
    want = poly_rows(q.to(cuda), k.to(cuda), v.to(cuda), scale, coeffs, chunk=512, exact_prefix=0)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(got).all())
    assert torch.equal(got, want)


def test_flags_skip_heads_and_coefficients_are_per_head(cuda):
    from techjam_amd.kernels.poly import poly_rows

    b, h, n = 2, 2, 1024
    q, k, v = _draw(b, h, n, seed=1)
    scale = 64 ** -0.5
    coeffs = coefficient_table(torch.tensor([[0.3, 0.1], [0.2, 0.35]])).float()
    flags = torch.tensor([1, 0, 0, 1], dtype=torch.int32)
    out = torch.full((b, h, n, 64), 5.0, device=cuda)
    poly_rows(q.to(cuda), k.to(cuda), v.to(cuda), scale, coeffs.reshape(-1, 3).to(cuda),
              flags=flags.to(cuda), chunk=512, exact_prefix=0, out=out)
    torch.cuda.synchronize()
    got = out.cpu()
    ref = poly_linear_attention(q, k, v, scale, chunk=512, exact_prefix=0, coeffs=coeffs.double())
    for bh, on in enumerate(flags.tolist()):
        bi, hi = divmod(bh, h)
        if on:
            assert _rel_rms(got[bi, hi], ref[bi, hi]) < 5e-3
        else:
            assert bool((got[bi, hi] == 5.0).all())


def test_fp16_inputs(cuda):
    from techjam_amd.kernels.poly import poly_rows

    q, k, v = (t.half() for t in _draw(1, 2, 1536, seed=2))
    scale = 64 ** -0.5
    c = torch.tensor(hermite_coefficients(0.334), dtype=torch.float32).repeat(2, 1)
    out = poly_rows(q.to(cuda), k.to(cuda), v.to(cuda), scale, c.to(cuda), chunk=512, exact_prefix=0)
    torch.cuda.synchronize()
    ref = poly_linear_attention(q.float(), k.float(), v.float(), scale, chunk=512, exact_prefix=0, sigma=0.334)
    assert out.dtype == torch.float16
    assert _rel_rms(out.float().cpu(), ref) < 5e-3


def test_deterministic(cuda):
    from techjam_amd.kernels.poly import poly_rows

    q, k, v = (t.to(cuda) for t in _draw(1, 2, 2048, seed=3))
    c = torch.tensor(hermite_coefficients(0.334), dtype=torch.float32, device=cuda).repeat(2, 1)
    a1 = poly_rows(q, k, v, 0.125, c, exact_prefix=512)
    a2 = poly_rows(q, k, v, 0.125, c, exact_prefix=512)
    torch.cuda.synchronize()
    assert torch.equal(a1[:, :, 512:], a2[:, :, 512:])


@pytest.mark.parametrize("n,prefix", [(2048, 512), (1536, 0), (300, 0), (9000, 4096)])
def test_result_does_not_depend_on_workspace_contents(cuda, n, prefix):
    """The call clears only what must start at zero (masters, shadow slot 0);
    a workspace full of 0xFF bytes (NaN in every float) must give the same
    bits as a fresh one."""
    from techjam_amd.kernels import _lib
    from techjam_amd.kernels.attention import _DTYPES, _stream_ptr, empty_like_heads
    from techjam_amd.kernels.poly import poly_rows, workspace_bytes

    q, k, v = (t.to(cuda).contiguous() for t in _draw(1, 2, n, seed=11))
    c = torch.tensor(hermite_coefficients(0.334), dtype=torch.float32, device=cuda).repeat(2, 1)
    ref = poly_rows(q, k, v, 0.125, c, exact_prefix=prefix)
    nbytes = workspace_bytes(1, 2, n, 64, 512)
    ws = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device=cuda)
    for _ in range(2):  # the second call sees the first call's leftovers
        out = empty_like_heads(q)
        code = _lib.lib().tj_poly_attn_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), _DTYPES[q.dtype], 1, 2, n, 64,
            _lib.strides4(q), _lib.strides4(k), _lib.strides4(v), _lib.strides4(out),
            0.125, 512, prefix, c.data_ptr(), None, ws.data_ptr(), nbytes, _stream_ptr(cuda))
        _lib.check(code, "tj_poly_attn_fwd")
        torch.cuda.synchronize()
        assert torch.equal(out[:, :, prefix:], ref[:, :, prefix:])


def test_poly_attention_forward_matches_oracle_including_prefix(cuda):
    from techjam_amd.implementations.poly_attention import poly_attention_forward

    q, k, v = _draw(1, 2, 6144, seed=4)
    scale = 64 ** -0.5
    got = poly_attention_forward(q.to(cuda), k.to(cuda), v.to(cuda), scale, sigma=0.334).cpu()
    ref = poly_linear_attention(q, k, v, scale, chunk=512, exact_prefix=4096, sigma=0.334)
    bad, mx = _or_failures(got, ref)
    assert bad == 0 and _rel_rms(got, ref) < 5e-3


def test_guarded_route_against_exact_attention(cuda):
    """q, k ~ N(0, 0.5^2) except head 0 ~ N(0, 2^2): 3 heads polynomial, head 0 exact."""
    from techjam_amd.implementations.poly_attention import guarded_attention

    b, h, n, d = 1, 4, 8192, 64
    g = torch.Generator().manual_seed(5)
    std = torch.tensor([2.0, 0.5, 0.5, 0.5]).view(1, h, 1, 1)
    q = (torch.randn(b, h, n, d, generator=g) * std).to(cuda)
    k = (torch.randn(b, h, n, d, generator=g) * std).to(cuda)
    v = torch.randn(b, h, n, d, generator=g).to(cuda)
    out, gr = guarded_attention(q, k, v, d ** -0.5)
    ref = blockwise_attention(q, k, v, d ** -0.5, True, block_q=2048, block_k=2048)
    torch.cuda.synchronize()
    assert gr.flags.cpu().tolist() == [0, 1, 1, 1]
    bad, mx = _or_failures(out.cpu(), ref.cpu())
    print(f"guarded S=8192: max_abs={mx:.2e} failed={bad}")
    assert bad == 0


@pytest.mark.slow
@pytest.mark.parametrize("seed", range(1234, 1239))
def test_extreme_length_workload_against_linear_memory_oracle(cuda, seed):
    """B=4, S=65536, H=16, D=64, fp32 io: zero failing elements, peak HBM < 8 GiB,
    on the harness's five accuracy seeds (1234+i; the seed drives the q/k/v draw)."""
    from techjam_amd.implementations.poly_attention import guarded_attention

    b, s, h, d = 4, 65536, 16, 64
    torch.cuda.empty_cache()
    g = torch.Generator(device=cuda).manual_seed(seed)
    q = torch.randn(b, s, h, d, generator=g, device=cuda) * 0.5
    k = torch.randn(b, s, h, d, generator=g, device=cuda) * 0.5
    v = torch.randn(b, s, h, d, generator=g, device=cuda)
    q[:, :, 0] = torch.randn(b, s, d, generator=g, device=cuda) * 2.0
    k[:, :, 0] = torch.randn(b, s, d, generator=g, device=cuda) * 2.0
    qh, kh, vh = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    out, gr = guarded_attention(qh, kh, vh, d ** -0.5)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - base + 3 * q.numel() * 4
    assert int(gr.flags.sum()) == 60 and not bool(gr.flags.view(b, h)[:, 0].any())
    assert peak < 8 * 2**30, f"peak {peak / 2**30:.2f} GiB"
    failed, mx = 0, 0.0
    for bi in range(b):  # the oracle per sample keeps its score tiles bounded
        ref = blockwise_attention(qh[bi:bi + 1], kh[bi:bi + 1], vh[bi:bi + 1], d ** -0.5, True,
                                  block_q=4096, block_k=4096)
        nb, m = _or_failures(out[bi:bi + 1], ref)
        failed += nb
        mx = max(mx, m)
        del ref
    print(f"extreme length, seed {seed}: peak={peak / 2**30:.2f} GiB max_abs={mx:.3e} failed={failed}")
    assert failed == 0


def _guard_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        b, h = int(rng.integers(1, 4)), int(rng.integers(1, 6))
        s = int(rng.choice([4097, 4608, 5000, 6144, 8192 + 77, 10240, 12288 + 5]))
        # per-head input std: score sigma = std^2 (D = 64), so 0.3 and 0.5
        # take the polynomial route, 1.0 and 2.0 the exact fallback
        stds = [float(x) for x in rng.choice([0.3, 0.5, 1.0, 2.0], size=h)]
        cases.append(dict(b=b, h=h, s=s, stds=stds, layout=str(rng.choice(["bhsd", "bshd", "packed"])),
                          f16=bool(rng.random() < 0.3), seed=500 + i))
    return cases


@pytest.mark.parametrize("case", _guard_cases(12, 7), ids=lambda c: "{seed}-b{b}h{h}s{s}-{layout}{}".format(
    "-f16" if c["f16"] else "", **c))
def test_guarded_route_random_configurations(cuda, case):
    """Seeded shapes past the exact prefix (ragged tails included), mixed
    per-head score ranges, three memory layouts and both input types, against
    exact attention in fp32 on the GPU: the guard's routing and zero OR-rule
    failures over every element."""
    from techjam_amd.implementations.poly_attention import guarded_attention

    b, h, s, d = case["b"], case["h"], case["s"], 64
    dt = torch.float16 if case["f16"] else torch.float32
    g = torch.Generator(device=cuda).manual_seed(case["seed"])
    std = torch.tensor(case["stds"], device=cuda).view(1, h, 1, 1)
    if case["layout"] == "packed":
        qkv = torch.randn(b, s, 3, h, d, generator=g, device=cuda)
        q, k, v = (qkv[:, :, j].transpose(1, 2) for j in range(3))
    elif case["layout"] == "bshd":
        q, k, v = (torch.randn(b, s, h, d, generator=g, device=cuda).transpose(1, 2) for _ in range(3))
    else:
        q, k, v = (torch.randn(b, h, s, d, generator=g, device=cuda) for _ in range(3))
    q, k = (q * std).to(dt), (k * std).to(dt)
    v = v.to(dt)
    out, gr = guarded_attention(q, k, v, d ** -0.5)
    prev = torch.get_float32_matmul_precision()
    torch.set_float32_matmul_precision("highest")
    try:
        ref = blockwise_attention(q.float(), k.float(), v.float(), d ** -0.5, True, block_q=2048, block_k=2048)
    finally:
        torch.set_float32_matmul_precision(prev)
    torch.cuda.synchronize()
    want_flags = [int(x <= 0.5) for x in case["stds"]] * b
    assert gr.flags.cpu().tolist() == want_flags
    bad, mx = _or_failures(out.float(), ref)
    print(f"{case}: max_abs={mx:.2e} failed={bad}")
    assert bad == 0
