"""Parity of the HIP exact-attention kernel with the oracle (GPU).

The oracle is ``oracle.attention``: float64 brute force for small shapes and
the blockwise online softmax in float64 on the CPU for larger ones. Inputs are
drawn on the CPU from seeded generators and copied to the GPU. The bar is the
benchmark's per-element rule ``|d| <= 2e-3 OR |d| <= 0.02*|ref|`` with zero
failures (``torch_transformer_benchmark.py:309-319``); fp16 operands with fp32
accumulation sit far inside it, so the tests also bound the max abs error.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.attention import blockwise_attention, brute_force_attention

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 0.02


def _draw(shape, seed, scale=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g, dtype=torch.float64) * scale).to(dtype)


def _assert_close(got: torch.Tensor, ref, max_abs=None, what=""):
    got = got.detach().double().cpu().numpy()
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref)
    ok = np.isfinite(got) & ((err <= ATOL) | (err <= RTOL * np.abs(ref)))
    n_bad = int((~ok).sum())
    assert n_bad == 0, f"{what}: {n_bad} failing elements, max abs err {err.max():.3e}"
    if max_abs is not None:
        assert err.max() <= max_abs, f"{what}: max abs err {err.max():.3e} > {max_abs}"


def _run(q, k, v, dev, **kw):
    from techjam_amd.kernels import scaled_dot_product_attention

    out = scaled_dot_product_attention(q.to(dev), k.to(dev), v.to(dev), **kw)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("d", [32, 64, 128, 256])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("s", [1, 7, 64, 100, 129, 300])
def test_matches_brute_force(cuda, s, causal, d):
    b, h = 2, 3
    q, k, v = (_draw((b, h, s, d), seed) for seed in (1, 2, 3))
    ref = brute_force_attention(q, k, v, d ** -0.5, causal)
    got = _run(q, k, v, cuda, is_causal=causal)
    _assert_close(got, ref, max_abs=4e-3, what=f"s={s} d={d} causal={causal}")


@pytest.mark.parametrize("d", [8, 16, 40, 100, 160])
@pytest.mark.parametrize("causal", [True, False])
def test_head_dims_served_by_zero_padding(cuda, causal, d):
    b, h, s = 2, 3, 200
    q, k, v = (_draw((b, h, s, d), seed) for seed in (4, 5, 6))
    ref = brute_force_attention(q, k, v, d ** -0.5, causal)
    got = _run(q, k, v, cuda, is_causal=causal)
    assert got.shape == (b, h, s, d)
    _assert_close(got, ref, max_abs=4e-3, what=f"d={d} causal={causal}")
    lens = torch.tensor([200, 77], dtype=torch.int32)
    got = _run(q, k, v, cuda, is_causal=causal, valid_len=lens.to(cuda))
    for i, n in enumerate(lens.tolist()):
        ref_i = brute_force_attention(q[i:i + 1, :, :n], k[i:i + 1, :, :n], v[i:i + 1, :, :n], d ** -0.5, causal)
        _assert_close(got[i:i + 1, :, :n], ref_i, max_abs=4e-3, what=f"d={d} sample {i}")
        assert float(got[i, :, n:].abs().max().cpu()) == 0.0 if n < s else True


@pytest.mark.parametrize("causal", [True, False])
def test_right_padding_valid_lengths(cuda, causal):
    b, h, s, d = 4, 2, 200, 64
    q, k, v = (_draw((b, h, s, d), seed) for seed in (4, 5, 6))
    lengths = [200, 77, 1, 0]
    ref = brute_force_attention(q, k, v, d ** -0.5, causal, valid_len=lengths)
    vl = torch.tensor(lengths, dtype=torch.int32, device=cuda)
    got = _run(q, k, v, cuda, is_causal=causal, valid_len=vl)
    _assert_close(got, ref, max_abs=4e-3, what=f"valid_len causal={causal}")
    # padded rows are exact zeros
    for bi, n in enumerate(lengths):
        assert torch.count_nonzero(got[bi, :, n:]).item() == 0


@pytest.mark.parametrize("causal", [True, False])
def test_projection_biases_folded_into_the_kernel(cuda, causal):
    """q_bias / v_bias on bias-free projections equal attention of the biased
    tensors; the key bias, which the kernel never sees, shifts whole score rows
    and drops out of the softmax. Padded rows stay exact zeros."""
    from techjam_amd.kernels import scaled_dot_product_attention

    b, h, s, d = 3, 4, 300, 64
    q, k, v = (_draw((b, h, s, d), seed) for seed in (31, 32, 33))
    bq, bk, bv = (_draw((h, d), seed, scale=0.5) for seed in (34, 35, 36))
    lengths = [300, 123, 0]
    ref = brute_force_attention(q + bq[None, :, None], k + bk[None, :, None], v + bv[None, :, None],
                                d ** -0.5, causal, valid_len=lengths)
    vl = torch.tensor(lengths, dtype=torch.int32, device=cuda)
    got = scaled_dot_product_attention(q.to(cuda), k.to(cuda), v.to(cuda), is_causal=causal, valid_len=vl,
                                       q_bias=bq.reshape(-1).to(cuda), v_bias=bv.reshape(-1).to(cuda))
    torch.cuda.synchronize()
    _assert_close(got, ref, max_abs=4e-3, what=f"folded biases causal={causal}")
    for bi, n in enumerate(lengths):
        assert torch.count_nonzero(got[bi, :, n:]).item() == 0
    with pytest.raises(ValueError):
        scaled_dot_product_attention(q.to(cuda), k.to(cuda), v.to(cuda), q_bias=bq.reshape(-1).to(cuda),
                                     row_limit=torch.zeros(b * h, dtype=torch.int32, device=cuda))


def test_row_limit_leaves_other_rows_untouched(cuda):
    from techjam_amd.kernels import scaled_dot_product_attention

    b, h, s, d = 2, 3, 300, 64
    q, k, v = (_draw((b, h, s, d), seed) for seed in (7, 8, 9))
    limits = torch.tensor([0, 1, 128, 129, 300, 1000], dtype=torch.int32)
    out = torch.full((b, h, s, d), 12345.0, device=cuda)
    scaled_dot_product_attention(q.to(cuda), k.to(cuda), v.to(cuda), is_causal=True,
                                 row_limit=limits.to(cuda), out=out)
    torch.cuda.synchronize()
    ref = brute_force_attention(q, k, v, d ** -0.5, True)
    got = out.cpu()
    for bh in range(b * h):
        bi, hi = divmod(bh, h)
        n = min(int(limits[bh]), s)
        _assert_close(got[bi, hi, :n], ref[bi, hi, :n], what=f"head {bh}")
        assert bool((got[bi, hi, n:] == 12345.0).all()), f"head {bh} rows >= {n} were written"


# Launches with row limits take the balanced tile order: (b, h) spread over
# the XCDs by their index digits, four ranks of a (b, h) per XCD, when B*H is
# a multiple of 8, and a plain rotation otherwise. (B, H, S): 128-row tiles
# below 1024 wide tiles, 256-row tiles at B=4 H=16 S=4096.
_ROW_LIMIT_ORDER_CASES = [(1, 8, 4096), (3, 8, 2048), (4, 16, 4096), (3, 4, 1500)]


@pytest.mark.parametrize("b,h,s", _ROW_LIMIT_ORDER_CASES, ids=lambda x: str(x))
def test_row_limited_tile_order_issues_every_query_tile(cuda, b, h, s):
    """NaN-prefilled output, a mix of per-head row limits (0, a 4096-row
    prefix, S, and odd values): every row below its head's limit against the
    blockwise oracle, every row at or past it still NaN."""
    from techjam_amd.kernels import scaled_dot_product_attention

    d = 64
    g = torch.Generator(device=cuda).manual_seed(5150)
    q, k, v = (torch.randn(b, s, h, d, generator=g, device=cuda).transpose(1, 2) for _ in range(3))
    choices = [s, min(s, 4096), 0, s - 1, (s // 3) | 1, 257]
    limits = torch.tensor([choices[i % len(choices)] for i in range(b * h)], dtype=torch.int32, device=cuda)
    out = torch.full((b, s, h, d), float("nan"), device=cuda).transpose(1, 2)
    scaled_dot_product_attention(q, k, v, is_causal=True, row_limit=limits, out=out)
    torch.cuda.synchronize()
    prev = torch.get_float32_matmul_precision()
    torch.set_float32_matmul_precision("highest")
    try:
        ref = blockwise_attention(q, k, v, d ** -0.5, True, block_q=1024, block_k=1024)
    finally:
        torch.set_float32_matmul_precision(prev)
    bad = 0
    for bh, n in enumerate(limits.tolist()):
        bi, hi = divmod(bh, h)
        got, want = out[bi, hi, :n], ref[bi, hi, :n]
        err = (got - want).abs()
        ok = torch.isfinite(got) & ((err <= ATOL) | (err <= RTOL * want.abs()))
        bad += int((~ok).sum())
        assert bool(torch.isnan(out[bi, hi, n:]).all()), f"head {bh}: rows >= {n} were written"
    assert bad == 0, f"{bad} failing elements"


def test_packed_qkv_strided_views(cuda):
    """q, k, v as views of one [B, S, 3, H, D] projection; output into [B, S, H, D]."""
    b, s, h, d = 2, 333, 4, 64
    packed = _draw((b, s, 3, h, d), 10)
    q, k, v = (packed[:, :, i].transpose(1, 2) for i in range(3))
    ref = brute_force_attention(q, k, v, d ** -0.5, True)
    from techjam_amd.kernels import scaled_dot_product_attention

    pk = packed.to(cuda)
    qg, kg, vg = (pk[:, :, i].transpose(1, 2) for i in range(3))
    assert qg.stride() == (s * 3 * h * d, d, 3 * h * d, 1)
    got = scaled_dot_product_attention(qg, kg, vg, is_causal=True)
    torch.cuda.synchronize()
    assert got.transpose(1, 2).is_contiguous()  # [B, S, H, D] storage, free reshape
    _assert_close(got, ref, max_abs=4e-3, what="packed views")


def test_float16_inputs(cuda):
    b, h, s, d = 2, 2, 257, 64
    q, k, v = (_draw((b, h, s, d), seed).half() for seed in (11, 12, 13))
    ref = brute_force_attention(q.double(), k.double(), v.double(), d ** -0.5, True)
    got = _run(q, k, v, cuda, is_causal=True)
    assert got.dtype == torch.float16
    _assert_close(got.float(), ref, max_abs=4e-3, what="fp16")


@pytest.mark.parametrize("scale_in", [0.1, 1.0])
def test_small_score_ranges_on_plain_fp16_scores(cuda, scale_in):
    """Score sigma 0.01 and 1: fp16 q/k operands are accurate enough."""
    b, h, s, d = 1, 2, 256, 64
    q, k = (_draw((b, h, s, d), seed, scale_in) for seed in (14, 15))
    v = _draw((b, h, s, d), 16)
    ref = brute_force_attention(q, k, v, d ** -0.5, True)
    got = _run(q, k, v, cuda, is_causal=True)
    _assert_close(got, ref, max_abs=2e-3, what=f"input scale {scale_in}")


@pytest.mark.parametrize("scale_in", [2.0, 6.0])
def test_wide_score_ranges_on_split_scores(cuda, scale_in):
    """Score sigma 4 and 36 (peaked softmax, max subtraction matters).

    Rounding q and k to fp16 perturbs scores by ~1e-3 at sigma 4, which the
    peaked softmax passes to the output; the split (hi + lo) score path
    restores fp32-level scores.
    """
    b, h, s, d = 2, 2, 256, 64
    q, k = (_draw((b, h, s, d), seed, scale_in) for seed in (14, 15))
    v = _draw((b, h, s, d), 16)
    ref = brute_force_attention(q, k, v, d ** -0.5, True)
    got = _run(q, k, v, cuda, is_causal=True, qk_split=True)
    _assert_close(got, ref, max_abs=2.5e-3, what=f"input scale {scale_in}")


def test_split_scores_per_head(cuda):
    """Only flagged heads take the split path; the others are unchanged bitwise."""
    from techjam_amd.kernels import scaled_dot_product_attention

    b, h, s, d = 1, 4, 300, 64
    q, k, v = (_draw((b, h, s, d), seed, 2.0).to(cuda) for seed in (23, 24, 25))
    flags = torch.tensor([0, 1, 0, 1], dtype=torch.int32, device=cuda)
    plain = scaled_dot_product_attention(q, k, v, is_causal=True)
    mixed = scaled_dot_product_attention(q, k, v, is_causal=True, qk_split=flags)
    split = scaled_dot_product_attention(q, k, v, is_causal=True, qk_split=True)
    torch.cuda.synchronize()
    assert torch.equal(mixed[:, 0], plain[:, 0]) and torch.equal(mixed[:, 2], plain[:, 2])
    assert torch.equal(mixed[:, 1], split[:, 1]) and torch.equal(mixed[:, 3], split[:, 3])
    ref = brute_force_attention(q.cpu(), k.cpu(), v.cpu(), d ** -0.5, True)
    _assert_close(split, ref, max_abs=2.5e-3, what="split all heads")


def test_long_sequence_against_blockwise_oracle(cuda):
    b, h, s, d = 1, 2, 4096, 64
    q, k, v = (_draw((b, h, s, d), seed) for seed in (17, 18, 19))
    ref = blockwise_attention(q.double(), k.double(), v.double(), d ** -0.5, True, acc_dtype=torch.float64)
    got = _run(q, k, v, cuda, is_causal=True)
    _assert_close(got, ref.numpy(), max_abs=4e-3, what="S=4096")


def test_deterministic_and_strictly_causal(cuda):
    from techjam_amd.kernels import scaled_dot_product_attention

    b, h, s, d = 1, 2, 512, 64
    q, k, v = (_draw((b, h, s, d), seed).to(cuda) for seed in (20, 21, 22))
    a1 = scaled_dot_product_attention(q, k, v, is_causal=True)
    a2 = scaled_dot_product_attention(q, k, v, is_causal=True)
    k2, v2 = k.clone(), v.clone()
    k2[:, :, 300:] *= 7.0
    v2[:, :, 300:] *= 7.0
    a3 = scaled_dot_product_attention(q, k2, v2, is_causal=True)
    torch.cuda.synchronize()
    assert torch.equal(a1, a2)
    assert torch.equal(a1[:, :, :300], a3[:, :, :300])
    assert not torch.equal(a1[:, :, 300:], a3[:, :, 300:])


@pytest.mark.parametrize("seed", [1234, 1235, 1236, 101234])
def test_full_benchmark_shape_every_head(cuda, seed):
    """B=64, S=4096, H=16, D=64 causal (the attention-core workload), every
    one of the 1024 (b, h) heads and every element checked, on the harness's
    accuracy seeds 1234+i and its timing seed 101234 (src/benchmark.py:80,
    :185-192, :379).

    ``out`` starts as NaN, so a query tile the XCD-aware tile order never
    issues (or a row it never writes) fails the finiteness half of the rule.
    The oracle is the blockwise online softmax in fp32 on the GPU under
    matmul precision "highest" (fp32 products and sums, ~1e-6 from fp64),
    eight samples at a time.
    """
    from techjam_amd.kernels import scaled_dot_product_attention

    b, s, h, d = 64, 4096, 16, 64
    g = torch.Generator(device=cuda).manual_seed(seed)
    q, k, v = (torch.randn(b, s, h, d, generator=g, device=cuda).transpose(1, 2) for _ in range(3))
    out = torch.full((b, s, h, d), float("nan"), device=cuda).transpose(1, 2)
    scaled_dot_product_attention(q, k, v, is_causal=True, out=out)
    torch.cuda.synchronize()
    prev = torch.get_float32_matmul_precision()
    torch.set_float32_matmul_precision("highest")
    try:
        failed, max_abs = 0, 0.0
        for b0 in range(0, b, 8):
            sl = slice(b0, b0 + 8)
            ref = blockwise_attention(q[sl], k[sl], v[sl], d ** -0.5, True, block_q=1024, block_k=1024)
            got = out[sl]
            err = (got - ref).abs()
            ok = torch.isfinite(got) & ((err <= ATOL) | (err <= RTOL * ref.abs()))
            failed += int((~ok).sum())
            max_abs = max(max_abs, float(torch.nan_to_num(err, nan=float("inf")).max()))
            del ref, err, ok
    finally:
        torch.set_float32_matmul_precision(prev)
    print(f"attention core, seed {seed}, all 1024 heads: failed={failed} max_abs={max_abs:.3e}")
    assert failed == 0 and max_abs <= 4e-3


# One shape per branch of the kernel's tile order (B, H, S, valid lengths):
# query tiles per (b, h) = S / 256 when B*H*S/256 >= 1024, else S / 128; a
# group holds max(1, 64 / tiles) (b, h); an XCD owns B*H/8 of them, walks all
# but the last group one (b, h) at a time when it owns more than two groups,
# and deals each list in snake rounds of four when the tile count allows.
_ORDER_CASES = {
    "per-head-snake-then-group-of-4": (5, 16, 4096, None),   # 16 tiles, 10 (b, h) per XCD
    "groups-of-2": (2, 16, 8192, None),                       # 32 tiles, 4 (b, h) per XCD
    "groups-of-2-ragged": (2, 16, 8192, [8192, 5000]),
    "groups-of-1": (1, 16, 16384, None),                      # 64 tiles, 2 (b, h) per XCD
    "full-and-partial-group": (3, 8, 4096, None),             # 128-row tiles: 32, 3 (b, h) per XCD
    "tile-count-not-multiple-of-4": (4, 8, 2900, None),       # 128-row tiles: 23
}


@pytest.mark.parametrize("name", list(_ORDER_CASES))
def test_every_tile_order_issues_every_query_tile(cuda, name):
    """``out`` starts as NaN: a query tile that a branch of the XCD /
    shader-engine tile order skipped or issued twice with another's rows
    would leave NaN or wrong rows. Every element against the blockwise
    oracle (fp32 on the GPU, matmul precision "highest")."""
    from techjam_amd.kernels import scaled_dot_product_attention

    b, h, s, lengths = _ORDER_CASES[name]
    d = 64
    g = torch.Generator(device=cuda).manual_seed(4242)
    q, k, v = (torch.randn(b, s, h, d, generator=g, device=cuda).transpose(1, 2) for _ in range(3))
    vl = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=cuda)
    out = torch.full((b, s, h, d), float("nan"), device=cuda).transpose(1, 2)
    scaled_dot_product_attention(q, k, v, is_causal=True, valid_len=vl, out=out)
    torch.cuda.synchronize()
    prev = torch.get_float32_matmul_precision()
    torch.set_float32_matmul_precision("highest")
    try:
        ref = blockwise_attention(q, k, v, d ** -0.5, True, valid_len=vl, block_q=1024, block_k=1024)
    finally:
        torch.set_float32_matmul_precision(prev)
    err = (out - ref).abs()
    ok = torch.isfinite(out) & ((err <= ATOL) | (err <= RTOL * ref.abs()))
    bad = int((~ok).sum())
    print(f"{name}: B={b} H={h} S={s}: failed={bad} max_abs={float(torch.nan_to_num(err, nan=float('inf')).max()):.3e}")
    assert bad == 0
    if lengths is not None:
        for bi, n in enumerate(lengths):
            assert torch.count_nonzero(out[bi, :, n:]).item() == 0


def _sweep_cases(n, seed):
    """Seeded random configurations: shape, head dim, causality, dtype,
    layout ([B, S, H, D] storage viewed as [B, H, S, D], or contiguous), valid
    lengths (0 and S included), split scores."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        b, h = int(rng.integers(1, 5)), int(rng.integers(1, 6))
        s = int(rng.choice([1, 2, 63, 64, 65, 127, 255, 256, 257, 511, 700, 1024, 1500]))
        d = int(rng.choice([32, 64, 128]))
        lengths = None
        if rng.random() < 0.6:
            lengths = [int(x) for x in rng.integers(0, s + 1, size=b)]
            lengths[int(rng.integers(0, b))] = s
        cases.append(dict(b=b, h=h, s=s, d=d, causal=bool(rng.random() < 0.6), lengths=lengths,
                          f16=bool(rng.random() < 0.3), bshd=bool(rng.random() < 0.5),
                          split=bool(rng.random() < 0.25), seed=1000 + i))
    return cases


@pytest.mark.parametrize("case", _sweep_cases(40, 2024), ids=lambda c: "{seed}-b{b}h{h}s{s}d{d}{}{}{}{}".format(
    "c" if c["causal"] else "", "L" if c["lengths"] else "", "h" if c["f16"] else "", "x" if c["split"] else "",
    **c))
def test_random_configurations_match_brute_force(cuda, case):
    """Every combination the dispatcher can hand the kernel, against the
    float64 brute force; ``out`` starts as NaN so an unwritten row fails."""
    from techjam_amd.kernels import scaled_dot_product_attention

    b, h, s, d = case["b"], case["h"], case["s"], case["d"]
    dt = torch.float16 if case["f16"] else torch.float32
    q, k, v = (_draw((b, s, h, d), case["seed"] + j, dtype=dt) for j in range(3))
    if case["bshd"]:
        views = [t.to(cuda).transpose(1, 2) for t in (q, k, v)]
        out = torch.full((b, s, h, d), float("nan"), device=cuda, dtype=dt).transpose(1, 2)
    else:
        views = [t.transpose(1, 2).contiguous().to(cuda) for t in (q, k, v)]
        out = torch.full((b, h, s, d), float("nan"), device=cuda, dtype=dt)
    vl = None if case["lengths"] is None else torch.tensor(case["lengths"], dtype=torch.int32, device=cuda)
    scaled_dot_product_attention(*views, is_causal=case["causal"], valid_len=vl, out=out,
                                 qk_split=True if case["split"] else None)
    torch.cuda.synchronize()
    ref = brute_force_attention(*(t.cpu() for t in views), d ** -0.5, case["causal"], valid_len=case["lengths"])
    _assert_close(out.float(), ref, max_abs=4e-3 if not case["f16"] else 6e-3, what=str(case))


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_rows_past_the_sequence_end_read_as_zeros(cuda, dtype, causal, split):
    """K and V views whose memory continues past row S - 1 with NaN. S = 1000
    is not a multiple of the 64-key tile, so the last tile reaches 24 rows
    past the end; the bounds-checked buffer loads must return zeros there (a
    NaN value row times a zero weight would still poison every output row)."""
    from techjam_amd.kernels import scaled_dot_product_attention

    b, h, s, d, pad = 2, 3, 1000, 64, 64
    q, k, v = (_draw((b, h, s, d), seed, dtype=dtype) for seed in (11, 12, 13))
    views = [q.to(cuda)]
    for t in (k, v):
        full = torch.full((b, h, s + pad, d), float("nan"), device=cuda, dtype=dtype)
        full[:, :, :s] = t.to(cuda)
        views.append(full[:, :, :s])
    out = torch.full((b, h, s, d), float("nan"), device=cuda, dtype=dtype)
    scaled_dot_product_attention(*views, is_causal=causal, out=out, qk_split=True if split else None)
    torch.cuda.synchronize()
    ref = brute_force_attention(q, k, v, d ** -0.5, causal)
    _assert_close(out.float(), ref, max_abs=4e-3 if dtype == torch.float32 else 6e-3,
                  what=f"{dtype} causal={causal} split={split}")


@pytest.mark.parametrize("causal", [True, False])
def test_wide_tiles_with_ragged_lengths(cuda, causal):
    """B=8 H=16 S=2048 takes the 256-row tile path (1024 wide tiles) with
    right padding: every (b, h) against the blockwise oracle on the GPU."""
    from techjam_amd.kernels import scaled_dot_product_attention

    b, s, h, d = 8, 2048, 16, 64
    g = torch.Generator(device=cuda).manual_seed(77)
    q, k, v = (torch.randn(b, s, h, d, generator=g, device=cuda).transpose(1, 2) for _ in range(3))
    lengths = torch.tensor([2048, 1, 0, 257, 1024, 2047, 700, 1500], dtype=torch.int32, device=cuda)
    out = torch.full((b, s, h, d), float("nan"), device=cuda).transpose(1, 2)
    scaled_dot_product_attention(q, k, v, is_causal=causal, valid_len=lengths, out=out)
    torch.cuda.synchronize()
    prev = torch.get_float32_matmul_precision()
    torch.set_float32_matmul_precision("highest")
    try:
        ref = blockwise_attention(q, k, v, d ** -0.5, causal, valid_len=lengths, block_q=512, block_k=512)
    finally:
        torch.set_float32_matmul_precision(prev)
    err = (out - ref).abs()
    ok = torch.isfinite(out) & ((err <= ATOL) | (err <= RTOL * ref.abs()))
    assert int((~ok).sum()) == 0, f"{int((~ok).sum())} failing, max abs {float(err.max()):.3e}"
    for bi, n in enumerate(lengths.tolist()):
        assert torch.count_nonzero(out[bi, :, n:]).item() == 0


@pytest.mark.parametrize("mode", ["causal", "padded", "row_limits", "ragged_s"])
def test_split_scores_on_wide_tiles(cuda, mode):
    """Split scores for every head on a grid of 1024 256-row tiles (B=8 H=16
    S=2048): the kernel with two query blocks per wave and 32-key tiles.
    Scores have sd ~4 (q, k ~ N(0, 2^2)), the range split scores exist for;
    every (b, h) against the blockwise oracle on the GPU in fp32. `padded`
    adds right padding without causality; `row_limits` computes only the
    first rows of some heads (the guarded route's launch) and must leave the
    others' rows untouched; `ragged_s` has a sequence length that is not a
    multiple of the key tile."""
    from techjam_amd.kernels import scaled_dot_product_attention

    b, s, h, d = 8, (2000 if mode == "ragged_s" else 2048), 16, 64  # 2000: the last 32-key tile is half past S
    g = torch.Generator(device=cuda).manual_seed(78)
    q, k = (torch.randn(b, s, h, d, generator=g, device=cuda).transpose(1, 2) * 2.0 for _ in range(2))
    v = torch.randn(b, s, h, d, generator=g, device=cuda).transpose(1, 2)
    causal = mode != "padded"
    lengths = (torch.tensor([2048, 1, 0, 257, 1024, 2047, 700, 1500], dtype=torch.int32, device=cuda)
               if mode == "padded" else None)
    limits = None
    if mode == "row_limits":
        limits = torch.full((b * h,), s, dtype=torch.int32, device=cuda)
        limits[1::3] = 300
        limits[2::5] = 0
    out = torch.full((b, s, h, d), float("nan"), device=cuda).transpose(1, 2)
    scaled_dot_product_attention(q, k, v, is_causal=causal, valid_len=lengths, out=out,
                                 qk_split=torch.ones(b * h, dtype=torch.int32, device=cuda),
                                 row_limit=limits)
    torch.cuda.synchronize()
    prev = torch.get_float32_matmul_precision()
    torch.set_float32_matmul_precision("highest")
    try:
        ref = blockwise_attention(q, k, v, d ** -0.5, causal, valid_len=lengths, block_q=512, block_k=512)
    finally:
        torch.set_float32_matmul_precision(prev)
    rows = torch.ones(b, h, s, dtype=torch.bool, device=cuda)
    if limits is not None:
        rows = torch.arange(s, device=cuda)[None, None, :] < limits.view(b, h, 1)
        assert bool(torch.isnan(out[~rows]).all()), "rows beyond a row limit were written"
    err = (out - ref).abs()[rows]
    ok = torch.isfinite(out[rows]) & ((err <= ATOL) | (err <= RTOL * ref[rows].abs()))
    assert int((~ok).sum()) == 0, f"{int((~ok).sum())} failing, max abs {float(err.max()):.3e}"
    assert float(err.max()) < 4e-3, f"max abs {float(err.max()):.3e}"


@pytest.mark.parametrize("seed", [78, 79, 80])
def test_split_heads_error_is_the_rounding_of_v(cuda, seed):
    """Split heads at score sd 4 (q, k ~ N(0, 2^2), B=8 H=16 S=2000, 16.4 M
    outputs per seed): scores from hi/lo fp16 parts of q and k, probabilities
    as hi/lo fp16 parts, so the only rounding left is v's to fp16 for the PV
    MFMA. An output then moves by at most 2^-11 * sum_j p_j |v_j| / l (the
    attention of |v|), below the OR rule's 2e-3 for |v| < 8. Asserted: zero
    failing elements; every error within that bound; and against the oracle
    run on v rounded to fp16, the kernel is fp32-accurate."""
    from techjam_amd.kernels import scaled_dot_product_attention

    b, s, h, d = 8, 2000, 16, 64
    g = torch.Generator(device=cuda).manual_seed(seed)
    q, k = (torch.randn(b, s, h, d, generator=g, device=cuda).transpose(1, 2) * 2.0 for _ in range(2))
    v = torch.randn(b, s, h, d, generator=g, device=cuda).transpose(1, 2)
    out = torch.empty(b, s, h, d, device=cuda).transpose(1, 2)
    scaled_dot_product_attention(q, k, v, is_causal=True, out=out,
                                 qk_split=torch.ones(b * h, dtype=torch.int32, device=cuda))
    torch.cuda.synchronize()
    qd, kd = q.double(), k.double()
    ref = blockwise_attention(qd, kd, v.double(), d ** -0.5, True, block_q=500, block_k=500, acc_dtype=torch.float64)
    err = (out.double() - ref).abs()
    ok = torch.isfinite(out) & ((err <= ATOL) | (err <= RTOL * ref.abs()))
    assert int((~ok).sum()) == 0, f"{int((~ok).sum())} outputs outside the OR rule, max abs {float(err.max()):.3e}"
    del ref
    v_abs = blockwise_attention(qd, kd, v.double().abs(), d ** -0.5, True, block_q=500, block_k=500,
                                acc_dtype=torch.float64)
    excess = err - (2.0 ** -11 * v_abs + 2e-5)
    assert float(excess.max()) <= 0.0, f"error exceeds v's rounding bound by {float(excess.max()):.3e}"
    del v_abs, excess
    ref_h = blockwise_attention(qd, kd, v.half().double(), d ** -0.5, True, block_q=500, block_k=500,
                                acc_dtype=torch.float64)
    assert float((out.double() - ref_h).abs().max()) <= 1e-4


def _midpoint_queries(n: int, d: int, qscale: float, seed: int) -> np.ndarray:
    """fp32 q values whose product with ``qscale`` rounds in fp32 onto a
    midpoint between two fp16 numbers while the exact product does not sit on
    it: fp16(fp32(q * qscale)) and fp16(q * qscale) then differ by an ulp."""
    rng = np.random.default_rng(seed)
    c32 = np.float32(qscale)
    picked = []
    need = n * d
    while need > 0:
        h = rng.uniform(0.5, 1.9, 4 * need).astype(np.float16)
        mid = (h.astype(np.float64) + np.nextafter(h, np.float16(2)).astype(np.float64)) / 2
        x0 = (mid / float(c32)).astype(np.float32)
        for x in (x0, np.nextafter(x0, np.float32(0)), np.nextafter(x0, np.float32(4))):
            y32 = (x * c32).astype(np.float32)
            exact = x.astype(np.float64) * float(c32)
            good = ((y32.astype(np.float64) == mid) & (exact != mid)
                    & (y32.astype(np.float16) != exact.astype(np.float16)))
            take = x[good][:need]
            picked.append(take)
            need -= take.size
            if need <= 0:
                break
    out = np.concatenate(picked)[: n * d]
    out *= np.where(rng.random(out.size) < 0.5, -1.0, 1.0).astype(np.float32)
    return out.reshape(n, d)


def test_split_scores_with_q_on_fp16_midpoints(cuda):
    """Every scaled query element rounds (in fp32) onto an fp16 midpoint, where
    rounding the fp32 product and rounding the exact product to fp16 pick
    different neighbours: the hi and lo parts of q must come from the same
    fp32 value, or hi + lo misses q by an fp16 ulp in every dimension and the
    scores lose the accuracy split heads exist for. Checked against the fp64
    brute force with v rounded to fp16 (so only the kernel's own arithmetic
    counts), on the 128-row and the 256-row split kernels."""
    from techjam_amd.kernels import scaled_dot_product_attention

    d = 64
    qscale = float(np.float32(d ** -0.5) * np.float32(1.4426950408889634))
    for b, h, s in ((1, 2, 256), (8, 16, 512)):
        g = torch.Generator().manual_seed(5)
        q = torch.from_numpy(_midpoint_queries(b * h * s, d, qscale, 6)).view(b, h, s, d)
        k = torch.randn(b, h, s, d, generator=g) * 0.5  # scores of sd ~3: rows mix several keys
        v = torch.randn(b, h, s, d, generator=g).half().float()
        out = scaled_dot_product_attention(q.to(cuda), k.to(cuda), v.to(cuda), is_causal=True,
                                           qk_split=torch.ones(b * h, dtype=torch.int32, device=cuda))
        torch.cuda.synchronize()
        ref = blockwise_attention(q.double().to(cuda), k.double().to(cuda), v.double().to(cuda), d ** -0.5, True,
                                  acc_dtype=torch.float64)
        err = float((out.double() - ref).abs().max())
        assert err <= 1e-4, f"B={b} H={h} S={s}: max abs {err:.3e}"


def test_keys_spanning_more_than_2_gib_are_copied_not_refused(cuda):
    """k and v rows 4 MiB apart (600 rows span 2.3 GiB, beyond the kernels'
    31-bit offsets): the wrapper reads them through a contiguous copy, and the
    result is bitwise that of contiguous inputs."""
    from techjam_amd.kernels import scaled_dot_product_attention

    b, h, s, d, row = 1, 2, 600, 64, 1 << 20
    g = torch.Generator(device=cuda).manual_seed(9)
    q = torch.randn(b, h, s, d, generator=g, device=cuda)
    big_k = torch.zeros(s, row, device=cuda)
    big_v = torch.zeros(s, row, device=cuda)
    big_k[:, : h * d] = torch.randn(s, h * d, generator=g, device=cuda)
    big_v[:, : h * d] = torch.randn(s, h * d, generator=g, device=cuda)
    k = big_k[:, : h * d].view(s, h, d).unsqueeze(0).transpose(1, 2)  # [1, H, S, D], row stride 2^20
    v = big_v[:, : h * d].view(s, h, d).unsqueeze(0).transpose(1, 2)
    assert ((s - 1) * k.stride(2) + d) * 4 >= 1 << 31
    got = scaled_dot_product_attention(q, k, v, is_causal=True)
    want = scaled_dot_product_attention(q, k.contiguous(), v.contiguous(), is_causal=True)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    del big_k, big_v, k, v
    torch.cuda.empty_cache()
