"""Python entry points of the HIP exact-attention and score-guard kernels.

``scaled_dot_product_attention`` stands where the reference calls
``torch.nn.functional.scaled_dot_product_attention``
(``src/implementations/sdpa.py:65-73``, ``:157-165``,
``src/implementations/extreme.py:227-236``); ``score_guard`` replaces
``estimate_sigma``/``poly_is_safe`` (``src/implementations/poly_guard.py:68-102``)
without a host synchronisation. Tensors stay where they are: strided
``[B, H, S, D]`` views are passed to the kernels by pointer and strides.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Union

import torch
import torch.nn.functional as F

from ..errors import UnsupportedCaseError
from . import _lib

SUPPORTED_HEAD_DIMS = (32, 64, 128, 256)

_DTYPES = {torch.float32: _lib.TJ_F32, torch.float16: _lib.TJ_F16}


def _stream_ptr(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _require_device(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise UnsupportedCaseError(
            "the HIP attention kernels require tensors on a ROCm GPU; "
            f"got device {dev} (there is no CPU implementation)"
        )
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"tensors are on different devices: {dev} and {t.device}")
    return dev


#: The kernels address the rows of one (b, h) with 31-bit byte offsets.
MAX_HEAD_SPAN_BYTES = 1 << 31


def _head_span_bytes(t: torch.Tensor) -> int:
    s, d = t.shape[2], t.shape[3]
    return ((s - 1) * t.stride(2) + d) * t.element_size() if s > 0 else 0


def _kernel_view(t: torch.Tensor, keys: bool = False) -> torch.Tensor:
    """``t`` itself when the kernels can read it in place, else a contiguous copy.

    In-place reading needs a unit innermost stride, 16-byte aligned rows and a
    16-byte aligned base, and for keys and values (``keys``) rows of one
    (b, h) spanning under 2 GiB; the model's projection views qualify. The
    copy is ``[B, H, S, D]`` contiguous, whose head span is ``S*D`` elements
    -- so keys of a long sequence in an interleaved ``[B, S, H, D]`` layout
    (over 2^31 / (H*D*4) tokens in fp32) cost one copy instead of being
    refused.
    """
    vec = 16 // t.element_size()
    st = t.stride()
    if (st[3] == 1 and all(s % vec == 0 for s in st[:3]) and t.data_ptr() % 16 == 0
            and (not keys or (st[2] >= 0 and _head_span_bytes(t) < MAX_HEAD_SPAN_BYTES))):
        return t
    return t.contiguous()


def _check_qkv(q, k, v):
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, v must be [B, H, S, D]")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"q, k, v shapes differ: {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if q.dtype not in _DTYPES:
        raise UnsupportedCaseError(f"dtype {q.dtype} is not supported (float32 or float16)")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k, v must share a dtype")
    if kernel_head_dim(q.shape[-1]) is None:
        raise UnsupportedCaseError(
            f"head_dim {q.shape[-1]} is not supported (at most {SUPPORTED_HEAD_DIMS[-1]}; "
            f"{SUPPORTED_HEAD_DIMS} natively, others zero-padded)"
        )


def kernel_head_dim(d: int) -> Optional[int]:
    """The kernel head_dim that serves ``d``: ``d`` itself when the kernel
    has it, else the next of ``SUPPORTED_HEAD_DIMS`` (q, k, v zero-padded to
    it), or ``None`` beyond the largest."""
    for p in SUPPORTED_HEAD_DIMS:
        if 0 < d <= p:
            return p
    return None


def empty_like_heads(q: torch.Tensor) -> torch.Tensor:
    """A ``[B, H, S, D]`` output whose storage is ``[B, S, H, D]``.

    The caller's ``transpose(1, 2).reshape(B, S, H*D)`` is then a free view
    instead of a copy.
    """
    b, h, s, d = q.shape
    return torch.empty(b, s, h, d, dtype=q.dtype, device=q.device).transpose(1, 2)


def scaled_dot_product_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    is_causal: bool = False,
    scale: Optional[float] = None,
    valid_len: Optional[torch.Tensor] = None,
    row_limit: Optional[torch.Tensor] = None,
    qk_split: Union[bool, torch.Tensor, None] = None,
    out: Optional[torch.Tensor] = None,
    q_bias: Optional[torch.Tensor] = None,
    v_bias: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Exact attention on the HIP kernel; ``[B, H, S, D]`` views in, ``[B, H, S, D]`` out.

    ``valid_len`` (int32 ``[B]`` on the device) masks keys ``j >= valid_len[b]``
    and zeroes rows ``i >= valid_len[b]``: the right-padding contract of the
    model, where those rows are zeroed after the output projection anyway.
    ``row_limit`` (int32 ``[B*H]``) restricts the rows computed per head; the
    other rows of ``out`` are left untouched. ``qk_split`` (``True`` for all
    heads, or an int32 ``[B*H]`` device flag tensor) selects the three-MFMA
    score path that keeps fp32-level score accuracy for wide score ranges.

    ``q_bias`` / ``v_bias`` (fp32 ``[H*D]``, contiguous, on the device) are the
    projection biases of bias-free q and v views: the result is the attention
    of ``q + q_bias`` and ``v + v_bias``. A key bias has no effect on the
    output (it shifts every score of a row by the same amount), so callers
    drop it. Not combined with ``row_limit`` or ``qk_split``.
    """
    _check_qkv(q, k, v)
    if out is not None and (out.shape != q.shape or out.dtype != q.dtype or out.device != q.device):
        raise ValueError("out must match q in shape, dtype and device")
    dev = _require_device(q, k, v)
    b, h, s, d = q.shape
    if scale is None:
        scale = d ** -0.5
    dp = kernel_head_dim(d)
    if dp != d:
        # Zero dims add nothing to q.k and give zero output columns: pad to the
        # kernel's head_dim (same scale) and return the first d columns.
        if out is not None:
            raise ValueError(f"out= is not supported for head_dim {d} (computed padded to {dp})")
        pad = (0, dp - d)
        q, k, v = (F.pad(t, pad) for t in (q, k, v))
        q_bias, v_bias = (None if t is None else F.pad(t.reshape(h, d), pad).reshape(-1)
                          for t in (q_bias, v_bias))
        res = scaled_dot_product_attention(q, k, v, is_causal=is_causal, scale=scale, valid_len=valid_len,
                                           row_limit=row_limit, qk_split=qk_split, q_bias=q_bias, v_bias=v_bias)
        return res[..., :d]
    q, k, v = _kernel_view(q), _kernel_view(k, keys=True), _kernel_view(v, keys=True)
    if out is None:
        out = empty_like_heads(q)
    elif out.shape != q.shape or out.dtype != q.dtype or out.device != dev:
        raise ValueError("out must match q in shape, dtype and device")
    if qk_split is True:
        qk_split = _all_heads(b * h, dev)
    elif qk_split is False:
        qk_split = None
    for name, t, n in (("valid_len", valid_len, b), ("row_limit", row_limit, b * h),
                       ("qk_split", qk_split, b * h)):
        if t is not None and (t.dtype != torch.int32 or t.device != dev or t.numel() != n
                              or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous int32 tensor of {n} elements on {dev}")
    if q_bias is not None or v_bias is not None:
        if row_limit is not None or qk_split is not None:
            raise ValueError("q_bias / v_bias do not combine with row_limit or qk_split")
        for name, t in (("q_bias", q_bias), ("v_bias", v_bias)):
            if t is not None and (t.dtype != torch.float32 or t.device != dev or t.numel() != h * d
                                  or not t.is_contiguous() or t.data_ptr() % 16):
                raise ValueError(f"{name} must be a contiguous, 16-byte aligned float32 tensor of {h * d} "
                                 f"elements on {dev}")
        code = _lib.lib().tj_attn_fwd_proj_bias(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), _DTYPES[q.dtype],
            b, h, s, d,
            _lib.strides4(q), _lib.strides4(k), _lib.strides4(v), _lib.strides4(out),
            float(scale), int(bool(is_causal)), _ptr(valid_len), _ptr(q_bias), _ptr(v_bias),
            _stream_ptr(dev),
        )
        _lib.check(code, "tj_attn_fwd_proj_bias")
        return out
    code = _lib.lib().tj_attn_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), _DTYPES[q.dtype],
        b, h, s, d,
        _lib.strides4(q), _lib.strides4(k), _lib.strides4(v), _lib.strides4(out),
        float(scale), int(bool(is_causal)), _ptr(valid_len), _ptr(row_limit), _ptr(qk_split),
        _stream_ptr(dev),
    )
    _lib.check(code, "tj_attn_fwd")
    return out


#: Entries kept by each of the small device-tensor caches below (oldest
#: dropped first), so that callers cycling through many shapes do not grow
#: them without bound.
CACHE_ENTRIES = 64

_ONES: dict = {}


def _cache_put(cache: dict, key, value):
    if len(cache) >= CACHE_ENTRIES:
        cache.pop(next(iter(cache)))
    cache[key] = value
    return value


def _all_heads(n: int, dev: torch.device) -> torch.Tensor:
    key = (n, str(dev))
    t = _ONES.get(key)
    if t is None:
        t = _cache_put(_ONES, key, torch.ones(n, dtype=torch.int32, device=dev))
    return t


@dataclass
class GuardResult:
    """Per-(b,h) outputs of the device-side guard (all device tensors, flattened ``[B*H]``)."""

    sigma: torch.Tensor       # float32 [B*H]
    mean: torch.Tensor        # float32 [B*H]
    smax: torch.Tensor        # float32 [B*H]
    flags: torch.Tensor       # int32   [B*H], 1 = polynomial route
    coeffs: torch.Tensor      # float32 [B*H, 3]
    row_limit: torch.Tensor   # int32   [B*H], rows the exact kernel computes
    split: torch.Tensor       # int32   [B*H], 1 = exact fallback with split scores


_SAMPLE_CACHE: dict = {}


def sample_index(n: int, samples: int, seed: int, device: torch.device) -> torch.Tensor:
    """Device copy of the guard's row sample: first ``min(samples, n)`` of a seeded permutation.

    Drawn with a CPU generator and cached per ``(n, samples, seed, device)``,
    so repeated forwards upload it once.
    """
    key = (n, samples, seed, str(device))
    idx = _SAMPLE_CACHE.get(key)
    if idx is None:
        gen = torch.Generator().manual_seed(seed)
        cpu = torch.randperm(n, generator=gen)[: min(samples, n)].to(torch.int32)
        idx = _cache_put(_SAMPLE_CACHE, key, cpu.to(device))
    return idx


def score_guard(
    q: torch.Tensor,
    k: torch.Tensor,
    scale: float,
    *,
    samples: int = 512,
    seed: int = 0,
    ceiling: float = 0.40,
    exact_prefix: int = 4096,
) -> GuardResult:
    """Per-head sigma, flag, Hermite coefficients and exact-row limit, on the device."""
    if q.ndim != 4 or k.ndim != 4:
        raise ValueError("q and k must be [B, H, N, D]")
    if q.shape != k.shape:
        raise ValueError("q and k shapes differ")
    if q.dtype not in _DTYPES or k.dtype != q.dtype:
        raise UnsupportedCaseError(f"dtype {q.dtype} is not supported")
    dev = _require_device(q, k)
    b, h, s, d = q.shape
    q, k = _kernel_view(q), _kernel_view(k)
    idx = sample_index(s, samples, seed, dev)
    m = b * h
    res = GuardResult(
        sigma=torch.empty(m, dtype=torch.float32, device=dev),
        mean=torch.empty(m, dtype=torch.float32, device=dev),
        smax=torch.empty(m, dtype=torch.float32, device=dev),
        flags=torch.empty(m, dtype=torch.int32, device=dev),
        coeffs=torch.empty(m, 3, dtype=torch.float32, device=dev),
        row_limit=torch.empty(m, dtype=torch.int32, device=dev),
        split=torch.empty(m, dtype=torch.int32, device=dev),
    )
    lib = _lib.lib()
    ws_bytes = lib.tj_score_guard_workspace_bytes(b, h, idx.numel())
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    code = lib.tj_score_guard(
        q.data_ptr(), k.data_ptr(), _DTYPES[q.dtype], b, h, s, d,
        _lib.strides4(q), _lib.strides4(k), float(scale), idx.data_ptr(), idx.numel(),
        float(ceiling), int(exact_prefix),
        res.sigma.data_ptr(), res.mean.data_ptr(), res.smax.data_ptr(), res.flags.data_ptr(),
        res.coeffs.data_ptr(), res.row_limit.data_ptr(), res.split.data_ptr(),
        ws.data_ptr(), ws.numel(), _stream_ptr(dev),
    )
    _lib.check(code, "tj_score_guard")
    return res
