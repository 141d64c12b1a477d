"""Exact attention modules on the HIP kernel: strided and packed-QKV projections.

Mirror ``src/implementations/sdpa.py:13-170``:

* ``StridedSDPASelfAttention`` projects q, k, v with separate ``nn.Linear``
  layers and hands ``[B, H, S, dh]`` strided views of the ``[B, S, D]``
  projections to the kernel (no ``.contiguous()`` copies, ``sdpa.py:32-34``).
* ``PackedQKVSDPASelfAttention`` keeps a derived ``[3D, D]`` weight, runs one
  GEMM and views the ``[B, S, 3, H, dh]`` result (strides
  ``(3SD, dh, 3D, 1)``, ``sdpa.py:127-138``); the derived buffers are rebuilt
  on ``load_state_dict`` and ``_apply`` (``sdpa.py:93``, ``:118-125``).

``drop_key_mask`` keeps its reference meaning -- the caller has established
causal attention with a right-padded mask -- but here it only decides whether
the kernel also receives the per-sample lengths; with or without them the
valid rows are identical (the lengths additionally skip padded query tiles).
The kernel writes its ``[B, H, S, dh]`` output in ``[B, S, H, dh]`` storage, so
the merge back to ``[B, S, D]`` before the output projection is a view.
"""

from __future__ import annotations

from typing import Optional

import torch

from ..kernels.attention import scaled_dot_product_attention
from ..model import HipSelfAttention, linear, project


class StridedSDPASelfAttention(HipSelfAttention):
    """q/k/v ``nn.Linear`` projections, strided head views, HIP exact attention."""

    drop_key_mask = False

    def context(self, x, valid_token_mask=None, causal=False, valid_len=None):
        b, s, _ = x.shape
        if self.folds_biases(x):
            q, k, v, qb, vb = self.project_qkv_folded(x)
            ctx = scaled_dot_product_attention(q, k, v, is_causal=causal, scale=self.scale, valid_len=valid_len,
                                               q_bias=qb, v_bias=vb)
        else:
            q, k, v = self.project_qkv(x)
            ctx = scaled_dot_product_attention(q, k, v, is_causal=causal, scale=self.scale, valid_len=valid_len)
        return ctx.transpose(1, 2).reshape(b, s, self.d_model)


class PackedQKVSDPASelfAttention(StridedSDPASelfAttention):
    """One ``[3D, D]`` GEMM feeding copy-free q/k/v views (inference only)."""

    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__(d_model, num_heads)
        self.register_buffer("_packed_qkv_weight", torch.empty(0), persistent=False)
        self.register_buffer("_packed_qkv_bias", torch.empty(0), persistent=False)
        self.refresh_packed_qkv()
        self.register_load_state_dict_post_hook(self._repack_after_load)

    @torch.no_grad()
    def refresh_packed_qkv(self) -> None:
        """Rebuild the derived packed weight after any parameter change."""
        weight = torch.cat((self.q_proj.weight, self.k_proj.weight, self.v_proj.weight), dim=0).detach()
        bias = torch.cat((self.q_proj.bias, self.k_proj.bias, self.v_proj.bias), dim=0).detach()
        same = (self._packed_qkv_weight.shape == weight.shape
                and self._packed_qkv_weight.device == weight.device
                and self._packed_qkv_weight.dtype == weight.dtype)
        if same:
            self._packed_qkv_weight.copy_(weight)
            self._packed_qkv_bias.copy_(bias)
        else:
            self._packed_qkv_weight = weight
            self._packed_qkv_bias = bias

    def _repack_after_load(self, module, incompatible_keys) -> None:
        del module, incompatible_keys
        self.refresh_packed_qkv()

    def _apply(self, fn, recurse: bool = True):
        result = super()._apply(fn, recurse=recurse)
        self.refresh_packed_qkv()
        return result

    def project_qkv(self, x: torch.Tensor):
        if torch.is_grad_enabled():
            # The packed buffers are inference caches, not trainable parameters.
            return super().project_qkv(x)
        b, s, _ = x.shape
        packed = linear(x, self._packed_qkv_weight, self._packed_qkv_bias)
        q, k, v = packed.view(b, s, 3, self.num_heads, self.head_dim).unbind(dim=2)
        return q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)

    def project_qkv_folded(self, x: torch.Tensor):
        """One bias-free ``[3D, D]`` GEMM (fp16 operands and result for an fp16
        ``x``); the q and v thirds of the packed bias go to the kernel (the key
        third never changes the output)."""
        b, s, _ = x.shape
        packed = project(x, self._packed_qkv_weight, self, "packed_qkv")
        q, k, v = packed.view(b, s, 3, self.num_heads, self.head_dim).unbind(dim=2)
        d = self.d_model
        return (q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                self._packed_qkv_bias[:d], self._packed_qkv_bias[2 * d:])


def attention_core(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool = True,
                   scale: Optional[float] = None, valid_len: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Exact attention core on ``[B, H, S, dh]`` tensors (the single-layer workloads)."""
    return scaled_dot_product_attention(q, k, v, is_causal=causal, scale=scale, valid_len=valid_len)
