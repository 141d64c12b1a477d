"""HIP kernel entry points (ctypes over the C ABI of ``include/techjam_attn.h``)."""

from .attention import scaled_dot_product_attention, score_guard

__all__ = ["scaled_dot_product_attention", "score_guard"]
