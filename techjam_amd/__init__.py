"""MI355X-native attention hot path of the techjam Transformer benchmark.

The package mirrors the reference's Python interface (``src.dispatcher``,
``src.implementations.*``, ``src.infra``) while every attention call runs the
hand-written gfx950 HIP kernels of ``libtechjam_attn.so`` through the C ABI
declared in ``include/techjam_attn.h``. There is no CPU or PyTorch fallback for
attention: without a ROCm GPU or without the built library the attention
entry points raise.
"""

from .errors import UnsupportedCaseError

__all__ = ["UnsupportedCaseError"]
