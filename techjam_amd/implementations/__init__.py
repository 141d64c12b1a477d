"""Attention modules, routing and streaming helpers of the HIP path.

Mirrors ``src/implementations`` of the reference: ``sdpa`` (exact strided and
packed-QKV attention), ``attention_routing`` (mask classification),
``extreme`` (batch/prefix streaming and the guarded polynomial module),
``poly_guard`` and ``poly_attention``.
"""
