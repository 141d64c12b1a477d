"""Exception types shared by the dispatcher and the kernel wrappers."""

from __future__ import annotations


class UnsupportedCaseError(RuntimeError):
    """A request the HIP path refuses before allocating anything.

    Same role as the reference's ``UnsupportedCaseError``
    (``src/dispatcher.py:141-142``): raised for contracts the MI355X path does
    not implement (CPU tensors, unsupported head sizes or dtypes). There is no
    silent fallback to another implementation.
    """
