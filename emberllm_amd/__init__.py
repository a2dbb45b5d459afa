"""emberllm_amd — emberllm's token loop on one MI355X (gfx950).

The product is ``libember.so`` (C11 host library with the ember.h API over
hand-written HIP kernels).  This package holds its sources (``csrc/``), the
ctypes prototypes (``_native``), a Python binding with the reference's
``Ember`` class API (``emberllm``) and the benchmark model shapes
(``configs``).
"""
from . import _native  # noqa: F401

__all__ = ["_native", "configs", "emberllm"]
