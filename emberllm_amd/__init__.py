"""emberllm_amd — emberllm's token loop on one MI355X (gfx950).

The product is ``libember.so`` (C11 host library with the ember.h API over
hand-written HIP kernels).  This package holds its sources (``csrc/``), the
ctypes prototypes (``_native``), ``emberllm.Engine`` (the numpy wrapper
the tests and the benchmark drive the C ABI through) and the benchmark model
shapes (``configs``).
"""
from . import _native  # noqa: F401

__all__ = ["_native", "configs", "emberllm"]
