"""ds4cuda_amd — MI355X (gfx950) implementation of ds4cuda's attention path.

The compute lives in libds4hip.so (hand-written HIP kernels behind the C-ABI
of include/ds4hip.h); this package is the Python host mirror of the
reference launchers (ds4cuda_amd.ops) plus the synthetic input generator.
"""
from ._lib import Ds4HipError, LIB_PATH, lib  # noqa: F401

__all__ = ["Ds4HipError", "LIB_PATH", "lib"]
