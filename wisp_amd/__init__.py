"""wisp_amd — MI355X (gfx950) rebuild of WISP's int4 routed-expert MoE path.

The product is the C-ABI shared library wisp_amd/libwisp_amd.so (declared in
include/wisp_amd.h). This package holds its sources (csrc/), the build
script, and thin ctypes front ends used by the tests and the benchmark.
"""
from ._lib import LIB_PATH, lib  # noqa: F401

__all__ = ["lib", "LIB_PATH"]
