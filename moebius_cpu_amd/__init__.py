"""moebius-hip: the MI355X (gfx950) conv/norm hot path of moebius-cpu.

The product is the C-ABI library `libmoebius_hip.so` (include/moebius_hip.h):
hand-written HIP kernels plus the C++ engine/model host code. This Python
package only loads it (ctypes) and mirrors the reference engine API for tests
and benchmarks; it has no compute path of its own and no CPU fallback.
"""
from ._lib import LIB_PATH, MoebiusError, lib  # noqa: F401

__all__ = ["LIB_PATH", "MoebiusError", "lib"]
