"""MI355X-native EFLA hot path: HIP kernels for gfx950 behind a C ABI.

``ceo_amd.efla`` (EFLA, reference ABI and chunked query readout),
``ceo_amd.nn`` (LayerNorm, GEMM) and ``ceo_amd.runtime`` (device layer and
launch profiler) all call libefla_hip.so through ctypes.
"""
from ._lib import HipError, build, lib  # noqa: F401

__all__ = ["HipError", "build", "lib"]
