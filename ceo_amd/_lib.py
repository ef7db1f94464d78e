"""ctypes binding of libefla_hip.so (the C ABI in include/efla_hip.h and
include/efla_runtime.h).

The library is built in-tree by ``make -C ceo_amd/csrc`` (see
``__graft_entry__.build``).  Loading never falls back to anything else: a
missing library raises, so nothing can silently run without the HIP kernels.
"""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(_HERE)
CSRC = os.path.join(_HERE, "csrc")
LIB_PATH = os.path.join(_HERE, "lib", "libefla_hip.so")
HEADERS = [os.path.join(ROOT, "include", "efla_hip.h"),
           os.path.join(ROOT, "include", "efla_runtime.h")]

_LIB = None

# hipError_t names for the codes this library returns
ERROR_NAMES = {
    0: "Success",
    1: "InvalidValue",
    2: "OutOfMemory",
    3: "NotInitialized",
    9: "InvalidConfiguration",
    98: "InvalidDeviceFunction",
    100: "NoDevice",
    101: "InvalidDevice",
    400: "InvalidHandle",
    700: "IllegalAddress",
    719: "LaunchFailure",
    801: "NotSupported",
}


class HipError(RuntimeError):
    """A non-zero hipError_t returned by an entry point."""

    def __init__(self, code: int, where: str):
        self.code = code
        self.name = ERROR_NAMES.get(code, f"hipError{code}")
        super().__init__(f"{where} failed: {self.name} ({code})")


def build(jobs: int = 8) -> None:
    subprocess.run(["make", "-s", "-C", CSRC, f"-j{jobs}"], check=True)


def header_functions() -> list[str]:
    """Names of the functions the public headers declare."""
    names = []
    pat = re.compile(r"^\s*(?:int|size_t|void)\s+(\w+)\s*\(", re.M)
    for h in HEADERS:
        with open(h) as f:
            names += pat.findall(f.read())
    return names


vp = ctypes.c_void_p
sz = ctypes.c_size_t
i32 = ctypes.c_int
f32 = ctypes.c_float

_SIGS = {
    # EFLA, reference ABI
    "efla_forward_hip": (i32, [vp, vp, vp, vp, sz, sz, sz, sz, f32, sz, vp]),
    "efla_backward_hip": (i32, [vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, f32, vp]),
    "efla_chunked_scan_hip": (i32, [ctypes.POINTER(vp), sz, sz, sz, vp]),
    "efla_affine_state_scan_hip": (i32, [ctypes.POINTER(vp), ctypes.POINTER(vp), sz, sz, sz, sz,
                                         vp]),
    # EFLA, query readout
    "efla_chunk_fwd_workspace_size": (sz, [sz, sz, sz, sz, sz, sz, i32]),
    "efla_chunk_bwd_workspace_size": (sz, [sz, sz, sz, sz, sz, sz, i32]),
    "efla_chunk_fwd_hip": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, sz, sz, sz,
                                 i32, vp, sz, ctypes.c_uint, vp]),
    "efla_chunk_bwd_hip": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, sz,
                                 sz, sz, sz, sz, sz, i32, vp, sz, ctypes.c_uint, vp]),
    "efla_chunk_fwd_noalloc_hip": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, sz,
                                         sz, sz, i32, vp]),
    "efla_chunk_fwd_strided_hip": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, sz,
                                         sz, sz, i32, vp, sz, ctypes.c_uint, vp, vp]),
    "efla_chunk_bwd_strided_hip": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                         sz, sz, sz, sz, sz, sz, sz, i32, vp, sz,
                                         ctypes.c_uint, vp, vp]),
    # LayerNorm
    "layernorm_forward_hip": (i32, [vp, vp, vp, vp, sz, sz, f32, vp]),
    "layernorm_forward_stats_hip": (i32, [vp, vp, vp, vp, vp, vp, sz, sz, f32, vp]),
    "layernorm_backward_hip": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, vp]),
    "layernorm_backward_residual_hip": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, vp]),
    "layernorm_backward_ex_hip": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, i32, vp]),
    "rmsnorm_forward_hip": (i32, [vp, vp, vp, sz, sz, f32, vp]),
    "rmsnorm_backward_hip": (i32, [vp, vp, vp, vp, vp, sz, sz, f32, vp]),
    "shortconv_forward_hip": (i32, [vp, vp, vp, sz, sz, sz, sz, vp]),
    "shortconv_backward_hip": (i32, [vp, vp, vp, vp, vp, sz, sz, sz, sz, vp]),
    "prism_forward_hip": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, sz, f32, vp]),
    "prism_backward_hip": (i32, [vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, sz, sz, vp]),
    # GEMM
    "gemm_forward_hip": (i32, [vp, vp, vp, vp, sz, sz, sz, i32, i32, i32, vp]),
    "gemm_backward_hip": (i32, [vp, vp, vp, vp, vp, vp, sz, sz, sz, vp]),
    "gemm_gelu_forward_hip": (i32, [vp, vp, vp, vp, vp, sz, sz, sz, vp]),
    "gemm_gelu_backward_hip": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, sz, sz, sz, vp]),
    # GELU, AdamW
    "gemm_ex_hip": (i32, [i32, i32, sz, sz, sz, f32, vp, sz, vp, sz, vp, f32, vp, sz, vp, sz,
                          i32, vp]),
    "gelu_forward_hip": (i32, [vp, vp, sz, ctypes.c_bool, vp]),
    "gelu_backward_hip": (i32, [vp, vp, vp, sz, ctypes.c_bool, vp]),
    "sigmoid_gate_forward_hip": (i32, [vp, sz, vp, sz, sz, vp]),
    "sigmoid_gate_backward_hip": (i32, [vp, vp, vp, sz, sz, sz, vp]),
    "adamw_step_hip": (i32, [vp, vp, vp, vp, sz, f32, f32, f32, f32, f32, sz, vp]),
    "adamw_step_master_hip": (i32, [vp, vp, vp, vp, vp, sz, f32, f32, f32, f32, f32, sz, vp]),
    # embedding, cross-entropy
    "embedding_forward_hip": (i32, [vp, vp, vp, sz, sz, vp]),
    "embedding_forward_checked_hip": (i32, [vp, vp, vp, sz, sz, sz, vp]),
    "embedding_backward_hip": (i32, [vp, vp, vp, sz, sz, sz, vp]),
    "cross_entropy_forward_hip": (i32, [vp, vp, vp, sz, sz, f32, vp]),
    "cross_entropy_backward_hip": (i32, [vp, vp, vp, vp, sz, sz, f32, vp]),
    "cross_entropy_forward_backward_hip": (i32, [vp, vp, vp, vp, vp, sz, sz, f32, vp]),
    # sequence packing (host)
    "efla_pack_sequences": (i32, [vp, vp, sz, sz, vp, vp, vp, vp, ctypes.POINTER(sz),
                                  ctypes.POINTER(sz)]),
    # runtime
    "efla_rt_device_count": (i32, [ctypes.POINTER(i32)]),
    "efla_rt_set_device": (i32, [i32]),
    "efla_rt_get_device": (i32, [ctypes.POINTER(i32)]),
    "efla_rt_device_synchronize": (i32, []),
    "efla_rt_device_info": (i32, [i32, ctypes.c_char_p, sz, ctypes.POINTER(i32),
                                  ctypes.POINTER(i32), ctypes.POINTER(sz), ctypes.POINTER(i32),
                                  ctypes.POINTER(i32)]),
    "efla_rt_malloc": (i32, [ctypes.POINTER(vp), sz]),
    "efla_rt_free": (i32, [vp]),
    "efla_rt_host_malloc": (i32, [ctypes.POINTER(vp), sz]),
    "efla_rt_host_free": (i32, [vp]),
    "efla_rt_memcpy": (i32, [vp, vp, sz, i32]),
    "efla_rt_memcpy_async": (i32, [vp, vp, sz, i32, vp]),
    "efla_rt_mem_get_info": (i32, [ctypes.POINTER(sz), ctypes.POINTER(sz)]),
    "efla_rt_fill": (i32, [vp, f32, sz, i32, vp]),
    "efla_rt_set_gemm_backend": (i32, [i32]),
    "efla_rt_stream_create": (i32, [ctypes.POINTER(vp)]),
    "efla_rt_stream_destroy": (i32, [vp]),
    "efla_rt_stream_synchronize": (i32, [vp]),
    "efla_rt_event_create": (i32, [ctypes.POINTER(vp)]),
    "efla_rt_event_destroy": (i32, [vp]),
    "efla_rt_event_record": (i32, [vp, vp]),
    "efla_rt_event_synchronize": (i32, [vp]),
    "efla_rt_event_elapsed_ms": (i32, [ctypes.POINTER(f32), vp, vp]),
    "efla_rt_workspace_bytes": (sz, []),
    "efla_rt_workspace_release": (i32, []),
    "efla_rt_workspace_release_stream": (i32, [vp]),
    "efla_prof_enable": (None, [i32]),
    "efla_prof_reset": (None, []),
    "efla_prof_collect": (i32, []),
    "efla_prof_count": (i32, []),
    "efla_prof_entry": (i32, [i32, ctypes.c_char_p, sz, ctypes.POINTER(ctypes.c_longlong),
                              ctypes.POINTER(ctypes.c_double)]),
}


def lib():
    """The loaded library; raises if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build the HIP library first "
            "(python -c 'import __graft_entry__ as g; g.build()')")
    L = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = L
    return L


def check(rc: int, where: str) -> None:
    if rc != 0:
        raise HipError(rc, where)
