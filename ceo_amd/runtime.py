"""HIP device layer helpers (include/efla_runtime.h) and the launch profiler."""
from __future__ import annotations

import ctypes

from ._lib import check, lib


def device_info(device: int = 0) -> dict:
    name = ctypes.create_string_buffer(128)
    cu, clk, lds, ws = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    mem = ctypes.c_size_t()
    check(lib().efla_rt_device_info(device, name, 128, ctypes.byref(cu), ctypes.byref(clk),
                                    ctypes.byref(mem), ctypes.byref(lds), ctypes.byref(ws)),
          "efla_rt_device_info")
    return {"arch": name.value.decode(), "compute_units": cu.value, "clock_khz": clk.value,
            "total_mem": mem.value, "lds_per_block": lds.value, "warp_size": ws.value}


class Profiler:
    """Per-kernel launch timing from hipEvents recorded on each launch's stream."""

    def __enter__(self):
        lib().efla_prof_reset()
        lib().efla_prof_enable(1)
        return self

    def __exit__(self, *exc):
        lib().efla_prof_enable(0)
        return False

    @staticmethod
    def results() -> dict:
        """{kernel name: (launches, total ms)}; waits for outstanding events."""
        check(lib().efla_prof_collect(), "efla_prof_collect")
        out = {}
        name = ctypes.create_string_buffer(256)
        n, ms = ctypes.c_longlong(), ctypes.c_double()
        for i in range(lib().efla_prof_count()):
            if lib().efla_prof_entry(i, name, 256, ctypes.byref(n), ctypes.byref(ms)) == 0:
                out[name.value.decode()] = (n.value, ms.value)
        return out


def workspace_bytes() -> int:
    return lib().efla_rt_workspace_bytes()


def release_workspace() -> None:
    check(lib().efla_rt_workspace_release(), "efla_rt_workspace_release")
