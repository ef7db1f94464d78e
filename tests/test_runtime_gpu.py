"""The HIP device layer (include/efla_runtime.h) that replaces the reference's
CUDA runtime bindings (src/runtime/cuda.zig: cudart externs 140-172,
CudaStream 291-314, CudaEvent 317-351, CudaDevice 354-402, the cudaMalloc
helper 461-467 and the no-op cudaFill stub 490-496), called through the C
ABI on the GPU."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import announce

pytestmark = pytest.mark.gpu

H2H, H2D, D2H, D2D, DEFAULT = 0, 1, 2, 3, 4


@pytest.fixture(scope="module")
def L():
    from ceo_amd import _lib

    torch.cuda.init()
    return _lib.lib()


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def test_device_queries(L):
    announce("runtime: device count / set / get / info / mem info")
    n = ctypes.c_int()
    assert L.efla_rt_device_count(ctypes.byref(n)) == 0 and n.value >= 1
    assert L.efla_rt_set_device(0) == 0
    d = ctypes.c_int(-1)
    assert L.efla_rt_get_device(ctypes.byref(d)) == 0 and d.value == 0
    name = ctypes.create_string_buffer(64)
    cu, clk, lds, ws = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    mem = ctypes.c_size_t()
    assert L.efla_rt_device_info(0, name, 64, ctypes.byref(cu), ctypes.byref(clk),
                                 ctypes.byref(mem), ctypes.byref(lds), ctypes.byref(ws)) == 0
    print(f"  {name.value.decode()} cus={cu.value} clock={clk.value} kHz mem={mem.value} "
          f"lds/block={lds.value} wave={ws.value}", flush=True)
    assert name.value.decode().startswith("gfx950")
    assert cu.value == torch.cuda.get_device_properties(0).multi_processor_count
    assert ws.value == 64 and lds.value >= 65536 and mem.value > (200 << 30)
    # every output pointer may be NULL
    assert L.efla_rt_device_info(0, None, 0, None, None, None, None, None) == 0
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert L.efla_rt_mem_get_info(ctypes.byref(free), ctypes.byref(total)) == 0
    assert 0 < free.value <= total.value and total.value == mem.value


@pytest.mark.parametrize("dtype,code", [(torch.float32, 0), (torch.float16, 2),
                                        (torch.bfloat16, 14)])
def test_fill(L, dtype, code):
    """fill writes exactly numel elements of value (rounded like torch's cast)
    and nothing around them, at odd sizes and at offsets that break 4- and
    16-byte alignment."""
    announce(f"runtime: fill {dtype}")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for n in (1, 3, 255, 257, 65537, 1000003):
        for off in (0, 1, 3):
            for value in (1.5, 0.1, -3.0e5):
                buf = torch.full((n + off + 2,), -7.0, dtype=dtype, device="cuda:0")
                view = buf[off + 1:]
                assert L.efla_rt_fill(_ptr(view), ctypes.c_float(value), n, code, stream) == 0
                torch.cuda.synchronize()
                want = torch.tensor(value, dtype=torch.float32).to(dtype)
                assert torch.equal(buf[off + 1:off + 1 + n], want.expand(n).to("cuda:0")), (n, off)
                assert (buf[:off + 1] == -7.0).all() and buf[-1] == -7.0, (n, off)
    # numel 0: nothing to do, any pointer
    assert L.efla_rt_fill(None, ctypes.c_float(1.0), 0, code, stream) == 0
    # NULL with elements, unknown dtype: InvalidValue, nothing launched
    assert L.efla_rt_fill(None, ctypes.c_float(1.0), 4, code, stream) == 1
    buf = torch.zeros(8, dtype=dtype, device="cuda:0")
    assert L.efla_rt_fill(_ptr(buf), ctypes.c_float(1.0), 8, 99, stream) == 1
    torch.cuda.synchronize()
    assert (buf == 0).all()


def test_malloc_memcpy_every_kind(L):
    announce("runtime: malloc / free / memcpy kinds / pinned host memory")
    n = 1 << 20
    src = (np.arange(n, dtype=np.uint32) * 2654435761).astype(np.uint32)
    dev_a, dev_b = ctypes.c_void_p(), ctypes.c_void_p()
    assert L.efla_rt_malloc(ctypes.byref(dev_a), n * 4) == 0 and dev_a.value
    assert L.efla_rt_malloc(ctypes.byref(dev_b), n * 4) == 0 and dev_b.value
    pinned = ctypes.c_void_p()
    assert L.efla_rt_host_malloc(ctypes.byref(pinned), n * 4) == 0 and pinned.value
    try:
        host = np.zeros(n, dtype=np.uint32)
        hp = src.ctypes.data_as(ctypes.c_void_p)
        outp = host.ctypes.data_as(ctypes.c_void_p)
        pin = np.ctypeslib.as_array((ctypes.c_uint32 * n).from_address(pinned.value))
        # host -> pinned host (H2H), pinned -> device (H2D), device -> device,
        # device -> pageable host (D2H)
        assert L.efla_rt_memcpy(pinned, hp, n * 4, H2H) == 0
        assert np.array_equal(pin, src)
        assert L.efla_rt_memcpy(dev_a, pinned, n * 4, H2D) == 0
        assert L.efla_rt_memcpy(dev_b, dev_a, n * 4, D2D) == 0
        assert L.efla_rt_memcpy(outp, dev_b, n * 4, D2H) == 0
        assert np.array_equal(host, src)
        # kind 4 (default): the runtime infers the direction from the pointers
        pin[:] = 0
        assert L.efla_rt_memcpy(pinned, dev_b, n * 4, DEFAULT) == 0
        assert np.array_equal(pin, src)
        # async copies on a library-created stream
        s = ctypes.c_void_p()
        assert L.efla_rt_stream_create(ctypes.byref(s)) == 0
        try:
            pin[:] = 0
            assert L.efla_rt_memcpy_async(dev_a, outp, n * 4, H2D, s) == 0  # same data
            assert L.efla_rt_fill(dev_b, ctypes.c_float(0.0), n, 0, s) == 0
            assert L.efla_rt_memcpy_async(dev_b, dev_a, n * 4, D2D, s) == 0
            assert L.efla_rt_memcpy_async(pinned, dev_b, n * 4, D2H, s) == 0
            assert L.efla_rt_stream_synchronize(s) == 0
            assert np.array_equal(pin, src)
        finally:
            assert L.efla_rt_stream_destroy(s) == 0
    finally:
        assert L.efla_rt_host_free(pinned) == 0
        assert L.efla_rt_free(dev_a) == 0
        assert L.efla_rt_free(dev_b) == 0
    assert L.efla_rt_free(None) == 0  # as cudaFree(NULL)


def test_streams_and_events(L):
    announce("runtime: stream / event create, record, synchronize, elapsed time")
    s = ctypes.c_void_p()
    e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
    assert L.efla_rt_stream_create(ctypes.byref(s)) == 0 and s.value
    assert L.efla_rt_event_create(ctypes.byref(e0)) == 0
    assert L.efla_rt_event_create(ctypes.byref(e1)) == 0
    buf = torch.empty(64 << 20, dtype=torch.float32, device="cuda:0")
    try:
        assert L.efla_rt_event_record(e0, s) == 0
        for _ in range(20):  # ~5 GB of stores: a measurable interval
            assert L.efla_rt_fill(_ptr(buf), ctypes.c_float(2.0), buf.numel(), 0, s) == 0
        assert L.efla_rt_event_record(e1, s) == 0
        assert L.efla_rt_event_synchronize(e1) == 0
        ms = ctypes.c_float(-1.0)
        assert L.efla_rt_event_elapsed_ms(ctypes.byref(ms), e0, e1) == 0
        print(f"  20 fills of 256 MiB: {ms.value:.3f} ms", flush=True)
        assert 0.0 < ms.value < 1000.0
        assert L.efla_rt_stream_synchronize(s) == 0
        assert L.efla_rt_device_synchronize() == 0
        assert bool((buf == 2.0).all())
    finally:
        assert L.efla_rt_event_destroy(e0) == 0
        assert L.efla_rt_event_destroy(e1) == 0
        assert L.efla_rt_stream_destroy(s) == 0


def test_workspace_bytes_and_release(L):
    from ceo_amd import efla, runtime

    announce("runtime: cached workspaces per stream, release")
    runtime.release_workspace()
    assert runtime.workspace_bytes() == 0
    g = torch.Generator(device="cuda:0").manual_seed(1)
    q = torch.randn(1, 256, 2, 64, generator=g, device="cuda:0").to(torch.bfloat16)
    beta = torch.rand(1, 256, 2, generator=g, device="cuda:0").to(torch.bfloat16)
    efla.chunk_efla_fwd(q, q, q, beta)  # NULL workspace: the current stream's cached one
    torch.cuda.synchronize()
    one = runtime.workspace_bytes()
    assert one > 0
    s2 = torch.cuda.Stream()
    with torch.cuda.stream(s2):
        efla.chunk_efla_fwd(q, q, q, beta)
    torch.cuda.synchronize()
    assert runtime.workspace_bytes() == 2 * one  # a second stream gets its own buffer
    runtime.release_workspace()
    assert runtime.workspace_bytes() == 0


def test_workspace_released_with_its_stream(L):
    """Four library streams each run the reference ABI's forward at the bench
    shape (B H = 128 takes the column split: one zeroed fp32 row-sum buffer,
    4 bytes per output element, after the per-token coefficients) and a
    chunked forward; destroying each stream through efla_rt_stream_destroy
    frees its cached buffers, and the device's total returns to zero."""
    from ceo_amd import efla, runtime

    announce("runtime: per-stream workspaces freed by efla_rt_stream_destroy")
    runtime.release_workspace()
    assert runtime.workspace_bytes() == 0
    B, T, H, d = 4, 8192, 32, 128
    g = torch.Generator(device="cuda:0").manual_seed(2)
    k = (0.08 * torch.randn(B, T, H, d, generator=g, device="cuda:0")).to(torch.bfloat16)
    v = torch.randn(B, T, H, d, generator=g, device="cuda:0").to(torch.bfloat16)
    q = torch.randn(1, 256, 2, 64, generator=g, device="cuda:0").to(torch.bfloat16)
    beta = torch.rand(1, 256, 2, generator=g, device="cuda:0").to(torch.bfloat16)
    states = [torch.zeros(B * H, d, d, dtype=torch.bfloat16, device="cuda:0") for _ in range(4)]
    ref_state = states[0].clone()
    ref_o = efla.efla_forward(k, v, ref_state, 0.5)
    torch.cuda.synchronize()
    runtime.release_workspace()
    ntok, elems = B * T * H, B * T * H * d
    step = 64 << 20
    bound = -(-(ntok * 4 + 256 + elems * 4) // step) * step  # the 64 MiB growth step
    streams, outs, totals = [], [], []
    try:
        for i in range(4):
            s = ctypes.c_void_p()
            assert L.efla_rt_stream_create(ctypes.byref(s)) == 0
            streams.append(s)
            with torch.cuda.stream(torch.cuda.ExternalStream(s.value)):
                outs.append(efla.efla_forward(k, v, states[i], 0.5))
                efla.chunk_efla_fwd(q, q, q, beta)
            assert L.efla_rt_stream_synchronize(s) == 0
            totals.append(runtime.workspace_bytes())
        per = [totals[0]] + [b - a for a, b in zip(totals, totals[1:])]
        print(f"  per-stream cached bytes {per}, Mode R bound {bound}", flush=True)
        assert all(p == per[0] for p in per)
        # the chunked forward reuses the stream's (larger) Mode R buffer
        assert per[0] <= bound
        for o, st in zip(outs, states):  # the same bits on every stream
            assert torch.equal(o, ref_o) and torch.equal(st, ref_state)
    finally:
        outs.clear()
        torch.cuda.synchronize()
        left = []
        for s in streams:
            left.append((L.efla_rt_stream_destroy(s), runtime.workspace_bytes()))
    print(f"  after each destroy: {left}", flush=True)
    assert all(rc == 0 for rc, _ in left)
    assert [b for _, b in left] == [(3 - j) * totals[0] for j in range(4)]
    assert runtime.workspace_bytes() == 0
