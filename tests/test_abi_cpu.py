"""The C ABI without a GPU: the library loads, exports every symbol the public
headers declare, and rejects bad arguments before touching a device, with the
reference's codes (0 success, 1 invalid value, 9 invalid configuration)."""
import ctypes

import pytest

from ceo_amd import _lib

NULL = None


@pytest.fixture(scope="module")
def L():
    return _lib.lib()


def test_exports_every_declared_symbol(L):
    names = _lib.header_functions()
    assert len(names) >= 40
    for n in names:
        assert hasattr(L, n), n
        assert n in _lib._SIGS, f"{n} has no ctypes signature"


def test_efla_forward_validation_order(L):
    p = ctypes.c_void_p(16)
    # B, H or d == 0 -> InvalidValue, before the T == 0 early return (efla.cu:497-502)
    assert L.efla_forward_hip(p, p, p, p, 0, 0, 1, 1, 1.0, 64, NULL) == 1
    assert L.efla_forward_hip(p, p, p, p, 1, 4, 0, 1, 1.0, 64, NULL) == 1
    assert L.efla_forward_hip(p, p, p, p, 1, 4, 1, 0, 1.0, 64, NULL) == 1
    # T == 0 -> success even with null pointers
    assert L.efla_forward_hip(NULL, NULL, NULL, NULL, 1, 0, 1, 1, 1.0, 64, NULL) == 0
    assert L.efla_forward_hip(p, NULL, p, p, 1, 1, 1, 1, 1.0, 64, NULL) == 1
    # B*H beyond the 32-bit grid -> InvalidConfiguration (efla.cu:507-513)
    assert L.efla_forward_hip(p, p, p, p, 1 << 31, 1, 4, 1, 1.0, 64, NULL) == 9


def test_efla_backward_validation_order(L):
    p = ctypes.c_void_p(16)
    assert L.efla_backward_hip(p, p, p, p, p, p, p, 0, 1, 1, 1, 1.0, NULL) == 1
    assert L.efla_backward_hip(p, p, p, NULL, p, p, p, 1, 1, 1, 1, 1.0, NULL) == 1
    assert L.efla_backward_hip(p, p, p, p, p, p, NULL, 1, 1, 1, 1, 1.0, NULL) == 1
    assert L.efla_backward_hip(NULL, p, p, p, p, p, p, 1, 1, 1, 2, 1.0, NULL) == 1
    assert L.efla_backward_hip(p, p, p, p, p, p, p, 1 << 31, 1, 4, 1, 1.0, NULL) == 9


def test_efla_chunked_scan_validation(L):
    arr = (ctypes.c_void_p * 2)(16, None)
    assert L.efla_chunked_scan_hip(arr, 0, 1, 1, NULL) == 1
    assert L.efla_chunked_scan_hip(arr, 2, 0, 1, NULL) == 1
    assert L.efla_chunked_scan_hip(NULL, 2, 1, 1, NULL) == 1
    assert L.efla_chunked_scan_hip(arr, 2, 1, 4, NULL) == 1  # a null chunk
    one = (ctypes.c_void_p * 1)(16)
    assert L.efla_chunked_scan_hip(one, 1, 1, 4, NULL) == 0  # nothing to add


def _fwd(L, **kw):
    a = dict(q=16, k=16, v=16, beta=16, s0=None, o=16, st=None, cu=None, B=2, T=128, N=0,
             H=2, K=64, V=64, C=64, dt=14, ws=None, wsb=0, flags=0)
    a.update(kw)
    vp = ctypes.c_void_p
    return L.efla_chunk_fwd_hip(vp(a["q"]), vp(a["k"]), vp(a["v"]), vp(a["beta"]), a["s0"],
                                vp(a["o"]) if a["o"] else None, a["st"], a["cu"], a["B"], a["T"],
                                a["N"], a["H"], a["K"], a["V"], a["C"], a["dt"], a["ws"],
                                a["wsb"], a["flags"], None)


def test_chunk_fwd_validation(L):
    assert _fwd(L, H=0) == 1
    assert _fwd(L, K=0) == 1
    assert _fwd(L, C=32) == 1          # only 64-token chunks
    assert _fwd(L, K=96) == 1          # unsupported head dim
    assert _fwd(L, dt=0, K=128) == 1   # fp32 only at 64 x 64
    assert _fwd(L, dt=2) == 1          # fp16 not supported
    assert _fwd(L, B=0) == 1
    assert _fwd(L, N=3) == 1           # num_seqs must match batch without cu_seqlens
    assert _fwd(L, cu=ctypes.c_void_p(16), B=2, N=2) == 1  # packed input has batch 1
    assert _fwd(L, T=0) == 0           # nothing to do, no final state requested
    assert _fwd(L, q=0) == 1
    assert _fwd(L, o=0) == 1
    assert _fwd(L, ws=ctypes.c_void_p(256), wsb=16) == 1   # workspace too small


def _bwd(L, flags=0, ws=None, wsb=0, T=128, **kw):
    vp = ctypes.c_void_p
    p = vp(16)
    return L.efla_chunk_bwd_hip(p, p, p, p, None, p, None, p, p, p, p, None, None, 2, T, 0, 2,
                                64, 64, 64, 14, ws, wsb, flags, None)


def test_chunk_bwd_flags(L):
    # unknown flag bits, and reusing the forward's factors without a workspace
    assert _bwd(L, flags=2) == 1
    assert _bwd(L, flags=1) == 1
    assert _bwd(L, flags=1, ws=ctypes.c_void_p(256), wsb=16) == 1  # workspace too small
    assert _bwd(L, flags=1, T=0) == 1   # flags are checked before the empty case
    assert _bwd(L, flags=0, T=0) == 0
    assert _bwd(L, flags=4) == 1
    assert _bwd(L, flags=3) == 1        # no workspace
    # saved states without the factors
    assert _bwd(L, flags=2, ws=ctypes.c_void_p(256), wsb=1 << 40) == 1


def test_chunk_fwd_flags(L):
    assert _fwd(L, flags=2) == 1        # unknown bit
    assert _fwd(L, flags=1) == 1        # saving states needs a caller workspace
    # the fwd-sized workspace has no room for the states
    fw = L.efla_chunk_fwd_workspace_size(2, 128, 0, 2, 64, 64, 14)
    assert _fwd(L, flags=1, ws=ctypes.c_void_p(256), wsb=fw) == 1
    assert _fwd(L, flags=1, T=0) == 1   # flags are checked before the empty case


def _fwd_strided(L, strides, q=16, B=2, T=128, dt=14):
    vp = ctypes.c_void_p
    arr = None if strides is None else (ctypes.c_int64 * 3)(*strides)
    return L.efla_chunk_fwd_strided_hip(vp(q), vp(16), vp(16), vp(16), None, vp(16), None, None,
                                        B, T, 0, 2, 64, 64, 64, dt, None, 0, 0, arr, None)


def test_chunk_fwd_strided_validation(L):
    # H = 2, d = 64: the packed token stride is 128 elements
    assert _fwd_strided(L, [120, 128, 128]) == 1           # below the packed row
    assert _fwd_strided(L, [132, 128, 128]) == 1           # not whole 16-byte pieces
    assert _fwd_strided(L, [1 << 24, 128, 128]) == 1       # beyond 32-bit chunk offsets
    assert _fwd_strided(L, [136, 128, 128], q=24) == 1     # pointer not 16-byte aligned
    assert _fwd_strided(L, [128, 128, 128], q=24, T=0) == 0  # packed: no alignment rule
    assert _fwd_strided(L, [136, 128, 128], dt=0) == 801   # fp32 path: packed only
    assert _fwd_strided(L, [128, 128, 128], dt=0, T=0) == 0
    assert _fwd_strided(L, [136, 256, 1000], T=0) == 0     # valid, nothing to do
    assert _fwd_strided(L, None, T=0) == 0                 # NULL: packed
    # the whole strided extent beyond 2^46 elements
    assert _fwd_strided(L, [1 << 17, 128, 128], B=1 << 22, T=256) == 9


def _bwd_strided(L, strides, dq=16, dt=14, T=128):
    vp = ctypes.c_void_p
    p = vp(16)
    arr = (ctypes.c_int64 * 6)(*strides)
    return L.efla_chunk_bwd_strided_hip(p, p, p, p, None, p, None, vp(dq), p, p, p, None, None,
                                        2, T, 0, 2, 64, 64, 64, dt, None, 0, 0, arr, None)


def test_chunk_bwd_strided_validation(L):
    packed = [128] * 6
    assert _bwd_strided(L, packed, T=0) == 0
    assert _bwd_strided(L, [128, 128, 128, 120, 128, 128]) == 1   # gradient rows overlap
    assert _bwd_strided(L, [128, 128, 128, 128, 128, 140]) == 1
    assert _bwd_strided(L, [128, 128, 128, 392, 392, 392], dq=40) == 1
    assert _bwd_strided(L, [392] * 6, dt=0) == 801
    assert _bwd_strided(L, [392] * 6, T=0) == 0


def test_sigmoid_gate_validation(L):
    p = ctypes.c_void_p(16)
    assert L.sigmoid_gate_forward_hip(p, 64, p, 0, 16, NULL) == 0      # nothing to do
    assert L.sigmoid_gate_forward_hip(NULL, 64, p, 4, 16, NULL) == 1
    assert L.sigmoid_gate_forward_hip(p, 8, p, 4, 16, NULL) == 1       # ld < cols
    assert L.sigmoid_gate_forward_hip(p, 1 << 24, p, 4, 16, NULL) == 9
    assert L.sigmoid_gate_backward_hip(p, p, p, 64, 4, 0, NULL) == 0
    assert L.sigmoid_gate_backward_hip(p, NULL, p, 64, 4, 16, NULL) == 1
    assert L.sigmoid_gate_backward_hip(p, p, p, 15, 4, 16, NULL) == 1


def test_workspace_sizes(L):
    f = L.efla_chunk_fwd_workspace_size
    b = L.efla_chunk_bwd_workspace_size
    # cfg3: B=4, T=8192, H=32, K=V=128 bf16
    fw = f(4, 8192, 0, 32, 128, 128, 14)
    bw = b(4, 8192, 0, 32, 128, 128, 14)
    slots, H = 4 * 8192 // 64, 32
    t_bytes = slots * H * (10 * 256 + 32) * 2  # bf16 T per chunk: ten lower 16x16 tiles
    state_bytes = slots * H * 128 * 128 * 2  # bf16 chunk states
    assert fw >= t_bytes
    assert fw < t_bytes + state_bytes        # no states unless asked for
    assert bw >= fw + 2 * state_bytes        # h and dh
    assert bw < fw + 2 * state_bytes + 2 * t_bytes  # P packed as T is
    assert bw < 16 * 2**30                   # fits comfortably in 288 GB
    assert f(4, 8192, 0, 32, 96, 128, 14) == 0
    assert f(1, 65536, 40, 16, 128, 256, 14) > 0   # packed, cfg5 shape


def test_gemm_validation(L):
    p = ctypes.c_void_p(16)
    assert L.gemm_forward_hip(NULL, p, NULL, p, 4, 4, 4, 14, 14, 14, NULL) == 1
    assert L.gemm_forward_hip(p, p, NULL, p, 4, 4, 4, 14, 14, 99, NULL) == 1
    assert L.gemm_forward_hip(p, p, NULL, p, 0, 4, 4, 14, 14, 14, NULL) == 0
    assert L.gemm_backward_hip(p, p, p, NULL, NULL, NULL, 4, 4, 4, NULL) == 0
    assert L.gemm_backward_hip(NULL, p, p, p, NULL, NULL, 4, 4, 4, NULL) == 1
    # column sums of grad_pre need grad_pre; grad_pre needs grad_c, b and pre
    assert L.gemm_gelu_backward_hip(p, p, p, p, NULL, NULL, NULL, p, 4, 4, 4, NULL) == 1
    assert L.gemm_gelu_backward_hip(NULL, p, p, p, p, NULL, NULL, p, 4, 4, 4, NULL) == 1
    assert L.gemm_gelu_backward_hip(p, p, p, NULL, p, NULL, NULL, NULL, 4, 4, 4, NULL) == 1


def test_layernorm_validation(L):
    p = ctypes.c_void_p(16)
    assert L.layernorm_forward_hip(p, p, NULL, p, 1024, 0, 1e-5, NULL) == 1
    assert L.layernorm_forward_hip(p, p, NULL, p, 0, 1024, 1e-5, NULL) == 0
    assert L.layernorm_forward_hip(NULL, p, NULL, p, 2048, 1024, 1e-5, NULL) == 1
    assert L.layernorm_forward_stats_hip(p, p, NULL, p, NULL, p, 2048, 1024, 1e-5, NULL) == 1
    # the _ex backward: D == 0 or a NULL operand -> 1; column sums past 8192 columns -> 9
    ex = L.layernorm_backward_ex_hip
    assert ex(p, p, p, p, p, NULL, p, NULL, NULL, p, 1024, 0, 0, NULL) == 1
    assert ex(p, p, p, p, p, NULL, NULL, NULL, NULL, p, 2048, 1024, 0, NULL) == 1
    assert ex(p, NULL, p, p, p, NULL, p, NULL, NULL, p, 2048, 1024, 1, NULL) == 1
    assert ex(p, p, p, p, p, NULL, p, NULL, NULL, p, 32768, 16384, 0, NULL) == 9
    assert ex(p, p, p, p, p, NULL, p, p, p, NULL, 32768, 16384, 1, NULL) == 9


def test_rmsnorm_validation(L):
    p = ctypes.c_void_p(16)
    assert L.rmsnorm_forward_hip(p, p, p, 1024, 0, 1e-6, NULL) == 1
    assert L.rmsnorm_forward_hip(p, p, p, 1000, 1024, 1e-6, NULL) == 0
    assert L.rmsnorm_forward_hip(NULL, p, p, 2048, 1024, 1e-6, NULL) == 1
    assert L.rmsnorm_backward_hip(p, p, p, p, NULL, 1024, 0, 1e-6, NULL) == 1
    assert L.rmsnorm_backward_hip(p, p, p, p, NULL, 0, 64, 1e-6, NULL) == 0
    assert L.rmsnorm_backward_hip(p, NULL, p, p, NULL, 128, 64, 1e-6, NULL) == 1
    assert L.rmsnorm_backward_hip(p, p, p, p, p, 32768, 32768, 1e-6, NULL) == 9


def test_shortconv_and_prism_validation(L):
    p = ctypes.c_void_p(16)
    # ShortConv: nothing to do -> 0; NULL -> 1; window beyond the limits -> 9
    assert L.shortconv_forward_hip(p, p, p, 0, 8, 8, 4, NULL) == 0
    assert L.shortconv_forward_hip(NULL, p, p, 1, 8, 8, 4, NULL) == 1
    assert L.shortconv_forward_hip(p, NULL, p, 1, 8, 8, 4, NULL) == 1
    assert L.shortconv_forward_hip(p, p, p, 1, 8, 8, 1 << 21, NULL) == 9
    assert L.shortconv_backward_hip(NULL, p, p, p, NULL, 1, 8, 8, 4, NULL) == 1
    assert L.shortconv_backward_hip(p, NULL, p, p, p, 1, 8, 8, 4, NULL) == 1
    assert L.shortconv_backward_hip(p, p, p, p, NULL, 0, 8, 8, 4, NULL) == 0
    # PRISM: head_dim 0 or above hidden_dim -> 1; > 16 iterations -> 9
    wp = (ctypes.c_void_p * 17)(*([16] * 17))
    assert L.prism_forward_hip(p, p, NULL, NULL, p, NULL, NULL, wp, 1, 4, 64, 0, 3, 0.99,
                               NULL) == 1
    assert L.prism_forward_hip(p, p, NULL, NULL, p, NULL, NULL, wp, 1, 4, 64, 65, 3, 0.99,
                               NULL) == 1
    assert L.prism_forward_hip(p, p, NULL, NULL, p, NULL, NULL, wp, 1, 4, 64, 64, 17, 0.99,
                               NULL) == 9
    assert L.prism_forward_hip(p, p, NULL, NULL, p, NULL, NULL, NULL, 1, 4, 64, 64, 3, 0.99,
                               NULL) == 1
    assert L.prism_forward_hip(NULL, p, NULL, NULL, p, NULL, NULL, wp, 1, 4, 64, 64, 3, 0.99,
                               NULL) == 1
    wnull = (ctypes.c_void_p * 3)(16, None, 16)
    assert L.prism_forward_hip(p, p, NULL, NULL, p, NULL, NULL, wnull, 1, 4, 64, 64, 3, 0.99,
                               NULL) == 1
    assert L.prism_forward_hip(p, p, NULL, NULL, p, NULL, NULL, wp, 0, 4, 64, 64, 3, 0.99,
                               NULL) == 0
    assert L.prism_backward_hip(p, p, p, wp, p, p, NULL, 1, 4, 64, 64, 17, NULL) == 9
    assert L.prism_backward_hip(p, p, p, wp, NULL, p, NULL, 1, 4, 64, 64, 3, NULL) == 1
    gnull = (ctypes.c_void_p * 3)(16, None, 16)
    assert L.prism_backward_hip(p, p, p, wp, p, p, gnull, 1, 4, 64, 64, 3, NULL) == 1


def test_gemm_ex_and_residual_validation(L):
    p = ctypes.c_void_p(16)
    bf = 14
    # m or n == 0 -> 0; bad transpose flag, short strides, NULL -> 1
    assert L.gemm_ex_hip(0, 0, 0, 8, 8, 1.0, p, 8, p, 8, NULL, 0.0, NULL, 0, p, 8, bf, NULL) == 0
    assert L.gemm_ex_hip(2, 0, 8, 8, 8, 1.0, p, 8, p, 8, NULL, 0.0, NULL, 0, p, 8, bf, NULL) == 1
    assert L.gemm_ex_hip(0, 0, 8, 8, 8, 1.0, p, 4, p, 8, NULL, 0.0, NULL, 0, p, 8, bf, NULL) == 1
    assert L.gemm_ex_hip(0, 0, 8, 8, 8, 1.0, p, 8, p, 8, NULL, 0.0, NULL, 0, p, 4, bf, NULL) == 1
    assert L.gemm_ex_hip(0, 0, 8, 8, 8, 1.0, p, 8, p, 8, NULL, 1.0, NULL, 8, p, 8, bf, NULL) == 1
    # k == 0 reads neither operand, but D's stride is still checked
    assert L.gemm_ex_hip(0, 0, 8, 8, 0, 1.0, NULL, 0, NULL, 0, NULL, 0.0, NULL, 0, p, 4, bf,
                         NULL) == 1
    assert L.layernorm_backward_residual_hip(p, p, p, p, p, NULL, p, NULL, NULL, 2048, 1024,
                                             NULL) == 1


def test_gelu_validation(L):
    p = ctypes.c_void_p(16)
    # numel == 0: the reference launches an empty grid -> InvalidConfiguration
    assert L.gelu_forward_hip(p, p, 0, True, NULL) == 9
    assert L.gelu_backward_hip(p, p, p, 0, False, NULL) == 9
    assert L.gelu_forward_hip(NULL, p, 8, True, NULL) == 1
    assert L.gelu_backward_hip(p, NULL, p, 8, True, NULL) == 1


def test_adamw_validation(L):
    p = ctypes.c_void_p(16)
    ok = (3e-4, 0.9, 0.999, 1e-8, 0.1, 1)

    def bf(*hp, n=8, ptrs=(p, p, p, p)):
        return L.adamw_step_hip(*ptrs, n, *hp, NULL)

    def ms(*hp, n=8, ptrs=(p, p, p, p, NULL)):
        return L.adamw_step_master_hip(*ptrs, n, *hp, NULL)

    for fn in (bf, ms):
        # optim.cu:671-690: numel == 0 first, then nulls, then hyper-parameters
        assert fn(*ok, n=0, ptrs=(NULL,) * (4 if fn is bf else 5)) == 0
        assert fn(*ok, ptrs=(p, NULL, p, p) if fn is bf else (p, NULL, p, p, NULL)) == 1
        assert fn(float("nan"), 0.9, 0.999, 1e-8, 0.1, 1) == 1
        assert fn(3e-4, 1.0, 0.999, 1e-8, 0.1, 1) == 1      # beta1 >= 1
        assert fn(3e-4, 0.9, -0.1, 1e-8, 0.1, 1) == 1       # beta2 < 0
        assert fn(3e-4, 0.9, 0.999, 0.0, 0.1, 1) == 1       # eps <= 0
        assert fn(3e-4, 0.9, 0.999, 1e-8, float("inf"), 1) == 1
        assert fn(3e-4, 0.9, 0.999, 1e-8, 0.1, 0) == 1      # step == 0


def test_embedding_and_cross_entropy_validation(L):
    p = ctypes.c_void_p(16)
    assert L.embedding_forward_hip(p, p, p, 0, 8, NULL) == 0
    assert L.embedding_forward_hip(NULL, p, p, 4, 8, NULL) == 1
    assert L.embedding_forward_hip(p, p, p, 4, 0, NULL) == 1
    assert L.embedding_forward_checked_hip(p, p, p, 4, 0, 8, NULL) == 1   # empty table
    assert L.embedding_backward_hip(p, p, p, 0, 10, 8, NULL) == 0
    assert L.embedding_backward_hip(p, NULL, p, 4, 10, 8, NULL) == 1
    assert L.cross_entropy_forward_hip(p, p, p, 0, 100, 0.0, NULL) == 0
    assert L.cross_entropy_forward_hip(NULL, p, p, 4, 100, 0.0, NULL) == 1
    assert L.cross_entropy_forward_hip(p, p, p, 4, 0, 0.0, NULL) == 1
    assert L.cross_entropy_forward_hip(p, p, p, 4, 100, 1.0, NULL) == 1   # eps outside [0, 1)
    assert L.cross_entropy_forward_hip(p, p, NULL, 4, 100, 0.0, NULL) == 1
    assert L.cross_entropy_backward_hip(NULL, p, p, p, 4, 100, 0.0, NULL) == 1
    assert L.cross_entropy_backward_hip(p, p, p, p, 4, 100, float("nan"), NULL) == 1
    assert L.cross_entropy_forward_backward_hip(p, p, NULL, p, p, 0, 100, 0.0, NULL) == 0
    assert L.cross_entropy_forward_backward_hip(NULL, p, NULL, p, p, 4, 100, 0.0, NULL) == 1
    assert L.cross_entropy_forward_backward_hip(p, p, NULL, NULL, p, 4, 100, 0.0, NULL) == 1
    assert L.cross_entropy_forward_backward_hip(p, p, NULL, p, NULL, 4, 100, 0.0, NULL) == 1
    assert L.cross_entropy_forward_backward_hip(p, p, NULL, p, p, 4, 100, 1.0, NULL) == 1


def test_affine_state_scan_validation(L):
    p = ctypes.c_void_p(16)
    arr = (ctypes.c_void_p * 2)(p, p)
    assert L.efla_affine_state_scan_hip(arr, arr, 0, 4, 64, 64, NULL) == 1
    assert L.efla_affine_state_scan_hip(NULL, arr, 2, 4, 64, 64, NULL) == 1
    assert L.efla_affine_state_scan_hip(arr, arr, 2, 4, 0, 64, NULL) == 1
    assert L.efla_affine_state_scan_hip(arr, arr, 2, 4, 512, 64, NULL) == 9
    holes = (ctypes.c_void_p * 2)(p, None)
    assert L.efla_affine_state_scan_hip(arr, holes, 2, 4, 64, 64, NULL) == 1
    assert L.efla_affine_state_scan_hip(holes, arr, 2, 4, 64, 64, NULL) == 1
    assert L.efla_affine_state_scan_hip(arr, arr, 1, 4, 64, 64, NULL) == 0   # nothing to combine


def test_runtime_validation(L):
    """Argument checks of the device layer that run before any HIP call."""
    p = ctypes.c_void_p(16)
    f = ctypes.c_float(1.0)
    assert L.efla_rt_fill(NULL, f, 0, 0, NULL) == 0  # nothing to fill
    assert L.efla_rt_fill(NULL, f, 5, 14, NULL) == 1  # NULL with elements
    for dt in (1, 3, 99, -1):  # only fp32 (0), fp16 (2), bf16 (14)
        assert L.efla_rt_fill(p, f, 5, dt, NULL) == 1
    assert L.efla_rt_set_gemm_backend(2) == 1
    assert L.efla_rt_set_gemm_backend(-1) == 1
    assert L.efla_rt_set_gemm_backend(0) == 0


def test_chunk_fwd_noalloc_validation(L):
    """Argument checks and the scratch-size refusal come before any HIP call."""
    p = ctypes.c_void_p(16)

    def call(B=2, T=128, H=2, K=64, V=64, dt=14, q=p):
        return L.efla_chunk_fwd_noalloc_hip(q, p, p, p, NULL, p, NULL, NULL, B, T, 0, H, K, V,
                                            64, dt, NULL)
    assert call(H=0) == 1
    assert call(K=96) == 1  # no kernel for this head size
    assert call(q=NULL) == 1
    # forward workspace beyond EFLA_NOALLOC_SCRATCH_BYTES (64 MiB) -> 2
    assert call(B=8, T=8192, H=32, K=128, V=128) == 2
