"""EFLA on MI355X: torch-facing wrappers over the C ABI.

Two families, mirroring the reference's kernel interface
(src/kernels/efla_kernels.zig:8-43, kernels/cuda/include/kernels.h:35-77):

* ``efla_forward`` / ``efla_backward`` / ``efla_chunked_scan`` -- the reference
  ABI (``eflaForwardCuda`` / ``eflaBackwardCuda`` / ``eflaChunkedScanCuda``):
  keys and values only, scalar beta, d_k == d_v, a bf16 (B*H, d, d) state
  updated in place, readout o_t = S_t k_t.
* ``chunk_efla_fwd`` / ``chunk_efla_bwd`` / ``chunk_efla`` -- the chunked
  query-readout form used by the benchmark configurations: q, per-token beta,
  d_k != d_v, optional fp32 initial / final state, varlen via ``cu_seqlens``.

Tensors are device tensors; torch only provides the memory and the current
stream.  Every call goes to libefla_hip.so and raises ``HipError`` on a
non-zero return code.
"""
from __future__ import annotations

import ctypes

import torch

from ._lib import check, lib

DTYPE_CODES = {torch.float32: 0, torch.float16: 2, torch.bfloat16: 14}


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _require(t, name, dtype=None, device=None, contiguous=True):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")


# ---------------------------------------------------------------------------
# reference ABI
# ---------------------------------------------------------------------------
def efla_forward(k: torch.Tensor, v: torch.Tensor, state: torch.Tensor, beta: float,
                 chunk_size: int = 64) -> torch.Tensor:
    """eflaForwardCuda: o_t = S_t k_t; ``state`` (B*H, d, d) bf16 is updated in place.

    ``chunk_size`` (ignored by the reference) is a tuning hint: for d = 64 / 128
    the number of tokens (16, 32 or 64) staged in LDS at once; the results do
    not depend on it."""
    B, T, H, d = k.shape
    for t, n in ((k, "k"), (v, "v"), (state, "state")):
        _require(t, n, torch.bfloat16, k.device)
    if v.shape != k.shape or state.shape != (B * H, d, d):
        raise ValueError("efla_forward: shapes must be k, v (B,T,H,d) and state (B*H,d,d)")
    out = torch.empty_like(k)
    rc = lib().efla_forward_hip(_p(k), _p(v), _p(state), _p(out), B, T, H, d, float(beta),
                                chunk_size, _stream(k))
    check(rc, "efla_forward_hip")
    return out


def efla_backward(grad_output: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                  state0: torch.Tensor, beta: float):
    """eflaBackwardCuda: (grad_k, grad_v, grad_state) for S_0 = ``state0``."""
    B, T, H, d = k.shape
    for t, n in ((grad_output, "grad_output"), (k, "k"), (v, "v"), (state0, "state")):
        _require(t, n, torch.bfloat16, k.device)
    gk = torch.empty_like(k)
    gv = torch.empty_like(v)
    gs = torch.empty_like(state0)
    rc = lib().efla_backward_hip(_p(grad_output), _p(k), _p(v), _p(state0), _p(gk), _p(gv),
                                 _p(gs), B, T, H, d, float(beta), _stream(k))
    check(rc, "efla_backward_hip")
    return gk, gv, gs


def efla_chunked_scan(chunk_states, num_heads: int, head_dim: int) -> None:
    """eflaChunkedScanCuda: in-place bf16 inclusive prefix sum over chunk states."""
    n = len(chunk_states)
    for i, t in enumerate(chunk_states):
        _require(t, f"chunk_states[{i}]", torch.bfloat16)
    arr = (ctypes.c_void_p * max(n, 1))(*[t.data_ptr() for t in chunk_states])
    st = _stream(chunk_states[0]) if n else None
    rc = lib().efla_chunked_scan_hip(arr, n, num_heads, head_dim, st)
    check(rc, "efla_chunked_scan_hip")


# ---------------------------------------------------------------------------
# chunked query readout
# ---------------------------------------------------------------------------
def token_stride(t: torch.Tensor, name: str = "tensor") -> int:
    """Elements from one token's row to the next of a (B, T, H, D) tensor whose
    heads are packed within each token row and whose batches follow each other
    (a contiguous tensor, or a column slice of a wider per-token row such as a
    fused projection, viewed as (B, T, H, D))."""
    B, T, H, D = t.shape
    if t.is_contiguous():
        return H * D
    s = t.stride()
    ts = s[1] if T > 1 else (s[0] if B > 1 else H * D)
    if s[3] != 1 or (H > 1 and s[2] != D) or (B > 1 and s[0] != T * ts):
        raise ValueError(f"{name} must be contiguous or a token-strided view "
                         "(heads packed within each token row)")
    return ts


def _q_shapes(q, k, v, beta, cu_seqlens):
    if q.dim() != 4 or k.shape != q.shape or v.dim() != 4 or v.shape[:3] != q.shape[:3]:
        raise ValueError("q, k must be (B,T,H,K) and v (B,T,H,V)")
    if beta.shape != q.shape[:3]:
        raise ValueError("beta must be (B,T,H)")
    dt = q.dtype
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _require(t, n, dt, q.device, contiguous=False)
    _require(beta, "beta", dt, q.device)
    if dt not in (torch.bfloat16, torch.float32):
        raise ValueError(f"unsupported dtype {dt}")
    B, T, H, K = q.shape
    V = v.shape[-1]
    if cu_seqlens is not None:
        _require(cu_seqlens, "cu_seqlens", torch.int32, q.device)
        if B != 1:
            raise ValueError("varlen inputs are packed with batch size 1")
        N = cu_seqlens.numel() - 1
    else:
        N = B
    return B, T, H, K, V, N, DTYPE_CODES[dt]


SAVE_STATES = 1  # EFLA_FWD_SAVE_STATES


def chunk_efla_fwd(q, k, v, beta, initial_state=None, output_final_state=False,
                   cu_seqlens=None, workspace=None, save_states=False):
    """Returns (o, final_state or None).

    With ``save_states`` the chunk start states (and, for bf16, each chunk's
    P = tril(Q K^T)) are also written into ``workspace`` (which must then be a
    backward-sized one, ``new_workspace``), for a backward call with
    ``reuse_states``."""
    if save_states and workspace is None:
        raise ValueError("save_states needs a caller workspace")
    B, T, H, K, V, N, dt = _q_shapes(q, k, v, beta, cu_seqlens)
    if initial_state is not None:
        _require(initial_state, "initial_state", torch.float32, q.device)
        if initial_state.shape != (N, H, K, V):
            raise ValueError("initial_state must be (N,H,K,V) fp32")
    o = torch.empty(B, T, H, V, dtype=q.dtype, device=q.device)
    st = torch.empty(N, H, K, V, dtype=torch.float32, device=q.device) \
        if output_final_state else None
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    args = (_p(q), _p(k), _p(v), _p(beta), _p(initial_state), _p(o), _p(st), _p(cu_seqlens),
            B, T, N if cu_seqlens is not None else 0, H, K, V, 64, dt, _p(workspace), ws_bytes,
            SAVE_STATES if save_states else 0)
    strides = [token_stride(t, n) for t, n in ((q, "q"), (k, "k"), (v, "v"))]
    if strides == [H * K, H * K, H * V]:
        rc = lib().efla_chunk_fwd_hip(*args, _stream(q))
        check(rc, "efla_chunk_fwd_hip")
    else:
        arr = (ctypes.c_int64 * 3)(*strides)
        rc = lib().efla_chunk_fwd_strided_hip(*args, arr, _stream(q))
        check(rc, "efla_chunk_fwd_strided_hip")
    return o, st


REUSE_FORWARD = 1  # EFLA_BWD_REUSE_FORWARD
REUSE_STATES = 2  # EFLA_BWD_REUSE_STATES


def chunk_efla_bwd(q, k, v, beta, do, initial_state=None, dht=None, cu_seqlens=None,
                   workspace=None, reuse_forward=False, reuse_states=False, grads_out=None):
    """Returns (dq, dk, dv, dbeta, dh0 or None).

    ``grads_out`` = (dq, dk, dv): tensors shaped like q, k, v to write the
    gradients into, which may be token-strided views (column slices of one
    fused gradient row); by default new contiguous tensors.

    With ``reuse_forward`` the ``workspace`` must be the one the forward call on
    the same inputs used (untouched since): the per-chunk WY factors are taken
    from it instead of being recomputed.  ``reuse_states`` (with
    ``reuse_forward``, after a forward with ``save_states``) takes the chunk
    states and P from it too."""
    if (reuse_forward or reuse_states) and workspace is None:
        raise ValueError("reuse_forward / reuse_states need the forward's workspace")
    if reuse_states and not reuse_forward:
        raise ValueError("reuse_states needs reuse_forward")
    B, T, H, K, V, N, dt = _q_shapes(q, k, v, beta, cu_seqlens)
    _require(do, "do", q.dtype, q.device)
    if do.shape != v.shape:
        raise ValueError("do must match v")
    for t, n in ((initial_state, "initial_state"), (dht, "dht")):
        if t is not None:
            _require(t, n, torch.float32, q.device)
            if t.shape != (N, H, K, V):
                raise ValueError(f"{n} must be (N,H,K,V) fp32")
    if grads_out is None:
        dq = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        dk = torch.empty(k.shape, dtype=q.dtype, device=q.device)
        dv = torch.empty(v.shape, dtype=q.dtype, device=q.device)
    else:
        dq, dk, dv = grads_out
        for t, ref, n in ((dq, q, "dq"), (dk, k, "dk"), (dv, v, "dv")):
            _require(t, n, q.dtype, q.device, contiguous=False)
            if t.shape != ref.shape:
                raise ValueError(f"{n} must be shaped like {n[1:]}")
    db = torch.empty_like(beta)
    dh0 = torch.empty(N, H, K, V, dtype=torch.float32, device=q.device) \
        if initial_state is not None else None
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    args = (_p(q), _p(k), _p(v), _p(beta), _p(initial_state), _p(do), _p(dht), _p(dq), _p(dk),
            _p(dv), _p(db), _p(dh0), _p(cu_seqlens), B, T,
            N if cu_seqlens is not None else 0, H, K, V, 64, dt, _p(workspace), ws_bytes,
            (REUSE_FORWARD if reuse_forward else 0) | (REUSE_STATES if reuse_states else 0))
    strides = [token_stride(t, n) for t, n in ((q, "q"), (k, "k"), (v, "v"), (dq, "dq"),
                                                (dk, "dk"), (dv, "dv"))]
    if strides == [H * K, H * K, H * V, H * K, H * K, H * V]:
        rc = lib().efla_chunk_bwd_hip(*args, _stream(q))
        check(rc, "efla_chunk_bwd_hip")
    else:
        arr = (ctypes.c_int64 * 6)(*strides)
        rc = lib().efla_chunk_bwd_strided_hip(*args, arr, _stream(q))
        check(rc, "efla_chunk_bwd_strided_hip")
    return dq, dk, dv, db, dh0


def new_workspace(q, v, cu_seqlens=None) -> torch.Tensor:
    """A workspace large enough for the backward of this problem (and so for its
    forward), for passing to both calls with save_states / reuse_forward."""
    B, T, H, K = q.shape
    N = 0 if cu_seqlens is None else cu_seqlens.numel() - 1
    n = workspace_bytes("bwd", B, T, H, K, v.shape[-1], q.dtype, N)
    return torch.empty(n, dtype=torch.uint8, device=q.device)


class ChunkEflaFunction(torch.autograd.Function):
    """Keeps the forward's workspace (the per-chunk WY factors and chunk start
    states) for the backward, which then recomputes nothing of the forward."""

    @staticmethod
    def forward(ctx, q, k, v, beta, initial_state, output_final_state, cu_seqlens):
        ws = new_workspace(q, v, cu_seqlens)
        o, st = chunk_efla_fwd(q, k, v, beta, initial_state, output_final_state, cu_seqlens,
                               workspace=ws, save_states=True)
        ctx.save_for_backward(q, k, v, beta, initial_state, cu_seqlens, ws)
        return o, st

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, beta, s0, cu, ws = ctx.saved_tensors
        dq, dk, dv, db, dh0 = chunk_efla_bwd(q, k, v, beta, do.contiguous(), s0,
                                             None if dht is None else dht.contiguous(), cu,
                                             workspace=ws, reuse_forward=True,
                                             reuse_states=True)
        return dq, dk, dv, db, dh0, None, None


def chunk_efla(q, k, v, beta, initial_state=None, output_final_state=False, cu_seqlens=None):
    """Differentiable chunked EFLA: returns (o, final_state or None)."""
    return ChunkEflaFunction.apply(q, k, v, beta, initial_state, output_final_state, cu_seqlens)


def workspace_bytes(kind: str, B: int, T: int, H: int, K: int, V: int, dtype, num_seqs=0):
    fn = lib().efla_chunk_fwd_workspace_size if kind == "fwd" else \
        lib().efla_chunk_bwd_workspace_size
    return fn(B, T, num_seqs, H, K, V, DTYPE_CODES[dtype])
