"""CPU oracle for the EFLA hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module.  It is the checker, never the product: the
HIP library in ``ceo_amd`` does not import it and fails loudly without its own
shared object.

Contents and what pins each part (tests/test_oracle_*.py):

* ``f32_to_bf16`` / ``bf16_to_f32`` -- RNE rounding of src/tensor/dtype.zig:370-390.
  Pinned by the reference's round-trip KAT (dtype.zig:653-665) and by
  torch's own bf16 cast on random data.
* ``coeff`` -- c(beta, lambda) and dc/dlambda of kernels/cuda/efla.cu:93-115.
  Pinned by the reference KAT (src/kernels/efla_kernels.zig:110-117), the closed
  forms, the Taylor/closed-form continuity at lambda = 1e-6, and central
  differences for dc/dlambda and dc/dbeta.
* ``r_forward`` / ``r_backward`` / ``r_chunked_scan`` -- the reference ABI
  (efla.cu:154-233, 235-454, 466-476, 482-748).  Pinned by the one-token
  closed form o_1 = c (v.k) k, by torch fp64 autograd of an independent
  restatement (rounding switched off via ``r_exact``), by the validation-order
  cases of the host code, and by the bf16 prefix sum.
* ``q_forward`` / ``q_backward`` -- the recurrence generalised to a query
  readout, per-token beta, d_k != d_v, varlen.  Pinned by the one-token closed
  form o_1 = c (q.k) v, the matrix-exponential form of one step (scipy expm),
  the residual contraction identity, beta -> 0, central differences, torch fp64
  autograd, varlen == independent runs and Mode R / Mode Q sharing S_T.
* ``chunk_forward`` / ``chunk_backward`` -- numpy fp64 restatement of the
  chunked (WY / UT-transform) algorithm the HIP kernels implement.  Pinned by
  equality with ``q_forward`` / ``q_backward`` for chunk sizes 1, 16, 64, T.
* ``layernorm_fwd`` / ``layernorm_bwd`` -- layernorm.cu:133-183 and the
  textbook gradient.  Pinned by the per-row mean 0 / variance 1 invariant and
  torch fp64 autograd.
* ``rmsnorm_fwd`` / ``rmsnorm_bwd`` -- layernorm.cu:15-127 with the exact
  gradient (the reference's dx drops a factor rs^2).  Pinned by the per-row
  mean(y^2) = 1 invariant (w = 1, eps = 0), torch's rms_norm and fp64
  autograd, and central differences that reject the reference's form.
* ``shortconv_fwd`` / ``shortconv_bwd`` -- prism.zig:448-473 in its own fp32
  order (bit-exact before the bf16 rounding) and the adjoint.  Pinned by
  torch's grouped conv1d (fp64) and its autograd, the impulse response (a unit
  input at t = 0 reads out the weights) and window 1 (y = x w exactly).
* ``prism_fwd`` / ``prism_bwd`` -- prism.zig:251-323 and its gradient.
  Pinned by a one-iteration closed form, a hand-unrolled two-iteration
  evaluation, torch fp64 autograd of an independent restatement and central
  differences.
* ``gelu_fwd`` / ``gelu_bwd`` -- layernorm.cu:189-250, tanh and erf forms.
  Pinned by torch's own GELU (both forms) and its autograd, and special values.
* ``adamw_step`` / ``adamw_step_bf16`` -- optim.cu:147-178, 657-709 with fp32
  and with bf16 state.  Pinned by an fp64 closed form at steps 1 and 7 and the
  zero-state identity p1 = p0 (1 - lr wd) - lr g / (|g| + eps); the bf16 form
  adds only the bf16 round trip, pinned by the reference's KAT (dtype.zig:654).
* ``cross_entropy_fwd`` / ``cross_entropy_bwd`` -- nn_kernels.zig:200-246.
  Pinned by torch's cross_entropy and its autograd (eps = 0), uniform logits
  (loss log V for every eps) and zero-sum gradient rows.
* ``embedding_fwd`` / ``embedding_bwd`` -- layers.zig:658-686 and its
  adjoint; pinned by a dense one-hot matmul (E = onehot W, dW = onehot^T dY).
* ``pack_sequences`` -- dataset.zig:421-465; pinned by the reference's own
  test (dataset.zig:467-481: 9 tokens, 3 sequences) and by invariants (packed
  tokens are the kept sequences in order, positions restart at 0).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

c_f32p = ctypes.POINTER(ctypes.c_float)
c_f64p = ctypes.POINTER(ctypes.c_double)
c_u16p = ctypes.POINTER(ctypes.c_uint16)
c_i32p = ctypes.POINTER(ctypes.c_int32)


def _host_has_avx2() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            flags = f.read()
        return " avx2" in flags and " fma" in flags
    except OSError:
        return False


def build(force: bool = False) -> None:
    """Compile the oracle shared objects in place with make."""
    args = ["make", "-s", "-C", _HERE]
    if force:
        args.insert(2, "-B")
    subprocess.run(args, check=True)


def lib():
    global _LIB
    if _LIB is not None:
        return _LIB
    name = "liboracle_avx2.so" if _host_has_avx2() else "liboracle.so"
    path = os.path.join(_HERE, name)
    if not os.path.exists(path):
        build()
    L = ctypes.CDLL(path)
    sz = ctypes.c_size_t
    i64 = ctypes.c_int64
    L.or_f32_to_bf16.restype = ctypes.c_uint16
    L.or_f32_to_bf16.argtypes = [ctypes.c_float]
    L.or_bf16_to_f32.restype = ctypes.c_float
    L.or_bf16_to_f32.argtypes = [ctypes.c_uint16]
    L.or_f32_to_bf16_array.argtypes = [c_f32p, c_u16p, sz]
    L.or_bf16_to_f32_array.argtypes = [c_u16p, c_f32p, sz]
    L.or_randn.argtypes = [ctypes.c_uint64, ctypes.c_uint64, c_f64p, sz]
    L.or_efla_coeff_f32.argtypes = [ctypes.c_float, ctypes.c_float, c_f32p, c_f32p]
    L.or_efla_coeff_f64.argtypes = [ctypes.c_double, ctypes.c_double, c_f64p, c_f64p, c_f64p]
    L.or_efla_r_forward.restype = ctypes.c_int
    L.or_efla_r_forward.argtypes = [c_u16p, c_u16p, c_u16p, c_u16p, sz, sz, sz, sz, ctypes.c_float]
    L.or_efla_r_backward.restype = ctypes.c_int
    L.or_efla_r_backward.argtypes = [c_u16p, c_u16p, c_u16p, c_u16p, c_u16p, c_u16p, c_u16p,
                                     sz, sz, sz, sz, ctypes.c_float]
    L.or_efla_r_chunked_scan.restype = ctypes.c_int
    L.or_efla_r_chunked_scan.argtypes = [ctypes.POINTER(c_u16p), sz, sz, sz]
    L.or_set_r_exact.argtypes = [ctypes.c_int]
    for sfx, p in (("f64", c_f64p), ("f32", c_f32p)):
        fwd = getattr(L, "or_efla_q_forward_" + sfx)
        fwd.argtypes = [p, p, p, p, c_i32p, i64, i64, i64, i64, i64, p, p, p]
        bwd = getattr(L, "or_efla_q_backward_" + sfx)
        bwd.argtypes = [p, p, p, p, p, c_i32p, i64, i64, i64, i64, i64, p, p,
                        p, p, p, p, p]
    L.or_layernorm_fwd.argtypes = [c_f32p, c_f32p, c_f32p, c_f32p, c_f32p, c_f32p, sz, sz,
                                   ctypes.c_float]
    L.or_layernorm_bwd.argtypes = [c_f32p, c_f32p, c_f32p, c_f32p, c_f32p, c_f32p, c_f64p,
                                   c_f64p, sz, sz]
    L.or_gelu_fwd.argtypes = [c_f32p, c_f32p, sz]
    L.or_gelu_bwd.argtypes = [c_f32p, c_f32p, c_f32p, sz]
    L.or_gelu_exact_fwd.argtypes = [c_f32p, c_f32p, sz]
    L.or_gelu_exact_bwd.argtypes = [c_f32p, c_f32p, c_f32p, sz]
    L.or_adamw_step.argtypes = [c_f32p, c_f32p, c_f32p, c_f32p, sz, ctypes.c_float,
                                ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                ctypes.c_float, sz]
    L.or_num_threads.restype = ctypes.c_int
    L.or_set_num_threads.argtypes = [ctypes.c_int]
    _LIB = L
    return L


def _p(a, t):
    if a is None:
        return None
    return a.ctypes.data_as(t)


# --------------------------------------------------------------------------
# bf16 and the input generator
# --------------------------------------------------------------------------
def f32_to_bf16(x) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), RNE as dtype.zig:370-384."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().or_f32_to_bf16_array(_p(x, c_f32p), _p(out, c_u16p), x.size)
    return out


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().or_bf16_to_f32_array(_p(h, c_u16p), _p(out, c_f32p), h.size)
    return out


def round_bf16(x) -> np.ndarray:
    """Values of x after a round trip through bf16, as float32."""
    return bf16_to_f32(f32_to_bf16(x))


def randn(seed: int, shape, offset: int = 0) -> np.ndarray:
    """Seeded N(0,1) in fp64 (splitmix64 + Box-Muller), portable across hosts."""
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, dtype=np.float64)
    lib().or_randn(ctypes.c_uint64(seed & 0xFFFFFFFFFFFFFFFF), ctypes.c_uint64(offset),
                   _p(out, c_f64p), n)
    return out.reshape(shape)


def make_efla_inputs(seed: int, n_tok: int, H: int, K: int, V: int, *, bf16: bool,
                     with_q: bool = True, with_do: bool = True):
    """Inputs with the distributions the benchmark configs name.

    q, k, v, dO ~ N(0,1); k L2-normalised per (token, head) in fp64 and then
    rounded; beta = sigmoid(N(0,1)).  Tensors come from independent streams
    (seed + tensor index << 40).  Returned as float32 arrays holding the
    bf16-rounded values when ``bf16`` is set.
    """
    def stream(i, shape):
        return randn(seed + (i << 40), shape)

    k = stream(1, (n_tok, H, K))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = stream(2, (n_tok, H, V))
    beta = 1.0 / (1.0 + np.exp(-stream(3, (n_tok, H))))
    out = {"k": k, "v": v, "beta": beta}
    if with_q:
        out["q"] = stream(0, (n_tok, H, K))
    if with_do:
        out["do"] = stream(4, (n_tok, H, V))
    conv = round_bf16 if bf16 else (lambda a: a.astype(np.float32))
    return {name: conv(a) for name, a in out.items()}


# --------------------------------------------------------------------------
# coefficient
# --------------------------------------------------------------------------
def coeff_f32(lam: float, beta: float):
    c = ctypes.c_float()
    d = ctypes.c_float()
    lib().or_efla_coeff_f32(lam, beta, ctypes.byref(c), ctypes.byref(d))
    return c.value, d.value


def coeff_f64(lam: float, beta: float):
    c = ctypes.c_double()
    dl = ctypes.c_double()
    db = ctypes.c_double()
    lib().or_efla_coeff_f64(lam, beta, ctypes.byref(c), ctypes.byref(dl), ctypes.byref(db))
    return c.value, dl.value, db.value


def coeff_np(lam, beta):
    """Vectorised fp64 c, dc/dlambda, dc/dbeta (same formulas as or_efla_coeff_f64)."""
    lam = np.asarray(lam, dtype=np.float64)
    beta = np.asarray(beta, dtype=np.float64)
    fn = np.vectorize(coeff_f64, otypes=[np.float64, np.float64, np.float64])
    return fn(lam, beta)


# --------------------------------------------------------------------------
# Mode R (reference ABI)
# --------------------------------------------------------------------------
def r_exact(flag: bool) -> None:
    """Switch the Mode R oracle's per-token bf16 state rounding off (True) or on."""
    lib().or_set_r_exact(1 if flag else 0)


def r_forward(k16, v16, state16, B, T, H, d, beta):
    """Reference efla_forward_cuda on bf16 bit patterns. Returns (rc, out16)."""
    out = np.zeros((B, T, H, d), dtype=np.uint16)
    st = state16
    rc = lib().or_efla_r_forward(_p(k16, c_u16p), _p(v16, c_u16p), _p(st, c_u16p),
                                 _p(out, c_u16p), B, T, H, d, float(beta))
    return rc, out


def r_backward(do16, k16, v16, state16, B, T, H, d, beta):
    """Reference efla_backward_cuda. Returns (rc, gk16, gv16, gs16)."""
    gk = np.zeros((B, T, H, d), dtype=np.uint16)
    gv = np.zeros((B, T, H, d), dtype=np.uint16)
    gs = np.zeros((B * H, d, d), dtype=np.uint16)
    rc = lib().or_efla_r_backward(_p(do16, c_u16p), _p(k16, c_u16p), _p(v16, c_u16p),
                                  _p(state16, c_u16p), _p(gk, c_u16p), _p(gv, c_u16p),
                                  _p(gs, c_u16p), B, T, H, d, float(beta))
    return rc, gk, gv, gs


def r_chunked_scan(chunks, H, d):
    """Reference efla_chunked_scan_cuda on a list of (H,d,d) uint16 arrays (in place)."""
    n = len(chunks)
    arr = (c_u16p * n)(*[_p(c, c_u16p) for c in chunks])
    return lib().or_efla_r_chunked_scan(arr, n, H, d)


# --------------------------------------------------------------------------
# Mode Q sequential recurrence
# --------------------------------------------------------------------------
def _qprep(dtype, *arrs):
    return [None if a is None else np.ascontiguousarray(a, dtype=dtype) for a in arrs]


def q_forward(q, k, v, beta, *, cu_seqlens=None, T=None, S0=None, dtype=np.float64):
    """o, S_T of the sequential recurrence.

    q, k: (n_tok, H, K); v: (n_tok, H, V); beta: (n_tok, H).  Without
    cu_seqlens the tokens are N = n_tok // T sequences of length T.
    """
    n_tok, H, K = q.shape
    V = v.shape[-1]
    if cu_seqlens is not None:
        cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
        N, T = len(cu) - 1, 0
    else:
        cu = None
        T = n_tok if T is None else T
        N = n_tok // T
    q, k, v, beta, S0 = _qprep(dtype, q, k, v, beta, S0)
    O = np.zeros((n_tok, H, V), dtype=dtype)
    ST = np.zeros((N, H, K, V), dtype=dtype)
    p = c_f64p if dtype == np.float64 else c_f32p
    fn = lib().or_efla_q_forward_f64 if dtype == np.float64 else lib().or_efla_q_forward_f32
    fn(_p(q, p), _p(k, p), _p(v, p), _p(beta, p), _p(cu, c_i32p), N, T, H, K, V,
       _p(S0, p), _p(O, p), _p(ST, p))
    return O, ST


def q_backward(q, k, v, beta, do, *, cu_seqlens=None, T=None, S0=None, dST=None,
               dtype=np.float64):
    """dq, dk, dv, dbeta, dS0 of the sequential recurrence (BPTT)."""
    n_tok, H, K = q.shape
    V = v.shape[-1]
    if cu_seqlens is not None:
        cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
        N, T = len(cu) - 1, 0
    else:
        cu = None
        T = n_tok if T is None else T
        N = n_tok // T
    q, k, v, beta, do, S0, dST = _qprep(dtype, q, k, v, beta, do, S0, dST)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    db = np.zeros_like(beta)
    dS0 = np.zeros((N, H, K, V), dtype=dtype)
    p = c_f64p if dtype == np.float64 else c_f32p
    fn = lib().or_efla_q_backward_f64 if dtype == np.float64 else lib().or_efla_q_backward_f32
    fn(_p(q, p), _p(k, p), _p(v, p), _p(beta, p), _p(do, p), _p(cu, c_i32p), N, T, H, K, V,
       _p(S0, p), _p(dST, p), _p(dq, p), _p(dk, p), _p(dv, p), _p(db, p), _p(dS0, p))
    return dq, dk, dv, db, dS0


# --------------------------------------------------------------------------
# Chunked (WY / UT transform) restatement in numpy fp64, one (sequence, head)
# --------------------------------------------------------------------------
def chunk_prep(k, v, beta):
    """For one chunk: b, dc/dlambda, dc/dbeta, T = (I + A)^-1, W = T D K, U = T D V."""
    lam = (k * k).sum(-1)
    b, dcl, dcb = coeff_np(lam, beta)
    C = k.shape[0]
    A = np.tril(b[:, None] * (k @ k.T), -1)
    Tm = np.linalg.inv(np.eye(C) + A)
    W = Tm @ (b[:, None] * k)
    U = Tm @ (b[:, None] * v)
    return b, dcl, dcb, Tm, W, U


def chunk_forward(q, k, v, beta, C=64, S0=None):
    """o, S_T and per-chunk (S_n, W, U, Vn) for one (sequence, head); fp64."""
    L, K = k.shape
    V = v.shape[1]
    S = np.zeros((K, V)) if S0 is None else np.array(S0, dtype=np.float64)
    O = np.zeros((L, V))
    inter = []
    for n0 in range(0, L, C):
        sl = slice(n0, min(n0 + C, L))
        qc, kc, vc = q[sl].astype(np.float64), k[sl].astype(np.float64), v[sl].astype(np.float64)
        b, _, _, Tm, W, U = chunk_prep(kc, vc, beta[sl].astype(np.float64))
        Vn = U - W @ S
        O[sl] = qc @ S + np.tril(qc @ kc.T) @ Vn
        inter.append({"S": S.copy(), "W": W, "U": U, "Vn": Vn, "T": Tm, "b": b})
        S = S + kc.T @ Vn
    return O, S, inter


def chunk_backward(q, k, v, beta, do, C=64, S0=None, dST=None):
    """dq, dk, dv, dbeta, dS0 of the chunked algorithm for one (sequence, head)."""
    L, K = k.shape
    V = v.shape[1]
    _, _, inter = chunk_forward(q, k, v, beta, C, S0)
    dS = np.zeros((K, V)) if dST is None else np.array(dST, dtype=np.float64)
    dq = np.zeros((L, K))
    dk = np.zeros((L, K))
    dv = np.zeros((L, V))
    dbeta = np.zeros(L)
    starts = list(range(0, L, C))
    for idx in reversed(range(len(starts))):
        n0 = starts[idx]
        sl = slice(n0, min(n0 + C, L))
        Q, Kc, Vc, dOc = (a[sl].astype(np.float64) for a in (q, k, v, do))
        it = inter[idx]
        S, W, Tm, b, Vn = it["S"], it["W"], it["T"], it["b"], it["Vn"]
        _, dcl, dcb, _, _, _ = chunk_prep(Kc, Vc, beta[sl].astype(np.float64))
        P = np.tril(Q @ Kc.T)
        dVn = P.T @ dOc + Kc @ dS
        M = np.tril(dOc @ Vn.T)
        dQ = dOc @ S.T + M @ Kc
        dK = M.T @ Q + Vn @ dS.T
        dW = -dVn @ S.T
        dU = dVn
        dS_prev = dS + Q.T @ dOc - W.T @ dVn
        DK = b[:, None] * Kc
        DV = b[:, None] * Vc
        dT = dW @ DK.T + dU @ DV.T
        dDK = Tm.T @ dW
        dDV = Tm.T @ dU
        dK += b[:, None] * dDK
        db = (dDK * Kc).sum(1) + (dDV * Vc).sum(1)
        dV = b[:, None] * dDV
        dA = np.tril(-(Tm.T @ dT @ Tm.T), -1)
        db += (dA * (Kc @ Kc.T)).sum(1)
        dK += b[:, None] * (dA @ Kc) + dA.T @ DK
        dK += 2.0 * (db * dcl)[:, None] * Kc
        dq[sl], dk[sl], dv[sl], dbeta[sl] = dQ, dK, dV, db * dcb
        dS = dS_prev
    return dq, dk, dv, dbeta, dS


# --------------------------------------------------------------------------
# LayerNorm, GELU, AdamW
# --------------------------------------------------------------------------
def layernorm_fwd(x, w, b, eps=1e-5):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, D = x.shape
    w = np.ascontiguousarray(w, dtype=np.float32)
    b = None if b is None else np.ascontiguousarray(b, dtype=np.float32)
    y = np.empty_like(x)
    mean = np.empty(rows, dtype=np.float32)
    rstd = np.empty(rows, dtype=np.float32)
    lib().or_layernorm_fwd(_p(x, c_f32p), _p(w, c_f32p), _p(b, c_f32p), _p(y, c_f32p),
                           _p(mean, c_f32p), _p(rstd, c_f32p), rows, D, float(eps))
    return y, mean, rstd


def layernorm_bwd(dy, x, w, mean, rstd):
    dy, x, w, mean, rstd = (np.ascontiguousarray(a, dtype=np.float32)
                            for a in (dy, x, w, mean, rstd))
    rows, D = x.shape
    dx = np.empty_like(x)
    dw = np.empty(D, dtype=np.float64)
    db = np.empty(D, dtype=np.float64)
    lib().or_layernorm_bwd(_p(dy, c_f32p), _p(x, c_f32p), _p(w, c_f32p), _p(mean, c_f32p),
                           _p(rstd, c_f32p), _p(dx, c_f32p), _p(dw, c_f64p), _p(db, c_f64p),
                           rows, D)
    return dx, dw, db


def rmsnorm_fwd(x, w, eps=1e-5):
    """y = x rs w with rs = 1 / sqrt(mean(x^2) + eps) per row, fp64
    (layernorm.cu:15-48).  Returns (y, rs)."""
    x = np.asarray(x, dtype=np.float64)
    rs = 1.0 / np.sqrt((x * x).mean(axis=-1) + eps)
    return x * rs[:, None] * np.asarray(w, dtype=np.float64), rs


def rmsnorm_bwd(dy, x, w, eps=1e-5, reference_form=False):
    """(dx, dw) of y = x rs w in fp64.  The exact gradient is
    dx = rs g - x rs^3 mean(g x) with g = dy w, dw = sum_rows dy x rs.
    ``reference_form`` gives the reference's dx instead (layernorm.cu:108-116:
    the second term scaled by rs rather than rs^3), which a finite-difference
    check rejects; the HIP kernels implement the exact gradient."""
    dy, x, w = (np.asarray(a, dtype=np.float64) for a in (dy, x, w))
    D = x.shape[-1]
    rs = 1.0 / np.sqrt((x * x).mean(axis=-1) + eps)
    g = dy * w
    sgx = (g * x).sum(axis=-1)
    scale = rs if reference_form else rs ** 3
    dx = rs[:, None] * g - x * (scale * sgx / D)[:, None]
    dw = (dy * x * rs[:, None]).sum(axis=0)
    return dx, dw


def shortconv_fwd(x, weight):
    """ShortConv.forwardCpu (src/model/prism.zig:448-473) in its own arithmetic:
    for x (B, T, C) and weight (C, W) holding bf16 values, every output is the
    fp32 sum over w = 0..W-1 (t - w >= 0), in increasing w, of the fp32-rounded
    products x[b,t-w,c] * weight[c,w], starting from +0.  numpy float32
    multiplies and adds round each operation (no fused multiply-add), so this is
    the reference's value before its bf16 rounding.  Returns fp32 (B, T, C)."""
    x = np.asarray(x, dtype=np.float32)
    wt = np.asarray(weight, dtype=np.float32)
    B, T, C = x.shape
    s = np.zeros((B, T, C), dtype=np.float32)
    for w in range(wt.shape[1]):
        if w >= T:
            break
        p = x[:, :T - w, :] * wt[None, None, :, w]
        s[:, w:, :] = s[:, w:, :] + p
    return s


def shortconv_bwd(dy, x, weight):
    """(dx, dweight) of y = ShortConv(x) in fp64: dx[t] = sum_w dy[t+w] w[c,w],
    dweight[c,w] = sum_{b,t>=w} dy[b,t,c] x[b,t-w,c]."""
    dy, x, wt = (np.asarray(a, dtype=np.float64) for a in (dy, x, weight))
    B, T, C = x.shape
    dx = np.zeros_like(x)
    dw = np.zeros_like(wt)
    for w in range(min(wt.shape[1], T)):
        dx[:, :T - w, :] += dy[:, w:, :] * wt[None, None, :, w]
        dw[:, w] = (dy[:, w:, :] * x[:, :T - w, :]).sum(axis=(0, 1))
    return dx, dw


def _gelu_tanh64(x):
    """0.5 x (1 + tanh u) written x / (1 + e^(-2u)): the same value without the
    cancellation of 1 + tanh u for x << 0."""
    u = np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)
    with np.errstate(over="ignore"):  # e^(-2u) = inf gives the limit -0
        return x / (1.0 + np.exp(-2.0 * u))


def _gelu_tanh64_grad(x):
    """s + 2 x s (1 - s) u' with s = 1 / (1 + e^(-2u)) = 0.5 (1 + tanh u)."""
    u = np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)
    with np.errstate(over="ignore"):
        s = 1.0 / (1.0 + np.exp(-2.0 * u))
    return s + 2.0 * x * s * (1.0 - s) * np.sqrt(2.0 / np.pi) * (1.0 + 3 * 0.044715 * x ** 2)


def prism_fwd(u, v, w_p, head_dim, round_output=True):
    """PrismLayer.prismForwardCpu (prism.zig:251-323): per row and channel
    d < head_dim, r = v - u; for each l: delta = GELU_tanh(p_l[d] r) with p_l
    the first head_dim values of w_p[l], o = o + 0.5 delta (rounded to fp32 and
    then bf16 after every step when ``round_output``), r -= delta.  Channels
    >= head_dim are 0.  fp64 math; returns float32 (B, T, C)."""
    u = np.asarray(u, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    out = np.zeros(u.shape, dtype=np.float64)
    r = v[..., :head_dim] - u[..., :head_dim]
    o = np.zeros_like(r)
    for wp in w_p:
        p = np.asarray(wp, dtype=np.float64).reshape(-1)[:head_dim]
        d = _gelu_tanh64(p * r)
        o = o + 0.5 * d
        if round_output:
            o = round_bf16(o.astype(np.float32)).astype(np.float64)
        r = r - d
    out[..., :head_dim] = o
    return out.astype(np.float32)


def prism_bwd(grad_output, u, v, w_p, head_dim):
    """(grad_u, grad_v, [grad p_l]) of prism_fwd without the bf16 rounding of o
    (fp64): the reverse of r_{l+1} = r_l - GELU(p_l r_l), o = 0.5 sum_l
    GELU(p_l r_l)."""
    g = np.asarray(grad_output, dtype=np.float64)[..., :head_dim]
    u = np.asarray(u, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    ps = [np.asarray(wp, dtype=np.float64).reshape(-1)[:head_dim] for wp in w_p]
    rs, xs = [], []
    r = v[..., :head_dim] - u[..., :head_dim]
    for p in ps:
        rs.append(r)
        xs.append(p * r)
        r = r - _gelu_tanh64(xs[-1])
    a = np.zeros_like(r)
    dps = [None] * len(ps)
    for l in range(len(ps) - 1, -1, -1):
        gx = (0.5 * g - a) * _gelu_tanh64_grad(xs[l])
        dps[l] = (gx * rs[l]).reshape(-1, head_dim).sum(axis=0)
        a = a + gx * ps[l]
    gu = np.zeros(u.shape)
    gv = np.zeros(u.shape)
    gv[..., :head_dim] = a
    gu[..., :head_dim] = -a
    return gu, gv, dps


def gelu_fwd(x, approximate=True):
    """GELU in fp64, rounded to fp32: the tanh form (layernorm.cu:189-194) or,
    with approximate=False, the erf form (layernorm.cu:196-200)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    fn = lib().or_gelu_fwd if approximate else lib().or_gelu_exact_fwd
    fn(_p(x, c_f32p), _p(y, c_f32p), x.size)
    return y


def gelu_bwd(dy, x, approximate=True):
    """dy * GELU'(x) in fp64 (layernorm.cu:216-250), rounded to fp32."""
    dy = np.ascontiguousarray(dy, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    dx = np.empty_like(x)
    fn = lib().or_gelu_bwd if approximate else lib().or_gelu_exact_bwd
    fn(_p(dy, c_f32p), _p(x, c_f32p), _p(dx, c_f32p), x.size)
    return dx


def adamw_step(p, g, m, v, lr, b1, b2, eps, wd, step):
    """In-place fp32 AdamW step on numpy arrays."""
    for a in (p, m, v):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    g = np.ascontiguousarray(g, dtype=np.float32)
    lib().or_adamw_step(_p(p, c_f32p), _p(g, c_f32p), _p(m, c_f32p), _p(v, c_f32p), p.size,
                        lr, b1, b2, eps, wd, step)


def adamw_step_bf16(p, g, m, v, lr, b1, b2, eps, wd, step):
    """The reference's bf16-state AdamW (optim.cu:147-178): bf16 p, g, m, v
    (given as uint16 bit patterns) read as fp32, the fp32 step above, each
    result rounded to bf16.  Returns the new (p, m, v) bit patterns."""
    pf, gf, mf, vf = (bf16_to_f32(a) for a in (p, g, m, v))
    adamw_step(pf, gf, mf, vf, lr, b1, b2, eps, wd, step)
    return f32_to_bf16(pf), f32_to_bf16(mf), f32_to_bf16(vf)


def cross_entropy_fwd(logits, targets, label_smoothing=0.0):
    """crossEntropyForwardCpu (nn_kernels.zig:200-246) in fp64: per-row
    ((1 - eps) (logsumexp - z_t) + eps log V) / B; NaN for a target outside
    [0, V).  Returns the (B,) array whose sum is the mean loss."""
    z = np.asarray(logits, dtype=np.float64)
    B, V = z.shape
    t = np.asarray(targets).astype(np.int64)
    m = z.max(axis=1, keepdims=True)
    lse = (m + np.log(np.exp(z - m).sum(axis=1, keepdims=True)))[:, 0]
    ok = (t >= 0) & (t < V)
    zt = np.where(ok, z[np.arange(B), np.clip(t, 0, V - 1)], 0.0)
    loss = ((1.0 - label_smoothing) * (lse - zt) + label_smoothing * np.log(V)) / B
    return np.where(ok, loss, np.nan)


def cross_entropy_bwd(grad_loss, logits, targets, label_smoothing=0.0):
    """d loss / d logits for the forward above: grad_loss[i] (1 - eps)
    (softmax_i - onehot(t_i)) / B, zero rows for invalid targets (fp64)."""
    z = np.asarray(logits, dtype=np.float64)
    B, V = z.shape
    t = np.asarray(targets).astype(np.int64)
    p = np.exp(z - z.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ok = (t >= 0) & (t < V)
    p[np.arange(B)[ok], t[ok]] -= 1.0
    coef = np.where(ok, np.asarray(grad_loss, dtype=np.float64) * (1 - label_smoothing) / B, 0.0)
    return p * coef[:, None]


def embedding_fwd(indices, weight):
    """Embedding.forward (layers.zig:658-686): rows of `weight`; an index
    outside the table gives a zero row (the checked entry's behaviour)."""
    w = np.asarray(weight)
    idx = np.asarray(indices).astype(np.int64)
    ok = (idx >= 0) & (idx < w.shape[0])
    out = np.zeros((idx.size, w.shape[1]), dtype=w.dtype)
    out[ok] = w[idx[ok]]
    return out


def embedding_bwd(grad_output, indices, num_embeddings):
    """sum of grad_output rows per index (fp64), out-of-range indices skipped."""
    g = np.asarray(grad_output, dtype=np.float64)
    idx = np.asarray(indices).astype(np.int64)
    ok = (idx >= 0) & (idx < num_embeddings)
    dw = np.zeros((num_embeddings, g.shape[1]))
    np.add.at(dw, idx[ok], g[ok])
    return dw


def pack_sequences(sequences, max_length):
    """packSequences (dataset.zig:421-465), pure Python: in order, a sequence
    is appended when it fits in what is left of max_length, else skipped.
    Returns (tokens, positions, sequence_ids, cumulative_lengths)."""
    toks, pos, sid, cum = [], [], [], []
    cur = 0
    for seq in sequences:
        if cur + len(seq) > max_length:
            continue
        for p, t in enumerate(seq):
            toks.append(int(t))
            pos.append(p)
            sid.append(len(cum))
        cur += len(seq)
        cum.append(cur)
    return toks, pos, sid, cum


def num_threads() -> int:
    return lib().or_num_threads()


def set_num_threads(n: int) -> None:
    lib().or_set_num_threads(int(n))
