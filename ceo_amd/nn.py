"""LayerNorm, GEMM, GELU and AdamW around EFLA: torch-facing wrappers over the C ABI.

Mirror the reference's ``layerNormForwardCuda`` / ``gemmForwardCuda`` /
``gemmBackwardCuda`` externs (src/kernels/nn_kernels.zig:28-76) and their
callers ``LayerNorm.forward`` (src/nn/layers.zig:226-245, eps 1e-5) and
``Linear.forward`` (src/nn/layers.zig:561-586, weight (in, out) row-major),
and the GELU / AdamW kernels of kernels/cuda/include/kernels.h:171-189, 309-322.
"""
from __future__ import annotations

import torch

from ._lib import check, lib
from .efla import DTYPE_CODES, _p, _require, _stream


def layernorm_forward(x: torch.Tensor, weight: torch.Tensor, bias=None, eps: float = 1e-5,
                      save_stats: bool = False):
    """y = LayerNorm(x) over the last dim (bf16); with save_stats also (mean, rstd) fp32."""
    D = x.shape[-1]
    _require(x, "x", torch.bfloat16)
    _require(weight, "weight", torch.bfloat16, x.device)
    if bias is not None:
        _require(bias, "bias", torch.bfloat16, x.device)
    y = torch.empty_like(x)
    if save_stats:
        rows = x.numel() // D
        mean = torch.empty(rows, dtype=torch.float32, device=x.device)
        rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
        rc = lib().layernorm_forward_stats_hip(_p(x), _p(weight), _p(bias), _p(y), _p(mean),
                                               _p(rstd), x.numel(), D, float(eps), _stream(x))
        check(rc, "layernorm_forward_stats_hip")
        return y, mean, rstd
    rc = lib().layernorm_forward_hip(_p(x), _p(weight), _p(bias), _p(y), x.numel(), D,
                                     float(eps), _stream(x))
    check(rc, "layernorm_forward_hip")
    return y


def layernorm_backward(dy, x, weight, mean, rstd, need_param_grads: bool = True,
                       residual=None, out_dx_colsum=None, out_dw=None, out_db=None):
    """(dx bf16, dweight, dbias); dweight / dbias are fp32 (None without
    need_param_grads), or the given ``out_dw`` / ``out_db`` ((D,) bf16, written
    in place, e.g. views of a bf16 gradient buffer).  With ``residual`` (bf16,
    x's shape) dx is LayerNorm's input gradient plus it; with
    ``out_dx_colsum`` ((D,) bf16) dx's column sums are written there."""
    D = x.shape[-1]
    for t, n in ((dy, "dy"), (x, "x"), (weight, "weight")):
        _require(t, n, torch.bfloat16, x.device)
    _require(mean, "mean", torch.float32, x.device)
    _require(rstd, "rstd", torch.float32, x.device)
    dx = torch.empty_like(x)
    pbf = out_dw is not None or out_db is not None
    if pbf:
        if out_dw is None or out_db is None or not need_param_grads:
            raise ValueError("out_dw and out_db go together (and need need_param_grads)")
        for t, n in ((out_dw, "out_dw"), (out_db, "out_db")):
            _require(t, n, torch.bfloat16, x.device)
            if t.numel() != D:
                raise ValueError(f"{n} must hold normalized_shape values")
        dw, db = out_dw, out_db
    else:
        dw = torch.empty(D, dtype=torch.float32, device=x.device) if need_param_grads else None
        db = torch.empty(D, dtype=torch.float32, device=x.device) if need_param_grads else None
    if residual is not None:
        _require(residual, "residual", torch.bfloat16, x.device)
        if residual.shape != x.shape:
            raise ValueError("residual must have x's shape")
    if out_dx_colsum is not None:
        _require(out_dx_colsum, "out_dx_colsum", torch.bfloat16, x.device)
        if out_dx_colsum.numel() != D:
            raise ValueError("out_dx_colsum must hold normalized_shape values")
    if out_dx_colsum is not None or pbf:
        rc = lib().layernorm_backward_ex_hip(_p(dy), _p(x), _p(weight), _p(mean), _p(rstd),
                                             _p(residual), _p(dx), _p(dw), _p(db),
                                             _p(out_dx_colsum), x.numel(), D, int(pbf),
                                             _stream(x))
        check(rc, "layernorm_backward_ex_hip")
    elif residual is None:
        rc = lib().layernorm_backward_hip(_p(dy), _p(x), _p(weight), _p(mean), _p(rstd), _p(dx),
                                          _p(dw), _p(db), x.numel(), D, _stream(x))
        check(rc, "layernorm_backward_hip")
    else:
        rc = lib().layernorm_backward_residual_hip(_p(dy), _p(x), _p(weight), _p(mean),
                                                   _p(rstd), _p(residual), _p(dx), _p(dw),
                                                   _p(db), x.numel(), D, _stream(x))
        check(rc, "layernorm_backward_residual_hip")
    return dx, dw, db


def rmsnorm_forward(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """y = x * rsqrt(mean(x^2) + eps) * weight over the last dim (bf16)."""
    D = x.shape[-1]
    _require(x, "x", torch.bfloat16)
    _require(weight, "weight", torch.bfloat16, x.device)
    y = torch.empty_like(x)
    rc = lib().rmsnorm_forward_hip(_p(x), _p(weight), _p(y), x.numel(), D, float(eps),
                                   _stream(x))
    check(rc, "rmsnorm_forward_hip")
    return y


def rmsnorm_backward(dy, x, weight, eps: float = 1e-5, grad_weight=None,
                     need_weight_grad: bool = True):
    """(dx bf16, dweight fp32 or None).  dweight is added into ``grad_weight``
    when given (fp32, (D,)), else into a new zero buffer."""
    D = x.shape[-1]
    for t, n in ((dy, "dy"), (x, "x"), (weight, "weight")):
        _require(t, n, torch.bfloat16, x.device)
    dx = torch.empty_like(x)
    dw = None
    if need_weight_grad:
        if grad_weight is None:
            dw = torch.zeros(D, dtype=torch.float32, device=x.device)
        else:
            _require(grad_weight, "grad_weight", torch.float32, x.device)
            if grad_weight.numel() != D:
                raise ValueError("grad_weight must hold normalized_shape values")
            dw = grad_weight
    rc = lib().rmsnorm_backward_hip(_p(dy), _p(x), _p(weight), _p(dx), _p(dw), x.numel(), D,
                                    float(eps), _stream(x))
    check(rc, "rmsnorm_backward_hip")
    return dx, dw


def gemm_forward(a: torch.Tensor, b: torch.Tensor, bias=None, out_dtype=None) -> torch.Tensor:
    """c = a @ b (+ bias), a (m,k), b (k,n) row-major; fp32 accumulation."""
    m, k = a.shape
    k2, n = b.shape
    if k2 != k:
        raise ValueError("gemm_forward: inner dimensions differ")
    _require(a, "a")
    _require(b, "b", device=a.device)
    out_dtype = out_dtype or a.dtype
    c = torch.empty(m, n, dtype=out_dtype, device=a.device)
    if bias is not None:
        _require(bias, "bias", out_dtype, a.device)
    rc = lib().gemm_forward_hip(_p(a), _p(b), _p(bias), _p(c), m, k, n, DTYPE_CODES[a.dtype],
                                DTYPE_CODES[b.dtype], DTYPE_CODES[out_dtype], _stream(a))
    check(rc, "gemm_forward_hip")
    return c


def _row_stride(t: torch.Tensor, name: str) -> int:
    """Row stride of a 2-D tensor whose rows are contiguous (a column block of
    a larger row-major matrix is fine)."""
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be 2-D with contiguous rows")
    return t.stride(0)


def gemm_ex(a, b, out, bias=None, c=None, alpha: float = 1.0, beta: float = 0.0,
            trans_a: bool = False, trans_b: bool = False) -> torch.Tensor:
    """out = alpha op(a) op(b) (+ bias) + beta c, row-major 2-D operands whose
    rows are contiguous (views of column blocks allowed); ``c`` may be ``out``
    itself.  Writes into ``out`` and returns it."""
    m, n = out.shape
    k = a.shape[0] if trans_a else a.shape[1]
    if (a.shape[1] if trans_a else a.shape[0]) != m:
        raise ValueError("gemm_ex: op(a) rows differ from out rows")
    if (b.shape[1] if trans_b else b.shape[0]) != k or \
            (b.shape[0] if trans_b else b.shape[1]) != n:
        raise ValueError("gemm_ex: op(b) must be k x n")
    for t, nme in ((a, "a"), (b, "b"), (out, "out")):
        if not t.is_cuda or t.dtype != out.dtype:
            raise ValueError(f"{nme} must be a device tensor of out's dtype")
    if bias is not None:
        _require(bias, "bias", out.dtype, out.device)
    ldc = 0
    if beta != 0.0:
        if c is None or c.shape != out.shape or c.dtype != out.dtype:
            raise ValueError("gemm_ex: beta != 0 needs c of out's shape and dtype")
        ldc = _row_stride(c, "c")
    rc = lib().gemm_ex_hip(int(trans_a), int(trans_b), m, n, k, float(alpha), _p(a),
                           _row_stride(a, "a"), _p(b), _row_stride(b, "b"), _p(bias),
                           float(beta), _p(c) if beta != 0.0 else None, ldc, _p(out),
                           _row_stride(out, "out"), DTYPE_CODES[out.dtype], _stream(out))
    check(rc, "gemm_ex_hip")
    return out


def gemm_backward(dc: torch.Tensor, a: torch.Tensor, b: torch.Tensor, need_a=True, need_b=True,
                  need_bias=False, out_a=None, out_b=None, out_bias=None):
    """(da, db, dbias) for c = a @ b + bias, all bf16; ``out_*`` (contiguous,
    right shape) receive the results instead of new tensors."""
    m, k = a.shape
    n = b.shape[1]
    for t, nme in ((dc, "dc"), (a, "a"), (b, "b")):
        _require(t, nme, torch.bfloat16, a.device)
    for t, nme, shape in ((out_a, "out_a", (m, k)), (out_b, "out_b", (k, n)),
                          (out_bias, "out_bias", (n,))):
        if t is not None:
            _require(t, nme, torch.bfloat16, a.device)
            if tuple(t.shape) != shape:
                raise ValueError(f"gemm_backward: {nme} must be {shape}")
    da = (out_a if out_a is not None else torch.empty_like(a)) if need_a else None
    dbm = (out_b if out_b is not None else torch.empty_like(b)) if need_b else None
    dbias = (out_bias if out_bias is not None else
             torch.empty(n, dtype=torch.bfloat16, device=a.device)) if need_bias else None
    rc = lib().gemm_backward_hip(_p(dc), _p(a), _p(b), _p(da), _p(dbm), _p(dbias), m, k, n,
                                 _stream(a))
    check(rc, "gemm_backward_hip")
    return da, dbm, dbias


def gemm_gelu_forward(a: torch.Tensor, b: torch.Tensor, bias=None):
    """(pre, out) with pre = a @ b (+ bias) and out = GELU_tanh(pre), bf16, in
    one product with the GELU in its epilogue."""
    m, k = a.shape
    k2, n = b.shape
    if k2 != k:
        raise ValueError("gemm_gelu_forward: inner dimensions differ")
    _require(a, "a", torch.bfloat16)
    _require(b, "b", torch.bfloat16, a.device)
    if bias is not None:
        _require(bias, "bias", torch.bfloat16, a.device)
    pre = torch.empty(m, n, dtype=torch.bfloat16, device=a.device)
    out = torch.empty_like(pre)
    rc = lib().gemm_gelu_forward_hip(_p(a), _p(b), _p(bias), _p(pre), _p(out), m, k, n,
                                     _stream(a))
    check(rc, "gemm_gelu_forward_hip")
    return pre, out


def gemm_gelu_backward(dc, a, b, pre, need_pre=True, need_b=True, need_bias=False,
                       out_b=None, out_bias=None, out_pre_bias=None):
    """(dpre, db, dbias) for c = a @ b + bias with a = GELU_tanh(pre): dpre =
    (dc @ b^T) * GELU'(pre) from one product with the derivative in its
    epilogue; bf16.  With ``out_pre_bias`` ((k,) bf16) the column sums of
    dpre (the gradient of the bias that made pre) are also written there."""
    m, k = a.shape
    n = b.shape[1]
    for t, nme in ((dc, "dc"), (a, "a"), (b, "b"), (pre, "pre")):
        _require(t, nme, torch.bfloat16, a.device)
    if pre.shape != a.shape:
        raise ValueError("gemm_gelu_backward: pre must have a's shape")
    for t, nme, shape in ((out_b, "out_b", (k, n)), (out_bias, "out_bias", (n,)),
                          (out_pre_bias, "out_pre_bias", (k,))):
        if t is not None:
            _require(t, nme, torch.bfloat16, a.device)
            if tuple(t.shape) != shape:
                raise ValueError(f"gemm_gelu_backward: {nme} must be {shape}")
    if out_pre_bias is not None and not need_pre:
        raise ValueError("gemm_gelu_backward: out_pre_bias needs need_pre")
    dpre = torch.empty_like(a) if need_pre else None
    dbm = (out_b if out_b is not None else torch.empty_like(b)) if need_b else None
    dbias = (out_bias if out_bias is not None else
             torch.empty(n, dtype=torch.bfloat16, device=a.device)) if need_bias else None
    rc = lib().gemm_gelu_backward_hip(_p(dc), _p(a), _p(b), _p(pre), _p(dpre), _p(dbm),
                                      _p(dbias), _p(out_pre_bias), m, k, n, _stream(a))
    check(rc, "gemm_gelu_backward_hip")
    return dpre, dbm, dbias


def gelu_forward(x: torch.Tensor, approximate: bool = True) -> torch.Tensor:
    """GELU of a bf16 tensor (tanh form unless approximate=False)."""
    _require(x, "x", torch.bfloat16)
    y = torch.empty_like(x)
    rc = lib().gelu_forward_hip(_p(x), _p(y), x.numel(), bool(approximate), _stream(x))
    check(rc, "gelu_forward_hip")
    return y


def gelu_backward(dy: torch.Tensor, x: torch.Tensor, approximate: bool = True) -> torch.Tensor:
    """dy * GELU'(x), bf16."""
    _require(x, "x", torch.bfloat16)
    _require(dy, "dy", torch.bfloat16, x.device)
    if dy.shape != x.shape:
        raise ValueError("gelu_backward: dy and x differ in shape")
    dx = torch.empty_like(x)
    rc = lib().gelu_backward_hip(_p(dy), _p(x), _p(dx), x.numel(), bool(approximate),
                                 _stream(x))
    check(rc, "gelu_backward_hip")
    return dx


def sigmoid_gate_forward(logits: torch.Tensor) -> torch.Tensor:
    """beta = bf16(sigmoid(float(logits))) of a (rows, cols) bf16 column block
    (row stride free, e.g. the end of a fused projection row); beta is packed."""
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be (rows, cols) with unit column stride")
    _require(logits, "logits", torch.bfloat16, contiguous=False)
    rows, cols = logits.shape
    beta = torch.empty(rows, cols, dtype=torch.bfloat16, device=logits.device)
    rc = lib().sigmoid_gate_forward_hip(_p(logits), logits.stride(0), _p(beta), rows, cols,
                                        _stream(logits))
    check(rc, "sigmoid_gate_forward_hip")
    return beta


def sigmoid_gate_backward(dbeta: torch.Tensor, beta: torch.Tensor, out: torch.Tensor) -> None:
    """out = bf16((float(dbeta) * b) * (1 - b)), b = float(beta), written into the
    (rows, cols) block ``out`` (row stride free); dbeta, beta packed."""
    _require(beta, "beta", torch.bfloat16)
    _require(dbeta, "dbeta", torch.bfloat16, beta.device)
    _require(out, "out", torch.bfloat16, beta.device, contiguous=False)
    if beta.dim() != 2 or dbeta.shape != beta.shape or out.shape != beta.shape \
            or out.stride(1) != 1:
        raise ValueError("sigmoid_gate_backward: dbeta, beta, out must be (rows, cols)")
    rows, cols = beta.shape
    rc = lib().sigmoid_gate_backward_hip(_p(dbeta), _p(beta), _p(out), out.stride(0), rows,
                                         cols, _stream(beta))
    check(rc, "sigmoid_gate_backward_hip")


def adamw_step(param, grad, exp_avg, exp_avg_sq, lr, beta1=0.9, beta2=0.999, eps=1e-8,
               weight_decay=0.0, step=1) -> None:
    """In-place AdamW step with bf16 parameters and state (the reference's layout)."""
    for t, n in ((param, "param"), (grad, "grad"), (exp_avg, "exp_avg"),
                 (exp_avg_sq, "exp_avg_sq")):
        _require(t, n, torch.bfloat16, param.device)
        if t.numel() != param.numel():
            raise ValueError(f"adamw_step: {n} size differs from param")
    rc = lib().adamw_step_hip(_p(param), _p(grad), _p(exp_avg), _p(exp_avg_sq), param.numel(),
                              float(lr), float(beta1), float(beta2), float(eps),
                              float(weight_decay), int(step), _stream(param))
    check(rc, "adamw_step_hip")


def adamw_step_master(param, grad, exp_avg, exp_avg_sq, lr, beta1=0.9, beta2=0.999, eps=1e-8,
                      weight_decay=0.0, step=1, param_bf16=None) -> None:
    """In-place AdamW step on fp32 master weights / moments with a bf16 gradient;
    ``param_bf16`` (optional) receives the new weights in bf16."""
    for t, n in ((param, "param"), (exp_avg, "exp_avg"), (exp_avg_sq, "exp_avg_sq")):
        _require(t, n, torch.float32, param.device)
    _require(grad, "grad", torch.bfloat16, param.device)
    if param_bf16 is not None:
        _require(param_bf16, "param_bf16", torch.bfloat16, param.device)
    for t in (grad, exp_avg, exp_avg_sq, param_bf16):
        if t is not None and t.numel() != param.numel():
            raise ValueError("adamw_step_master: sizes differ")
    rc = lib().adamw_step_master_hip(_p(param), _p(grad), _p(exp_avg), _p(exp_avg_sq),
                                     _p(param_bf16), param.numel(), float(lr), float(beta1),
                                     float(beta2), float(eps), float(weight_decay), int(step),
                                     _stream(param))
    check(rc, "adamw_step_master_hip")


def embedding_forward(indices: torch.Tensor, weight: torch.Tensor,
                      checked: bool = True) -> torch.Tensor:
    """weight[indices] for int32 indices and a (vocab, dim) bf16 table; with
    ``checked`` an out-of-range index gives a zero row."""
    _require(indices, "indices", torch.int32)
    _require(weight, "weight", torch.bfloat16, indices.device)
    V, D = weight.shape
    out = torch.empty(*indices.shape, D, dtype=torch.bfloat16, device=weight.device)
    if checked:
        rc = lib().embedding_forward_checked_hip(_p(indices), _p(weight), _p(out),
                                                 indices.numel(), V, D, _stream(weight))
        check(rc, "embedding_forward_checked_hip")
    else:
        rc = lib().embedding_forward_hip(_p(indices), _p(weight), _p(out), indices.numel(), D,
                                         _stream(weight))
        check(rc, "embedding_forward_hip")
    return out


def embedding_backward(grad_output: torch.Tensor, indices: torch.Tensor, grad_weight) -> None:
    """grad_weight (vocab, dim) fp32 += scatter of grad_output rows by index."""
    _require(indices, "indices", torch.int32)
    _require(grad_output, "grad_output", torch.bfloat16, indices.device)
    _require(grad_weight, "grad_weight", torch.float32, indices.device)
    V, D = grad_weight.shape
    rc = lib().embedding_backward_hip(_p(grad_output), _p(indices), _p(grad_weight),
                                      indices.numel(), V, D, _stream(grad_weight))
    check(rc, "embedding_backward_hip")


def cross_entropy_forward(logits: torch.Tensor, targets: torch.Tensor,
                          label_smoothing: float = 0.0) -> torch.Tensor:
    """Per-row loss / batch, fp32 (B,): its sum is the mean loss."""
    _require(logits, "logits", torch.bfloat16)
    _require(targets, "targets", torch.int32, logits.device)
    B, V = logits.shape
    loss = torch.empty(B, dtype=torch.float32, device=logits.device)
    rc = lib().cross_entropy_forward_hip(_p(logits), _p(targets), _p(loss), B, V,
                                         float(label_smoothing), _stream(logits))
    check(rc, "cross_entropy_forward_hip")
    return loss


def cross_entropy_forward_backward(logits: torch.Tensor, targets: torch.Tensor,
                                   label_smoothing: float = 0.0,
                                   grad_loss=None, in_place: bool = False):
    """(per-row loss / batch fp32 (B,), dL/dlogits bf16) from one read of the
    logits; dL/dloss[i] = grad_loss[i], or 1 for every row when None.  With
    in_place the gradient overwrites ``logits``."""
    _require(logits, "logits", torch.bfloat16)
    _require(targets, "targets", torch.int32, logits.device)
    if grad_loss is not None:
        _require(grad_loss, "grad_loss", torch.float32, logits.device)
    B, V = logits.shape
    loss = torch.empty(B, dtype=torch.float32, device=logits.device)
    g = logits if in_place else torch.empty_like(logits)
    rc = lib().cross_entropy_forward_backward_hip(_p(logits), _p(targets), _p(grad_loss),
                                                  _p(loss), _p(g), B, V,
                                                  float(label_smoothing), _stream(logits))
    check(rc, "cross_entropy_forward_backward_hip")
    return loss, g


def cross_entropy_backward(grad_loss: torch.Tensor, logits: torch.Tensor, targets: torch.Tensor,
                           label_smoothing: float = 0.0) -> torch.Tensor:
    """dL/dlogits (bf16) given dL/dloss[i] (fp32, (B,))."""
    _require(logits, "logits", torch.bfloat16)
    _require(targets, "targets", torch.int32, logits.device)
    _require(grad_loss, "grad_loss", torch.float32, logits.device)
    B, V = logits.shape
    g = torch.empty_like(logits)
    rc = lib().cross_entropy_backward_hip(_p(grad_loss), _p(logits), _p(targets), _p(g), B, V,
                                          float(label_smoothing), _stream(logits))
    check(rc, "cross_entropy_backward_hip")
    return g
