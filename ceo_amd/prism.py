"""ShortConv and the PRISM layer that consumes the EFLA output.

Mirrors the reference's ``ShortConv`` (src/model/prism.zig:359-474: weight
(hidden_dim, window) ~ N(0, 1/window), causal depthwise convolution) and
``PrismLayer`` (prism.zig:41-357: ``forward(input, v)`` runs ShortConv on the
normed input to get the proxy u, then the iterative refinement on (u, v)),
as its ``TransformerBlock`` calls them (src/model/model.zig:169-176).  The
refinement is the one the reference executes (``prismForwardCpu``,
prism.zig:251-323); the backward is the gradient of that forward (the
reference's ``backward`` returns zeros, prism.zig:326-356).  All compute is in
``libefla_hip.so``.
"""
from __future__ import annotations

import ctypes
import math

import torch

from ._lib import check, lib
from .efla import _p, _require, _stream

MAX_ITERATIONS = 16


def shortconv_forward(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """y = ShortConv(x) for x (B, T, C) bf16 and weight (C, W) bf16."""
    _require(x, "x", torch.bfloat16)
    _require(weight, "weight", torch.bfloat16, x.device)
    B, T, C = x.shape
    if weight.dim() != 2 or weight.shape[0] != C:
        raise ValueError("weight must be (hidden_dim, window)")
    y = torch.empty_like(x)
    rc = lib().shortconv_forward_hip(_p(x), _p(weight), _p(y), B, T, C, weight.shape[1],
                                     _stream(x))
    check(rc, "shortconv_forward_hip")
    return y


def shortconv_backward(dy, x, weight, grad_weight=None, need_input_grad: bool = True,
                       need_weight_grad: bool = True):
    """(dx bf16 or None, dweight fp32 or None); dweight is added into
    ``grad_weight`` when given, else into a new zero buffer."""
    for t, n in ((dy, "dy"), (x, "x"), (weight, "weight")):
        _require(t, n, torch.bfloat16, x.device)
    B, T, C = x.shape
    W = weight.shape[1]
    dx = torch.empty_like(x) if need_input_grad else None
    dw = None
    if need_weight_grad:
        if grad_weight is None:
            dw = torch.zeros(C, W, dtype=torch.float32, device=x.device)
        else:
            _require(grad_weight, "grad_weight", torch.float32, x.device)
            dw = grad_weight
    rc = lib().shortconv_backward_hip(_p(dy), _p(x), _p(weight), _p(dx), _p(dw), B, T, C, W,
                                      _stream(x))
    check(rc, "shortconv_backward_hip")
    return dx, dw


def _ptr_array(ts):
    return (ctypes.c_void_p * max(1, len(ts)))(*[t.data_ptr() for t in ts])


def prism_forward(u, v, w_p, head_dim: int, w_beta=None, w_k=None, prev_state=None,
                  alpha: float = 0.99, want_state: bool = True):
    """(output (B, T, C) bf16, new_state (1, head_dim, head_dim) bf16 or None)."""
    _require(u, "u", torch.bfloat16)
    _require(v, "v", torch.bfloat16, u.device)
    if u.shape != v.shape:
        raise ValueError("u and v must have the same shape")
    for i, w in enumerate(w_p):
        _require(w, f"w_p[{i}]", torch.bfloat16, u.device)
        if w.numel() < head_dim:
            raise ValueError("each w_p[l] must hold at least head_dim values")
    B, T, C = u.shape
    out = torch.empty_like(u)
    state = (torch.empty(1, head_dim, head_dim, dtype=torch.bfloat16, device=u.device)
             if want_state else None)
    wb = _ptr_array(w_beta) if w_beta else None
    wk = _ptr_array(w_k) if w_k else None
    rc = lib().prism_forward_hip(_p(u), _p(v), _p(prev_state), _p(state), _p(out), wb, wk,
                                 _ptr_array(w_p), B, T, C, head_dim, len(w_p), float(alpha),
                                 _stream(u))
    check(rc, "prism_forward_hip")
    return out, state


def prism_backward(grad_output, u, v, w_p, head_dim: int, grad_w_p=None):
    """(grad_u, grad_v) bf16; the w_p gradients are added into ``grad_w_p``
    (a list of fp32 tensors, one per iteration) when given."""
    for t, n in ((grad_output, "grad_output"), (u, "u"), (v, "v")):
        _require(t, n, torch.bfloat16, u.device)
    B, T, C = u.shape
    gu = torch.empty_like(u)
    gv = torch.empty_like(v)
    gw = None
    if grad_w_p is not None:
        if len(grad_w_p) != len(w_p):
            raise ValueError("grad_w_p needs one tensor per iteration")
        for i, g in enumerate(grad_w_p):
            _require(g, f"grad_w_p[{i}]", torch.float32, u.device)
        gw = (ctypes.c_void_p * max(1, len(grad_w_p)))(*[g.data_ptr() for g in grad_w_p])
    rc = lib().prism_backward_hip(_p(grad_output), _p(u), _p(v), _ptr_array(w_p), _p(gu),
                                  _p(gv), gw, B, T, C, head_dim, len(w_p), _stream(u))
    check(rc, "prism_backward_hip")
    return gu, gv


class ShortConv:
    """Causal depthwise convolution, weight (hidden_dim, window) bf16
    (prism.zig:359-410)."""

    def __init__(self, hidden_dim: int, window_size: int, device="cuda", generator=None):
        std = math.sqrt(1.0 / window_size)
        w = torch.randn(hidden_dim, window_size, generator=generator) * std
        self.weight = w.to(torch.bfloat16).to(device)
        self.grad_weight = torch.zeros(hidden_dim, window_size, dtype=torch.float32,
                                       device=device)

    def forward(self, x):
        return shortconv_forward(x, self.weight)

    def backward(self, dy, x):
        dx, _ = shortconv_backward(dy, x, self.weight, grad_weight=self.grad_weight)
        return dx


class PrismLayer:
    """The reference's PrismLayer with its parameters (per iteration W_beta,
    W_k, W_p of (hidden_dim, head_dim) ~ N(0, 2/hidden_dim), prism.zig:217-236)
    and the refinement it executes.  ``forward(input, v)`` returns
    (output, new_state); ``backward(grad_output)`` returns (grad_input, grad_v)
    and adds into ``shortconv.grad_weight`` and ``grad_w_p``."""

    def __init__(self, hidden_dim: int, head_dim: int, num_iterations: int = 3,
                 window_size: int = 64, forget_factor: float = 0.99, device="cuda", seed=0):
        if num_iterations > MAX_ITERATIONS:
            raise ValueError(f"at most {MAX_ITERATIONS} iterations")
        g = torch.Generator().manual_seed(seed)
        self.hidden_dim, self.head_dim = hidden_dim, head_dim
        self.alpha = forget_factor
        self.shortconv = ShortConv(hidden_dim, window_size, device, g)
        std = math.sqrt(2.0 / hidden_dim)

        def mats():
            return [(torch.randn(hidden_dim, head_dim, generator=g) * std)
                    .to(torch.bfloat16).to(device) for _ in range(num_iterations)]

        self.w_beta, self.w_k, self.w_p = mats(), mats(), mats()
        self.grad_w_p = [torch.zeros(hidden_dim, head_dim, dtype=torch.float32, device=device)
                         for _ in range(num_iterations)]
        self._saved = None

    def forward(self, x, v, state=None):
        u = self.shortconv.forward(x)
        out, new_state = prism_forward(u, v, self.w_p, self.head_dim, self.w_beta, self.w_k,
                                       state, self.alpha)
        self._saved = (x, u, v)
        return out, new_state

    def backward(self, grad_output):
        if self._saved is None:
            raise RuntimeError("backward before forward")
        x, u, v = self._saved
        gu, gv = prism_backward(grad_output, u, v, self.w_p, self.head_dim,
                                [g.view(-1) for g in self.grad_w_p])
        grad_input = self.shortconv.backward(gu, x)
        return grad_input, gv
