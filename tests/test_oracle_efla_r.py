"""Pins for the Mode R oracle: the reference ABI (efla.cu:482-748) restated."""
import ctypes

import numpy as np
import pytest
import torch


def _bf16_inputs(oracle, seed, B, T, H, d):
    x = oracle.make_efla_inputs(seed, B * T, H, d, d, bf16=True, with_q=False)
    k = oracle.f32_to_bf16(x["k"]).reshape(B, T, H, d)
    v = oracle.f32_to_bf16(x["v"]).reshape(B, T, H, d)
    do = oracle.f32_to_bf16(x["do"]).reshape(B, T, H, d)
    return k, v, do


def test_forward_validation_order(oracle):
    L = oracle.lib()
    buf = np.zeros(16, dtype=np.uint16)
    p = buf.ctypes.data_as(oracle.c_u16p)
    null = oracle.c_u16p()
    # zero B/H/d -> InvalidValue, checked before T == 0 (efla.cu:497-502)
    assert L.or_efla_r_forward(p, p, p, p, 0, 0, 1, 1, 1.0) == 1
    assert L.or_efla_r_forward(p, p, p, p, 1, 1, 0, 1, 1.0) == 1
    assert L.or_efla_r_forward(p, p, p, p, 1, 1, 1, 0, 1.0) == 1
    # T == 0 -> success even with null pointers (checked before the null checks)
    assert L.or_efla_r_forward(null, null, null, null, 1, 0, 1, 1, 1.0) == 0
    assert L.or_efla_r_forward(p, null, p, p, 1, 1, 1, 1, 1.0) == 1
    # B*H beyond the 32-bit grid -> InvalidConfiguration (efla.cu:507-513)
    assert L.or_efla_r_forward(p, p, p, p, 1 << 31, 1, 4, 1, 1.0) == 9


def test_backward_validation_order(oracle):
    L = oracle.lib()
    buf = np.full(64, 0x3F80, dtype=np.uint16)
    p = buf.ctypes.data_as(oracle.c_u16p)
    null = oracle.c_u16p()
    assert L.or_efla_r_backward(p, p, p, p, p, p, p, 0, 1, 1, 1, 1.0) == 1
    assert L.or_efla_r_backward(p, p, p, null, p, p, p, 1, 1, 1, 1, 1.0) == 1
    assert L.or_efla_r_backward(p, p, p, p, p, p, null, 1, 1, 1, 1, 1.0) == 1
    # T == 0 zeroes grad_state and ignores the other pointers (efla.cu:582-584)
    gs = np.full(4, 0x3F80, dtype=np.uint16)
    assert L.or_efla_r_backward(null, null, null, p, null, null,
                                gs.ctypes.data_as(oracle.c_u16p), 1, 0, 1, 2, 1.0) == 0
    assert not gs.any()
    assert L.or_efla_r_backward(null, p, p, p, p, p, p, 1, 1, 1, 2, 1.0) == 1
    assert L.or_efla_r_backward(p, p, p, p, p, p, p, 1 << 31, 1, 4, 1, 1.0) == 9


def test_one_token_closed_form(oracle):
    # S_0 = 0, one token: S_1 = c k v^T and o_1 = S_1 k = c (v.k) k.
    B, T, H, d = 1, 1, 2, 16
    k, v, _ = _bf16_inputs(oracle, 5, B, T, H, d)
    st = np.zeros((B * H, d, d), dtype=np.uint16)
    beta = 0.7
    rc, out = oracle.r_forward(k, v, st, B, T, H, d, beta)
    assert rc == 0
    kf, vf = oracle.bf16_to_f32(k)[0, 0], oracle.bf16_to_f32(v)[0, 0]
    for h in range(H):
        lam = float((kf[h].astype(np.float64) ** 2).sum())
        c = -np.expm1(-beta * lam) / lam
        ref = c * (vf[h] @ kf[h]) * kf[h]
        np.testing.assert_allclose(oracle.bf16_to_f32(out[0, 0, h]), ref, rtol=8e-3, atol=1e-6)
        np.testing.assert_allclose(oracle.bf16_to_f32(st[h]), c * np.outer(kf[h], vf[h]),
                                   rtol=8e-3, atol=1e-6)


def _torch_mode_r(k, v, beta, S0):
    """Independent restatement: S <- (I - c k k^T) S + c k v^T, o = S k."""
    T, H, d = k.shape
    eye = torch.eye(d, dtype=k.dtype)
    S = S0
    outs = []
    for t in range(T):
        kt = k[t]
        lam = (kt * kt).sum(-1)
        c = -torch.expm1(-beta * lam) / lam
        S = (eye - c[:, None, None] * kt[:, :, None] * kt[:, None, :]) @ S + \
            c[:, None, None] * kt[:, :, None] * v[t][:, None, :]
        outs.append(torch.einsum("hij,hj->hi", S, kt))
    return torch.stack(outs), S


def test_backward_formulas_match_autograd(oracle):
    # With the per-token bf16 rounding switched off the restated backward
    # (efla.cu:315-454) must be the exact gradient of the restated forward.
    B, T, H, d = 1, 24, 2, 16
    k, v, do = _bf16_inputs(oracle, 7, B, T, H, d)
    rng = np.random.default_rng(4)
    S0 = oracle.f32_to_bf16((rng.standard_normal((H, d, d)) * 0.2).astype(np.float32))
    beta = 0.9
    oracle.r_exact(True)
    try:
        st = S0.copy()
        rc, out = oracle.r_forward(k, v, st, B, T, H, d, beta)
        assert rc == 0
        rc, gk, gv, gs = oracle.r_backward(do, k, v, S0, B, T, H, d, beta)
        assert rc == 0
    finally:
        oracle.r_exact(False)
    tk = torch.tensor(oracle.bf16_to_f32(k)[0].astype(np.float64), requires_grad=True)
    tv = torch.tensor(oracle.bf16_to_f32(v)[0].astype(np.float64), requires_grad=True)
    tS = torch.tensor(oracle.bf16_to_f32(S0).astype(np.float64), requires_grad=True)
    o, _ = _torch_mode_r(tk, tv, beta, tS)
    (o * torch.tensor(oracle.bf16_to_f32(do)[0].astype(np.float64))).sum().backward()
    np.testing.assert_allclose(oracle.bf16_to_f32(out)[0], o.detach().numpy(), rtol=1e-2,
                               atol=2e-3)
    for ours, ref in ((gk[0], tk.grad), (gv[0], tv.grad), (gs, tS.grad)):
        got = oracle.bf16_to_f32(ours).astype(np.float64)
        r = ref.numpy()
        assert np.linalg.norm(got - r) / np.linalg.norm(r) < 4e-3


def test_bf16_trajectory_stays_near_exact(oracle):
    # Rounding the state to bf16 every token (efla.cu:218-220) drifts from the
    # fp32 trajectory but stays bounded (the update is a contraction).
    B, T, H, d = 2, 256, 4, 64
    k, v, _ = _bf16_inputs(oracle, 8, B, T, H, d)
    st0 = np.zeros((B * H, d, d), dtype=np.uint16)
    st = st0.copy()
    _, out = oracle.r_forward(k, v, st, B, T, H, d, 0.6)
    oracle.r_exact(True)
    try:
        st2 = st0.copy()
        _, out2 = oracle.r_forward(k, v, st2, B, T, H, d, 0.6)
    finally:
        oracle.r_exact(False)
    a, b = oracle.bf16_to_f32(out), oracle.bf16_to_f32(out2)
    rel = np.linalg.norm(a - b) / np.linalg.norm(b)
    assert 1e-4 < rel < 3e-2


def test_mode_r_and_q_share_final_state(oracle):
    # Both readouts run the same state recurrence; with scalar beta and the same
    # k, v the Mode Q fp64 final state matches Mode R's up to its bf16 drift.
    B, T, H, d = 1, 96, 2, 32
    k, v, _ = _bf16_inputs(oracle, 9, B, T, H, d)
    st = np.zeros((B * H, d, d), dtype=np.uint16)
    oracle.r_exact(True)
    try:
        oracle.r_forward(k, v, st, B, T, H, d, 0.5)
    finally:
        oracle.r_exact(False)
    kf = oracle.bf16_to_f32(k).reshape(T, H, d).astype(np.float64)
    vf = oracle.bf16_to_f32(v).reshape(T, H, d).astype(np.float64)
    _, ST = oracle.q_forward(kf, kf, vf, np.full((T, H), 0.5))
    got = oracle.bf16_to_f32(st)
    assert np.linalg.norm(got - ST[0]) / np.linalg.norm(ST[0]) < 5e-3


def test_chunked_scan_is_bf16_prefix_sum(oracle):
    rng = np.random.default_rng(1)
    H, d, n = 2, 8, 5
    vals = [rng.standard_normal((H, d, d)).astype(np.float32) for _ in range(n)]
    chunks = [oracle.f32_to_bf16(x) for x in vals]
    assert oracle.r_chunked_scan(chunks, H, d) == 0
    run = oracle.bf16_to_f32(oracle.f32_to_bf16(vals[0]))
    for i in range(1, n):
        run = oracle.round_bf16(run + oracle.round_bf16(vals[i]))
        np.testing.assert_array_equal(oracle.bf16_to_f32(chunks[i]), run)
    L = oracle.lib()
    arr = (oracle.c_u16p * 2)(chunks[0].ctypes.data_as(oracle.c_u16p), oracle.c_u16p())
    assert L.or_efla_r_chunked_scan(arr, 2, H, d) == 1
    assert L.or_efla_r_chunked_scan(arr, 0, H, d) == 1
    assert L.or_efla_r_chunked_scan(ctypes.cast(None, ctypes.POINTER(oracle.c_u16p)), 2, H,
                                    d) == 1
