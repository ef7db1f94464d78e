"""Pins for the Mode Q oracle (query readout, per-token beta, d_k != d_v, varlen).

Every check here compares the oracle with something it does not contain:
closed forms, a library matrix exponential, central differences, torch
autograd, or a different algorithm (the chunked WY form).
"""
import numpy as np
import pytest
import scipy.linalg
import torch


def _inputs(oracle, seed, n_tok, H, K, V, bf16=False):
    d = oracle.make_efla_inputs(seed, n_tok, H, K, V, bf16=bf16)
    return {k: v.astype(np.float64) for k, v in d.items()}


def test_one_token_closed_form(oracle):
    # From S_0 = 0 one token gives S_1 = c k v^T, hence o_1 = c (q.k) v.
    d = _inputs(oracle, 11, 1, 3, 8, 5)
    o, st = oracle.q_forward(d["q"], d["k"], d["v"], d["beta"])
    for h in range(3):
        k, v, q, b = d["k"][0, h], d["v"][0, h], d["q"][0, h], d["beta"][0, h]
        lam = k @ k
        c = -np.expm1(-b * lam) / lam
        np.testing.assert_allclose(o[0, h], c * (q @ k) * v, rtol=1e-13, atol=1e-15)
        np.testing.assert_allclose(st[0, h], c * np.outer(k, v), rtol=1e-13, atol=1e-15)


def test_one_step_matrix_exponential(oracle):
    # The EFLA step is the exact solution of dS/dt = -k k^T S + k v^T over time
    # beta: S_1 = expm(-beta k k^T) S_0 + (I - expm(-beta k k^T)) k v^T / lambda.
    rng = np.random.default_rng(3)
    K, V = 7, 4
    for trial in range(5):
        k = rng.standard_normal(K) * rng.uniform(0.2, 2.0)
        v = rng.standard_normal(V)
        q = rng.standard_normal(K)
        b = rng.uniform(0.05, 2.0)
        S0 = rng.standard_normal((K, V))
        _, st = oracle.q_forward(q[None, None], k[None, None], v[None, None],
                                 np.array([[b]]), S0=S0[None, None])
        E = scipy.linalg.expm(-b * np.outer(k, k))
        ref = E @ S0 + (np.eye(K) - E) @ np.outer(k, v) / (k @ k)
        np.testing.assert_allclose(st[0, 0], ref, rtol=1e-12, atol=1e-12)


def test_residual_contraction(oracle):
    # v_t - S_t^T k_t = exp(-beta lambda) (v_t - S_{t-1}^T k_t)
    rng = np.random.default_rng(5)
    K, V = 6, 9
    S0 = rng.standard_normal((K, V))
    k, v, q = rng.standard_normal(K), rng.standard_normal(V), rng.standard_normal(K)
    b = 0.8
    _, st = oracle.q_forward(q[None, None], k[None, None], v[None, None], np.array([[b]]),
                             S0=S0[None, None])
    lhs = v - st[0, 0].T @ k
    rhs = np.exp(-b * (k @ k)) * (v - S0.T @ k)
    np.testing.assert_allclose(lhs, rhs, rtol=1e-12, atol=1e-13)


def test_beta_zero_keeps_state(oracle):
    d = _inputs(oracle, 12, 20, 2, 8, 8)
    S0 = np.random.default_rng(0).standard_normal((1, 2, 8, 8))
    o, st = oracle.q_forward(d["q"], d["k"], d["v"], np.zeros_like(d["beta"]), S0=S0)
    np.testing.assert_array_equal(st, S0)
    np.testing.assert_allclose(o, np.einsum("thk,hkv->thv", d["q"], S0[0]), rtol=1e-13)


def _torch_recurrence(q, k, v, beta, S0):
    """Independent restatement in matrix form: S <- (I - c k k^T) S + c k v^T."""
    T, H, K = q.shape
    outs = []
    S = S0
    eye = torch.eye(K, dtype=q.dtype)
    for t in range(T):
        kt = k[t]
        lam = (kt * kt).sum(-1)
        c = -torch.expm1(-beta[t] * lam) / lam
        A = eye - c[:, None, None] * kt[:, :, None] * kt[:, None, :]
        S = A @ S + c[:, None, None] * kt[:, :, None] * v[t][:, None, :]
        outs.append(torch.einsum("hkv,hk->hv", S, q[t]))
    return torch.stack(outs), S


@pytest.mark.parametrize("K,V", [(8, 8), (6, 10)])
def test_backward_matches_autograd(oracle, K, V):
    T, H = 37, 2
    d = _inputs(oracle, 21, T, H, K, V)
    rng = np.random.default_rng(9)
    S0 = rng.standard_normal((1, H, K, V)) * 0.3
    dST = rng.standard_normal((1, H, K, V))
    tq, tk, tv, tb = (torch.tensor(d[n], requires_grad=True) for n in ("q", "k", "v", "beta"))
    tS0 = torch.tensor(S0[0], requires_grad=True)
    o, st = _torch_recurrence(tq, tk, tv, tb, tS0)
    loss = (o * torch.tensor(d["do"])).sum() + (st * torch.tensor(dST[0])).sum()
    loss.backward()
    o_or, st_or = oracle.q_forward(d["q"], d["k"], d["v"], d["beta"], S0=S0)
    np.testing.assert_allclose(o_or, o.detach().numpy(), rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(st_or[0], st.detach().numpy(), rtol=1e-11, atol=1e-12)
    dq, dk, dv, db, dS0 = oracle.q_backward(d["q"], d["k"], d["v"], d["beta"], d["do"],
                                            S0=S0, dST=dST)
    for ours, ref in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad), (db, tb.grad),
                      (dS0[0], tS0.grad)):
        np.testing.assert_allclose(ours, ref.numpy(), rtol=1e-10, atol=1e-11)


def test_backward_central_differences(oracle):
    T, H, K, V = 9, 1, 4, 3
    d = _inputs(oracle, 31, T, H, K, V)
    do = d["do"]

    def loss(q, k, v, b):
        o, _ = oracle.q_forward(q, k, v, b)
        return float((o * do).sum())

    dq, dk, dv, db, _ = oracle.q_backward(d["q"], d["k"], d["v"], d["beta"], do)
    eps = 1e-6
    for name, grad in (("q", dq), ("k", dk), ("v", dv), ("beta", db)):
        arr = d[name]
        flat = arr.reshape(-1)
        g = grad.reshape(-1)
        for i in range(0, flat.size, max(1, flat.size // 12)):
            args = {n: d[n].copy() for n in ("q", "k", "v", "beta")}
            args[name].reshape(-1)[i] += eps
            lp = loss(args["q"], args["k"], args["v"], args["beta"])
            args[name].reshape(-1)[i] -= 2 * eps
            lm = loss(args["q"], args["k"], args["v"], args["beta"])
            assert g[i] == pytest.approx((lp - lm) / (2 * eps), rel=1e-5, abs=1e-7), (name, i)


def test_varlen_equals_independent_runs(oracle):
    H, K, V = 2, 8, 16
    lens = [5, 64, 1, 70, 33]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    d = _inputs(oracle, 41, int(cu[-1]), H, K, V)
    rng = np.random.default_rng(1)
    S0 = rng.standard_normal((len(lens), H, K, V)) * 0.2
    dST = rng.standard_normal((len(lens), H, K, V))
    o, st = oracle.q_forward(d["q"], d["k"], d["v"], d["beta"], cu_seqlens=cu, S0=S0)
    g = oracle.q_backward(d["q"], d["k"], d["v"], d["beta"], d["do"], cu_seqlens=cu, S0=S0,
                          dST=dST)
    for i in range(len(lens)):
        sl = slice(cu[i], cu[i + 1])
        oi, sti = oracle.q_forward(d["q"][sl], d["k"][sl], d["v"][sl], d["beta"][sl],
                                   S0=S0[i:i + 1])
        np.testing.assert_array_equal(o[sl], oi)
        np.testing.assert_array_equal(st[i], sti[0])
        gi = oracle.q_backward(d["q"][sl], d["k"][sl], d["v"][sl], d["beta"][sl], d["do"][sl],
                               S0=S0[i:i + 1], dST=dST[i:i + 1])
        for a, b in zip(g[:4], gi[:4]):
            np.testing.assert_array_equal(a[sl], b)
        np.testing.assert_array_equal(g[4][i], gi[4][0])


def test_batch_layout_equals_varlen(oracle):
    B, T, H, K, V = 3, 20, 2, 8, 8
    d = _inputs(oracle, 42, B * T, H, K, V)
    o1, s1 = oracle.q_forward(d["q"], d["k"], d["v"], d["beta"], T=T)
    cu = np.arange(0, B * T + 1, T, dtype=np.int32)
    o2, s2 = oracle.q_forward(d["q"], d["k"], d["v"], d["beta"], cu_seqlens=cu)
    np.testing.assert_array_equal(o1, o2)
    np.testing.assert_array_equal(s1, s2)


@pytest.mark.parametrize("C", [1, 16, 64, 150])
def test_chunked_algorithm_equals_sequential(oracle, C):
    L, H, K, V = 150, 1, 16, 24
    d = _inputs(oracle, 51, L, H, K, V)
    rng = np.random.default_rng(2)
    S0 = rng.standard_normal((K, V)) * 0.3
    dST = rng.standard_normal((K, V))
    o_seq, st_seq = oracle.q_forward(d["q"], d["k"], d["v"], d["beta"], S0=S0[None, None])
    q, k, v, b, do = (d[n][:, 0] for n in ("q", "k", "v", "beta", "do"))
    o_ch, st_ch, _ = oracle.chunk_forward(q, k, v, b, C=C, S0=S0)
    np.testing.assert_allclose(o_ch, o_seq[:, 0], rtol=1e-10, atol=1e-11)
    np.testing.assert_allclose(st_ch, st_seq[0, 0], rtol=1e-10, atol=1e-11)
    g_seq = oracle.q_backward(d["q"], d["k"], d["v"], d["beta"], d["do"], S0=S0[None, None],
                              dST=dST[None, None])
    g_ch = oracle.chunk_backward(q, k, v, b, do, C=C, S0=S0, dST=dST)
    for a, bb in zip(g_ch[:4], g_seq[:4]):
        np.testing.assert_allclose(a, bb[:, 0], rtol=1e-9, atol=1e-10)
    np.testing.assert_allclose(g_ch[4], g_seq[4][0, 0], rtol=1e-9, atol=1e-10)


def test_fp32_oracle_tracks_fp64(oracle):
    B, T, H, K, V = 2, 256, 4, 64, 64
    d = oracle.make_efla_inputs(61, B * T, H, K, V, bf16=False)
    o64, _ = oracle.q_forward(d["q"], d["k"], d["v"], d["beta"], T=T)
    o32, _ = oracle.q_forward(d["q"], d["k"], d["v"], d["beta"], T=T, dtype=np.float32)
    rel = np.linalg.norm(o32 - o64) / np.linalg.norm(o64)
    assert rel < 1e-5
    g64 = oracle.q_backward(d["q"], d["k"], d["v"], d["beta"], d["do"], T=T)
    g32 = oracle.q_backward(d["q"], d["k"], d["v"], d["beta"], d["do"], T=T, dtype=np.float32)
    for a, b in zip(g32, g64):
        assert np.linalg.norm(a - b) / np.linalg.norm(b) < 1e-5


def test_segments_compose_affinely(oracle):
    """The state after two segments is A2 (A1 S0 + B1) + B2 with A the
    product of (I - c k k^T) and B the final state from zero; A is also the
    recurrence's final state from S0 = I with v = 0 (the transition the
    affine state scan consumes)."""
    rng = np.random.default_rng(21)
    H, K, V, T1, T2 = 2, 6, 5, 9, 7
    x = oracle.make_efla_inputs(31, T1 + T2, H, K, V, bf16=False)
    q, k, v, b = x["q"], x["k"], x["v"], x["beta"]
    S0 = rng.standard_normal((1, H, K, V))

    def prod(kk, bb):
        A = np.broadcast_to(np.eye(K), (H, K, K)).copy()
        for t in range(kk.shape[0]):
            kt = kk[t].astype(np.float64)
            lam = (kt ** 2).sum(-1)
            c = -np.expm1(-bb[t].astype(np.float64) * lam) / lam
            M = np.eye(K) - c[:, None, None] * np.einsum("hi,hj->hij", kt, kt)
            A = M @ A
        return A

    s1, s2 = slice(0, T1), slice(T1, T1 + T2)
    A1, A2 = prod(k[s1], b[s1]), prod(k[s2], b[s2])
    _, B1 = oracle.q_forward(q[s1], k[s1], v[s1], b[s1], T=T1)
    _, B2 = oracle.q_forward(q[s2], k[s2], v[s2], b[s2], T=T2)
    _, S_ref = oracle.q_forward(q, k, v, b, T=T1 + T2, S0=S0)
    S_comp = A2 @ (A1 @ S0[0] + B1[0]) + B2[0]
    assert np.abs(S_comp - S_ref[0]).max() < 1e-12
    eye = np.broadcast_to(np.eye(K), (1, H, K, K)).copy()
    _, A1_rec = oracle.q_forward(q[s1], k[s1], np.zeros((T1, H, K)), b[s1], T=T1, S0=eye)
    assert np.abs(A1_rec[0] - A1).max() < 1e-12
