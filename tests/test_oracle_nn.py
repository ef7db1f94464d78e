"""Pins for the oracle's LayerNorm, GELU and AdamW (CPU only).

LayerNorm follows layernorm.cu:133-183 (eps inside the rsqrt, optional bias);
its gradient is the textbook one.  GELU is the tanh approximation of
layernorm.cu:189-250.  AdamW is optim.cu:147-178 with fp32 master weights.
Each is checked against an independent statement: numpy fp64 formulas, torch
fp64 autograd / torch's own GELU, invariants and a one-step closed form.
"""
import numpy as np
import pytest
import torch


def test_layernorm_forward_formula_and_invariants(oracle):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((7, 96)) * 3 + 2).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(96)).astype(np.float32)
    b = (0.1 * rng.standard_normal(96)).astype(np.float32)
    y, mean, rstd = oracle.layernorm_fwd(x, w, b, 1e-5)
    xd = x.astype(np.float64)
    mu = xd.mean(1, keepdims=True)
    var = ((xd - mu) ** 2).mean(1, keepdims=True)
    ref = (xd - mu) / np.sqrt(var + 1e-5) * w + b
    assert np.abs(y - ref).max() < 1e-5
    assert np.allclose(mean, mu[:, 0], rtol=1e-6)
    assert np.allclose(rstd, 1 / np.sqrt(var[:, 0] + 1e-5), rtol=1e-5)
    # w = 1, b = 0: each row has mean 0 and variance var / (var + eps)
    y1, _, _ = oracle.layernorm_fwd(x, np.ones(96, np.float32), None, 1e-5)
    assert np.abs(y1.mean(1)).max() < 1e-6
    assert np.abs(y1.var(1) - var[:, 0] / (var[:, 0] + 1e-5)).max() < 1e-5


def test_layernorm_backward_matches_autograd(oracle):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 48)).astype(np.float32)
    w = (1 + 0.2 * rng.standard_normal(48)).astype(np.float32)
    b = (0.1 * rng.standard_normal(48)).astype(np.float32)
    dy = rng.standard_normal((5, 48)).astype(np.float32)
    _, mean, rstd = oracle.layernorm_fwd(x, w, b, 1e-5)
    dx, dw, db = oracle.layernorm_bwd(dy, x, w, mean, rstd)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    bt = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    yt = torch.nn.functional.layer_norm(xt, (48,), wt, bt, 1e-5)
    (yt * torch.tensor(dy, dtype=torch.float64)).sum().backward()
    assert np.abs(dx - xt.grad.numpy()).max() < 1e-4
    assert np.abs(dw - wt.grad.numpy()).max() < 1e-4
    assert np.abs(db - bt.grad.numpy()).max() < 1e-6


def test_gelu_matches_torch_tanh_gelu(oracle):
    x = np.linspace(-8, 8, 1001).astype(np.float32)
    y = oracle.gelu_fwd(x)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    yt = torch.nn.functional.gelu(xt, approximate="tanh")
    assert np.abs(y - yt.detach().numpy()).max() < 1e-6
    dy = np.cos(x).astype(np.float32)
    (yt * torch.tensor(dy, dtype=torch.float64)).sum().backward()
    assert np.abs(oracle.gelu_bwd(dy, x) - xt.grad.numpy()).max() < 1e-6
    # special values: gelu(0) = 0, gelu(x) -> x for large x, -> 0 for very negative x
    assert oracle.gelu_fwd(np.array([0.0, 30.0, -30.0], np.float32)).tolist() == [0.0, 30.0, 0.0]


@pytest.mark.parametrize("step", [1, 7])
def test_adamw_step_closed_form(oracle, step):
    rng = np.random.default_rng(3)
    n = 64
    p = rng.standard_normal(n).astype(np.float32)
    g = rng.standard_normal(n).astype(np.float32)
    m = (0.1 * rng.standard_normal(n)).astype(np.float32) if step > 1 else np.zeros(n, np.float32)
    v = np.abs(0.1 * rng.standard_normal(n)).astype(np.float32) if step > 1 else np.zeros(n, np.float32)
    lr, b1, b2, eps, wd = 3e-4, 0.9, 0.999, 1e-8, 0.1
    p0, m0, v0 = p.astype(np.float64), m.astype(np.float64), v.astype(np.float64)
    mn = b1 * m0 + (1 - b1) * g
    vn = b2 * v0 + (1 - b2) * g.astype(np.float64) ** 2
    ref = p0 * (1 - lr * wd) - lr * (mn / (1 - b1 ** step)) / (np.sqrt(vn / (1 - b2 ** step)) + eps)
    oracle.adamw_step(p, g, m, v, lr, b1, b2, eps, wd, step)
    assert np.abs(p - ref).max() < 1e-6
    assert np.abs(m - mn).max() < 1e-7 and np.abs(v - vn).max() < 1e-7
    if step == 1:
        # from a zero state one step is p(1 - lr wd) - lr g / (|g| + eps)
        kat = p0 * (1 - lr * wd) - lr * g / (np.abs(g) + eps)
        assert np.abs(p - kat).max() < 1e-6


def test_gelu_erf_form_matches_torch(oracle):
    x = np.linspace(-8, 8, 1001).astype(np.float32)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    yt = torch.nn.functional.gelu(xt, approximate="none")
    assert np.abs(oracle.gelu_fwd(x, approximate=False) - yt.detach().numpy()).max() < 1e-6
    dy = np.sin(x).astype(np.float32)
    (yt * torch.tensor(dy, dtype=torch.float64)).sum().backward()
    assert np.abs(oracle.gelu_bwd(dy, x, approximate=False) - xt.grad.numpy()).max() < 1e-6
    # Phi(0) = 1/2: gelu(0) = 0 with slope 1/2; the two forms agree to ~1e-3
    assert oracle.gelu_bwd(np.ones(1, np.float32), np.zeros(1, np.float32), False)[0] == 0.5
    assert np.abs(oracle.gelu_fwd(x, False) - oracle.gelu_fwd(x, True)).max() < 2e-3


def test_adamw_bf16_state_is_the_fp32_step_rounded(oracle):
    rng = np.random.default_rng(4)
    n = 257
    f = [rng.standard_normal(n).astype(np.float32) for _ in range(2)]
    m = (0.01 * rng.standard_normal(n)).astype(np.float32)
    v = (1e-4 * np.abs(rng.standard_normal(n))).astype(np.float32)
    bits = [oracle.f32_to_bf16(a) for a in (f[0], f[1], m, v)]
    p2, m2, v2 = oracle.adamw_step_bf16(*bits, 1e-3, 0.9, 0.999, 1e-8, 0.1, 5)
    # independent: fp64 closed form on the bf16 values, then bf16 rounding
    pf, gf, mf, vf = (oracle.bf16_to_f32(b).astype(np.float64) for b in bits)
    mn = 0.9 * mf + 0.1 * gf
    vn = 0.999 * vf + 0.001 * gf * gf
    pn = pf * (1 - 1e-4) - 1e-3 * (mn / (1 - 0.9 ** 5)) / (np.sqrt(vn / (1 - 0.999 ** 5)) + 1e-8)
    for got, ref in ((p2, pn), (m2, mn), (v2, vn)):
        g = oracle.bf16_to_f32(got).astype(np.float64)
        # one bf16 step at most (the fp32 step can sit on the other side of a boundary)
        assert np.all(np.abs(g - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-30)


def test_cross_entropy_matches_torch(oracle):
    rng = np.random.default_rng(5)
    B, V = 7, 33
    z = rng.standard_normal((B, V)) * 3
    t = rng.integers(0, V, B)
    zt = torch.tensor(z, requires_grad=True)
    ref = torch.nn.functional.cross_entropy(zt, torch.tensor(t), reduction="mean")
    loss = oracle.cross_entropy_fwd(z, t)
    assert abs(loss.sum() - ref.item()) < 1e-12
    ref.backward()
    assert np.abs(oracle.cross_entropy_bwd(np.ones(B), z, t) - zt.grad.numpy()).max() < 1e-12
    # label smoothing as the CPU reference: (1 - eps) loss_0 + eps log V, per row / B
    l2 = oracle.cross_entropy_fwd(z, t, 0.1)
    assert np.allclose(l2, 0.9 * loss + 0.1 * np.log(V) / B)
    # uniform logits: log V for any eps; gradient rows sum to zero
    assert np.allclose(oracle.cross_entropy_fwd(np.zeros((B, V)), t, 0.3).sum(), np.log(V))
    g = oracle.cross_entropy_bwd(rng.standard_normal(B), z, t, 0.2)
    assert np.abs(g.sum(axis=1)).max() < 1e-12
    # invalid target: NaN loss, zero gradient row
    t2 = t.copy()
    t2[2] = V
    assert np.isnan(oracle.cross_entropy_fwd(z, t2)[2])
    assert not oracle.cross_entropy_bwd(np.ones(B), z, t2)[2].any()


def test_embedding_is_a_one_hot_product(oracle):
    rng = np.random.default_rng(6)
    V, D, N = 11, 5, 40
    w = rng.standard_normal((V, D))
    idx = rng.integers(0, V, N)
    onehot = np.eye(V)[idx]
    assert np.array_equal(oracle.embedding_fwd(idx, w), onehot @ w)
    dy = rng.standard_normal((N, D))
    assert np.allclose(oracle.embedding_bwd(dy, idx, V), onehot.T @ dy)
    bad = idx.copy()
    bad[3] = V
    assert not oracle.embedding_fwd(bad, w)[3].any()


def test_rmsnorm_forward_invariant_and_torch(oracle):
    """RMSNorm (layernorm.cu:15-48): rows of x rs have mean square 1 when
    eps = 0, and the fp64 form equals torch's rms_norm."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((6, 80)) * 2 + 0.5).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(80)).astype(np.float32)
    y1, rs = oracle.rmsnorm_fwd(x, np.ones(80), eps=0.0)
    assert np.abs((y1 ** 2).mean(1) - 1).max() < 1e-12
    assert np.allclose(rs, 1 / np.sqrt((x.astype(np.float64) ** 2).mean(1)), rtol=1e-14)
    y, _ = oracle.rmsnorm_fwd(x, w, eps=1e-5)
    ref = torch.nn.functional.rms_norm(torch.tensor(x, dtype=torch.float64), (80,),
                                       torch.tensor(w, dtype=torch.float64), 1e-5)
    assert np.abs(y - ref.numpy()).max() < 1e-12


def test_rmsnorm_backward_autograd_and_reference_form(oracle):
    """The exact gradient matches torch fp64 autograd and central differences;
    the reference's dx (rs in place of rs^3 in the second term) fails them."""
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((4, 32)) * 1.7).astype(np.float64)
    w = 1 + 0.2 * rng.standard_normal(32)
    dy = rng.standard_normal((4, 32))
    eps = 1e-5
    dx, dw = oracle.rmsnorm_bwd(dy, x, w, eps)
    xt = torch.tensor(x, requires_grad=True)
    wt = torch.tensor(w, requires_grad=True)
    yt = torch.nn.functional.rms_norm(xt, (32,), wt, eps)
    (yt * torch.tensor(dy)).sum().backward()
    assert np.abs(dx - xt.grad.numpy()).max() < 1e-10
    assert np.abs(dw - wt.grad.numpy()).max() < 1e-10
    # central differences of <dy, y(x)> at a few coordinates
    f = lambda xx: float((dy * oracle.rmsnorm_fwd(xx, w, eps)[0]).sum())
    h = 1e-6
    for r, c in ((0, 0), (1, 7), (3, 31)):
        e = np.zeros_like(x)
        e[r, c] = h
        fd = (f(x + e) - f(x - e)) / (2 * h)
        assert abs(dx[r, c] - fd) < 1e-6
    dx_ref_form, _ = oracle.rmsnorm_bwd(dy, x, w, eps, reference_form=True)
    assert np.abs(dx_ref_form - xt.grad.numpy()).max() > 1e-2


def test_rmsnorm_reference_known_answer(oracle):
    """nn_kernels.zig:250-264: rows [1, 2, 3, 4], w = 1, eps = 1e-6 give a
    mean square of 1 within 1%; the closed form is x / sqrt(7.5 + eps)."""
    x = np.array([[1.0, 2.0, 3.0, 4.0], [1.0, 2.0, 3.0, 4.0]])
    y, rs = oracle.rmsnorm_fwd(x, np.ones(4), eps=1e-6)
    assert abs((y[0] ** 2).mean() - 1.0) < 0.01
    assert np.allclose(y, x / np.sqrt(7.5 + 1e-6), rtol=1e-15)
