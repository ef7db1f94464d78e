"""Pins for the oracle's ShortConv and PRISM refinement (CPU only).

ShortConv follows ShortConv.forwardCpu (src/model/prism.zig:448-473): a causal
depthwise convolution whose fp32 terms are added in increasing lag.  PRISM
follows PrismLayer.prismForwardCpu (prism.zig:251-323).  Each is checked
against an independent statement: torch's grouped conv1d and autograd, an
impulse response, a summation-order known answer, closed forms and central
differences.
"""
import numpy as np
import torch


def _conv_torch(x, w):
    """Causal depthwise conv as torch computes it: left-pad W-1, flip the taps."""
    B, T, C = x.shape
    W = w.shape[1]
    xt = torch.nn.functional.pad(x.permute(0, 2, 1), (W - 1, 0))
    y = torch.nn.functional.conv1d(xt, w.flip(-1).unsqueeze(1), groups=C)
    return y.permute(0, 2, 1)


def test_shortconv_matches_grouped_conv1d(oracle):
    rng = np.random.default_rng(1)
    for B, T, C, W in ((2, 37, 24, 5), (1, 9, 8, 16), (3, 64, 16, 64)):
        x = oracle.round_bf16(rng.standard_normal((B, T, C)))
        w = oracle.round_bf16(rng.standard_normal((C, W)) / np.sqrt(W))
        y = oracle.shortconv_fwd(x, w)
        ref = _conv_torch(torch.tensor(x, dtype=torch.float64), torch.tensor(w, dtype=torch.float64))
        assert np.abs(y - ref.numpy()).max() < 1e-5 * max(1.0, np.abs(ref.numpy()).max())


def test_shortconv_impulse_and_window_one(oracle):
    """A unit input at t = 0 reads the taps out in order; W = 1 is x * w."""
    C, W, T = 4, 6, 10
    w = oracle.round_bf16(np.arange(1, C * W + 1, dtype=np.float64).reshape(C, W) / 7)
    x = np.zeros((1, T, C), dtype=np.float32)
    x[0, 0, :] = 1
    y = oracle.shortconv_fwd(x, w)
    assert np.array_equal(y[0, :W, :], w.T)
    assert not y[0, W:, :].any()
    rng = np.random.default_rng(2)
    x = oracle.round_bf16(rng.standard_normal((2, 5, 3)))
    w1 = oracle.round_bf16(rng.standard_normal((3, 1)))
    assert np.array_equal(oracle.shortconv_fwd(x, w1), x * w1[:, 0])


def test_shortconv_summation_order_known_answer(oracle):
    """Terms added in increasing lag (the reference loop's order) round
    1.15625 + 2^-8 + 2^-24 + 2^-24 to 1.15625 + 2^-8 in fp32 (two ties to
    even), which bf16 rounds down to 1.15625; the opposite order reaches
    1.15625 + 2^-8 + 2^-23, which rounds up to 1.1640625."""
    x = np.array([[[1.0], [1.0], [1.0 + 2.0 ** -5]]], dtype=np.float32)
    w = np.array([[1.125, 2.0 ** -24, 2.0 ** -24]], dtype=np.float32)
    y = oracle.shortconv_fwd(x, w)
    assert y[0, 2, 0] == np.float32(1.15625 + 2.0 ** -8)
    assert oracle.round_bf16(y)[0, 2, 0] == np.float32(1.15625)
    rev = np.float32(2.0 ** -24) + np.float32(2.0 ** -24) + np.float32(1.15625 + 2.0 ** -8)
    assert oracle.round_bf16(np.array([rev]))[0] == np.float32(1.1640625)
    assert oracle.round_bf16(y)[0, 0, 0] == np.float32(1.125)
    assert oracle.round_bf16(y)[0, 1, 0] == np.float32(1.125)


def test_shortconv_backward_matches_autograd(oracle):
    rng = np.random.default_rng(3)
    B, T, C, W = 2, 21, 6, 4
    x = rng.standard_normal((B, T, C))
    w = rng.standard_normal((C, W))
    dy = rng.standard_normal((B, T, C))
    dx, dw = oracle.shortconv_bwd(dy, x, w)
    xt = torch.tensor(x, requires_grad=True)
    wt = torch.tensor(w, requires_grad=True)
    (_conv_torch(xt, wt) * torch.tensor(dy)).sum().backward()
    assert np.abs(dx - xt.grad.numpy()).max() < 1e-12
    assert np.abs(dw - wt.grad.numpy()).max() < 1e-12


def _gelu(x):
    """torch's tanh GELU in fp64 (the textbook 0.5 x (1 + tanh u))."""
    return torch.nn.functional.gelu(torch.tensor(x, dtype=torch.float64),
                                    approximate="tanh").numpy()


def test_prism_forward_closed_forms(oracle):
    rng = np.random.default_rng(4)
    B, T, C, HD = 2, 3, 10, 6
    u = oracle.round_bf16(rng.standard_normal((B, T, C)))
    v = oracle.round_bf16(rng.standard_normal((B, T, C)))
    w_p = [oracle.round_bf16(rng.standard_normal((C, HD))) for _ in range(2)]
    # one iteration: o = bf16(0.5 GELU(p (v - u))); channels >= head_dim are 0
    o1 = oracle.prism_fwd(u, v, w_p[:1], HD)
    p0 = w_p[0].reshape(-1)[:HD].astype(np.float64)
    r = (v - u)[..., :HD].astype(np.float64)
    ref1 = oracle.round_bf16((0.5 * _gelu(p0 * r)).astype(np.float32))
    assert np.abs(o1[..., :HD] - ref1).max() <= 2.0 ** -8 * np.abs(ref1).max()
    assert (o1[..., :HD] == ref1).mean() > 0.95
    assert not o1[..., HD:].any()
    # two iterations unrolled by hand, without the rounding
    p1 = w_p[1].reshape(-1)[:HD].astype(np.float64)
    d0 = _gelu(p0 * r)
    d1 = _gelu(p1 * (r - d0))
    o2 = oracle.prism_fwd(u, v, w_p, HD, round_output=False)
    assert np.abs(o2[..., :HD] - (0.5 * d0 + 0.5 * d1)).max() < 1e-6
    # no iterations: all zero
    assert not oracle.prism_fwd(u, v, [], HD).any()


def test_prism_backward_autograd_and_differences(oracle):
    rng = np.random.default_rng(5)
    B, T, C, HD, L = 2, 4, 7, 5, 3
    u = rng.standard_normal((B, T, C))
    v = rng.standard_normal((B, T, C))
    w_p = [rng.standard_normal((C, HD)) for _ in range(L)]
    g = rng.standard_normal((B, T, C))
    gu, gv, dps = oracle.prism_bwd(g, u, v, w_p, HD)
    # torch fp64 autograd of the same refinement
    ut = torch.tensor(u, requires_grad=True)
    vt = torch.tensor(v, requires_grad=True)
    pts = [torch.tensor(w.reshape(-1)[:HD].copy(), requires_grad=True) for w in w_p]
    r = vt[..., :HD] - ut[..., :HD]
    o = torch.zeros_like(r)
    for p in pts:
        d = torch.nn.functional.gelu(p * r, approximate="tanh")
        o = o + 0.5 * d
        r = r - d
    (o * torch.tensor(g[..., :HD])).sum().backward()
    assert np.abs(gu - ut.grad.numpy()).max() < 1e-12
    assert np.abs(gv - vt.grad.numpy()).max() < 1e-12
    for l in range(L):
        assert np.abs(dps[l] - pts[l].grad.numpy()).max() < 1e-12
    # central differences of <g, o(v)> on the oracle forward itself
    f = lambda vv: float((g * oracle.prism_fwd(u, vv, w_p, HD, round_output=False)).sum())
    h = 1e-3
    for idx in ((0, 0, 0), (1, 3, 4), (0, 2, 6)):
        e = np.zeros_like(v)
        e[idx] = h
        fd = (f(v + e) - f(v - e)) / (2 * h)
        assert abs(gv[idx] - fd) < 2e-3 * max(1.0, abs(fd))


def test_gelu_form_without_cancellation(oracle):
    """The oracle's x / (1 + e^(-2u)) equals torch's 0.5 x (1 + tanh u) where
    the latter does not cancel, equals the cancellation-free rewrite
    1 + tanh u = 2 e^(2u) / (1 + e^(2u)) in the far negative tail, and its
    derivative matches central differences."""
    x = np.linspace(-3, 6, 301)
    assert np.allclose(oracle._gelu_tanh64(x), _gelu(x), rtol=1e-13, atol=1e-300)
    # far tail: 1 + tanh u = 2 e^(2u) / (1 + e^(2u)) exactly, no cancellation
    xt = np.array([-8.0, -10.0, -12.0])
    u = np.sqrt(2 / np.pi) * (xt + 0.044715 * xt ** 3)
    exact = 0.5 * xt * (2 * np.exp(2 * u) / (1 + np.exp(2 * u)))
    assert np.allclose(oracle._gelu_tanh64(xt), exact, rtol=1e-13)
    # derivative by central differences
    xs = np.array([-4.0, -1.3, 0.0, 0.7, 2.5])
    h = 1e-6
    fd = (oracle._gelu_tanh64(xs + h) - oracle._gelu_tanh64(xs - h)) / (2 * h)
    assert np.allclose(oracle._gelu_tanh64_grad(xs), fd, rtol=1e-7, atol=1e-9)
