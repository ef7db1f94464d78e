"""ShortConv and the PRISM refinement on the GPU against the oracle.

ShortConv's forward is bit-exact with the reference loop's arithmetic
(prism.zig:448-473: fp32 terms added in increasing lag, then bf16); its
backward and the PRISM kernels are checked to bf16 output rounding.
"""
import numpy as np
import pytest
import torch

from helpers import announce, rel_l2

pytestmark = pytest.mark.gpu


def _bf(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)


def _bits(t):
    return (t.view(torch.int16).cpu().numpy().astype(np.int32) & 0xFFFF).astype(np.uint16)


# (4, 650, 1024, 64) and (4, 1300, 1024, 37) are large enough in channel tiles x
# batch rows for the token-walking kernel (two and three tiles per workgroup)
@pytest.mark.parametrize("B,T,C,W", [(2, 100, 96, 16), (1, 300, 1024, 64), (2, 65, 70, 3),
                                     (1, 50, 64, 80), (1, 40, 32, 100), (1, 8, 16, 1),
                                     (1, 10, 64, 64), (3, 129, 130, 17), (4, 650, 1024, 64),
                                     (4, 1300, 1024, 37)])
def test_shortconv_forward_bit_exact(oracle, B, T, C, W):
    from ceo_amd.prism import shortconv_forward

    announce(f"shortconv_forward B={B} T={T} C={C} W={W}")
    rng = np.random.default_rng(B * 1000 + T + C + W)
    x = _bf(rng.standard_normal((B, T, C)))
    w = _bf(rng.standard_normal((C, W)) / np.sqrt(W))
    y = shortconv_forward(x.cuda(), w.cuda())
    torch.cuda.synchronize()
    ref = oracle.f32_to_bf16(oracle.shortconv_fwd(x.float().numpy(), w.float().numpy()))
    got = _bits(y)
    mism = int((got != ref).sum())
    print(f"  mismatching bf16 values: {mism} of {got.size}", flush=True)
    assert mism == 0


@pytest.mark.parametrize("W", [3, 100])
def test_shortconv_summation_order_known_answer(W):
    """Increasing-lag fp32 order: 1.15625 + 2^-8 + 2^-24 + 2^-24 stays a bf16
    tie and rounds to 1.15625 (the reverse order would give 1.1640625); the
    taps beyond the third are zero, so the tiled (W = 3) and direct (W = 100)
    kernels must agree."""
    from ceo_amd.prism import shortconv_forward

    announce(f"shortconv order known answer W={W}")
    x = torch.tensor([[[1.0], [1.0], [1.0 + 2.0 ** -5]]], dtype=torch.bfloat16).cuda()
    w = torch.zeros(1, W, dtype=torch.bfloat16)
    w[0, :3] = torch.tensor([1.125, 2.0 ** -24, 2.0 ** -24])
    y = shortconv_forward(x, w.cuda()).float().cpu().numpy()
    assert y[0, 2, 0] == 1.15625 and y[0, 1, 0] == 1.125 and y[0, 0, 0] == 1.125


@pytest.mark.parametrize("B,T,C,W", [(2, 100, 96, 16), (1, 256, 1024, 64), (2, 65, 70, 3),
                                     (1, 40, 32, 100), (1, 10, 64, 64), (4, 650, 1024, 64)])
def test_shortconv_backward(oracle, B, T, C, W):
    from ceo_amd.prism import shortconv_backward

    announce(f"shortconv_backward B={B} T={T} C={C} W={W}")
    rng = np.random.default_rng(7 + W)
    x = _bf(rng.standard_normal((B, T, C)))
    w = _bf(rng.standard_normal((C, W)) / np.sqrt(W))
    dy = _bf(rng.standard_normal((B, T, C)))
    acc = torch.zeros(C, W, dtype=torch.float32, device="cuda")
    dx, _ = shortconv_backward(dy.cuda(), x.cuda(), w.cuda(), grad_weight=acc)
    dx2, _ = shortconv_backward(dy.cuda(), x.cuda(), w.cuda(), grad_weight=acc)
    torch.cuda.synchronize()
    rdx, rdw = oracle.shortconv_bwd(dy.double().numpy(), x.double().numpy(), w.double().numpy())
    e_dx, e_dw = rel_l2(dx, rdx), rel_l2(acc, 2 * rdw)
    print(f"  rel-L2 dx={e_dx:.2e} dw(2 calls)={e_dw:.2e}", flush=True)
    assert e_dx <= 1e-2 and e_dw <= 1e-5
    assert torch.equal(dx, dx2)


@pytest.mark.parametrize("B,T,C,W", [(4, 650, 1024, 64), (4, 1300, 1024, 37),
                                     (8, 333, 1024, 16)])
def test_shortconv_walk_matches_tiles(B, T, C, W):
    """The token-walking kernel (rows handed from one tile to the next) and the
    one-tile kernels (taken for rows that are not 16-byte aligned) give
    bit-identical outputs and input gradients."""
    from ceo_amd.prism import shortconv_backward, shortconv_forward

    announce(f"shortconv walk vs tiles B={B} T={T} C={C} W={W}")
    g = torch.Generator().manual_seed(B + T + W)
    x = torch.randn(B, T, C, generator=g).to(torch.bfloat16).cuda()
    dy = torch.randn(B, T, C, generator=g).to(torch.bfloat16).cuda()
    w = (torch.randn(C, W, generator=g) / W ** 0.5).to(torch.bfloat16).cuda()
    y_w = shortconv_forward(x, w)
    y_t = shortconv_forward(_misaligned(x), w)
    dx_w, _ = shortconv_backward(dy, x, w)
    dx_t, _ = shortconv_backward(_misaligned(dy), x, w)
    torch.cuda.synchronize()
    assert (_bits(y_w) == _bits(y_t)).all()
    assert (_bits(dx_w) == _bits(dx_t)).all()


# (2, 64, 256, 64, 3), (1, 1000, 512, 128, 4), (3, 77, 96, 32, 2) and
# (1, 50, 16, 8, 1) take the 16-row block kernels (16-byte rows, head_dim / 8
# dividing 256, L <= 4; 1000 rows leave a partial last block); the others the
# lane-per-channel kernels.
@pytest.mark.parametrize("B,T,C,HD,L", [(2, 64, 256, 64, 3), (1, 33, 100, 37, 1),
                                        (2, 16, 64, 64, 16), (1, 8, 300, 128, 0),
                                        (1, 1000, 512, 128, 4), (3, 77, 96, 32, 2),
                                        (1, 50, 16, 8, 1)])
def test_prism_forward(oracle, B, T, C, HD, L):
    from ceo_amd.prism import prism_forward

    announce(f"prism_forward B={B} T={T} C={C} head_dim={HD} L={L}")
    rng = np.random.default_rng(11 + C + L)
    u = _bf(rng.standard_normal((B, T, C)))
    v = _bf(rng.standard_normal((B, T, C)) * 1.5)
    w_p = [_bf(rng.standard_normal((C, HD)) * np.sqrt(2.0 / C) * 8) for _ in range(L)]
    out, state = prism_forward(u.cuda(), v.cuda(), [w.cuda() for w in w_p], HD)
    torch.cuda.synchronize()
    ref = oracle.prism_fwd(u.float().numpy(), v.float().numpy(), [w.float().numpy() for w in w_p],
                           HD)
    got = out.float().cpu().numpy()
    diff = np.abs(got - ref)
    exact = float((diff == 0).mean())
    print(f"  exact {exact:.4f}, max diff {diff.max():.2e}", flush=True)
    # fp32 vs fp64 GELU can move a value across a bf16 rounding boundary: one ulp
    assert (diff <= 2.0 ** -7 * np.abs(ref) + 1e-30).all()
    assert exact >= 0.99
    assert not got[..., HD:].any()
    assert not state.float().abs().sum().item()


@pytest.mark.parametrize("B,T,C,HD,L", [(2, 64, 256, 64, 3), (1, 33, 100, 37, 2),
                                        (1, 1000, 512, 128, 4), (3, 77, 96, 32, 3),
                                        (1, 50, 16, 8, 1)])
def test_prism_backward(oracle, B, T, C, HD, L):
    from ceo_amd.prism import prism_backward

    announce(f"prism_backward B={B} T={T} C={C} head_dim={HD} L={L}")
    rng = np.random.default_rng(21 + C)
    u = _bf(rng.standard_normal((B, T, C)))
    v = _bf(rng.standard_normal((B, T, C)) * 1.5)
    g = _bf(rng.standard_normal((B, T, C)))
    w_p = [_bf(rng.standard_normal((C, HD)) * 0.7) for _ in range(L)]
    gw = [torch.zeros(C * HD, dtype=torch.float32, device="cuda") for _ in range(L)]
    gu, gv = prism_backward(g.cuda(), u.cuda(), v.cuda(), [w.cuda() for w in w_p], HD, gw)
    torch.cuda.synchronize()
    rgu, rgv, rdp = oracle.prism_bwd(g.double().numpy(), u.double().numpy(), v.double().numpy(),
                                     [w.double().numpy() for w in w_p], HD)
    errs = [rel_l2(gu, rgu), rel_l2(gv, rgv)]
    errs += [rel_l2(gw[l][:HD], rdp[l]) for l in range(L)]
    print("  rel-L2 gu, gv, dp_l:", [f"{e:.2e}" for e in errs], flush=True)
    assert errs[0] <= 1e-2 and errs[1] <= 1e-2
    assert max(errs[2:]) <= 1e-4
    assert not gw[0][HD:].any()
    assert not gu.float()[..., HD:].any() and not gv.float()[..., HD:].any()


def _misaligned(t):
    """A contiguous copy of t whose data starts 2 bytes past a 16-byte
    boundary (the PRISM entries then take the lane-per-channel kernels)."""
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    m = buf[1:].view(t.shape)
    m.copy_(t)
    assert m.data_ptr() % 16 == 2
    return m


def test_prism_row_blocks_match_lane_kernels():
    """The 16-row block kernels and the lane-per-channel kernels compute the
    same per-channel arithmetic: outputs and input gradients bit-identical,
    the w_p gradients equal up to summation order; the block kernels' w_p
    gradient (per-block partials added in block order) is the same on every
    run."""
    from ceo_amd.prism import prism_backward, prism_forward

    B, T, C, HD, L = 2, 500, 256, 64, 3
    announce(f"prism row-block vs lane kernels B={B} T={T} C={C} head_dim={HD} L={L}")
    rng = np.random.default_rng(5)
    u = _bf(rng.standard_normal((B, T, C))).cuda()
    v = _bf(rng.standard_normal((B, T, C)) * 1.5).cuda()
    g = _bf(rng.standard_normal((B, T, C))).cuda()
    w_p = [_bf(rng.standard_normal((C, HD)) * 0.7).cuda() for _ in range(L)]
    um, vm, gm = _misaligned(u), _misaligned(v), _misaligned(g)
    out_f, _ = prism_forward(u, v, w_p, HD)
    out_l, _ = prism_forward(um, vm, w_p, HD)
    gws = [[torch.zeros(C * HD, dtype=torch.float32, device="cuda") for _ in range(L)]
           for _ in range(3)]
    gu_f, gv_f = prism_backward(g, u, v, w_p, HD, gws[0])
    gu_f2, gv_f2 = prism_backward(g, u, v, w_p, HD, gws[1])
    gu_l, gv_l = prism_backward(gm, um, vm, w_p, HD, gws[2])
    torch.cuda.synchronize()
    assert (_bits(out_f) == _bits(out_l)).all()
    assert (_bits(gu_f) == _bits(gu_l)).all() and (_bits(gv_f) == _bits(gv_l)).all()
    assert torch.equal(gu_f, gu_f2) and torch.equal(gv_f, gv_f2)
    for l in range(L):
        assert torch.equal(gws[0][l], gws[1][l])
        assert rel_l2(gws[0][l], gws[2][l].cpu().numpy()) <= 1e-5


def test_prism_layer_against_torch_autograd():
    """PrismLayer (ShortConv then refinement) forward and backward against a
    torch fp32 autograd restatement on the same bf16 weights."""
    from ceo_amd.prism import PrismLayer

    announce("PrismLayer vs torch autograd (B=2, T=96, C=128, head_dim=64, L=3, W=16)")
    B, T, C, HD = 2, 96, 128, 64
    layer = PrismLayer(C, HD, num_iterations=3, window_size=16, seed=3)
    for w in layer.w_p:
        w.mul_(4)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(B, T, C, generator=g).to(torch.bfloat16).cuda()
    v = (torch.randn(B, T, C, generator=g) * 1.5).to(torch.bfloat16).cuda()
    dy = torch.randn(B, T, C, generator=g).to(torch.bfloat16).cuda()
    out, _ = layer.forward(x, v)
    gx, gv = layer.backward(dy)
    torch.cuda.synchronize()

    xt = x.float().requires_grad_(True)
    vt = v.float().requires_grad_(True)
    wc = layer.shortconv.weight.float().requires_grad_(True)
    pts = [w.float().reshape(-1)[:HD].clone().requires_grad_(True) for w in layer.w_p]
    xp = torch.nn.functional.pad(xt.permute(0, 2, 1), (wc.shape[1] - 1, 0))
    u = torch.nn.functional.conv1d(xp, wc.flip(-1).unsqueeze(1), groups=C).permute(0, 2, 1)
    r = vt[..., :HD] - u[..., :HD]
    o = torch.zeros_like(r)
    for p in pts:
        d = torch.nn.functional.gelu(p * r, approximate="tanh")
        o = o + 0.5 * d
        r = r - d
    (o * dy.float()[..., :HD]).sum().backward()
    e_o = rel_l2(out[..., :HD], o.detach().cpu().numpy())
    e_gx, e_gv = rel_l2(gx, xt.grad.cpu().numpy()), rel_l2(gv, vt.grad.cpu().numpy())
    e_wc = rel_l2(layer.shortconv.grad_weight, wc.grad.cpu().numpy())
    e_wp = max(rel_l2(layer.grad_w_p[l].reshape(-1)[:HD], pts[l].grad.cpu().numpy())
               for l in range(3))
    print(f"  rel-L2 out={e_o:.2e} gx={e_gx:.2e} gv={e_gv:.2e} dWconv={e_wc:.2e} dWp={e_wp:.2e}",
          flush=True)
    assert e_o <= 2e-2 and e_gx <= 2e-2 and e_gv <= 2e-2 and e_wc <= 2e-2 and e_wp <= 2e-2
