"""Embedding and cross-entropy kernels on the GPU against the oracle."""
import numpy as np
import pytest
import torch

from helpers import announce, rel_l2

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,V,D", [(1000, 300, 1024), (77, 50, 100), (5, 7, 8)])
def test_embedding(oracle, N, V, D):
    from ceo_amd.nn import embedding_backward, embedding_forward

    announce(f"embedding N={N} V={V} D={D}")
    rng = np.random.default_rng(N + V)
    w = torch.randn(V, D, generator=torch.Generator().manual_seed(N)).to(torch.bfloat16)
    idx = rng.integers(0, V, N).astype(np.int32)
    idx[1] = V + 3  # out of range: zero row (checked entry), skipped in the backward
    idx[2] = -1
    idd = torch.from_numpy(idx).cuda()
    out = embedding_forward(idd, w.cuda())
    torch.cuda.synchronize()
    ref = oracle.embedding_fwd(idx, w.float().numpy())
    assert np.array_equal(out.float().cpu().numpy(), ref)
    # the unchecked reference entry on valid indices only
    good = torch.from_numpy(np.clip(idx, 0, V - 1)).cuda()
    out2 = embedding_forward(good, w.cuda(), checked=False)
    assert torch.equal(out2.cpu(), w[np.clip(idx, 0, V - 1)])
    dy = torch.randn(N, D, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16)
    dw = torch.full((V, D), 0.5, device="cuda")  # accumulated into
    embedding_backward(dy.cuda(), idd, dw)
    torch.cuda.synchronize()
    rdw = oracle.embedding_bwd(dy.float().numpy(), idx, V) + 0.5
    e = rel_l2(dw, rdw)
    print(f"  dW rel-L2={e:.2e}", flush=True)
    assert e <= 1e-6


@pytest.mark.parametrize("B,V,eps", [(64, 32000, 0.0), (37, 32000, 0.1), (16, 50257, 0.0),
                                     (9, 1000, 0.0), (5, 77, 0.2), (3, 70000, 0.0)])
def test_cross_entropy(oracle, B, V, eps):
    from ceo_amd.nn import cross_entropy_backward, cross_entropy_forward

    announce(f"cross_entropy B={B} V={V} eps={eps}")
    g = torch.Generator().manual_seed(B * V)
    z = (torch.randn(B, V, generator=g) * 4).to(torch.bfloat16)
    t = torch.randint(0, V, (B,), generator=g, dtype=torch.int32)
    t[0] = V  # invalid target -> NaN loss, zero gradient row
    gl = torch.rand(B, generator=g) + 0.5
    zd, td = z.cuda(), t.cuda()
    loss = cross_entropy_forward(zd, td, eps)
    grad = cross_entropy_backward(gl.cuda(), zd, td, eps)
    torch.cuda.synchronize()
    rl = oracle.cross_entropy_fwd(z.float().numpy(), t.numpy(), eps)
    rg = oracle.cross_entropy_bwd(gl.numpy(), z.float().numpy(), t.numpy(), eps)
    ln = loss.cpu().numpy()
    assert np.isnan(ln[0]) and not grad[0].any()
    err = np.abs(ln[1:] - rl[1:]).max() / np.abs(rl[1:]).max()
    eg = rel_l2(grad[1:], rg[1:])
    print(f"  loss max rel {err:.2e}, grad rel-L2 {eg:.2e}", flush=True)
    assert err <= 1e-5 and eg <= 1e-2


@pytest.mark.parametrize("B,V,eps", [(37, 32000, 0.1), (9, 1000, 0.0), (3, 70000, 0.0)])
def test_cross_entropy_forward_backward_fused(B, V, eps):
    """The one-pass entry gives the two entries' results bit for bit: with a
    per-row grad_loss, with grad_loss NULL (= ones) and in place over the
    logits (the row-in-registers path and the looped path for V = 70000)."""
    from ceo_amd.nn import (cross_entropy_backward, cross_entropy_forward,
                            cross_entropy_forward_backward)

    announce(f"cross_entropy fused fwd+bwd B={B} V={V} eps={eps}")
    g = torch.Generator().manual_seed(B + V)
    z = (torch.randn(B, V, generator=g) * 4).to(torch.bfloat16).cuda()
    t = torch.randint(0, V, (B,), generator=g, dtype=torch.int32)
    t[1] = -1  # invalid target: NaN loss, zero gradient row
    t = t.cuda()
    gl = (torch.rand(B, generator=g) + 0.5).cuda()
    loss_ref = cross_entropy_forward(z, t, eps)
    grad_ref = cross_entropy_backward(gl, z, t, eps)
    ones_ref = cross_entropy_backward(torch.ones(B, device="cuda"), z, t, eps)
    loss, grad = cross_entropy_forward_backward(z, t, eps, grad_loss=gl)
    assert torch.equal(loss.nan_to_num(), loss_ref.nan_to_num()) and torch.isnan(loss[1])
    assert torch.equal(grad, grad_ref)
    zc = z.clone()
    loss2, grad2 = cross_entropy_forward_backward(zc, t, eps, in_place=True)
    assert grad2.data_ptr() == zc.data_ptr()
    assert torch.equal(loss2.nan_to_num(), loss_ref.nan_to_num())
    assert torch.equal(grad2, ones_ref)


def test_cross_entropy_uniform_logits():
    from ceo_amd.nn import cross_entropy_forward

    announce("cross_entropy uniform logits")
    B, V = 8, 32000
    loss = cross_entropy_forward(torch.zeros(B, V, dtype=torch.bfloat16, device="cuda"),
                                 torch.arange(B, dtype=torch.int32, device="cuda"), 0.3)
    assert abs(loss.sum().item() - np.log(V)) < 1e-5
