"""Affine combine of segment states and the sequence-sharded forward built on it."""
import numpy as np
import pytest
import torch

from helpers import announce, rel_l2, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,NH,K,V", [(5, 6, 128, 96), (3, 4, 64, 256), (1, 2, 64, 64),
                                      (4, 3, 256, 70)])
def test_affine_state_scan_matches_sequential_products(n, NH, K, V):
    from ceo_amd.state import affine_state_scan

    announce(f"affine state scan n={n} NH={NH} K={K} V={V}")
    g = torch.Generator().manual_seed(n * K + V)
    A = [torch.randn(1, NH, K, K, generator=g) / K ** 0.5 for _ in range(n)]
    Bs = [torch.randn(1, NH, K, V, generator=g) for _ in range(n)]
    dev = [b.cuda() for b in Bs]
    affine_state_scan([a.cuda() for a in A], dev)
    torch.cuda.synchronize()
    ref = Bs[0].double()
    for i in range(1, n):
        ref = A[i].double() @ ref + Bs[i].double()
        e = rel_l2(dev[i], ref.numpy())
        assert e <= 1e-6, (i, e)
    assert torch.equal(dev[0].cpu(), Bs[0])


@pytest.mark.parametrize("dtype,K,V,segments,tol", [(torch.float32, 64, 64, 4, 1e-5),
                                                    (torch.bfloat16, 128, 128, 4, 2e-2),
                                                    (torch.bfloat16, 64, 256, 2, 2e-2)])
def test_sharded_forward_matches_one_pass(oracle, dtype, K, V, segments, tol):
    from ceo_amd.efla import chunk_efla_fwd
    from ceo_amd.state import sharded_forward

    announce(f"sharded forward {dtype} K={K} V={V} segments={segments}")
    B, T, H = 2, 512, 2
    x = oracle.make_efla_inputs(17, B * T, H, K, V, bf16=dtype == torch.bfloat16)
    g = {n: to_dev(a, dtype, (B, T, H, K) if n in "qk" else
                   (B, T, H) if n == "beta" else (B, T, H, V)) for n, a in x.items()}
    s0 = 0.3 * torch.randn(B, H, K, V, generator=torch.Generator().manual_seed(2)).cuda()
    o, st = sharded_forward(g["q"], g["k"], g["v"], g["beta"], segments, initial_state=s0)
    o1, st1 = chunk_efla_fwd(g["q"], g["k"], g["v"], g["beta"], s0, True)
    ro, rs = oracle.q_forward(x["q"], x["k"], x["v"], x["beta"], T=T,
                              S0=s0.cpu().double().numpy())
    torch.cuda.synchronize()
    eo, es = rel_l2(o, ro.reshape(B, T, H, V)), rel_l2(st, rs)
    e1 = rel_l2(o, o1.float().cpu().numpy())
    print(f"  vs oracle o {eo:.2e} S_T {es:.2e}; vs one pass {e1:.2e}", flush=True)
    assert eo <= tol and es <= tol and e1 <= tol
