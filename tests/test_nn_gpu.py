"""LayerNorm and GEMM kernels on the GPU against the oracle / an fp64 reference."""
import numpy as np
import pytest
import torch

from helpers import announce, rel_l2

pytestmark = pytest.mark.gpu


def _bf(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)


@pytest.mark.parametrize("rows,D,bias", [(64, 1024, True), (37, 512, False), (16, 4096, True),
                                         (9, 1000, True), (5, 96, False)])
def test_layernorm_forward(oracle, rows, D, bias):
    from ceo_amd.nn import layernorm_forward

    announce(f"layernorm_forward rows={rows} D={D} bias={bias}")
    rng = np.random.default_rng(rows + D)
    x = _bf(rng.standard_normal((rows, D)) * 2 + 0.5)
    w = _bf(1 + 0.1 * rng.standard_normal(D))
    b = _bf(0.1 * rng.standard_normal(D)) if bias else None
    y, mean, rstd = layernorm_forward(x.cuda(), w.cuda(), None if b is None else b.cuda(),
                                      1e-5, save_stats=True)
    torch.cuda.synchronize()
    ry, rm, rr = oracle.layernorm_fwd(x.float().numpy(), w.float().numpy(),
                                      None if b is None else b.float().numpy(), 1e-5)
    e = rel_l2(y, ry)
    print(f"  rel-L2 y={e:.2e}", flush=True)
    assert e <= 1e-2
    assert rel_l2(mean, rm) <= 1e-5 and rel_l2(rstd, rr) <= 1e-5
    # invariant: with w = 1, b = 0 each row has mean 0 and variance 1
    y1 = layernorm_forward(x.cuda(), torch.ones(D, dtype=torch.bfloat16, device="cuda"))
    y1 = y1.float().cpu().numpy()
    assert np.abs(y1.mean(1)).max() < 2e-2 and np.abs(y1.var(1) - 1).max() < 3e-2


@pytest.mark.parametrize("rows,D", [(64, 1024), (50, 96), (5000, 1024), (33, 1536), (300, 2048),
                                    (17, 4096)])
def test_layernorm_backward(oracle, rows, D):
    from ceo_amd.nn import layernorm_backward, layernorm_forward

    announce(f"layernorm_backward rows={rows} D={D}")
    rng = np.random.default_rng(7)
    x = _bf(rng.standard_normal((rows, D)))
    w = _bf(1 + 0.1 * rng.standard_normal(D))
    dy = _bf(rng.standard_normal((rows, D)))
    _, mean, rstd = layernorm_forward(x.cuda(), w.cuda(), None, 1e-5, save_stats=True)
    dx, dw, db = layernorm_backward(dy.cuda(), x.cuda(), w.cuda(), mean, rstd)
    torch.cuda.synchronize()
    _, rm, rr = oracle.layernorm_fwd(x.float().numpy(), w.float().numpy(), None, 1e-5)
    rdx, rdw, rdb = oracle.layernorm_bwd(dy.float().numpy(), x.float().numpy(),
                                         w.float().numpy(), rm, rr)
    errs = (rel_l2(dx, rdx), rel_l2(dw, rdw), rel_l2(db, rdb))
    print("  rel-L2 dx,dw,db:", errs, flush=True)
    assert errs[0] <= 1e-2 and errs[1] <= 1e-4 and errs[2] <= 1e-5


@pytest.mark.parametrize("rows,D", [(64, 1024), (37, 96), (16, 4096), (9, 1000), (5, 512),
                                    (3, 8192)])
def test_rmsnorm_forward(oracle, rows, D):
    from ceo_amd.nn import rmsnorm_forward

    announce(f"rmsnorm_forward rows={rows} D={D}")
    rng = np.random.default_rng(rows * 7 + D)
    x = _bf(rng.standard_normal((rows, D)) * 1.5 + 0.3)
    w = _bf(1 + 0.1 * rng.standard_normal(D))
    y = rmsnorm_forward(x.cuda(), w.cuda(), 1e-6)
    torch.cuda.synchronize()
    ry, _ = oracle.rmsnorm_fwd(x.double().numpy(), w.double().numpy(), 1e-6)
    e = rel_l2(y, ry)
    print(f"  rel-L2 y={e:.2e}", flush=True)
    assert e <= 1e-2
    # invariant: with w = 1 every row has mean square 1 (up to bf16 rounding)
    y1 = rmsnorm_forward(x.cuda(), torch.ones(D, dtype=torch.bfloat16, device="cuda"), 0.0)
    ms = (y1.float() ** 2).mean(1).cpu().numpy()
    assert np.abs(ms - 1).max() < 1e-2


@pytest.mark.parametrize("D", [96, 128, 1000, 2048])
def test_norm_backward_weight_grads_repeat_bit_for_bit(D):
    # widths off the register path loop over the row; up to D = 2048 each wave
    # sums its dw (and db) columns in an LDS slice of its own and the slices
    # are added in wave order, so repeated calls give the same bits (LDS
    # atomics across the waves would not).  Enough rows for several per wave.
    from ceo_amd.nn import layernorm_backward, layernorm_forward, rmsnorm_backward

    announce(f"norm backward repeatability D={D}")
    rows = 4099
    rng = np.random.default_rng(5 + D)
    x = _bf(rng.standard_normal((rows, D))).cuda()
    w = _bf(1 + 0.1 * rng.standard_normal(D)).cuda()
    dy = _bf(rng.standard_normal((rows, D))).cuda()
    _, mean, rstd = layernorm_forward(x, w, None, 1e-5, save_stats=True)
    ln = [layernorm_backward(dy, x, w, mean, rstd) for _ in range(4)]
    rms = [rmsnorm_backward(dy, x, w, 1e-6) for _ in range(4)]
    torch.cuda.synchronize()
    for i in range(1, 4):
        for a, b in zip(ln[0], ln[i]):
            assert torch.equal(a, b)
        for a, b in zip(rms[0], rms[i]):
            assert torch.equal(a, b)


@pytest.mark.parametrize("rows,D", [(64, 1024), (50, 96), (5000, 1024), (33, 1536), (300, 2048),
                                    (17, 4096), (6, 16384), (4, 20000)])
def test_rmsnorm_backward(oracle, rows, D):
    from ceo_amd.nn import rmsnorm_backward

    announce(f"rmsnorm_backward rows={rows} D={D}")
    rng = np.random.default_rng(11 + D)
    x = _bf(rng.standard_normal((rows, D)) * 1.3)
    w = _bf(1 + 0.1 * rng.standard_normal(D))
    dy = _bf(rng.standard_normal((rows, D)))
    need_w = D <= 16384
    dx, dw = rmsnorm_backward(dy.cuda(), x.cuda(), w.cuda(), 1e-6, need_weight_grad=need_w)
    torch.cuda.synchronize()
    rdx, rdw = oracle.rmsnorm_bwd(dy.double().numpy(), x.double().numpy(), w.double().numpy(),
                                  1e-6)
    e_dx = rel_l2(dx, rdx)
    e_dw = rel_l2(dw, rdw) if need_w else 0.0
    print(f"  rel-L2 dx={e_dx:.2e} dw={e_dw:.2e}", flush=True)
    assert e_dx <= 1e-2 and e_dw <= 1e-4


def test_rmsnorm_backward_accumulates_and_misaligned(oracle):
    """grad_weight is added into (two calls give twice the sum); inputs that
    are not 16-byte aligned take the looping kernels with the same results."""
    from ceo_amd.nn import rmsnorm_backward, rmsnorm_forward

    announce("rmsnorm_backward accumulate + misaligned rows=40 D=1024")
    rows, D = 40, 1024
    rng = np.random.default_rng(21)
    x = _bf(rng.standard_normal((rows, D)))
    w = _bf(1 + 0.1 * rng.standard_normal(D))
    dy = _bf(rng.standard_normal((rows, D)))
    xd, wd, dyd = x.cuda(), w.cuda(), dy.cuda()
    acc = torch.zeros(D, dtype=torch.float32, device="cuda")
    dx1, _ = rmsnorm_backward(dyd, xd, wd, 1e-6, grad_weight=acc)
    dx2, _ = rmsnorm_backward(dyd, xd, wd, 1e-6, grad_weight=acc)
    torch.cuda.synchronize()
    _, rdw = oracle.rmsnorm_bwd(dy.double().numpy(), x.double().numpy(), w.double().numpy(), 1e-6)
    assert rel_l2(acc, 2 * rdw) <= 1e-4
    assert torch.equal(dx1, dx2)

    def shifted(t):  # same values at an address 2 bytes past a 16-byte boundary
        buf = torch.empty(t.numel() + 1, dtype=t.dtype, device="cuda")
        v = buf[1:].view(t.shape)
        v.copy_(t)
        return v

    xs, ws, dys = shifted(xd), shifted(wd), shifted(dyd)
    assert xs.data_ptr() % 16 != 0
    y_al = rmsnorm_forward(xd, wd, 1e-6)
    y_mis = rmsnorm_forward(xs, ws, 1e-6)
    dxs, dws = rmsnorm_backward(dys, xs, ws, 1e-6)
    dxa, dwa = rmsnorm_backward(dyd, xd, wd, 1e-6)
    torch.cuda.synchronize()
    assert rel_l2(y_mis, y_al.float().cpu().numpy()) <= 1e-2
    assert rel_l2(dxs, dxa.float().cpu().numpy()) <= 1e-2
    assert rel_l2(dws, dwa.cpu().numpy()) <= 1e-5


@pytest.mark.parametrize("trans_a,trans_b", [(False, False), (True, False), (False, True),
                                             (True, True)])
def test_gemm_ex_strided_accumulating(trans_a, trans_b):
    """gemm_ex on column-block views with bias and beta accumulation, against
    an fp32 torch product of the same bf16 values."""
    from ceo_amd.nn import gemm_ex

    announce(f"gemm_ex trans_a={trans_a} trans_b={trans_b}")
    g = torch.Generator().manual_seed(3 + 2 * trans_a + trans_b)
    m, n, k = 192, 160, 96
    # operands as column blocks of wider matrices
    a_full = torch.randn(k if trans_a else m, (m if trans_a else k) + 40, generator=g)
    b_full = torch.randn(n if trans_b else k, (k if trans_b else n) + 24, generator=g)
    a = a_full.to(torch.bfloat16).cuda()[:, 8:8 + (m if trans_a else k)]
    b = b_full.to(torch.bfloat16).cuda()[:, 16:16 + (k if trans_b else n)]
    bias = (0.1 * torch.randn(n, generator=g)).to(torch.bfloat16).cuda()
    c = torch.randn(m, n, generator=g).to(torch.bfloat16).cuda()
    out_full = torch.zeros(m, n + 32, dtype=torch.bfloat16, device="cuda")
    out = out_full[:, 32:]
    gemm_ex(a, b, out, bias=bias, c=c, alpha=0.5, beta=2.0, trans_a=trans_a, trans_b=trans_b)
    torch.cuda.synchronize()
    af, bf = a.float(), b.float()
    ref = 0.5 * ((af.T if trans_a else af) @ (bf.T if trans_b else bf)) + bias.float() + 2.0 * c.float()
    e = rel_l2(out, ref.cpu().numpy())
    print(f"  rel-L2 {e:.2e}", flush=True)
    assert e <= 1e-2
    assert not out_full[:, :32].float().abs().sum().item()  # nothing written outside the view
    # in-place accumulation: out += a b
    before = out.float().clone()
    gemm_ex(a, b, out, c=out, beta=1.0, trans_a=trans_a, trans_b=trans_b)
    torch.cuda.synchronize()
    ref2 = before + (af.T if trans_a else af) @ (bf.T if trans_b else bf)
    assert rel_l2(out, ref2.cpu().numpy()) <= 1e-2


def test_layernorm_backward_residual(oracle):
    """layernorm_backward with a residual: the input gradient plus it."""
    from ceo_amd.nn import layernorm_backward, layernorm_forward

    rows, D = 300, 1024
    announce(f"layernorm_backward residual rows={rows} D={D}")
    rng = np.random.default_rng(17)
    x = _bf(rng.standard_normal((rows, D)))
    w = _bf(1 + 0.1 * rng.standard_normal(D))
    dy = _bf(rng.standard_normal((rows, D)))
    res = _bf(rng.standard_normal((rows, D)))
    for D2, sl in ((D, slice(None)), (96, slice(0, 96))):
        xs, ws, dys, rs = (x[:, sl].contiguous(), w[sl].contiguous(), dy[:, sl].contiguous(),
                           res[:, sl].contiguous())
        _, mean, rstd = layernorm_forward(xs.cuda(), ws.cuda(), None, 1e-5, save_stats=True)
        dx, dw, db = layernorm_backward(dys.cuda(), xs.cuda(), ws.cuda(), mean, rstd,
                                        residual=rs.cuda())
        torch.cuda.synchronize()
        _, rm, rr = oracle.layernorm_fwd(xs.float().numpy(), ws.float().numpy(), None, 1e-5)
        rdx, rdw, _ = oracle.layernorm_bwd(dys.float().numpy(), xs.float().numpy(),
                                           ws.float().numpy(), rm, rr)
        e = rel_l2(dx, rdx + rs.float().numpy())
        print(f"  D={D2} rel-L2 dx+res {e:.2e}", flush=True)
        assert e <= 1e-2 and rel_l2(dw, rdw) <= 1e-4


@pytest.mark.parametrize("rows,D", [(300, 1024), (4097, 2048), (513, 1536), (300, 96)])
def test_layernorm_backward_dx_colsum(rows, D):
    """layernorm_backward with out_dx_colsum: dx bit-identical to the call
    without it (dw and db too on the register path, D a multiple of 512 up to
    2048), and the column sums of the returned dx (from the register kernel's
    partials, or a separate pass on the looped path)."""
    from ceo_amd.nn import layernorm_backward, layernorm_forward

    announce(f"layernorm_backward dx colsum rows={rows} D={D}")
    g = torch.Generator(device="cuda").manual_seed(rows + D)
    x = torch.randn(rows, D, generator=g, device="cuda").to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(D, generator=g, device="cuda")).to(torch.bfloat16)
    dy = torch.randn(rows, D, generator=g, device="cuda").to(torch.bfloat16)
    res = torch.randn(rows, D, generator=g, device="cuda").to(torch.bfloat16)
    _, mean, rstd = layernorm_forward(x, w, None, 1e-5, save_stats=True)
    for r in (None, res):
        dx0, dw0, db0 = layernorm_backward(dy, x, w, mean, rstd, residual=r)
        cs = torch.full((D,), 7.0, dtype=torch.bfloat16, device="cuda")
        dx1, dw1, db1 = layernorm_backward(dy, x, w, mean, rstd, residual=r, out_dx_colsum=cs)
        # without dw / db the sums are still produced
        cs2 = torch.zeros_like(cs)
        dx2, _, _ = layernorm_backward(dy, x, w, mean, rstd, need_param_grads=False, residual=r,
                                       out_dx_colsum=cs2)
        torch.cuda.synchronize()
        assert torch.equal(dx0, dx1) and torch.equal(dx0, dx2)
        if D % 512 == 0:
            assert torch.equal(dw0, dw1) and torch.equal(db0, db1)
        else:
            # the looped kernel adds dw / db with LDS atomics: the order, and
            # so the last bits, vary from call to call
            torch.testing.assert_close(dw0, dw1, rtol=1e-5, atol=1e-4)
            torch.testing.assert_close(db0, db1, rtol=1e-5, atol=1e-4)
        ref = dx0.double().sum(0)
        e = rel_l2(cs, ref.cpu().numpy())
        print(f"  residual={r is not None} rel-L2 colsum {e:.2e}", flush=True)
        assert e <= 1e-2 and torch.equal(cs, cs2)
        # dw / db straight into bf16 buffers: the fp32 sums rounded once
        bw = torch.zeros(D, dtype=torch.bfloat16, device="cuda")
        bb = torch.zeros_like(bw)
        dx3, _, _ = layernorm_backward(dy, x, w, mean, rstd, residual=r, out_dw=bw, out_db=bb)
        torch.cuda.synchronize()
        assert torch.equal(dx3, dx0)
        if D % 512 == 0:
            assert torch.equal(bw, dw0.to(torch.bfloat16)) and torch.equal(bb, db0.to(torch.bfloat16))
        else:
            assert rel_l2(bw, dw0.cpu().numpy()) <= 1e-2 and rel_l2(bb, db0.cpu().numpy()) <= 1e-2


@pytest.fixture(params=[0, 1], ids=["mfma", "generic"])
def gemm_backend(request):
    """Runs a GEMM test on the library's kernels (the large-tile MFMA kernel
    where it takes the shape) and on its generic kernel only
    (efla_rt_set_gemm_backend), restoring the default afterwards."""
    from ceo_amd._lib import lib

    assert lib().efla_rt_set_gemm_backend(request.param) == 0
    yield request.param
    assert lib().efla_rt_set_gemm_backend(0) == 0


@pytest.mark.parametrize("m,k,n", [(256, 128, 384), (100, 70, 33), (1, 64, 8), (300, 1024, 260),
                                   (777, 3088, 520)])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
def test_gemm_forward(m, k, n, dt, gemm_backend):
    from ceo_amd.nn import gemm_forward

    announce(f"gemm_forward {m}x{k}x{n} {dt} backend={gemm_backend}")
    g = torch.Generator().manual_seed(m * 7 + n)
    a = torch.randn(m, k, generator=g).to(dt)
    b = torch.randn(k, n, generator=g).to(dt)
    bias = torch.randn(n, generator=g).to(dt)
    c = gemm_forward(a.cuda(), b.cuda(), bias.cuda())
    torch.cuda.synchronize()
    ref = a.double() @ b.double() + bias.double()
    e = rel_l2(c, ref.numpy())
    print(f"  rel-L2={e:.2e}", flush=True)
    assert e <= (1e-5 if dt == torch.float32 else 1e-2)


def test_gemm_forward_mixed_dtypes():
    from ceo_amd.nn import gemm_forward

    announce("gemm_forward mixed")
    a = torch.randn(70, 48).to(torch.bfloat16)
    b = torch.randn(48, 90)
    c = gemm_forward(a.cuda(), b.cuda(), None, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert rel_l2(c, (a.double() @ b.double()).numpy()) <= 1e-5


def test_gemm_bias_epilogue_at_layer_shape():
    """The bias epilogue on a config-4 projection shape, against torch."""
    from ceo_amd.nn import gemm_forward

    announce("gemm_forward 2048x1024x3072 bf16 + bias")
    g = torch.Generator(device="cuda").manual_seed(3)
    a = torch.randn(2048, 1024, generator=g, device="cuda").to(torch.bfloat16)
    b = (0.03 * torch.randn(1024, 3072, generator=g, device="cuda")).to(torch.bfloat16)
    bias = torch.randn(3072, generator=g, device="cuda").to(torch.bfloat16)
    c = gemm_forward(a, b, bias)
    ref = a.float() @ b.float() + bias.float()
    e = rel_l2(c, ref.cpu().numpy())
    print(f"  rel-L2={e:.2e}", flush=True)
    assert e <= 1e-2


def test_gemm_k0_gives_bias():
    announce("gemm_forward k=0")
    import ctypes

    from ceo_amd._lib import lib

    # gemm.cu:316-318 rejects null a/b even when k == 0 (torch hands out null
    # data pointers for empty tensors), so the C ABI gets real allocations
    m, n = 5, 7
    buf = torch.empty(8, dtype=torch.bfloat16, device="cuda")
    bias = torch.arange(n, dtype=torch.bfloat16, device="cuda")
    c = torch.full((m, n), 3.0, dtype=torch.bfloat16, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib().gemm_forward_hip(P(buf), P(buf), P(bias), P(c), m, 0, n, 14, 14, 14, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(c, bias.expand(m, n))
    assert lib().gemm_forward_hip(P(buf), P(buf), None, P(c), m, 0, n, 14, 14, 14, st) == 0
    torch.cuda.synchronize()
    assert torch.count_nonzero(c) == 0
    # null operands: InvalidValue (1), as the reference
    assert lib().gemm_forward_hip(None, P(buf), None, P(c), m, 0, n, 14, 14, 14, st) == 1


@pytest.mark.parametrize("case", ["bias", "beta_c", "bias_beta_c", "alias"])
def test_gemm_ex_k0_null_operands(case):
    """gemm_ex_hip with k = 0 and NULL a, b: D = bias + beta C with nothing to
    contract, bit for bit (beta is a power of two, so beta C is exact and the
    one rounding is bf16(fp32(bias + beta C)) in any evaluation order); C may
    be D itself."""
    import ctypes

    from ceo_amd._lib import lib

    announce(f"gemm_ex k=0 {case}")
    m, n, ld = 37, 24, 40  # D, C with a row stride wider than n
    g = torch.Generator(device="cuda").manual_seed(5 + len(case))
    bias = torch.randn(n, generator=g, device="cuda").to(torch.bfloat16)
    cbuf = torch.randn(m, ld, generator=g, device="cuda").to(torch.bfloat16)
    dbuf = torch.full((m, ld), float("nan"), device="cuda", dtype=torch.bfloat16)
    use_bias = case != "beta_c"
    beta = {"bias": 0.0, "beta_c": 0.5, "bias_beta_c": -2.0, "alias": 0.5}[case]
    if case == "alias":
        dbuf = cbuf.clone()
    c_in = (dbuf if case == "alias" else cbuf)[:, :n].float().clone()
    want = (bias.float() if use_bias else torch.zeros(n, device="cuda")) + beta * c_in
    want = want.to(torch.bfloat16)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    c_ptr = P(dbuf) if case == "alias" else (P(cbuf) if beta != 0.0 else None)
    rc = lib().gemm_ex_hip(0, 0, m, n, 0, ctypes.c_float(1.0), None, 0, None, 0,
                           P(bias) if use_bias else None, ctypes.c_float(beta), c_ptr, ld,
                           P(dbuf), ld, 14, st)
    torch.cuda.synchronize()
    assert rc == 0
    assert torch.equal(dbuf[:, :n], want)
    if case != "alias":  # the columns past n are not written
        assert torch.isnan(dbuf[:, n:]).all()


@pytest.mark.parametrize("m,k,n", [(256, 128, 384), (100, 70, 33), (513, 200, 129),
                                   (4096, 1032, 264)])
def test_gemm_backward(m, k, n, gemm_backend):
    from ceo_amd.nn import gemm_backward

    announce(f"gemm_backward {m}x{k}x{n} backend={gemm_backend}")
    g = torch.Generator().manual_seed(m + k + n)
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    b = torch.randn(k, n, generator=g).to(torch.bfloat16)
    dc = torch.randn(m, n, generator=g).to(torch.bfloat16)
    da, db, dbias = gemm_backward(dc.cuda(), a.cuda(), b.cuda(), need_bias=True)
    torch.cuda.synchronize()
    assert rel_l2(da, (dc.double() @ b.double().T).numpy()) <= 1e-2
    assert rel_l2(db, (a.double().T @ dc.double()).numpy()) <= 1e-2
    assert rel_l2(dbias, dc.double().sum(0).numpy()) <= 1e-2


def test_sigmoid_gate_forward_backward_vs_torch():
    # beta = sigmoid of the last H columns of a fused projection row, and its
    # gradient written back into that block of the fused gradient row
    from ceo_amd import nn

    announce("sigmoid gate: fused-row block vs torch")
    torch.manual_seed(7)
    N, W, H = 3000, 3088, 16
    p = (torch.randn(N, W, device="cuda:0") * 4).to(torch.bfloat16)
    beta = nn.sigmoid_gate_forward(p[:, W - H:])
    ref = torch.sigmoid(p[:, W - H:].float()).to(torch.bfloat16)
    # fp32 sigmoid then bf16 rounding: at most one bf16 step apart from torch's
    diff = (beta.float() - ref.float()).abs()
    assert (diff <= ref.float().abs() * 2.0 ** -7).all()
    print(f"  forward: {(diff > 0).sum().item()} of {N * H} differ by one bf16 step",
          flush=True)
    g = torch.randn(N, H, device="cuda:0").to(torch.bfloat16)
    dp = torch.full((N, W), float("nan"), device="cuda:0", dtype=torch.bfloat16)
    nn.sigmoid_gate_backward(g, beta, dp[:, W - H:])
    bf = beta.float()
    want = (g.float() * bf * (1.0 - bf)).to(torch.bfloat16)
    assert torch.equal(dp[:, W - H:], want)
    assert torch.isnan(dp[:, :W - H]).all()  # nothing written outside the block


# ---------------------------------------------------------------------------
# the large-tile kernel (gemm_fast.hpp): transposes, residual, split-K, GELU
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("m,k,n", [(600, 1000, 328), (256, 64, 256), (40, 8, 8)])
def test_gemm_ex_transposes_residual(m, k, n, ta, tb, gemm_backend):
    """out = 0.5 op(a) op(b) + bias + out, for every transpose combination,
    against torch fp32; shapes with k-tails (1000 = 15 x 64 + 40) and edge tiles."""
    from ceo_amd import nn

    announce(f"gemm_ex {m}x{k}x{n} ta={ta} tb={tb} backend={gemm_backend}")
    g = torch.Generator(device="cuda").manual_seed(m + 3 * k + 7 * n + 2 * ta + tb)
    a = torch.randn(m, k, generator=g, device="cuda").to(torch.bfloat16)
    b = (0.1 * torch.randn(k, n, generator=g, device="cuda")).to(torch.bfloat16)
    bias = torch.randn(n, generator=g, device="cuda").to(torch.bfloat16)
    out = torch.randn(m, n, generator=g, device="cuda").to(torch.bfloat16)
    ref = 0.5 * (a.float() @ b.float()) + bias.float() + out.float()
    A = a.t().contiguous() if ta else a
    B = b.t().contiguous() if tb else b
    nn.gemm_ex(A, B, out, bias=bias, c=out, alpha=0.5, beta=1.0, trans_a=bool(ta),
               trans_b=bool(tb))
    e = rel_l2(out, ref.cpu().numpy())
    print(f"  rel-L2={e:.2e}", flush=True)
    assert e <= 1e-2


def test_gemm_split_k_deterministic():
    """An output with few tiles and a long contraction (the weight gradient of
    a config-4 projection) runs split along k with an ordered reduction: the
    same inputs give the same bits, and the result matches fp64 (sampled)."""
    from ceo_amd import nn

    announce("gemm_backward dB 16384 x 1024 x 1024 (split-K), twice")
    g = torch.Generator(device="cuda").manual_seed(11)
    a = torch.randn(16384, 1024, generator=g, device="cuda").to(torch.bfloat16)
    w = torch.randn(1024, 1024, generator=g, device="cuda").to(torch.bfloat16)
    dc = torch.randn(16384, 1024, generator=g, device="cuda").to(torch.bfloat16)
    _, db1, _ = nn.gemm_backward(dc, a, w, need_a=False)
    _, db2, _ = nn.gemm_backward(dc, a, w, need_a=False)
    torch.cuda.synchronize()
    assert torch.equal(db1, db2)
    cols = torch.arange(0, 1024, 37, device="cuda")
    ref = a.double().t() @ dc.double()[:, cols]
    e = rel_l2(db1[:, cols], ref.cpu().numpy())
    print(f"  rel-L2={e:.2e}", flush=True)
    assert e <= 1e-2


@pytest.mark.parametrize("m,k,n", [(2048, 1024, 4096), (300, 200, 264), (130, 70, 33)])
def test_gemm_gelu_fused(m, k, n):
    """gemm_gelu_forward / gemm_gelu_backward: pre = a b + bias, out =
    GELU_tanh(bf16(pre)); dpre = bf16(dc b2^T) GELU'(pre), db2 = out^T dc,
    dbias = colsum(dc), against torch fp32 with the same bf16 roundings
    (the last shape is not one the large-tile kernel takes: fallback path)."""
    from ceo_amd import nn

    announce(f"gemm_gelu fused {m}x{k}x{n}")
    g = torch.Generator(device="cuda").manual_seed(m + k + n)
    a = torch.randn(m, k, generator=g, device="cuda").to(torch.bfloat16)
    w = (0.05 * torch.randn(k, n, generator=g, device="cuda")).to(torch.bfloat16)
    bias = torch.randn(n, generator=g, device="cuda").to(torch.bfloat16)
    pre, out = nn.gemm_gelu_forward(a, w, bias)
    pre_ref = (a.float() @ w.float() + bias.float()).to(torch.bfloat16)
    out_ref = torch.nn.functional.gelu(pre_ref.float(), approximate="tanh")
    e1, e2 = rel_l2(pre, pre_ref.float().cpu().numpy()), rel_l2(out, out_ref.cpu().numpy())
    # the MLP's second product and its backward through the GELU
    w2 = (0.05 * torch.randn(n, k, generator=g, device="cuda")).to(torch.bfloat16)
    dc = torch.randn(m, k, generator=g, device="cuda").to(torch.bfloat16)
    dpb = torch.full((n,), 3.0, dtype=torch.bfloat16, device="cuda")
    dpre, dw2, dbias = nn.gemm_gelu_backward(dc, out, w2, pre, need_bias=True,
                                             out_pre_bias=dpb)
    x = pre.float().requires_grad_(True)
    gl = torch.nn.functional.gelu(x, approximate="tanh")
    (gl * (dc.float() @ w2.float().t()).to(torch.bfloat16).float()).sum().backward()
    e3 = rel_l2(dpre, x.grad.cpu().numpy())
    e4 = rel_l2(dw2, (out.float().t() @ dc.float()).cpu().numpy())
    e5 = rel_l2(dbias, dc.float().sum(0).cpu().numpy())
    # the pre-activation bias gradient: column sums of the dpre returned
    e6 = rel_l2(dpb, dpre.double().sum(0).cpu().numpy())
    dpre2, _, _ = nn.gemm_gelu_backward(dc, out, w2, pre, need_b=False)
    torch.cuda.synchronize()
    assert torch.equal(dpre, dpre2)
    print(f"  rel-L2 pre {e1:.2e} out {e2:.2e} dpre {e3:.2e} dw2 {e4:.2e} dbias {e5:.2e} "
          f"dpre colsum {e6:.2e}", flush=True)
    assert max(e1, e2, e3, e4, e5, e6) <= 1e-2


@pytest.mark.parametrize("name,m,k,n", [("qkv", 16384, 1024, 3088), ("out", 16384, 1024, 1024),
                                        ("up", 16384, 1024, 4096), ("down", 16384, 4096, 1024)])
def test_gemm_config4_products(name, m, k, n):
    """Every product of a config-4 layer at its full size on the default
    (hand-written) kernel: the forward with bias, the input gradient, the
    weight gradient (split-K) and the bias gradient, against torch fp32."""
    from ceo_amd import nn

    announce(f"gemm config-4 {name} {m}x{k}x{n}: forward, dA, dB, dbias")
    g = torch.Generator(device="cuda").manual_seed(k + n)
    a = torch.randn(m, k, generator=g, device="cuda").to(torch.bfloat16)
    w = (0.03 * torch.randn(k, n, generator=g, device="cuda")).to(torch.bfloat16)
    bias = torch.randn(n, generator=g, device="cuda").to(torch.bfloat16)
    dc = torch.randn(m, n, generator=g, device="cuda").to(torch.bfloat16)
    c = nn.gemm_forward(a, w, bias)
    e0 = rel_l2(c, (a.float() @ w.float() + bias.float()).cpu().numpy())
    da, dw, db = nn.gemm_backward(dc, a, w, need_bias=True)
    e1 = rel_l2(da, (dc.float() @ w.float().t()).cpu().numpy())
    e2 = rel_l2(dw, (a.float().t() @ dc.float()).cpu().numpy())
    e3 = rel_l2(db, dc.float().sum(0).cpu().numpy())
    print(f"  rel-L2 fwd {e0:.2e} dA {e1:.2e} dB {e2:.2e} dbias {e3:.2e}", flush=True)
    assert max(e0, e1, e2, e3) <= 1e-2


def test_gemm_gelu_config4_mlp():
    """The config-4 MLP's fused products at full size: up-projection with bias
    and GELU (pre-activation kept), and the down-projection's input gradient
    through GELU', against torch fp32 with the same bf16 roundings."""
    from ceo_amd import nn

    m, d, f = 16384, 1024, 4096
    announce(f"gemm_gelu config-4 MLP {m}x{d}x{f}")
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(m, d, generator=g, device="cuda").to(torch.bfloat16)
    w_up = (0.03 * torch.randn(d, f, generator=g, device="cuda")).to(torch.bfloat16)
    b_up = torch.randn(f, generator=g, device="cuda").to(torch.bfloat16)
    w_down = (0.02 * torch.randn(f, d, generator=g, device="cuda")).to(torch.bfloat16)
    pre, out = nn.gemm_gelu_forward(x, w_up, b_up)
    pre_ref = (x.float() @ w_up.float() + b_up.float()).to(torch.bfloat16)
    e1 = rel_l2(pre, pre_ref.float().cpu().numpy())
    e2 = rel_l2(out, torch.nn.functional.gelu(pre_ref.float(), approximate="tanh").cpu().numpy())
    dy = torch.randn(m, d, generator=g, device="cuda").to(torch.bfloat16)
    db_up = torch.empty(f, dtype=torch.bfloat16, device="cuda")
    dpre, dw, db = nn.gemm_gelu_backward(dy, out, w_down, pre, need_bias=True,
                                         out_pre_bias=db_up)
    t = pre.float().requires_grad_(True)
    gl = torch.nn.functional.gelu(t, approximate="tanh")
    (gl * (dy.float() @ w_down.float().t()).to(torch.bfloat16).float()).sum().backward()
    e3 = rel_l2(dpre, t.grad.cpu().numpy())
    e4 = rel_l2(dw, (out.float().t() @ dy.float()).cpu().numpy())
    e5 = rel_l2(db, dy.float().sum(0).cpu().numpy())
    e6 = rel_l2(db_up, dpre.double().sum(0).cpu().numpy())
    print(f"  rel-L2 pre {e1:.2e} out {e2:.2e} dpre {e3:.2e} dw {e4:.2e} dbias {e5:.2e} "
          f"dpre colsum {e6:.2e}", flush=True)
    assert max(e1, e2, e3, e4, e5, e6) <= 1e-2
