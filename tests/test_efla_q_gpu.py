"""Chunked query-readout EFLA on the GPU against the fp64 oracle.

Tolerances: rel-L2 <= 1e-4 for the fp32 path,
<= 2e-2 for bf16 inputs with fp32 accumulation, on O, dq, dk, dv, dbeta (and
the final / initial state and their gradients when present).
"""
import numpy as np
import pytest
import torch

from helpers import announce, rel_l2, to_dev

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


def _case(oracle, seed, B, T, H, K, V, dtype, *, s0=False, dst=False, cu=None, xform=None):
    from ceo_amd.efla import chunk_efla_bwd, chunk_efla_fwd

    announce(f"chunk_efla B={B} T={T} H={H} K={K} V={V} {dtype} s0={s0} dst={dst} "
             f"varlen={cu is not None}" + (f" {xform.__name__}" if xform else ""))
    ntok = B * T
    x = oracle.make_efla_inputs(seed, ntok, H, K, V, bf16=dtype == torch.bfloat16)
    if xform is not None:
        x = xform(oracle, x, dtype == torch.bfloat16)
    N = B if cu is None else len(cu) - 1
    rng = np.random.default_rng(seed)
    S0 = (rng.standard_normal((N, H, K, V)) * 0.3).astype(np.float32) if s0 else None
    dST = rng.standard_normal((N, H, K, V)).astype(np.float32) if dst else None
    g = {n: to_dev(a, dtype, (B, T, H, K) if n in "qk" else
                   (B, T, H) if n == "beta" else (B, T, H, V)) for n, a in x.items()}
    cu_t = None if cu is None else torch.tensor(cu, dtype=torch.int32, device="cuda:0")
    s0_t = None if S0 is None else torch.from_numpy(S0).cuda()
    dst_t = None if dST is None else torch.from_numpy(dST).cuda()
    o, st = chunk_efla_fwd(g["q"], g["k"], g["v"], g["beta"], s0_t, True, cu_t)
    dq, dk, dv, db, ds0 = chunk_efla_bwd(g["q"], g["k"], g["v"], g["beta"], g["do"], s0_t,
                                         dst_t, cu_t)
    torch.cuda.synchronize()
    kw = dict(cu_seqlens=cu) if cu is not None else dict(T=T)
    ro, rst = oracle.q_forward(x["q"], x["k"], x["v"], x["beta"], S0=S0, **kw)
    rg = oracle.q_backward(x["q"], x["k"], x["v"], x["beta"], x["do"], S0=S0, dST=dST, **kw)
    errs = {"o": rel_l2(o, ro), "S_T": rel_l2(st, rst), "dq": rel_l2(dq, rg[0]),
            "dk": rel_l2(dk, rg[1]), "dv": rel_l2(dv, rg[2]), "dbeta": rel_l2(db, rg[3])}
    if s0:
        errs["dS0"] = rel_l2(ds0, rg[4])
    print("  rel-L2:", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    tol = TOL[dtype]
    bad = {k: v for k, v in errs.items() if not v <= tol}
    assert not bad, bad


def test_cfg1_fp32(oracle):
    # B=2, T=256, H=4, d_k=d_v=64, chunk 64, fp32
    _case(oracle, 0xEF1A0000, 2, 256, 4, 64, 64, torch.float32)


def test_fp32_ragged_with_states(oracle):
    _case(oracle, 11, 2, 200, 3, 64, 64, torch.float32, s0=True, dst=True)


@pytest.mark.parametrize("K,V", [(64, 64), (128, 128), (128, 256), (64, 128), (128, 64),
                                 (64, 256)])
def test_bf16_shapes(oracle, K, V):
    _case(oracle, 100 + K + V, 2, 192, 2, K, V, torch.bfloat16)


def test_bf16_ragged_states(oracle):
    _case(oracle, 21, 2, 301, 2, 128, 128, torch.bfloat16, s0=True, dst=True)


@pytest.mark.parametrize("T", [1, 63, 64, 65])
def test_bf16_short_sequences(oracle, T):
    _case(oracle, 30 + T, 3, T, 2, 64, 64, torch.bfloat16, s0=True, dst=True)


@pytest.mark.parametrize("K,V", [(128, 128), (128, 256)])
def test_bf16_long_sequence(oracle, K, V):
    # full benchmark sequence length: rounding must not accumulate over 128
    # chunks of the state recurrence
    _case(oracle, 0xEF1A0002 + V, 1, 8192, 2, K, V, torch.bfloat16, s0=True, dst=True)


# lambda = |k|^2 per token, cycling over the coefficient's regimes: below the
# reference's series branch point (lambda <= 1e-6, efla.cu:93-115), inside this
# library's series range (beta lambda < 0.03, beta < 1), and one all-zero k per
# head (lambda = 0, where c = beta and dc/dlambda = -beta^2 / 2 exactly).
SMALL_K_SCALES = (3e-4, 9e-4, 0.05, 0.15, 0.1)


def small_lambda(oracle, x, bf16):
    k = x["k"].astype(np.float64).copy()
    scale = np.array([SMALL_K_SCALES[i % len(SMALL_K_SCALES)] for i in range(k.shape[0])])
    k *= scale[:, None, None]
    k[5] = 0.0
    x = dict(x)
    x["k"] = oracle.round_bf16(k) if bf16 else k.astype(np.float32)
    lam = (x["k"].astype(np.float64) ** 2).sum(-1)
    assert lam.max() < 0.03 and (lam[1::len(SMALL_K_SCALES)] <= 1e-6).all() and lam[5].max() == 0
    return x


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_small_lambda_coefficient_branch(oracle, dtype):
    """Every token's coefficient comes from the short-lambda series (and the
    lambda -> 0 limit of dc/dlambda drives dk): the fp32 path must hold
    1e-4 against the fp64 oracle, which evaluates c with expm1."""
    _case(oracle, 0x5A11, 2, 150, 2, 64, 64, dtype, s0=True, dst=True, xform=small_lambda)


@pytest.mark.parametrize("K,V", [(128, 128), (64, 64)])
def test_small_lambda_bf16_fast_kernels(oracle, K, V):
    _case(oracle, 0x5A12 + K, 2, 200, 2, K, V, torch.bfloat16, s0=True, dst=True,
          xform=small_lambda)


def zero_beta(oracle, x, bf16):
    """beta = 0 on a few tokens inside the sequences (b = c(0, lambda) = 0):
    the bf16 gradient kernel then forms dL/db of those 16-token blocks from
    rowsum(Y o R) + rowsum(dA o G) instead of rowsum(Y o Vn) / b."""
    beta = x["beta"].copy()
    beta[[5, 81, 150, 263, 300]] = 0.0
    x = dict(x)
    x["beta"] = beta
    return x


@pytest.mark.parametrize("K,V", [(128, 128), (64, 64)])
def test_zero_beta_tokens_bf16_fast_kernels(oracle, K, V):
    _case(oracle, 0x0B0 + K, 2, 200, 2, K, V, torch.bfloat16, s0=True, dst=True, xform=zero_beta)


def test_nan_inf_stay_in_their_sequence_and_head(oracle):
    """A NaN in one token's k and an Inf in another sequence's v contaminate
    only their own (sequence, head): every other (sequence, head) gets outputs
    and gradients bit-identical to a clean run, and finite; the contaminated
    ones carry non-finite values from the next chunk on (failure detection:
    a NaN or Inf injected into the inputs must propagate, and only there)."""
    from ceo_amd.efla import chunk_efla_bwd, chunk_efla_fwd

    B, T, H, K, V = 3, 200, 2, 128, 128
    announce(f"chunk_efla NaN/Inf isolation B={B} T={T} H={H} K={K} V={V}")
    x = oracle.make_efla_inputs(0xBAD, B * T, H, K, V, bf16=True)
    g = {n: to_dev(a, torch.bfloat16, (B, T, H, K) if n in "qk" else
                   (B, T, H) if n == "beta" else (B, T, H, V)) for n, a in x.items()}

    def run(gg):
        o, st = chunk_efla_fwd(gg["q"], gg["k"], gg["v"], gg["beta"], None, True)
        grads = chunk_efla_bwd(gg["q"], gg["k"], gg["v"], gg["beta"], gg["do"])
        torch.cuda.synchronize()
        return [o, st] + list(grads[:4])

    clean = run(g)
    bad = {n: t.clone() for n, t in g.items()}
    bad["k"][0, 70, 0, 3] = float("nan")
    bad["v"][2, 150, 1, 5] = float("inf")
    dirty = run(bad)
    names = ["o", "S_T", "dq", "dk", "dv", "dbeta"]
    hit = {(0, 0), (2, 1)}
    for n, a, b in zip(names, clean, dirty):
        for bb in range(B):
            for hh in range(H):
                sa, sb = (a[bb, hh], b[bb, hh]) if n == "S_T" else (a[bb, :, hh], b[bb, :, hh])
                if (bb, hh) in hit:
                    continue
                assert torch.isfinite(sb.float()).all(), (n, bb, hh)
                assert torch.equal(sa, sb), (n, bb, hh)
    # propagation: from the chunk after the bad token on, the output is not finite
    assert not torch.isfinite(dirty[0][0, 128:, 0].float()).any()
    assert not torch.isfinite(dirty[0][2, 192:, 1].float()).all()
    assert not torch.isfinite(dirty[1][0, 0].float()).all()
    for i in range(2, 6):  # every gradient of the NaN's (sequence, head) is hit
        d = dirty[i]
        assert not torch.isfinite(d[0, :, 0].float()).all(), names[i]


def test_varlen_bf16(oracle):
    lens = [1, 63, 64, 65, 130, 7, 0, 200]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    _case(oracle, 41, 1, int(cu[-1]), 2, 128, 256, torch.bfloat16, s0=True, dst=True,
          cu=cu)


def test_varlen_fp32(oracle):
    lens = [17, 64, 100]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    _case(oracle, 42, 1, int(cu[-1]), 2, 64, 64, torch.float32, s0=True, dst=True, cu=cu)


def test_empty_sequence_passes_state_through(oracle):
    from ceo_amd.efla import chunk_efla_bwd, chunk_efla_fwd

    announce("chunk_efla T=0")
    q = torch.zeros(2, 0, 2, 64, dtype=torch.bfloat16, device="cuda:0")
    beta = torch.zeros(2, 0, 2, dtype=torch.bfloat16, device="cuda:0")
    s0 = torch.randn(2, 2, 64, 64, device="cuda:0")
    o, st = chunk_efla_fwd(q, q, q, beta, s0, True)
    assert o.numel() == 0
    assert torch.equal(st, s0)
    dht = torch.randn_like(s0)
    *_, dh0 = chunk_efla_bwd(q, q, q, beta, q, s0, dht)
    assert torch.equal(dh0, dht)


def test_caller_workspace_matches_cached(oracle):
    from ceo_amd.efla import chunk_efla_fwd, workspace_bytes

    announce("chunk_efla caller workspace")
    B, T, H, K, V = 2, 128, 2, 128, 128
    x = oracle.make_efla_inputs(77, B * T, H, K, V, bf16=True)
    g = {n: to_dev(a, torch.bfloat16, (B, T, H, K) if n in "qk" else
                   (B, T, H) if n == "beta" else (B, T, H, V)) for n, a in x.items()}
    o1, _ = chunk_efla_fwd(g["q"], g["k"], g["v"], g["beta"])
    nbytes = workspace_bytes("fwd", B, T, H, K, V, torch.bfloat16)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda:0")
    o2, _ = chunk_efla_fwd(g["q"], g["k"], g["v"], g["beta"], workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


def test_autograd_function(oracle):
    from ceo_amd.efla import chunk_efla

    announce("chunk_efla autograd")
    B, T, H, K, V = 1, 130, 2, 64, 64
    x = oracle.make_efla_inputs(88, B * T, H, K, V, bf16=False)
    g = {n: to_dev(a, torch.float32, (B, T, H, K) if n in "qk" else
                   (B, T, H) if n == "beta" else (B, T, H, V)).requires_grad_(n != "do")
         for n, a in x.items()}
    o, _ = chunk_efla(g["q"], g["k"], g["v"], g["beta"])
    (o * g["do"]).sum().backward()
    rg = oracle.q_backward(x["q"], x["k"], x["v"], x["beta"], x["do"], T=T)
    for name, ref in zip(("q", "k", "v", "beta"), rg[:4]):
        assert rel_l2(g[name].grad, ref) <= 1e-4, name


@pytest.mark.parametrize("states", [False, True], ids=["factors", "factors+states"])
@pytest.mark.parametrize("dtype,K,V", [(torch.bfloat16, 128, 128), (torch.bfloat16, 64, 256),
                                       (torch.float32, 64, 64)])
def test_backward_reusing_forward_factors(oracle, dtype, K, V, states):
    from ceo_amd.efla import chunk_efla_bwd, chunk_efla_fwd, new_workspace

    announce(f"chunk_efla reuse_forward states={states} {dtype} K={K} V={V}")
    B, T, H = 2, 200, 2
    x = oracle.make_efla_inputs(91, B * T, H, K, V, bf16=dtype == torch.bfloat16)
    g = {n: to_dev(a, dtype, (B, T, H, K) if n in "qk" else
                   (B, T, H) if n == "beta" else (B, T, H, V)) for n, a in x.items()}
    s0 = 0.1 * torch.randn(B, H, K, V, generator=torch.Generator().manual_seed(5)).cuda()
    ws = new_workspace(g["q"], g["v"])
    o_ws, _ = chunk_efla_fwd(g["q"], g["k"], g["v"], g["beta"], s0, workspace=ws,
                             save_states=states)
    got = chunk_efla_bwd(g["q"], g["k"], g["v"], g["beta"], g["do"], s0, workspace=ws,
                         reuse_forward=True, reuse_states=states)
    o_ref, _ = chunk_efla_fwd(g["q"], g["k"], g["v"], g["beta"], s0)
    ref = chunk_efla_bwd(g["q"], g["k"], g["v"], g["beta"], g["do"], s0)
    torch.cuda.synchronize()
    assert torch.equal(o_ws, o_ref)
    for a, b, n in zip(got, ref, ("dq", "dk", "dv", "dbeta", "dh0")):
        if dtype == torch.bfloat16:
            assert torch.equal(a, b), n  # same kernels, same order: bit-identical
        else:
            # the generic fp32 path sums dL/db with LDS float atomics, whose order varies
            assert rel_l2(a, b.float().cpu().numpy()) <= 1e-6, n


def test_packed_batch_runs_sequences_independently(oracle):
    """efla_pack_sequences output drives the varlen entries: each packed
    sequence's outputs and gradients equal a separate run on that sequence."""
    from ceo_amd.data import pack_sequences
    from ceo_amd.efla import chunk_efla_bwd, chunk_efla_fwd

    announce("packed sequences -> varlen EFLA == per-sequence runs")
    rng = np.random.default_rng(12)
    H, K, V = 2, 64, 128
    lens = [int(x) for x in rng.integers(1, 300, 12)]
    ids = [np.arange(sum(lens[:i]), sum(lens[:i]) + n) for i, n in enumerate(lens)]
    p = pack_sequences(ids, 1500)
    assert 0 < p.num_sequences < len(lens)  # some sequences skipped
    ntok = int(p.cu_seqlens[-1])
    x = oracle.make_efla_inputs(5, sum(lens), H, K, V, bf16=True)
    rows = p.tokens.astype(np.int64)  # packed token -> row of the unpacked inputs
    g = {n: to_dev(a[rows], torch.bfloat16, (1, ntok, H, K) if n in "qk" else
                   (1, ntok, H) if n == "beta" else (1, ntok, H, V)) for n, a in x.items()}
    cu = p.cu_seqlens_device()
    o, _ = chunk_efla_fwd(g["q"], g["k"], g["v"], g["beta"], cu_seqlens=cu)
    grads = chunk_efla_bwd(g["q"], g["k"], g["v"], g["beta"], g["do"], cu_seqlens=cu)
    for s in range(p.num_sequences):
        a, b = int(p.cu_seqlens[s]), int(p.cu_seqlens[s + 1])
        one = {n: t[:, a:b].contiguous() for n, t in g.items()}
        o1, _ = chunk_efla_fwd(one["q"], one["k"], one["v"], one["beta"])
        g1 = chunk_efla_bwd(one["q"], one["k"], one["v"], one["beta"], one["do"])
        assert torch.equal(o[:, a:b], o1), s
        for big, small in zip(grads[:4], g1[:4]):
            assert torch.equal(big[:, a:b], small), s


@pytest.mark.parametrize("reuse", [False, True], ids=["recompute", "reuse-states"])
def test_many_sequences_scans_match_per_sequence_runs(oracle, reuse):
    """A varlen batch whose state scans have more (sequence, head, value
    slice) workgroups than the GPU has CUs, so they run in several rounds,
    and whose gradient kernel meets sequence boundaries inside its items'
    loop: each sequence's outputs and gradients must match its own run bit
    for bit, with the forward's states reused and recomputed."""
    from ceo_amd.efla import chunk_efla_bwd, chunk_efla_fwd, new_workspace

    H, K, V = 4, 128, 128
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    nseq = cus // (H * V // 64) + 9  # scan grid above the CU count
    announce(f"{nseq} sequences (scan grid {nseq * H * V // 64} > {cus} CUs) == per-sequence runs")
    rng = np.random.default_rng(21)
    lens = [int(x) for x in rng.integers(1, 200, nseq)]
    ntok = sum(lens)
    cu_np = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    x = oracle.make_efla_inputs(6, ntok, H, K, V, bf16=True)
    g = {n: to_dev(a, torch.bfloat16, (1, ntok, H, K) if n in "qk" else
                   (1, ntok, H) if n == "beta" else (1, ntok, H, V)) for n, a in x.items()}
    cu = torch.from_numpy(cu_np).to("cuda")

    def run(t, cu_t):
        if reuse:
            ws = new_workspace(t["q"], t["v"], cu_t)
            o, _ = chunk_efla_fwd(t["q"], t["k"], t["v"], t["beta"], cu_seqlens=cu_t, workspace=ws,
                                  save_states=True)
            gr = chunk_efla_bwd(t["q"], t["k"], t["v"], t["beta"], t["do"], cu_seqlens=cu_t,
                                workspace=ws, reuse_forward=True, reuse_states=True)
        else:
            o, _ = chunk_efla_fwd(t["q"], t["k"], t["v"], t["beta"], cu_seqlens=cu_t)
            gr = chunk_efla_bwd(t["q"], t["k"], t["v"], t["beta"], t["do"], cu_seqlens=cu_t)
        torch.cuda.synchronize()
        return o.clone(), [u.clone() for u in gr[:4]]

    o, grads = run(g, cu)
    for s in range(nseq):
        a, b = int(cu_np[s]), int(cu_np[s + 1])
        one = {n: t[:, a:b].contiguous() for n, t in g.items()}
        o1, g1 = run(one, None)
        assert torch.equal(o[:, a:b], o1), s
        for big, small in zip(grads, g1):
            assert torch.equal(big[:, a:b], small), s


# The gradient kernel is persistent: min(#CUs, items) workgroups each loop over
# (chunk, head) items, copying the next item's inputs into LDS while the
# current one finishes.  At test sizes every workgroup would get one item, so
# EFLA_GRAD_WORKGROUPS caps the grid and makes each workgroup run many items,
# including partial chunks and sequence boundaries in the middle of its loop.
def _grads(g, cu_t, s0_t, dst_t, reuse):
    from ceo_amd.efla import chunk_efla_bwd, chunk_efla_fwd, new_workspace

    if reuse:
        ws = new_workspace(g["q"], g["v"], cu_t)
        chunk_efla_fwd(g["q"], g["k"], g["v"], g["beta"], s0_t, cu_seqlens=cu_t, workspace=ws,
                       save_states=True)
        out = chunk_efla_bwd(g["q"], g["k"], g["v"], g["beta"], g["do"], s0_t, dst_t,
                             cu_seqlens=cu_t, workspace=ws, reuse_forward=True,
                             reuse_states=True)
    else:
        out = chunk_efla_bwd(g["q"], g["k"], g["v"], g["beta"], g["do"], s0_t, dst_t,
                             cu_seqlens=cu_t)
    torch.cuda.synchronize()
    return [t.clone() for t in out]


@pytest.mark.parametrize("reuse", [False, True], ids=["recompute", "reuse-states"])
@pytest.mark.parametrize("K,V", [(128, 128), (64, 256), (64, 64)])
def test_grad_kernel_grid_cap_bit_exact(oracle, monkeypatch, K, V, reuse):
    announce(f"grad kernel grid cap K={K} V={V} reuse={reuse}")
    lens = [130, 64, 1, 0, 257, 63, 65, 200, 9, 128]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    ntok, H = int(cu[-1]), 3
    x = oracle.make_efla_inputs(57 + K + V, ntok, H, K, V, bf16=True)
    g = {n: to_dev(a, torch.bfloat16, (1, ntok, H, K) if n in "qk" else
                   (1, ntok, H) if n == "beta" else (1, ntok, H, V)) for n, a in x.items()}
    cu_t = torch.tensor(cu, dtype=torch.int32, device="cuda:0")
    rng = np.random.default_rng(3)
    s0_t = torch.from_numpy((rng.standard_normal((len(lens), H, K, V)) * 0.3)
                            .astype(np.float32)).cuda()
    dst_t = torch.from_numpy(rng.standard_normal((len(lens), H, K, V)).astype(np.float32)).cuda()
    monkeypatch.delenv("EFLA_GRAD_WORKGROUPS", raising=False)
    ref = _grads(g, cu_t, s0_t, dst_t, reuse)
    for cap in ("1", "3", "7"):
        monkeypatch.setenv("EFLA_GRAD_WORKGROUPS", cap)
        got = _grads(g, cu_t, s0_t, dst_t, reuse)
        for a, b, n in zip(got, ref, ("dq", "dk", "dv", "dbeta", "dS0")):
            assert torch.equal(a, b), (cap, n)


def test_grad_kernel_many_items_per_workgroup_vs_oracle(oracle, monkeypatch):
    # the varlen case above, with 3 workgroups looping over all the items
    monkeypatch.setenv("EFLA_GRAD_WORKGROUPS", "3")
    lens = [1, 63, 64, 65, 130, 7, 0, 200]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    _case(oracle, 43, 1, int(cu[-1]), 2, 128, 256, torch.bfloat16, s0=True, dst=True, cu=cu)


# Token-strided I/O: q, k, v read as column slices of one fused row per token
# and dq, dk, dv written into the slices of a fused gradient row, as a model
# with a fused q/k/v/beta projection holds them.  The pad columns hold NaN, so
# a read outside the slices would show in the outputs, and a write outside
# them in the pad; the results must equal the packed call's bit for bit.
def _fused(parts, pad, fill):
    N = parts[0].shape[0] * parts[0].shape[1]
    widths = [p.shape[2] * p.shape[3] for p in parts]
    buf = torch.full((N, sum(widths) + pad), fill, dtype=torch.bfloat16, device="cuda:0")
    views, c = [], 0
    for p, w in zip(parts, widths):
        buf[:, c:c + w] = p.reshape(N, w)
        views.append(buf[:, c:c + w].view(p.shape))
        c += w
    return buf, views


@pytest.mark.parametrize("reuse", [False, True], ids=["recompute", "reuse-states"])
@pytest.mark.parametrize("layout", ["fixed", "varlen"])
@pytest.mark.parametrize("K,V", [(64, 64), (128, 128), (64, 256)])
def test_token_strided_io_bit_exact(oracle, K, V, layout, reuse):
    from ceo_amd.efla import chunk_efla_bwd, chunk_efla_fwd, new_workspace, token_stride

    announce(f"token-strided io K={K} V={V} {layout} reuse={reuse}")
    H = 3
    if layout == "fixed":
        B, T, cu = 2, 200, None
    else:
        lens = [70, 1, 130, 0, 64, 99]
        cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        B, T = 1, int(cu[-1])
    N = B if cu is None else len(cu) - 1
    x = oracle.make_efla_inputs(91 + K + V, B * T, H, K, V, bf16=True)
    g = {n: to_dev(a, torch.bfloat16, (B, T, H, K) if n in "qk" else
                   (B, T, H) if n == "beta" else (B, T, H, V)) for n, a in x.items()}
    cu_t = None if cu is None else torch.tensor(cu, dtype=torch.int32, device="cuda:0")
    rng = np.random.default_rng(5)
    s0 = torch.from_numpy((rng.standard_normal((N, H, K, V)) * 0.3).astype(np.float32)).cuda()
    dst = torch.from_numpy(rng.standard_normal((N, H, K, V)).astype(np.float32)).cuda()
    nan = float("nan")
    _, (q, k, v) = _fused([g["q"], g["k"], g["v"]], 24, nan)
    assert token_stride(q) == H * (2 * K + V) + 24
    gbuf, gviews = _fused([torch.empty_like(g["q"]), torch.empty_like(g["k"]),
                           torch.empty_like(g["v"])], 24, nan)

    def run(qq, kk, vv, grads_out):
        ws = new_workspace(g["q"], g["v"], cu_t)
        o, st = chunk_efla_fwd(qq, kk, vv, g["beta"], s0, True, cu_t, workspace=ws,
                               save_states=reuse)
        out = chunk_efla_bwd(qq, kk, vv, g["beta"], g["do"], s0, dst, cu_t, workspace=ws,
                             reuse_forward=reuse, reuse_states=reuse, grads_out=grads_out)
        torch.cuda.synchronize()
        return [o.clone(), st.clone()] + [t.clone() for t in out]

    ref = run(g["q"], g["k"], g["v"], None)
    got = run(q, k, v, tuple(gviews))
    for a, b, n in zip(got, ref, ("o", "S_T", "dq", "dk", "dv", "dbeta", "dS0")):
        assert torch.equal(a, b), n
    for a, b in zip(gviews, ref[2:5]):
        assert torch.equal(a, b)
    assert torch.isnan(gbuf[:, -24:]).all()  # nothing written outside the slices
    assert all(torch.isfinite(t).all() for t in ref)


def test_token_stride_rejects_other_layouts():
    from ceo_amd.efla import token_stride

    x = torch.zeros(2, 5, 3, 64, device="cuda:0", dtype=torch.bfloat16)
    assert token_stride(x) == 192
    assert token_stride(torch.zeros(2, 5, 400, device="cuda:0")[:, :, :192]
                        .view(2, 5, 3, 64)) == 400
    with pytest.raises(ValueError):
        token_stride(x.transpose(1, 2))  # heads outside the token row
    with pytest.raises(ValueError):
        token_stride(torch.zeros(3, 5, 3, 64, device="cuda:0")[::2])  # a gap between batches
