"""Parity at the benchmark configurations' full workloads (BASELINE.json
configs 2-5; config 1 runs at its exact shape in test_efla_q_gpu.py).

Each EFLA case runs the library on the workload's full shape, on inputs drawn
with the distributions the configs name (the oracle's seeded generator, bf16
rounded), and compares with the fp64 sequential oracle (oracle/efla_q_body.h,
the recurrence of kernels/cuda/efla.cu:154-233 with the BPTT of
efla.cu:315-454 generalised to a query readout and per-token beta).
Tolerance: rel-L2 <= 2e-2 for bf16 inputs with fp32 accumulation
(BASELINE.json north_star).

Config 3 goes through the path bench.py times: one backward-sized workspace,
a forward that saves T, b, the chunk states and P, and a backward that reuses
all of them; the gradients are then compared bit for bit with the backward
that recomputes the states (north_star's design) on the same inputs.
"""
import math
import os
import sys

import numpy as np
import pytest
import torch

from helpers import announce, rel_l2, to_dev

pytestmark = pytest.mark.gpu

TOL = 2e-2
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _inputs(oracle, seed, B, T, H, K, V):
    x = oracle.make_efla_inputs(seed, B * T, H, K, V, bf16=True)
    g = {n: to_dev(a, torch.bfloat16, (B, T, H, K) if n in "qk" else
                   (B, T, H) if n == "beta" else (B, T, H, V)) for n, a in x.items()}
    return x, g


def _check(errs):
    print("  rel-L2:", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    bad = {k: v for k, v in errs.items() if not v <= TOL}
    assert not bad, bad


def test_cfg3_bench_path(oracle):
    """B=4, T=8192, H=32, d=128, bf16 fwd+bwd, bench.py's path."""
    from ceo_amd import efla

    B, T, H, K, V = 4, 8192, 32, 128, 128
    announce(f"cfg3 bench path B={B} T={T} H={H} K={K} V={V} bf16")
    x, g = _inputs(oracle, 0xEF1A0002, B, T, H, K, V)
    ws = efla.new_workspace(g["q"], g["v"])
    o, _ = efla.chunk_efla_fwd(g["q"], g["k"], g["v"], g["beta"], workspace=ws,
                               save_states=True)
    dq, dk, dv, db, _ = efla.chunk_efla_bwd(g["q"], g["k"], g["v"], g["beta"], g["do"],
                                            workspace=ws, reuse_forward=True,
                                            reuse_states=True)
    # the recompute path (states rebuilt in the backward), same inputs
    r = efla.chunk_efla_bwd(g["q"], g["k"], g["v"], g["beta"], g["do"])
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv", "dbeta"), (dq, dk, dv, db), r[:4]):
        assert torch.equal(a, b), f"{name}: reuse and recompute paths differ"
    ro, _ = oracle.q_forward(x["q"], x["k"], x["v"], x["beta"], T=T)
    errs = {"o": rel_l2(o, ro)}
    del ro
    rg = oracle.q_backward(x["q"], x["k"], x["v"], x["beta"], x["do"], T=T)
    errs.update(dq=rel_l2(dq, rg[0]), dk=rel_l2(dk, rg[1]), dv=rel_l2(dv, rg[2]),
                dbeta=rel_l2(db, rg[3]))
    _check(errs)


def test_cfg2_forward(oracle):
    """B=8, T=2048, H=16, d=128, bf16 forward from a zero state."""
    from ceo_amd import efla

    B, T, H, K, V = 8, 2048, 16, 128, 128
    announce(f"cfg2 forward B={B} T={T} H={H} K={K} V={V} bf16")
    x, g = _inputs(oracle, 0xEF1A0001, B, T, H, K, V)
    o, st = efla.chunk_efla_fwd(g["q"], g["k"], g["v"], g["beta"], output_final_state=True)
    torch.cuda.synchronize()
    ro, rst = oracle.q_forward(x["q"], x["k"], x["v"], x["beta"], T=T)
    _check({"o": rel_l2(o, ro), "S_T": rel_l2(st, rst)})


def test_cfg5_varlen(oracle):
    """65,536 packed tokens, log-uniform lengths in [64, 8192]
    (bench.py's draw), H=16, d_k=128, d_v=256, state reset per sequence."""
    sys.path.insert(0, ROOT)
    import bench
    from ceo_amd import efla

    total, H, K, V = 65536, 16, 128, 256
    lens = bench.varlen_lengths(total, 0xEF1A0002)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    assert cu[-1] == total
    announce(f"cfg5 varlen {len(lens)} sequences, {total} tokens, H={H} K={K} V={V} bf16")
    x, g = _inputs(oracle, 0xEF1A0004, 1, total, H, K, V)
    cu_t = torch.from_numpy(cu).to("cuda:0")
    ws = efla.new_workspace(g["q"], g["v"], cu_t)
    o, st = efla.chunk_efla_fwd(g["q"], g["k"], g["v"], g["beta"], output_final_state=True,
                                cu_seqlens=cu_t, workspace=ws, save_states=True)
    dq, dk, dv, db, _ = efla.chunk_efla_bwd(g["q"], g["k"], g["v"], g["beta"], g["do"],
                                            cu_seqlens=cu_t, workspace=ws,
                                            reuse_forward=True, reuse_states=True)
    torch.cuda.synchronize()
    ro, rst = oracle.q_forward(x["q"], x["k"], x["v"], x["beta"], cu_seqlens=cu)
    errs = {"o": rel_l2(o, ro), "S_T": rel_l2(st, rst)}
    del ro, rst
    rg = oracle.q_backward(x["q"], x["k"], x["v"], x["beta"], x["do"], cu_seqlens=cu)
    errs.update(dq=rel_l2(dq, rg[0]), dk=rel_l2(dk, rg[1]), dv=rel_l2(dv, rg[2]),
                dbeta=rel_l2(db, rg[3]))
    _check(errs)


# ---------------------------------------------------------------------------
# config 4: the full 24-layer model
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def lm4():
    from ceo_amd.lm_step import EflaLM, LMConfig, synthetic_batch

    cfg = LMConfig()
    model = EflaLM(cfg, device="cuda:0", seed=7)
    tokens, targets = synthetic_batch(cfg, 8, 2048, seed=8, device="cuda:0")
    return cfg, model, tokens, targets


def test_cfg4_layer_efla_vs_oracle(oracle, lm4):
    """One layer of the config-4 forward: its EFLA inputs as the model forms
    them (column slices of the fused projection rows, beta from the gate),
    its output and, through the same workspace, the gradients for a random
    dO, against the fp64 oracle."""
    from ceo_amd import efla

    cfg, model, tokens, targets = lm4
    announce("cfg4 layer-12 EFLA inputs vs oracle (B=8 T=2048 H=16 d=64)")
    with torch.no_grad():
        _, saved = model.forward(tokens, targets)
    s = saved["layers"][12]
    B, T, H, dh = 8, 2048, cfg.n_heads, cfg.head_dim
    ws = model._workspaces(B, T)[12]
    host = {n: s[n].float().cpu().numpy().reshape(B * T, H, -1) for n in ("q", "k", "v")}
    host["beta"] = s["beta"].float().cpu().numpy().reshape(B * T, H)
    rng = np.random.default_rng(12)
    do = oracle.round_bf16(rng.standard_normal((B * T, H, dh)))
    do_t = torch.from_numpy(do).to("cuda:0").to(torch.bfloat16).view(B, T, H, dh)
    dq, dk, dv, db, _ = efla.chunk_efla_bwd(s["q"], s["k"], s["v"], s["beta"], do_t,
                                            workspace=ws, reuse_forward=True,
                                            reuse_states=True)
    torch.cuda.synchronize()
    ro, _ = oracle.q_forward(host["q"], host["k"], host["v"], host["beta"], T=T)
    rg = oracle.q_backward(host["q"], host["k"], host["v"], host["beta"], do, T=T)
    _check({"o": rel_l2(s["o"], ro), "dq": rel_l2(dq, rg[0]), "dk": rel_l2(dk, rg[1]),
            "dv": rel_l2(dv, rg[2]), "dbeta": rel_l2(db, rg[3])})


def test_cfg4_lm_head_gemm_fp64(lm4):
    """The full-size LM-head products (16384 x 1024 x 32000) against fp64 on
    sampled rows / columns: the forward, and the backward's dA and dB."""
    from ceo_amd import nn

    cfg, model, tokens, targets = lm4
    announce("cfg4 LM head GEMM 16384 x 1024 x 32000 vs fp64 (sampled)")
    g = torch.Generator(device="cuda:0").manual_seed(3)
    M, Kd, N = 16384, cfg.d_model, cfg.vocab
    a = torch.randn(M, Kd, generator=g, device="cuda:0").to(torch.bfloat16)
    w = model.w("head")
    c = nn.gemm_forward(a, w)
    dc = (torch.randn(M, N, generator=g, device="cuda:0") * 0.01).to(torch.bfloat16)
    da, dw, _ = nn.gemm_backward(dc, a, w)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(1).choice(M, 192, replace=False))
    cols = np.sort(np.random.default_rng(2).choice(N, 96, replace=False))
    a64 = a.double().cpu().numpy()
    w64 = w.double().cpu().numpy()
    dc64 = dc.double().cpu().numpy()
    errs = {
        "C rows": rel_l2(c[rows], a64[rows] @ w64),
        "dA rows": rel_l2(da[rows], dc64[rows] @ w64.T),
        "dB cols": rel_l2(dw[:, cols], a64.T @ dc64[:, cols]),
    }
    print("  rel-L2:", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    # bf16 outputs of fp32-accumulated products: rounding alone is ~2e-3
    assert all(v <= 1e-2 for v in errs.values()), errs


def test_cfg4_training_steps(lm4):
    """Three AdamW steps of the full model on one batch: the loss starts near
    log(vocab), stays finite and falls."""
    cfg, model, tokens, targets = lm4
    announce("cfg4 full 24-layer model, 3 training steps")
    losses = []
    for _ in range(3):
        losses.append(model.train_step(tokens, targets).item())
        print(f"  loss {losses[-1]:.5f}", flush=True)
    assert all(math.isfinite(v) for v in losses), losses
    assert abs(losses[0] - math.log(cfg.vocab)) < 0.5, losses
    assert losses[2] < losses[1] < losses[0], losses
    assert torch.isfinite(model.master).all()
