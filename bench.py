"""EFLA fwd+bwd throughput on one MI355X (the headline benchmark).

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--config cfg3|cfg1|cfg2|cfg4|cfg5] [--no-cpu] [--cpu-budget SECONDS]
                    [--aux] [--no-recompute]

A step is one chunked EFLA forward plus one backward over one batch of
synthetic inputs already resident in HBM.  As the library's autograd function
runs it, the forward writes its per-chunk factors (T, b), chunk start states
and P = tril(Q K^T) into a caller workspace and the backward reuses them, so
the backward runs no forward recompute.  The design north_star names (the
backward recomputes the chunk states instead of storing them) is timed in a
second pass and reported as ``recompute``.  Default workload: configs[2] of
the benchmark definition, B=4, T=8192, H=32, d_k=d_v=128, chunk 64, bf16
storage with fp32 accumulation.

Timing: W untimed steps, then K timed steps between torch.cuda.synchronize()
calls, with a hipEvent pair per step on the launch stream; ``ms_per_step`` is
the median step (by default the median of 50 timed steps after 10 warm-up
steps), ``mean_ms_per_step`` the mean.  The per-kernel split
comes from a separate pass of K steps with the library's launch profiler
(an event pair around each launch, which would inflate the timed steps).

Prints ONE JSON line with the metric, the per-kernel split, the roofline of
the dominant kernel and of the step, and a CPU baseline: the scalar fp32
restatement of the same recurrence (oracle/, OpenMP over (sequence, head))
timed on a bounded sample of the same workload on this host.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

C = 64  # chunk length
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_FP32_TFLOPS = 157.3  # MI355X dense fp32 MFMA
PEAK_HBM_GBS = 8000.0

CONFIGS = {
    # name: (B, T, H, K, V, dtype, fwd+bwd?, varlen?)
    "cfg3": dict(B=4, T=8192, H=32, K=128, V=128, dtype="bf16", bwd=True, varlen=False),
    "cfg1": dict(B=2, T=256, H=4, K=64, V=64, dtype="fp32", bwd=True, varlen=False),
    "cfg2": dict(B=8, T=2048, H=16, K=128, V=128, dtype="bf16", bwd=False, varlen=False),
    "cfg5": dict(B=1, T=65536, H=16, K=128, V=256, dtype="bf16", bwd=True, varlen=True),
}


# ---------------------------------------------------------------------------
# FLOP model (algorithmic; recompute is not counted)
# ---------------------------------------------------------------------------
def f_fwd_per_token_head(K: int, V: int, c: int = C) -> float:
    """C(6K + 4V) + 6KV + (2/3)C^2 per (token, head): per chunk the products
    KK^T, W = T(bK), U = T(bV), QK^T (2C^2K each but U, 2C^2V), P Vn (2C^2V),
    WS, QS, K^T Vn (2CKV each) and the UT solve (2/3)C^3."""
    return c * (6 * K + 4 * V) + 6 * K * V + (2.0 / 3.0) * c * c


def kernel_flops_per_chunk(K: int, V: int, c: int = C) -> dict:
    """Algorithmic FLOPs of each library kernel per (chunk, head), assigned so
    that the forward kernels sum to F_fwd and the backward ones to 2 F_fwd
    (the backward's re-run of prep and of the state scan is recompute: 0)."""
    c2, c3, ckv = c * c, c ** 3, c * K * V
    return {
        # forward: WY prep (K K^T, UT solve, W, U) and the fused scan + output
        # (W S, K^T Vn, Q S, Q K^T, P Vn)
        "efla_q_fwd_prep": 4 * c2 * K + 2 * c2 * V + (2.0 / 3.0) * c3,
        "efla_q_fwd_scan": 6 * ckv + 2 * c2 * K + 2 * c2 * V,
        # backward: reverse scan (K dS, Q^T dO, W^T dVn, P^T dO) and the
        # per-chunk gradients (the rest of 2 F_fwd)
        "efla_q_bwd_re_prep": 0.0,
        "efla_q_bwd_re_state": 0.0,
        "efla_q_bwd_state": 6 * ckv + 2 * c2 * V,
        "efla_q_bwd_grad": 12 * c2 * K + 6 * c2 * V + 6 * ckv + (4.0 / 3.0) * c3,
        # fp32 path (generic kernels)
        "efla_q_fwd_state": 4 * ckv,
        "efla_q_fwd_o": 2 * c2 * K + 2 * c2 * V + 2 * ckv,
        "efla_q_bwd_dvloc": 2 * c2 * K + 2 * c2 * V,
        "efla_q_bwd_dqkw": 4 * c2 * K + 2 * c2 * V + 6 * ckv,
        "efla_q_bwd_wy": 6 * c2 * K + 4 * c2 * V + 4 * c3,
    }


def io_bytes(ntok: int, H: int, K: int, V: int, bwd: bool, esize: int = 2) -> float:
    """Algorithmic HBM bytes: fwd reads q, k, v, beta and writes o; bwd reads
    q, k, v, beta, dO and writes dq, dk, dv, dbeta."""
    per_tok = H * (2 * K + 2 * V + 1) * esize  # fwd: q k (K each) v o (V each) beta
    if bwd:
        per_tok += H * (2 * K + V + 1 + V + 2 * K + V + 1) * esize
    return float(ntok) * per_tok


def kernel_io_bytes_per_token_head(K: int, V: int, esize: int = 2) -> dict:
    """The op's own I/O bytes each kernel accounts for, per (token, head):
    what it reads of the op's inputs and writes of its outputs.  Intermediates
    (T, b, chunk states, P) are not algorithmic bytes; the gradient kernel is
    charged the whole backward I/O (q, k, v, dO, beta in; dq, dk, dv, dbeta
    out), the forward scan the forward's (q, k, v in, o out)."""
    return {
        "efla_q_fwd_prep": (K + 1) * esize,
        "efla_q_fwd_scan": (2 * K + 2 * V) * esize,
        "efla_q_bwd_state": (2 * K + V) * esize,
        "efla_q_bwd_grad": (4 * K + 4 * V + 2) * esize,
    }


# ---------------------------------------------------------------------------
# inputs
# ---------------------------------------------------------------------------
def varlen_lengths(total: int, seed: int):
    """Log-uniform lengths in [64, 8192], the last one truncated to fill `total`."""
    import numpy as np

    rng = np.random.default_rng(seed)
    lens = []
    while sum(lens) < total:
        lens.append(int(math.floor(math.exp(rng.uniform(math.log(64), math.log(8192))))))
    lens[-1] -= sum(lens) - total
    return [x for x in lens if x > 0]


def make_inputs(cfg: dict, seed: int, device):
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    B, T, H, K, V = cfg["B"], cfg["T"], cfg["H"], cfg["K"], cfg["V"]
    dt = torch.bfloat16 if cfg["dtype"] == "bf16" else torch.float32

    def randn(*shape):
        return torch.randn(*shape, generator=g, device=device, dtype=torch.float32)

    q = randn(B, T, H, K)
    k = randn(B, T, H, K)
    k = k / k.norm(dim=-1, keepdim=True)
    v = randn(B, T, H, V)
    beta = torch.sigmoid(randn(B, T, H))
    do = randn(B, T, H, V)
    out = {n: t.to(dt).contiguous() for n, t in
           (("q", q), ("k", k), ("v", v), ("beta", beta), ("do", do))}
    out["cu"] = None
    if cfg["varlen"]:
        lens = varlen_lengths(B * T, seed)
        cu = [0]
        for x in lens:
            cu.append(cu[-1] + x)
        out["cu"] = torch.tensor(cu, dtype=torch.int32, device=device)
    return out


# ---------------------------------------------------------------------------
# CPU baseline
# ---------------------------------------------------------------------------
def cpu_baseline(cfg: dict, seed: int, budget_s: float) -> dict:
    """Scalar fp32 restatement of the same recurrence (oracle/efla_q_body.h),
    OpenMP over (sequence, head), on whole sequences of the workload's shape
    until `budget_s` is spent (at least one).  Scaled to the metric's unit:
    workload tokens (all H heads) per second."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle  # the checker / baseline only; never on the measured GPU path

    oracle.lib()
    T, H, K, V = cfg["T"], cfg["H"], cfg["K"], cfg["V"]
    if cfg["varlen"]:
        T = 8192  # the longest sequence length the varlen draw allows
    n_seq = cfg["B"] if not cfg["varlen"] else max(1, cfg["B"] * cfg["T"] // T)
    inputs = {}
    done, elapsed = 0, 0.0
    # whole sequences, cycling through the workload's n_seq inputs, until the
    # budget is spent (at least one sequence)
    while True:
        s = done % n_seq
        if s not in inputs:
            inputs[s] = oracle.make_efla_inputs(seed + s, T, H, K, V,
                                                bf16=cfg["dtype"] == "bf16",
                                                with_do=cfg["bwd"])
        x = inputs[s]
        t0 = time.perf_counter()
        oracle.q_forward(x["q"], x["k"], x["v"], x["beta"], T=T, dtype=np.float32)
        if cfg["bwd"]:
            oracle.q_backward(x["q"], x["k"], x["v"], x["beta"], x["do"], T=T,
                              dtype=np.float32)
        elapsed += time.perf_counter() - t0
        done += 1
        print(f"[bench] cpu baseline: sequence {done} ({elapsed:.1f} s)",
              file=sys.stderr, flush=True)
        if elapsed >= budget_s:
            break
    cores = oracle.num_threads()
    # one thread on a slice of the heads of the first sequence (the recurrence
    # is independent per head), scaled to whole-sequence tokens per second
    x = inputs[0]
    heads = 0
    t1 = 0.0
    oracle.set_num_threads(1)
    try:
        while heads < H and t1 < min(5.0, budget_s / 3):
            hs = slice(heads, heads + 1)
            part = {n: np.ascontiguousarray(a[:, hs]) for n, a in x.items()}
            t0 = time.perf_counter()
            oracle.q_forward(part["q"], part["k"], part["v"], part["beta"], T=T,
                             dtype=np.float32)
            if cfg["bwd"]:
                oracle.q_backward(part["q"], part["k"], part["v"], part["beta"], part["do"],
                                  T=T, dtype=np.float32)
            t1 += time.perf_counter() - t0
            heads += 1
    finally:
        oracle.set_num_threads(cores)
    return {
        "value": done * T / elapsed,
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{done} sequences (cycling the workload's {n_seq}) of T={T}, H={H}, "
                  f"d_k={K}, d_v={V} "
                  f"({'fwd+bwd' if cfg['bwd'] else 'fwd'}, fp32 math on "
                  f"{'bf16-rounded ' if cfg['dtype'] == 'bf16' else ''}inputs), "
                  f"{elapsed:.2f} s",
        "single_thread": {
            "value": T * heads / H / t1,
            "unit": "tokens/s",
            "cores": 1,
            "sample": f"{heads} of the {H} heads of one T={T} sequence, one thread, "
                      f"{t1:.2f} s, scaled by heads / {H}",
        },
    }


# ---------------------------------------------------------------------------
# HBM traffic of the dominant kernel (from committed rocprofv3 counter runs)
# ---------------------------------------------------------------------------
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def copy_calibration(mib: int) -> int:
    """A plain copy of known size: FETCH_SIZE and WRITE_SIZE of its kernel
    divided into the true byte count give the counters' scale factors."""
    import torch

    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": n}), flush=True)
    return 0


def measured_traffic(config: str, kernel: str):
    """HBM bytes per launch of `kernel` recorded in profiles/traffic.json by the
    FETCH_SIZE / WRITE_SIZE runs (already scaled by the copy calibration), or
    None when that file does not cover this kernel and workload."""
    try:
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f)
        k = rec[config]["kernels"][kernel]
        return float(k["fetch_bytes"]) + float(k["write_bytes"])
    except (OSError, KeyError, ValueError, TypeError):
        return None


# ---------------------------------------------------------------------------
# HBM-bound kernels of the config-4 step (LayerNorm, GELU, AdamW)
# ---------------------------------------------------------------------------
CFG4 = {"tokens": 16384, "d_model": 1024, "mlp": 4096, "params": 368_000_000}


def aux_bench(steps: int, warmup: int, ops_only: int = 0) -> int:
    """Times the kernels around EFLA at config-4 shapes: the GEMMs of one layer
    and the LM head against the bf16 MFMA roof (their FLOPs over the average
    hipEvent duration), LayerNorm / GELU / AdamW and the reference model's
    RMSNorm / ShortConv / PRISM against the HBM roof (algorithmic bytes per
    launch: what each must read and write once).
    With ``ops_only`` = N it instead runs each HBM-bound op N times, untimed
    (the program that rocprofv3 FETCH_SIZE / WRITE_SIZE passes profile).
    Prints one JSON line."""
    import torch

    from ceo_amd import nn, prism, runtime

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(4)
    N, D, F, P = CFG4["tokens"], CFG4["d_model"], CFG4["mlp"], CFG4["params"]

    def bf(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g, device=dev) * scale).to(torch.bfloat16)

    x, w, b, dy = bf(N, D), bf(D), bf(D, scale=0.1), bf(N, D)
    h, dh = bf(N, F), bf(N, F)
    p32 = torch.randn(P, generator=g, device=dev)
    m32 = torch.zeros(P, device=dev)
    v32 = torch.zeros(P, device=dev)
    gp = bf(P, scale=0.01)
    pcopy = torch.empty(P, dtype=torch.bfloat16, device=dev)
    y, mean, rstd = nn.layernorm_forward(x, w, b, save_stats=True)
    # the reference model's RMSNorm, ShortConv (window 64, configs/train.yaml)
    # and 3-iteration PRISM refinement on the same activations, as (8, 2048, 1024)
    rms_dw = torch.zeros(D, device=dev)
    x3, dy3 = x.view(8, N // 8, D), dy.view(8, N // 8, D)
    conv_w = bf(D, 64, scale=0.125)
    conv_dw = torch.zeros(D, 64, device=dev)
    w_p = [bf(D, 64, scale=0.04) for _ in range(3)]
    gw_p = [torch.zeros(D * 64, device=dev) for _ in range(3)]
    cases = {
        # name: (callable, algorithmic bytes per launch, what)
        "layernorm_fwd": (lambda: nn.layernorm_forward(x, w, b, save_stats=True),
                          N * D * 4 + N * 8, "x in, y out (bf16), mean/rstd out"),
        "layernorm_bwd": (lambda: nn.layernorm_backward(dy, x, w, mean, rstd),
                          N * D * 6 + N * 8, "dy, x in, dx out (bf16), mean/rstd in"),
        "gelu_fwd": (lambda: nn.gelu_forward(h), N * F * 4, "x in, y out (bf16)"),
        "gelu_bwd": (lambda: nn.gelu_backward(dh, h), N * F * 6, "dy, x in, dx out (bf16)"),
        "adamw_master": (lambda: nn.adamw_step_master(p32, gp, m32, v32, 3e-4, 0.9, 0.999,
                                                      1e-8, 0.1, 1, param_bf16=pcopy),
                         P * 28, "p, m, v fp32 in+out, g bf16 in, bf16 copy out"),
        "rmsnorm_fwd": (lambda: nn.rmsnorm_forward(x, w, 1e-6), N * D * 4,
                        "x in, y out (bf16)"),
        "rmsnorm_bwd": (lambda: nn.rmsnorm_backward(dy, x, w, 1e-6, grad_weight=rms_dw),
                        N * D * 6, "dy, x in, dx out (bf16)"),
        "shortconv_fwd_w64": (lambda: prism.shortconv_forward(x3, conv_w), N * D * 4,
                              "x in, y out (bf16); 64 taps per output"),
        "shortconv_bwd_w64": (lambda: prism.shortconv_backward(dy3, x3, conv_w,
                                                               grad_weight=conv_dw),
                              N * D * 6, "dy, x in, dx out (bf16), dW partials"),
        "prism_fwd_l3": (lambda: prism.prism_forward(x3, dy3, w_p, 64), N * 64 * 4 + N * D * 2,
                         "u, v in over head_dim 64, output rows out (bf16)"),
        "prism_bwd_l3": (lambda: prism.prism_backward(dy3, x3, dy3, w_p, 64, gw_p),
                         N * 64 * 6 + N * D * 4, "g, u, v in over head_dim 64, du, dv rows out"),
    }
    if ops_only:
        for name, (fn, nbytes, _) in cases.items():
            for _ in range(ops_only):
                fn()
            torch.cuda.synchronize()
        print(json.dumps({"aux_ops": {k: v[1] for k, v in cases.items()},
                          "launches_each": ops_only}), flush=True)
        return 0
    # GEMMs of one config-4 layer and the LM head (MFMA-bound: FLOPs, not bytes)
    wq, wu, wd, wh = bf(D, 3 * D, scale=0.03), bf(D, F, scale=0.03), bf(F, D, scale=0.02), \
        bf(D, 32000, scale=0.03)
    xu = bf(N, F)
    dcu = bf(N, F)
    gemms = {
        "gemm_qkv_fwd": (lambda: nn.gemm_forward(x, wq), 2.0 * N * D * 3 * D),
        "gemm_up_fwd": (lambda: nn.gemm_forward(x, wu), 2.0 * N * D * F),
        "gemm_down_fwd": (lambda: nn.gemm_forward(xu, wd), 2.0 * N * F * D),
        "gemm_lm_head_fwd": (lambda: nn.gemm_forward(x, wh), 2.0 * N * D * 32000),
        "gemm_up_bwd": (lambda: nn.gemm_backward(dcu, x, wu, need_bias=False), 4.0 * N * D * F),
    }
    out = {}
    stream = torch.cuda.current_stream(dev)

    def run(fn, n_warm, n, graph=True):
        """Average ms per call over n back-to-back calls between one event pair.
        With ``graph`` the n calls are captured in one HIP graph on a side
        stream (warmed first, so its cached workspace exists before capture)
        and the graph is replayed between the events: the Python wrappers cost
        several microseconds of host time per call, which would otherwise show
        up as GPU idle time between the short HBM-bound kernels.  Then the
        per-kernel split from an eager profiled pass."""
        for _ in range(n_warm):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        avg, mode = None, "eager"
        if graph:
            try:
                cs = torch.cuda.Stream()
                cs.wait_stream(stream)
                with torch.cuda.stream(cs):
                    for _ in range(2):
                        fn()
                torch.cuda.synchronize()
                gr = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gr, stream=cs):
                    for _ in range(n):
                        fn()
                gr.replay()
                torch.cuda.synchronize()
                e0.record(stream)
                gr.replay()
                e1.record(stream)
                torch.cuda.synchronize()
                avg, mode = e0.elapsed_time(e1) / n, "graph"
                del gr
            except Exception as exc:  # capture refused: time the eager calls
                print(f"[bench] graph capture failed ({exc}); eager timing", file=sys.stderr,
                      flush=True)
                torch.cuda.synchronize()
        if avg is None:
            e0.record(stream)
            for _ in range(n):
                fn()
            e1.record(stream)
            torch.cuda.synchronize()
            avg = e0.elapsed_time(e1) / n
        with runtime.Profiler() as prof:
            for _ in range(n):
                fn()
        res = prof.results()
        return avg, {k: round(tot / cnt, 4) for k, (cnt, tot) in res.items()}, mode

    for name, (fn, flops) in gemms.items():
        avg_ms, kms, mode = run(fn, warmup, steps)
        tf = flops / (avg_ms * 1e-3) / 1e12
        out[name] = {"avg_ms": round(avg_ms, 4), "flops": flops, "TFLOP/s": round(tf, 1),
                     "frac_of_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4),
                     "timing": mode, "kernels_ms": kms}
        print(f"[bench] {name}: {avg_ms:.4f} ms, {tf:.0f} TFLOP/s", file=sys.stderr, flush=True)
    del xu, dcu
    # the practical HBM ceiling for a read + write stream: a device copy of
    # 1 GiB (too large for the 256 MB MALL to hold across calls)
    csrc = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
    cdst = torch.empty_like(csrc)
    c_ms, _, c_mode = run(lambda: cdst.copy_(csrc), 2, 10)
    copy_gbs = 2 * csrc.numel() * 4 / (c_ms * 1e-3) / 1e9
    out["copy_1GiB_ceiling"] = {"avg_ms": round(c_ms, 4), "bytes": 2 * csrc.numel() * 4,
                                "bytes_are": "1 GiB fp32 in, 1 GiB out (torch copy_)",
                                "GB/s": round(copy_gbs, 1),
                                "frac_of_hbm_peak": round(copy_gbs / PEAK_HBM_GBS, 4),
                                "timing": c_mode}
    print(f"[bench] copy_1GiB_ceiling: {c_ms:.4f} ms, {copy_gbs:.0f} GB/s", file=sys.stderr,
          flush=True)
    del csrc, cdst
    for name, (fn, nbytes, what) in cases.items():
        # the op's time: every kernel it launched (LayerNorm's backward has a
        # second, small reduction kernel), averaged over the timed calls
        avg_ms, kms, mode = run(fn, warmup, steps)
        gbs = nbytes / (avg_ms * 1e-3) / 1e9
        out[name] = {"avg_ms": round(avg_ms, 4), "bytes": nbytes, "bytes_are": what,
                     "GB/s": round(gbs, 1), "frac_of_hbm_peak": round(gbs / PEAK_HBM_GBS, 4),
                     "frac_of_copy_ceiling": round(gbs / copy_gbs, 4) if copy_gbs else None,
                     "timing": mode, "kernels_ms": kms}
        print(f"[bench] {name}: {avg_ms:.4f} ms, {gbs:.0f} GB/s", file=sys.stderr, flush=True)
    del cases, x, dy, h, dh, p32, m32, v32, gp, pcopy
    # the reference ABI's entries (efla_forward_hip / efla_backward_hip, Mode R:
    # scalar beta, key readout, bf16 state rounded per token) at cfg3's shape
    from ceo_amd import efla

    B, T, H, d = 4, 8192, 32, 128
    kr = torch.randn(B, T, H, d, generator=g, device=dev)
    kr = (kr / kr.norm(dim=-1, keepdim=True)).to(torch.bfloat16)
    vr, dor = bf(B, T, H, d), bf(B, T, H, d)
    s0 = torch.zeros(B * H, d, d, dtype=torch.bfloat16, device=dev)
    state = s0.clone()
    mode_r = {
        "efla_forward_hip_cfg3": lambda: efla.efla_forward(kr, vr, state.copy_(s0), 0.5, 64),
        "efla_backward_hip_cfg3": lambda: efla.efla_backward(dor, kr, vr, s0, 0.5),
    }
    for name, fn in mode_r.items():
        avg_ms, kms, _ = run(fn, 1, 3, graph=False)
        out[name] = {"avg_ms": round(avg_ms, 3), "tokens_per_s": round(B * T / (avg_ms * 1e-3), 1),
                     "shape": f"B={B} T={T} H={H} d={d} bf16", "kernels_ms": kms}
        print(f"[bench] {name}: {avg_ms:.3f} ms", file=sys.stderr, flush=True)
    print(json.dumps({"aux": "config-4 kernels around EFLA, and the reference-ABI EFLA "
                             "entries at cfg3's shape", "shapes": CFG4, "steps": steps,
                      "kernels": out}), flush=True)
    return 0


# ---------------------------------------------------------------------------
# config 4: the full training step of the decoder LM
# ---------------------------------------------------------------------------
def lm_bench(steps: int, warmup: int, seed: int) -> int:
    """Times forwardStep + backwardStep + updateStep of the config-4 model
    (random init, synthetic uniform token ids, batch 8 x 2048).  Prints one
    JSON line: tokens/s and model FLOP utilisation, with the per-kernel split."""
    import torch

    from ceo_amd import runtime
    from ceo_amd.lm_step import EflaLM, LMConfig, step_flops, synthetic_batch

    dev = torch.device("cuda:0")
    cfg = LMConfig()
    B, T = 8, 2048
    model = EflaLM(cfg, device=dev, seed=seed)
    tokens, targets = synthetic_batch(cfg, B, T, seed=seed + 1, device=dev)
    print(f"[bench] cfg4: {model.n_params / 1e6:.1f} M parameters, batch {B} x {T}",
          file=sys.stderr, flush=True)
    losses = []
    for _ in range(warmup):
        losses.append(model.train_step(tokens, targets))
    torch.cuda.synchronize()
    print("[bench] warmup done", file=sys.stderr, flush=True)
    stream = torch.cuda.current_stream(dev)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # the timed steps run without the per-launch profiler (an event pair around
    # each of the step's ~600 launches would be counted in the step time); a
    # second, profiled pass of the same length gives the per-kernel split
    ev0.record(stream)
    for _ in range(steps):
        losses.append(model.train_step(tokens, targets))
    ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    prof = runtime.Profiler()
    pe0, pe1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with prof:
        pe0.record(stream)
        for _ in range(steps):
            losses.append(model.train_step(tokens, targets))
        pe1.record(stream)
    torch.cuda.synchronize()
    profiled_ms = pe0.elapsed_time(pe1) / steps
    kern = prof.results()
    lib_ms = sum(tot for _, tot in kern.values()) / steps
    groups = {}
    for name, (n, tot) in kern.items():
        key = ("gemm" if name.startswith("gemm") else "efla" if name.startswith("efla")
               else name.split("_")[0])
        groups[key] = groups.get(key, 0.0) + tot / steps
    flops = step_flops(cfg, B * T, T)
    line = {
        "metric": "config-4 training step tokens/s (fwd + bwd + AdamW)",
        "value": round(B * T / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (uniform token ids, random init)",
        "config": {"workload": "cfg4: d_model 1024, 24 layers, 16 EFLA heads x 64, MLP 4096, "
                               "vocab 32000, batch 8 x 2048, fp32 master + AdamW",
                   "params": model.n_params, "tokens_per_step": B * T},
        "model_tflops": round(flops / (ms * 1e-3) / 1e12, 1),
        "mfu_bf16": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "library_kernel_ms": round(lib_ms, 3),
        "profiled_pass_ms_per_step": round(profiled_ms, 3),
        "kernel_ms_by_group": {k: round(v, 3) for k, v in sorted(groups.items(),
                                                                 key=lambda kv: -kv[1])},
        "kernels": {k: {"launches_per_step": n / steps, "ms_per_step": round(tot / steps, 3)}
                    for k, (n, tot) in sorted(kern.items(), key=lambda kv: -kv[1][1])},
        "loss_first_last": [round(losses[0].item(), 4), round(losses[-1].item(), 4)],
    }
    print(json.dumps(line), flush=True)
    return 0


# ---------------------------------------------------------------------------
# main
# ---------------------------------------------------------------------------
def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="cfg3", choices=sorted(CONFIGS) + ["cfg4"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-recompute", action="store_true",
                    help="skip the pass timing the recompute variant")
    ap.add_argument("--no-ref-abi", action="store_true",
                    help="skip timing the reference ABI's efla_forward_hip / efla_backward_hip "
                         "(cfg3 only)")
    ap.add_argument("--cpu-budget", type=float, default=15.0,
                    help="seconds of CPU-baseline work (whole sequences, at least one)")
    ap.add_argument("--seed", type=int, default=0xEF1A0002)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB five times "
                         "(the known-size kernel that calibrates rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE readings) and exit")
    ap.add_argument("--aux-ops", type=int, default=0, metavar="N",
                    help="only run each --aux HBM-bound op N times, untimed, and exit "
                         "(for rocprofv3 counter passes)")
    ap.add_argument("--aux", action="store_true",
                    help="only time the config-4 LayerNorm / GELU / AdamW kernels against "
                         "the HBM roof (one JSON line) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    if args.aux_ops:
        return aux_bench(0, 0, ops_only=args.aux_ops)
    if args.aux:
        return aux_bench(args.steps, args.warmup)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the EFLA path here has no multi-GPU mode "
              f"(--gpus {args.gpus}, WORLD_SIZE={world} requested)", file=sys.stderr)
        return 2

    import torch

    from ceo_amd import efla, runtime

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    if args.config == "cfg4":
        return lm_bench(args.steps, args.warmup, args.seed & 0xFFFF)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = CONFIGS[args.config]
    B, T, H, K, V = cfg["B"], cfg["T"], cfg["H"], cfg["K"], cfg["V"]
    ntok = B * T
    x = make_inputs(cfg, args.seed, dev)
    cu = x["cu"]
    print(f"[bench] {args.config}: B={B} T={T} H={H} K={K} V={V} {cfg['dtype']} "
          f"{'fwd+bwd' if cfg['bwd'] else 'fwd'}{' varlen' if cu is not None else ''}",
          file=sys.stderr, flush=True)

    # one workspace for both calls, as the autograd function uses it: the
    # forward leaves its per-chunk factors, chunk start states and P there and
    # the backward reads them instead of recomputing them
    ws = efla.new_workspace(x["q"], x["v"], cu)

    def step():
        o, _ = efla.chunk_efla_fwd(x["q"], x["k"], x["v"], x["beta"], cu_seqlens=cu,
                                   workspace=ws, save_states=cfg["bwd"])
        if cfg["bwd"]:
            efla.chunk_efla_bwd(x["q"], x["k"], x["v"], x["beta"], x["do"], cu_seqlens=cu,
                                workspace=ws, reuse_forward=True, reuse_states=True)
        return o

    def step_recompute():
        # north_star's design: nothing handed over, the backward rebuilds the
        # chunk factors and states (into the library's cached workspace)
        efla.chunk_efla_fwd(x["q"], x["k"], x["v"], x["beta"], cu_seqlens=cu)
        efla.chunk_efla_bwd(x["q"], x["k"], x["v"], x["beta"], x["do"], cu_seqlens=cu)

    def step_recompute_states():
        # the forward hands over its per-chunk factors (T, b and the
        # coefficient derivatives, 5.9 KB per chunk and head) but not the chunk
        # states or P: the backward recomputes the states
        efla.chunk_efla_fwd(x["q"], x["k"], x["v"], x["beta"], cu_seqlens=cu, workspace=ws,
                            save_states=False)
        efla.chunk_efla_bwd(x["q"], x["k"], x["v"], x["beta"], x["do"], cu_seqlens=cu,
                            workspace=ws, reuse_forward=True, reuse_states=False)

    stream = torch.cuda.current_stream(dev)

    def timed(fn, n):
        """Per-step milliseconds from a hipEvent pair per step on the launch
        stream, and the total between the first and the last event."""
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
        torch.cuda.synchronize()
        evs[0].record(stream)
        for i in range(n):
            fn()
            evs[i + 1].record(stream)
        torch.cuda.synchronize()
        per = [evs[i].elapsed_time(evs[i + 1]) for i in range(n)]
        return per, evs[0].elapsed_time(evs[n])

    def median(xs):
        ys = sorted(xs)
        m = len(ys) // 2
        return ys[m] if len(ys) % 2 else 0.5 * (ys[m - 1] + ys[m])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    print(f"[bench] warmup done ({args.warmup} steps)", file=sys.stderr, flush=True)
    per_step, ms_total = timed(step, args.steps)
    ms_step = median(per_step)
    print(f"[bench] timed {args.steps} steps: median {ms_step:.4f} ms/step, "
          f"mean {ms_total / args.steps:.4f}", file=sys.stderr, flush=True)
    # the per-kernel split, from a second pass with the launch profiler
    prof = runtime.Profiler()
    with prof:
        _, prof_total = timed(step, args.steps)
    kern = prof.results()
    print(f"[bench] profiled pass: {prof_total / args.steps:.4f} ms/step", file=sys.stderr,
          flush=True)
    recompute = None
    if cfg["bwd"] and not args.no_recompute:
        for _ in range(args.warmup):
            step_recompute()
        per_re, _ = timed(step_recompute, args.steps)
        recompute = median(per_re)
        print(f"[bench] recompute variant: median {recompute:.4f} ms/step", file=sys.stderr,
              flush=True)
        for _ in range(args.warmup):
            step_recompute_states()
        per_rs, _ = timed(step_recompute_states, args.steps)
        recompute_states = median(per_rs)
        print(f"[bench] states-only recompute: median {recompute_states:.4f} ms/step",
              file=sys.stderr, flush=True)

    ref_abi = None
    if args.config == "cfg3" and not args.no_ref_abi:
        # the reference ABI's own entries on the same k, v, dO: the token-by-token
        # recurrence with the bf16 state re-rounded every token (efla.cu:154-233,
        # 315-454; no chunked form reproduces it), scalar beta, zero initial state
        s0 = torch.zeros(B * H, K, K, dtype=torch.bfloat16, device=dev)
        st = s0.clone()

        def fwd_r():
            efla.efla_forward(x["k"], x["v"], st.copy_(s0), 0.5, C)

        def bwd_r():
            efla.efla_backward(x["do"], x["k"], x["v"], s0, 0.5)

        fwd_r()
        bwd_r()
        per_f, _ = timed(fwd_r, 3)
        per_b, _ = timed(bwd_r, 3)
        mf_, mb_ = median(per_f), median(per_b)
        ref_abi = {
            "what": "efla_forward_hip / efla_backward_hip (the reference's token-serial "
                    "recurrence, state re-rounded to bf16 per token), median of 3 calls",
            "forward_ms": round(mf_, 3), "backward_ms": round(mb_, 3),
            "forward_tokens_per_s": round(ntok / (mf_ * 1e-3), 1),
            "backward_tokens_per_s": round(ntok / (mb_ * 1e-3), 1),
        }
        print(f"[bench] reference ABI: forward {mf_:.3f} ms, backward {mb_:.3f} ms",
              file=sys.stderr, flush=True)

    # FLOPs / bytes
    if cu is not None:
        lens = (cu[1:] - cu[:-1]).tolist()
        n_chunks = sum((L + C - 1) // C for L in lens)
        fwd_flops = float(sum(lens)) * H * f_fwd_per_token_head(K, V)
    else:
        n_chunks = B * ((T + C - 1) // C)
        fwd_flops = float(ntok) * H * f_fwd_per_token_head(K, V)
    step_flops = fwd_flops * (3 if cfg["bwd"] else 1)
    per_chunk = kernel_flops_per_chunk(K, V)
    kernels = {}
    for name, (launches, tot_ms) in sorted(kern.items(), key=lambda kv: -kv[1][1]):
        avg_ms = tot_ms / max(launches, 1)
        fl = per_chunk.get(name, 0.0) * n_chunks * H
        kernels[name] = {
            "launches": launches, "avg_ms": round(avg_ms, 4),
            "share": round(tot_ms / max(prof_total, 1e-9), 4),
            "tflops": round(fl / (avg_ms * 1e-3) / 1e12, 2) if fl else None,
        }
    dom = max(kern.items(), key=lambda kv: kv[1][1])[0] if kern else None
    # the MFMA rate the path computes at: bf16 operands, or fp32 for cfg1
    peak = PEAK_BF16_TFLOPS if cfg["dtype"] == "bf16" else PEAK_FP32_TFLOPS
    roof = None
    if dom is not None:
        launches, tot_ms = kern[dom]
        avg_ms = tot_ms / launches
        fl = per_chunk.get(dom, 0.0) * n_chunks * H
        ach = fl / (avg_ms * 1e-3) / 1e12
        alg_bytes = kernel_io_bytes_per_token_head(
            K, V, 2 if cfg["dtype"] == "bf16" else 4).get(dom, 0) * ntok * H
        gbs = alg_bytes / (avg_ms * 1e-3) / 1e9
        traffic = measured_traffic(args.config, dom)
        mfma = {"achieved": round(ach, 2), "peak": peak, "unit": "TFLOP/s",
                "frac": round(ach / peak, 4), "flops_per_launch": fl}
        hbm = {"achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
               "frac": round(gbs / PEAK_HBM_GBS, 4), "algorithmic_bytes_per_launch": alg_bytes}
        if traffic:
            # what the launch moves (FETCH_SIZE + WRITE_SIZE) over its time
            hbm["measured_gbs"] = round(traffic / (avg_ms * 1e-3) / 1e9, 1)
        # the bound is the roof the kernel is closer to
        bound = "hbm" if hbm["frac"] > mfma["frac"] else "mfma"
        top = hbm if bound == "hbm" else mfma
        roof = {"kernel": dom, "bound": bound, "achieved": top["achieved"],
                "peak": top["peak"], "unit": top["unit"], "frac": top["frac"],
                "traffic": traffic, "avg_ms": round(avg_ms, 4), "mfma": mfma, "hbm": hbm}
    step_tflops = step_flops / (ms_step * 1e-3) / 1e12
    io = io_bytes(ntok, H, K, V, cfg["bwd"], esize=2 if cfg["dtype"] == "bf16" else 4)
    if recompute is not None:
        recompute = {
            "what": "north_star's design: no workspace handed over, the backward "
                    "recomputes the chunk factors and states",
            "ms_per_step": round(recompute, 4),
            "tokens_per_s": round(ntok / (recompute * 1e-3), 1),
            "pct_mfma_peak": round(100 * step_flops / (recompute * 1e-3) / 1e12 / peak, 3),
            "states_only": {
                "what": "the forward hands over its per-chunk factors (T, b, dc) but not "
                        "the chunk states or P; the backward recomputes the states",
                "ms_per_step": round(recompute_states, 4),
                "tokens_per_s": round(ntok / (recompute_states * 1e-3), 1),
                "pct_mfma_peak": round(
                    100 * step_flops / (recompute_states * 1e-3) / 1e12 / peak, 3),
            },
        }

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(cfg, args.seed, args.cpu_budget)

    info = runtime.device_info(0)
    tokens_per_s = ntok / (ms_step * 1e-3)
    line = {
        "metric": "EFLA fwd+bwd tokens/s at H=32,d=128,T=8192 bf16; % bf16 MFMA peak"
                  if args.config == "cfg3" else f"EFLA {args.config} tokens/s",
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "mean_ms_per_step": round(ms_total / args.steps, 4),
        "timing": "median of the timed steps (hipEvent pair per step on the launch stream)",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (seeded torch N(0,1) q/k/v/dO, k L2-normalised, "
                "beta=sigmoid(N(0,1)))",
        "config": {"workload": f"{args.config}: EFLA {'fwd+bwd' if cfg['bwd'] else 'fwd'} "
                               f"B={B} T={T} H={H} d_k={K} d_v={V} chunk={C} "
                               f"{cfg['dtype']}{' varlen' if cu is not None else ''}",
                   "tokens_per_step": ntok, "parallelism": "single GPU"},
        "pct_bf16_mfma_peak": round(100 * step_tflops / PEAK_BF16_TFLOPS, 3),
        "pct_mfma_peak": round(100 * step_tflops / peak, 3),
        "mfma_peak_tflops": peak,
        "step_tflops": round(step_tflops, 2),
        "step_flops": step_flops,
        "step_io_gbs": round(io / (ms_step * 1e-3) / 1e9, 1),
        "roofline": roof,
        "recompute": recompute,
        "reference_abi": ref_abi,
        "kernels": kernels,
        "cpu_baseline": cpu,
        "device": {"arch": info["arch"], "cus": info["compute_units"],
                   "clock_mhz": info["clock_khz"] // 1000},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
