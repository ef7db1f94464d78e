"""Concurrent callers: entry points that take their scratch from the library's
cached workspace (efla_chunk_bwd_hip with a NULL workspace, efla_backward_hip,
layernorm_backward_hip) called from two host threads on two streams, and from
two threads sharing one stream, must give results bit-identical to the same
calls made one after another.  The reference allocates its scratch per call
(kernels/cuda/efla.cu:631-647), so its callers never share it; here the cached
buffers are per (device, stream) and leased while a call queues its work."""
import threading

import pytest
import torch

from helpers import announce

pytestmark = pytest.mark.gpu


def _problem(seed):
    g = torch.Generator(device="cuda:0").manual_seed(seed)

    def bf(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g, device="cuda:0") * scale).to(torch.bfloat16)

    B, T, H, K = 2, 1000 + 37 * (seed % 5), 4, 128
    k = torch.randn(B, T, H, K, generator=g, device="cuda:0")
    k = (k / k.norm(dim=-1, keepdim=True)).to(torch.bfloat16)
    x = {"q": bf(B, T, H, K), "k": k, "v": bf(B, T, H, K), "do": bf(B, T, H, K),
         "beta": torch.sigmoid(torch.randn(B, T, H, generator=g, device="cuda:0"))
         .to(torch.bfloat16)}
    # Mode R (reference ABI): k, v (B, T, H, d), S_0 (B*H, d, d) bf16, scalar beta
    d = 64
    kr = torch.randn(1, 300, 2, d, generator=g, device="cuda:0")
    x["kr"] = (kr / kr.norm(dim=-1, keepdim=True)).to(torch.bfloat16)
    x["vr"], x["dor"] = bf(1, 300, 2, d), bf(1, 300, 2, d)
    x["s0"] = bf(2, d, d, scale=0.1)
    # LayerNorm rows
    x["ln_x"], x["ln_dy"] = bf(4096, 1024), bf(4096, 1024)
    x["ln_w"] = bf(1024, scale=0.5)
    x["ln_b"] = bf(1024, scale=0.1)
    return x


def _run(x):
    from ceo_amd import efla, nn

    out = list(efla.chunk_efla_bwd(x["q"], x["k"], x["v"], x["beta"], x["do"])[:4])
    out += list(efla.efla_backward(x["dor"], x["kr"], x["vr"], x["s0"], 0.7))
    _, mean, rstd = nn.layernorm_forward(x["ln_x"], x["ln_w"], x["ln_b"], save_stats=True)
    out += list(nn.layernorm_backward(x["ln_dy"], x["ln_x"], x["ln_w"], mean, rstd))
    return out


def _threads(problems, streams, reps=4):
    results = [None] * len(problems)
    errors = []
    start = threading.Barrier(len(problems))

    def worker(i):
        try:
            with torch.cuda.stream(streams[i]):
                start.wait()
                res = [_run(problems[i]) for _ in range(reps)]
            streams[i].synchronize()
            results[i] = res
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(repr(e))

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(len(problems))]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors
    return results


def _compare(results, refs):
    for i, (res, ref) in enumerate(zip(results, refs)):
        for rep, out in enumerate(res):
            for j, (a, b) in enumerate(zip(out, ref)):
                assert torch.equal(a, b), f"caller {i}, repeat {rep}, output {j} differs"


@pytest.mark.parametrize("shared_stream", [False, True])
def test_two_threads(shared_stream):
    from ceo_amd import runtime

    announce(f"concurrency: two threads, {'one shared stream' if shared_stream else 'two streams'}")
    problems = [_problem(1), _problem(2)]
    refs = [_run(p) for p in problems]  # one after another, default stream
    torch.cuda.synchronize()
    # start from empty caches so the concurrent calls also allocate and grow
    runtime.release_workspace()
    s = torch.cuda.Stream()
    streams = [s, s] if shared_stream else [s, torch.cuda.Stream()]
    results = _threads(problems, streams)
    torch.cuda.synchronize()
    _compare(results, refs)
