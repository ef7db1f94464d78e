"""efla_chunk_fwd_noalloc_hip, the forward for callers that cannot allocate:
through the C ABI its results must equal efla_chunk_fwd_hip's bit for bit,
on two calls in a row (the second smaller, so the fixed scratch array holds
the first call's data when the second starts), it must not touch the
library's cached workspaces, and a problem beyond the fixed scratch size is
refused with 2 before anything is queued."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import announce

pytestmark = pytest.mark.gpu

BF16, F32 = 14, 0


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _inputs(seed, B, T, H, K, V, dtype, cu=None, states=False):
    g = torch.Generator(device="cuda:0").manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=g, device="cuda:0")
    k = torch.randn(B, T, H, K, generator=g, device="cuda:0")
    k = k / k.norm(dim=-1, keepdim=True)
    v = torch.randn(B, T, H, V, generator=g, device="cuda:0")
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g, device="cuda:0"))
    x = {n: t.to(dtype).contiguous() for n, t in (("q", q), ("k", k), ("v", v), ("beta", beta))}
    N = B if cu is None else len(cu) - 1
    x["cu"] = None if cu is None else torch.tensor(cu, dtype=torch.int32, device="cuda:0")
    x["s0"] = (torch.randn(N, H, K, V, generator=g, device="cuda:0") * 0.3) if states else None
    x.update(B=B, T=T, H=H, K=K, V=V, N=N, dt=BF16 if dtype == torch.bfloat16 else F32)
    return x


def _call(L, x, noalloc):
    """One forward through the C ABI; returns (rc, o, S_T or None)."""
    o = torch.full((x["B"], x["T"], x["H"], x["V"]), 7.0, dtype=x["q"].dtype, device="cuda:0")
    st = None
    if x["s0"] is not None:
        st = torch.full((x["N"], x["H"], x["K"], x["V"]), 7.0, device="cuda:0")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nseq = x["N"] if x["cu"] is not None else 0
    args = (_p(x["q"]), _p(x["k"]), _p(x["v"]), _p(x["beta"]), _p(x["s0"]), _p(o), _p(st),
            _p(x["cu"]), x["B"], x["T"], nseq, x["H"], x["K"], x["V"], 64, x["dt"])
    if noalloc:
        rc = L.efla_chunk_fwd_noalloc_hip(*args, stream)
    else:
        rc = L.efla_chunk_fwd_hip(*args, None, 0, 0, stream)
    torch.cuda.synchronize()
    return rc, o, st


CASES = [
    # two calls in a row, the second with a smaller input
    ("bf16 B=2 T=2048 H=16 K=V=128, then varlen 3 seqs H=4 K=64 V=128 with states",
     [dict(seed=1, B=2, T=2048, H=16, K=128, V=128, dtype=torch.bfloat16),
      dict(seed=2, B=1, T=300, H=4, K=64, V=128, dtype=torch.bfloat16, cu=[0, 65, 129, 300],
           states=True)]),
    ("fp32 B=2 T=256 H=4 K=V=64 with states, then B=1 T=70",
     [dict(seed=3, B=2, T=256, H=4, K=64, V=64, dtype=torch.float32, states=True),
      dict(seed=4, B=1, T=70, H=4, K=64, V=64, dtype=torch.float32)]),
]


@pytest.mark.parametrize("name,calls", CASES, ids=["bf16", "fp32"])
def test_noalloc_matches_forward(name, calls):
    from ceo_amd import _lib, runtime

    L = _lib.lib()
    announce(f"noalloc forward: {name}")
    runtime.release_workspace()
    xs = [_inputs(**c) for c in calls]
    got = [_call(L, x, True) for x in xs]  # back to back on the fixed scratch
    assert runtime.workspace_bytes() == 0, "the no-alloc entry used a cached workspace"
    for i, (x, (rc, o, st)) in enumerate(zip(xs, got)):
        assert rc == 0, (i, rc)
        rc2, o2, st2 = _call(L, x, False)
        assert rc2 == 0
        assert torch.equal(o, o2), f"call {i}: output differs from efla_chunk_fwd_hip"
        if st is not None:
            assert torch.equal(st, st2), f"call {i}: final state differs"
        assert bool(torch.isfinite(o.float()).all())
    # the same calls again, now after other work has used the scratch
    for i, x in enumerate(xs):
        rc, o, _ = _call(L, x, True)
        assert rc == 0 and torch.equal(o, got[i][1]), f"repeat of call {i} differs"


def test_noalloc_runs_just_inside_scratch():
    """A problem whose forward workspace just fits the fixed scratch runs and
    matches the allocating entry point bit for bit.  (The refusal of larger
    problems is pinned without a GPU: test_abi_cpu.py's
    test_chunk_fwd_noalloc_validation.)"""
    from ceo_amd import _lib, efla

    L = _lib.lib()
    announce("noalloc forward: problem just inside the fixed scratch")
    limit = 64 << 20  # EFLA_NOALLOC_SCRATCH_BYTES
    x = _inputs(5, 1, 64 * 11000 // 16, 16, 64, 64, torch.bfloat16)  # 11,000 chunk-heads
    assert efla.workspace_bytes("fwd", 1, x["T"], 16, 64, 64, torch.bfloat16) <= limit
    rc, o, _ = _call(L, x, True)
    assert rc == 0
    rc2, o2, _ = _call(L, x, False)
    assert rc2 == 0 and torch.equal(o, o2)
