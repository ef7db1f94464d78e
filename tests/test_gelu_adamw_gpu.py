"""GELU and AdamW kernels on the GPU against the oracle.

GELU is compared in bf16 units with the oracle's fp64 value rounded to bf16:
the kernel computes in fp32, so an element may land one bf16 step away where
the exact value sits next to a rounding boundary.  AdamW with bf16 state is
compared with the oracle's fp32 step rounded to bf16 the same way; the
fp32-master variant within 1e-6 relative.  Sizes are ragged (a tail past the
8-element vectors) and one case uses buffers offset by one element, which
takes the unaligned scalar path.
"""
import numpy as np
import pytest
import torch

from helpers import announce, rel_l2

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    """bf16 bit patterns as int32 in 0 .. 0xFFFF."""
    return t.contiguous().view(torch.int16).cpu().numpy().astype(np.int32) & 0xFFFF


def _bf16_steps(got_bits, ref_bits) -> np.ndarray:
    """Distance in bf16 steps between two arrays of bf16 bit patterns (same sign)."""
    def ordered(b):
        b = b & 0xFFFF
        return np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(ordered(got_bits) - ordered(ref_bits))


def _dev_bf16(a, offset=False):
    """bf16 device tensor holding `a`; with offset, a view one element into a
    larger buffer (2-byte aligned only)."""
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)
    if not offset:
        return t.cuda()
    buf = torch.zeros(t.numel() + 1, dtype=torch.bfloat16, device="cuda")
    v = buf[1:]
    v.copy_(t.cuda())
    return v


def _check_bf16(got: torch.Tensor, ref32: np.ndarray, oracle, what: str, x=None):
    """At most one bf16 step from the oracle.  Where x < -9 (|GELU|, |GELU'|
    below 1e-16 in both forms) only to 1e-16 absolute: the kernel's v_exp_f32 /
    v_rcp_f32 / erfcf flush subnormal intermediates, which starts near x = -10."""
    ref_bits = oracle.f32_to_bf16(ref32).astype(np.int32)
    steps = _bf16_steps(_bits(got), ref_bits)
    tail = np.zeros(ref32.shape, bool) if x is None else x < -9
    g = got.float().cpu().numpy()
    assert np.all(np.abs(g[tail] - ref32[tail]) <= 1e-16), what
    steps = np.where(tail, 0, steps)
    frac = float((steps > 0).mean())
    print(f"  {what}: max {int(steps.max())} bf16 steps, {frac:.2e} of elements differ, "
          f"{int(tail.sum())} in the x < -9 tail", flush=True)
    assert steps.max() <= 1 and frac <= 2e-3, what


@pytest.mark.parametrize("approximate", [True, False], ids=["tanh", "erf"])
@pytest.mark.parametrize("n,offset", [(1_000_003, False), (4099, True), (8, False), (1, False)])
def test_gelu(oracle, approximate, n, offset):
    from ceo_amd.nn import gelu_backward, gelu_forward

    announce(f"gelu approximate={approximate} n={n} offset={offset}")
    rng = np.random.default_rng(n)
    x = oracle.round_bf16((rng.standard_normal(n) * 3).astype(np.float32))
    dy = oracle.round_bf16(rng.standard_normal(n).astype(np.float32))
    xd, dyd = _dev_bf16(x, offset), _dev_bf16(dy, offset)
    y = gelu_forward(xd, approximate)
    dx = gelu_backward(dyd, xd, approximate)
    torch.cuda.synchronize()
    _check_bf16(y, oracle.gelu_fwd(x, approximate), oracle, "y", x)
    _check_bf16(dx, oracle.gelu_bwd(dy, x, approximate), oracle, "dx", x)


def test_gelu_special_values(oracle):
    from ceo_amd.nn import gelu_backward, gelu_forward

    announce("gelu special values")
    x = np.array([0.0, 30.0, -30.0, 1e-20, -1e-20, 6.0, -6.0, 2.0], np.float32)
    for approximate in (True, False):
        xd = _dev_bf16(x)
        y = gelu_forward(xd, approximate).float().cpu().numpy()
        dx = gelu_backward(torch.ones_like(xd), xd, approximate).float().cpu().numpy()
        assert y[0] == 0.0 and y[1] == 30.0 and y[2] == 0.0
        assert dx[0] == 0.5 and dx[1] == 1.0 and dx[2] == 0.0
        _check_bf16(torch.from_numpy(y).to(torch.bfloat16), oracle.gelu_fwd(oracle.round_bf16(x),
                    approximate), oracle, "special y")


@pytest.mark.parametrize("n,offset", [(1_000_003, False), (999, True)])
@pytest.mark.parametrize("step", [1, 10])
def test_adamw_bf16_state(oracle, n, offset, step):
    from ceo_amd.nn import adamw_step

    announce(f"adamw bf16 n={n} offset={offset} step={step}")
    rng = np.random.default_rng(step + n)
    p = rng.standard_normal(n).astype(np.float32)
    g = (0.1 * rng.standard_normal(n)).astype(np.float32)
    m = (0.01 * rng.standard_normal(n)).astype(np.float32) if step > 1 else np.zeros(n, np.float32)
    v = (1e-4 * np.abs(rng.standard_normal(n))).astype(np.float32) if step > 1 else \
        np.zeros(n, np.float32)
    hp = dict(lr=3e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.1, step=step)
    pd, gd, md, vd = (_dev_bf16(a, offset) for a in (p, g, m, v))
    adamw_step(pd, gd, md, vd, **hp)
    torch.cuda.synchronize()
    rp, rm, rv = oracle.adamw_step_bf16(*(oracle.f32_to_bf16(a) for a in (p, g, m, v)),
                                        hp["lr"], hp["beta1"], hp["beta2"], hp["eps"],
                                        hp["weight_decay"], step)
    for got, ref, name in ((pd, rp, "param"), (md, rm, "exp_avg"), (vd, rv, "exp_avg_sq")):
        steps = _bf16_steps(_bits(got), ref.astype(np.int32))
        frac = float((steps > 0).mean())
        print(f"  {name}: max {int(steps.max())} bf16 steps, {frac:.2e} differ", flush=True)
        assert steps.max() <= 1 and frac <= 1e-3, name


@pytest.mark.parametrize("n", [1_000_003, 5])
@pytest.mark.parametrize("step", [1, 7])
def test_adamw_master(oracle, n, step):
    from ceo_amd.nn import adamw_step_master

    announce(f"adamw master n={n} step={step}")
    rng = np.random.default_rng(7 * step + n)
    p = rng.standard_normal(n).astype(np.float32)
    g = oracle.round_bf16((0.1 * rng.standard_normal(n)).astype(np.float32))
    m = (0.01 * rng.standard_normal(n)).astype(np.float32) if step > 1 else np.zeros(n, np.float32)
    v = (1e-4 * np.abs(rng.standard_normal(n))).astype(np.float32) if step > 1 else \
        np.zeros(n, np.float32)
    hp = dict(lr=3e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.1, step=step)
    pd, md, vd = (torch.from_numpy(a.copy()).cuda() for a in (p, m, v))
    gd = _dev_bf16(g)
    pb = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    adamw_step_master(pd, gd, md, vd, param_bf16=pb, **hp)
    torch.cuda.synchronize()
    rp, rm, rv = p.copy(), m.copy(), v.copy()
    oracle.adamw_step(rp, g, rm, rv, hp["lr"], hp["beta1"], hp["beta2"], hp["eps"],
                      hp["weight_decay"], step)
    for got, ref, name in ((pd, rp, "param"), (md, rm, "exp_avg"), (vd, rv, "exp_avg_sq")):
        gg = got.cpu().numpy()
        err = np.abs(gg - ref) / (np.abs(ref) + 1e-30)
        print(f"  {name}: max rel {err.max():.2e}", flush=True)
        assert err.max() <= 1e-6, name
    assert np.array_equal(_bits(pb), oracle.f32_to_bf16(pd.cpu().numpy()).astype(np.int32))
    if step == 1:
        # from a zero state one step is p (1 - lr wd) - lr g / (|g| + eps)
        kat = p.astype(np.float64) * (1 - 3e-4 * 0.1) - 3e-4 * g / (np.abs(g) + 1e-8)
        assert np.abs(pd.cpu().numpy() - kat).max() < 1e-6


def test_adamw_matches_a_torch_adamw_run(oracle):
    """Ten master-weight steps track torch.optim.AdamW (fp32, decoupled decay)."""
    from ceo_amd.nn import adamw_step_master

    announce("adamw master vs torch.optim.AdamW, 10 steps")
    rng = np.random.default_rng(11)
    n = 4096
    p0 = rng.standard_normal(n).astype(np.float32)
    ref = torch.nn.Parameter(torch.from_numpy(p0.copy()))
    opt = torch.optim.AdamW([ref], lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    pd = torch.from_numpy(p0.copy()).cuda()
    md = torch.zeros(n, device="cuda")
    vd = torch.zeros(n, device="cuda")
    for step in range(1, 11):
        g = oracle.round_bf16(rng.standard_normal(n).astype(np.float32))
        ref.grad = torch.from_numpy(g.copy())
        opt.step()
        adamw_step_master(pd, _dev_bf16(g), md, vd, 1e-3, 0.9, 0.95, 1e-8, 0.1, step)
    torch.cuda.synchronize()
    e = rel_l2(pd, ref.detach().numpy())
    print(f"  rel-L2 after 10 steps {e:.2e}", flush=True)
    assert e <= 1e-6
