"""Pins for the oracle's scalar pieces: bf16 rounding and the EFLA coefficient."""
import math

import numpy as np
import pytest
import torch


def test_bf16_roundtrip_kat(oracle):
    # The reference's own KAT values (src/tensor/dtype.zig:653-665).
    vals = np.array([0.0, -0.0, 1.0, -1.0, 100.0, -100.0, 0.5, -0.5, 1.17549435e-38,
                     -1.17549435e-38, 9.1835496e-41, -9.1835496e-41, np.inf, -np.inf],
                    dtype=np.float32)
    back = oracle.bf16_to_f32(oracle.f32_to_bf16(vals))
    assert np.array_equal(back.view(np.uint32), vals.view(np.uint32))
    nan = oracle.bf16_to_f32(oracle.f32_to_bf16(np.array([np.nan], dtype=np.float32)))
    assert np.isnan(nan).all()


def test_bf16_rne_matches_torch(oracle):
    # torch's fp32 -> bf16 cast is round-to-nearest-even as well.
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(200_000) * np.exp(rng.uniform(-20, 20, 200_000))).astype(np.float32)
    # exact ties: low 16 bits == 0x8000
    ties = (rng.integers(0, 2**31, 4096, dtype=np.uint32) & 0xFFFF0000) | 0x8000
    x = np.concatenate([x, ties.view(np.float32)])
    x = x[np.isfinite(x)]
    ours = oracle.f32_to_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)


def test_coeff_reference_kat(oracle):
    # src/kernels/efla_kernels.zig:110-117
    c1, _ = oracle.coeff_f32(1e-8, 1.0)
    assert abs(c1 - 1.0) <= 1e-3
    c2, _ = oracle.coeff_f32(1.0, 1.0)
    assert abs(c2 - (1.0 - math.exp(-1.0))) <= 1e-3 * (1.0 - math.exp(-1.0))


@pytest.mark.parametrize("beta", [0.05, 0.5, 1.0, 3.0])
def test_coeff_taylor_branch_and_cancellation(oracle, beta):
    # efla.cu:94 switches to a 4-term series at lambda <= 1e-6.  The series side
    # matches the exact function; the closed-form side (1 - expf(-x))/lambda
    # cancels for x = beta*lambda << 1, with error bounded by ulp(1)/x.  The
    # fp64 function is continuous across the cutoff.
    lo, dlo = oracle.coeff_f32(1e-6, beta)
    c64, d64, _ = oracle.coeff_f64(1e-6, beta)
    assert abs(lo - c64) <= 1e-6 * beta
    assert abs(dlo - d64) <= 1e-6 * beta * beta
    lam_hi = 1.0001e-6
    hi, _ = oracle.coeff_f32(lam_hi, beta)
    c64_hi, _, _ = oracle.coeff_f64(lam_hi, beta)
    x = beta * lam_hi
    assert abs(hi - c64_hi) <= 2.0 * 2.0**-23 / x * c64_hi
    assert abs(c64 - c64_hi) <= 1e-9


@pytest.mark.parametrize("lam,beta", [(1e-9, 0.7), (1e-4, 0.3), (0.9, 0.6), (1.0, 1.0),
                                      (3.7, 0.25), (40.0, 0.9), (0.02, 0.4)])
def test_coeff_f64_closed_forms(oracle, lam, beta):
    c, dl, db = oracle.coeff_f64(lam, beta)
    # definition (mpmath-free high-precision form through expm1)
    assert c == pytest.approx(-math.expm1(-beta * lam) / lam, rel=1e-13)
    # central differences of the definition
    f = lambda l, b: -math.expm1(-b * l) / l
    h = 1e-6 * lam if lam > 1e-3 else 1e-5 * (1.0 + 1e-3)  # c extends analytically to lambda < 0
    fd_l = (f(lam + h, beta) - f(lam - h, beta)) / (2 * h)
    fd_b = (f(lam, beta + 1e-6) - f(lam, beta - 1e-6)) / 2e-6
    assert dl == pytest.approx(fd_l, rel=1e-5, abs=1e-9)
    assert db == pytest.approx(fd_b, rel=1e-6)
    assert db == pytest.approx(math.exp(-beta * lam), rel=1e-14)
    # fp32 reference formula agrees up to its cancellation bound ulp(1)/x
    c32, d32 = oracle.coeff_f32(lam, beta)
    x = beta * lam
    bound = 2e-6 + (0.0 if lam <= 1e-6 else 2.0 * 2.0**-23 / x)
    assert c32 == pytest.approx(c, rel=bound, abs=1e-7)
    if x > 0.1:
        assert d32 == pytest.approx(dl, rel=1e-4, abs=1e-6)


def test_coeff_limits(oracle):
    # lambda -> 0 gives c -> beta (the plain delta rule step); beta = 0 gives c = 0.
    c, _, _ = oracle.coeff_f64(1e-15, 0.37)
    assert c == pytest.approx(0.37, rel=1e-12)
    c, dl, db = oracle.coeff_f64(1.3, 0.0)
    assert c == 0.0 and dl == 0.0 and db == 1.0


def test_randn_is_standard_normal_and_sliceable(oracle):
    x = oracle.randn(1234, (200_000,))
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    part = oracle.randn(1234, (1000,), offset=5000)
    assert np.array_equal(part, x[5000:6000])
