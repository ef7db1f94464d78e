// EFLA step coefficient on the device.
//
// c(beta, lambda) = (1 - exp(-beta lambda)) / lambda, its lambda derivative,
// and dc/dbeta = exp(-beta lambda) -- the function of
// kernels/cuda/efla.cu:93-115.  For x = beta*lambda < 0.03 (which contains the
// reference's lambda <= 1e-6 branch) the power series
//   c      = beta * sum_{n>=0} (-x)^n / (n+1)!
//   dc/dl  = beta^2 * sum_{n>=0} (-1)^{n+1} (n+1) x^n / (n+2)!
// is summed to x^5; above it the closed form is evaluated through expm1f.
// The reference's (1 - expf(-x)) / lambda cancels for small x (19% error at
// lambda = 1e-6, beta = 0.05); this form does not.
#pragma once
#include <hip/hip_runtime.h>

namespace efla {

__device__ __forceinline__ void efla_coeff(float lam, float beta, float& c, float& dcl,
                                           float& dcb) {
    const float x = beta * lam;
    if (fabsf(x) < 0.03f) {
        c = beta * (1.f + x * (-0.5f + x * (1.f / 6.f + x * (-1.f / 24.f +
                                                              x * (1.f / 120.f + x * (-1.f / 720.f))))));
        dcl = beta * beta *
              (-0.5f + x * (1.f / 3.f + x * (-1.f / 8.f + x * (1.f / 30.f +
                                                               x * (-1.f / 144.f + x * (1.f / 840.f))))));
    } else {
        const float em1 = expm1f(-x);
        c = -em1 / lam;
        dcl = (x * (em1 + 1.f) + em1) / (lam * lam);
    }
    dcb = expf(-x);
}

}  // namespace efla
