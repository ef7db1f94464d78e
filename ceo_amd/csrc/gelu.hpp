// GELU in fp32 for device code: the tanh form via the logistic identity
// 0.5 (1 + tanh u) = 1 / (1 + e^(-2u)) (one v_exp_f32, one v_rcp_f32, no
// cancellation for x << 0) and the erf form via erfcf.  The formulas behind
// the reference's gelu kernels (layernorm.cu:189-250) and its PRISM
// refinement step (src/model/prism.zig:293-300).
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>

namespace efla {
namespace gelu {

constexpr float kS2Pi = 0.7978845608028654f;  // sqrt(2 / pi)
constexpr float kCube = 0.044715f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kInvSqrt2 = 0.7071067811865476f;
constexpr float kInvSqrt2Pi = 0.3989422804014327f;

// s = 0.5 (1 + tanh u) = 1 / (1 + e^(-2u)); also returns u'
__device__ __forceinline__ float gelu_s(float x, float& du) {
    const float x2 = x * x;
    const float u = x * (kS2Pi + kS2Pi * kCube * x2);
    du = kS2Pi * (1.f + 3.f * kCube * x2);
    const float e = __builtin_amdgcn_exp2f(-2.f * kLog2e * u);  // e^(-2u); +inf -> s = 0
    return __builtin_amdgcn_rcpf(1.f + e);
}

template <bool APPROX>
__device__ __forceinline__ float gelu_f(float x) {
    if constexpr (APPROX) {
        float du;
        return x * gelu_s(x, du);
    } else {
        return 0.5f * x * erfcf(-x * kInvSqrt2);  // 1 + erf(x / sqrt 2) without cancellation
    }
}

template <bool APPROX>
__device__ __forceinline__ float gelu_df(float x) {
    if constexpr (APPROX) {
        float du;
        const float s = gelu_s(x, du);
        return s + 2.f * x * s * (1.f - s) * du;
    } else {
        const float cdf = 0.5f * erfcf(-x * kInvSqrt2);
        return cdf + x * (expf(-0.5f * x * x) * kInvSqrt2Pi);
    }
}

}  // namespace gelu
}  // namespace efla
