// GELU forward / backward and the AdamW step for gfx950.  All are HBM-bound
// elementwise passes: 16-byte loads and stores (8 bf16 or 4 fp32 per access),
// a grid-stride loop over at most kMaxBlocks workgroups, and a scalar tail.
// Buffers not 16-byte aligned take the scalar loop throughout.
//
// GELU (replaces gelu_forward_cuda / gelu_backward_cuda, layernorm.cu:189-250,
// 385-425): bf16 in / out, fp32 math.
//   tanh form  0.5 x (1 + tanh u), u = sqrt(2/pi) (x + 0.044715 x^3), written
//              x * s with s = 1 / (1 + e^(-2u)) by the logistic identity
//              0.5 (1 + tanh u) = 1 / (1 + e^(-2u)): one v_exp_f32 and one
//              v_rcp_f32 per element.  Derivative s + 2 x s (1 - s) u' with
//              u' = sqrt(2/pi) (1 + 3 * 0.044715 x^2) (since 1 - tanh^2 u =
//              4 s (1 - s)).
//   erf form   x Phi(x) with Phi(x) = erfc(-x / sqrt 2) / 2 (the library
//              erfcf: no cancellation of 1 + erf for x << 0, where the
//              reference's fp32 1 + erff loses its relative accuracy);
//              derivative Phi(x) + x phi(x).
//   Both forms stay accurate relative to the (small) result for x << 0; the
//   reference's 1 + tanhf(u) and 1 + erff cancel there (below x = -4 or so,
//   where |GELU(x)| < 1e-4 and its absolute error stays below 1e-7).
//
// AdamW (replaces adamw_step_cuda, optim.cu:147-178, 657-709): bf16 param,
// grad, exp_avg, exp_avg_sq; fp32 math in the reference's order; each new
// value rounded to bf16; bias corrections 1 - beta^step formed in double on
// the host.  adamw_step_master_hip runs the same step on fp32 master weights
// and fp32 moments with a bf16 gradient, and optionally writes a bf16 copy of
// the new weights (what a bf16 model with fp32 master weights needs).
#include <hip/hip_runtime.h>
#include <math.h>

#include "../../include/efla_hip.h"
#include "common.hpp"
#include "gelu.hpp"
#include "internal.hpp"

namespace efla {
namespace ew {

constexpr int NTH = 256;
constexpr long kMaxBlocks = 4096;  // 16 workgroups per CU on 256 CUs

typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

__device__ __forceinline__ long gid() { return (long)blockIdx.x * NTH + threadIdx.x; }
__device__ __forceinline__ long gstride() { return (long)gridDim.x * NTH; }

// ---------------------------------------------------------------------------
// GELU
// ---------------------------------------------------------------------------
using namespace ::efla::gelu;

template <bool APPROX>
__global__ void __launch_bounds__(NTH) gelu_fwd_kernel(const bf16* __restrict__ x,
                                                       bf16* __restrict__ y, long n, long n8) {
    for (long i = gid(); i < n8; i += gstride()) {
        const bf16x8 a = reinterpret_cast<const bf16x8*>(x)[i];
        bf16x8 r;
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = (bf16)gelu_f<APPROX>((float)a[j]);
        reinterpret_cast<bf16x8*>(y)[i] = r;
    }
    for (long i = n8 * 8 + gid(); i < n; i += gstride()) y[i] = (bf16)gelu_f<APPROX>((float)x[i]);
}

template <bool APPROX>
__global__ void __launch_bounds__(NTH) gelu_bwd_kernel(const bf16* __restrict__ dy,
                                                       const bf16* __restrict__ x,
                                                       bf16* __restrict__ dx, long n, long n8) {
    for (long i = gid(); i < n8; i += gstride()) {
        const bf16x8 a = reinterpret_cast<const bf16x8*>(x)[i];
        const bf16x8 g = reinterpret_cast<const bf16x8*>(dy)[i];
        bf16x8 r;
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = (bf16)((float)g[j] * gelu_df<APPROX>((float)a[j]));
        reinterpret_cast<bf16x8*>(dx)[i] = r;
    }
    for (long i = n8 * 8 + gid(); i < n; i += gstride())
        dx[i] = (bf16)((float)dy[i] * gelu_df<APPROX>((float)x[i]));
}

// ---------------------------------------------------------------------------
// AdamW
// ---------------------------------------------------------------------------
struct AdamArgs {
    float lr, beta1, beta2, bc1, bc2, eps, weight_decay;
};

// one element, optim.cu:164-176 order; p, m, v updated in place
__device__ __forceinline__ void adam1(float& p, float g, float& m, float& v, const AdamArgs& a) {
    m = a.beta1 * m + (1.0f - a.beta1) * g;
    v = a.beta2 * v + (1.0f - a.beta2) * g * g;
    const float mh = m / a.bc1;
    const float vh = v / a.bc2;
    const float den = sqrtf(fmaxf(vh, 0.0f)) + a.eps;
    p = p * (1.0f - a.lr * a.weight_decay) - a.lr * (mh / den);
}

__global__ void __launch_bounds__(NTH) adamw_bf16_kernel(bf16* __restrict__ p,
                                                         const bf16* __restrict__ g,
                                                         bf16* __restrict__ m,
                                                         bf16* __restrict__ v, long n, long n8,
                                                         AdamArgs a) {
    for (long i = gid(); i < n8; i += gstride()) {
        bf16x8 pv = reinterpret_cast<bf16x8*>(p)[i];
        const bf16x8 gv = reinterpret_cast<const bf16x8*>(g)[i];
        bf16x8 mv = reinterpret_cast<bf16x8*>(m)[i];
        bf16x8 vv = reinterpret_cast<bf16x8*>(v)[i];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float pf = (float)pv[j], mf = (float)mv[j], vf = (float)vv[j];
            adam1(pf, (float)gv[j], mf, vf, a);
            pv[j] = (bf16)pf;
            mv[j] = (bf16)mf;
            vv[j] = (bf16)vf;
        }
        reinterpret_cast<bf16x8*>(p)[i] = pv;
        reinterpret_cast<bf16x8*>(m)[i] = mv;
        reinterpret_cast<bf16x8*>(v)[i] = vv;
    }
    for (long i = n8 * 8 + gid(); i < n; i += gstride()) {
        float pf = (float)p[i], mf = (float)m[i], vf = (float)v[i];
        adam1(pf, (float)g[i], mf, vf, a);
        p[i] = (bf16)pf;
        m[i] = (bf16)mf;
        v[i] = (bf16)vf;
    }
}

// fp32 p, m, v; bf16 g; optional bf16 copy of p.  8 elements per iteration.
__global__ void __launch_bounds__(NTH) adamw_master_kernel(float* __restrict__ p,
                                                           const bf16* __restrict__ g,
                                                           float* __restrict__ m,
                                                           float* __restrict__ v,
                                                           bf16* __restrict__ pcopy, long n,
                                                           long n8, AdamArgs a) {
    for (long i = gid(); i < n8; i += gstride()) {
        f32x4 p0 = reinterpret_cast<f32x4*>(p)[2 * i], p1 = reinterpret_cast<f32x4*>(p)[2 * i + 1];
        f32x4 m0 = reinterpret_cast<f32x4*>(m)[2 * i], m1 = reinterpret_cast<f32x4*>(m)[2 * i + 1];
        f32x4 v0 = reinterpret_cast<f32x4*>(v)[2 * i], v1 = reinterpret_cast<f32x4*>(v)[2 * i + 1];
        const bf16x8 gv = reinterpret_cast<const bf16x8*>(g)[i];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float pa = p0[j], ma = m0[j], va = v0[j], pb = p1[j], mb = m1[j], vb = v1[j];
            adam1(pa, (float)gv[j], ma, va, a);
            adam1(pb, (float)gv[4 + j], mb, vb, a);
            p0[j] = pa, m0[j] = ma, v0[j] = va, p1[j] = pb, m1[j] = mb, v1[j] = vb;
        }
        reinterpret_cast<f32x4*>(p)[2 * i] = p0;
        reinterpret_cast<f32x4*>(p)[2 * i + 1] = p1;
        reinterpret_cast<f32x4*>(m)[2 * i] = m0;
        reinterpret_cast<f32x4*>(m)[2 * i + 1] = m1;
        reinterpret_cast<f32x4*>(v)[2 * i] = v0;
        reinterpret_cast<f32x4*>(v)[2 * i + 1] = v1;
        if (pcopy) {
            bf16x8 c;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                c[j] = (bf16)p0[j];
                c[4 + j] = (bf16)p1[j];
            }
            reinterpret_cast<bf16x8*>(pcopy)[i] = c;
        }
    }
    for (long i = n8 * 8 + gid(); i < n; i += gstride()) {
        adam1(p[i], (float)g[i], m[i], v[i], a);
        if (pcopy) pcopy[i] = (bf16)p[i];
    }
}

// ---------------------------------------------------------------------------
// host helpers
// ---------------------------------------------------------------------------
inline bool aligned16(const void* q) { return q == nullptr || ((uintptr_t)q & 15) == 0; }

// Vector count (0: scalar loop only) and grid for n elements.
inline void plan(size_t n, bool vec, long* n8, dim3* grid, long max_blocks = kMaxBlocks) {
    *n8 = vec ? (long)(n / 8) : 0;
    const long work = vec ? *n8 : (long)n;
    long blocks = (work + NTH - 1) / NTH;
    if (blocks < 1) blocks = 1;
    if (blocks > max_blocks) blocks = max_blocks;
    *grid = dim3((unsigned)blocks);
}

// optim.cu:671-690: hyper-parameter checks and the double-precision bias
// corrections; returns kSuccess and fills `a`, or kInvalidValue.
int adam_args(float lr, float beta1, float beta2, float eps, float weight_decay, size_t step,
              AdamArgs* a) {
    if (!isfinite(lr) || !isfinite(beta1) || !isfinite(beta2) || !isfinite(eps) ||
        !isfinite(weight_decay))
        return kInvalidValue;
    if (beta1 < 0.0f || beta1 >= 1.0f || beta2 < 0.0f || beta2 >= 1.0f || eps <= 0.0f || step == 0)
        return kInvalidValue;
    const double bc1 = 1.0 - pow((double)beta1, (double)step);
    const double bc2 = 1.0 - pow((double)beta2, (double)step);
    if (!(bc1 > 0.0) || !(bc2 > 0.0) || !isfinite(bc1) || !isfinite(bc2)) return kInvalidValue;
    *a = AdamArgs{lr, beta1, beta2, (float)bc1, (float)bc2, eps, weight_decay};
    return kSuccess;
}

// ---------------------------------------------------------------------------
// Per-token beta gate of a fused projection row: the row ends in `cols` beta
// logits at row stride `ld`; beta is packed (rows, cols).  fp32 math, bf16
// rounding of each result, as torch's sigmoid(x.float()).to(bf16) forward and
// (g.float() * b) * (1 - b) backward.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(NTH) gate_fwd_kernel(const bf16* __restrict__ x, long ld,
                                                       bf16* __restrict__ y, long n, int cols) {
    for (long i = gid(); i < n; i += gstride()) {
        const long r = i / cols;
        const float v = (float)x[r * ld + (i - r * cols)];
        y[i] = (bf16)(1.f / (1.f + expf(-v)));
    }
}

__global__ void __launch_bounds__(NTH) gate_bwd_kernel(const bf16* __restrict__ g,
                                                       const bf16* __restrict__ b,
                                                       bf16* __restrict__ dx, long ld, long n,
                                                       int cols) {
    for (long i = gid(); i < n; i += gstride()) {
        const long r = i / cols;
        const float bb = (float)b[i];
        dx[r * ld + (i - r * cols)] = (bf16)(((float)g[i] * bb) * (1.f - bb));
    }
}

}  // namespace ew
}  // namespace efla

using namespace efla;

static int gate_args(size_t ld, size_t rows, size_t cols, size_t* n) {
    if (ld < cols || cols > (size_t)INT32_MAX) return kInvalidValue;
    if (rows > ((size_t)1 << 40) || ld >= ((size_t)1 << 24)) return kInvalidConfiguration;
    *n = rows * cols;
    return kSuccess;
}

extern "C" int sigmoid_gate_forward_hip(const void* logits, size_t ld, void* beta, size_t rows,
                                        size_t cols, hipStream_t stream) {
    if (rows == 0 || cols == 0) return kSuccess;
    if (!logits || !beta) return kInvalidValue;
    size_t n;
    const int rc = gate_args(ld, rows, cols, &n);
    if (rc != kSuccess) return rc;
    long n8;
    dim3 grid;
    ew::plan(n, false, &n8, &grid);
    EFLA_LAUNCH("sigmoid_gate_fwd", ew::gate_fwd_kernel, grid, dim3(ew::NTH), stream,
                (const bf16*)logits, (long)ld, (bf16*)beta, (long)n, (int)cols);
    return (int)hipPeekAtLastError();
}

extern "C" int sigmoid_gate_backward_hip(const void* grad_beta, const void* beta,
                                         void* grad_logits, size_t ld, size_t rows, size_t cols,
                                         hipStream_t stream) {
    if (rows == 0 || cols == 0) return kSuccess;
    if (!grad_beta || !beta || !grad_logits) return kInvalidValue;
    size_t n;
    const int rc = gate_args(ld, rows, cols, &n);
    if (rc != kSuccess) return rc;
    long n8;
    dim3 grid;
    ew::plan(n, false, &n8, &grid);
    EFLA_LAUNCH("sigmoid_gate_bwd", ew::gate_bwd_kernel, grid, dim3(ew::NTH), stream,
                (const bf16*)grad_beta, (const bf16*)beta, (bf16*)grad_logits, (long)ld,
                (long)n, (int)cols);
    return (int)hipPeekAtLastError();
}

// gelu_forward_cuda (layernorm.cu:385-403) launches ceil(numel / 256) blocks
// without checking numel: an empty grid, which the runtime rejects as an
// invalid configuration.  numel == 0 therefore returns 9 here too.
extern "C" int gelu_forward_hip(const void* input, void* output, size_t numel, bool approximate,
                                hipStream_t stream) {
    if (numel == 0) return kInvalidConfiguration;
    if (!input || !output) return kInvalidValue;
    long n8;
    dim3 grid;
    ew::plan(numel, ew::aligned16(input) && ew::aligned16(output), &n8, &grid);
    if (approximate)
        EFLA_LAUNCH("gelu_fwd", ew::gelu_fwd_kernel<true>, grid, dim3(ew::NTH), stream,
                    (const bf16*)input, (bf16*)output, (long)numel, n8);
    else
        EFLA_LAUNCH("gelu_fwd", ew::gelu_fwd_kernel<false>, grid, dim3(ew::NTH), stream,
                    (const bf16*)input, (bf16*)output, (long)numel, n8);
    return (int)hipPeekAtLastError();
}

extern "C" int gelu_backward_hip(const void* grad_output, const void* input, void* grad_input,
                                 size_t numel, bool approximate, hipStream_t stream) {
    if (numel == 0) return kInvalidConfiguration;
    if (!grad_output || !input || !grad_input) return kInvalidValue;
    long n8;
    dim3 grid;
    ew::plan(numel,
             ew::aligned16(grad_output) && ew::aligned16(input) && ew::aligned16(grad_input), &n8,
             &grid);
    if (approximate)
        EFLA_LAUNCH("gelu_bwd", ew::gelu_bwd_kernel<true>, grid, dim3(ew::NTH), stream,
                    (const bf16*)grad_output, (const bf16*)input, (bf16*)grad_input,
                    (long)numel, n8);
    else
        EFLA_LAUNCH("gelu_bwd", ew::gelu_bwd_kernel<false>, grid, dim3(ew::NTH), stream,
                    (const bf16*)grad_output, (const bf16*)input, (bf16*)grad_input,
                    (long)numel, n8);
    return (int)hipPeekAtLastError();
}

extern "C" int adamw_step_hip(void* param, const void* grad, void* exp_avg, void* exp_avg_sq,
                              size_t numel, float lr, float beta1, float beta2, float eps,
                              float weight_decay, size_t step, hipStream_t stream) {
    if (numel == 0) return kSuccess;
    if (!param || !grad || !exp_avg || !exp_avg_sq) return kInvalidValue;
    ew::AdamArgs a;
    const int rc = ew::adam_args(lr, beta1, beta2, eps, weight_decay, step, &a);
    if (rc != kSuccess) return rc;
    long n8;
    dim3 grid;
    ew::plan(numel,
             ew::aligned16(param) && ew::aligned16(grad) && ew::aligned16(exp_avg) &&
                 ew::aligned16(exp_avg_sq),
             &n8, &grid);
    EFLA_LAUNCH("adamw_bf16", ew::adamw_bf16_kernel, grid, dim3(ew::NTH), stream, (bf16*)param,
                (const bf16*)grad, (bf16*)exp_avg, (bf16*)exp_avg_sq, (long)numel, n8, a);
    return (int)hipPeekAtLastError();
}

extern "C" int adamw_step_master_hip(float* param, const void* grad, float* exp_avg,
                                     float* exp_avg_sq, void* param_bf16, size_t numel, float lr,
                                     float beta1, float beta2, float eps, float weight_decay,
                                     size_t step, hipStream_t stream) {
    if (numel == 0) return kSuccess;
    if (!param || !grad || !exp_avg || !exp_avg_sq) return kInvalidValue;
    ew::AdamArgs a;
    const int rc = ew::adam_args(lr, beta1, beta2, eps, weight_decay, step, &a);
    if (rc != kSuccess) return rc;
    long n8;
    dim3 grid;
    ew::plan(numel,
             ew::aligned16(param) && ew::aligned16(grad) && ew::aligned16(exp_avg) &&
                 ew::aligned16(exp_avg_sq) && ew::aligned16(param_bf16),
             &n8, &grid, 4 * ew::kMaxBlocks);  // 2-3 % faster than 4096 on 368M values
    EFLA_LAUNCH("adamw_master", ew::adamw_master_kernel, grid, dim3(ew::NTH), stream, param,
                (const bf16*)grad, exp_avg, exp_avg_sq, (bf16*)param_bf16, (long)numel, n8, a);
    return (int)hipPeekAtLastError();
}
