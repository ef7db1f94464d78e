// RMSNorm forward / backward for gfx950, bf16 rows with fp32 statistics.
//
// Forward (replaces rmsnorm_forward_cuda, kernels.h:125-133,
// layernorm.cu:15-48, 307-329): rows = numel / D,
//   rs = rsqrt(mean(x^2) + eps),  y = x rs w.
// Backward (replaces rmsnorm_backward_cuda, kernels.h:138-148,
// layernorm.cu:51-127), with g = dy w:
//   dx = rs g - x rs^3 mean(g x),   dw += sum_rows dy x rs.
// The reference's backward differs from this gradient: it multiplies the
// second term by rs / D instead of rs^3 / D (layernorm.cu:113-115), and adds
// fp32 values through a float pointer into its bf16 grad_weight buffer
// (layernorm.cu:119-123).  Here grad_weight is an fp32 buffer that the
// backward adds into (it may be NULL).
//
// Layout as the LayerNorm kernels: one row per wavefront; for D a multiple of
// 512 (up to 4096 forward, 2048 backward) the row lives in registers with
// 16-byte accesses and the backward accumulates dw per lane across its rows,
// combined per workgroup in LDS; other widths loop over the row (dw through
// LDS atomics).  A second kernel sums the per-workgroup dw partials in a fixed
// order and adds them to grad_weight.
#include <hip/hip_runtime.h>

#include "../../include/efla_hip.h"
#include "common.hpp"
#include "internal.hpp"
#include "reduce.hpp"

namespace efla {
namespace rms {

constexpr int NTH = 256;
constexpr int RPB = NTH / kWave;  // rows per workgroup and round

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
    return x;
}

template <int NV>
__global__ void __launch_bounds__(NTH) fwd_reg_kernel(const bf16* __restrict__ x,
                                                      const bf16* __restrict__ w,
                                                      bf16* __restrict__ y, long rows,
                                                      float eps) {
    constexpr int D = NV * 512;
    const long row = (long)blockIdx.x * RPB + wave_id();
    if (row >= rows) return;
    const int lane = lane_id();
    bf16x8 xv[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) xv[j] = *reinterpret_cast<const bf16x8*>(x + row * D + (j * 64 + lane) * 8);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += (float)xv[j][i] * (float)xv[j][i];
    const float rs = 1.0f / sqrtf(wave_sum(ss) * (1.0f / D) + eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = (j * 64 + lane) * 8;
        const bf16x8 wv = *reinterpret_cast<const bf16x8*>(w + c);
        bf16x8 o;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (bf16)((float)xv[j][i] * rs * (float)wv[i]);
        *reinterpret_cast<bf16x8*>(y + row * D + c) = o;
    }
}

__global__ void __launch_bounds__(NTH) fwd_loop_kernel(const bf16* __restrict__ x,
                                                       const bf16* __restrict__ w,
                                                       bf16* __restrict__ y, long rows, long D,
                                                       float eps) {
    const long row = (long)blockIdx.x * RPB + wave_id();
    if (row >= rows) return;
    const int lane = lane_id();
    const bf16* xr = x + row * D;
    float ss = 0.f;
    for (long c = lane; c < D; c += kWave) ss += (float)xr[c] * (float)xr[c];
    const float rs = 1.0f / sqrtf(wave_sum(ss) / (float)D + eps);
    for (long c = lane; c < D; c += kWave) y[row * D + c] = (bf16)((float)xr[c] * rs * (float)w[c]);
}

// part[blockIdx.x][0..D) = this workgroup's sum of dy x rs
template <int NV>
__global__ void __launch_bounds__(NTH) bwd_reg_kernel(const bf16* __restrict__ dy,
                                                      const bf16* __restrict__ x,
                                                      const bf16* __restrict__ w,
                                                      bf16* __restrict__ dx,
                                                      float* __restrict__ part, long rows,
                                                      float eps, int want_w) {
    constexpr int D = NV * 512;
    __shared__ float red[RPB][D];
    const int lane = lane_id(), wv = wave_id();
    float wf[NV][8], dwa[NV][8];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const bf16x8 t = *reinterpret_cast<const bf16x8*>(w + (j * 64 + lane) * 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            wf[j][i] = (float)t[i];
            dwa[j][i] = 0.f;
        }
    }
    const long waves = (long)gridDim.x * RPB;
    for (long row = (long)blockIdx.x * RPB + wv; row < rows; row += waves) {
        bf16x8 xv[NV], gv[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            xv[j] = *reinterpret_cast<const bf16x8*>(x + row * D + (j * 64 + lane) * 8);
            gv[j] = *reinterpret_cast<const bf16x8*>(dy + row * D + (j * 64 + lane) * 8);
        }
        float ss = 0.f, sgx = 0.f;
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float xf = (float)xv[j][i];
                ss += xf * xf;
                sgx += (float)gv[j][i] * wf[j][i] * xf;
            }
        const float rs = 1.0f / sqrtf(wave_sum(ss) * (1.0f / D) + eps);
        const float c2 = rs * rs * rs * wave_sum(sgx) * (1.0f / D);
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            bf16x8 o;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float xf = (float)xv[j][i], gy = (float)gv[j][i];
                o[i] = (bf16)(rs * gy * wf[j][i] - xf * c2);
                dwa[j][i] += gy * xf * rs;
            }
            *reinterpret_cast<bf16x8*>(dx + row * D + (j * 64 + lane) * 8) = o;
        }
    }
    if (!want_w) return;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) red[wv][(j * 64 + lane) * 8 + i] = dwa[j][i];
    __syncthreads();
    for (int c = threadIdx.x; c < D; c += NTH) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < RPB; ++k) s += red[k][c];
        part[(long)blockIdx.x * D + c] = s;
    }
}

__global__ void __launch_bounds__(NTH) bwd_loop_kernel(const bf16* __restrict__ dy,
                                                       const bf16* __restrict__ x,
                                                       const bf16* __restrict__ w,
                                                       bf16* __restrict__ dx,
                                                       float* __restrict__ part, long rows,
                                                       int D, float eps, int want_w,
                                                       int per_wave) {
    // dw partials: one D-float slice per wave (column c belongs to one lane of
    // the wave; the slices are added in wave order, so the sums do not depend
    // on timing) when per_wave, else one slice updated with atomics
    extern __shared__ float acc[];
    const int lane = lane_id();
    const int nacc = per_wave ? RPB * D : D;
    float* wacc = acc + (per_wave ? wave_id() * D : 0);
    if (want_w)
        for (int i = threadIdx.x; i < nacc; i += NTH) acc[i] = 0.f;
    __syncthreads();
    const long waves = (long)gridDim.x * RPB;
    for (long row = (long)blockIdx.x * RPB + wave_id(); row < rows; row += waves) {
        const bf16* xr = x + row * D;
        const bf16* gr = dy + row * D;
        float ss = 0.f, sgx = 0.f;
        for (int c = lane; c < D; c += kWave) {
            const float xf = (float)xr[c];
            ss += xf * xf;
            sgx += (float)gr[c] * (float)w[c] * xf;
        }
        const float rs = 1.0f / sqrtf(wave_sum(ss) / (float)D + eps);
        const float c2 = rs * rs * rs * wave_sum(sgx) / (float)D;
        for (int c = lane; c < D; c += kWave) {
            const float xf = (float)xr[c], gy = (float)gr[c];
            dx[row * D + c] = (bf16)(rs * gy * (float)w[c] - xf * c2);
            if (want_w) {
                if (per_wave)
                    wacc[c] += gy * xf * rs;
                else
                    atomicAdd(&acc[c], gy * xf * rs);
            }
        }
    }
    if (!want_w) return;
    __syncthreads();
    for (int i = threadIdx.x; i < D; i += NTH) {
        float v = acc[i];
        if (per_wave)
            for (int ww = 1; ww < RPB; ++ww) v += acc[ww * D + i];
        part[(long)blockIdx.x * D + i] = v;
    }
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace rms
}  // namespace efla

using namespace efla;

extern "C" int rmsnorm_forward_hip(const void* input, const void* weight, void* output,
                                   size_t numel, size_t normalized_shape, float eps,
                                   hipStream_t stream) {
    const size_t D = normalized_shape;
    if (D == 0) return kInvalidValue;
    const size_t rows = numel / D;
    if (rows == 0) return kSuccess;
    if (!input || !weight || !output) return kInvalidValue;
    if (rows > ((size_t)1 << 40) || (rows + rms::RPB - 1) / rms::RPB > 0x7FFFFFFFull)
        return kInvalidConfiguration;
    const bf16 *x = (const bf16*)input, *w = (const bf16*)weight;
    bf16* y = (bf16*)output;
    const dim3 grid((unsigned)((rows + rms::RPB - 1) / rms::RPB)), block(rms::NTH);
    const bool vec = rms::aligned16(x) && rms::aligned16(w) && rms::aligned16(y);
    if (vec && D % 512 == 0 && D <= 4096) {
        switch (D / 512) {
#define RMS_FWD(nv)                                                                            \
    case nv:                                                                                   \
        EFLA_LAUNCH("rmsnorm_fwd", rms::fwd_reg_kernel<nv>, grid, block, stream, x, w, y,      \
                    (long)rows, eps);                                                          \
        return (int)hipPeekAtLastError();
            RMS_FWD(1) RMS_FWD(2) RMS_FWD(3) RMS_FWD(4) RMS_FWD(5) RMS_FWD(6) RMS_FWD(7)
            RMS_FWD(8)
#undef RMS_FWD
        }
    }
    EFLA_LAUNCH("rmsnorm_fwd_loop", rms::fwd_loop_kernel, grid, block, stream, x, w, y,
                (long)rows, (long)D, eps);
    return (int)hipPeekAtLastError();
}

extern "C" int rmsnorm_backward_hip(const void* grad_output, const void* input,
                                    const void* weight, void* grad_input, float* grad_weight,
                                    size_t numel, size_t normalized_shape, float eps,
                                    hipStream_t stream) {
    const size_t D = normalized_shape;
    if (D == 0) return kInvalidValue;
    const size_t rows = numel / D;
    if (rows == 0) return kSuccess;
    if (!grad_output || !input || !weight || !grad_input) return kInvalidValue;
    if ((grad_weight && D > 16384) || rows > ((size_t)1 << 40)) return kInvalidConfiguration;
    size_t nblk = (rows + rms::RPB - 1) / rms::RPB;
    if (nblk > 512) nblk = 512;
    float* part = nullptr;
    WsLease lease;
    if (grad_weight) {
        void* ws = nullptr;
        const int rc = workspace_acquire(nblk * D * sizeof(float), stream, &ws, lease);
        if (rc != kSuccess) return rc;
        part = (float*)ws;
    }
    const bf16 *g = (const bf16*)grad_output, *x = (const bf16*)input, *w = (const bf16*)weight;
    bf16* dx = (bf16*)grad_input;
    const bool vec = rms::aligned16(g) && rms::aligned16(x) && rms::aligned16(w) &&
                     rms::aligned16(dx);
    const int nv = (vec && D % 512 == 0 && D <= 2048) ? (int)(D / 512) : 0;
    const dim3 grid((unsigned)nblk), block(rms::NTH);
    const int want = grad_weight ? 1 : 0;
    switch (nv) {
#define RMS_BWD(n)                                                                            \
    case n:                                                                                   \
        EFLA_LAUNCH("rmsnorm_bwd", rms::bwd_reg_kernel<n>, grid, block, stream, g, x, w, dx,  \
                    part, (long)rows, eps, want);                                             \
        break;
        RMS_BWD(1) RMS_BWD(2) RMS_BWD(3) RMS_BWD(4)
#undef RMS_BWD
        default: {
            // per-wave dw slices (timing-independent sums) while they fit in
            // 64 KB of LDS
            const bool per_wave = want && D * rms::RPB <= 16384;
            ::efla::ProfScope ps("rmsnorm_bwd_loop", stream);
            hipLaunchKernelGGL(rms::bwd_loop_kernel, grid, block,
                               want ? (per_wave ? rms::RPB : 1) * D * sizeof(float) : 0, stream, g,
                               x, w, dx, part, (long)rows, (int)D, eps, want, per_wave ? 1 : 0);
        }
    }
    EFLA_CHECK(hipPeekAtLastError());
    if (grad_weight) {
        EFLA_LAUNCH("rmsnorm_bwd_reduce", partial_colsum_add_kernel,
                    partial_colsum_grid((long)D), dim3(256), stream, (const float*)part,
                    (int)nblk, (long)D, grad_weight);
    }
    return (int)hipPeekAtLastError();
}
