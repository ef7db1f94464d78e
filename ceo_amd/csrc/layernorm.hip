// LayerNorm forward / backward for gfx950, bf16 rows with fp32 statistics.
//
// Forward (replaces layernorm_forward_cuda, layernorm.cu:133-183, 359-383):
//   y = (x - mean) * rsqrt(var + eps) * w + b,  bias optional.
// One row per wavefront.  When D is a multiple of 512 and at most 4096 the
// row stays in registers (8 bf16 per lane per 512 columns, 16-byte coalesced
// loads), so HBM sees one read of x and one write of y; the variance is taken
// about the mean from those registers instead of the reference's
// E[x^2] - mean^2, which cancels when |mean| >> std.  Other widths take a
// looped path that re-reads the row (from cache for typical widths).
//
// Backward (no reference counterpart): with xhat = (x - mean) * rstd, g = dy*w
//   dx = rstd * (g - mean(g) - xhat * mean(g * xhat))
//   dw = sum_rows dy * xhat,  db = sum_rows dy      (fp32)
// One row per wavefront, grid-stride over rows.  For D a multiple of 512 up
// to 2048 the rows of x and dy stay in registers (16-byte loads, one HBM pass)
// and each lane accumulates dw/db for its own columns in registers across its
// rows; the 4 waves of a workgroup combine theirs in LDS and write one partial
// row.  Other widths loop over the row; up to D = 2048 each wave accumulates
// dw/db in an LDS slice of its own (a column belongs to one lane of the wave)
// and the four slices are added in wave order, so the sums do not depend on
// timing; wider rows accumulate with LDS atomics (order-dependent in the last
// bits).  A second kernel sums the per-workgroup partials, 16 row groups per
// column block (D <= 8192 when dw/db are wanted).
#include <hip/hip_runtime.h>

#include "../../include/efla_hip.h"
#include "common.hpp"
#include "internal.hpp"

namespace efla {
namespace ln {

constexpr int NTH = 256;

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
    return x;
}

// Row held in registers: lane owns columns (j*64 + lane)*8 .. +8 for j < NV.
template <int NV>
__global__ void __launch_bounds__(NTH) fwd_reg_kernel(const bf16* __restrict__ x,
                                                      const bf16* __restrict__ w,
                                                      const bf16* __restrict__ b,
                                                      bf16* __restrict__ y,
                                                      float* __restrict__ mean_out,
                                                      float* __restrict__ rstd_out, long rows,
                                                      float eps) {
    constexpr int D = NV * 512;
    const long row = (long)blockIdx.x * (NTH / kWave) + wave_id();
    if (row >= rows) return;
    const int lane = lane_id();
    const bf16* xr = x + row * D;
    bf16x8 xv[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) xv[j] = *reinterpret_cast<const bf16x8*>(xr + (j * 64 + lane) * 8);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) s += (float)xv[j][i];
    const float mean = wave_sum(s) * (1.0f / D);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float d = (float)xv[j][i] - mean;
            ss += d * d;
        }
    const float var = wave_sum(ss) * (1.0f / D);
    const float rstd = 1.0f / sqrtf(var + eps);
    bf16* yr = y + row * D;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = (j * 64 + lane) * 8;
        const bf16x8 wv = *reinterpret_cast<const bf16x8*>(w + c);
        bf16x8 bv;
        if (b) bv = *reinterpret_cast<const bf16x8*>(b + c);
        bf16x8 o;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float bb = b ? (float)bv[i] : 0.f;
            o[i] = (bf16)(((float)xv[j][i] - mean) * rstd * (float)wv[i] + bb);
        }
        *reinterpret_cast<bf16x8*>(yr + c) = o;
    }
    if (lane == 0) {
        if (mean_out) mean_out[row] = mean;
        if (rstd_out) rstd_out[row] = rstd;
    }
}

// Any width: three passes over the row with stride-64 scalar access.
__global__ void __launch_bounds__(NTH) fwd_loop_kernel(const bf16* __restrict__ x,
                                                       const bf16* __restrict__ w,
                                                       const bf16* __restrict__ b,
                                                       bf16* __restrict__ y,
                                                       float* __restrict__ mean_out,
                                                       float* __restrict__ rstd_out, long rows,
                                                       long D, float eps) {
    const long row = (long)blockIdx.x * (NTH / kWave) + wave_id();
    if (row >= rows) return;
    const int lane = lane_id();
    const bf16* xr = x + row * D;
    float s = 0.f;
    for (long c = lane; c < D; c += kWave) s += (float)xr[c];
    const float mean = wave_sum(s) / (float)D;
    float ss = 0.f;
    for (long c = lane; c < D; c += kWave) {
        const float d = (float)xr[c] - mean;
        ss += d * d;
    }
    const float rstd = 1.0f / sqrtf(wave_sum(ss) / (float)D + eps);
    bf16* yr = y + row * D;
    for (long c = lane; c < D; c += kWave) {
        const float bb = b ? (float)b[c] : 0.f;
        yr[c] = (bf16)(((float)xr[c] - mean) * rstd * (float)w[c] + bb);
    }
    if (lane == 0) {
        if (mean_out) mean_out[row] = mean;
        if (rstd_out) rstd_out[row] = rstd;
    }
}

// dx per row; dw/db partials per workgroup in LDS, written to
// part[blockIdx.x][0..D) (dw) and part[blockIdx.x][D..2D) (db): per wave
// (4 * 2D floats, added in wave order) when per_wave, else one 2D block
// updated with atomics.
__global__ void __launch_bounds__(NTH) bwd_kernel(const bf16* __restrict__ dy,
                                                  const bf16* __restrict__ x,
                                                  const bf16* __restrict__ w,
                                                  const float* __restrict__ mean,
                                                  const float* __restrict__ rstd,
                                                  const bf16* __restrict__ res,
                                                  bf16* __restrict__ dx,
                                                  float* __restrict__ part, long rows, int D,
                                                  int want_params, int per_wave) {
    extern __shared__ float acc[];  // 2*D (4 * 2*D per_wave) when want_params
    const int lane = lane_id();
    const int nacc = per_wave ? (NTH / kWave) * 2 * D : 2 * D;
    float* wacc = acc + (per_wave ? wave_id() * 2 * D : 0);
    if (want_params)
        for (int i = threadIdx.x; i < nacc; i += NTH) acc[i] = 0.f;
    __syncthreads();
    const long waves = (long)gridDim.x * (NTH / kWave);
    for (long row = (long)blockIdx.x * (NTH / kWave) + wave_id(); row < rows; row += waves) {
        const bf16* xr = x + row * D;
        const bf16* gr = dy + row * D;
        const float mu = mean[row], rs = rstd[row];
        float sg = 0.f, sgx = 0.f;
        for (int c = lane; c < D; c += kWave) {
            const float xh = ((float)xr[c] - mu) * rs;
            const float g = (float)gr[c] * (float)w[c];
            sg += g;
            sgx += g * xh;
        }
        sg = wave_sum(sg) / (float)D;
        sgx = wave_sum(sgx) / (float)D;
        bf16* dxr = dx + row * D;
        for (int c = lane; c < D; c += kWave) {
            const float xh = ((float)xr[c] - mu) * rs;
            const float gy = (float)gr[c];
            const float g = gy * (float)w[c];
            const float add = res ? (float)res[row * D + c] : 0.f;
            dxr[c] = (bf16)(rs * (g - sg - xh * sgx) + add);
            if (want_params) {
                if (per_wave) {  // column c is this lane's alone within the wave
                    wacc[c] += gy * xh;
                    wacc[D + c] += gy;
                } else {
                    atomicAdd(&acc[c], gy * xh);
                    atomicAdd(&acc[D + c], gy);
                }
            }
        }
    }
    if (!want_params) return;
    __syncthreads();
    float* pr = part + (long)blockIdx.x * 2 * D;
    for (int i = threadIdx.x; i < 2 * D; i += NTH) {
        float v = acc[i];
        if (per_wave)
            for (int ww = 1; ww < NTH / kWave; ++ww) v += acc[ww * 2 * D + i];
        pr[i] = v;
    }
}

// Register-resident backward for D = NV * 512 (NV <= 4): lane owns columns
// (j * 64 + lane) * 8 + i.  part[blockIdx.x][0..D) = dw, [D..2D) = db
// partials, and with NS = 3 [2D..3D) = the column sums of dx (as written).
template <int NV, int NS>
__global__ void __launch_bounds__(NTH) bwd_reg_kernel(const bf16* __restrict__ dy,
                                                      const bf16* __restrict__ x,
                                                      const bf16* __restrict__ w,
                                                      const float* __restrict__ mean,
                                                      const float* __restrict__ rstd,
                                                      const bf16* __restrict__ res,
                                                      bf16* __restrict__ dx,
                                                      float* __restrict__ part, long rows,
                                                      int want_params) {
    constexpr int D = NV * 512;
    __shared__ float red[NTH / kWave][NS * D];  // 32 KB per 1024 columns and sum
    const int lane = lane_id(), wv = wave_id();
    float wf[NV][8], dwa[NV][8], dba[NV][8], dxa[NV][8];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const bf16x8 t = *reinterpret_cast<const bf16x8*>(w + (j * 64 + lane) * 8);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            wf[j][i] = (float)t[i];
            dwa[j][i] = dba[j][i] = dxa[j][i] = 0.f;
        }
    }
    const long waves = (long)gridDim.x * (NTH / kWave);
    long row = (long)blockIdx.x * (NTH / kWave) + wv;
    // the next two rows' x, dy (and the residual gradient) and their mean and
    // rstd are in flight while this one computes: with one row a wave kept too
    // few bytes in flight to cover the loaded memory latency.  The statistics
    // travel with the rows: loaded at their use, after the prefetch, their
    // wait (one in-order counter for all vector-memory loads) would also wait
    // for the rows just prefetched.
    bf16x8 xn[2][NV], gn[2][NV], rn[2][NV] = {};
    float mun[2] = {0.f, 0.f}, rsn[2] = {0.f, 0.f};
    auto fetch = [&](long r, int sl) {
        mun[sl] = mean[r];
        rsn[sl] = rstd[r];
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            xn[sl][j] = *reinterpret_cast<const bf16x8*>(x + r * D + (j * 64 + lane) * 8);
            gn[sl][j] = *reinterpret_cast<const bf16x8*>(dy + r * D + (j * 64 + lane) * 8);
            if (res) rn[sl][j] = *reinterpret_cast<const bf16x8*>(res + r * D + (j * 64 + lane) * 8);
        }
    };
    if (row < rows) fetch(row, 0);
    if (row + waves < rows) fetch(row + waves, 1);
    for (; row < rows; row += waves) {
        bf16x8 xv[NV], gv[NV], rv[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            xv[j] = xn[0][j];
            gv[j] = gn[0][j];
            rv[j] = rn[0][j];
            xn[0][j] = xn[1][j];
            gn[0][j] = gn[1][j];
            rn[0][j] = rn[1][j];
        }
        const float mu = mun[0], rs = rsn[0];
        mun[0] = mun[1];
        rsn[0] = rsn[1];
        if (row + 2 * waves < rows) fetch(row + 2 * waves, 1);
        float sg = 0.f, sgx = 0.f;
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float g = (float)gv[j][i] * wf[j][i];
                sg += g;
                sgx += g * (((float)xv[j][i] - mu) * rs);
            }
        sg = wave_sum(sg) * (1.0f / D);
        sgx = wave_sum(sgx) * (1.0f / D);
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            bf16x8 o;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float xh = ((float)xv[j][i] - mu) * rs;
                const float gy = (float)gv[j][i];
                const float add = res ? (float)rv[j][i] : 0.f;
                o[i] = (bf16)(rs * (gy * wf[j][i] - sg - xh * sgx) + add);
                dwa[j][i] += gy * xh;
                dba[j][i] += gy;
                if constexpr (NS == 3) dxa[j][i] += (float)o[i];
            }
            *reinterpret_cast<bf16x8*>(dx + row * D + (j * 64 + lane) * 8) = o;
        }
    }
    if (!want_params) return;
    // combine the 4 waves' column sums, then one partial row per workgroup
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            red[wv][(j * 64 + lane) * 8 + i] = dwa[j][i];
            red[wv][D + (j * 64 + lane) * 8 + i] = dba[j][i];
            if constexpr (NS == 3) red[wv][2 * D + (j * 64 + lane) * 8 + i] = dxa[j][i];
        }
    __syncthreads();
    float* pr = part + (long)blockIdx.x * NS * D;
    for (int c = threadIdx.x; c < NS * D; c += NTH) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < NTH / kWave; ++k) s += red[k][c];
        pr[c] = s;
    }
}

// out[c] = sum_b part[b][c] for c < NS D (dw = out[0..D), db = out[D..2D),
// fp32 or with pbf bf16, and with NS = 3 the dx column sums out[2D..3D) as
// bf16 into dxs).
// Workgroup: 64 row groups x 4 lanes of 4 columns (16-byte loads), 16 columns
// per workgroup, so the grid has NS D / 16 workgroups and each thread's rows
// (b = rg, rg + 64, ...; at most 8 for the 512 partial rows) are all in flight
// at once.  Row group rg sums its rows in increasing b, then the 64 group
// sums are added in increasing rg: a fixed order.  Odd D reads scalars.
constexpr int RED_RG = 64, RED_U = 8;
__global__ void __launch_bounds__(NTH) reduce_kernel(const float* __restrict__ part, int nblk,
                                                     int D, int NS, void* __restrict__ dw,
                                                     void* __restrict__ db, int pbf,
                                                     bf16* __restrict__ dxs) {
    __shared__ float acc[RED_RG][16 + 1];
    const int q = threadIdx.x & 3, rg = threadIdx.x >> 2;
    const int c0 = blockIdx.x * 16 + 4 * q;
    const int W = NS * D;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    if (W % 4 == 0 && c0 + 4 <= W) {
        for (int b0 = rg; b0 < nblk; b0 += RED_RG * RED_U) {
            floatx4 v[RED_U];
#pragma unroll
            for (int u = 0; u < RED_U; ++u) {  // rows past the end re-read the last row
                const int b = min(b0 + RED_RG * u, nblk - 1);
                v[u] = *reinterpret_cast<const floatx4*>(part + (long)b * W + c0);
            }
#pragma unroll
            for (int u = 0; u < RED_U; ++u)
                if (b0 + RED_RG * u < nblk)
#pragma unroll
                    for (int i = 0; i < 4; ++i) s[i] += v[u][i];
        }
    } else {
        for (int b = rg; b < nblk; b += RED_RG)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (c0 + i < W) s[i] += part[(long)b * W + c0 + i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[rg][4 * q + i] = s[i];
    __syncthreads();
    if (threadIdx.x < 16) {
        const int c = blockIdx.x * 16 + threadIdx.x;
        float t = 0.f;
#pragma unroll 8
        for (int k = 0; k < RED_RG; ++k) t += acc[k][threadIdx.x];
        if (c < D) {
            if (dw && pbf) static_cast<bf16*>(dw)[c] = (bf16)t;
            else if (dw) static_cast<float*>(dw)[c] = t;
        } else if (c < 2 * D) {
            if (db && pbf) static_cast<bf16*>(db)[c - D] = (bf16)t;
            else if (db) static_cast<float*>(db)[c - D] = t;
        } else if (c < W && dxs) {
            dxs[c - 2 * D] = (bf16)t;
        }
    }
}

static int forward(const void* input, const void* weight, const void* bias, void* output,
                   float* mean, float* rstd, size_t numel, size_t D, float eps,
                   hipStream_t stream) {
    if (D == 0) return kInvalidValue;
    const size_t rows = numel / D;
    if (rows == 0) return kSuccess;
    if (!input || !weight || !output) return kInvalidValue;
    if (rows > ((size_t)1 << 40)) return kInvalidConfiguration;
    const size_t rpb = NTH / kWave;
    const size_t grid = (rows + rpb - 1) / rpb;
    if (grid > 0x7FFFFFFFull) return kInvalidConfiguration;
    const bf16* x = (const bf16*)input;
    const bf16* w = (const bf16*)weight;
    const bf16* b = (const bf16*)bias;
    bf16* y = (bf16*)output;
    const bool aligned = (((uintptr_t)x | (uintptr_t)w | (uintptr_t)y |
                           (uintptr_t)(b ? b : w)) & 15u) == 0;
    const dim3 g((unsigned)grid), bl(NTH);
    if (aligned && D % 512 == 0 && D <= 4096) {
        switch (D / 512) {
#define LN_CASE(nv)                                                                            \
    case nv:                                                                                   \
        EFLA_LAUNCH("layernorm_fwd", fwd_reg_kernel<nv>, g, bl, stream, x, w, b, y, mean, rstd, \
                    (long)rows, eps);                                                          \
        return (int)hipPeekAtLastError();
            LN_CASE(1) LN_CASE(2) LN_CASE(3) LN_CASE(4) LN_CASE(5) LN_CASE(6) LN_CASE(7)
            LN_CASE(8)
#undef LN_CASE
        }
    }
    EFLA_LAUNCH("layernorm_fwd_loop", fwd_loop_kernel, g, bl, stream, x, w, b, y, mean, rstd,
                (long)rows, (long)D, eps);
    return (int)hipPeekAtLastError();
}

}  // namespace ln
}  // namespace efla

using namespace efla;

extern "C" int layernorm_forward_hip(const void* input, const void* weight, const void* bias,
                                     void* output, size_t numel, size_t normalized_shape,
                                     float eps, hipStream_t stream) {
    return ln::forward(input, weight, bias, output, nullptr, nullptr, numel, normalized_shape,
                       eps, stream);
}

extern "C" int layernorm_forward_stats_hip(const void* input, const void* weight,
                                           const void* bias, void* output, float* mean,
                                           float* rstd, size_t numel, size_t normalized_shape,
                                           float eps, hipStream_t stream) {
    if (!mean || !rstd) return kInvalidValue;
    return ln::forward(input, weight, bias, output, mean, rstd, numel, normalized_shape, eps,
                       stream);
}

static int ln_backward(const void* grad_output, const void* input, const void* weight,
                       const float* mean, const float* rstd, const void* residual,
                       void* grad_input, void* grad_weight, void* grad_bias,
                       void* grad_input_colsum, size_t numel, size_t normalized_shape,
                       bool pbf, hipStream_t stream) {
    const size_t D = normalized_shape;
    if (D == 0) return kInvalidValue;
    const size_t rows = numel / D;
    const bool params = grad_weight || grad_bias;
    if (rows == 0) {
        const size_t pb = pbf ? 2 : 4;
        if (grad_weight) EFLA_CHECK((hipError_t)fill_zero(grad_weight, D * pb, stream));
        if (grad_bias) EFLA_CHECK((hipError_t)fill_zero(grad_bias, D * pb, stream));
        if (grad_input_colsum) EFLA_CHECK((hipError_t)fill_zero(grad_input_colsum, D * 2, stream));
        return kSuccess;
    }
    if (!grad_output || !input || !weight || !mean || !rstd || !grad_input) return kInvalidValue;
    if (((params || grad_input_colsum) && D > 8192) || rows > ((size_t)1 << 40))
        return kInvalidConfiguration;
    const bool aligned = ((uintptr_t)grad_output | (uintptr_t)input | (uintptr_t)weight |
                          (uintptr_t)grad_input | (uintptr_t)residual) % 16 == 0;
    const int nv = (aligned && D % 512 == 0 && D <= 2048) ? (int)(D / 512) : 0;
    // the register path sums dx's columns with dw and db (a third partial);
    // the looped path sums them in a pass of their own afterwards
    const int ns = (nv && grad_input_colsum) ? 3 : 2;
    const bool parts = params || ns == 3;
    // two workgroups per CU; each wave then takes several rows, which keeps the
    // per-workgroup dw/db partials (and their reduction) small
    size_t nblk = (rows + 3) / 4;
    if (nblk > 512) nblk = 512;
    float* part = nullptr;
    WsLease lease;
    if (parts) {
        void* ws = nullptr;
        int rc = workspace_acquire(nblk * ns * D * sizeof(float), stream, &ws, lease);
        if (rc != kSuccess) return rc;
        part = (float*)ws;
    }
    const bf16 *g = (const bf16*)grad_output, *x = (const bf16*)input, *w = (const bf16*)weight;
    const bf16* res = (const bf16*)residual;
    bf16* dx = (bf16*)grad_input;
    const dim3 grid((unsigned)nblk), block(ln::NTH);
    switch (nv * 4 + ns) {
#define LN_BWD_CASE(n, s)                                                                        \
    case n * 4 + s:                                                                              \
        EFLA_LAUNCH("layernorm_bwd", (ln::bwd_reg_kernel<n, s>), grid, block, stream, g, x, w, mean, \
                    rstd, res, dx, part, (long)rows, parts ? 1 : 0);                              \
        break;
        LN_BWD_CASE(1, 2) LN_BWD_CASE(2, 2) LN_BWD_CASE(3, 2) LN_BWD_CASE(4, 2)
        LN_BWD_CASE(1, 3) LN_BWD_CASE(2, 3) LN_BWD_CASE(3, 3) LN_BWD_CASE(4, 3)
#undef LN_BWD_CASE
        default: {
            // per-wave dw/db slices (timing-independent sums) while they fit
            // in 64 KB of LDS
            const bool per_wave = params && D <= 2048;
            const size_t smem =
                params ? (per_wave ? (ln::NTH / kWave) : 1) * 2 * D * sizeof(float) : 0;
            ::efla::ProfScope ps("layernorm_bwd_loop", stream);
            hipLaunchKernelGGL(ln::bwd_kernel, grid, block, smem, stream, g, x, w, mean, rstd, res,
                               dx, part, (long)rows, (int)D, params ? 1 : 0, per_wave ? 1 : 0);
        }
    }
    EFLA_CHECK(hipPeekAtLastError());
    if (parts) {
        const unsigned gr = (unsigned)((ns * D + 15) / 16);
        EFLA_LAUNCH("layernorm_bwd_reduce", ln::reduce_kernel, dim3(gr), dim3(ln::NTH), stream,
                    (const float*)part, (int)nblk, (int)D, ns, grad_weight, grad_bias, pbf ? 1 : 0,
                    ns == 3 ? (bf16*)grad_input_colsum : (bf16*)nullptr);
    }
    if (grad_input_colsum && ns == 2) {
        // the column pass leases this stream's workspace itself: hand back the
        // partials' lease first (its kernels are already queued on the stream)
        lease.release();
        EFLA_CHECK((hipError_t)colsum_bf16_rows(dx, (long)rows, (long)D, (bf16*)grad_input_colsum,
                                                stream));
    }
    return (int)hipPeekAtLastError();
}

extern "C" int layernorm_backward_hip(const void* grad_output, const void* input,
                                      const void* weight, const float* mean, const float* rstd,
                                      void* grad_input, float* grad_weight, float* grad_bias,
                                      size_t numel, size_t normalized_shape,
                                      hipStream_t stream) {
    return ln_backward(grad_output, input, weight, mean, rstd, nullptr, grad_input, grad_weight,
                       grad_bias, nullptr, numel, normalized_shape, false, stream);
}

extern "C" int layernorm_backward_residual_hip(const void* grad_output, const void* input,
                                               const void* weight, const float* mean,
                                               const float* rstd, const void* residual,
                                               void* grad_input, float* grad_weight,
                                               float* grad_bias, size_t numel,
                                               size_t normalized_shape, hipStream_t stream) {
    if (!residual && numel / (normalized_shape ? normalized_shape : 1) > 0) return kInvalidValue;
    return ln_backward(grad_output, input, weight, mean, rstd, residual, grad_input, grad_weight,
                       grad_bias, nullptr, numel, normalized_shape, false, stream);
}

extern "C" int layernorm_backward_ex_hip(const void* grad_output, const void* input,
                                         const void* weight, const float* mean, const float* rstd,
                                         const void* residual, void* grad_input,
                                         void* grad_weight, void* grad_bias,
                                         void* grad_input_colsum, size_t numel,
                                         size_t normalized_shape, int param_grads_bf16,
                                         hipStream_t stream) {
    return ln_backward(grad_output, input, weight, mean, rstd, residual, grad_input, grad_weight,
                       grad_bias, grad_input_colsum, numel, normalized_shape,
                       param_grads_bf16 != 0, stream);
}
