// ShortConv (causal depthwise convolution) and the PRISM refinement that
// consumes the EFLA output, for gfx950.
//
// ShortConv forward (replaces shortconv_forward_cuda, kernels.h:107-116, which
// is declared only; the executed semantics are ShortConv.forwardCpu,
// src/model/prism.zig:448-473):
//   y[b,t,c] = bf16( sum over w = 0..W-1 with t-w >= 0 of x[b,t-w,c] * weight[c,w] )
// with every product rounded to fp32 and the terms added in increasing w, as
// the reference loop does (no fused multiply-add), so the output is
// bit-identical to it.
// ShortConv backward (shortConvBackwardCuda, src/kernels/prism_kernels.zig:
// 50-60, declared only, no body anywhere):
//   grad_input[b,t,c] = sum over w with t+w < T of dy[b,t+w,c] weight[c,w]  (bf16)
//   grad_weight[c,w] += sum over b, t >= w of dy[b,t,c] x[b,t-w,c]          (fp32)
//
// PRISM forward (replaces prism_forward_cuda, kernels.h:86-102, declared only;
// the executed semantics are PrismLayer.prismForwardCpu, prism.zig:251-323):
// for every token row and channel d < head_dim,
//   r = v - u;  for l = 0..L-1:  x = p_l[d] r,  delta = GELU_tanh(x),
//               o = bf16(o + 0.5 delta),  r = r - delta,
// where p_l holds the first head_dim entries of w_p[l]; output channels
// d >= head_dim are 0.  That path reads neither w_beta, w_k, prev_state nor
// alpha and leaves the new state at zero; so does this one (new_state, a
// head_dim x head_dim bf16 matrix, is zero-filled when given).
// PRISM backward (no usable counterpart: prismBackwardCuda,
// prism_kernels.zig:24-37, takes no weights, and PrismLayer.backward,
// prism.zig:326-356, returns zeros): the gradient of the forward above with
// the bf16 rounding of o passed straight through,
//   gd_l = 0.5 g - a_{l+1},  gx_l = gd_l GELU'(x_l),  a_l = a_{l+1} + gx_l p_l,
//   a_L = 0,  grad_v = a_0,  grad_u = -a_0,  grad_w_p[l][d] += sum_rows gx_l r_l.
//
// Layout.  The ShortConv kernels tile 64 channels x 64 tokens per workgroup
// with the token rows and the weights staged as fp32 in LDS: one lane per
// channel, one wave per 16 tokens.  A lane keeps 16 outputs (or 16 lags) and
// walks the window in blocks of 16 lags, reading 31 staged values and 16
// weights for 256 multiply-adds.  Windows longer than 80 take direct kernels
// that read through the caches.  The weight gradient splits the token tiles
// over workgroups; each writes a partial, which a second pass sums in a fixed
// order into grad_weight.  PRISM runs one lane per channel over blocks of 32
// rows.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/efla_hip.h"
#include "common.hpp"
#include "gelu.hpp"
#include "internal.hpp"

namespace efla {
namespace prism {

using ::efla::gelu::gelu_df;
using ::efla::gelu::gelu_f;

constexpr int NTH = 256;
constexpr int CT = 64;   // channels per tile, one per lane
constexpr int TT = 64;   // tokens per tile, 16 per wave
constexpr int JB = 16;   // outputs (or lags) per lane and lag block
constexpr int kMaxTiledW = 80;  // keeps every tile within 64 KiB of LDS
constexpr int kMaxLagBlocks = kMaxTiledW / JB;
constexpr int kMaxIter = 16;
constexpr int RB = 32;  // PRISM rows per workgroup
constexpr long kMaxBlocks = 16384;

struct WPtrs {
    const bf16* p[kMaxIter];
};

__device__ __forceinline__ int padded_window(int W) { return (W + JB - 1) & ~(JB - 1); }

// dst[r][c] = src[b, t_lo + r, c0 + c] as fp32, 0 outside [0, T) x [0, C)
__device__ __forceinline__ void stage_rows(float* dst, const bf16* __restrict__ src, long b,
                                           long t_lo, int nrows, int T, int C, int c0) {
    for (int i = threadIdx.x; i < nrows * CT; i += NTH) {
        const int r = i / CT, c = i % CT;
        const long t = t_lo + r;
        float val = 0.f;
        if (t >= 0 && t < T && c0 + c < C) val = (float)src[(b * T + t) * C + c0 + c];
        dst[r * CT + c] = val;
    }
}

// ws[w][c] (row stride CT + 1) = weight[c0 + c][w], 0 for w >= W or c >= C
__device__ __forceinline__ void stage_weights(float* ws, const bf16* __restrict__ wt, int W, int Wp,
                                              int C, int c0) {
    for (int i = threadIdx.x; i < CT * Wp; i += NTH) {
        const int c = i / Wp, w = i % Wp;
        ws[w * (CT + 1) + c] = (w < W && c0 + c < C) ? (float)wt[(long)(c0 + c) * W + w] : 0.f;
    }
}

// y = ShortConv(x) for one 64 x 64 tile; grid (token tiles, channel tiles, B)
template <bool EDGE>
__device__ __forceinline__ void conv_fwd_lane(float (&acc)[JB], const float* xs, const float* ws,
                                              int W, int Wp, int g, int c, int tj0) {
#pragma clang fp contract(off)
    for (int w0 = 0; w0 < Wp; w0 += JB) {
        // xr[m] = x[tj0 + m - (JB-1) - w0]
        const int rbase = g * JB - (JB - 1) - w0 + (Wp - 1);
        float xr[2 * JB - 1], wv[JB];
#pragma unroll
        for (int m = 0; m < 2 * JB - 1; ++m) xr[m] = xs[(rbase + m) * CT + c];
#pragma unroll
        for (int k = 0; k < JB; ++k) wv[k] = ws[(w0 + k) * (CT + 1) + c];
#pragma unroll
        for (int k = 0; k < JB; ++k) {
            if (w0 + k < W) {
#pragma unroll
                for (int j = 0; j < JB; ++j) {
                    const float p = xr[j - k + JB - 1] * wv[k];
                    if (EDGE)
                        acc[j] = (tj0 + j - w0 - k >= 0) ? acc[j] + p : acc[j];
                    else
                        acc[j] = acc[j] + p;
                }
            }
        }
    }
}

__global__ void __launch_bounds__(NTH) conv_fwd_kernel(const bf16* __restrict__ x,
                                                       const bf16* __restrict__ wt,
                                                       bf16* __restrict__ y, int T, int C, int W) {
    extern __shared__ float smem[];
    const int Wp = padded_window(W);
    const int nrows = TT + Wp - 1;
    float* xs = smem;                // [nrows][CT]: tokens t0 - (Wp-1) ..
    float* ws = smem + nrows * CT;   // [Wp][CT + 1]
    const long b = blockIdx.z;
    const int t0 = blockIdx.x * TT, c0 = blockIdx.y * CT;
    stage_rows(xs, x, b, (long)t0 - (Wp - 1), nrows, T, C, c0);
    stage_weights(ws, wt, W, Wp, C, c0);
    __syncthreads();
    const int c = lane_id(), g = __builtin_amdgcn_readfirstlane(wave_id());
    const int tj0 = t0 + g * JB;
    float acc[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) acc[j] = 0.f;
    if (tj0 < W - 1)
        conv_fwd_lane<true>(acc, xs, ws, W, Wp, g, c, tj0);
    else
        conv_fwd_lane<false>(acc, xs, ws, W, Wp, g, c, tj0);
    if (c0 + c < C) {
#pragma unroll
        for (int j = 0; j < JB; ++j)
            if (tj0 + j < T) y[(b * T + tj0 + j) * C + c0 + c] = (bf16)acc[j];
    }
}

// windows beyond the tiled limit: one output per lane, reads through the caches
__global__ void __launch_bounds__(NTH) conv_fwd_direct_kernel(const bf16* __restrict__ x,
                                                              const bf16* __restrict__ wt,
                                                              bf16* __restrict__ y, long n, int T,
                                                              int C, int W) {
#pragma clang fp contract(off)
    for (long i = (long)blockIdx.x * NTH + threadIdx.x; i < n; i += (long)gridDim.x * NTH) {
        const int c = (int)(i % C);
        const long bt = i / C;
        const int t = (int)(bt % T);
        const int wmax = min(W - 1, t);
        float s = 0.f;
        for (int w = 0; w <= wmax; ++w) s = s + (float)x[(bt - w) * C + c] * (float)wt[(long)c * W + w];
        y[i] = (bf16)s;
    }
}

// grad_input for one tile: dx[t] = sum_w dy[t + w] weight[w]
__global__ void __launch_bounds__(NTH) conv_dx_kernel(const bf16* __restrict__ dy,
                                                      const bf16* __restrict__ wt,
                                                      bf16* __restrict__ dx, int T, int C, int W) {
    extern __shared__ float smem[];
    const int Wp = padded_window(W);
    const int nrows = TT + Wp - 1;
    float* ds = smem;               // [nrows][CT]: tokens t0 ..
    float* ws = smem + nrows * CT;  // [Wp][CT + 1]
    const long b = blockIdx.z;
    const int t0 = blockIdx.x * TT, c0 = blockIdx.y * CT;
    stage_rows(ds, dy, b, t0, nrows, T, C, c0);
    stage_weights(ws, wt, W, Wp, C, c0);
    __syncthreads();
    const int c = lane_id(), g = __builtin_amdgcn_readfirstlane(wave_id());
    float acc[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) acc[j] = 0.f;
    for (int w0 = 0; w0 < Wp; w0 += JB) {
        float dr[2 * JB - 1], wv[JB];
#pragma unroll
        for (int m = 0; m < 2 * JB - 1; ++m) dr[m] = ds[(g * JB + w0 + m) * CT + c];
#pragma unroll
        for (int k = 0; k < JB; ++k) wv[k] = ws[(w0 + k) * (CT + 1) + c];
#pragma unroll
        for (int k = 0; k < JB; ++k)
#pragma unroll
            for (int j = 0; j < JB; ++j) acc[j] = fmaf(dr[j + k], wv[k], acc[j]);
    }
    const int tj0 = t0 + g * JB;
    if (c0 + c < C) {
#pragma unroll
        for (int j = 0; j < JB; ++j)
            if (tj0 + j < T) dx[(b * T + tj0 + j) * C + c0 + c] = (bf16)acc[j];
    }
}

__global__ void __launch_bounds__(NTH) conv_dx_direct_kernel(const bf16* __restrict__ dy,
                                                             const bf16* __restrict__ wt,
                                                             bf16* __restrict__ dx, long n, int T,
                                                             int C, int W) {
    for (long i = (long)blockIdx.x * NTH + threadIdx.x; i < n; i += (long)gridDim.x * NTH) {
        const int c = (int)(i % C);
        const long bt = i / C;
        const int t = (int)(bt % T);
        const int wmax = min(W - 1, T - 1 - t);
        float s = 0.f;
        for (int w = 0; w <= wmax; ++w) s = fmaf((float)dy[(bt + w) * C + c], (float)wt[(long)c * W + w], s);
        dx[i] = (bf16)s;
    }
}

// part[split][c][w] = sum over this split's token tiles of dy[t] x[t - w].
// Wave g takes tokens 16g..16g+15 of every tile for all lags; the four waves'
// sums are added in LDS in wave order at the end.
__global__ void __launch_bounds__(NTH) conv_dw_kernel(const bf16* __restrict__ dy,
                                                      const bf16* __restrict__ x,
                                                      float* __restrict__ part, int B, int T,
                                                      int C, int W, int tiles_t) {
    extern __shared__ float smem[];
    const int Wp = padded_window(W);
    const int nlb = Wp / JB;
    const int nrx = TT + Wp - 1;
    float* xs = smem;             // [nrx][CT]: tokens t0 - (Wp-1) ..
    float* ds = xs + nrx * CT;    // [TT][CT]: tokens t0 ..
    const int c0 = blockIdx.x * CT;
    const int c = lane_id(), g = __builtin_amdgcn_readfirstlane(wave_id());
    float acc[kMaxLagBlocks][JB];
#pragma unroll
    for (int q = 0; q < kMaxLagBlocks; ++q)
#pragma unroll
        for (int k = 0; k < JB; ++k) acc[q][k] = 0.f;
    const long ntiles = (long)B * tiles_t;
    for (long tile = blockIdx.y; tile < ntiles; tile += gridDim.y) {
        const long b = tile / tiles_t;
        const int t0 = (int)(tile % tiles_t) * TT;
        __syncthreads();
        stage_rows(xs, x, b, (long)t0 - (Wp - 1), nrx, T, C, c0);
        stage_rows(ds, dy, b, t0, TT, T, C, c0);
        __syncthreads();
        float dr[JB];
#pragma unroll
        for (int j = 0; j < JB; ++j) dr[j] = ds[(g * JB + j) * CT + c];
#pragma unroll
        for (int q = 0; q < kMaxLagBlocks; ++q) {
            if (q < nlb) {
                const int w0 = q * JB;
                // xr[m] = x[t0 + 16g + m - (JB-1) - w0]
                const int rbase = g * JB - (JB - 1) - w0 + (Wp - 1);
                float xr[2 * JB - 1];
#pragma unroll
                for (int m = 0; m < 2 * JB - 1; ++m) xr[m] = xs[(rbase + m) * CT + c];
#pragma unroll
                for (int j = 0; j < JB; ++j)
#pragma unroll
                    for (int k = 0; k < JB; ++k) acc[q][k] = fmaf(dr[j], xr[j - k + JB - 1], acc[q][k]);
            }
        }
    }
    // add the four waves' sums: red[w][c], wave 0 writes, waves 1..3 add in turn
    __syncthreads();
    float* red = smem;  // [Wp][CT]
    for (int turn = 0; turn < NTH / kWave; ++turn) {
        if (g == turn) {
#pragma unroll
            for (int q = 0; q < kMaxLagBlocks; ++q) {
                if (q < nlb) {
#pragma unroll
                    for (int k = 0; k < JB; ++k) {
                        float* r = &red[(q * JB + k) * CT + c];
                        *r = turn == 0 ? acc[q][k] : *r + acc[q][k];
                    }
                }
            }
        }
        __syncthreads();
    }
    for (int i = threadIdx.x; i < CT * W; i += NTH) {
        const int cc = i / W, w = i % W;
        if (c0 + cc < C) part[((long)blockIdx.y * C + c0 + cc) * W + w] = red[w * CT + cc];
    }
}

// windows beyond the tiled limit: one (c, w) per lane over a slice of the rows
__global__ void __launch_bounds__(NTH) conv_dw_direct_kernel(const bf16* __restrict__ dy,
                                                             const bf16* __restrict__ x,
                                                             float* __restrict__ part, int B,
                                                             int T, int C, int W) {
    const long cw = (long)C * W;
    const long i = (long)blockIdx.x * NTH + threadIdx.x;
    if (i >= cw) return;
    const int c = (int)(i / W), w = (int)(i % W);
    const long rows = (long)B * T;
    const long per = (rows + gridDim.y - 1) / gridDim.y;
    const long r0 = (long)blockIdx.y * per, r1 = min(rows, r0 + per);
    float s = 0.f;
    for (long r = r0; r < r1; ++r) {
        const int t = (int)(r % T);
        if (t >= w) s = fmaf((float)dy[r * C + c], (float)x[(r - w) * C + c], s);
    }
    part[(long)blockIdx.y * cw + i] = s;
}

// out[i] += sum_s part[s][i], s in order
__global__ void __launch_bounds__(NTH) sum_parts_kernel(const float* __restrict__ part, int nsplit,
                                                        long n, long stride,
                                                        float* __restrict__ out) {
    for (long i = (long)blockIdx.x * NTH + threadIdx.x; i < n; i += (long)gridDim.x * NTH) {
        float s = 0.f;
        for (int k = 0; k < nsplit; ++k) s += part[(long)k * stride + i];
        out[i] += s;
    }
}

// ---------------------------------------------------------------------------
// PRISM
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(NTH) prism_fwd_kernel(const bf16* __restrict__ u,
                                                        const bf16* __restrict__ v, WPtrs wp,
                                                        bf16* __restrict__ out, long rows, int C,
                                                        int HD, int L) {
    const int c = blockIdx.y * NTH + threadIdx.x;
    if (c >= C) return;
    const long r0 = (long)blockIdx.x * RB, r1 = min(rows, r0 + RB);
    if (c >= HD) {
        for (long r = r0; r < r1; ++r) out[r * C + c] = (bf16)0.f;
        return;
    }
    float p[kMaxIter];
#pragma unroll
    for (int l = 0; l < kMaxIter; ++l) p[l] = l < L ? (float)wp.p[l][c] : 0.f;
    for (long r = r0; r < r1; ++r) {
        float res = (float)v[r * C + c] - (float)u[r * C + c];
        float o = 0.f;
#pragma unroll
        for (int l = 0; l < kMaxIter; ++l) {
            if (l < L) {
                const float d = gelu_f<true>(p[l] * res);
                o = (float)(bf16)(o + 0.5f * d);
                res -= d;
            }
        }
        out[r * C + c] = (bf16)o;
    }
}

// part[blk][l][c] (c < HD) = this block's sum over rows of gx_l r_l
__global__ void __launch_bounds__(NTH) prism_bwd_kernel(const bf16* __restrict__ go,
                                                        const bf16* __restrict__ u,
                                                        const bf16* __restrict__ v, WPtrs wp,
                                                        bf16* __restrict__ gu,
                                                        bf16* __restrict__ gv,
                                                        float* __restrict__ part, long rows,
                                                        int C, int HD, int L) {
    const int c = blockIdx.y * NTH + threadIdx.x;
    if (c >= C) return;
    const long r0 = (long)blockIdx.x * RB, r1 = min(rows, r0 + RB);
    if (c >= HD) {
        for (long r = r0; r < r1; ++r) {
            gu[r * C + c] = (bf16)0.f;
            gv[r * C + c] = (bf16)0.f;
        }
        return;
    }
    float p[kMaxIter], dp[kMaxIter];
#pragma unroll
    for (int l = 0; l < kMaxIter; ++l) {
        p[l] = l < L ? (float)wp.p[l][c] : 0.f;
        dp[l] = 0.f;
    }
    for (long r = r0; r < r1; ++r) {
        float res[kMaxIter], xl[kMaxIter];
        float rr = (float)v[r * C + c] - (float)u[r * C + c];
#pragma unroll
        for (int l = 0; l < kMaxIter; ++l) {
            res[l] = rr;
            xl[l] = p[l] * rr;
            if (l < L) rr -= gelu_f<true>(xl[l]);
        }
        const float g = (float)go[r * C + c];
        float a = 0.f;
#pragma unroll
        for (int l = kMaxIter - 1; l >= 0; --l) {
            if (l < L) {
                const float gx = (0.5f * g - a) * gelu_df<true>(xl[l]);
                dp[l] = fmaf(gx, res[l], dp[l]);
                a = fmaf(gx, p[l], a);
            }
        }
        gv[r * C + c] = (bf16)a;
        gu[r * C + c] = (bf16)(-a);
    }
    if (part) {
#pragma unroll
        for (int l = 0; l < kMaxIter; ++l)
            if (l < L) part[((long)blockIdx.x * L + l) * HD + c] = dp[l];
    }
}

inline size_t conv_lds_bytes(int W, bool dw) {
    const int Wp = (W + JB - 1) & ~(JB - 1);
    const size_t rows = (size_t)(TT + Wp - 1) + (dw ? TT : 0);
    const size_t a = rows * CT * sizeof(float);
    const size_t wts = dw ? 0 : (size_t)Wp * (CT + 1) * sizeof(float);
    return a + wts;
}

inline unsigned grid_1d(long n) {
    long g = (n + NTH - 1) / NTH;
    return (unsigned)(g < 1 ? 1 : (g > kMaxBlocks ? kMaxBlocks : g));
}

}  // namespace prism
}  // namespace efla

using namespace efla;

namespace {

int conv_check(size_t B, size_t T, size_t C, size_t W) {
    if (B * T * C > ((size_t)1 << 40) || T > 0x7FFFFFFFull || C > 0x7FFFFFFFull ||
        W > ((size_t)1 << 20) || C * W > 0x7FFFFFFFull || B > 65535)
        return kInvalidConfiguration;
    return kSuccess;
}

}  // namespace

extern "C" int shortconv_forward_hip(const void* input, const void* weight, void* output,
                                     size_t batch_size, size_t seq_len, size_t hidden_dim,
                                     size_t window_size, hipStream_t stream) {
    const size_t n = batch_size * seq_len * hidden_dim;
    if (n == 0) return kSuccess;
    if (!input || !output || (window_size > 0 && !weight)) return kInvalidValue;
    const int rc = conv_check(batch_size, seq_len, hidden_dim, window_size);
    if (rc != kSuccess) return rc;
    const bf16* x = (const bf16*)input;
    const bf16* wt = (const bf16*)weight;
    bf16* y = (bf16*)output;
    const int T = (int)seq_len, C = (int)hidden_dim, W = (int)window_size;
    if (W >= 1 && W <= prism::kMaxTiledW) {
        const dim3 grid((unsigned)((T + prism::TT - 1) / prism::TT),
                        (unsigned)((C + prism::CT - 1) / prism::CT), (unsigned)batch_size);
        ::efla::ProfScope ps("shortconv_fwd", stream);
        hipLaunchKernelGGL(prism::conv_fwd_kernel, grid, dim3(prism::NTH),
                           prism::conv_lds_bytes(W, false), stream, x, wt, y, T, C, W);
    } else {
        EFLA_LAUNCH("shortconv_fwd_direct", prism::conv_fwd_direct_kernel,
                    dim3(prism::grid_1d((long)n)), dim3(prism::NTH), stream, x, wt, y, (long)n, T,
                    C, W);
    }
    return (int)hipPeekAtLastError();
}

extern "C" int shortconv_backward_hip(const void* grad_output, const void* input,
                                      const void* weight, void* grad_input, float* grad_weight,
                                      size_t batch_size, size_t seq_len, size_t hidden_dim,
                                      size_t window_size, hipStream_t stream) {
    const size_t n = batch_size * seq_len * hidden_dim;
    if (n == 0 || window_size == 0) {
        if (n > 0 && grad_input) return fill_zero(grad_input, n * sizeof(bf16), stream);
        return kSuccess;
    }
    if (!grad_output || !weight || (grad_weight && !input)) return kInvalidValue;
    const int rc = conv_check(batch_size, seq_len, hidden_dim, window_size);
    if (rc != kSuccess) return rc;
    const bf16* dy = (const bf16*)grad_output;
    const bf16* x = (const bf16*)input;
    const bf16* wt = (const bf16*)weight;
    const int B = (int)batch_size, T = (int)seq_len, C = (int)hidden_dim, W = (int)window_size;
    const bool tiled = W <= prism::kMaxTiledW;
    const int ctiles = (C + prism::CT - 1) / prism::CT;
    const int ttiles = (T + prism::TT - 1) / prism::TT;
    if (grad_input) {
        bf16* dx = (bf16*)grad_input;
        if (tiled) {
            const dim3 grid((unsigned)ttiles, (unsigned)ctiles, (unsigned)B);
            ::efla::ProfScope ps("shortconv_dx", stream);
            hipLaunchKernelGGL(prism::conv_dx_kernel, grid, dim3(prism::NTH),
                               prism::conv_lds_bytes(W, false), stream, dy, wt, dx, T, C, W);
        } else {
            EFLA_LAUNCH("shortconv_dx_direct", prism::conv_dx_direct_kernel,
                        dim3(prism::grid_1d((long)n)), dim3(prism::NTH), stream, dy, wt, dx,
                        (long)n, T, C, W);
        }
        EFLA_CHECK(hipPeekAtLastError());
    }
    if (grad_weight) {
        const long cw = (long)C * W;
        long nsplit;
        if (tiled) {
            const long tiles = (long)B * ttiles;
            nsplit = std::max(1L, std::min({tiles, 256L, 1024L / ctiles}));
        } else {
            nsplit = std::max(1L, std::min((long)B * T, 4096L / (long)prism::grid_1d(cw)));
        }
        void* ws = nullptr;
        const int wrc = workspace_acquire((size_t)nsplit * cw * sizeof(float), stream, &ws);
        if (wrc != kSuccess) return wrc;
        float* part = (float*)ws;
        if (tiled) {
            ::efla::ProfScope ps("shortconv_dw", stream);
            hipLaunchKernelGGL(prism::conv_dw_kernel, dim3((unsigned)ctiles, (unsigned)nsplit),
                               dim3(prism::NTH), prism::conv_lds_bytes(W, true), stream, dy, x,
                               part, B, T, C, W, ttiles);
        } else {
            EFLA_LAUNCH("shortconv_dw_direct", prism::conv_dw_direct_kernel,
                        dim3((unsigned)((cw + prism::NTH - 1) / prism::NTH), (unsigned)nsplit),
                        dim3(prism::NTH), stream, dy, x, part, B, T, C, W);
        }
        EFLA_CHECK(hipPeekAtLastError());
        EFLA_LAUNCH("shortconv_dw_sum", prism::sum_parts_kernel, dim3(prism::grid_1d(cw)),
                    dim3(prism::NTH), stream, (const float*)part, (int)nsplit, cw, cw,
                    grad_weight);
    }
    return (int)hipPeekAtLastError();
}

namespace {

int prism_check(size_t B, size_t T, size_t hidden, size_t head_dim, size_t L,
                const void* const* w_p, prism::WPtrs* wp) {
    if (hidden == 0 || head_dim == 0 || head_dim > hidden) return kInvalidValue;
    if (L > (size_t)prism::kMaxIter || B * T * hidden > ((size_t)1 << 40) ||
        hidden > 0x7FFFFFFFull)
        return kInvalidConfiguration;
    if (L > 0 && !w_p) return kInvalidValue;
    for (size_t l = 0; l < (size_t)prism::kMaxIter; ++l) {
        wp->p[l] = l < L ? (const bf16*)w_p[l] : nullptr;
        if (l < L && !wp->p[l]) return kInvalidValue;
    }
    return kSuccess;
}

}  // namespace

extern "C" int prism_forward_hip(const void* u, const void* v, const void* prev_state,
                                 void* new_state, void* output, const void** w_beta,
                                 const void** w_k, const void** w_p, size_t batch_size,
                                 size_t seq_len, size_t hidden_dim, size_t head_dim,
                                 size_t num_iterations, float alpha, hipStream_t stream) {
    (void)prev_state;
    (void)w_beta;
    (void)w_k;
    (void)alpha;
    prism::WPtrs wp;
    int rc = prism_check(batch_size, seq_len, hidden_dim, head_dim, num_iterations, w_p, &wp);
    if (rc != kSuccess) return rc;
    const long rows = (long)(batch_size * seq_len);
    if (rows > 0 && (!u || !v || !output)) return kInvalidValue;
    if (new_state) {
        rc = fill_zero(new_state, head_dim * head_dim * sizeof(bf16), stream);
        if (rc != kSuccess) return rc;
    }
    if (rows == 0) return kSuccess;
    const dim3 grid((unsigned)((rows + prism::RB - 1) / prism::RB),
                    (unsigned)((hidden_dim + prism::NTH - 1) / prism::NTH));
    if (grid.x > 0x7FFFFFFFu) return kInvalidConfiguration;
    EFLA_LAUNCH("prism_fwd", prism::prism_fwd_kernel, grid, dim3(prism::NTH), stream,
                (const bf16*)u, (const bf16*)v, wp, (bf16*)output, rows, (int)hidden_dim,
                (int)head_dim, (int)num_iterations);
    return (int)hipPeekAtLastError();
}

extern "C" int prism_backward_hip(const void* grad_output, const void* u, const void* v,
                                  const void** w_p, void* grad_u, void* grad_v,
                                  float** grad_w_p, size_t batch_size, size_t seq_len,
                                  size_t hidden_dim, size_t head_dim, size_t num_iterations,
                                  hipStream_t stream) {
    prism::WPtrs wp;
    int rc = prism_check(batch_size, seq_len, hidden_dim, head_dim, num_iterations, w_p, &wp);
    if (rc != kSuccess) return rc;
    const long rows = (long)(batch_size * seq_len);
    if (rows == 0) return kSuccess;
    if (!grad_output || !u || !v || !grad_u || !grad_v) return kInvalidValue;
    const int L = (int)num_iterations;
    if (grad_w_p)
        for (int l = 0; l < L; ++l)
            if (!grad_w_p[l]) return kInvalidValue;
    const dim3 grid((unsigned)((rows + prism::RB - 1) / prism::RB),
                    (unsigned)((hidden_dim + prism::NTH - 1) / prism::NTH));
    if (grid.x > 0x7FFFFFFFu) return kInvalidConfiguration;
    float* part = nullptr;
    const bool want_w = grad_w_p && L > 0;
    if (want_w) {
        void* ws = nullptr;
        rc = workspace_acquire((size_t)grid.x * L * head_dim * sizeof(float), stream, &ws);
        if (rc != kSuccess) return rc;
        part = (float*)ws;
    }
    EFLA_LAUNCH("prism_bwd", prism::prism_bwd_kernel, grid, dim3(prism::NTH), stream,
                (const bf16*)grad_output, (const bf16*)u, (const bf16*)v, wp, (bf16*)grad_u,
                (bf16*)grad_v, part, rows, (int)hidden_dim, (int)head_dim, L);
    EFLA_CHECK(hipPeekAtLastError());
    if (want_w) {
        for (int l = 0; l < L; ++l) {
            EFLA_LAUNCH("prism_bwd_sum", prism::sum_parts_kernel,
                        dim3(prism::grid_1d((long)head_dim)), dim3(prism::NTH), stream,
                        (const float*)(part + (size_t)l * head_dim), (int)grid.x, (long)head_dim,
                        (long)L * head_dim, grad_w_p[l]);
            EFLA_CHECK(hipPeekAtLastError());
        }
    }
    return kSuccess;
}
