// ShortConv (causal depthwise convolution) and the PRISM refinement that
// consumes the EFLA output, for gfx950.
//
// ShortConv forward (replaces shortconv_forward_cuda, kernels.h:107-116, which
// is declared only; the executed semantics are ShortConv.forwardCpu,
// src/model/prism.zig:448-473):
//   y[b,t,c] = bf16( sum over w = 0..W-1 with t-w >= 0 of x[b,t-w,c] * weight[c,w] )
// with the terms added in fp32 in increasing w, as the reference loop does, so
// the output is bit-identical to it.  The product of two bf16 values has at
// most 16 significant bits and is exact in fp32 (unless it falls below fp32's
// normal range), so a fused multiply-add rounds exactly as the reference's
// separate multiply and add.
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
// weights for 256 multiply-adds.  For 16-byte rows and windows up to 64 the
// forward and grad_input walk several consecutive token tiles per workgroup
// (about two workgroups per CU): the upper half of a tile's staged rows is
// the next tile's lower half, and the next 64 rows are loaded into registers
// while the tile is formed.  Windows longer than 80 take direct kernels that
// read through the caches.  The weight gradient splits the token tiles over
// workgroups (for 16-byte rows, runs of consecutive tiles with the next
// tile's rows loaded during the current one); each writes a partial, which a
// second pass sums in a fixed order into grad_weight.  PRISM, for 16-byte rows and up to four iterations
// (the reference config runs three), takes blocks of 16 rows per workgroup:
// eight active channels per lane as one 16-byte piece of each input and
// output, and the columns past head_dim cleared by the same workgroup with
// 16-byte stores; the w_p gradient of a block is summed in LDS into a
// per-block partial, and a second kernel adds the partials in block order
// (the same result on every run).  Other shapes run one lane per active
// channel and one wave per row phase over blocks of 64 rows, with the columns
// cleared by a separate pass and the w_p gradient added with one float atomic
// per workgroup and value (the order of those additions varies between runs).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <initializer_list>

#include "../../include/efla_hip.h"
#include "common.hpp"
#include "gelu.hpp"
#include "internal.hpp"
#include "reduce.hpp"

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
constexpr int PRB = 64;  // PRISM rows per workgroup (16 per wave)
constexpr long kMaxBlocks = 16384;
constexpr int kDwPipeBlocks = 512;  // conv_dw_pipe_kernel workgroups (all splits)

struct WPtrs {
    const bf16* p[kMaxIter];
};
struct GPtrs {
    float* p[kMaxIter];
};

__device__ __forceinline__ int padded_window(int W) { return (W + JB - 1) & ~(JB - 1); }

constexpr int kStageIt = (TT + kMaxTiledW - 1 + 31) / 32;  // 16-byte row chunks per thread
constexpr int kStageEl = ((TT + kMaxTiledW - 1) * CT + NTH - 1) / NTH;  // scalar elements

// Rows t_lo .. t_lo + nrows - 1 (nrows <= 32 IT) of channels c0 .. c0 + 63 as
// 16-byte pieces held in registers (thread: channel group threadIdx % 8, rows
// threadIdx / 8 + 32 it), 0 outside [0, T) x [0, C); store() writes them to
// LDS as fp32 [row][CT].
template <int IT>
struct RowsVec {
    bf16x8 v[IT];
    __device__ __forceinline__ void load(const bf16* __restrict__ src, long b, long t_lo,
                                         int nrows, int T, int C, int c0) {
        const int q = threadIdx.x & 7, ro = threadIdx.x >> 3;
        const bool cok = c0 + q * 8 < C;
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int r = ro + 32 * it;
            const long t = t_lo + r;
            if (r < nrows && t >= 0 && t < T && cok) {
                v[it] = *reinterpret_cast<const bf16x8*>(src + (b * T + t) * C + c0 + q * 8);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[it][i] = (bf16)0.f;
            }
        }
    }
    __device__ __forceinline__ void store(float* dst, int nrows) const {
        const int q = threadIdx.x & 7, ro = threadIdx.x >> 3;
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int r = ro + 32 * it;
            if (r < nrows) {
                floatx4 lo, hi;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    lo[i] = (float)v[it][i];
                    hi[i] = (float)v[it][4 + i];
                }
                *reinterpret_cast<floatx4*>(&dst[r * CT + q * 8]) = lo;
                *reinterpret_cast<floatx4*>(&dst[r * CT + q * 8 + 4]) = hi;
            }
        }
    }
};

// dst[r][c] = src[b, t_lo + r, c0 + c] as fp32 for r < nrows, 0 outside
// [0, T) x [0, C).  Every load is issued before the first LDS write.  VEC:
// 16-byte loads of 8 channels (C % 8 == 0 and src 16-byte aligned).
template <bool VEC>
__device__ __forceinline__ void stage_rows(float* dst, const bf16* __restrict__ src, long b,
                                           long t_lo, int nrows, int T, int C, int c0) {
    if constexpr (VEC) {
        RowsVec<kStageIt> rv;
        rv.load(src, b, t_lo, nrows, T, C, c0);
        rv.store(dst, nrows);
    } else {
        float v[kStageEl];
#pragma unroll
        for (int k = 0; k < kStageEl; ++k) {
            const int i = threadIdx.x + k * NTH;
            const int r = i / CT, c = i % CT;
            const long t = t_lo + r;
            v[k] = (r < nrows && t >= 0 && t < T && c0 + c < C)
                       ? (float)src[(b * T + t) * C + c0 + c] : 0.f;
        }
#pragma unroll
        for (int k = 0; k < kStageEl; ++k) {
            const int i = threadIdx.x + k * NTH;
            if (i < nrows * CT) dst[i] = v[k];
        }
    }
}

// ws[w][c] (row stride CT + 1) = weight[c0 + c][w], 0 for w >= W or c >= C.
// The tile's weights are one contiguous run of 64 W values (rows c0..c0+63).
__device__ __forceinline__ void stage_weights(float* ws, const bf16* __restrict__ wt, int W, int Wp,
                                              int C, int c0) {
    const bf16* base = wt + (long)c0 * W;
    const int nvalid = min(CT, C - c0) * W;
    const bool vec = ((uintptr_t)wt & 15) == 0;
    constexpr int kIt = (CT * kMaxTiledW / 8 + NTH - 1) / NTH;
    bf16x8 v[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
        const int e = 8 * (threadIdx.x + it * NTH);
        if (vec && e + 8 <= nvalid) {
            v[it] = *reinterpret_cast<const bf16x8*>(base + e);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[it][i] = e + i < nvalid ? base[e + i] : (bf16)0.f;
        }
    }
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
        const int e = 8 * (threadIdx.x + it * NTH);
        if (e < CT * W) {
            int c = e / W, w = e - c * W;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                ws[w * (CT + 1) + c] = (float)v[it][i];
                if (++w == W) {
                    w = 0;
                    ++c;
                }
            }
        }
    }
    for (int i = threadIdx.x; i < (Wp - W) * CT; i += NTH) {
        const int w = W + i / CT, c = i % CT;
        ws[w * (CT + 1) + c] = 0.f;
    }
}

// y = ShortConv(x) for one 64 x 64 tile; grid (token tiles, channel tiles, B)
// One block of 16 lags starting at w0.  EDGE: some x index t - w may be
// negative (skip those terms, as the reference loop does); TAIL: lags at or
// beyond W exist in this block (skip them).
template <bool EDGE, bool TAIL>
__device__ __forceinline__ void conv_fwd_block(float (&acc)[JB], const float* xs, const float* ws,
                                               int W, int Wp, int g, int c, int tj0, int w0) {
    // xr[m] = x[tj0 + m - (JB-1) - w0]
    const int rbase = g * JB - (JB - 1) - w0 + (Wp - 1);
    float xr[2 * JB - 1], wv[JB];
#pragma unroll
    for (int m = 0; m < 2 * JB - 1; ++m) xr[m] = xs[(rbase + m) * CT + c];
#pragma unroll
    for (int k = 0; k < JB; ++k) wv[k] = ws[(w0 + k) * (CT + 1) + c];
#pragma unroll
    for (int k = 0; k < JB; ++k) {
        if (!TAIL || w0 + k < W) {
#pragma unroll
            for (int j = 0; j < JB; ++j) {
                const float s = fmaf(xr[j - k + JB - 1], wv[k], acc[j]);
                acc[j] = (!EDGE || tj0 + j - w0 - k >= 0) ? s : acc[j];
            }
        }
    }
}

__device__ __forceinline__ void conv_fwd_lane(float (&acc)[JB], const float* xs, const float* ws,
                                              int W, int Wp, int g, int c, int tj0) {
    const int wfull = W & ~(JB - 1);
    for (int w0 = 0; w0 < wfull; w0 += JB) {
        if (tj0 - w0 - (JB - 1) >= 0)
            conv_fwd_block<false, false>(acc, xs, ws, W, Wp, g, c, tj0, w0);
        else
            conv_fwd_block<true, false>(acc, xs, ws, W, Wp, g, c, tj0, w0);
    }
    if (wfull < W) {
        if (tj0 - wfull - (JB - 1) >= 0)
            conv_fwd_block<false, true>(acc, xs, ws, W, Wp, g, c, tj0, wfull);
        else
            conv_fwd_block<true, true>(acc, xs, ws, W, Wp, g, c, tj0, wfull);
    }
}

template <bool VEC>
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
    stage_rows<VEC>(xs, x, b, (long)t0 - (Wp - 1), nrows, T, C, c0);
    stage_weights(ws, wt, W, Wp, C, c0);
    __syncthreads();
    const int c = lane_id(), g = __builtin_amdgcn_readfirstlane(wave_id());
    const int tj0 = t0 + g * JB;
    float acc[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) acc[j] = 0.f;
    conv_fwd_lane(acc, xs, ws, W, Wp, g, c, tj0);
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
    for (long i = (long)blockIdx.x * NTH + threadIdx.x; i < n; i += (long)gridDim.x * NTH) {
        const int c = (int)(i % C);
        const long bt = i / C;
        const int t = (int)(bt % T);
        const int wmax = min(W - 1, t);
        float s = 0.f;
        for (int w = 0; w <= wmax; ++w) s = fmaf((float)x[(bt - w) * C + c], (float)wt[(long)c * W + w], s);
        y[i] = (bf16)s;
    }
}

// acc[j] = sum over lags w < Wp of ds[g JB + j + w][c] ws[w][c] (the rows past
// T and the lags past W are staged as zeros)
__device__ __forceinline__ void conv_dx_lane(float (&acc)[JB], const float* ds, const float* ws,
                                             int Wp, int g, int c) {
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
}

// grad_input for one tile: dx[t] = sum_w dy[t + w] weight[w]
template <bool VEC>
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
    stage_rows<VEC>(ds, dy, b, t0, nrows, T, C, c0);
    stage_weights(ws, wt, W, Wp, C, c0);
    __syncthreads();
    const int c = lane_id(), g = __builtin_amdgcn_readfirstlane(wave_id());
    float acc[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) acc[j] = 0.f;
    conv_dx_lane(acc, ds, ws, Wp, g, c);
    const int tj0 = t0 + g * JB;
    if (c0 + c < C) {
#pragma unroll
        for (int j = 0; j < JB; ++j)
            if (tj0 + j < T) dx[(b * T + tj0 + j) * C + c0 + c] = (bf16)acc[j];
    }
}

// The forward (DX false) or grad_input (DX true) over the token tiles
// [n0, n0 + tps) of one (channel tile, batch row), for 16-byte rows and
// windows of at most TT.  Tile n reads 64 + Wp - 1 staged rows, of which the
// upper 64 are tile n + 1's lower 64: the workgroup keeps 2 TT rows (row i =
// token t0 + OFF + i, OFF = -TT forward, 0 grad_input), and while a tile is
// formed each thread loads its share of the next tile's 64 new rows into
// registers; after the tile, each thread moves the pieces it is about to
// replace from the upper to the lower half and writes the new rows in their
// place (no thread touches another's pieces, so two barriers per tile).
// The per-output arithmetic is that of conv_fwd_kernel / conv_dx_kernel.
template <bool DX>
__global__ void __launch_bounds__(NTH) conv_walk_kernel(const bf16* __restrict__ src,
                                                        const bf16* __restrict__ wt,
                                                        bf16* __restrict__ dst, int T, int C,
                                                        int W, int tps) {
    extern __shared__ float smem[];
    constexpr int OFF = DX ? 0 : -TT;
    const int Wp = padded_window(W);
    float* rows = smem;                // [2 TT][CT]
    float* ws = smem + 2 * TT * CT;    // [Wp][CT + 1]
    const long b = blockIdx.y;
    const int c0 = blockIdx.x * CT;
    const int n0 = blockIdx.z * tps, n1 = min((T + TT - 1) / TT, n0 + tps);
    stage_rows<true>(rows, src, b, (long)n0 * TT + OFF, 2 * TT, T, C, c0);
    stage_weights(ws, wt, W, Wp, C, c0);
    __syncthreads();
    const int c = lane_id(), g = __builtin_amdgcn_readfirstlane(wave_id());
    const int q = threadIdx.x & 7, ro = threadIdx.x >> 3;
    const bool cok = c0 + 8 * q < C;
    for (int n = n0; n < n1; ++n) {
        const int t0 = n * TT;
        const bool more = n + 1 < n1;
        bf16x8 nx[2];
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const long t = (long)t0 + OFF + 2 * TT + ro + 32 * it;
            if (more && cok && t < T) {
                nx[it] = *reinterpret_cast<const bf16x8*>(src + (b * T + t) * C + c0 + 8 * q);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) nx[it][i] = (bf16)0.f;
            }
        }
        const int tj0 = t0 + g * JB;
        float acc[JB];
#pragma unroll
        for (int j = 0; j < JB; ++j) acc[j] = 0.f;
        if constexpr (DX)
            conv_dx_lane(acc, rows, ws, Wp, g, c);
        else
            conv_fwd_lane(acc, rows + (TT - (Wp - 1)) * CT, ws, W, Wp, g, c, tj0);
        if (c0 + c < C) {
#pragma unroll
            for (int j = 0; j < JB; ++j)
                if (tj0 + j < T) dst[(b * T + tj0 + j) * C + c0 + c] = (bf16)acc[j];
        }
        if (!more) break;
        __syncthreads();  // every wave is done with this tile's rows
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            float* up = rows + (TT + ro + 32 * it) * CT + 8 * q;
            float* lo = rows + (ro + 32 * it) * CT + 8 * q;
            const floatx4 a0 = *reinterpret_cast<const floatx4*>(up);
            const floatx4 a1 = *reinterpret_cast<const floatx4*>(up + 4);
            *reinterpret_cast<floatx4*>(lo) = a0;
            *reinterpret_cast<floatx4*>(lo + 4) = a1;
            floatx4 n0v, n1v;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                n0v[i] = (float)nx[it][i];
                n1v[i] = (float)nx[it][4 + i];
            }
            *reinterpret_cast<floatx4*>(up) = n0v;
            *reinterpret_cast<floatx4*>(up + 4) = n1v;
        }
        __syncthreads();
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
template <bool VEC>
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
        stage_rows<VEC>(xs, x, b, (long)t0 - (Wp - 1), nrx, T, C, c0);
        stage_rows<VEC>(ds, dy, b, t0, TT, T, C, c0);
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

// conv_dw_kernel for 16-byte rows with the token tiles of a split taken in
// order (tiles [blockIdx.y tpw, (blockIdx.y + 1) tpw) of the B x tiles_t
// sequence) and the next tile's x and dy rows loaded into registers while the
// current tile is formed, so the loads' latency is not paid once per tile.
__global__ void __launch_bounds__(NTH) conv_dw_pipe_kernel(const bf16* __restrict__ dy,
                                                           const bf16* __restrict__ x,
                                                           float* __restrict__ part, int B,
                                                           int T, int C, int W, int tiles_t,
                                                           int tpw) {
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
    const long tl0 = (long)blockIdx.y * tpw, tl1 = min(ntiles, tl0 + tpw);
    RowsVec<kStageIt> px;
    RowsVec<TT / 32> pd;
    auto load = [&](long tile) {
        const long b = tile / tiles_t;
        const int t0 = (int)(tile % tiles_t) * TT;
        px.load(x, b, (long)t0 - (Wp - 1), nrx, T, C, c0);
        pd.load(dy, b, t0, TT, T, C, c0);
    };
    if (tl0 < tl1) {
        load(tl0);
        px.store(xs, nrx);
        pd.store(ds, TT);
    }
    __syncthreads();
    for (long tile = tl0; tile < tl1; ++tile) {
        const bool more = tile + 1 < tl1;
        if (more) load(tile + 1);
        float dr[JB];
#pragma unroll
        for (int j = 0; j < JB; ++j) dr[j] = ds[(g * JB + j) * CT + c];
#pragma unroll
        for (int q = 0; q < kMaxLagBlocks; ++q) {
            if (q < nlb) {
                const int w0 = q * JB;
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
        if (more) {
            __syncthreads();
            px.store(xs, nrx);
            pd.store(ds, TT);
            __syncthreads();
        }
    }
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

// ---------------------------------------------------------------------------
// PRISM
// ---------------------------------------------------------------------------
// Lane = channel c = 64 blockIdx.y + lane (active when c < HD); wave g takes
// rows r0 + g, r0 + g + 4, ... of the block's PRB rows.
__global__ void __launch_bounds__(NTH) prism_fwd_kernel(const bf16* __restrict__ u,
                                                        const bf16* __restrict__ v, WPtrs wp,
                                                        bf16* __restrict__ out, long rows, int C,
                                                        int HD, int L) {
    const int c = blockIdx.y * kWave + lane_id();
    if (c >= HD) return;
    const int g = wave_id();
    const long r0 = (long)blockIdx.x * PRB;
    float p[kMaxIter];
#pragma unroll
    for (int l = 0; l < kMaxIter; ++l) p[l] = l < L ? (float)wp.p[l][c] : 0.f;
#pragma unroll 4
    for (int i = 0; i < PRB / 4; ++i) {
        const long r = r0 + g + 4 * i;
        if (r >= rows) break;
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

// grad_w_p[l][c] += this block's sum of gx_l r_l (one atomic add per block,
// so the order of the additions varies from run to run)
__global__ void __launch_bounds__(NTH) prism_bwd_kernel(const bf16* __restrict__ go,
                                                        const bf16* __restrict__ u,
                                                        const bf16* __restrict__ v, WPtrs wp,
                                                        bf16* __restrict__ gu,
                                                        bf16* __restrict__ gv, GPtrs gw,
                                                        long rows, int C, int HD, int L) {
    __shared__ float red[NTH / kWave][kMaxIter][kWave];
    const int lane = lane_id(), g = wave_id();
    const int c = blockIdx.y * kWave + lane;
    const bool active = c < HD;
    const long r0 = (long)blockIdx.x * PRB;
    float p[kMaxIter], dp[kMaxIter];
#pragma unroll
    for (int l = 0; l < kMaxIter; ++l) {
        p[l] = (active && l < L) ? (float)wp.p[l][c] : 0.f;
        dp[l] = 0.f;
    }
    if (active) {
#pragma unroll 2
        for (int i = 0; i < PRB / 4; ++i) {
            const long r = r0 + g + 4 * i;
            if (r >= rows) break;
            float res[kMaxIter], xl[kMaxIter];
            float rr = (float)v[r * C + c] - (float)u[r * C + c];
            const float gr = (float)go[r * C + c];
#pragma unroll
            for (int l = 0; l < kMaxIter; ++l) {
                res[l] = rr;
                xl[l] = p[l] * rr;
                if (l < L) rr -= gelu_f<true>(xl[l]);
            }
            float a = 0.f;
#pragma unroll
            for (int l = kMaxIter - 1; l >= 0; --l) {
                if (l < L) {
                    const float gx = (0.5f * gr - a) * gelu_df<true>(xl[l]);
                    dp[l] = fmaf(gx, res[l], dp[l]);
                    a = fmaf(gx, p[l], a);
                }
            }
            gv[r * C + c] = (bf16)a;
            gu[r * C + c] = (bf16)(-a);
        }
    }
    if (!gw.p[0]) return;
#pragma unroll
    for (int l = 0; l < kMaxIter; ++l)
        if (l < L) red[g][l][lane] = dp[l];
    __syncthreads();
    if (g == 0 && active) {
#pragma unroll
        for (int l = 0; l < kMaxIter; ++l) {
            if (l < L) {
                float t = 0.f;
#pragma unroll
                for (int k = 0; k < NTH / kWave; ++k) t += red[k][l][lane];
                atomicAdd(&gw.p[l][c], t);
            }
        }
    }
}

// a[r, HD..C) = 0 and b[r, HD..C) = 0 (b may be NULL) for every row, with
// 16-byte stores when VEC (C and HD multiples of 8, 16-byte aligned rows);
// the first workgroup also clears extra[0..extra_n).
template <bool VEC>
__global__ void __launch_bounds__(NTH) zero_cols_kernel(bf16* __restrict__ a, bf16* __restrict__ b,
                                                        long rows, int C, int HD,
                                                        bf16* __restrict__ extra, long extra_n) {
    if (blockIdx.x == 0)
        for (long i = threadIdx.x; i < extra_n; i += NTH) extra[i] = (bf16)0.f;
    const long gtid = (long)blockIdx.x * NTH + threadIdx.x, gstride = (long)gridDim.x * NTH;
    if (VEC) {
        const int per = (C - HD) / 8;
        bf16x8 z;
#pragma unroll
        for (int i = 0; i < 8; ++i) z[i] = (bf16)0.f;
        for (long i = gtid; i < rows * per; i += gstride) {
            const long r = i / per;
            const long off = r * C + HD + 8 * (i - r * per);
            *reinterpret_cast<bf16x8*>(a + off) = z;
            if (b) *reinterpret_cast<bf16x8*>(b + off) = z;
        }
    } else {
        const int per = C - HD;
        for (long i = gtid; i < rows * per; i += gstride) {
            const long r = i / per;
            const long off = r * C + HD + (i - r * per);
            a[off] = (bf16)0.f;
            if (b) b[off] = (bf16)0.f;
        }
    }
}

// Row-block forms of the PRISM kernels for 16-byte rows (hidden and head_dim
// multiples of 8, head_dim / 8 dividing NTH, 16-byte aligned activations, at
// most kFastIter iterations).  A workgroup owns PRR consecutive rows: its
// threads form the head_dim active channels eight per lane (one 16-byte piece
// of each input and output per row, the lane's channel group fixed) and clear
// the rows' columns past head_dim with 16-byte stores, so one launch writes
// every output byte and each CU keeps several row blocks' accesses in flight
// (the one-lane-per-channel kernels above keep one 2-byte access per lane).
constexpr int PRR = 16;
constexpr int kFastIter = 4;
constexpr long kMaxFastBlocks = 1L << 20;

__device__ __forceinline__ void zero_row_tails(bf16* __restrict__ a, bf16* __restrict__ b,
                                               long r0, long rows, int C, int HD) {
    const int per = (C - HD) / 8;
    const int n = (int)min((long)PRR, rows - r0) * per;
    bf16x8 z;
#pragma unroll
    for (int i = 0; i < 8; ++i) z[i] = (bf16)0.f;
    for (int i = threadIdx.x; i < n; i += NTH) {
        const int rr = i / per;
        const long off = (r0 + rr) * C + HD + 8 * (i - rr * per);
        *reinterpret_cast<bf16x8*>(a + off) = z;
        if (b) *reinterpret_cast<bf16x8*>(b + off) = z;
    }
}

// p[l][e] = w_p[l][8 j + e] for l < L, else 0
__device__ __forceinline__ void load_p8(const WPtrs& wp, int L, int j, float (&p)[kFastIter][8]) {
#pragma unroll
    for (int l = 0; l < kFastIter; ++l)
#pragma unroll
        for (int e = 0; e < 8; ++e) p[l][e] = l < L ? (float)wp.p[l][8 * j + e] : 0.f;
}

// The forward of prism_fwd_kernel per channel, plus the column clearing of
// zero_cols_kernel (and of new_state, `extra`, by the first workgroup).
__global__ void __launch_bounds__(NTH) prism_fwd_rows_kernel(const bf16* __restrict__ u,
                                                             const bf16* __restrict__ v, WPtrs wp,
                                                             bf16* __restrict__ out, long rows,
                                                             int C, int HD, int L,
                                                             bf16* __restrict__ extra,
                                                             long extra_n) {
    if (blockIdx.x == 0)
        for (long i = threadIdx.x; i < extra_n; i += NTH) extra[i] = (bf16)0.f;
    const long r0 = (long)blockIdx.x * PRR;
    const int PH = HD / 8, j = threadIdx.x % PH;
    float p[kFastIter][8];
    load_p8(wp, L, j, p);
    for (int rr = threadIdx.x / PH; rr < PRR; rr += NTH / PH) {
        const long r = r0 + rr;
        if (r >= rows) break;
        const bf16x8 uu = *reinterpret_cast<const bf16x8*>(u + r * C + 8 * j);
        const bf16x8 vv = *reinterpret_cast<const bf16x8*>(v + r * C + 8 * j);
        bf16x8 oo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float res = (float)vv[e] - (float)uu[e];
            float o = 0.f;
#pragma unroll
            for (int l = 0; l < kFastIter; ++l) {
                if (l < L) {
                    const float d = gelu_f<true>(p[l][e] * res);
                    o = (float)(bf16)(o + 0.5f * d);
                    res -= d;
                }
            }
            oo[e] = (bf16)o;
        }
        *reinterpret_cast<bf16x8*>(out + r * C + 8 * j) = oo;
    }
    zero_row_tails(out, nullptr, r0, rows, C, HD);
}

// The backward of prism_bwd_kernel per channel and the column clearing of
// grad_u and grad_v.  The w_p gradient of the block's rows goes to
// part[block][l * HD + c], summed over the block's threads in a fixed order;
// prism_wgrad_sum_kernel then adds the blocks' partials in block order, so the
// result is the same on every run.
__global__ void __launch_bounds__(NTH) prism_bwd_rows_kernel(
    const bf16* __restrict__ go, const bf16* __restrict__ u, const bf16* __restrict__ v, WPtrs wp,
    bf16* __restrict__ gu, bf16* __restrict__ gv, float* __restrict__ part, long rows, int C,
    int HD, int L) {
    __shared__ float red[kFastIter * NTH * 8];
    const long r0 = (long)blockIdx.x * PRR;
    const int PH = HD / 8, j = threadIdx.x % PH, k0 = threadIdx.x / PH, KB = NTH / PH;
    float p[kFastIter][8], dp[kFastIter][8];
    load_p8(wp, L, j, p);
#pragma unroll
    for (int l = 0; l < kFastIter; ++l)
#pragma unroll
        for (int e = 0; e < 8; ++e) dp[l][e] = 0.f;
    for (int rr = k0; rr < PRR; rr += KB) {
        const long r = r0 + rr;
        if (r >= rows) break;
        const long off = r * C + 8 * j;
        const bf16x8 gg = *reinterpret_cast<const bf16x8*>(go + off);
        const bf16x8 uu = *reinterpret_cast<const bf16x8*>(u + off);
        const bf16x8 vv = *reinterpret_cast<const bf16x8*>(v + off);
        bf16x8 ou, ov;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float res[kFastIter], xl[kFastIter];
            float rv = (float)vv[e] - (float)uu[e];
            const float gr = (float)gg[e];
#pragma unroll
            for (int l = 0; l < kFastIter; ++l) {
                res[l] = rv;
                xl[l] = p[l][e] * rv;
                if (l < L) rv -= gelu_f<true>(xl[l]);
            }
            float a = 0.f;
#pragma unroll
            for (int l = kFastIter - 1; l >= 0; --l) {
                if (l < L) {
                    const float gx = (0.5f * gr - a) * gelu_df<true>(xl[l]);
                    dp[l][e] = fmaf(gx, res[l], dp[l][e]);
                    a = fmaf(gx, p[l][e], a);
                }
            }
            ov[e] = (bf16)a;
            ou[e] = (bf16)(-a);
        }
        *reinterpret_cast<bf16x8*>(gv + off) = ov;
        *reinterpret_cast<bf16x8*>(gu + off) = ou;
    }
    zero_row_tails(gu, gv, r0, rows, C, HD);
    if (!part) return;
    // red[l][k][c]: thread (k, j) holds channels 8 j .. 8 j + 7 of row set k
#pragma unroll
    for (int l = 0; l < kFastIter; ++l)
        if (l < L)
#pragma unroll
            for (int e = 0; e < 8; ++e) red[(l * KB + k0) * HD + 8 * j + e] = dp[l][e];
    __syncthreads();
    for (int i = threadIdx.x; i < L * HD; i += NTH) {
        const int l = i / HD, c = i - l * HD;
        float t = 0.f;
        for (int k = 0; k < KB; ++k) t += red[(l * KB + k) * HD + c];
        part[(long)blockIdx.x * L * HD + i] = t;
    }
}

// grad_w_p[l][c] += sum over blocks b (in order) of part[b][l * HD + c];
// grid (ceil(HD / 16), L): 16 columns per workgroup as 4 lanes of 4 (HD is a
// multiple of 8), 64 block groups each taking every 64th block with eight
// 16-byte loads in flight
__global__ void __launch_bounds__(256) prism_wgrad_sum_kernel(const float* __restrict__ part,
                                                              int nblk, int HD, int L, GPtrs gw) {
    __shared__ float acc[64][16 + 1];
    const int q = threadIdx.x & 3, rg = threadIdx.x >> 2, l = blockIdx.y;
    const int c0 = blockIdx.x * 16 + 4 * q;
    const float* base = part + (long)l * HD + c0;
    const long stride = (long)L * HD;
    floatx4 s = {0.f, 0.f, 0.f, 0.f};
    if (c0 < HD)
#pragma unroll 8
        for (int b = rg; b < nblk; b += 64)
            s += *reinterpret_cast<const floatx4*>(base + b * stride);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[rg][4 * q + i] = s[i];
    __syncthreads();
    const int c = blockIdx.x * 16 + threadIdx.x;
    if (threadIdx.x < 16 && c < HD) {
        float t = 0.f;
#pragma unroll 8
        for (int k = 0; k < 64; ++k) t += acc[k][threadIdx.x];
        gw.p[l][c] += t;
    }
}

inline size_t conv_lds_bytes(int W, bool dw) {
    const int Wp = (W + JB - 1) & ~(JB - 1);
    const size_t rows = (size_t)(TT + Wp - 1) + (dw ? TT : 0);
    const size_t a = rows * CT * sizeof(float);
    const size_t wts = dw ? 0 : (size_t)Wp * (CT + 1) * sizeof(float);
    return a + wts;
}

inline bool vec_ok(const void* p, int C) { return ((uintptr_t)p & 15) == 0 && C % 8 == 0; }

// Token tiles per workgroup of conv_walk_kernel: enough segments per
// (channel tile, batch row) for about two workgroups per CU, 1 when the
// window is too long for its two-tile row buffer or the rows are not 16-byte.
inline int walk_tiles(int B, int T, int C, int W, bool vec) {
    if (!vec || W > TT) return 1;
    const int ttiles = (T + TT - 1) / TT, ctiles = (C + CT - 1) / CT;
    const long pairs = (long)B * ctiles;
    const long segs = std::max(1L, std::min((long)ttiles, (512 + pairs - 1) / pairs));
    return (int)((ttiles + segs - 1) / segs);
}

inline size_t walk_lds_bytes(int W) {
    const int Wp = (W + JB - 1) & ~(JB - 1);
    return (size_t)(2 * TT * CT + Wp * (CT + 1)) * sizeof(float);
}

// whether the row-block kernels take this problem (the pointers are the
// activations they read and write with 16-byte accesses)
inline bool rows_form_ok(long rows, size_t C, size_t HD, size_t L,
                         std::initializer_list<const void*> ptrs) {
    if (C % 8 != 0 || HD % 8 != 0 || HD == 0 || NTH % (HD / 8) != 0 || L > (size_t)kFastIter)
        return false;
    if ((rows + PRR - 1) / PRR > kMaxFastBlocks) return false;
    for (const void* p : ptrs)
        if ((uintptr_t)p & 15) return false;
    return true;
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
    const int tps = prism::walk_tiles((int)batch_size, T, C, W, prism::vec_ok(x, C));
    if (W >= 1 && tps > 1) {
        const int ttiles = (T + prism::TT - 1) / prism::TT;
        const dim3 grid((unsigned)((C + prism::CT - 1) / prism::CT), (unsigned)batch_size,
                        (unsigned)((ttiles + tps - 1) / tps));
        ::efla::ProfScope ps("shortconv_fwd", stream);
        hipLaunchKernelGGL(prism::conv_walk_kernel<false>, grid, dim3(prism::NTH),
                           prism::walk_lds_bytes(W), stream, x, wt, y, T, C, W, tps);
    } else if (W >= 1 && W <= prism::kMaxTiledW) {
        const dim3 grid((unsigned)((T + prism::TT - 1) / prism::TT),
                        (unsigned)((C + prism::CT - 1) / prism::CT), (unsigned)batch_size);
        ::efla::ProfScope ps("shortconv_fwd", stream);
        if (prism::vec_ok(x, C))
            hipLaunchKernelGGL(prism::conv_fwd_kernel<true>, grid, dim3(prism::NTH),
                               prism::conv_lds_bytes(W, false), stream, x, wt, y, T, C, W);
        else
            hipLaunchKernelGGL(prism::conv_fwd_kernel<false>, grid, dim3(prism::NTH),
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
        const int tps = prism::walk_tiles(B, T, C, W, prism::vec_ok(dy, C));
        if (tps > 1) {
            const dim3 grid((unsigned)ctiles, (unsigned)B, (unsigned)((ttiles + tps - 1) / tps));
            ::efla::ProfScope ps("shortconv_dx", stream);
            hipLaunchKernelGGL(prism::conv_walk_kernel<true>, grid, dim3(prism::NTH),
                               prism::walk_lds_bytes(W), stream, dy, wt, dx, T, C, W, tps);
        } else if (tiled) {
            const dim3 grid((unsigned)ttiles, (unsigned)ctiles, (unsigned)B);
            ::efla::ProfScope ps("shortconv_dx", stream);
            if (prism::vec_ok(dy, C))
                hipLaunchKernelGGL(prism::conv_dx_kernel<true>, grid, dim3(prism::NTH),
                                   prism::conv_lds_bytes(W, false), stream, dy, wt, dx, T, C, W);
            else
                hipLaunchKernelGGL(prism::conv_dx_kernel<false>, grid, dim3(prism::NTH),
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
        const bool pipe = tiled && prism::vec_ok(dy, C) && prism::vec_ok(x, C);
        long nsplit, tpw = 1;
        if (pipe) {  // about two workgroups per CU, each a run of consecutive tiles
            const long tiles = (long)B * ttiles;
            nsplit = std::max(1L, std::min(tiles, (long)prism::kDwPipeBlocks / ctiles));
            tpw = (tiles + nsplit - 1) / nsplit;
            nsplit = (tiles + tpw - 1) / tpw;
        } else if (tiled) {
            const long tiles = (long)B * ttiles;
            nsplit = std::max(1L, std::min({tiles, 256L, 1024L / ctiles}));
        } else {
            nsplit = std::max(1L, std::min((long)B * T, 4096L / (long)prism::grid_1d(cw)));
        }
        void* ws = nullptr;
        WsLease lease;
        const int wrc = workspace_acquire((size_t)nsplit * cw * sizeof(float), stream, &ws, lease);
        if (wrc != kSuccess) return wrc;
        float* part = (float*)ws;
        if (pipe) {
            ::efla::ProfScope ps("shortconv_dw", stream);
            hipLaunchKernelGGL(prism::conv_dw_pipe_kernel, dim3((unsigned)ctiles, (unsigned)nsplit),
                               dim3(prism::NTH), prism::conv_lds_bytes(W, true), stream, dy, x,
                               part, B, T, C, W, ttiles, (int)tpw);
        } else if (tiled) {
            ::efla::ProfScope ps("shortconv_dw", stream);
            const dim3 grid((unsigned)ctiles, (unsigned)nsplit);
            if (prism::vec_ok(dy, C) && prism::vec_ok(x, C))
                hipLaunchKernelGGL(prism::conv_dw_kernel<true>, grid, dim3(prism::NTH),
                                   prism::conv_lds_bytes(W, true), stream, dy, x, part, B, T, C,
                                   W, ttiles);
            else
                hipLaunchKernelGGL(prism::conv_dw_kernel<false>, grid, dim3(prism::NTH),
                                   prism::conv_lds_bytes(W, true), stream, dy, x, part, B, T, C,
                                   W, ttiles);
        } else {
            EFLA_LAUNCH("shortconv_dw_direct", prism::conv_dw_direct_kernel,
                        dim3((unsigned)((cw + prism::NTH - 1) / prism::NTH), (unsigned)nsplit),
                        dim3(prism::NTH), stream, dy, x, part, B, T, C, W);
        }
        EFLA_CHECK(hipPeekAtLastError());
        EFLA_LAUNCH("shortconv_dw_sum", partial_colsum_add_kernel, partial_colsum_grid(cw),
                    dim3(256), stream, (const float*)part, (int)nsplit, cw, grad_weight);
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
    if ((B * T + prism::PRB - 1) / prism::PRB > 0x7FFFFFFFull) return kInvalidConfiguration;
    if (L > 0 && !w_p) return kInvalidValue;
    for (size_t l = 0; l < (size_t)prism::kMaxIter; ++l) {
        wp->p[l] = l < L ? (const bf16*)w_p[l] : nullptr;
        if (l < L && !wp->p[l]) return kInvalidValue;
    }
    return kSuccess;
}

}  // namespace

namespace {

// zero the columns [head_dim, hidden_dim) of a and b (b may be NULL) and the
// extra_n values at extra
int zero_tail(bf16* a, bf16* b, long rows, size_t hidden, size_t head_dim, bf16* extra,
              long extra_n, hipStream_t stream) {
    const long n = rows * (long)(hidden - head_dim);
    if (n == 0 && extra_n == 0) return kSuccess;
    const bool vec = hidden % 8 == 0 && head_dim % 8 == 0 && ((uintptr_t)a & 15) == 0 &&
                     ((uintptr_t)b & 15) == 0;
    const dim3 grid(prism::grid_1d(vec ? n / 8 : n));
    if (vec)
        EFLA_LAUNCH("prism_zero_cols", prism::zero_cols_kernel<true>, grid, dim3(prism::NTH),
                    stream, a, b, rows, (int)hidden, (int)head_dim, extra, extra_n);
    else
        EFLA_LAUNCH("prism_zero_cols", prism::zero_cols_kernel<false>, grid, dim3(prism::NTH),
                    stream, a, b, rows, (int)hidden, (int)head_dim, extra, extra_n);
    return (int)hipPeekAtLastError();
}

dim3 prism_grid(long rows, size_t head_dim) {
    return dim3((unsigned)((rows + prism::PRB - 1) / prism::PRB),
                (unsigned)((head_dim + kWave - 1) / kWave));
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
    if (rows == 0) {
        return new_state ? fill_zero(new_state, head_dim * head_dim * sizeof(bf16), stream)
                         : kSuccess;
    }
    if (prism::rows_form_ok(rows, hidden_dim, head_dim, num_iterations, {u, v, output})) {
        EFLA_LAUNCH("prism_fwd", prism::prism_fwd_rows_kernel,
                    dim3((unsigned)((rows + prism::PRR - 1) / prism::PRR)), dim3(prism::NTH),
                    stream, (const bf16*)u, (const bf16*)v, wp, (bf16*)output, rows,
                    (int)hidden_dim, (int)head_dim, (int)num_iterations, (bf16*)new_state,
                    new_state ? (long)(head_dim * head_dim) : 0L);
        return (int)hipPeekAtLastError();
    }
    const dim3 grid = prism_grid(rows, head_dim);
    EFLA_LAUNCH("prism_fwd", prism::prism_fwd_kernel, grid, dim3(prism::NTH), stream,
                (const bf16*)u, (const bf16*)v, wp, (bf16*)output, rows, (int)hidden_dim,
                (int)head_dim, (int)num_iterations);
    EFLA_CHECK(hipPeekAtLastError());
    return zero_tail((bf16*)output, nullptr, rows, hidden_dim, head_dim, (bf16*)new_state,
                     new_state ? (long)(head_dim * head_dim) : 0, stream);
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
    prism::GPtrs gw;
    for (int l = 0; l < prism::kMaxIter; ++l) {
        gw.p[l] = (grad_w_p && l < L) ? grad_w_p[l] : nullptr;
        if (grad_w_p && l < L && !gw.p[l]) return kInvalidValue;
    }
    if (prism::rows_form_ok(rows, hidden_dim, head_dim, num_iterations,
                            {grad_output, u, v, grad_u, grad_v})) {
        const long nblk = (rows + prism::PRR - 1) / prism::PRR;
        float* part = nullptr;
        WsLease lease;
        if (grad_w_p && L > 0) {
            void* ws = nullptr;
            const int wrc = workspace_acquire((size_t)nblk * L * head_dim * sizeof(float),
                                              stream, &ws, lease);
            if (wrc != kSuccess) return wrc;
            part = (float*)ws;
        }
        EFLA_LAUNCH("prism_bwd", prism::prism_bwd_rows_kernel, dim3((unsigned)nblk),
                    dim3(prism::NTH), stream, (const bf16*)grad_output, (const bf16*)u,
                    (const bf16*)v, wp, (bf16*)grad_u, (bf16*)grad_v, part, rows,
                    (int)hidden_dim, (int)head_dim, L);
        EFLA_CHECK(hipPeekAtLastError());
        if (part)
            EFLA_LAUNCH("prism_bwd_wsum", prism::prism_wgrad_sum_kernel,
                        dim3((unsigned)((head_dim + 15) / 16), (unsigned)L), dim3(256), stream,
                        (const float*)part, (int)nblk, (int)head_dim, L, gw);
        return (int)hipPeekAtLastError();
    }
    const dim3 grid = prism_grid(rows, head_dim);
    EFLA_LAUNCH("prism_bwd", prism::prism_bwd_kernel, grid, dim3(prism::NTH), stream,
                (const bf16*)grad_output, (const bf16*)u, (const bf16*)v, wp, (bf16*)grad_u,
                (bf16*)grad_v, gw, rows, (int)hidden_dim, (int)head_dim, L);
    EFLA_CHECK(hipPeekAtLastError());
    return zero_tail((bf16*)grad_u, (bf16*)grad_v, rows, hidden_dim, head_dim, nullptr, 0, stream);
}
