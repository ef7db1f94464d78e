// EFLA behind the reference ABI ("Mode R"): efla_forward_hip,
// efla_backward_hip, efla_chunked_scan_hip.
//
// Semantics follow kernels/cuda/efla.cu exactly: per (b, h) and token t
//   lambda = |k_t|^2, c = c(beta, lambda)
//   u = S^T k_t, S <- bf16(S + (c k_t)(v_t - u)^T)   (state re-rounded every token)
//   o_t = S k_t                                        (needs d_k == d_v)
// One workgroup of 256 threads owns one (b, h).  The bf16 state lives in LDS
// (row stride d+2 to spread banks) instead of global memory, so a token costs
// two passes over LDS and four barriers, against three global passes and ~13
// barriers in the reference.  Reduction order differs from the reference's
// serial sums; values differ at fp32 rounding level before each bf16 rounding.
//
// The backward recomputes states from bf16 checkpoints taken every 64 tokens
// (exact, since the states are bf16 values), rebuilds the 65 states of one
// segment at a time into a workspace, and runs the reference's BPTT
// (efla.cu:315-454) over the segment in reverse with the fp32 dL/dS in LDS
// (d <= 128) or in the workspace (d <= 256).
#include <hip/hip_runtime.h>

#include "../../include/efla_hip.h"
#include "common.hpp"
#include "efla_coeff.hpp"
#include "internal.hpp"

namespace efla {
namespace r {

constexpr int NTH = 256;
constexpr int MAXD = 256;
constexpr int SEG = 64;  // checkpoint spacing of the backward

__device__ __forceinline__ float block_sum(float x, float* red) {
    // wave reduction then across the 4 waves
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
    __syncthreads();
    if (lane_id() == 0) red[wave_id()] = x;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// One forward token on the LDS state S (row stride lds).  kf, vf hold k_t, v_t
// in fp32; on return S holds the new state.  `red` needs 2*MAXD + 8 floats.
// If `out` is set, o_t = S k_t is written there (bf16).
__device__ void step(bf16* S, int lds, int d, const float* kf, const float* vf, float c,
                     float* red, float* rv, bf16* out) {
    const int t = threadIdx.x;
    const int P = NTH / d;  // threads per column / row
    const int col = t % d, part = t / d;
    const bool act = part < P;
    // u = S^T k (column sums)
    if (act) {
        float s = 0.f;
        for (int row = part; row < d; row += P) s = fmaf(kf[row], to_f(S[row * lds + col]), s);
        red[part * d + col] = s;
    }
    __syncthreads();
    if (t < d) {
        float u = 0.f;
        for (int p = 0; p < P; ++p) u += red[p * d + t];
        rv[t] = vf[t] - u;
    }
    __syncthreads();
    // S <- bf16(S + (c k_row) r_col); row sums of the new S against k
    if (act) {
        const int row = col;  // reuse the mapping: thread owns a row here
        const float ck = c * kf[row];
        float o = 0.f;
        for (int cc = part; cc < d; cc += P) {
            const bf16 nv = (bf16)fmaf(ck, rv[cc], to_f(S[row * lds + cc]));
            S[row * lds + cc] = nv;
            o = fmaf((float)nv, kf[cc], o);
        }
        red[MAXD + part * d + row] = o;
    }
    __syncthreads();
    if (out && t < d) {
        float o = 0.f;
        for (int p = 0; p < P; ++p) o += red[MAXD + p * d + t];
        out[t] = (bf16)o;
    }
}

__device__ __forceinline__ void load_vec(const bf16* __restrict__ src, float* dst, int d) {
    for (int i = threadIdx.x; i < d; i += NTH) dst[i] = to_f(src[i]);
}

__device__ __forceinline__ float token_coeff(const float* kf, int d, float beta, float* red,
                                             float* dc_out) {
    float s = 0.f;
    for (int i = threadIdx.x; i < d; i += NTH) s += kf[i] * kf[i];
    const float lam = block_sum(s, red);
    float c, dcl, dcb;
    efla_coeff(lam, beta, c, dcl, dcb);
    if (dc_out) *dc_out = dcl;
    return c;
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(NTH) r_forward_kernel(const bf16* __restrict__ k,
                                                        const bf16* __restrict__ v,
                                                        bf16* __restrict__ state,
                                                        bf16* __restrict__ out, int H, long T,
                                                        int d, float beta) {
    __shared__ bf16 S[MAXD * (MAXD + 2)];
    __shared__ float kf[MAXD], vf[MAXD], rv[MAXD], red[2 * MAXD + 8];
    const int bh = blockIdx.x, b = bh / H, h = bh % H;
    const int lds = d + 2;
    bf16* st = state + (long)bh * d * d;
    for (int i = threadIdx.x; i < d * d; i += NTH) S[(i / d) * lds + i % d] = st[i];
    __syncthreads();
    for (long t = 0; t < T; ++t) {
        const long base = ((long)b * T + t) * H * d + (long)h * d;
        load_vec(k + base, kf, d);
        load_vec(v + base, vf, d);
        __syncthreads();
        const float c = token_coeff(kf, d, beta, red + 2 * MAXD, nullptr);
        step(S, lds, d, kf, vf, c, red, rv, out + base);
        __syncthreads();
    }
    for (int i = threadIdx.x; i < d * d; i += NTH) st[i] = S[(i / d) * lds + i % d];
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------
// Phase 1 of the backward: run the forward once and store the state before
// every SEG-th token (bf16, exact) into ck[(bh * nseg + j) * d * d].
__global__ void __launch_bounds__(NTH) r_checkpoint_kernel(const bf16* __restrict__ k,
                                                           const bf16* __restrict__ v,
                                                           const bf16* __restrict__ state0,
                                                           bf16* __restrict__ ck, int H, long T,
                                                           int d, float beta) {
    __shared__ bf16 S[MAXD * (MAXD + 2)];
    __shared__ float kf[MAXD], vf[MAXD], rv[MAXD], red[2 * MAXD + 8];
    const int bh = blockIdx.x, b = bh / H, h = bh % H;
    const int lds = d + 2;
    const long dd = (long)d * d;
    const long nseg = (T + SEG - 1) / SEG;
    const bf16* s0 = state0 + (long)bh * dd;
    for (int i = threadIdx.x; i < d * d; i += NTH) S[(i / d) * lds + i % d] = s0[i];
    __syncthreads();
    for (long t = 0; t < T; ++t) {
        if (t % SEG == 0) {
            bf16* dst = ck + ((long)bh * nseg + t / SEG) * dd;
            for (int i = threadIdx.x; i < d * d; i += NTH) dst[i] = S[(i / d) * lds + i % d];
        }
        const long base = ((long)b * T + t) * H * d + (long)h * d;
        load_vec(k + base, kf, d);
        load_vec(v + base, vf, d);
        __syncthreads();
        const float c = token_coeff(kf, d, beta, red + 2 * MAXD, nullptr);
        step(S, lds, d, kf, vf, c, red, rv, nullptr);
        __syncthreads();
    }
}

// Phase 2: per segment (last to first) rebuild its states into hist (SEG+1
// states of d*d bf16 per (b,h)) and run the reference BPTT over it.
// G: dL/dS after the current token, fp32, in LDS when GL is false.
template <bool GL>
__global__ void __launch_bounds__(NTH) r_backward_kernel(
    const bf16* __restrict__ dO, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const bf16* __restrict__ ck, bf16* __restrict__ hist_all, float* __restrict__ G_all,
    bf16* __restrict__ grad_k, bf16* __restrict__ grad_v, bf16* __restrict__ grad_state, int H,
    long T, int d, float beta) {
    constexpr int GMAX = GL ? 1 : 128 * 129;
    constexpr int SMAX = GL ? MAXD * (MAXD + 2) : 128 * 130;
    __shared__ float Gl[GMAX];
    __shared__ bf16 S[SMAX];
    __shared__ float kf[MAXD], vf[MAXD], go[MAXD], w1[MAXD], w2[MAXD], gk[MAXD];
    __shared__ float red[3 * MAXD + 8];
    const int bh = blockIdx.x, b = bh / H, h = bh % H;
    const int tid = threadIdx.x;
    const int lds = d + 2;
    const long dd = (long)d * d;
    const long nseg = (T + SEG - 1) / SEG;
    const int P = NTH / d;
    const int col = tid % d, part = tid / d;
    const bool act = part < P;
    bf16* hist = hist_all + (long)bh * (SEG + 1) * dd;
    float* G = GL ? G_all + (long)bh * dd : Gl;
    const int ldg = GL ? d : d + 1;
    for (int i = tid; i < d * d; i += NTH) G[(i / d) * ldg + i % d] = 0.f;
    for (long seg = nseg - 1; seg >= 0; --seg) {
        const long t0 = seg * SEG;
        const long t1 = (t0 + SEG < T) ? t0 + SEG : T;
        // rebuild the segment: hist[j] = state before token t0 + j
        const bf16* c0 = ck + ((long)bh * nseg + seg) * dd;
        __syncthreads();
        for (int i = tid; i < d * d; i += NTH) {
            S[(i / d) * lds + i % d] = c0[i];
            hist[i] = c0[i];
        }
        __syncthreads();
        for (long t = t0; t < t1; ++t) {
            const long base = ((long)b * T + t) * H * d + (long)h * d;
            load_vec(k + base, kf, d);
            load_vec(v + base, vf, d);
            __syncthreads();
            const float c = token_coeff(kf, d, beta, red + 3 * MAXD, nullptr);
            step(S, lds, d, kf, vf, c, red, w1, nullptr);
            __syncthreads();
            bf16* dst = hist + (t - t0 + 1) * dd;
            for (int i = tid; i < d * d; i += NTH) dst[i] = S[(i / d) * lds + i % d];
        }
        __syncthreads();
        // reverse BPTT over the segment (efla.cu:355-453)
        for (long t = t1 - 1; t >= t0; --t) {
            const long base = ((long)b * T + t) * H * d + (long)h * d;
            const bf16* Sp = hist + (t - t0) * dd;
            const bf16* Sn = Sp + dd;
            load_vec(k + base, kf, d);
            load_vec(v + base, vf, d);
            load_vec(dO + base, go, d);
            __syncthreads();
            float dc;
            const float c = token_coeff(kf, d, beta, red + 3 * MAXD, &dc);
            // column sums: u = Sp^T k, gk = Sn^T go, w1 = c g^T k  (g = G + go k^T)
            if (act) {
                float su = 0.f, sg = 0.f, sw = 0.f;
                const float kc = kf[col];
                for (int row = part; row < d; row += P) {
                    const float kr = kf[row];
                    su = fmaf(kr, to_f(Sp[(long)row * d + col]), su);
                    sg = fmaf(to_f(Sn[(long)row * d + col]), go[row], sg);
                    const float g = fmaf(go[row], kc, G[row * ldg + col]);
                    sw = fmaf(g, kr, sw);
                }
                red[part * d + col] = su;
                red[MAXD + part * d + col] = sg;
                red[2 * MAXD + part * d + col] = sw;
            }
            __syncthreads();
            if (tid < d) {
                float su = 0.f, sg = 0.f, sw = 0.f;
                for (int p = 0; p < P; ++p) {
                    su += red[p * d + tid];
                    sg += red[MAXD + p * d + tid];
                    sw += red[2 * MAXD + p * d + tid];
                }
                w2[tid] = vf[tid] - su;
                gk[tid] = sg;
                w1[tid] = c * sw;
            }
            __syncthreads();
            // row sums: ex = g w2, up = Sp w1; G <- g - k w1^T
            float gc_part = 0.f;
            if (act) {
                const int row = col;
                const float kr = kf[row], gor = go[row];
                float ex = 0.f, up = 0.f;
                for (int cc = part; cc < d; cc += P) {
                    const float g = fmaf(gor, kf[cc], G[row * ldg + cc]);
                    ex = fmaf(g, w2[cc], ex);
                    up = fmaf(to_f(Sp[(long)row * d + cc]), w1[cc], up);
                    G[row * ldg + cc] = fmaf(-kr, w1[cc], g);
                }
                red[part * d + row] = ex;
                red[MAXD + part * d + row] = up;
            }
            __syncthreads();
            float ex_r = 0.f, up_r = 0.f;
            if (tid < d) {
                for (int p = 0; p < P; ++p) {
                    ex_r += red[p * d + tid];
                    up_r += red[MAXD + p * d + tid];
                }
                gc_part = kf[tid] * ex_r;  // grad_c = sum_row k_row (g w2)_row
            }
            const float grad_c = block_sum(gc_part, red + 3 * MAXD);
            const float grad_lambda = grad_c * dc;
            if (tid < d) {
                const float g = fmaf(2.f * grad_lambda, kf[tid], fmaf(c, ex_r, gk[tid]) - up_r);
                grad_v[base + tid] = (bf16)w1[tid];
                grad_k[base + tid] = (bf16)g;
            }
            __syncthreads();
        }
    }
    __syncthreads();
    bf16* gs = grad_state + (long)bh * dd;
    for (int i = tid; i < d * d; i += NTH) gs[i] = (bf16)G[(i / d) * ldg + i % d];
}

// chunk_states[i] <- bf16(chunk_states[i-1] + chunk_states[i]), one thread per
// element walking the chunks in order.
__global__ void __launch_bounds__(NTH) r_prefix_kernel(bf16* const* __restrict__ ptrs, long n,
                                                       long nchunks) {
    const long stride = (long)gridDim.x * blockDim.x;
    for (long j = (long)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += stride) {
        float run = to_f(ptrs[0][j]);
        for (long i = 1; i < nchunks; ++i) {
            const bf16 nv = (bf16)(run + to_f(ptrs[i][j]));
            ptrs[i][j] = nv;
            run = (float)nv;
        }
    }
}

}  // namespace r
}  // namespace efla

using namespace efla;
using namespace efla::r;

extern "C" int efla_forward_hip(const void* k, const void* v, void* state, void* output,
                                size_t batch_size, size_t seq_len, size_t num_heads,
                                size_t head_dim, float beta, size_t chunk_size,
                                hipStream_t stream) {
    (void)chunk_size;  // accepted and ignored, as efla.cu:495
    if (batch_size == 0 || num_heads == 0 || head_dim == 0) return kInvalidValue;
    if (seq_len == 0) return kSuccess;
    if (!k || !v || !state || !output) return kInvalidValue;
    size_t nbh, elems;
    if (!mul_ok(batch_size, num_heads, &nbh) || nbh > 0xFFFFFFFFull) return kInvalidConfiguration;
    if (!mul_ok(nbh, seq_len, head_dim, &elems) || elems > ((size_t)1 << 50))
        return kInvalidConfiguration;
    // the LDS-resident state holds head_dim <= 256 (the reference's bound is
    // its shared-memory limit; see the header)
    if (head_dim > (size_t)MAXD || nbh > (size_t)INT32_MAX) return kInvalidConfiguration;
    EFLA_LAUNCH("efla_r_forward", r_forward_kernel, dim3((unsigned)nbh), dim3(NTH), stream,
                (const bf16*)k, (const bf16*)v, (bf16*)state, (bf16*)output, (int)num_heads,
                (long)seq_len, (int)head_dim, beta);
    return (int)hipPeekAtLastError();
}

extern "C" int efla_backward_hip(const void* grad_output, const void* k, const void* v,
                                 const void* state, void* grad_k, void* grad_v,
                                 void* grad_state, size_t batch_size, size_t seq_len,
                                 size_t num_heads, size_t head_dim, float beta,
                                 hipStream_t stream) {
    if (batch_size == 0 || num_heads == 0 || head_dim == 0) return kInvalidValue;
    if (!state || !grad_state) return kInvalidValue;
    size_t nbh, gse, gsb;
    if (!mul_ok(batch_size, num_heads, &nbh) || nbh > 0xFFFFFFFFull) return kInvalidConfiguration;
    if (!mul_ok(nbh, head_dim, head_dim, &gse) || !mul_ok(gse, 2, &gsb))
        return kInvalidConfiguration;
    if (seq_len == 0) return fill_zero(grad_state, gsb, stream);
    if (!grad_output || !k || !v || !grad_k || !grad_v) return kInvalidValue;
    if (head_dim > (size_t)MAXD || nbh > (size_t)INT32_MAX) return kInvalidConfiguration;
    const size_t nseg = (seq_len + SEG - 1) / SEG;
    size_t ck_elems, hist_elems, g_elems = 0;
    if (!mul_ok(gse, nseg, &ck_elems) || !mul_ok(gse, SEG + 1, &hist_elems))
        return kInvalidConfiguration;
    const bool gl = head_dim > 128;
    if (gl) g_elems = gse;
    const size_t off_hist = (ck_elems * 2 + 255) & ~(size_t)255;
    const size_t off_g = (off_hist + hist_elems * 2 + 255) & ~(size_t)255;
    const size_t need = off_g + g_elems * 4 + 256;
    void* ws = nullptr;
    WsLease lease;
    int rc = workspace_acquire(need, stream, &ws, lease);
    if (rc != kSuccess) return rc;
    bf16* ck = (bf16*)ws;
    bf16* hist = (bf16*)((char*)ws + off_hist);
    float* G = gl ? (float*)((char*)ws + off_g) : nullptr;
    EFLA_LAUNCH("efla_r_checkpoint", r_checkpoint_kernel, dim3((unsigned)nbh), dim3(NTH), stream,
                (const bf16*)k, (const bf16*)v, (const bf16*)state, ck, (int)num_heads,
                (long)seq_len, (int)head_dim, beta);
    if (gl) {
        EFLA_LAUNCH("efla_r_backward", r_backward_kernel<true>, dim3((unsigned)nbh), dim3(NTH),
                    stream, (const bf16*)grad_output, (const bf16*)k, (const bf16*)v, ck, hist,
                    G, (bf16*)grad_k, (bf16*)grad_v, (bf16*)grad_state, (int)num_heads,
                    (long)seq_len, (int)head_dim, beta);
    } else {
        EFLA_LAUNCH("efla_r_backward", r_backward_kernel<false>, dim3((unsigned)nbh), dim3(NTH),
                    stream, (const bf16*)grad_output, (const bf16*)k, (const bf16*)v, ck, hist,
                    G, (bf16*)grad_k, (bf16*)grad_v, (bf16*)grad_state, (int)num_heads,
                    (long)seq_len, (int)head_dim, beta);
    }
    return (int)hipPeekAtLastError();
}

extern "C" int efla_chunked_scan_hip(void** chunk_states, size_t num_chunks, size_t num_heads,
                                     size_t head_dim, hipStream_t stream) {
    if (num_chunks == 0 || num_heads == 0 || head_dim == 0) return kInvalidValue;
    if (chunk_states == nullptr) return kInvalidValue;
    size_t n;
    if (!mul_ok(1, num_heads, head_dim, &n) || !mul_ok(n, head_dim, &n))
        return kInvalidConfiguration;
    for (size_t i = 0; i < num_chunks; ++i)
        if (chunk_states[i] == nullptr) return kInvalidValue;
    if (num_chunks == 1) return kSuccess;
    size_t pbytes;
    if (!mul_ok(num_chunks, sizeof(void*), &pbytes)) return kInvalidConfiguration;
    void* ws = nullptr;
    WsLease lease;
    int rc = workspace_acquire(pbytes, stream, &ws, lease);
    if (rc != kSuccess) return rc;
    // pageable source: the runtime stages it before returning, so the caller's
    // array may be released as soon as this call returns
    EFLA_CHECK(hipMemcpyAsync(ws, chunk_states, pbytes, hipMemcpyHostToDevice, stream));
    size_t g = (n + NTH - 1) / NTH;
    if (g > 65535) g = 65535;
    EFLA_LAUNCH("efla_r_prefix", r_prefix_kernel, dim3((unsigned)g), dim3(NTH), stream,
                (bf16* const*)ws, (long)n, (long)num_chunks);
    return (int)hipPeekAtLastError();
}
