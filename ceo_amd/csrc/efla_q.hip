// Chunked EFLA with a query readout ("Mode Q") for gfx950.
//
// Recurrence per (sequence, head), tokens t (generalises efla.cu:154-233):
//   lambda_t = |k_t|^2, b_t = c(beta_t, lambda_t)
//   S_t = S_{t-1} + b_t k_t (v_t - S_{t-1}^T k_t)^T,   o_t = S_t^T q_t
// This is the delta rule with step b_t, so the chunked WY / UT-transform form
// applies.  For a chunk of C = 64 tokens with start state S:
//   A  = strict_lower(diag(b) K K^T),  T = (I + A)^{-1}
//   W  = T diag(b) K,  U = T diag(b) V
//   Vn = U - W S                       (the chunk's effective values)
//   O  = Q S + tril(Q K^T) Vn
//   S' = S + K^T Vn
// Two kernel sets implement it.  bf16 runs on the gfx950 kernels of
// efla_q_fast.hpp (prep, forward scan with the output) and efla_q_bwd.hpp
// (state recompute, reverse state scan, persistent per-chunk gradient
// kernel); their headers describe them.  fp32 runs on the generic kernels in
// this file.  Generic forward: prep (b,
// T, W, U; parallel over chunks), state (serial over chunks, one workgroup
// per (sequence, head, 64-wide value slice), S held in MFMA accumulators),
// output (parallel over chunks).  Generic backward: it recomputes b, W, U and
// the chunk states, then runs dv_local (tril(QK^T)^T dO), a reverse state
// scan for dS, dq/dk/dw per chunk, and the WY backward that carries dW, dU
// through T and b (including the dc/dlambda term of efla.cu:384-451 and
// dbeta = dc * exp(-beta lambda)).  This file also holds the host side:
// validation, workspace layout and the launches.
#include <hip/hip_runtime.h>
#include <stdlib.h>

#include <mutex>

#include "../../include/efla_hip.h"
#include "common.hpp"
#include "efla_coeff.hpp"
#include "internal.hpp"
#include "efla_q_seq.hpp"
#include "efla_q_fast.hpp"
#include "efla_q_bwd.hpp"

namespace efla {
namespace q {

constexpr int NTH = 256;  // threads per workgroup
constexpr int NW = 4;     // waves per workgroup
constexpr int LDF = 68;   // row stride of the 64x64 fp32 LDS matrices

template <typename T>
constexpr int pad() {
    return 16 / (int)sizeof(T);
}

// Sanitise cu_seqlens into [0, ntok] (non-decreasing) and build chunk offsets.
// One workgroup of 1024 threads; each owns a contiguous run of sequences.
// With `order` (N <= LPT_MAX_SEQS) it also ranks the sequences by decreasing
// chunk count, ties in index order, and writes order[rank] = sequence.
__global__ void __launch_bounds__(1024) chunk_offsets_kernel(const int32_t* __restrict__ cu,
                                                             int N, long ntok,
                                                             int32_t* __restrict__ cu_s,
                                                             int32_t* __restrict__ coff,
                                                             int32_t* __restrict__ order) {
    __shared__ int part[1024];
    __shared__ int runmax[1024];
    const int tid = threadIdx.x;
    const int per = (N + 1023) / 1024;
    const int s0 = min(N, tid * per), s1 = min(N, s0 + per);
    // pass 1: clamp each entry and take the running max inside the run
    int m = 0;
    for (int i = s0; i < s1; ++i) {
        long c = cu[i];
        c = c < 0 ? 0 : (c > ntok ? ntok : c);
        m = max(m, (int)c);
    }
    runmax[tid] = m;
    __syncthreads();
    // prefix max of run maxima (exclusive) so the sanitised offsets never decrease
    for (int off = 1; off < 1024; off <<= 1) {
        const int v = tid >= off ? runmax[tid - off] : 0;
        __syncthreads();
        runmax[tid] = max(runmax[tid], v);
        __syncthreads();
    }
    int prev = tid > 0 ? runmax[tid - 1] : 0;
    int sum = 0;
    for (int i = s0; i < s1; ++i) {
        long c = cu[i];
        c = c < 0 ? 0 : (c > ntok ? ntok : c);
        prev = max(prev, (int)c);
        cu_s[i] = prev;
    }
    __syncthreads();
    if (tid == 1023) {
        long c = cu[N];
        c = c < 0 ? 0 : (c > ntok ? ntok : c);
        cu_s[N] = max((int)c, runmax[1023]);
    }
    __syncthreads();
    for (int i = s0; i < s1; ++i) {
        const int L = cu_s[i + 1] - cu_s[i];
        sum += (L + BT - 1) / BT;
    }
    part[tid] = sum;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
        const int v = tid >= off ? part[tid - off] : 0;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    int run = part[tid] - sum;
    for (int i = s0; i < s1; ++i) {
        coff[i] = run;
        const int L = cu_s[i + 1] - cu_s[i];
        run += (L + BT - 1) / BT;
    }
    if (tid == 1023) coff[N] = part[1023];
    if (order && N <= LPT_MAX_SEQS) {
        __syncthreads();  // every chunk count below is read from part[]
        int key = 0;
        if (tid < N) key = (cu_s[tid + 1] - cu_s[tid] + BT - 1) / BT;
        __syncthreads();  // part[] is free again
        part[tid] = key;
        __syncthreads();
        if (tid < N) {
            int rank = 0;
            for (int j = 0; j < N; ++j) {
                const int kj = part[j];
                rank += (kj > key || (kj == key && j < tid)) ? 1 : 0;
            }
            order[rank] = tid;
        }
    }
}

// ---------------------------------------------------------------------------
// T = (I + A)^{-1}, A = strict_lower(diag(b) K K^T), in fp32 LDS.
// Gs receives K K^T (lower tiles incl. the diagonal tiles), Ts the inverse.
// Diagonal 16x16 blocks by forward substitution, then the off-diagonal blocks
// by increasing distance: T_IJ = -T_II sum_{m=J}^{I-1} A_Im T_mJ.
// Ends with a workgroup barrier.
// ---------------------------------------------------------------------------
template <typename MT, int K, typename TK>
__device__ void compute_T(const TK* Ks, int ldk, const float* bs, float* Gs, float* Ts,
                          float* Ysc) {
    block_gemm<MT, 64, 64, K, NW>(view_k(Ks, ldk), view_k(Ks, ldk), SkipUpper{},
                                  [&](int r, int c, floatx4 acc) {
#pragma unroll
                                      for (int i = 0; i < 4; ++i) Gs[(r + i) * LDF + c] = acc[i];
                                  });
    for (int i = threadIdx.x; i < 64 * LDF; i += NTH) Ts[i] = 0.f;
    __syncthreads();
    const int w = wave_id(), l = lane_id();
    if (l < 16) {
        const int base = 16 * w, c = l;
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float s = (i == c) ? 1.f : 0.f;
            const float bi = bs[base + i];
#pragma unroll
            for (int j = 0; j < i; ++j) s -= bi * Gs[(base + i) * LDF + base + j] * x[j];
            x[i] = s;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) Ts[(base + i) * LDF + base + c] = x[i];
    }
    __syncthreads();
    const int r = l >> 2, c0 = 4 * (l & 3);
    float* Y = Ysc + w * 16 * 17;
    for (int d = 1; d < 4; ++d) {
        const int I = w + d, J = w;
        if (w < 4 - d) {
            float y[4] = {0.f, 0.f, 0.f, 0.f};
            const float bi = bs[16 * I + r];
            for (int m = 16 * J; m < 16 * I; ++m) {
                const float a = bi * Gs[(16 * I + r) * LDF + m];
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) y[qq] += a * Ts[m * LDF + 16 * J + c0 + qq];
            }
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) Y[r * 17 + c0 + qq] = y[qq];
        }
        __syncthreads();
        if (w < 4 - d) {
            float t[4] = {0.f, 0.f, 0.f, 0.f};
            for (int m = 0; m < 16; ++m) {
                const float a = Ts[(16 * I + r) * LDF + 16 * I + m];
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) t[qq] += a * Y[m * 17 + c0 + qq];
            }
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) Ts[(16 * I + r) * LDF + 16 * J + c0 + qq] = -t[qq];
        }
        __syncthreads();
    }
}

// lambda, b, dc/dlambda, dc/dbeta for the 64 tokens of a chunk (4 threads per
// token); padding tokens get b = 0.  Ends with a barrier.
template <typename T, int K>
__device__ __forceinline__ void chunk_coeffs(const T* Ks, int ldk, const T* __restrict__ beta,
                                             long bos, int H, int h, int len, float* bs,
                                             float* dcls, float* dcbs, float* bco_out) {
    const int t = threadIdx.x >> 2, part = threadIdx.x & 3;
    float s = 0.f;
    for (int d = part; d < K; d += 4) {
        const float x = to_f(Ks[t * ldk + d]);
        s += x * x;
    }
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    if (part == 0) {
        float c = 0.f, dcl = 0.f, dcb = 0.f;
        if (t < len) {
            efla_coeff(s, to_f(beta[(bos + t) * H + h]), c, dcl, dcb);
            if (bco_out) bco_out[(bos + t) * H + h] = c;
        }
        bs[t] = c;
        if (dcls) dcls[t] = dcl;
        if (dcbs) dcbs[t] = dcb;
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// forward: prep.  grid (chunk slots, H)
// ---------------------------------------------------------------------------
template <typename T, int K, int V>
__global__ void __launch_bounds__(NTH) fwd_prep_kernel(const T* __restrict__ k,
                                                       const T* __restrict__ v,
                                                       const T* __restrict__ beta, SeqInfo si,
                                                       int H, float* __restrict__ bco,
                                                       T* __restrict__ Wout,
                                                       T* __restrict__ Uout) {
    constexpr int P = pad<T>(), LDK = K + P, LDV = V + P;
    __shared__ __attribute__((aligned(16))) T Ks[64 * LDK];
    __shared__ __attribute__((aligned(16))) T Vs[64 * LDV];
    __shared__ __attribute__((aligned(16))) float Gs[64 * LDF];
    __shared__ __attribute__((aligned(16))) float Ts[64 * LDF];
    __shared__ float Ysc[4 * 16 * 17];
    __shared__ float bs[64];
    const int slot = blockIdx.x, h = blockIdx.y;
    long bos;
    int len;
    if (!locate_chunk(si, slot, bos, len)) return;
    load_rows<T, 64, K, NTH>(Ks, LDK, k + (bos * H + h) * K, (long)H * K, len);
    load_rows<T, 64, V, NTH>(Vs, LDV, v + (bos * H + h) * V, (long)H * V, len);
    __syncthreads();
    chunk_coeffs<T, K>(Ks, LDK, beta, bos, H, h, len, bs, nullptr, nullptr, bco);
    compute_T<T, K>(Ks, LDK, bs, Gs, Ts, Ysc);
    T* Wb = Wout + (bos * H + h) * K;
    T* Ub = Uout + (bos * H + h) * V;
    block_gemm<T, 64, K, 64, NW>(view_k((const float*)Ts, LDF), view_t((const T*)Ks, LDK, nullptr, bs),
                                 NoSkip{}, [&](int r, int c, floatx4 acc) {
                                     store_frag(Wb, (long)H * K, r, c, acc, len);
                                 });
    block_gemm<T, 64, V, 64, NW>(view_k((const float*)Ts, LDF), view_t((const T*)Vs, LDV, nullptr, bs),
                                 NoSkip{}, [&](int r, int c, floatx4 acc) {
                                     store_frag(Ub, (long)H * V, r, c, acc, len);
                                 });
}

// ---------------------------------------------------------------------------
// forward: state scan.  grid (N*H, V/VS).  One workgroup carries S[:, slice]
// (K x VS, fp32) through all chunks of its sequence in MFMA accumulators:
// wave w owns key rows [w*K/4, (w+1)*K/4).  Per chunk it stores the chunk
// start state (bf16/fp32; transposed [v][k] when HT, else [k][v]) and Vn.
// ---------------------------------------------------------------------------
template <typename T, int K, int V, int VS, bool HT>
__global__ void __launch_bounds__(NTH) fwd_state_kernel(const T* __restrict__ k,
                                                        const T* __restrict__ W,
                                                        const T* __restrict__ U, SeqInfo si,
                                                        int H, const float* __restrict__ S0,
                                                        float* __restrict__ ST,
                                                        T* __restrict__ hout,
                                                        T* __restrict__ Vnout) {
    constexpr int P = pad<T>();
    constexpr int LDW = K + P, LDKT = 64 + P, LDST = K + P, LDU = VS + P, LDVN = 64 + P;
    __shared__ __attribute__((aligned(16))) T Ws[64 * LDW];
    __shared__ __attribute__((aligned(16))) T KTs[K * LDKT];
    __shared__ __attribute__((aligned(16))) T STs[VS * LDST];
    __shared__ __attribute__((aligned(16))) T Us[64 * LDU];
    __shared__ __attribute__((aligned(16))) T VnT[VS * LDVN];
    constexpr int RT = K / 64;  // 16-row tiles per wave
    constexpr int CT = VS / 16;
    const int seq = blockIdx.x / H, h = blockIdx.x % H, v0 = blockIdx.y * VS;
    const int w = wave_id(), lane = lane_id();
    long sbos, slen;
    int slot0;
    seq_bounds(si, seq, sbos, slen, slot0);
    const int nch = (int)((slen + BT - 1) / BT);
    const long sbase = ((long)seq * H + h) * K * V;
    floatx4 S[RT][CT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            const int row = w * (K / 4) + rt * 16 + 4 * (lane >> 4);
            const int col = v0 + ct * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                S[rt][ct][i] = S0 ? S0[sbase + (long)(row + i) * V + col] : 0.f;
        }
    for (int n = 0; n < nch; ++n) {
        const long bos = sbos + (long)n * BT;
        const int len = (int)min((long)BT, slen - (long)n * BT);
        const long slot = slot0 + n;
        load_rows<T, 64, K, NTH>(Ws, LDW, W + (bos * H + h) * K, (long)H * K, len);
        load_rows_t<T, 64, K, NTH>(KTs, LDKT, k + (bos * H + h) * K, (long)H * K, len);
        load_rows<T, 64, VS, NTH>(Us, LDU, U + (bos * H + h) * V + v0, (long)H * V, len);
        T* hb = hout + (slot * H + h) * (long)K * V;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                const int row = w * (K / 4) + rt * 16 + 4 * (lane >> 4);
                const int col = ct * 16 + (lane & 15);
                store_frag_t(STs, LDST, row, col, S[rt][ct]);
                if (HT) {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        hb[(long)(v0 + col) * K + row + i] = from_f<T>(S[rt][ct][i]);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        hb[(long)(row + i) * V + v0 + col] = from_f<T>(S[rt][ct][i]);
                }
            }
        __syncthreads();
        T* vnb = Vnout + (bos * H + h) * V + v0;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            floatx4 acc = {0.f, 0.f, 0.f, 0.f};
            acc = tile_mma<T, K>(acc, view_k((const T*)Ws, LDW), 16 * w,
                                 view_k((const T*)STs, LDST), ct * 16, lane);
            const int r = 16 * w + 4 * (lane >> 4), c = ct * 16 + (lane & 15);
            floatx4 vn;
#pragma unroll
            for (int i = 0; i < 4; ++i) vn[i] = to_f(Us[(r + i) * LDU + c]) - acc[i];
            store_frag(vnb, (long)H * V, r, c, vn, len);
            store_frag_t(VnT, LDVN, r, c, vn);
        }
        __syncthreads();
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
                S[rt][ct] = tile_mma<T, 64>(S[rt][ct], view_k((const T*)KTs, LDKT),
                                            w * (K / 4) + rt * 16, view_k((const T*)VnT, LDVN),
                                            ct * 16, lane);
        __syncthreads();
    }
    if (ST) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                const int row = w * (K / 4) + rt * 16 + 4 * (lane >> 4);
                const int col = v0 + ct * 16 + (lane & 15);
#pragma unroll
                for (int i = 0; i < 4; ++i) ST[sbase + (long)(row + i) * V + col] = S[rt][ct][i];
            }
    }
}

// ---------------------------------------------------------------------------
// forward: output.  grid (chunk slots, H, V/VO).  O = Q S + tril(Q K^T) Vn.
// ---------------------------------------------------------------------------
template <typename T, int K, int V, int VO>
__global__ void __launch_bounds__(NTH) fwd_o_kernel(const T* __restrict__ q,
                                                    const T* __restrict__ k,
                                                    const T* __restrict__ hT,
                                                    const T* __restrict__ Vn, SeqInfo si, int H,
                                                    T* __restrict__ o) {
    constexpr int P = pad<T>(), LDQ = K + P, LDP = 64 + P, LDH = K + P, LDVN = 64 + P;
    __shared__ __attribute__((aligned(16))) T Qs[64 * LDQ];
    __shared__ __attribute__((aligned(16))) T Ks[64 * LDQ];
    __shared__ __attribute__((aligned(16))) T Ps[64 * LDP];
    __shared__ __attribute__((aligned(16))) T hTs[VO * LDH];
    __shared__ __attribute__((aligned(16))) T VnT[VO * LDVN];
    const int slot = blockIdx.x, h = blockIdx.y, v0 = blockIdx.z * VO;
    long bos;
    int len;
    if (!locate_chunk(si, slot, bos, len)) return;
    load_rows<T, 64, K, NTH>(Qs, LDQ, q + (bos * H + h) * K, (long)H * K, len);
    load_rows<T, 64, K, NTH>(Ks, LDQ, k + (bos * H + h) * K, (long)H * K, len);
    load_rows<T, VO, K, NTH>(hTs, LDH, hT + (((long)slot * H + h) * V + v0) * K, K, VO);
    load_rows_t<T, 64, VO, NTH>(VnT, LDVN, Vn + (bos * H + h) * V + v0, (long)H * V, len);
    for (int i = threadIdx.x; i < 64 * LDP; i += NTH) Ps[i] = from_f<T>(0.f);
    __syncthreads();
    block_gemm<T, 64, 64, K, NW>(view_k((const T*)Qs, LDQ), view_k((const T*)Ks, LDQ),
                                 SkipUpper{}, [&](int r, int c, floatx4 acc) {
#pragma unroll
                                     for (int i = 0; i < 4; ++i)
                                         if (c <= r + i) Ps[(r + i) * LDP + c] = from_f<T>(acc[i]);
                                 });
    __syncthreads();
    const int w = wave_id(), lane = lane_id();
    T* ob = o + (bos * H + h) * V + v0;
    constexpr int TN = VO / 16;
    for (int t = w; t < 4 * TN; t += NW) {
        const int tm = t / TN, tn = t % TN;
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        acc = tile_mma<T, K>(acc, view_k((const T*)Qs, LDQ), tm * 16, view_k((const T*)hTs, LDH),
                             tn * 16, lane);
        acc = tile_mma<T, 64>(acc, view_k((const T*)Ps, LDP), tm * 16,
                              view_k((const T*)VnT, LDVN), tn * 16, lane);
        store_frag(ob, (long)H * V, tm * 16 + 4 * (lane >> 4), tn * 16 + (lane & 15), acc, len);
    }
}

// ---------------------------------------------------------------------------
// backward: dv_local = tril(Q K^T)^T dO.  grid (chunk slots, H, V/VO)
// ---------------------------------------------------------------------------
template <typename T, int K, int V, int VO>
__global__ void __launch_bounds__(NTH) bwd_dvloc_kernel(const T* __restrict__ q,
                                                        const T* __restrict__ k,
                                                        const T* __restrict__ dO, SeqInfo si,
                                                        int H, T* __restrict__ dVloc) {
    constexpr int P = pad<T>(), LDQ = K + P, LDP = 64 + P, LDO = 64 + P;
    __shared__ __attribute__((aligned(16))) T Qs[64 * LDQ];
    __shared__ __attribute__((aligned(16))) T Ks[64 * LDQ];
    __shared__ __attribute__((aligned(16))) T Pts[64 * LDP];
    __shared__ __attribute__((aligned(16))) T dOT[VO * LDO];
    const int slot = blockIdx.x, h = blockIdx.y, v0 = blockIdx.z * VO;
    long bos;
    int len;
    if (!locate_chunk(si, slot, bos, len)) return;
    load_rows<T, 64, K, NTH>(Qs, LDQ, q + (bos * H + h) * K, (long)H * K, len);
    load_rows<T, 64, K, NTH>(Ks, LDQ, k + (bos * H + h) * K, (long)H * K, len);
    load_rows_t<T, 64, VO, NTH>(dOT, LDO, dO + (bos * H + h) * V + v0, (long)H * V, len);
    for (int i = threadIdx.x; i < 64 * LDP; i += NTH) Pts[i] = from_f<T>(0.f);
    __syncthreads();
    // Pt[j][i] = k_j . q_i for i >= j
    block_gemm<T, 64, 64, K, NW>(view_k((const T*)Ks, LDQ), view_k((const T*)Qs, LDQ),
                                 SkipLower{}, [&](int r, int c, floatx4 acc) {
#pragma unroll
                                     for (int i = 0; i < 4; ++i)
                                         if (c >= r + i) Pts[(r + i) * LDP + c] = from_f<T>(acc[i]);
                                 });
    __syncthreads();
    T* db = dVloc + (bos * H + h) * V + v0;
    block_gemm<T, 64, VO, 64, NW>(view_k((const T*)Pts, LDP), view_k((const T*)dOT, LDO),
                                  NoSkip{}, [&](int r, int c, floatx4 acc) {
                                      store_frag(db, (long)H * V, r, c, acc, len);
                                  });
}

// ---------------------------------------------------------------------------
// backward: reverse state scan.  grid (N*H, V/VS).  dS (K x VS) in MFMA
// accumulators; per chunk (last to first):
//   dh_n = dS                         (gradient of the chunk's end state)
//   dVn  = dv_local + K dS
//   dS  += Q^T dO - W^T dVn
// ---------------------------------------------------------------------------
template <typename T, int K, int V, int VS>
__global__ void __launch_bounds__(NTH) bwd_state_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ W,
    const T* __restrict__ dO, const T* __restrict__ dVloc, SeqInfo si, int H,
    const float* __restrict__ dST, float* __restrict__ dS0, T* __restrict__ dhout,
    T* __restrict__ dVnout) {
    constexpr int P = pad<T>();
    constexpr int LDK = K + P, LDA = 128 + P, LDB = 128 + P, LDS = K + P, LDV = VS + P;
    __shared__ __attribute__((aligned(16))) T Ks[64 * LDK];
    __shared__ __attribute__((aligned(16))) T AT[K * LDA];   // [Q^T | W^T]
    __shared__ __attribute__((aligned(16))) T BTs[VS * LDB]; // [dO ; -dVn] as [v][token]
    __shared__ __attribute__((aligned(16))) T dSTs[VS * LDS];
    __shared__ __attribute__((aligned(16))) T dVl[64 * LDV];
    constexpr int RT = K / 64, CT = VS / 16;
    const int seq = blockIdx.x / H, h = blockIdx.x % H, v0 = blockIdx.y * VS;
    const int w = wave_id(), lane = lane_id();
    long sbos, slen;
    int slot0;
    seq_bounds(si, seq, sbos, slen, slot0);
    const int nch = (int)((slen + BT - 1) / BT);
    const long sbase = ((long)seq * H + h) * K * V;
    floatx4 dS[RT][CT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            const int row = w * (K / 4) + rt * 16 + 4 * (lane >> 4);
            const int col = v0 + ct * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                dS[rt][ct][i] = dST ? dST[sbase + (long)(row + i) * V + col] : 0.f;
        }
    for (int n = nch - 1; n >= 0; --n) {
        const long bos = sbos + (long)n * BT;
        const int len = (int)min((long)BT, slen - (long)n * BT);
        const long slot = slot0 + n;
        load_rows<T, 64, K, NTH>(Ks, LDK, k + (bos * H + h) * K, (long)H * K, len);
        load_rows_t<T, 64, K, NTH>(AT, LDA, q + (bos * H + h) * K, (long)H * K, len);
        load_rows_t<T, 64, K, NTH>(AT + 64, LDA, W + (bos * H + h) * K, (long)H * K, len);
        load_rows_t<T, 64, VS, NTH>(BTs, LDB, dO + (bos * H + h) * V + v0, (long)H * V, len);
        load_rows<T, 64, VS, NTH>(dVl, LDV, dVloc + (bos * H + h) * V + v0, (long)H * V, len);
        T* dhb = dhout + (slot * H + h) * (long)K * V;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                const int row = w * (K / 4) + rt * 16 + 4 * (lane >> 4);
                const int col = ct * 16 + (lane & 15);
                store_frag_t(dSTs, LDS, row, col, dS[rt][ct]);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    dhb[(long)(row + i) * V + v0 + col] = from_f<T>(dS[rt][ct][i]);
            }
        __syncthreads();
        T* dvnb = dVnout + (bos * H + h) * V + v0;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            floatx4 acc = {0.f, 0.f, 0.f, 0.f};
            acc = tile_mma<T, K>(acc, view_k((const T*)Ks, LDK), 16 * w,
                                 view_k((const T*)dSTs, LDS), ct * 16, lane);
            const int r = 16 * w + 4 * (lane >> 4), c = ct * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += to_f(dVl[(r + i) * LDV + c]);
            store_frag(dvnb, (long)H * V, r, c, acc, len);
#pragma unroll
            for (int i = 0; i < 4; ++i) BTs[c * LDB + 64 + r + i] = from_f<T>(-acc[i]);
        }
        __syncthreads();
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
                dS[rt][ct] = tile_mma<T, 128>(dS[rt][ct], view_k((const T*)AT, LDA),
                                              w * (K / 4) + rt * 16, view_k((const T*)BTs, LDB),
                                              ct * 16, lane);
        __syncthreads();
    }
    if (dS0) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                const int row = w * (K / 4) + rt * 16 + 4 * (lane >> 4);
                const int col = v0 + ct * 16 + (lane & 15);
#pragma unroll
                for (int i = 0; i < 4; ++i) dS0[sbase + (long)(row + i) * V + col] = dS[rt][ct][i];
            }
    }
}

// ---------------------------------------------------------------------------
// backward: per chunk dq, the direct part of dk, and dW.  grid (chunk slots, H)
//   Dm = tril(dO Vn^T)
//   dq  = dO h^T + Dm K
//   dk' = Dm^T Q + Vn dh^T
//   dW  = -dVn h^T
// h = chunk start state, dh = gradient of the chunk end state, both [k][v].
// ---------------------------------------------------------------------------
template <typename T, int K, int V>
__global__ void __launch_bounds__(NTH) bwd_dqkw_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ dO,
    const T* __restrict__ Vn, const T* __restrict__ dVn, const T* __restrict__ hst,
    const T* __restrict__ dhst, SeqInfo si, int H, T* __restrict__ dq,
    float* __restrict__ dKp, T* __restrict__ dW) {
    constexpr int P = pad<T>();
    constexpr int LD64 = 64 + P;
    constexpr int SZ_A = 64 * LD64;  // one 64x64 tile buffer
    constexpr int SZ_H = K * LD64;   // one K x 64 buffer
    // phase 1: dOs, Vns, dVns (SZ_A each), hs, dhs (SZ_H each)
    // phase 2: Ds, DsT (overlay dOs, Vns), QT, KT (overlay hs, dhs)
    __shared__ __attribute__((aligned(16))) T smem[3 * SZ_A + 2 * SZ_H];
    T* dOs = smem;
    T* Vns = smem + SZ_A;
    T* dVns = smem + 2 * SZ_A;
    T* hs = smem + 3 * SZ_A;
    T* dhs = hs + SZ_H;
    T* Ds = dOs;
    T* DsT = Vns;
    T* QT = hs;
    T* KT = dhs;
    const int slot = blockIdx.x, h = blockIdx.y;
    long bos;
    int len;
    if (!locate_chunk(si, slot, bos, len)) return;
    const int w = wave_id(), lane = lane_id();
    constexpr int TNK = K / 16;
    constexpr int TPW = 4 * TNK / NW;  // 64 x K tiles per wave
    floatx4 aq[TPW], ak[TPW], aw[TPW], am[4];
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) aq[j][i] = ak[j][i] = aw[j][i] = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) am[j][i] = 0.f;
    const long hbase = ((long)slot * H + h) * K * V;
    for (int vt = 0; vt < V / 64; ++vt) {
        const int v0 = vt * 64;
        load_rows<T, 64, 64, NTH>(dOs, LD64, dO + (bos * H + h) * V + v0, (long)H * V, len);
        load_rows<T, 64, 64, NTH>(Vns, LD64, Vn + (bos * H + h) * V + v0, (long)H * V, len);
        load_rows<T, 64, 64, NTH>(dVns, LD64, dVn + (bos * H + h) * V + v0, (long)H * V, len);
        load_rows<T, K, 64, NTH>(hs, LD64, hst + hbase + v0, V, K);
        load_rows<T, K, 64, NTH>(dhs, LD64, dhst + hbase + v0, V, K);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = w + NW * j, tm = t / 4, tn = t % 4;
            am[j] = tile_mma<T, 64>(am[j], view_k((const T*)dOs, LD64), tm * 16,
                                    view_k((const T*)Vns, LD64), tn * 16, lane);
        }
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
            const int t = w + NW * j, tm = t / TNK, tn = t % TNK;
            aq[j] = tile_mma<T, 64>(aq[j], view_k((const T*)dOs, LD64), tm * 16,
                                    view_k((const T*)hs, LD64), tn * 16, lane);
            ak[j] = tile_mma<T, 64>(ak[j], view_k((const T*)Vns, LD64), tm * 16,
                                    view_k((const T*)dhs, LD64), tn * 16, lane);
            aw[j] = tile_mma<T, 64>(aw[j], view_k((const T*)dVns, LD64), tm * 16,
                                    view_k((const T*)hs, LD64), tn * 16, lane);
        }
        __syncthreads();
    }
    // phase 2
    for (int i = threadIdx.x; i < 2 * SZ_A; i += NTH) smem[i] = from_f<T>(0.f);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int t = w + NW * j, tm = t / 4, tn = t % 4;
        const int r = tm * 16 + 4 * (lane >> 4), c = tn * 16 + (lane & 15);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float x = (c <= r + i) ? am[j][i] : 0.f;
            Ds[(r + i) * LD64 + c] = from_f<T>(x);
            DsT[c * LD64 + r + i] = from_f<T>(x);
        }
    }
    load_rows_t<T, 64, K, NTH>(QT, LD64, q + (bos * H + h) * K, (long)H * K, len);
    load_rows_t<T, 64, K, NTH>(KT, LD64, k + (bos * H + h) * K, (long)H * K, len);
    __syncthreads();
    T* dqb = dq + (bos * H + h) * K;
    float* dkb = dKp + (bos * H + h) * K;
    T* dwb = dW + (bos * H + h) * K;
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
        const int t = w + NW * j, tm = t / TNK, tn = t % TNK;
        aq[j] = tile_mma<T, 64>(aq[j], view_k((const T*)Ds, LD64), tm * 16,
                                view_k((const T*)KT, LD64), tn * 16, lane);
        ak[j] = tile_mma<T, 64>(ak[j], view_k((const T*)DsT, LD64), tm * 16,
                                view_k((const T*)QT, LD64), tn * 16, lane);
        const int r = tm * 16 + 4 * (lane >> 4), c = tn * 16 + (lane & 15);
        floatx4 nw;
#pragma unroll
        for (int i = 0; i < 4; ++i) nw[i] = -aw[j][i];
        store_frag(dqb, (long)H * K, r, c, aq[j], len);
        store_frag(dkb, (long)H * K, r, c, ak[j], len);
        store_frag(dwb, (long)H * K, r, c, nw, len);
    }
}

// Sum x over the 16 lanes that share (lane >> 4), i.e. over the columns of a
// C fragment row group; every lane receives the sum.
__device__ __forceinline__ float sum16(float x) {
    x += __shfl_xor(x, 1);
    x += __shfl_xor(x, 2);
    x += __shfl_xor(x, 4);
    x += __shfl_xor(x, 8);
    return x;
}

// ---------------------------------------------------------------------------
// backward: WY part.  grid (chunk slots, H).  Carries dW (C x K) and dU = dVn
// (C x V) through W = T D K, U = T D V, T = (I + A)^{-1},
// A = strict_lower(D K K^T) and b = c(beta, |k|^2):
//   dT  = dW (DK)^T + dU (DV)^T
//   dk  = dk' + D T^T dW + (E + E^T) K + 2 db dc/dlambda k,  E = D dA
//   dv  = D T^T dU
//   dA  = strict_lower(-T^T dT T^T)
//   db  = rowsum(T^T dW o K) + rowsum(T^T dU o V) + rowsum(dA o K K^T)
//   dbeta = db * exp(-beta lambda)
// ---------------------------------------------------------------------------
template <typename T, int K, int V>
__global__ void __launch_bounds__(NTH) bwd_wy_kernel(
    const T* __restrict__ k, const T* __restrict__ v, const T* __restrict__ beta,
    const T* __restrict__ dWg, const T* __restrict__ dUg, const float* __restrict__ dKp,
    SeqInfo si, int H, T* __restrict__ dk, T* __restrict__ dv, T* __restrict__ dbeta) {
    constexpr int P = pad<T>(), LDK = K + P, LD64 = 64 + P;
    __shared__ __attribute__((aligned(16))) T Ks[64 * LDK];
    __shared__ __attribute__((aligned(16))) T dWs[64 * LDK];
    __shared__ __attribute__((aligned(16))) T Vt[64 * LD64];
    __shared__ __attribute__((aligned(16))) T dUt[64 * LD64];
    __shared__ __attribute__((aligned(16))) float Gs[64 * LDF];
    __shared__ __attribute__((aligned(16))) float Ts[64 * LDF];
    __shared__ __attribute__((aligned(16))) float As[64 * LDF];
    __shared__ __attribute__((aligned(16))) float Xs[64 * LDF];
    __shared__ float Ysc[4 * 16 * 17];
    __shared__ float bs[64], dcls[64], dcbs[64], dbs[64];
    const int slot = blockIdx.x, h = blockIdx.y;
    long bos;
    int len;
    if (!locate_chunk(si, slot, bos, len)) return;
    const int w = wave_id(), lane = lane_id();
    load_rows<T, 64, K, NTH>(Ks, LDK, k + (bos * H + h) * K, (long)H * K, len);
    load_rows<T, 64, K, NTH>(dWs, LDK, dWg + (bos * H + h) * K, (long)H * K, len);
    if (threadIdx.x < 64) dbs[threadIdx.x] = 0.f;
    __syncthreads();
    chunk_coeffs<T, K>(Ks, LDK, beta, bos, H, h, len, bs, dcls, dcbs, nullptr);
    compute_T<T, K>(Ks, LDK, bs, Gs, Ts, Ysc);

    // dT (all 16 tiles, 4 per wave) and dv, tile by tile over V
    floatx4 dT[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int t = w + NW * j, tm = t / 4, tn = t % 4;
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        dT[j] = tile_mma<T, K>(acc, view_k((const T*)dWs, LDK), tm * 16,
                               view_k((const T*)Ks, LDK, (const float*)bs), tn * 16, lane);
    }
    T* dvb = dv + (bos * H + h) * V;
    for (int vt = 0; vt < V / 64; ++vt) {
        const int v0 = vt * 64;
        load_rows<T, 64, 64, NTH>(Vt, LD64, v + (bos * H + h) * V + v0, (long)H * V, len);
        load_rows<T, 64, 64, NTH>(dUt, LD64, dUg + (bos * H + h) * V + v0, (long)H * V, len);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = w + NW * j, tm = t / 4, tn = t % 4;
            dT[j] = tile_mma<T, 64>(dT[j], view_k((const T*)dUt, LD64), tm * 16,
                                    view_k((const T*)Vt, LD64, (const float*)bs), tn * 16, lane);
            floatx4 acc = {0.f, 0.f, 0.f, 0.f};
            acc = tile_mma<T, 64>(acc, view_t((const float*)Ts, LDF), tm * 16,
                                  view_t((const T*)dUt, LD64), tn * 16, lane);
            const int r = tm * 16 + 4 * (lane >> 4), c = tn * 16 + (lane & 15);
            floatx4 dvv;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                dvv[i] = bs[r + i] * acc[i];
                const float part = sum16(acc[i] * to_f(Vt[(r + i) * LD64 + c]));
                if ((lane & 15) == 0) atomicAdd(&dbs[r + i], part);
            }
            store_frag(dvb + v0, (long)H * V, r, c, dvv, len);
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int t = w + NW * j, tm = t / 4, tn = t % 4;
        const int r = tm * 16 + 4 * (lane >> 4), c = tn * 16 + (lane & 15);
#pragma unroll
        for (int i = 0; i < 4; ++i) As[(r + i) * LDF + c] = dT[j][i];
    }
    // dk accumulation: dk' + D T^T dW
    constexpr int TNK = K / 16;
    constexpr int TPW = 4 * TNK / NW;
    floatx4 akk[TPW];
    const float* dkp = dKp + (bos * H + h) * K;
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
        const int t = w + NW * j, tm = t / TNK, tn = t % TNK;
        const int r = tm * 16 + 4 * (lane >> 4), c = tn * 16 + (lane & 15);
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        acc = tile_mma<T, 64>(acc, view_t((const float*)Ts, LDF), tm * 16,
                              view_t((const T*)dWs, LDK), tn * 16, lane);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float base = (r + i < len) ? dkp[(long)(r + i) * H * K + c] : 0.f;
            akk[j][i] = base + bs[r + i] * acc[i];
            const float part = sum16(acc[i] * to_f(Ks[(r + i) * LDK + c]));
            if ((lane & 15) == 0) atomicAdd(&dbs[r + i], part);
        }
    }
    __syncthreads();
    // X = dT T^T
    block_gemm<T, 64, 64, 64, NW>(view_k((const float*)As, LDF), view_k((const float*)Ts, LDF),
                                  NoSkip{}, [&](int r, int c, floatx4 acc) {
#pragma unroll
                                      for (int i = 0; i < 4; ++i) Xs[(r + i) * LDF + c] = acc[i];
                                  });
    __syncthreads();
    // dA = strict_lower(-T^T X); E = D dA -> As; db += rowsum(dA o G)
    block_gemm<T, 64, 64, 64, NW>(view_t((const float*)Ts, LDF), view_t((const float*)Xs, LDF),
                                  NoSkip{}, [&](int r, int c, floatx4 acc) {
#pragma unroll
                                      for (int i = 0; i < 4; ++i) {
                                          const int row = r + i;
                                          const float da = (c < row) ? -acc[i] : 0.f;
                                          As[row * LDF + c] = bs[row] * da;
                                          const float g = (c < row) ? Gs[row * LDF + c] : 0.f;
                                          const float part = sum16(da * g);
                                          if ((lane & 15) == 0) atomicAdd(&dbs[row], part);
                                      }
                                  });
    __syncthreads();
    // F = E + E^T -> Xs
    for (int idx = threadIdx.x; idx < 64 * 64; idx += NTH) {
        const int i = idx >> 6, j = idx & 63;
        Xs[i * LDF + j] = As[i * LDF + j] + As[j * LDF + i];
    }
    __syncthreads();
    T* dkb = dk + (bos * H + h) * K;
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
        const int t = w + NW * j, tm = t / TNK, tn = t % TNK;
        akk[j] = tile_mma<T, 64>(akk[j], view_k((const float*)Xs, LDF), tm * 16,
                                 view_t((const T*)Ks, LDK), tn * 16, lane);
        const int r = tm * 16 + 4 * (lane >> 4), c = tn * 16 + (lane & 15);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            akk[j][i] += 2.f * dbs[r + i] * dcls[r + i] * to_f(Ks[(r + i) * LDK + c]);
        store_frag(dkb, (long)H * K, r, c, akk[j], len);
    }
    if (threadIdx.x < len)
        dbeta[(bos + threadIdx.x) * H + h] = from_f<T>(dbs[threadIdx.x] * dcbs[threadIdx.x]);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct Carve {
    char* base;
    size_t off = 0;
    explicit Carve(void* b) : base((char*)b) {}
    template <typename X>
    X* take(size_t n) {
        off = (off + 255) & ~(size_t)255;
        X* p = base ? (X*)(base + off) : nullptr;
        off += n * sizeof(X);
        return p;
    }
};

struct Problem {
    long ntok;      // total tokens
    int N;          // sequences
    long T;         // tokens per sequence (fixed-length case)
    int H, K, V;
    bool varlen;
    long slots;     // chunk slots launched for per-chunk kernels
    int nt;         // chunks per sequence (fixed-length case)
    TokLd ld;       // token strides of q, k, v, dq, dk, dv (bf16 path)
};

// Workspace layouts.  The forward's layout is a prefix of the backward's:
// sequence offsets, the per-chunk WY data (bf16 T and fp32 b on the bf16 path;
// W, U and per-token b on the generic path), then the chunk states h and, on
// the bf16 path, the chunks' P = tril(Q K^T) (on the generic path, Vn).  A backward call given the forward's workspace finds
// the forward's factors, and its saved states, in place.
template <typename T>
struct FwdWs {
    int32_t *cu_s, *coff, *order;
    T *W, *U;     // generic path
    bf16* Tc;     // bf16 path
    float* bc;    // bf16 path
    float* dcc;   // bf16 path: dc/dlambda, dc/dbeta per token
    float* bco;   // generic path
    T* h;         // generic path; bf16 path when the states are saved
    bf16* Pc;     // bf16 path when the states are saved
    T* Vn;        // generic path
};

template <typename T>
struct BwdWs {
    int32_t *cu_s, *coff, *order;
    T *W, *U;
    bf16* Tc;
    float* bc;
    float* dcc;  // bf16 path: dc/dlambda, dc/dbeta per token, as the forward's prep wrote them
    float* bco;  // generic path
    T* h;        // chunk start states
    bf16* Pc;    // bf16 path: tril(Q K^T) per chunk, as the forward saved it
    T* Vn;       // generic path
    T* dh;       // chunk end-state gradients
    T *dvloc, *dVn, *dW;  // generic path
    float* dKp;           // generic path
};

// Takes the common prefix; returns with `c` at the end of h (and Vn).
template <typename T>
static void carve_prefix(const Problem& p, Carve& c, int32_t** cu_s, int32_t** coff,
                         int32_t** order, T** W, T** U, bf16** Tc, float** bc, float** dcc,
                         float** bco, T** h, bf16** Pc, T** Vn, bool with_h) {
    *cu_s = c.take<int32_t>(p.N + 1);
    *coff = c.take<int32_t>(p.N + 1);
    // room for the sequence order whenever it can be used (the size queries
    // do not know whether the call will be varlen)
    *order = p.N <= LPT_MAX_SEQS ? c.take<int32_t>(p.N) : nullptr;
    *W = *U = nullptr;
    *Tc = nullptr;
    *bc = *dcc = *bco = nullptr;
    *h = *Vn = nullptr;
    *Pc = nullptr;
    if (__is_same(T, bf16)) {
        *Tc = c.take<bf16>((size_t)p.slots * p.H * fast::TRI_ELEMS);
        *bc = c.take<float>((size_t)p.slots * p.H * 64);
        *dcc = c.take<float>((size_t)p.slots * p.H * 128);
        if (with_h) {
            *h = c.take<T>((size_t)p.slots * p.H * p.K * p.V);
            *Pc = c.take<bf16>((size_t)p.slots * p.H * fast::TRI_ELEMS);
        }
    } else {
        *W = c.take<T>((size_t)p.ntok * p.H * p.K);
        *U = c.take<T>((size_t)p.ntok * p.H * p.V);
        *bco = c.take<float>((size_t)p.ntok * p.H);
        *h = c.take<T>((size_t)p.slots * p.H * p.K * p.V);
        *Vn = c.take<T>((size_t)p.ntok * p.H * p.V);
    }
}

// with_states: room for the bf16 path's chunk states (the generic path always
// keeps them)
template <typename T>
static size_t carve_fwd(const Problem& p, void* base, FwdWs<T>* out, bool with_states) {
    Carve c(base);
    FwdWs<T> w{};
    carve_prefix<T>(p, c, &w.cu_s, &w.coff, &w.order, &w.W, &w.U, &w.Tc, &w.bc, &w.dcc,
                    &w.bco, &w.h, &w.Pc, &w.Vn, with_states);
    if (out) *out = w;
    return c.off + 256;
}

template <typename T>
static size_t carve_bwd(const Problem& p, void* base, BwdWs<T>* out) {
    Carve c(base);
    BwdWs<T> w{};
    carve_prefix<T>(p, c, &w.cu_s, &w.coff, &w.order, &w.W, &w.U, &w.Tc, &w.bc, &w.dcc,
                    &w.bco, &w.h, &w.Pc, &w.Vn, true);
    w.dh = c.take<T>((size_t)p.slots * p.H * p.K * p.V);
    if (!__is_same(T, bf16)) {
        w.dvloc = c.take<T>((size_t)p.ntok * p.H * p.V);
        w.dVn = c.take<T>((size_t)p.ntok * p.H * p.V);
        w.dW = c.take<T>((size_t)p.ntok * p.H * p.K);
        w.dKp = c.take<float>((size_t)p.ntok * p.H * p.K);
    }
    if (out) *out = w;
    return c.off + 256;
}

constexpr int VS = 64;  // value slice of the state scans
constexpr int VO = 64;  // value tile of the per-chunk output kernels

static SeqInfo make_seqinfo(const Problem& p, const int32_t* cu_s, const int32_t* coff,
                           const int32_t* order) {
    SeqInfo s;
    s.cu = p.varlen ? cu_s : nullptr;
    s.coff = p.varlen ? coff : nullptr;
    s.order = p.varlen ? order : nullptr;
    s.N = p.N;
    s.T = p.T;
    s.nt = p.nt;
    return s;
}

static int build_offsets(const Problem& p, const int32_t* cu, int32_t* cu_s, int32_t* coff,
                         int32_t* order, hipStream_t st) {
    if (!p.varlen) return kSuccess;
    EFLA_LAUNCH("efla_q_chunk_offsets", chunk_offsets_kernel, dim3(1), dim3(1024), st, cu, p.N,
                p.ntok, cu_s, coff, order);
    return (int)hipPeekAtLastError();
}

template <typename T, int K, int V>
static int run_fwd(const Problem& p, const T* q, const T* k, const T* v, const T* beta,
                   const float* S0, T* o, float* ST, const int32_t* cu, void* ws,
                   bool save_states, hipStream_t st) {
    FwdWs<T> w;
    carve_fwd<T>(p, ws, &w, save_states);
    EFLA_CHECK((hipError_t)build_offsets(p, cu, w.cu_s, w.coff, w.order, st));
    const SeqInfo si = make_seqinfo(p, w.cu_s, w.coff, w.order);
    const int H = p.H;
    if constexpr (__is_same(T, bf16)) {
        EFLA_LAUNCH("efla_q_fwd_prep", (fast::prep_kernel<K>), dim3(H, p.slots),
                    dim3(fast::NT), st, k, beta, si, H, w.Tc, w.bc, w.dcc, p.ld.k);
        EFLA_LAUNCH("efla_q_fwd_scan", (fast::scan_o_kernel<K, V>),
                    dim3(p.N * H * (V / fast::VS)), dim3(fast::NTS), st, q, k, v, w.Tc, w.bc, si,
                    H, S0, ST, o, w.h, w.Pc, p.ld);
        return (int)hipPeekAtLastError();
    }
    EFLA_LAUNCH("efla_q_fwd_prep", (fwd_prep_kernel<T, K, V>), dim3(p.slots, H), dim3(NTH), st,
                k, v, beta, si, H, w.bco, w.W, w.U);
    EFLA_LAUNCH("efla_q_fwd_state", (fwd_state_kernel<T, K, V, VS, true>),
                dim3(p.N * H, V / VS), dim3(NTH), st, k, w.W, w.U, si, H, S0, ST, w.h, w.Vn);
    EFLA_LAUNCH("efla_q_fwd_o", (fwd_o_kernel<T, K, V, VO>), dim3(p.slots, H, V / VO),
                dim3(NTH), st, q, k, w.h, w.Vn, si, H, o);
    return (int)hipPeekAtLastError();
}

template <typename T, int K, int V>
static int run_bwd(const Problem& p, const T* q, const T* k, const T* v, const T* beta,
                   const float* S0, const T* dO, const float* dST, T* dq, T* dk, T* dv,
                   T* dbeta, float* dS0, const int32_t* cu, void* ws, bool reuse,
                   bool reuse_states, hipStream_t st) {
    BwdWs<T> w;
    carve_bwd<T>(p, ws, &w);
    EFLA_CHECK((hipError_t)build_offsets(p, cu, w.cu_s, w.coff, w.order, st));
    const SeqInfo si = make_seqinfo(p, w.cu_s, w.coff, w.order);
    const int H = p.H;
    // forward recompute: the WY factors unless the forward's are in the
    // workspace (reuse), the chunk states unless the forward saved them
    if constexpr (__is_same(T, bf16)) {
        const dim3 scan_grid(p.N * H * (V / fast::VS));
        if (!reuse)
            EFLA_LAUNCH("efla_q_bwd_re_prep", (fast::prep_kernel<K>), dim3(H, p.slots),
                        dim3(fast::NT), st, k, beta, si, H, w.Tc, w.bc, w.dcc, p.ld.k);
        if (!reuse_states)
            EFLA_LAUNCH("efla_q_bwd_re_state", (fast::scan_h_kernel<K, V>), scan_grid,
                        dim3(fast::NT), st, k, v, (const bf16*)w.Tc, (const float*)w.bc, si, H,
                        S0, w.h, p.ld);
        // persistent gradient kernel: one workgroup per CU (its LDS allows no
        // more), each looping over (chunk, head) items.  EFLA_GRAD_WORKGROUPS
        // caps the grid (tests use it to run many items per workgroup at
        // small sizes; the results do not depend on the grid)
        const int nitems = H * p.slots;
        int ncu = device_cu_count();
        if (const char* cap = getenv("EFLA_GRAD_WORKGROUPS")) {
            const int c = atoi(cap);
            if (c > 0 && (ncu <= 0 || c < ncu)) ncu = c;
        }
        const dim3 grad_grid((unsigned)(ncu > 0 && ncu < nitems ? ncu : nitems));
        // the forward that saved the states also saved each chunk's P.  The
        // gradient kernel runs 16 waves (four per SIMD) where its registers
        // allow it without spills (d_v <= 128), else 8
        constexpr int NG = V <= 128 ? 4 : 2;
        if (reuse_states) {
            EFLA_LAUNCH("efla_q_bwd_state", (fast::scan_dh_kernel<K, V, true>), scan_grid,
                        dim3(fast::dh_threads<K>()), st, q, k, dO, (const bf16*)w.Tc, (const float*)w.bc,
                        (const bf16*)w.Pc, si, H, dST, dS0, w.dh, p.ld);
            EFLA_LAUNCH("efla_q_bwd_grad", (fast::grad_kernel<K, V, true, NG>), grad_grid,
                        dim3(fast::grad_threads<NG>()), st, q, k, v, dO, (const bf16*)w.Tc,
                        (const float*)w.bc, (const float*)w.dcc, (const bf16*)w.Pc, w.h, w.dh,
                        si, H, nitems, dq, dk, dv, dbeta, p.ld);
        } else {
            EFLA_LAUNCH("efla_q_bwd_state", (fast::scan_dh_kernel<K, V, false>), scan_grid,
                        dim3(fast::dh_threads<K>()), st, q, k, dO, (const bf16*)w.Tc, (const float*)w.bc,
                        (const bf16*)nullptr, si, H, dST, dS0, w.dh, p.ld);
            EFLA_LAUNCH("efla_q_bwd_grad", (fast::grad_kernel<K, V, false, NG>), grad_grid,
                        dim3(fast::grad_threads<NG>()), st, q, k, v, dO, (const bf16*)w.Tc,
                        (const float*)w.bc, (const float*)w.dcc, (const bf16*)nullptr, w.h, w.dh,
                        si, H, nitems, dq, dk, dv, dbeta, p.ld);
        }
        return (int)hipPeekAtLastError();
    } else if (!reuse) {
        EFLA_LAUNCH("efla_q_bwd_re_prep", (fwd_prep_kernel<T, K, V>), dim3(p.slots, H),
                    dim3(NTH), st, k, v, beta, si, H, w.bco, w.W, w.U);
    }
    // the generic forward keeps its states transposed for its output kernel,
    // so this path recomputes them whatever reuse_states says
    EFLA_LAUNCH("efla_q_bwd_re_state", (fwd_state_kernel<T, K, V, VS, false>),
                dim3(p.N * H, V / VS), dim3(NTH), st, k, w.W, w.U, si, H, S0, (float*)nullptr,
                w.h, w.Vn);
    EFLA_LAUNCH("efla_q_bwd_dvloc", (bwd_dvloc_kernel<T, K, V, VO>), dim3(p.slots, H, V / VO),
                dim3(NTH), st, q, k, dO, si, H, w.dvloc);
    EFLA_LAUNCH("efla_q_bwd_state", (bwd_state_kernel<T, K, V, VS>), dim3(p.N * H, V / VS),
                dim3(NTH), st, q, k, w.W, dO, w.dvloc, si, H, dST, dS0, w.dh, w.dVn);
    EFLA_LAUNCH("efla_q_bwd_dqkw", (bwd_dqkw_kernel<T, K, V>), dim3(p.slots, H), dim3(NTH), st,
                q, k, dO, w.Vn, w.dVn, w.h, w.dh, si, H, dq, w.dKp, w.dW);
    EFLA_LAUNCH("efla_q_bwd_wy", (bwd_wy_kernel<T, K, V>), dim3(p.slots, H), dim3(NTH), st, k,
                v, beta, w.dW, w.dVn, w.dKp, si, H, dk, dv, dbeta);
    return (int)hipPeekAtLastError();
}

// (dtype, K, V) combinations compiled in.
static bool supported(int dtype, size_t K, size_t V) {
    if (dtype == kDtypeBF16)
        return (K == 64 || K == 128) && (V == 64 || V == 128 || V == 256);
    if (dtype == kDtypeF32) return K == 64 && V == 64;
    return false;
}

#define EFLA_Q_DISPATCH_BF16(FN, ...)                                           \
    do {                                                                        \
        if (p.K == 64 && p.V == 64) return FN<bf16, 64, 64>(__VA_ARGS__);       \
        if (p.K == 64 && p.V == 128) return FN<bf16, 64, 128>(__VA_ARGS__);     \
        if (p.K == 64 && p.V == 256) return FN<bf16, 64, 256>(__VA_ARGS__);     \
        if (p.K == 128 && p.V == 64) return FN<bf16, 128, 64>(__VA_ARGS__);     \
        if (p.K == 128 && p.V == 128) return FN<bf16, 128, 128>(__VA_ARGS__);   \
        if (p.K == 128 && p.V == 256) return FN<bf16, 128, 256>(__VA_ARGS__);   \
    } while (0)

// Validates the Mode Q arguments and fills `p`.  Returns kSuccess, or the
// error code to return; *empty is set when there are no tokens to process.
static int make_problem(const void* q, const void* k, const void* v, const void* beta,
                        const int32_t* cu, size_t batch, size_t seq_len, size_t num_seqs,
                        size_t H, size_t K, size_t V, size_t chunk, int dtype, Problem* p,
                        bool* empty) {
    *empty = false;
    if (H == 0 || K == 0 || V == 0) return kInvalidValue;
    if (chunk != 0 && chunk != (size_t)BT) return kInvalidValue;
    if (!supported(dtype, K, V)) return kInvalidValue;
    if (cu == nullptr) {
        if (batch == 0) return kInvalidValue;
        if (num_seqs != 0 && num_seqs != batch) return kInvalidValue;
        num_seqs = batch;
    } else {
        if (batch != 1 || num_seqs == 0) return kInvalidValue;
    }
    size_t ntok, elems;
    if (!mul_ok(batch, seq_len, &ntok)) return kInvalidConfiguration;
    if (!mul_ok(ntok, H, (K > V ? K : V), &elems) || elems > ((size_t)1 << 46))
        return kInvalidConfiguration;
    // 64 token rows of a chunk span < 2^32 bytes (32-bit tile offsets)
    if (H >= ((size_t)1 << 24) || H * (K > V ? K : V) >= ((size_t)1 << 24))
        return kInvalidConfiguration;
    if (num_seqs > (size_t)INT32_MAX / 2 || ntok > (size_t)INT32_MAX)
        return kInvalidConfiguration;
    p->ntok = (long)ntok;
    p->N = (int)num_seqs;
    p->H = (int)H;
    p->K = (int)K;
    p->V = (int)V;
    p->varlen = cu != nullptr;
    p->T = p->varlen ? 0 : (long)seq_len;
    p->nt = p->varlen ? 0 : (int)((seq_len + BT - 1) / BT);
    p->slots = p->varlen ? (long)(ntok / BT + num_seqs) : (long)num_seqs * p->nt;
    p->ld = TokLd{(long)(H * K), (long)(H * K), (long)(H * V), (long)(H * K), (long)(H * K),
                  (long)(H * V)};
    if ((size_t)p->N * H > (size_t)INT32_MAX || (size_t)p->slots > (size_t)INT32_MAX)
        return kInvalidConfiguration;
    if (seq_len == 0) {
        *empty = true;
        return kSuccess;
    }
    if (!q || !k || !v || !beta) return kInvalidValue;
    return kSuccess;
}

}  // namespace q
}  // namespace efla

using namespace efla;
using namespace efla::q;

// Workspace bound covering both the fixed-length and the packed layout of
// batch_size * seq_len tokens in max(num_seqs, batch_size) sequences.
static bool ws_problem(size_t batch, size_t seq_len, size_t num_seqs, size_t H, size_t K,
                       size_t V, int dtype, Problem* p) {
    if (H == 0 || K == 0 || V == 0 || !supported(dtype, K, V)) return false;
    size_t ntok;
    if (!mul_ok(batch, seq_len, &ntok) || ntok > (size_t)INT32_MAX) return false;
    const size_t N = num_seqs > batch ? num_seqs : batch;
    if (N == 0 || N > (size_t)INT32_MAX / 2) return false;
    p->ntok = (long)ntok;
    p->N = (int)N;
    p->H = (int)H;
    p->K = (int)K;
    p->V = (int)V;
    p->varlen = false;
    p->T = (long)seq_len;
    p->nt = (int)((seq_len + BT - 1) / BT);
    const size_t fixed = batch * (size_t)p->nt;
    const size_t packed = ntok / BT + N;
    p->slots = (long)(fixed > packed ? fixed : packed);
    return true;
}

extern "C" size_t efla_chunk_fwd_workspace_size(size_t batch_size, size_t seq_len,
                                                size_t num_seqs, size_t num_heads,
                                                size_t head_dim_k, size_t head_dim_v,
                                                int dtype) {
    Problem p;
    if (!ws_problem(batch_size, seq_len, num_seqs, num_heads, head_dim_k, head_dim_v, dtype, &p))
        return 0;
    return dtype == kDtypeBF16 ? carve_fwd<bf16>(p, nullptr, nullptr, false)
                               : carve_fwd<float>(p, nullptr, nullptr, false);
}

extern "C" size_t efla_chunk_bwd_workspace_size(size_t batch_size, size_t seq_len,
                                                size_t num_seqs, size_t num_heads,
                                                size_t head_dim_k, size_t head_dim_v,
                                                int dtype) {
    Problem p;
    if (!ws_problem(batch_size, seq_len, num_seqs, num_heads, head_dim_k, head_dim_v, dtype, &p))
        return 0;
    return dtype == kDtypeBF16 ? carve_bwd<bf16>(p, nullptr, nullptr)
                               : carve_bwd<float>(p, nullptr, nullptr);
}

// Token strides of the strided entry points (NULL: packed), in the order
// q, k, v[, dq, dk, dv].  A stride other than the packed one (H*K or H*V
// elements) is at least that, a multiple of 8 elements (whole 16-byte row
// pieces) and below 2^24 (the kernels' 32-bit offsets within a 64-token
// chunk); its pointer must then be 16-byte aligned.  Only the bf16 kernels
// take non-packed strides.
static int apply_strides(Problem* p, const int64_t* ts, int n, int dtype,
                         const void* const* ptrs) {
    if (ts == nullptr) return kSuccess;
    long ld[6] = {p->ld.q, p->ld.k, p->ld.v, p->ld.dq, p->ld.dk, p->ld.dv};
    bool custom = false;
    for (int i = 0; i < n; ++i) {
        const int64_t s = ts[i];
        if (s == ld[i]) continue;
        if (s < ld[i] || s % 8 != 0 || s >= ((int64_t)1 << 24)) return kInvalidValue;
        if (ptrs[i] != nullptr && ((uintptr_t)ptrs[i] & 15) != 0) return kInvalidValue;
        if ((uint64_t)p->ntok * (uint64_t)s > ((uint64_t)1 << 46)) return kInvalidConfiguration;
        ld[i] = (long)s;
        custom = true;
    }
    if (custom && dtype != kDtypeBF16) return kNotSupported;
    p->ld = TokLd{ld[0], ld[1], ld[2], ld[3], ld[4], ld[5]};
    return kSuccess;
}

static int chunk_fwd(const void* q, const void* k, const void* v, const void* beta,
                     const float* initial_state, void* output, float* final_state,
                     const int32_t* cu_seqlens, size_t batch_size, size_t seq_len,
                     size_t num_seqs, size_t num_heads, size_t head_dim_k, size_t head_dim_v,
                     size_t chunk_size, int dtype, void* workspace, size_t workspace_bytes,
                     unsigned flags, const int64_t* token_strides, hipStream_t stream) {
    Problem p;
    bool empty;
    int rc = make_problem(q, k, v, beta, cu_seqlens, batch_size, seq_len, num_seqs, num_heads,
                          head_dim_k, head_dim_v, chunk_size, dtype, &p, &empty);
    if (rc != kSuccess) return rc;
    {
        const void* ptrs[3] = {q, k, v};
        rc = apply_strides(&p, token_strides, 3, dtype, ptrs);
        if (rc != kSuccess) return rc;
    }
    if ((flags & ~(unsigned)EFLA_FWD_SAVE_STATES) != 0) return kInvalidValue;
    const bool save = (flags & EFLA_FWD_SAVE_STATES) != 0;
    if (save && workspace == nullptr) return kInvalidValue;
    const size_t sbytes = (size_t)p.N * p.H * p.K * p.V * sizeof(float);
    if (empty) {
        if (final_state == nullptr) return kSuccess;
        if (initial_state)
            return (int)hipMemcpyAsync(final_state, initial_state, sbytes,
                                       hipMemcpyDeviceToDevice, stream);
        return fill_zero(final_state, sbytes, stream);
    }
    if (output == nullptr) return kInvalidValue;
    const size_t need = dtype == kDtypeBF16 ? carve_fwd<bf16>(p, nullptr, nullptr, save)
                                            : carve_fwd<float>(p, nullptr, nullptr, save);
    void* ws = workspace;
    WsLease lease;
    if (ws == nullptr) {
        rc = workspace_acquire(need, stream, &ws, lease);
        if (rc != kSuccess) return rc;
    } else if (workspace_bytes < need) {
        return kInvalidValue;
    }
    if (dtype == kDtypeBF16) {
        EFLA_Q_DISPATCH_BF16(run_fwd, p, (const bf16*)q, (const bf16*)k, (const bf16*)v,
                             (const bf16*)beta, initial_state, (bf16*)output, final_state,
                             cu_seqlens, ws, save, stream);
    } else {
        return run_fwd<float, 64, 64>(p, (const float*)q, (const float*)k, (const float*)v,
                                      (const float*)beta, initial_state, (float*)output,
                                      final_state, cu_seqlens, ws, save, stream);
    }
    return kInvalidValue;
}

static int chunk_bwd(const void* q, const void* k, const void* v, const void* beta,
                     const float* initial_state, const void* grad_output,
                     const float* grad_final_state, void* grad_q, void* grad_k, void* grad_v,
                     void* grad_beta, float* grad_initial_state, const int32_t* cu_seqlens,
                     size_t batch_size, size_t seq_len, size_t num_seqs, size_t num_heads,
                     size_t head_dim_k, size_t head_dim_v, size_t chunk_size, int dtype,
                     void* workspace, size_t workspace_bytes, unsigned flags,
                     const int64_t* token_strides, hipStream_t stream) {
    Problem p;
    bool empty;
    int rc = make_problem(q, k, v, beta, cu_seqlens, batch_size, seq_len, num_seqs, num_heads,
                          head_dim_k, head_dim_v, chunk_size, dtype, &p, &empty);
    if (rc != kSuccess) return rc;
    {
        const void* ptrs[6] = {q, k, v, grad_q, grad_k, grad_v};
        rc = apply_strides(&p, token_strides, 6, dtype, ptrs);
        if (rc != kSuccess) return rc;
    }
    if ((flags & ~(unsigned)(EFLA_BWD_REUSE_FORWARD | EFLA_BWD_REUSE_STATES)) != 0)
        return kInvalidValue;
    const bool reuse = (flags & EFLA_BWD_REUSE_FORWARD) != 0;
    const bool reuse_states = (flags & EFLA_BWD_REUSE_STATES) != 0;
    if ((reuse || reuse_states) && workspace == nullptr) return kInvalidValue;
    if (reuse_states && !reuse) return kInvalidValue;
    const size_t sbytes = (size_t)p.N * p.H * p.K * p.V * sizeof(float);
    if (empty) {
        if (grad_initial_state == nullptr) return kSuccess;
        if (grad_final_state)
            return (int)hipMemcpyAsync(grad_initial_state, grad_final_state, sbytes,
                                       hipMemcpyDeviceToDevice, stream);
        return fill_zero(grad_initial_state, sbytes, stream);
    }
    if (!grad_output || !grad_q || !grad_k || !grad_v || !grad_beta) return kInvalidValue;
    const size_t need = dtype == kDtypeBF16 ? carve_bwd<bf16>(p, nullptr, nullptr)
                                            : carve_bwd<float>(p, nullptr, nullptr);
    void* ws = workspace;
    WsLease lease;
    if (ws == nullptr) {
        rc = workspace_acquire(need, stream, &ws, lease);
        if (rc != kSuccess) return rc;
    } else if (workspace_bytes < need) {
        return kInvalidValue;
    }
    if (dtype == kDtypeBF16) {
        EFLA_Q_DISPATCH_BF16(run_bwd, p, (const bf16*)q, (const bf16*)k, (const bf16*)v,
                             (const bf16*)beta, initial_state, (const bf16*)grad_output,
                             grad_final_state, (bf16*)grad_q, (bf16*)grad_k, (bf16*)grad_v,
                             (bf16*)grad_beta, grad_initial_state, cu_seqlens, ws, reuse,
                             reuse_states, stream);
    } else {
        return run_bwd<float, 64, 64>(p, (const float*)q, (const float*)k, (const float*)v,
                                      (const float*)beta, initial_state,
                                      (const float*)grad_output, grad_final_state,
                                      (float*)grad_q, (float*)grad_k, (float*)grad_v,
                                      (float*)grad_beta, grad_initial_state, cu_seqlens, ws,
                                      reuse, reuse_states, stream);
    }
    return kInvalidValue;
}

extern "C" int efla_chunk_fwd_hip(const void* q, const void* k, const void* v, const void* beta,
                                  const float* initial_state, void* output, float* final_state,
                                  const int32_t* cu_seqlens, size_t batch_size, size_t seq_len,
                                  size_t num_seqs, size_t num_heads, size_t head_dim_k,
                                  size_t head_dim_v, size_t chunk_size, int dtype,
                                  void* workspace, size_t workspace_bytes, unsigned flags,
                                  hipStream_t stream) {
    return chunk_fwd(q, k, v, beta, initial_state, output, final_state, cu_seqlens, batch_size,
                     seq_len, num_seqs, num_heads, head_dim_k, head_dim_v, chunk_size, dtype,
                     workspace, workspace_bytes, flags, nullptr, stream);
}

// ---------------------------------------------------------------------------
// Forward without allocation: the per-chunk factors go to a fixed device array
// ---------------------------------------------------------------------------
// Each GPU the library runs on holds its own copy of `scratch` from the first
// call there until the process ends.  Host code never passes the array's name
// to a kernel (on the host it is only a stand-in for the symbol): the address
// of the current device's copy comes from hipGetSymbolAddress, taken once per
// device on the first call with that device current.
static __device__ __align__(256) unsigned char scratch[EFLA_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDev = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDev];  // per device: its copy of `scratch`
}  // namespace

static int scratch_address(void** out) {
    int dev = 0;
    EFLA_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxScratchDev) return kInvalidValue;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        EFLA_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (ptr == nullptr) return kInvalidValue;
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return kSuccess;
}

extern "C" int efla_chunk_fwd_noalloc_hip(const void* q, const void* k, const void* v,
                                          const void* beta, const float* initial_state,
                                          void* output, float* final_state,
                                          const int32_t* cu_seqlens, size_t batch_size,
                                          size_t seq_len, size_t num_seqs, size_t num_heads,
                                          size_t head_dim_k, size_t head_dim_v,
                                          size_t chunk_size, int dtype, hipStream_t stream) {
    Problem p;
    bool empty;
    int rc = make_problem(q, k, v, beta, cu_seqlens, batch_size, seq_len, num_seqs, num_heads,
                          head_dim_k, head_dim_v, chunk_size, dtype, &p, &empty);
    if (rc != kSuccess) return rc;
    if (!empty) {
        // the forward's factors (T, b and the coefficients, or W, U, h, Vn on
        // the fp32 path) must fit in the fixed array; nothing else is used
        const size_t need = dtype == kDtypeBF16 ? carve_fwd<bf16>(p, nullptr, nullptr, false)
                                                : carve_fwd<float>(p, nullptr, nullptr, false);
        if (need > EFLA_NOALLOC_SCRATCH_BYTES) return kOutOfMemory;
    }
    void* scr = nullptr;
    rc = scratch_address(&scr);
    if (rc != kSuccess) return rc;
    // every kernel writes what it reads back of the scratch before reading it,
    // so nothing has to be cleared between calls
    return chunk_fwd(q, k, v, beta, initial_state, output, final_state, cu_seqlens, batch_size,
                     seq_len, num_seqs, num_heads, head_dim_k, head_dim_v, chunk_size, dtype,
                     scr, EFLA_NOALLOC_SCRATCH_BYTES, 0u, nullptr, stream);
}

extern "C" int efla_chunk_fwd_strided_hip(
    const void* q, const void* k, const void* v, const void* beta, const float* initial_state,
    void* output, float* final_state, const int32_t* cu_seqlens, size_t batch_size,
    size_t seq_len, size_t num_seqs, size_t num_heads, size_t head_dim_k, size_t head_dim_v,
    size_t chunk_size, int dtype, void* workspace, size_t workspace_bytes, unsigned flags,
    const int64_t* token_strides, hipStream_t stream) {
    return chunk_fwd(q, k, v, beta, initial_state, output, final_state, cu_seqlens, batch_size,
                     seq_len, num_seqs, num_heads, head_dim_k, head_dim_v, chunk_size, dtype,
                     workspace, workspace_bytes, flags, token_strides, stream);
}

extern "C" int efla_chunk_bwd_hip(const void* q, const void* k, const void* v, const void* beta,
                                  const float* initial_state, const void* grad_output,
                                  const float* grad_final_state, void* grad_q, void* grad_k,
                                  void* grad_v, void* grad_beta, float* grad_initial_state,
                                  const int32_t* cu_seqlens, size_t batch_size, size_t seq_len,
                                  size_t num_seqs, size_t num_heads, size_t head_dim_k,
                                  size_t head_dim_v, size_t chunk_size, int dtype,
                                  void* workspace, size_t workspace_bytes, unsigned flags,
                                  hipStream_t stream) {
    return chunk_bwd(q, k, v, beta, initial_state, grad_output, grad_final_state, grad_q, grad_k,
                     grad_v, grad_beta, grad_initial_state, cu_seqlens, batch_size, seq_len,
                     num_seqs, num_heads, head_dim_k, head_dim_v, chunk_size, dtype, workspace,
                     workspace_bytes, flags, nullptr, stream);
}

extern "C" int efla_chunk_bwd_strided_hip(
    const void* q, const void* k, const void* v, const void* beta, const float* initial_state,
    const void* grad_output, const float* grad_final_state, void* grad_q, void* grad_k,
    void* grad_v, void* grad_beta, float* grad_initial_state, const int32_t* cu_seqlens,
    size_t batch_size, size_t seq_len, size_t num_seqs, size_t num_heads, size_t head_dim_k,
    size_t head_dim_v, size_t chunk_size, int dtype, void* workspace, size_t workspace_bytes,
    unsigned flags, const int64_t* token_strides, hipStream_t stream) {
    return chunk_bwd(q, k, v, beta, initial_state, grad_output, grad_final_state, grad_q, grad_k,
                     grad_v, grad_beta, grad_initial_state, cu_seqlens, batch_size, seq_len,
                     num_seqs, num_heads, head_dim_k, head_dim_v, chunk_size, dtype, workspace,
                     workspace_bytes, flags, token_strides, stream);
}
