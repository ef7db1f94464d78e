// bf16 chunked EFLA backward for gfx950 (included by efla_q.hip after
// efla_q_fast.hpp).
//
// Per chunk of C = 64 tokens with start state h (= S_n), end-state gradient
// dh (= dL/dS_{n+1}), b = c(beta, |k|^2), D = diag(b), G = K K^T,
// T = (I + strict_lower(D G))^{-1}, P = tril(Q K^T):
//   R  = V - K h,  Vn = T D R,  O = Q h + P Vn,  S_{n+1} = h + K^T Vn
// the chunk's gradients are
//   dVn = P^T dO + K dh,   Y = T^T dVn,   dv = D Y
//   Dm  = tril(dO Vn^T)
//   dq  = dO h^T + Dm K
//   dk  = Dm^T Q + Vn dh^T - D Y h^T + (dG + dG^T) K + 2 db c'(lambda) k
//   dT  = dVn (D R)^T,  dA = -strict_lower(T^T dT T^T),  dG = D dA
//   db  = rowsum(Y o R) + rowsum(dA o G),  dbeta = db exp(-beta lambda)
// and the state gradient runs backwards as dS_n = dS_{n+1} + Q^T dO - K^T D Y
// (= dS_{n+1} + Q^T dO - W^T dVn with W = T D K).  These restate the BPTT of
// kernels/cuda/efla.cu:315-454 chunk-wise (including its dc/dlambda term of
// efla.cu:384-451) for the query readout.
//
// scan_h_kernel   (forward recompute, grid: sequences x H x V/64)
//   S through the chunks as in scan_o_kernel; writes each chunk's start state
//   h_n to `hist` as bf16 [chunk][head][v][f].
// scan_dh_kernel  (reverse, same grid)
//   dS through the chunks backwards; writes each chunk's end-state gradient to
//   `dhist` in the same layout, and dS_0.
// grad_kernel     (grid: chunk slots x H)
//   everything above for one chunk from q, k, v, beta, dO, h, dh, looping over
//   64-wide value slices; writes dq, dk, dv, dbeta.
#pragma once
#include "efla_q_fast.hpp"

namespace efla {
namespace q {
namespace fast {

using mf::frag_row;
using mf::frag_tr;
using mf::tr_rows4;

constexpr int LD64 = ldb<64>();

__device__ __forceinline__ void store4(bf16* p, floatx4 a) {
    *reinterpret_cast<bf16x4*>(p) = bf16x4{(bf16)a[0], (bf16)a[1], (bf16)a[2], (bf16)a[3]};
}
__device__ __forceinline__ void store4s(bf16* p, floatx4 a, float s) {
    *reinterpret_cast<bf16x4*>(p) =
        bf16x4{(bf16)(a[0] * s), (bf16)(a[1] * s), (bf16)(a[2] * s), (bf16)(a[3] * s)};
}
__device__ __forceinline__ floatx4 load4(const bf16* p) {
    const bf16x4 x = *reinterpret_cast<const bf16x4*>(p);
    return floatx4{(float)x[0], (float)x[1], (float)x[2], (float)x[3]};
}
// keep the compiler from moving LDS accesses across this point and wait for
// this wave's outstanding LDS operations (a wave reads back what it wrote)
__device__ __forceinline__ void lds_fence_wave() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Write the C tiles of a K x 64 state slice (S[fb] rows pim(fb, 4g + i),
// column v0 + 16 w + r) to hist[v][f] (row stride K) as bf16, 8 bytes a lane.
template <int K>
__device__ __forceinline__ void store_state_vf(bf16* __restrict__ hist, const floatx4* S, int vcol) {
    const int g = mf::lane() >> 4;
#pragma unroll
    for (int fb = 0; fb < K / 16; ++fb) store4(hist + (long)vcol * K + pim(fb, 4 * g), S[fb]);
}

// ---------------------------------------------------------------------------
// forward recompute: chunk start states
// ---------------------------------------------------------------------------
template <int K>
struct ScanHSmem {
    bf16 W[64 * ldb<K>()];
    bf16 Kr[64 * ldb<K>()];
    bf16 U[64 * LD64];
};

template <int K, int V>
__global__ void __launch_bounds__(NT) scan_h_kernel(const bf16* __restrict__ k,
                                                    const bf16* __restrict__ W,
                                                    const bf16* __restrict__ U, SeqInfo si,
                                                    int H, const float* __restrict__ S0,
                                                    bf16* __restrict__ hist) {
    constexpr int LDK = ldb<K>(), NVS = V / VS;
    __shared__ __attribute__((aligned(16))) ScanHSmem<K> sm;
    const int w = mf::wave(), l = mf::lane(), g = l >> 4, r = l & 15;
    int bh, vsl;
    scan_map(blockIdx.x, si.N * H, NVS, bh, vsl);
    const int seq = bh / H, h = bh % H, v0 = vsl * VS;
    long sbos, slen;
    int slot0;
    seq_bounds(si, seq, sbos, slen, slot0);
    const int nch = (int)((slen + 63) / 64);
    const long sbase = (long)bh * K * V;
    const int vcol = v0 + 16 * w + r;
    floatx4 S[K / 16];
#pragma unroll
    for (int fb = 0; fb < K / 16; ++fb) S[fb] = zero4();
    if (S0) {
#pragma unroll
        for (int fb = 0; fb < K / 16; ++fb)
#pragma unroll
            for (int i = 0; i < 4; ++i) S[fb][i] = S0[sbase + (long)pim(fb, 4 * g + i) * V + vcol];
    }
    mf::TileRegs<64, K, NT> rw, rk;
    mf::TileRegs<64, VS, NT> ru;
    auto prefetch = [&](int n) {
        const long bos = sbos + (long)n * 64;
        const int len = (int)min((long)64, slen - (long)n * 64);
        rw.load(W + (bos * H + h) * K, (long)H * K, len);
        rk.load(k + (bos * H + h) * K, (long)H * K, len);
        ru.load(U + (bos * H + h) * V + v0, (long)H * V, len);
    };
    if (nch > 0) prefetch(0);
    for (int n = 0; n < nch; ++n) {
        __syncthreads();
        rw.store_rows(sm.W, LDK);
        rk.store_rows(sm.Kr, LDK);
        ru.store_rows(sm.U, LD64);
        __syncthreads();
        if (n + 1 < nch) prefetch(n + 1);
        store_state_vf<K>(hist + ((long)(slot0 + n) * H + h) * V * K, S, vcol);
        bf16x8 sb[K / 32];
#pragma unroll
        for (int kb = 0; kb < K / 32; ++kb) sb[kb] = mf::neg(frag_from_c(S[2 * kb], S[2 * kb + 1]));
        floatx4 vn[4];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            const bf16x4 u = tr_rows4(sm.U, LD64, 32 * (tb >> 1) + 4 * (tb & 1), 16 * w, 4);
            vn[tb] = floatx4{(float)u[0], (float)u[1], (float)u[2], (float)u[3]};
            const int row = pim(tb, r);
#pragma unroll
            for (int kb = 0; kb < K / 32; ++kb)
                vn[tb] = mma(frag_row(sm.W, LDK, row, 32 * kb), sb[kb], vn[tb]);
        }
        const bf16x8 vb0 = frag_from_c(vn[0], vn[1]), vb1 = frag_from_c(vn[2], vn[3]);
#pragma unroll
        for (int fb = 0; fb < K / 16; ++fb) {
            const int c0 = 32 * (fb >> 1) + 4 * (fb & 1);
            S[fb] = mma(frag_tr(sm.Kr, LDK, 0, c0, 8), vb0, S[fb]);
            S[fb] = mma(frag_tr(sm.Kr, LDK, 32, c0, 8), vb1, S[fb]);
        }
    }
}

// ---------------------------------------------------------------------------
// reverse scan: chunk end-state gradients
// ---------------------------------------------------------------------------
template <int K>
struct ScanDhSmem {
    bf16 Q[64 * ldb<K>()];
    bf16 Kr[64 * ldb<K>()];
    bf16 W[64 * ldb<K>()];
    bf16 dO[64 * LD64];  // dO[:, slice]
    bf16 P[64 * LD64];   // tril(Q K^T) [t][t']
};

template <int K, int V>
__global__ void __launch_bounds__(NT) scan_dh_kernel(const bf16* __restrict__ q,
                                                     const bf16* __restrict__ k,
                                                     const bf16* __restrict__ W,
                                                     const bf16* __restrict__ dO, SeqInfo si,
                                                     int H, const float* __restrict__ dST,
                                                     float* __restrict__ dS0,
                                                     bf16* __restrict__ dhist) {
    constexpr int LDK = ldb<K>(), NVS = V / VS;
    __shared__ __attribute__((aligned(16))) ScanDhSmem<K> sm;
    const int w = mf::wave(), l = mf::lane(), g = l >> 4, r = l & 15;
    int bh, vsl;
    scan_map(blockIdx.x, si.N * H, NVS, bh, vsl);
    const int seq = bh / H, h = bh % H, v0 = vsl * VS;
    long sbos, slen;
    int slot0;
    seq_bounds(si, seq, sbos, slen, slot0);
    const int nch = (int)((slen + 63) / 64);
    const long sbase = (long)bh * K * V;
    const int vcol = v0 + 16 * w + r;
    floatx4 dS[K / 16];
#pragma unroll
    for (int fb = 0; fb < K / 16; ++fb) dS[fb] = zero4();
    if (dST) {
#pragma unroll
        for (int fb = 0; fb < K / 16; ++fb)
#pragma unroll
            for (int i = 0; i < 4; ++i) dS[fb][i] = dST[sbase + (long)pim(fb, 4 * g + i) * V + vcol];
    }
    for (int i = threadIdx.x; i < 64 * LD64; i += NT) sm.P[i] = (bf16)0.f;
    mf::TileRegs<64, K, NT> rq, rk, rw;
    mf::TileRegs<64, VS, NT> rd;
    auto prefetch = [&](int n) {
        const long bos = sbos + (long)n * 64;
        const int len = (int)min((long)64, slen - (long)n * 64);
        rq.load(q + (bos * H + h) * K, (long)H * K, len);
        rk.load(k + (bos * H + h) * K, (long)H * K, len);
        rw.load(W + (bos * H + h) * K, (long)H * K, len);
        rd.load(dO + (bos * H + h) * V + v0, (long)H * V, len);
    };
    if (nch > 0) prefetch(nch - 1);
    for (int n = nch - 1; n >= 0; --n) {
        __syncthreads();
        rq.store_rows(sm.Q, LDK);
        rk.store_rows(sm.Kr, LDK);
        rw.store_rows(sm.W, LDK);
        rd.store_rows(sm.dO, LD64);
        __syncthreads();
        if (n > 0) prefetch(n - 1);
        store_state_vf<K>(dhist + ((long)(slot0 + n) * H + h) * V * K, dS, vcol);
        for (int nt = w; nt < 10; nt += 4) {
            int I, J;
            lower_tile(nt, I, J);
            floatx4 acc = zero4();
#pragma unroll
            for (int k0 = 0; k0 < K; k0 += 32)
                acc = mma(frag_nat(sm.Kr, LDK, 16 * J, k0), frag_nat(sm.Q, LDK, 16 * I, k0), acc);
            const int tq = 16 * I + r, tk = 16 * J + 4 * g;
            *reinterpret_cast<bf16x4*>(sm.P + tq * LD64 + tk) =
                bf16x4{(bf16)(tk + 0 <= tq ? acc[0] : 0.f), (bf16)(tk + 1 <= tq ? acc[1] : 0.f),
                       (bf16)(tk + 2 <= tq ? acc[2] : 0.f), (bf16)(tk + 3 <= tq ? acc[3] : 0.f)};
        }
        bf16x8 sb[K / 32];
#pragma unroll
        for (int kb = 0; kb < K / 32; ++kb) sb[kb] = frag_from_c(dS[2 * kb], dS[2 * kb + 1]);
        const bf16x8 do0 = frag_tr(sm.dO, LD64, 0, 16 * w), do1 = frag_tr(sm.dO, LD64, 32, 16 * w);
        __syncthreads();
        // dVn = P^T dO + K dS; tile tb row 4g + i is token pim(tb, 4g + i)
        floatx4 dvn[4];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            const int row = pim(tb, r), c0 = 32 * (tb >> 1) + 4 * (tb & 1);
            floatx4 acc = zero4();
            if (tb < 2) acc = mma(frag_tr(sm.P, LD64, 0, c0, 8), do0, acc);
            acc = mma(frag_tr(sm.P, LD64, 32, c0, 8), do1, acc);
#pragma unroll
            for (int kb = 0; kb < K / 32; ++kb) acc = mma(frag_row(sm.Kr, LDK, row, 32 * kb), sb[kb], acc);
            dvn[tb] = acc;
        }
        const bf16x8 nd0 = mf::neg(frag_from_c(dvn[0], dvn[1]));
        const bf16x8 nd1 = mf::neg(frag_from_c(dvn[2], dvn[3]));
        // dS <- dS + Q^T dO - W^T dVn
#pragma unroll
        for (int fb = 0; fb < K / 16; ++fb) {
            const int c0 = 32 * (fb >> 1) + 4 * (fb & 1);
            floatx4 acc = dS[fb];
            acc = mma(frag_tr(sm.Q, LDK, 0, c0, 8), do0, acc);
            acc = mma(frag_tr(sm.Q, LDK, 32, c0, 8), do1, acc);
            acc = mma(frag_tr(sm.W, LDK, 0, c0, 8), nd0, acc);
            acc = mma(frag_tr(sm.W, LDK, 32, c0, 8), nd1, acc);
            dS[fb] = acc;
        }
    }
    if (dS0) {
#pragma unroll
        for (int fb = 0; fb < K / 16; ++fb)
#pragma unroll
            for (int i = 0; i < 4; ++i) dS0[sbase + (long)pim(fb, 4 * g + i) * V + vcol] = dS[fb][i];
    }
}

// ---------------------------------------------------------------------------
// per-chunk gradients
// ---------------------------------------------------------------------------
template <int K>
struct GradSmem {
    bf16 Qs[64 * ldb<K>()];
    bf16 Ks[64 * ldb<K>()];
    bf16 Ps[64 * LD64];  // P[t][t'] (t' <= t)
    bf16 Tb[64 * LD64];  // bf16(T)[t][t'] (t' <= t), from the WY prep
    float lam[64], b[64], dcl[64], dcb[64];
    union {
        struct {  // one 64-wide value slice
            bf16 V[64 * LD64];   // v[:, slice]; each wave's rows later hold D Y
            bf16 dO[64 * LD64];  // dO[:, slice]
            bf16 h[64 * ldb<K>()];   // h[v][f] for the slice's v
            bf16 dh[64 * ldb<K>()];  // dh[v][f]
            bf16 DR[64 * LD64];  // D R [t][v]
            bf16 Vn[64 * LD64];  // Vn [t][v]
            bf16 dVn[64 * LD64]; // dVn [t][v]
        } s;
        struct {  // closing products
            bf16 Dm[64 * LD64];  // Dm [t][t']
            bf16 X[64 * LD64];   // dT T^T [t][t'']
            bf16 dG[64 * LD64];  // dG [i][j]
        } e;
    } u;
};

template <int K, int V>
__global__ void __launch_bounds__(NT) grad_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const bf16* __restrict__ beta, const bf16* __restrict__ dO, const bf16* __restrict__ Tws,
    const bf16* __restrict__ hist, const bf16* __restrict__ dhist, SeqInfo si, int H,
    bf16* __restrict__ dq, bf16* __restrict__ dk, bf16* __restrict__ dv,
    bf16* __restrict__ dbeta) {
    constexpr int LDK = ldb<K>(), NS = V / VS;
    __shared__ __attribute__((aligned(16))) GradSmem<K> sm;
    const int slot = blockIdx.x, h = blockIdx.y;
    long bos;
    int len;
    if (!locate_chunk(si, slot, bos, len)) return;
    const int w = mf::wave(), l = mf::lane(), g = l >> 4, r = l & 15;
    const int t = 16 * w + r;  // this lane's token (column of the transposed tiles)
    const long chb = ((long)slot * H + h) * V * K;  // this chunk's h / dh block

    mf::TileRegs<64, VS, NT> rv, rd;
    mf::TileRegs<64, K, NT> rh, rdh;
    auto prefetch = [&](int s) {
        const int vv = s * VS;
        rv.load(v + (bos * H + h) * V + vv, (long)H * V, len);
        rd.load(dO + (bos * H + h) * V + vv, (long)H * V, len);
        rh.load(hist + chb + (long)vv * K, K, 64);
        rdh.load(dhist + chb + (long)vv * K, K, 64);
    };
    // ---- chunk setup: q, k, T, b, P ----
    {
        mf::TileRegs<64, K, NT> rq, rk;
        mf::TileRegs<64, 64, NT> rt;
        rq.load(q + (bos * H + h) * K, (long)H * K, len);
        rk.load(k + (bos * H + h) * K, (long)H * K, len);
        rt.load(Tws + ((long)slot * H + h) * 64 * 64, 64, 64);
        prefetch(0);
        rq.store_rows(sm.Qs, LDK);
        rk.store_rows(sm.Ks, LDK);
        rt.store_rows(sm.Tb, LD64);
#pragma unroll
        for (int j = 0; j < rk.TPT; ++j) {
            const float s = rk.row_sumsq(j);
            if (rk.fg() == 0) sm.lam[rk.t0() + j] = s;
        }
        for (int i = threadIdx.x; i < 64 * LD64; i += NT) sm.Ps[i] = (bf16)0.f;
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const int tt = threadIdx.x;
        float c = 0.f, dcl = 0.f, dcb = 0.f;
        if (tt < len) efla_coeff(sm.lam[tt], (float)beta[(bos + tt) * H + h], c, dcl, dcb);
        sm.b[tt] = c;
        sm.dcl[tt] = dcl;
        sm.dcb[tt] = dcb;
    }
    for (int n = w; n < 10; n += 4) {
        int I, J;
        lower_tile(n, I, J);
        floatx4 accp = zero4();
#pragma unroll
        for (int k0 = 0; k0 < K; k0 += 32)
            accp = mma(frag_nat(sm.Ks, LDK, 16 * J, k0), frag_nat(sm.Qs, LDK, 16 * I, k0), accp);
        const int tq = 16 * I + r, tk = 16 * J + 4 * g;
        *reinterpret_cast<bf16x4*>(sm.Ps + tq * LD64 + tk) =
            bf16x4{(bf16)(tk + 0 <= tq ? accp[0] : 0.f), (bf16)(tk + 1 <= tq ? accp[1] : 0.f),
                   (bf16)(tk + 2 <= tq ? accp[2] : 0.f), (bf16)(tk + 3 <= tq ? accp[3] : 0.f)};
    }
    // B operand (line t, k = t') of T
    const bf16x8 tfr[2] = {frag_nat(sm.Tb, LD64, 16 * w, 0), frag_nat(sm.Tb, LD64, 16 * w, 32)};
    __syncthreads();
    const float bt = sm.b[t];
    const int nks = w >= 2 ? 1 : 0;  // first k-step (of 32) that reaches t'' >= t

    // ---- value slices ----
    floatx4 dqa[K / 16], dka[K / 16], dma[4], dta[4];
#pragma unroll
    for (int fb = 0; fb < K / 16; ++fb) dqa[fb] = dka[fb] = zero4();
#pragma unroll
    for (int j = 0; j < 4; ++j) dma[j] = dta[j] = zero4();
    float dbp = 0.f;
    for (int s = 0; s < NS; ++s) {
        const int vv = s * VS;
        if (s > 0) __syncthreads();
        rv.store_rows(sm.u.s.V, LD64);
        rd.store_rows(sm.u.s.dO, LD64);
        rh.store_rows(sm.u.s.h, LDK);
        rdh.store_rows(sm.u.s.dh, LDK);
        __syncthreads();
        if (s + 1 < NS) prefetch(s + 1);
        // R^T = V^T - h K^T and dVn^T = dO^T P + dh K^T, tile vb: (value 16vb + 4g + i, token t)
        floatx4 rT[4];
#pragma unroll
        for (int vb = 0; vb < 4; ++vb) {
            floatx4 ra = load4(sm.u.s.V + t * LD64 + 16 * vb + 4 * g);
            floatx4 da = zero4();
#pragma unroll
            for (int kb = 0; kb < K / 32; ++kb) {
                const bf16x8 kt = frag_nat(sm.Ks, LDK, 16 * w, 32 * kb);
                ra = mma(frag_nat(sm.u.s.h, LDK, 16 * vb, 32 * kb), mf::neg(kt), ra);
                da = mma(frag_nat(sm.u.s.dh, LDK, 16 * vb, 32 * kb), kt, da);
            }
            if (nks == 0) da = mma(frag_tr(sm.u.s.dO, LD64, 0, 16 * vb), frag_tr(sm.Ps, LD64, 0, 16 * w), da);
            da = mma(frag_tr(sm.u.s.dO, LD64, 32, 16 * vb), frag_tr(sm.Ps, LD64, 32, 16 * w), da);
            rT[vb] = ra;
            store4s(sm.u.s.DR + t * LD64 + 16 * vb + 4 * g, ra, bt);
            store4(sm.u.s.dVn + t * LD64 + 16 * vb + 4 * g, da);
        }
        __syncthreads();
        // Vn^T = (D R)^T T^T; Y^T = dVn^T T; dv = D Y; db += sum_v Y R; D Y -> own rows of V
        bf16* vrow = dv + ((bos + t) * H + h) * V + vv + 4 * g;
#pragma unroll
        for (int vb = 0; vb < 4; ++vb) {
            floatx4 vn = mma(frag_tr(sm.u.s.DR, LD64, 0, 16 * vb), tfr[0], zero4());
            if (w >= 2) vn = mma(frag_tr(sm.u.s.DR, LD64, 32, 16 * vb), tfr[1], vn);
            store4(sm.u.s.Vn + t * LD64 + 16 * vb + 4 * g, vn);
            floatx4 y = zero4();
            if (nks == 0)
                y = mma(frag_tr(sm.u.s.dVn, LD64, 0, 16 * vb), frag_tr(sm.Tb, LD64, 0, 16 * w), y);
            y = mma(frag_tr(sm.u.s.dVn, LD64, 32, 16 * vb), frag_tr(sm.Tb, LD64, 32, 16 * w), y);
#pragma unroll
            for (int i = 0; i < 4; ++i) dbp += y[i] * rT[vb][i];
            if (t < len) store4s(vrow + 16 * vb, y, bt);
            store4s(sm.u.s.V + t * LD64 + 16 * vb + 4 * g, y, bt);
        }
        lds_fence_wave();
        // dq^T += h^T dO^T;  dk^T -= h^T (D Y)^T;  dT^T[t'][t] += sum_v D R[t'] dVn[t]
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const bf16x8 dob = frag_nat(sm.u.s.dO, LD64, 16 * w, 32 * ks);
            const bf16x8 dyb = mf::neg(frag_nat(sm.u.s.V, LD64, 16 * w, 32 * ks));
            const bf16x8 dvb = frag_nat(sm.u.s.dVn, LD64, 16 * w, 32 * ks);
#pragma unroll
            for (int fb = 0; fb < K / 16; ++fb) {
                const bf16x8 ha = frag_tr(sm.u.s.h, LDK, 32 * ks, 16 * fb);
                dqa[fb] = mma(ha, dob, dqa[fb]);
                dka[fb] = mma(ha, dyb, dka[fb]);
            }
#pragma unroll
            for (int J = 0; J < 4; ++J)
                if (J < 2 || w >= 2)
                    dta[J] = mma(frag_row(sm.u.s.DR, LD64, pim(J, r), 32 * ks), dvb, dta[J]);
        }
        __syncthreads();
        // Dm^T[t'][t] += sum_v Vn[t'] dO[t];  dk^T += dh^T Vn^T
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const bf16x8 dob = frag_nat(sm.u.s.dO, LD64, 16 * w, 32 * ks);
            const bf16x8 vnb = frag_nat(sm.u.s.Vn, LD64, 16 * w, 32 * ks);
#pragma unroll
            for (int J = 0; J < 4; ++J)
                if (J < 2 || w >= 2)
                    dma[J] = mma(frag_row(sm.u.s.Vn, LD64, pim(J, r), 32 * ks), dob, dma[J]);
#pragma unroll
            for (int fb = 0; fb < K / 16; ++fb)
                dka[fb] = mma(frag_tr(sm.u.s.dh, LDK, 32 * ks, 16 * fb), vnb, dka[fb]);
        }
    }
    // db from Y o R: sum over the 4 lane groups holding token t
    dbp += __shfl_xor(dbp, 16);
    dbp += __shfl_xor(dbp, 32);
    __syncthreads();  // slice buffers are free

    // ---- closing products ----
    // masks: Dm[t][t'] needs t' <= t, dT[t][t'] needs t' < t
#pragma unroll
    for (int J = 0; J < 4; ++J)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tp = pim(J, 4 * g + i);
            if (tp > t) dma[J][i] = 0.f;
            if (tp >= t) dta[J][i] = 0.f;
        }
    // dq^T += K^T Dm^T (k = t'), Dm from registers
    {
        const bf16x8 m0 = frag_from_c(dma[0], dma[1]), m1 = frag_from_c(dma[2], dma[3]);
#pragma unroll
        for (int fb = 0; fb < K / 16; ++fb) {
            dqa[fb] = mma(frag_tr(sm.Ks, LDK, 0, 16 * fb), m0, dqa[fb]);
            if (w >= 2) dqa[fb] = mma(frag_tr(sm.Ks, LDK, 32, 16 * fb), m1, dqa[fb]);
        }
    }
    // share Dm [t][t'] and X^T: X[t][t''] = sum_t' dT[t][t'] T[t''][t']
#pragma unroll
    for (int J = 0; J < 4; ++J) store4(sm.u.e.Dm + t * LD64 + pim(J, 4 * g), dma[J]);
    {
        const bf16x8 d0 = frag_from_c(dta[0], dta[1]), d1 = frag_from_c(dta[2], dta[3]);
#pragma unroll
        for (int J = 0; J < 4; ++J) {
            floatx4 x = mma(frag_nat(sm.Tb, LD64, 16 * J, 0), d0, zero4());
            x = mma(frag_nat(sm.Tb, LD64, 16 * J, 32), d1, x);
            store4(sm.u.e.X + t * LD64 + 16 * J + 4 * g, x);
        }
    }
    __syncthreads();
    // dk^T += Q^T Dm (token t' = t owned here, k = t >= t')
#pragma unroll
    for (int fb = 0; fb < K / 16; ++fb) {
        if (nks == 0)
            dka[fb] = mma(frag_tr(sm.Qs, LDK, 0, 16 * fb), frag_tr(sm.u.e.Dm, LD64, 0, 16 * w), dka[fb]);
        dka[fb] = mma(frag_tr(sm.Qs, LDK, 32, 16 * fb), frag_tr(sm.u.e.Dm, LD64, 32, 16 * w), dka[fb]);
    }
    // M^T[j][i] = sum_t X[t][j] T[t][i] for i = t owned here, rows j = pim(J, .) < i;
    // dA = -M (strict lower), G recomputed; db += sum_j dA G; dG = b_i dA
    float dbg = 0.f;
    floatx4 dgt[4];
#pragma unroll
    for (int J = 0; J < 4; ++J) {
        dgt[J] = zero4();
        if (J < 2 || w >= 2) {
            const int c0 = 32 * (J >> 1) + 4 * (J & 1);
            floatx4 m = zero4();
            if (nks == 0) m = mma(frag_tr(sm.u.e.X, LD64, 0, c0, 8), frag_tr(sm.Tb, LD64, 0, 16 * w), m);
            m = mma(frag_tr(sm.u.e.X, LD64, 32, c0, 8), frag_tr(sm.Tb, LD64, 32, 16 * w), m);
            floatx4 gg = zero4();
#pragma unroll
            for (int k0 = 0; k0 < K; k0 += 32)
                gg = mma(frag_row(sm.Ks, LDK, pim(J, r), k0), frag_nat(sm.Ks, LDK, 16 * w, k0), gg);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = pim(J, 4 * g + i);
                const float da = (j < t) ? -m[i] : 0.f;
                dbg += da * gg[i];
                dgt[J][i] = bt * da;
            }
        }
    }
    dbg += __shfl_xor(dbg, 16);
    dbg += __shfl_xor(dbg, 32);
    const float dbt = dbp + dbg;  // dL/db for token t (all lanes of the column)
    // dk^T += K^T dG^T (k = j < i = t), from registers; share dG [i][j]
    {
        const bf16x8 g0 = frag_from_c(dgt[0], dgt[1]), g1 = frag_from_c(dgt[2], dgt[3]);
#pragma unroll
        for (int fb = 0; fb < K / 16; ++fb) {
            dka[fb] = mma(frag_tr(sm.Ks, LDK, 0, 16 * fb), g0, dka[fb]);
            if (w >= 2) dka[fb] = mma(frag_tr(sm.Ks, LDK, 32, 16 * fb), g1, dka[fb]);
        }
    }
#pragma unroll
    for (int J = 0; J < 4; ++J) store4(sm.u.e.dG + t * LD64 + pim(J, 4 * g), dgt[J]);
    __syncthreads();
    // dk^T += K^T dG (token j = t owned here, k = i > j)
#pragma unroll
    for (int fb = 0; fb < K / 16; ++fb) {
        if (nks == 0)
            dka[fb] = mma(frag_tr(sm.Ks, LDK, 0, 16 * fb), frag_tr(sm.u.e.dG, LD64, 0, 16 * w), dka[fb]);
        dka[fb] = mma(frag_tr(sm.Ks, LDK, 32, 16 * fb), frag_tr(sm.u.e.dG, LD64, 32, 16 * w), dka[fb]);
    }
    // dk += 2 db c'(lambda) k; write dq, dk, dbeta
    if (t < len) {
        const float s2 = 2.f * dbt * sm.dcl[t];
        bf16* qrow = dq + ((bos + t) * H + h) * K + 4 * g;
        bf16* krow = dk + ((bos + t) * H + h) * K + 4 * g;
#pragma unroll
        for (int fb = 0; fb < K / 16; ++fb) {
            store4(qrow + 16 * fb, dqa[fb]);
            const floatx4 kk = load4(sm.Ks + t * LDK + 16 * fb + 4 * g);
            floatx4 a = dka[fb];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] += s2 * kk[i];
            store4(krow + 16 * fb, a);
        }
        if (g == 0) dbeta[(bos + t) * H + h] = (bf16)(dbt * sm.dcb[t]);
    }
}

}  // namespace fast
}  // namespace q
}  // namespace efla
