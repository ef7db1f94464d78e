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
// efla.cu:384-451) for the query readout.  Since
// T^T dT T^T = (T^T dVn)(T D R)^T = Y Vn^T, the gradient kernel forms
//   dA = -strict_lower(Y Vn^T)
// as a sum over the value slices, like Dm, and never forms dT.
//
// scan_h_kernel   (forward recompute, grid: sequences x H x V/64)
//   S through the chunks as in scan_o_kernel; writes each chunk's start state
//   h_n to `hist` as bf16 [chunk][head][v][f].
// scan_dh_kernel  (reverse, same grid)
//   dS through the chunks backwards (dVn = P^T dO + K dS, Z = D T^T dVn,
//   dS <- dS + Q^T dO - K^T Z); writes each chunk's end-state gradient to
//   `dhist` in the same layout, and dS_0.
// grad_kernel     (persistent, one workgroup per CU over the chunk x H items)
//   everything above for one chunk from q, k, v, beta, dO, h, dh, looping over
//   64-wide value slices; writes dq, dk, dv, dbeta.
#pragma once
#include "efla_q_fast.hpp"

namespace efla {
namespace q {
namespace fast {

using mf::frag_row;
using mf::frag_tr;
using mf::frag_trc;
using mf::tr_rows4;

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

// ---------------------------------------------------------------------------
// forward recompute: chunk start states
// ---------------------------------------------------------------------------
template <int K>
struct ScanHBuf {
    bf16 Kr[64 * ldb<K>()];
    bf16 Vs[64 * LD64];  // v[:, slice]
    bf16 T[64 * LD64];
    float b[64];
};

template <int K>
struct ScanHSmem {
    ScanHBuf<K> buf[2];  // chunk n in buf[n & 1]
};

template <int K, int V>
__global__ void __launch_bounds__(NT) scan_h_kernel(const bf16* __restrict__ k,
                                                    const bf16* __restrict__ v,
                                                    const bf16* __restrict__ Tc,
                                                    const float* __restrict__ bc, SeqInfo si,
                                                    int H, const float* __restrict__ S0,
                                                    bf16* __restrict__ hist, TokLd ld) {
    constexpr int LDK = ldb<K>(), NVS = V / VS;
    __shared__ __attribute__((aligned(16))) ScanHSmem<K> sm;
    const int w = mf::wave(), l = mf::lane(), g = l >> 4, r = l & 15;
    int bh, vsl;
    scan_map(blockIdx.x, si.N * H, NVS, bh, vsl);
    bh = scan_seq_head(si, bh, H);
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
        mf::dma_wait();  // retired here, not by a vmcnt(0) inside the chunk loop
    }
    ChunkRegs<K, false, true> pre;
    auto prefetch = [&](int n) {
        const long bos = sbos + (long)n * 64;
        const int len = (int)min((long)64, slen - (long)n * 64);
        pre.load(nullptr, k, v, Tc, bc, bos, len, h, V, v0, (long)(slot0 + n) * H + h, 0, ld.k,
                 ld.v);
    };
    if (nch > 0) {
        prefetch(0);
        pre.stage(sm.buf[0]);
        if (nch > 1) prefetch(1);
    }
    for (int n = 0; n < nch; ++n) {
        const ScanHBuf<K>& cb = sm.buf[n & 1];
        __syncthreads();  // chunk n staged; everyone is done with chunk n - 1
        bf16x8 sb[K / 32];
#pragma unroll
        for (int kb = 0; kb < K / 32; ++kb) sb[kb] = frag_from_c(S[2 * kb], S[2 * kb + 1]);
        store_state_frag<K>(hist + ((long)(slot0 + n) * H + h) * V * K, sb, vcol);
        floatx4 vn[4];
        chunk_vn<K>(cb, w, sb, vn);
        const bf16x8 vb0 = frag_from_c(vn[0], vn[1]), vb1 = frag_from_c(vn[2], vn[3]);
#pragma unroll
        for (int fb = 0; fb < K / 16; ++fb) {
            const int c0 = 32 * (fb >> 1) + 4 * (fb & 1);
            S[fb] = mma(frag_tr(cb.Kr, LDK, 0, c0, 8), vb0, S[fb]);
            S[fb] = mma(frag_tr(cb.Kr, LDK, 32, c0, 8), vb1, S[fb]);
        }
        if (n + 1 < nch) {
            pre.stage(sm.buf[(n + 1) & 1]);
            if (n + 2 < nch) prefetch(n + 2);
        }
    }
}

// ---------------------------------------------------------------------------
// reverse scan: chunk end-state gradients
// ---------------------------------------------------------------------------
// PS: the forward saved each chunk's P = tril(Q K^T); it is staged with the
// other chunk inputs instead of being recomputed.
template <int K, bool PS>
struct ScanDhBuf {
    bf16 Q[64 * ldb<K>()];
    bf16 Kr[64 * ldb<K>()];
    bf16 Vs[64 * LD64];  // dO[:, slice]
    bf16 T[64 * LD64];
    bf16 P[PS ? 64 * LD64 : 8];  // the forward's P [t][t'] (PS)
    float b[64];
};

template <int K, bool PS>
struct ScanDhSmem {
    ScanDhBuf<K, PS> buf[2];  // chunk n in buf[n & 1]
    // P [t][t'] computed here (not PS): with copy waves chunk n's in P + (n & 1) *
    // 64 * LD64, formed by the copy waves during chunk n + 1
    bf16 P[PS ? 8 : (K > 64 ? 2 : 1) * 64 * LD64];
};

// P = tril(Q K^T) of a staged chunk into P [t][t'] (row stride LD64): lower
// 16x16 tiles nt0, nt0 + 4, ... of 10 (I = t block, J = t' block), computed
// transposed so each lane writes 4 consecutive t'; upper tiles untouched.
template <int K, typename Buf>
__device__ __forceinline__ void chunk_p_tiles(const Buf& cb, bf16* P, int nt0) {
    constexpr int LDK = ldb<K>();
    const int l = mf::lane(), g = l >> 4, r = l & 15;
    for (int nt = nt0; nt < 10; nt += 4) {
        int I, J;
        lower_tile(nt, I, J);
        floatx4 acc = zero4();
#pragma unroll
        for (int k0 = 0; k0 < K; k0 += 32)
            acc = mma(frag_nat(cb.Kr, LDK, 16 * J, k0), frag_nat(cb.Q, LDK, 16 * I, k0), acc);
        const int tq = 16 * I + r, tk = 16 * J + 4 * g;
        *reinterpret_cast<bf16x4*>(P + tq * LD64 + tk) =
            bf16x4{(bf16)(tk + 0 <= tq ? acc[0] : 0.f), (bf16)(tk + 1 <= tq ? acc[1] : 0.f),
                   (bf16)(tk + 2 <= tq ? acc[2] : 0.f), (bf16)(tk + 3 <= tq ? acc[3] : 0.f)};
    }
}

// d_k = 128: waves 0..3 compute, waves 4..7 write chunk n - 1 into LDS during
// chunk n (as in scan_o_kernel, one register set: more loads in flight
// measured slower here).  d_k = 64: four waves that also stage the next
// chunk themselves (copy waves measured 1.14x slower at that size).
template <int K>
constexpr bool dh_copy_waves() {
    return K > 64;
}
template <int K>
constexpr int dh_threads() {
    return dh_copy_waves<K>() ? NTS : NT;
}
template <int K, int V, bool PS>
__global__ void __launch_bounds__(dh_threads<K>()) scan_dh_kernel(const bf16* __restrict__ q,
                                                      const bf16* __restrict__ k,
                                                      const bf16* __restrict__ dO,
                                                      const bf16* __restrict__ Tc,
                                                      const float* __restrict__ bc,
                                                      const bf16* __restrict__ Pc, SeqInfo si,
                                                      int H, const float* __restrict__ dST,
                                                      float* __restrict__ dS0,
                                                      bf16* __restrict__ dhist, TokLd ld) {
    constexpr int LDK = ldb<K>(), NVS = V / VS;
    __shared__ __attribute__((aligned(16))) ScanDhSmem<K, PS> sm;
    const int w = mf::wave(), l = mf::lane(), g = l >> 4, r = l & 15;
    int bh, vsl;
    scan_map(blockIdx.x, si.N * H, NVS, bh, vsl);
    bh = scan_seq_head(si, bh, H);
    const int seq = bh / H, h = bh % H, v0 = vsl * VS;
    long sbos, slen;
    int slot0;
    seq_bounds(si, seq, sbos, slen, slot0);
    const int nch = (int)((slen + 63) / 64);
    constexpr bool CW = dh_copy_waves<K>();
    if (CW && w >= NCW) {  // copy waves: chunk n - 1 into buf[(n - 1) & 1] during chunk n
        const int ct = (int)threadIdx.x - NT;
        struct Regs {
            ChunkRegs<K, true, true> c;
            mf::TileRegs<64, 64, NT> p;  // PS: the chunk's P
        };
        // chunk n's loads (clamped to chunk 0, so every iteration issues the
        // same loads and the staging's waits stay exact)
        auto load = [&](Regs& R, int n) {
            n = max(n, 0);
            const long bos = sbos + (long)n * 64;
            const int len = (int)min((long)64, slen - (long)n * 64);
            const long cid = (long)(slot0 + n) * H + h;
            R.c.load(q, k, dO, Tc, bc, bos, len, h, V, v0, cid, ld.q, ld.k, (long)H * V, ct);
            if constexpr (PS) load_tri(R.p, Pc + cid * TRI_ELEMS, ct);
        };
        auto stage = [&](Regs& R, ScanDhBuf<K, PS>& bf) {
            R.c.stage(bf);
            if constexpr (PS) R.p.store_rows(bf.P, LD64);
        };
        // not PS: the copy waves also form each chunk's P once it is staged
        auto ptiles = [&](int m) {
            chunk_p_tiles<K>(sm.buf[m & 1], sm.P + (m & 1) * 64 * LD64, w - NCW);
        };
        Regs ra;
        if (nch > 0) {
            load(ra, nch - 1);
            stage(ra, sm.buf[(nch - 1) & 1]);
            load(ra, nch - 2);
            if constexpr (!PS) {
                __syncthreads();  // chunk nch - 1 staged
                ptiles(nch - 1);
            }
        }
        for (int n = nch - 1; n >= 0; --n) {
            __syncthreads();  // chunk n staged; everyone is done with chunk n + 1
            if (n > 0) stage(ra, sm.buf[(n - 1) & 1]);
            load(ra, n - 2);
            if constexpr (!PS) {
                __syncthreads();  // chunk n - 1 staged
                if (n > 0) ptiles(n - 1);
            }
        }
        return;
    }
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
        mf::dma_wait();  // retired here, not by a vmcnt(0) inside the chunk loop
    }
    if constexpr (!PS) {
        for (int i = threadIdx.x; i < (CW ? 2 : 1) * 64 * LD64; i += NT) sm.P[i] = (bf16)0.f;
        if (CW && nch > 0) __syncthreads();  // zeros in place before the copy waves' P tiles
    }
    // without copy waves: chunk n - 1 staged from registers during chunk n,
    // chunk n - 2's loads issued right after
    ChunkRegs<K, true, true> pre;
    mf::TileRegs<64, 64, NT> rp;  // PS: the chunk's P
    auto prefetch = [&](int n) {
        const long bos = sbos + (long)n * 64;
        const int len = (int)min((long)64, slen - (long)n * 64);
        const long cid = (long)(slot0 + n) * H + h;
        pre.load(q, k, dO, Tc, bc, bos, len, h, V, v0, cid, ld.q, ld.k, (long)H * V);
        if constexpr (PS) load_tri(rp, Pc + cid * TRI_ELEMS);
    };
    auto stage = [&](ScanDhBuf<K, PS>& bf) {
        pre.stage(bf);
        if constexpr (PS) rp.store_rows(bf.P, LD64);
    };
    if (!CW && nch > 0) {
        prefetch(nch - 1);
        stage(sm.buf[(nch - 1) & 1]);
        if (nch > 1) prefetch(nch - 2);
    }
    for (int n = nch - 1; n >= 0; --n) {
        const ScanDhBuf<K, PS>& cb = sm.buf[n & 1];
        const bf16* Pm = PS ? cb.P : sm.P + (CW ? (n & 1) * 64 * LD64 : 0);
        __syncthreads();  // chunk n staged; everyone is done with chunk n + 1
        if (!PS && !CW) chunk_p_tiles<K>(cb, sm.P, w);
        bf16x8 sb[K / 32];
#pragma unroll
        for (int kb = 0; kb < K / 32; ++kb) sb[kb] = frag_from_c(dS[2 * kb], dS[2 * kb + 1]);
        store_state_frag<K>(dhist + ((long)(slot0 + n) * H + h) * V * K, sb, vcol);
        // dO^T in c-order over the tokens; its partners (P, Q) are read the same way
        const bf16x8 do0 = mf::frag_trc(cb.Vs, LD64, 0, 16 * w), do1 = mf::frag_trc(cb.Vs, LD64, 32, 16 * w);
        // K dS part of dVn (P^T dO is added once P is complete); tile tb row
        // 4g + i is token pim(tb, 4g + i)
        floatx4 dvn[4];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            const int row = pim(tb, r);
            floatx4 acc = zero4();
#pragma unroll
            for (int kb = 0; kb < K / 32; ++kb) acc = mma(frag_row(cb.Kr, LDK, row, 32 * kb), sb[kb], acc);
            dvn[tb] = acc;
        }
        if (!CW && n > 0) {
            stage(sm.buf[(n - 1) & 1]);
            if (n > 1) prefetch(n - 2);
        }
        // not PS: P complete (without copy waves); chunk n - 1 staged for the
        // copy waves' P tiles (with them)
        if constexpr (!PS) __syncthreads();
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            const int c0 = 32 * (tb >> 1) + 4 * (tb & 1);
            if (tb < 2) dvn[tb] = mma(mf::frag_trc(Pm, LD64, 0, c0, 8), do0, dvn[tb]);
            dvn[tb] = mma(mf::frag_trc(Pm, LD64, 32, c0, 8), do1, dvn[tb]);
        }
        // Z = D T^T dVn (k = t'' >= t)
        const bf16x8 dv0 = frag_from_c(dvn[0], dvn[1]), dv1 = frag_from_c(dvn[2], dvn[3]);
        floatx4 z[4];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            const int c0 = 32 * (tb >> 1) + 4 * (tb & 1);
            floatx4 acc = zero4();
            if (tb < 2) acc = mma(frag_tr(cb.T, LD64, 0, c0, 8), dv0, acc);
            acc = mma(frag_tr(cb.T, LD64, 32, c0, 8), dv1, acc);
            const floatx4 bb = *reinterpret_cast<const floatx4*>(cb.b + pim(tb, 4 * g));
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] *= -bb[i];  // -D Y
            z[tb] = acc;
        }
        const bf16x8 nz0 = frag_from_c(z[0], z[1]), nz1 = frag_from_c(z[2], z[3]);
        // dS <- dS + Q^T dO - K^T Z
#pragma unroll
        for (int fb = 0; fb < K / 16; ++fb) {
            const int c0 = 32 * (fb >> 1) + 4 * (fb & 1);
            floatx4 acc = dS[fb];
            acc = mma(mf::frag_trc(cb.Q, LDK, 0, c0, 8), do0, acc);
            acc = mma(mf::frag_trc(cb.Q, LDK, 32, c0, 8), do1, acc);
            acc = mma(frag_tr(cb.Kr, LDK, 0, c0, 8), nz0, acc);
            acc = mma(frag_tr(cb.Kr, LDK, 32, c0, 8), nz1, acc);
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
template <int K, int NG>
struct GradSmem {
    bf16 Qs[64 * ldb<K>()];
    bf16 Ks[64 * ldb<K>()];
    bf16 Ps[64 * LD64];  // P[t][t'] (t' <= t)
    bf16 Tb[64 * LD64];  // bf16(T)[t][t'] (t' <= t), from the WY prep
    // b, dc/dlambda, dc/dbeta per token for items of even / odd position in
    // this workgroup's sequence (the next item's arrive during the closing)
    float coef[2][3][64];
    float dbh[NG][64];   // per-group partial dL/db
    // one 64-wide value slice's inputs; during an item's closing products the
    // next item's first slice is copied in here
    bf16 V[64 * LD64];   // v[:, slice]; each wave's (rows, value tiles) later hold D Y
    bf16 dO[64 * LD64];  // dO[:, slice]
    bf16 h[64 * ldb<K>()];   // h[v][f] for the slice's v
    bf16 dh[64 * ldb<K>()];  // dh[v][f]
    union {
        struct {  // one 64-wide value slice
            bf16 DR[64 * LD64];  // D R [t][v]; after the last slice, dG [i][j] (j < i)
            bf16 Vn[64 * LD64];  // Vn [t][v]
            bf16 dVn[64 * LD64]; // dVn [t][v]; after the last slice, Dm [t][t'] (t' <= t)
            bf16 Y[64 * LD64];   // Y [t][v]
        } s;
        struct {  // the item's dq, dk rows on their way out
            bf16 dq[64 * ldb<K>()];
            bf16 dk[64 * ldb<K>()];
        } o;
    } u;
};

// A 64 x K bf16 LDS tile: one [64][ldb<K>()] block, or (SPLIT_, K > 64)
// K / 64 column halves of 64 with row stride 72.  at(base, c) is the block
// holding column c, read at column col(c).
template <int K, bool SPLIT_>
struct KTile {
    static constexpr bool SPLIT = SPLIT_ && K > 64;
    static constexpr int KH = SPLIT ? K / 64 : 1, LD = SPLIT ? 72 : ldb<K>(), HALF = 64 * LD;
    static_assert(K % 64 == 0 && KH * HALF <= 64 * ldb<K>(), "K = 64 or 128");
    static __device__ __forceinline__ const bf16* at(const bf16* base, int c) {
        return SPLIT ? base + (c >> 6) * HALF : base;
    }
    static __device__ __forceinline__ int col(int c) { return SPLIT ? (c & 63) : c; }
    // every 16-byte piece of the 64 x K tile at src (row stride ld) into dst
    template <int NW>
    static __device__ __forceinline__ void copy(bf16* dst, const bf16* src, long ld, int nvalid,
                                                int rot, int l) {
        if constexpr (!SPLIT) {
            mf::dma_tile<64, K, ldb<K>(), NW>(dst, src, ld, nvalid, rot, l);
        } else {
#pragma unroll
            for (int hh = 0; hh < KH; ++hh)
                mf::dma_tile<64, 64, LD, NW>(dst + hh * HALF, src + 64 * hh, ld, nvalid, rot + hh, l);
        }
    }
    // offset of element (row, c) (c a multiple of 8)
    static __device__ __forceinline__ int off(int row, int c) {
        return (SPLIT ? (c >> 6) * HALF : 0) + row * LD + col(c);
    }
};

// Wave (tb, gq): tb = wave & 3 owns tokens 16tb .. 16tb+15 (the columns of
// every transposed tile it computes); gq = wave >> 2 picks one of NG groups of
// the value tiles (slice phase), of the key tiles (dq / dk) and of the 16-token
// blocks of the 64 x 64 chunk matrices: 4 / NG of each.  NG = 2 is 8 waves, NG
// = 4 is 16 (four per SIMD, half the tiles per wave).
//
// Persistent: workgroup b (one per CU) takes the (chunk, head) items b,
// b + gridDim.x, ... in heads-fastest order (the heads of one chunk are
// neighbouring row pieces of the same token rows).  An item's inputs are
// copied straight into LDS (global_load_lds) while the previous item ends:
// P once the last value slice's first phase is done, T after its second, the
// first value slice's v, dO, h and the per-token coefficients as soon as the
// slices end (the closing reads none of them), q and dh after the closing's
// Q^T Dm product and k after the last product that reads K.  Nothing of the next
// item passes through registers, so the copies never make a wave wait.
template <int NG>
constexpr int grad_threads() {
    return 256 * NG;
}

template <int K, int V, bool PS, int NG>
__global__ void __launch_bounds__(grad_threads<NG>()) grad_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const bf16* __restrict__ dO, const bf16* __restrict__ Tws, const float* __restrict__ bws,
    const float* __restrict__ dcws, const bf16* __restrict__ Pws, const bf16* __restrict__ hist,
    const bf16* __restrict__ dhist, SeqInfo si, int H, int nitems,
    bf16* __restrict__ dq, bf16* __restrict__ dk, bf16* __restrict__ dv,
    bf16* __restrict__ dbeta, TokLd ld) {
    constexpr int NTG = grad_threads<NG>(), NW = NTG / 64;  // threads, waves
    constexpr int LDK = ldb<K>(), NS = V / VS, NF = K / 16 / NG;  // NF key tiles per group
    // K-wide operand tiles: Qs and Ks are one [64][LDK] block each (Lk); the
    // 16-wave kernel keeps h and dh as K / 64 column halves of 64 with row
    // stride 72 (Lh; the same 64 x LDK elements), every fragment's k or line
    // range inside one half.  Measured at cfg3 against the other three
    // combinations, this one is 1-3 % faster.  (The 8-wave d_v = 256
    // instantiation keeps [64][LDK] tiles: with the halves, hipcc's register
    // allocation fails on it.)
    using Lk = KTile<K, false>;
    using Lh = KTile<K, NG == 4>;
    auto kh = [](const bf16* base, int c) { return Lk::at(base, c); };
    auto kcol = [](int c) { return Lk::col(c); };
    constexpr int LDH = Lk::LD;
    auto hh_ = [](const bf16* base, int c) { return Lh::at(base, c); };
    auto hcol = [](int c) { return Lh::col(c); };
    constexpr int LDS_H = Lh::LD;
    constexpr int EG = 4 / NG;  // value tiles / 16-token blocks per group
    // threads holding the v, dO slice and the h, dh slice prefetches (one
    // 16-byte piece each at most)
    constexpr int NTV = NTG < 64 * VS / 8 ? NTG : 64 * VS / 8;
    constexpr int NTH = NTG < 64 * K / 8 ? NTG : 64 * K / 8;
    static_assert(NG == 2 || NG == 4, "8 or 16 waves");
    __shared__ __attribute__((aligned(16))) GradSmem<K, NG> sm;
    const int w8 = mf::wave(), tb = w8 & 3, hf = w8 >> 2;
    const int nks = tb >= 2 ? 1 : 0;  // first k-step (of 32) that reaches t'' >= t
    const int f0 = hf * NF;            // first key tile of this group

    struct Item {
        int h, slot, len;
        long bos;
    };
    auto locate = [&](int it, Item& I) -> bool {
        if (it >= nitems) return false;
        I.h = it % H;
        I.slot = it / H;
        return locate_chunk(si, I.slot, I.bos, I.len);
    };
    // copies into LDS (l: lane); each is issued by all waves
    auto copy_p = [&](const Item& I, int l) {
        if constexpr (PS)
            dma_tri<NW>(sm.Ps, Pws + ((long)I.slot * H + I.h) * TRI_ELEMS, 2, l);
    };
    auto copy_dh0 = [&](const Item& I, int l) {
        Lh::template copy<NW>(sm.dh, dhist + ((long)I.slot * H + I.h) * V * K, K, 64, 6, l);
    };
    auto copy_slice0 = [&](const Item& I, int par, int l, bool with_p, bool with_dh = true) {
        const long cid = (long)I.slot * H + I.h, chb = cid * V * K;
        mf::dma_tile<64, VS, LD64, NW>(sm.V, v + I.bos * ld.v + (long)I.h * V, ld.v, I.len, 0, l);
        mf::dma_tile<64, VS, LD64, NW>(sm.dO, dO + (I.bos * H + I.h) * V, (long)H * V, I.len, 2, l);
        Lh::template copy<NW>(sm.h, hist + chb, K, 64, 4, l);
        if (with_dh) copy_dh0(I, l);
        if (with_p) copy_p(I, l);
        // b (16 chunks of 16 bytes) and dc/dlambda, dc/dbeta (32 chunks)
        if (w8 == NW - 1 && l < 16) mf::dma16(bws + cid * 64, 16u * l, sm.coef[par][0]);
        if (w8 == NW - 2 && l < 32) mf::dma16(dcws + cid * 128, 16u * l, sm.coef[par][1]);
    };
    auto copy_q = [&](const Item& I, int l) {
        Lk::template copy<NW>(sm.Qs, q + I.bos * ld.q + (long)I.h * K, ld.q, I.len, 3, l);
    };
    auto copy_t = [&](const Item& I, int l) {
        dma_tri<NW>(sm.Tb, Tws + ((long)I.slot * H + I.h) * TRI_ELEMS, 5, l);
    };
    auto copy_k = [&](const Item& I, int l) {
        Lk::template copy<NW>(sm.Ks, k + I.bos * ld.k + (long)I.h * K, ld.k, I.len, 1, l);
    };

    int it = blockIdx.x, par = 0;
    Item cur;
    if (!locate(it, cur)) return;  // uniform over the workgroup
    if constexpr (!PS)  // P's tiles above the diagonal are never written
        for (int i = threadIdx.x; i < 64 * LD64; i += NTG) sm.Ps[i] = (bf16)0.f;
    copy_slice0(cur, par, mf::lane(), true);
    copy_q(cur, mf::lane());
    copy_t(cur, mf::lane());
    copy_k(cur, mf::lane());
    for (;;) {
    // lane-dependent values are derived per item (see mf::tid_in)
    const int tid = mf::tid_in(it);
    const int l = tid & 63, g = l >> 4, r = l & 15;
    const int t = 16 * tb + r;  // this lane's token (column of the transposed tiles)
    const int h = cur.h, slot = cur.slot, len = cur.len;
    const long bos = cur.bos;
    const long chb = ((long)slot * H + h) * V * K;  // this chunk's h / dh block
    const float* cf = sm.coef[par][0];  // b, dc/dlambda, dc/dbeta at cf[0, 64, 128 + t]

    mf::TileRegs<64, VS, NTV> rv, rd;
    mf::TileRegs<64, K, NTH> rh, rdh;
    auto prefetch = [&](int s) {
        const int vv = s * VS;
        if (NTV == NTG || tid < NTV) {
            rv.load(v + bos * ld.v + (long)h * V + vv, ld.v, len, tid);
            rd.load(dO + (bos * H + h) * V + vv, (long)H * V, len, tid);
        }
        if (NTH == NTG || tid < NTH) {
            rh.load(hist + chb + (long)vv * K, K, 64, tid);
            rdh.load(dhist + chb + (long)vv * K, K, 64, tid);
        }
    };
    // ---- item setup: every input of the item's first slice is in flight
    mf::dma_wait();
    // the next item, looked up here where nothing is in flight (the varlen
    // lookup reads cu_seqlens offsets and waits for its loads)
    Item nxt;
    const bool more = locate(it + (int)gridDim.x, nxt);
    __syncthreads();  // every wave's copies have landed
    if (len < 64) {  // a sequence's last chunk: token rows past its end read as zero
        for (int i = tid; i < (64 - len) * (K / 8); i += NTG) {
            const int c = 8 * (i % (K / 8));
            const int o = Lk::off(len + i / (K / 8), c);
            *reinterpret_cast<bf16x8*>(sm.Qs + o) = bf16x8{};
            *reinterpret_cast<bf16x8*>(sm.Ks + o) = bf16x8{};
        }
        for (int i = tid; i < (64 - len) * (VS / 8); i += NTG) {
            const int o = (len + i / (VS / 8)) * LD64 + 8 * (i % (VS / 8));
            *reinterpret_cast<bf16x8*>(sm.V + o) = bf16x8{};
            *reinterpret_cast<bf16x8*>(sm.dO + o) = bf16x8{};
        }
        __syncthreads();
    }
    if constexpr (!PS) {
        for (int n = w8; n < 10; n += NW) {
            int I, J;
            lower_tile(n, I, J);
            floatx4 accp = zero4();
#pragma unroll
            for (int k0 = 0; k0 < K; k0 += 32)
                accp = mma(frag_nat(l, kh(sm.Ks, k0), LDH, 16 * J, kcol(k0)),
                           frag_nat(l, kh(sm.Qs, k0), LDH, 16 * I, kcol(k0)), accp);
            const int tq = 16 * I + r, tk = 16 * J + 4 * g;
            *reinterpret_cast<bf16x4*>(sm.Ps + tq * LD64 + tk) =
                bf16x4{(bf16)(tk + 0 <= tq ? accp[0] : 0.f), (bf16)(tk + 1 <= tq ? accp[1] : 0.f),
                       (bf16)(tk + 2 <= tq ? accp[2] : 0.f), (bf16)(tk + 3 <= tq ? accp[3] : 0.f)};
        }
        __syncthreads();
    }
    // B operand (line t, k = t') of T
    const bf16x8 tfr0 = frag_nat(l, sm.Tb, LD64, 16 * tb, 0), tfr1 = frag_nat(l, sm.Tb, LD64, 16 * tb, 32);
    const float bt = cf[t];
    // dL/db: (I + D strict_lower(G)) Vn = D R gives strict_lower(G) Vn =
    // R - D^-1 Vn, so rowsum(Y o R) + rowsum(dA o G) = rowsum(Y o Vn) / b, with
    // no G.  A 16-token block holding a b near 0 takes the explicit sum
    // instead (wave-uniform: every wave of the block sees the same 16 b).
    const bool dbx = __any(t < len && !(fabsf(bt) >= 1e-20f));

    // ---- value slices ----
    floatx4 dqa[NF], dka[NF], dma[EG], dya[EG];
#pragma unroll
    for (int fb = 0; fb < NF; ++fb) dqa[fb] = dka[fb] = zero4();
#pragma unroll
    for (int e = 0; e < EG; ++e) dma[e] = dya[e] = zero4();
    // this group's t' blocks reach t' <= t: block J holds tokens of
    // 32 (J >> 1) .. 32 (J >> 1) + 31 (pim interleaves J and J ^ 1)
    const bool jlive = 32 * ((EG * hf) >> 1) <= 16 * tb + 15;
    float dbp = 0.f;
    for (int s = 0; s < NS; ++s) {
        const int vv = s * VS;
        if (s > 0) {  // slice 0 was copied in with the item's other inputs
            __syncthreads();
            if (NTV == NTG || tid < NTV) {
                rv.store_rows(sm.V, LD64);
                rd.store_rows(sm.dO, LD64);
            }
            if (NTH == NTG || tid < NTH) {
                if constexpr (Lh::KH > 1) {
                    rh.store_rows_split(sm.h, Lh::LD, Lh::HALF);
                    rdh.store_rows_split(sm.dh, Lh::LD, Lh::HALF);
                } else {
                    rh.store_rows(sm.h, Lh::LD);
                    rdh.store_rows(sm.dh, Lh::LD);
                }
            }
            __syncthreads();
        }
        if (s + 1 < NS) prefetch(s + 1);
        // R^T = V^T - h K^T and dVn^T = dO^T P + dh K^T for value tiles
        // EG hf .. EG hf + EG - 1: tile (value 16vb + 4g + i, token t)
#pragma unroll
        for (int e = 0; e < EG; ++e) {
            const int vb = EG * hf + e;
            floatx4 ra = load4(sm.V + t * LD64 + 16 * vb + 4 * g);
            floatx4 da = zero4();
#pragma unroll
            for (int kb = 0; kb < K / 32; ++kb) {
                const int kc = 32 * kb;
                const bf16x8 kt = frag_nat(l, kh(sm.Ks, kc), LDH, 16 * tb, kcol(kc));
                ra = mma(frag_nat(l, hh_(sm.h, kc), LDS_H, 16 * vb, hcol(kc)), mf::neg(kt), ra);
                da = mma(frag_nat(l, hh_(sm.dh, kc), LDS_H, 16 * vb, hcol(kc)), kt, da);
            }
            // (both operands transposed: c-order rows, see mf::frag_trc)
            if (nks == 0) da = mma(frag_trc(l, sm.dO, LD64, 0, 16 * vb), frag_trc(l, sm.Ps, LD64, 0, 16 * tb), da);
            da = mma(frag_trc(l, sm.dO, LD64, 32, 16 * vb), frag_trc(l, sm.Ps, LD64, 32, 16 * tb), da);
            store4s(sm.u.s.DR + t * LD64 + 16 * vb + 4 * g, ra, bt);
            store4(sm.u.s.dVn + t * LD64 + 16 * vb + 4 * g, da);
            // the explicit db needs R itself: parked where this wave's Y goes
            if (dbx) store4(sm.u.s.Y + t * LD64 + 16 * vb + 4 * g, ra);
        }
        __syncthreads();
        // the last slice no longer reads P: the next item's P goes in now
        if (s == NS - 1 && more) copy_p(nxt, l);
        // Vn^T = (D R)^T T^T; Y^T = dVn^T T; db += sum_v Y R; Y -> Y, D Y -> V (and dv)
#pragma unroll
        for (int e = 0; e < EG; ++e) {
            const int vb = EG * hf + e;
            floatx4 vn = mma(frag_tr(l, sm.u.s.DR, LD64, 0, 16 * vb), tfr0, zero4());
            if (tb >= 2) vn = mma(frag_tr(l, sm.u.s.DR, LD64, 32, 16 * vb), tfr1, vn);
            store4(sm.u.s.Vn + t * LD64 + 16 * vb + 4 * g, vn);
            floatx4 y = zero4();
            if (nks == 0)
                y = mma(frag_trc(l, sm.u.s.dVn, LD64, 0, 16 * vb), frag_trc(l, sm.Tb, LD64, 0, 16 * tb), y);
            y = mma(frag_trc(l, sm.u.s.dVn, LD64, 32, 16 * vb), frag_trc(l, sm.Tb, LD64, 32, 16 * tb), y);
            if (dbx) {
                const floatx4 ra = load4(sm.u.s.Y + t * LD64 + 16 * vb + 4 * g);
#pragma unroll
                for (int i = 0; i < 4; ++i) dbp += y[i] * ra[i];
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) dbp += y[i] * vn[i];
            }
            store4(sm.u.s.Y + t * LD64 + 16 * vb + 4 * g, y);
            store4s(sm.V + t * LD64 + 16 * vb + 4 * g, y, bt);
        }
        __syncthreads();
        // nor T (its fragments for Vn are in registers since the item start)
        if (s == NS - 1 && more) copy_t(nxt, l);
        if (NTV == NTG || tid < NTV) {  // dv = D Y of this slice from its bf16 copy in V, as whole 16-byte row pieces
            static_assert(NTV == 64 * (VS / 8), "one piece per thread");
            const int tt = tid / (VS / 8), f = 8 * (tid % (VS / 8));
            if (tt < len)
                *reinterpret_cast<bf16x8*>(dv + (bos + tt) * ld.dv + (long)h * V + vv + f) =
                    *reinterpret_cast<const bf16x8*>(sm.V + tt * LD64 + f);
        }
        // dq^T += h^T dO^T; dk^T += dh^T Vn^T - h^T (D Y)^T  (key tiles f0 .. f0+NF-1)
        // (Y Vn^T)^T[t'][t] += sum_v Vn[t'] Y[t]; Dm^T[t'][t] += sum_v Vn[t'] dO[t]
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const bf16x8 dob = frag_nat(l, sm.dO, LD64, 16 * tb, 32 * ks);
            const bf16x8 dyb = mf::neg(frag_nat(l, sm.V, LD64, 16 * tb, 32 * ks));
            const bf16x8 vnb = frag_nat(l, sm.u.s.Vn, LD64, 16 * tb, 32 * ks);
#pragma unroll
            for (int fb = 0; fb < NF; ++fb) {
                const int fcl = 16 * (f0 + fb);
                const bf16x8 ha = frag_tr(l, hh_(sm.h, fcl), LDS_H, 32 * ks, hcol(fcl));
                dqa[fb] = mma(ha, dob, dqa[fb]);
                dka[fb] = mma(ha, dyb, dka[fb]);
                dka[fb] = mma(frag_tr(l, hh_(sm.dh, fcl), LDS_H, 32 * ks, hcol(fcl)), vnb, dka[fb]);
            }
            if (jlive) {
                const bf16x8 yb = frag_nat(l, sm.u.s.Y, LD64, 16 * tb, 32 * ks);
#pragma unroll
                for (int e = 0; e < EG; ++e) {
                    const int J = EG * hf + e;
                    const bf16x8 vr = frag_row(l, sm.u.s.Vn, LD64, pim(J, r), 32 * ks);
                    dya[e] = mma(vr, yb, dya[e]);
                    dma[e] = mma(vr, dob, dma[e]);
                }
            }
        }
    }
    // ---- closing products ----
    // dA[t][j] = -sum_v Y[t][v] Vn[j][v] (j < t) is complete in this wave's
    // tiles; dG = b dA (and, in blocks taking the explicit db, G recomputed
    // and db += sum_j dA G).  Dm (j <= t)
    // goes into dVn's tile, dG into D R's (both last read by the slices' second
    // phase), so one barrier ends the slices and the stores.
    bf16* const Dm = sm.u.s.dVn;
    bf16* const dGm = sm.u.s.DR;
    float dbg = 0.f;
#pragma unroll
    for (int e = 0; e < EG; ++e) {
        const int J = EG * hf + e;
        floatx4 dg = zero4();
        if (jlive) {
#pragma unroll
            for (int i = 0; i < 4; ++i) dg[i] = (pim(J, 4 * g + i) < t) ? -dya[e][i] : 0.f;  // dA
            if (dbx) {
                floatx4 gg = zero4();
#pragma unroll
                for (int k0 = 0; k0 < K; k0 += 32)
                    gg = mma(frag_row(l, kh(sm.Ks, k0), LDH, pim(J, r), kcol(k0)),
                             frag_nat(l, kh(sm.Ks, k0), LDH, 16 * tb, kcol(k0)), gg);
#pragma unroll
                for (int i = 0; i < 4; ++i) dbg += dg[i] * gg[i];
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) dg[i] *= bt;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (pim(J, 4 * g + i) > t) dma[e][i] = 0.f;
        store4(Dm + t * LD64 + pim(J, 4 * g), dma[e]);
        store4(dGm + t * LD64 + pim(J, 4 * g), dg);
    }
    // db: sum over the 4 lane groups holding token t, then over the groups
    // (rows past the sequence's end have b = 0 and are never written)
    dbp = dbx ? dbp + dbg : (t < len ? dbp / bt : 0.f);
    dbp += __shfl_xor(dbp, 16);
    dbp += __shfl_xor(dbp, 32);
    if (g == 0) sm.dbh[hf][t] = dbp;
    __syncthreads();  // slice buffers are free; Dm, dG, db complete
    // the next item's v, dO and h slices and coefficients into the free
    // buffers (the closing products read none of them); its dh below
    if (more) copy_slice0(nxt, par ^ 1, l, false, false);
    // dk^T += Q^T Dm (token t' = t, k = t >= t'), first, so Q is free early
    {
        const bf16x8 c1 = frag_trc(l, Dm, LD64, 32, 16 * tb);
        bf16x8 c0 = c1;
        if (nks == 0) c0 = frag_trc(l, Dm, LD64, 0, 16 * tb);
#pragma unroll
        for (int fb = 0; fb < NF; ++fb) {
            const int fc = 16 * (f0 + fb);
            if (nks == 0) dka[fb] = mma(frag_trc(l, kh(sm.Qs, fc), LDH, 0, kcol(fc)), c0, dka[fb]);
            dka[fb] = mma(frag_trc(l, kh(sm.Qs, fc), LDH, 32, kcol(fc)), c1, dka[fb]);
        }
    }
    __syncthreads();  // Q is read
    if (more) {
        copy_q(nxt, l);
        copy_dh0(nxt, l);
    }
    // dq^T += K^T Dm^T (k = t' <= t); dk^T += K^T dG^T (k = j < i = t) +
    // K^T dG (token j = t, k = i > j): the K fragments serve both
    {
        const bf16x8 m0 = frag_nat(l, Dm, LD64, 16 * tb, 0), m1 = frag_nat(l, Dm, LD64, 16 * tb, 32);
        const bf16x8 a0 = frag_nat(l, dGm, LD64, 16 * tb, 0), a1 = frag_nat(l, dGm, LD64, 16 * tb, 32);
        const bf16x8 b1 = frag_tr(l, dGm, LD64, 32, 16 * tb);
        bf16x8 b0 = b1;
        if (nks == 0) b0 = frag_tr(l, dGm, LD64, 0, 16 * tb);
#pragma unroll
        for (int fb = 0; fb < NF; ++fb) {
            const int fc = 16 * (f0 + fb);
            const bf16x8 k0 = frag_tr(l, kh(sm.Ks, fc), LDH, 0, kcol(fc)),
                         k1 = frag_tr(l, kh(sm.Ks, fc), LDH, 32, kcol(fc));
            dqa[fb] = mma(k0, m0, dqa[fb]);
            if (tb >= 2) dqa[fb] = mma(k1, m1, dqa[fb]);
            dka[fb] = mma(k0, a0, dka[fb]);
            if (tb >= 2) dka[fb] = mma(k1, a1, dka[fb]);
            if (nks == 0) dka[fb] = mma(k0, b0, dka[fb]);
            dka[fb] = mma(k1, b1, dka[fb]);
        }
    }
    // k of this lane's token and key tiles for the last term, then K is free
    bf16x4 kfin[NF];
#pragma unroll
    for (int fb = 0; fb < NF; ++fb)
        kfin[fb] = *reinterpret_cast<const bf16x4*>(kh(sm.Ks, 16 * (f0 + fb)) + t * LDH +
                                                    kcol(16 * (f0 + fb)) + 4 * g);
    __syncthreads();
    if (more) copy_k(nxt, l);  // nor K
    float dbt = sm.dbh[0][t];  // dL/db for token t
#pragma unroll
    for (int gg = 1; gg < NG; ++gg) dbt += sm.dbh[gg][t];
    // dk += 2 db c'(lambda) k; dq, dk (this half's key tiles) into LDS (the
    // closing buffers are free), then written out as whole 16-byte row pieces
    {
        const float s2 = 2.f * dbt * cf[64 + t];
        bf16* qs = sm.u.o.dq;  // [t][f], row stride LDK
        bf16* ks = sm.u.o.dk;
#pragma unroll
        for (int fb = 0; fb < NF; ++fb) {
            const int fc = 16 * (f0 + fb);
            store4(qs + t * LDK + fc + 4 * g, dqa[fb]);
            floatx4 a = dka[fb];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] += s2 * (float)kfin[fb][i];
            store4(ks + t * LDK + fc + 4 * g, a);
        }
        if (t < len && hf == 0 && g == 0) dbeta[(bos + t) * H + h] = (bf16)(dbt * cf[128 + t]);
        __syncthreads();
        for (int i = tid; i < 64 * (K / 8); i += NTG) {
            const int tt = i / (K / 8), f = 8 * (i % (K / 8));
            if (tt < len) {
                const long o = (long)h * K + f;
                *reinterpret_cast<bf16x8*>(dq + (bos + tt) * ld.dq + o) =
                    *reinterpret_cast<const bf16x8*>(qs + tt * LDK + f);
                *reinterpret_cast<bf16x8*>(dk + (bos + tt) * ld.dk + o) =
                    *reinterpret_cast<const bf16x8*>(ks + tt * LDK + f);
            }
        }
    }
    if (!more) break;
    it += (int)gridDim.x;
    par ^= 1;
    cur = nxt;
    }  // items
}

}  // namespace fast
}  // namespace q
}  // namespace efla
