// bf16 chunked EFLA kernels tuned for gfx950 (included by efla_q.hip after
// the SeqInfo helpers).  Same algorithm and workspace layout as the generic
// kernels in efla_q.hip; these keep operands in MFMA fragment registers
// instead of re-staging them, read LDS with 8/16-byte vectors, write global
// memory in 16-byte row segments, and prefetch the next chunk while the
// current one computes.
//
// prep_kernel   (grid: chunk slots x H)
//   b = c(beta, |k|^2); T = (I + strict_lower(diag(b) K K^T))^{-1} in fp32;
//   W = T diag(b) K, U = T diag(b) V (bf16, token layout like k / v).
// scan_kernel   (grid: sequences x H x V/64, one 64-wide value slice each)
//   carries S[:, slice] (K x 64, fp32) through the chunks of one sequence in
//   MFMA accumulators (wave w owns value columns 16w..16w+15) and per chunk
//     Vn = U - W S,  o = Q S + tril(Q K^T) Vn,  S <- S + K^T Vn.
#pragma once
#include "mfma.hpp"

namespace efla {
namespace q {
namespace fast {

using mf::bf16x4;
using mf::bf16x8;
using mf::floatx4;
using mf::frag_cc;
using mf::frag_from_c;
using mf::frag_nat;
using mf::mma;
using mf::mma_f32;
using mf::zero4;

constexpr int NT = 256;      // 4 waves
constexpr int LDF = 64 + 8;  // 64 x 64 fp32 matrices

// lower-triangular 16x16 tile (I >= J) number -> (I, J)
__device__ __forceinline__ void lower_tile(int n, int& I, int& J) {
    I = n < 1 ? 0 : n < 3 ? 1 : n < 6 ? 2 : 3;
    J = n - I * (I + 1) / 2;
}

// Pair-interleaved row map of a C tile: row r = 4g + i of tile `tile` stands
// for index 32 (tile >> 1) + 8g + 4 (tile & 1) + i.  Two tiles 2m, 2m+1 held
// this way are one natural-order MFMA operand over indices 32m .. 32m+31
// (frag_from_c), so results feed the next product straight from registers.
__device__ __forceinline__ int pim(int tile, int r) {
    return 32 * (tile >> 1) + 8 * (r >> 2) + 4 * (tile & 1) + (r & 3);
}

template <int D>
constexpr int ldb() {  // bf16 row stride: D + 16 keeps b128, b64 and tr16 reads conflict-free
    return D + 16;
}

// ---------------------------------------------------------------------------
// prep
// ---------------------------------------------------------------------------
template <int K, int V>
struct PrepSmem {
    bf16 Kr[64 * ldb<K>()];
    bf16 Vr[64 * ldb<V>()];
    float G[64 * LDF];  // K K^T (lower tiles)
    float T[64 * LDF];  // (I + A)^{-1}
    float lam[64];
    float b[64];
};

template <int K, int V>
__global__ void __launch_bounds__(NT) prep_kernel(const bf16* __restrict__ k,
                                                  const bf16* __restrict__ v,
                                                  const bf16* __restrict__ beta, SeqInfo si,
                                                  int H, bf16* __restrict__ Wout,
                                                  bf16* __restrict__ Uout,
                                                  bf16* __restrict__ Tout) {
    constexpr int LDK = ldb<K>(), LDV = ldb<V>();
    __shared__ __attribute__((aligned(16))) PrepSmem<K, V> sm;
    const int h = blockIdx.x, slot = blockIdx.y;  // heads fastest: one chunk's rows stay together
    long bos;
    int len;
    if (!locate_chunk(si, slot, bos, len)) return;
    const int w = mf::wave(), l = mf::lane(), g = l >> 4, r = l & 15;
    {
        mf::TileRegs<64, K, NT> kt;
        mf::TileRegs<64, V, NT> vt;
        kt.load(k + (bos * H + h) * K, (long)H * K, len);
        vt.load(v + (bos * H + h) * V, (long)H * V, len);
        kt.store_rows(sm.Kr, LDK);
        vt.store_rows(sm.Vr, LDV);
#pragma unroll
        for (int j = 0; j < kt.TPT; ++j) {
            const float s = kt.row_sumsq(j);
            if (kt.fg() == 0) sm.lam[kt.t0() + j] = s;
        }
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const int t = threadIdx.x;
        float c = 0.f, dcl, dcb;
        if (t < len) efla_coeff(sm.lam[t], (float)beta[(bos + t) * H + h], c, dcl, dcb);
        sm.b[t] = c;
    }
    // G = K K^T, lower tiles
    for (int n = w; n < 10; n += 4) {
        int I, J;
        lower_tile(n, I, J);
        floatx4 acc = zero4();
#pragma unroll
        for (int k0 = 0; k0 < K; k0 += 32)
            acc = mma(frag_nat(sm.Kr, LDK, 16 * I, k0), frag_nat(sm.Kr, LDK, 16 * J, k0), acc);
#pragma unroll
        for (int i = 0; i < 4; ++i) sm.G[(16 * I + 4 * g + i) * LDF + 16 * J + r] = acc[i];
    }
    __syncthreads();
    float* T = sm.T;
    // diagonal 16x16 blocks of T by forward substitution (lane = column)
    if (l < 16) {
        const int base = 16 * w;
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < i; ++j) s += sm.G[(base + i) * LDF + base + j] * x[j];
            x[i] = (i == l ? 1.f : 0.f) - sm.b[base + i] * s;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) T[(base + i) * LDF + base + l] = x[i];
    }
    __syncthreads();
    // off-diagonal blocks by distance d: T_IJ = -T_II sum_{m=J}^{I-1} A_Im T_mJ
    for (int d = 1; d < 4; ++d) {
        if (w < 4 - d) {
            const int I = w + d, J = w;
            const float bi = sm.b[16 * I + r];
            floatx4 y = zero4();
            for (int m = 16 * J; m < 16 * I; m += 4)
                y = mma_f32(bi * sm.G[(16 * I + r) * LDF + m + g], T[(m + g) * LDF + 16 * J + r], y);
            floatx4 t = zero4();
#pragma unroll
            for (int i = 0; i < 4; ++i) t = mma_f32(T[(16 * I + r) * LDF + 16 * I + 4 * g + i], y[i], t);
#pragma unroll
            for (int i = 0; i < 4; ++i) T[(16 * I + 4 * g + i) * LDF + 16 * J + r] = -t[i];
        }
        __syncthreads();
    }
    // optional bf16 copy of T for the backward: [t][t'], zero above the diagonal
    if (Tout) {
        const int tr = threadIdx.x >> 2, c0 = 16 * (threadIdx.x & 3);
        bf16x8 lo, hi;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            lo[c] = (bf16)(c0 + c <= tr ? T[tr * LDF + c0 + c] : 0.f);
            hi[c] = (bf16)(c0 + 8 + c <= tr ? T[tr * LDF + c0 + 8 + c] : 0.f);
        }
        bf16* dst = Tout + ((long)slot * H + h) * 64 * 64 + tr * 64 + c0;
        *reinterpret_cast<bf16x8*>(dst) = lo;
        *reinterpret_cast<bf16x8*>(dst + 8) = hi;
    }
    // W^T = K^T (T diag(b))^T and U^T likewise, for token block w.  B operand
    // (k = t', column t = 16w + r): (T diag(b))[t][t'], zero above the diagonal.
    const int t = 16 * w + r;
    const int nks = w >= 2 ? 2 : 1;
    bf16x8 tb[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int k0 = 32 * ks + 8 * g;
        const floatx4 t0 = *reinterpret_cast<const floatx4*>(T + t * LDF + k0);
        const floatx4 t1 = *reinterpret_cast<const floatx4*>(T + t * LDF + k0 + 4);
        const floatx4 b0 = *reinterpret_cast<const floatx4*>(sm.b + k0);
        const floatx4 b1 = *reinterpret_cast<const floatx4*>(sm.b + k0 + 4);
        bf16x8 f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            f[s] = (bf16)((k0 + s <= t) ? t0[s] * b0[s] : 0.f);
            f[4 + s] = (bf16)((k0 + 4 + s <= t) ? t1[s] * b1[s] : 0.f);
        }
        tb[ks] = f;
    }
    const bool live = t < len;
    bf16* wrow = Wout + ((bos + t) * H + h) * K + 4 * g;
    bf16* urow = Uout + ((bos + t) * H + h) * V + 4 * g;
#pragma unroll
    for (int fb = 0; fb < K / 16; ++fb) {
        floatx4 acc = mma(mf::frag_tr(sm.Kr, LDK, 0, 16 * fb), tb[0], zero4());
        if (nks > 1) acc = mma(mf::frag_tr(sm.Kr, LDK, 32, 16 * fb), tb[1], acc);
        if (live)
            *reinterpret_cast<bf16x4*>(wrow + 16 * fb) =
                bf16x4{(bf16)acc[0], (bf16)acc[1], (bf16)acc[2], (bf16)acc[3]};
    }
#pragma unroll
    for (int vb = 0; vb < V / 16; ++vb) {
        floatx4 acc = mma(mf::frag_tr(sm.Vr, LDV, 0, 16 * vb), tb[0], zero4());
        if (nks > 1) acc = mma(mf::frag_tr(sm.Vr, LDV, 32, 16 * vb), tb[1], acc);
        if (live)
            *reinterpret_cast<bf16x4*>(urow + 16 * vb) =
                bf16x4{(bf16)acc[0], (bf16)acc[1], (bf16)acc[2], (bf16)acc[3]};
    }
}

// ---------------------------------------------------------------------------
// forward scan + output
// ---------------------------------------------------------------------------
constexpr int VS = 64;  // value slice per workgroup

template <int K>
struct ScanBuf {
    bf16 W[64 * ldb<K>()];
    bf16 Q[64 * ldb<K>()];
    bf16 Kr[64 * ldb<K>()];
    bf16 U[64 * ldb<VS>()];  // U[:, slice]
};

template <int K>
struct ScanSmem {
    ScanBuf<K> buf[2];       // chunk n in buf[n & 1]; chunk n + 1 is stored meanwhile
    bf16 P[64 * ldb<64>()];  // tril(Q K^T) [t][t'] (upper tiles stay zero)
};

// Workgroup -> (sequence * H + head, value slice).  When the head count
// allows, the slices of one head get ids that are equal modulo 8 so they run
// on the same XCD and share its L2 for the W / Q / K tiles they all read.
__device__ __forceinline__ void scan_map(int id, int NH, int nvs, int& bh, int& vs) {
    if ((NH & 7) == 0) {
        const int grp = id / (8 * nvs), rem = id % (8 * nvs);
        bh = grp * 8 + (rem & 7);
        vs = rem >> 3;
    } else {
        bh = id / nvs;
        vs = id % nvs;
    }
}

// State layout in registers: S[fb] is a C tile whose row r = 4g + i is key
// index pim(fb, r) and whose column is value v0 + 16 w + (lane & 15).
template <int K, int V>
__global__ void __launch_bounds__(NT) scan_o_kernel(const bf16* __restrict__ q,
                                                    const bf16* __restrict__ k,
                                                    const bf16* __restrict__ W,
                                                    const bf16* __restrict__ U, SeqInfo si,
                                                    int H, const float* __restrict__ S0,
                                                    float* __restrict__ ST,
                                                    bf16* __restrict__ o) {
    constexpr int LDK = ldb<K>(), LDU = ldb<VS>(), LDP = ldb<64>(), NVS = V / VS;
    __shared__ __attribute__((aligned(16))) ScanSmem<K> sm;
    const int w = mf::wave(), l = mf::lane(), g = l >> 4, r = l & 15;
    int bh, vsl;
    scan_map(blockIdx.x, si.N * H, NVS, bh, vsl);
    const int seq = bh / H, h = bh % H, v0 = vsl * VS;
    long sbos, slen;
    int slot0;
    seq_bounds(si, seq, sbos, slen, slot0);
    const int nch = (int)((slen + 63) / 64);
    const long sbase = (long)bh * K * V;
    const int vcol = v0 + 16 * w + r;  // this lane's state column
    floatx4 S[K / 16];
#pragma unroll
    for (int fb = 0; fb < K / 16; ++fb) S[fb] = zero4();
    if (S0) {
#pragma unroll
        for (int fb = 0; fb < K / 16; ++fb)
#pragma unroll
            for (int i = 0; i < 4; ++i) S[fb][i] = S0[sbase + (long)pim(fb, 4 * g + i) * V + vcol];
    }
    for (int i = threadIdx.x; i < 64 * LDP; i += NT) sm.P[i] = (bf16)0.f;

    mf::TileRegs<64, K, NT> rw, rq, rk;
    mf::TileRegs<64, VS, NT> ru;
    auto prefetch = [&](int n) {
        const long bos = sbos + (long)n * 64;
        const int len = (int)min((long)64, slen - (long)n * 64);
        rw.load(W + (bos * H + h) * K, (long)H * K, len);
        rq.load(q + (bos * H + h) * K, (long)H * K, len);
        rk.load(k + (bos * H + h) * K, (long)H * K, len);
        ru.load(U + (bos * H + h) * V + v0, (long)H * V, len);
    };
    auto stage = [&](ScanBuf<K>& b) {
        rw.store_rows(b.W, LDK);
        rq.store_rows(b.Q, LDK);
        rk.store_rows(b.Kr, LDK);
        ru.store_rows(b.U, LDU);
    };
    if (nch > 0) {
        prefetch(0);
        stage(sm.buf[0]);
        if (nch > 1) prefetch(1);
    }
    for (int n = 0; n < nch; ++n) {
        const long bos = sbos + (long)n * 64;
        const int len = (int)min((long)64, slen - (long)n * 64);
        const ScanBuf<K>& cb = sm.buf[n & 1];
        __syncthreads();  // chunk n staged; everyone is done with chunk n - 1
        // P[t][t'] = q_t . k_t' for t' <= t, lower 16x16 tiles (I = t block,
        // J = t' block) computed transposed so each lane writes 4 consecutive t'
        for (int nt = w; nt < 10; nt += 4) {
            int I, J;
            lower_tile(nt, I, J);
            floatx4 acc = zero4();
#pragma unroll
            for (int k0 = 0; k0 < K; k0 += 32)
                acc = mma(frag_nat(cb.Kr, LDK, 16 * J, k0), frag_nat(cb.Q, LDK, 16 * I, k0), acc);
            const int tq = 16 * I + r, tk = 16 * J + 4 * g;
            *reinterpret_cast<bf16x4*>(sm.P + tq * LDP + tk) =
                bf16x4{(bf16)(tk + 0 <= tq ? acc[0] : 0.f), (bf16)(tk + 1 <= tq ? acc[1] : 0.f),
                       (bf16)(tk + 2 <= tq ? acc[2] : 0.f), (bf16)(tk + 3 <= tq ? acc[3] : 0.f)};
        }
        bf16x8 sb[K / 32];
#pragma unroll
        for (int kb = 0; kb < K / 32; ++kb) sb[kb] = frag_from_c(S[2 * kb], S[2 * kb + 1]);
        // Vn = U - W S; tile tb row 4g + i is token pim(tb, 4g + i)
        floatx4 vn[4];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            const bf16x4 u = mf::tr_rows4(cb.U, LDU, 32 * (tb >> 1) + 4 * (tb & 1), 16 * w, 4);
            vn[tb] = floatx4{(float)u[0], (float)u[1], (float)u[2], (float)u[3]};
            const int row = pim(tb, r);
#pragma unroll
            for (int kb = 0; kb < K / 32; ++kb)
                vn[tb] = mma(mf::frag_row(cb.W, LDK, row, 32 * kb), mf::neg(sb[kb]), vn[tb]);
        }
        // stage chunk n + 1 (its loads were issued one chunk ago), fetch n + 2
        if (n + 1 < nch) {
            stage(sm.buf[(n + 1) & 1]);
            if (n + 2 < nch) prefetch(n + 2);
        }
        __syncthreads();  // P complete
        const bf16x8 vb0 = frag_from_c(vn[0], vn[1]), vb1 = frag_from_c(vn[2], vn[3]);
        // o^T = S^T Q^T + Vn^T P^T: tile tb holds (value 16w + 4g + i, token 16tb + r)
        bf16* orow = o + (bos * H + h) * V + v0 + 16 * w + 4 * g;
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            floatx4 acc = zero4();
#pragma unroll
            for (int kb = 0; kb < K / 32; ++kb)
                acc = mma(sb[kb], frag_nat(cb.Q, LDK, 16 * tb, 32 * kb), acc);
            acc = mma(vb0, frag_nat(sm.P, LDP, 16 * tb, 0), acc);
            if (tb >= 2) acc = mma(vb1, frag_nat(sm.P, LDP, 16 * tb, 32), acc);
            const int t = 16 * tb + r;
            if (t < len)
                *reinterpret_cast<bf16x4*>(orow + (long)t * H * V) =
                    bf16x4{(bf16)acc[0], (bf16)acc[1], (bf16)acc[2], (bf16)acc[3]};
        }
        // S <- S + K^T Vn; A rows follow the state's key map pim(fb, r)
#pragma unroll
        for (int fb = 0; fb < K / 16; ++fb) {
            const int c0 = 32 * (fb >> 1) + 4 * (fb & 1);
            S[fb] = mma(mf::frag_tr(cb.Kr, LDK, 0, c0, 8), vb0, S[fb]);
            S[fb] = mma(mf::frag_tr(cb.Kr, LDK, 32, c0, 8), vb1, S[fb]);
        }
    }
    if (ST) {
#pragma unroll
        for (int fb = 0; fb < K / 16; ++fb)
#pragma unroll
            for (int i = 0; i < 4; ++i) ST[sbase + (long)pim(fb, 4 * g + i) * V + vcol] = S[fb][i];
    }
}

}  // namespace fast
}  // namespace q
}  // namespace efla
