// EFLA behind the reference ABI ("Mode R"): efla_forward_hip,
// efla_backward_hip, efla_chunked_scan_hip.
//
// Semantics follow kernels/cuda/efla.cu exactly: per (b, h) and token t
//   lambda = |k_t|^2, c = c(beta, lambda)
//   u = S^T k_t, S <- bf16(S + (c k_t)(v_t - u)^T)   (state re-rounded every token)
//   o_t = S k_t                                        (needs d_k == d_v)
// The work of a token is serial per (b, h), so a token's cost is its chain of
// dependent steps.  For d = 64 and 128 (k, v, dO aligned to d / 8 bytes) the
// state lives in registers (r_fast_kernel): consecutive lanes own one value
// column, S^T k and the update are lane-local, and o = S k (a sum over
// columns) is formed by MFMAs from a transposed LDS copy of the new state, one
// barrier per token pair.  The value columns evolve independently, so when
// B H leaves half of the CUs idle each (b, h) is split over two workgroups of
// half the columns (their fp32 row sums meet in one zeroed fp32 buffer by
// atomic adds, rounded once by r_combine_kernel).  Each
// segment's k, c k and v are staged in LDS at once, the next segment's reads
// in flight; every token's c(beta, |k|^2) comes from a separate parallel
// kernel.  Other d keep one workgroup per (b, h) and the state in LDS (row
// stride d+2): two LDS passes and four barriers per token against the
// reference's three global passes and ~13 barriers (r_forward_kernel).
// Reduction order differs from the reference's serial sums; values differ at
// fp32 rounding level before each bf16 rounding.
//
// The backward recomputes states from bf16 checkpoints (exact, since the
// states are bf16 values), rebuilds one segment's states at a time into a
// workspace, and runs the reference's BPTT (efla.cu:315-454) over the segment
// in reverse: for d = 64 / 128 with 32-token segments, dL/dS in fp32
// registers and the same column split (r_ckpt_kernel for the checkpoints,
// r_bwd_fast_kernel: a barrier-free rebuild, one barrier per reverse token),
// otherwise with 64-token segments and dL/dS in LDS (d <= 128) or the
// workspace (d <= 256).
#include <hip/hip_runtime.h>

#include "../../include/efla_hip.h"
#include "common.hpp"
#include "efla_coeff.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace efla {
namespace r {

constexpr int NTH = 256;
constexpr int MAXD = 256;
constexpr int SEG = 64;   // checkpoint spacing of the backward
constexpr int SEGF = 32;  // the same for the register-resident backward (d = 64, 128)

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
// forward, register-resident state (d = 64 or 128; other d take
// r_forward_kernel)
// ---------------------------------------------------------------------------
// c(beta, |k_t|^2) of every token, [b * H + h][t] (fp32), and dc/dlambda
// when dcout is set: 16 lanes per
// (token, head) row of d = 16 P values (P = 4 or 8), 16-byte loads, the
// squares summed per lane and then across the 16 lanes.
template <int P>
__global__ void __launch_bounds__(NTH) r_coeff_kernel(const bf16* __restrict__ k,
                                                      float* __restrict__ cout,
                                                      float* __restrict__ dcout, int H, long T,
                                                      float beta, long n) {
    const long i = ((long)blockIdx.x * NTH + threadIdx.x) / 16;  // (b, t, h), h fastest
    const int q = threadIdx.x & 15;
    float s = 0.f;
    if (i < n) {
        typedef __attribute__((__vector_size__(P * sizeof(__bf16)))) __bf16 bfP;
        const bfP x = *reinterpret_cast<const bfP*>(k + i * (16 * P) + P * q);
#pragma unroll
        for (int e = 0; e < P; ++e) s = fmaf((float)x[e], (float)x[e], s);
    }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) s += __shfl_xor(s, off);
    if (i < n && q == 0) {
        float c, dcl, dcb;
        efla_coeff(s, beta, c, dcl, dcb);
        const long h = i % H, bt = i / H, t = bt % T, b = bt / T;
        cout[(b * H + h) * T + t] = c;
        if (dcout) dcout[(b * H + h) * T + t] = dcl;
    }
}

// The token step with the state in registers: LPC lanes (consecutive) own
// value column c of S, each holding its RPL rows as packed bf16 pairs.
// Per token
//   u_c = sum_row k_row S[row][c]     bf16 dot2 over row pairs, then across
//                                     the LPC lanes of the column
//   S[row][c] = bf16(S + (c k_row) (v_c - u_c))       lane-local
//   o_row = sum_c S[row][c] k_c        the new state's columns go to LDS as
//                                      [c][row] and 16x16x32 MFMAs contract
//                                      them with k
// The updates need only the lane's own column, so tokens go in pairs: both
// updates, both new states to LDS, one barrier, then both o products.  Each
// segment of SEGF tokens has its k (bf16), c k (fp32, c from r_coeff_kernel)
// and v columns staged in LDS at once (SegRows, the global reads a segment
// ahead).  The o products of a pair read their fragments right after its
// barrier and run their MFMAs after the next pair's updates, so the reads
// overlap that work.  The bf16 roundings and the (c k) r product are the
// reference's; the sums run in another order (fp32 rounding level before each
// bf16 rounding).
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;

// Cross-lane moves through DPP (a VALU operand modifier) instead of the LDS
// permute unit: the lane's partner within its quad (xor 1, xor 2) and a
// rotation within its row of 16 lanes.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL,
                                                               0xF, 0xF, true));
}
// sum over the L (1, 2, 4 or 8) consecutive lanes of an aligned group, in every lane
template <int L>
__device__ __forceinline__ float quad_sum(float x) {
    if constexpr (L >= 2) x += dpp_f<0xB1>(x);   // quad_perm [1, 0, 3, 2]
    if constexpr (L >= 4) x += dpp_f<0x4E>(x);   // quad_perm [2, 3, 0, 1]
    if constexpr (L >= 8) x += dpp_f<0x141>(x);  // row_half_mirror: lane 7 - i of its 8
    return x;
}
// x from lane (row r, i) of the rows in ROWMASK (the DPP source lane), 0 elsewhere
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_rows(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                                  CTRL, ROWMASK, 0xF, false));
}
// sum over the wave of the values in lanes 4i (other lanes are ignored),
// uniform; all VALU: lane 4i's value to its quad, rotations within each row of
// 16 (every lane then holds its row's sum), then the GFX9 row broadcasts (lane
// 15 into rows 1 and 3, lane 31 into rows 2 and 3) leave the total in lane 63
__device__ __forceinline__ float wave_sum_q4(float x) {
    x = dpp_f<0x00>(x);            // quad_perm [0, 0, 0, 0]
    x += dpp_f<0x124>(x);          // row_ror:4
    x += dpp_f<0x128>(x);          // row_ror:8
    x += dpp_rows<0x142, 0xA>(x);  // row_bcast:15
    x += dpp_rows<0x143, 0xC>(x);  // row_bcast:31
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}

// Column split: the state's value columns evolve independently (the update
// and S^T k touch only their own column), so one (b, h) may be spread over NS
// workgroups of D / NS columns each, LPC lanes per column.  Only the row sums
// (o, and the backward's grad_k) span columns: with NS = 2 each workgroup
// adds its part into `part` (one zeroed fp32 buffer in the output's layout)
// with fp32 atomics, and r_combine_kernel rounds the sum once to bf16.  Each
// element receives exactly two addends onto zero, and fl(fl(0 + x) + y) =
// fl(x + y) = fl(fl(0 + y) + x), so the result does not depend on which
// workgroup adds first (4 bytes of scratch per output element).
// NS = 1, LPC = 4 is one workgroup per (b, h); NS = 2, LPC = 8 gives a grid of
// 2 B H with half the rows per lane (for B H below the CU count).
// a[i] for a lane-dependent i in 0..3 (a select chain, no scratch indexing)
__device__ __forceinline__ float pick4(const mf::floatx4& a, int i) {
    return i == 0 ? a[0] : i == 1 ? a[1] : i == 2 ? a[2] : a[3];
}

template <int D, int NS, int LPC>
constexpr int rfast_threads() {
    return D / NS * LPC;
}

// ---------------------------------------------------------------------------
// segment staging (forward, checkpoint pass, backward)
// ---------------------------------------------------------------------------
// A segment's (SEGF tokens) per-token rows in LDS: k, c k in fp32 (CKS), dO
// (DO), this workgroup's NC value columns of v (VS), c and dc/dlambda (DC).
template <int D, int NC, bool DO, bool CKS, bool VS, bool DC, int SG = SEGF>
struct SegLds {
    bf16 kb[SG][D];
    bf16 gb[DO ? SG : 1][D];
    float ckf[CKS ? SG : 1][D];
    bf16 vb[VS ? SG : 1][NC];
    float cc[SG], dcc[DC ? SG : 1];
};

// The same rows on their way in: load() issues the global reads of a segment
// into registers (a segment ahead of use, so their latency overlaps the
// current segment's work); store() writes them to SegLds once the current
// segment's readers are done.  Pieces of VW = d / 16 elements (d / 8 bytes,
// the alignment the host checks for k, dO and v) spread over the NT threads.
template <int D, int NC, int NT, bool DO, bool CKS, bool VS, bool DC, int SG = SEGF>
struct SegRows {
    static constexpr int VW = D / 16;
    static constexpr int NKP = SG * D / VW, IK = (NKP + NT - 1) / NT;   // k / dO pieces
    static constexpr int NVP = SG * NC / VW, IV = (NVP + NT - 1) / NT;  // v pieces
    typedef __attribute__((__vector_size__(VW * sizeof(__bf16)))) __bf16 bfV;
    bfV kx[IK], gx[DO ? IK : 1], vx[VS ? IV : 1];
    float cx[CKS ? IK : 1], cs, dcs;

    __device__ __forceinline__ void load(const bf16* __restrict__ k, const bf16* __restrict__ dO,
                                         const bf16* __restrict__ v, const float* __restrict__ cbh,
                                         const float* __restrict__ dcbh, long base0, long tstride,
                                         long t0, int n, int vcol0, int tid) {
#pragma unroll
        for (int it = 0; it < IK; ++it) {
            const int i = tid + it * NT, j = i / (D / VW), e0 = (i % (D / VW)) * VW;
            if (i < NKP && j < n) {
                const long o = base0 + (t0 + j) * tstride + e0;
                kx[it] = *reinterpret_cast<const bfV*>(k + o);
                if constexpr (DO) gx[it] = *reinterpret_cast<const bfV*>(dO + o);
                if constexpr (CKS) cx[it] = cbh[t0 + j];
            }
        }
        if constexpr (VS)
#pragma unroll
            for (int it = 0; it < IV; ++it) {
                const int i = tid + it * NT, j = i / (NC / VW), e0 = (i % (NC / VW)) * VW;
                if (i < NVP && j < n)
                    vx[it] = *reinterpret_cast<const bfV*>(v + base0 + (t0 + j) * tstride + vcol0 + e0);
            }
        if (tid < n) {
            cs = cbh[t0 + tid];
            if constexpr (DC) dcs = dcbh[t0 + tid];
        }
    }

    __device__ __forceinline__ void store(SegLds<D, NC, DO, CKS, VS, DC, SG>& sl, int n, int tid) const {
#pragma unroll
        for (int it = 0; it < IK; ++it) {
            const int i = tid + it * NT, j = i / (D / VW), e0 = (i % (D / VW)) * VW;
            if (i < NKP && j < n) {
                *reinterpret_cast<bfV*>(&sl.kb[j][e0]) = kx[it];
                if constexpr (DO) *reinterpret_cast<bfV*>(&sl.gb[j][e0]) = gx[it];
                if constexpr (CKS)
#pragma unroll
                    for (int e = 0; e < VW; ++e) sl.ckf[j][e0 + e] = cx[it] * (float)kx[it][e];
            }
        }
        if constexpr (VS)
#pragma unroll
            for (int it = 0; it < IV; ++it) {
                const int i = tid + it * NT, j = i / (NC / VW), e0 = (i % (NC / VW)) * VW;
                if (i < NVP && j < n) *reinterpret_cast<bfV*>(&sl.vb[j][e0]) = vx[it];
            }
        if (tid < n) {
            sl.cc[tid] = cs;
            if constexpr (DC) sl.dcc[tid] = dcs;
        }
    }
};

template <int D, int NS, int SG>
struct RFastSmem {
    static constexpr bool CKS = NS > 1;  // c k staged (fp32); else formed per row
    bf16 Sl[4][(D / NS) * (D + 8)];      // new states [c][row]: two tokens, double-buffered
    SegLds<D, D / NS, false, CKS, true, false, SG> seg;
};

// SG: tokens staged per segment (chunk_size's tuning hint; the results do not
// depend on it)
template <int D, int NS, int LPC, int SG>
__global__ void __launch_bounds__((rfast_threads<D, NS, LPC>())) r_fast_kernel(
    const bf16* __restrict__ k, const bf16* __restrict__ v, const float* __restrict__ coef,
    bf16* __restrict__ state, bf16* __restrict__ out, float* __restrict__ part_out,
    int H, long T) {
    constexpr int NC = D / NS, NT = rfast_threads<D, NS, LPC>(), NW = NT / 64;
    constexpr int RPL = D / LPC, NP = RPL / 2, LDS = D + 8;
    constexpr bool CKS = RFastSmem<D, NS, SG>::CKS;
    static_assert(RPL % 8 == 0 && (D == 64 || D == 128) && NC % 32 == 0 && NT % 64 == 0 &&
                      NT <= 1024 && D % (16 * NW) == 0 && SG % 2 == 0,
                  "d = 64 or 128, 32-column multiples per workgroup");
    __shared__ __attribute__((aligned(16))) RFastSmem<D, NS, SG> sm;
    const int tid = threadIdx.x, w = mf::wave(), l = mf::lane();
    const int bh = blockIdx.x / NS, cb = blockIdx.x % NS;
    const int col = cb * NC + tid / LPC, lcol = tid / LPC, part = tid % LPC, r0 = part * RPL;
    const int b = bh / H, h = bh % H;
    const long dd = (long)D * D, nsegf = (T + SG - 1) / SG;
    const long tstride = (long)H * D;  // elements between tokens
    const long base0 = (long)b * T * tstride + (long)h * D;
    const float* cbh = coef + (long)bh * T;
    bf16* st = state + (long)bh * dd;

    bf16x2 Sp[NP];  // rows r0 + 2p (low half) and r0 + 2p + 1 (high half)
#pragma unroll
    for (int p = 0; p < NP; ++p)
        Sp[p] = bf16x2{st[(long)(r0 + 2 * p) * D + col], st[(long)(r0 + 2 * p + 1) * D + col]};

    // o products of the last pair, fragments in registers
    constexpr int MT = D / 16 / NW, NK = NC / 32;
    bf16x8 af[2][MT][NK], bk[2][NK];
    long pp = -1;  // that pair's first token
    const int g = l >> 4, j = l & 15;
    auto o_reads = [&](long t, int jj, int sb) {  // token t (segment row jj), Sl buffer sb
        pp = t;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if (t + i >= T) break;
            const bf16* kb = sm.seg.kb[jj + i];
            const bf16* slt = sm.Sl[sb + i];
#pragma unroll
            for (int q = 0; q < NK; ++q) {
                const bf16x4 lo = *reinterpret_cast<const bf16x4*>(kb + cb * NC + 32 * q + 4 * g);
                const bf16x4 hi = *reinterpret_cast<const bf16x4*>(kb + cb * NC + 32 * q + 16 + 4 * g);
                bk[i][q] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    af[i][m][q] = mf::frag_trc(l, slt, LDS, 32 * q, 16 * (MT * w + m));
            }
        }
    };
    // A = S[row][c] (c-order k over c), B = k broadcast over the 16 columns
    auto o_products = [&]() {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const long t = pp + i;
            if (t >= T) break;
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                mf::floatx4 acc = mf::zero4();
#pragma unroll
                for (int q = 0; q < NK; ++q) acc = mf::mma(af[i][m][q], bk[i][q], acc);
                // the 16 columns of acc are equal (B is a broadcast of k)
                const long o = base0 + t * tstride + 16 * (MT * w + m) + 4 * g;
                if constexpr (NS == 1) {
                    if (j == 0) {
                        bf16x4 ov;
#pragma unroll
                        for (int e = 0; e < 4; ++e) ov[e] = (bf16)acc[e];
                        *reinterpret_cast<bf16x4*>(out + o) = ov;
                    }
                } else if (j < 4) {
                    // lanes 0..3 of each row group add one row each: the wave's
                    // 16 rows in one atomic instruction on one 64-byte line
                    unsafeAtomicAdd(part_out + o + j, pick4(acc, j));
                }
            }
        }
    };
    // one token's update from segment row jj; the new column piece to sl
    auto update = [&](int jj, bf16* sl) {
        // this lane's rows of k (bf16 pairs) and c k, all reads issued first
        bf16x8 kq[NP / 4];
        float ckr[RPL];
#pragma unroll
        for (int q = 0; q < NP / 4; ++q)
            kq[q] = *reinterpret_cast<const bf16x8*>(&sm.seg.kb[jj][r0 + 8 * q]);
        if constexpr (CKS) {
#pragma unroll
            for (int q = 0; q < RPL / 4; ++q) {
                const mf::floatx4 x = *reinterpret_cast<const mf::floatx4*>(&sm.seg.ckf[jj][r0 + 4 * q]);
#pragma unroll
                for (int e = 0; e < 4; ++e) ckr[4 * q + e] = x[e];
            }
        } else {
            const float cj = sm.seg.cc[jj];
#pragma unroll
            for (int i = 0; i < RPL; ++i) ckr[i] = cj * (float)kq[i / 8][i % 8];
        }
        const float vt = to_f(sm.seg.vb[jj][lcol]);
        // u = S^T k for this column (four partial sums, then the lanes of the column)
        float ua[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const bf16x2 kp = bf16x2{kq[p / 4][2 * (p % 4)], kq[p / 4][2 * (p % 4) + 1]};
            ua[p % 4] = __builtin_amdgcn_fdot2_f32_bf16(kp, Sp[p], ua[p % 4], false);
        }
        const float u = quad_sum<LPC>((ua[0] + ua[1]) + (ua[2] + ua[3]));
        const float rc = vt - u;
        // S <- bf16(S + (c k) r); the new column piece as bf16 into LDS
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const float lo = fmaf(ckr[2 * p], rc, (float)Sp[p][0]);
            const float hi = fmaf(ckr[2 * p + 1], rc, (float)Sp[p][1]);
            Sp[p] = bf16x2{(bf16)lo, (bf16)hi};
        }
#pragma unroll
        for (int q = 0; q < NP / 4; ++q)
            *reinterpret_cast<bf16x8*>(sl + 8 * q) =
                bf16x8{Sp[4 * q][0], Sp[4 * q][1], Sp[4 * q + 1][0], Sp[4 * q + 1][1],
                       Sp[4 * q + 2][0], Sp[4 * q + 2][1], Sp[4 * q + 3][0], Sp[4 * q + 3][1]};
    };

    SegRows<D, NC, NT, false, CKS, true, false, SG> rows;
    rows.load(k, nullptr, v, cbh, nullptr, base0, tstride, 0, (int)(T < SG ? T : SG), cb * NC,
              tid);
    long P = 0;  // token pairs so far (selects the Sl buffers)
    for (long seg = 0; seg < nsegf; ++seg) {
        const long t0 = seg * SG;
        const int n = (int)(T - t0 < SG ? T - t0 : SG);
        __syncthreads();  // the previous segment's rows read (its last o_reads)
        rows.store(sm.seg, n, tid);
        __syncthreads();
        if (seg + 1 < nsegf) {
            const long t2 = t0 + SG;
            rows.load(k, nullptr, v, cbh, nullptr, base0, tstride, t2,
                      (int)(T - t2 < SG ? T - t2 : SG), cb * NC, tid);
        }
        // pairs of tokens: both updates, both new states to LDS, the previous
        // pair's o products, one barrier, this pair's o fragments
        for (int jj = 0; jj < n; jj += 2, ++P) {
            const int sb = 2 * (int)(P & 1);
            update(jj, sm.Sl[sb] + lcol * LDS + r0);
            if (jj + 1 < n) update(jj + 1, sm.Sl[sb + 1] + lcol * LDS + r0);
            if (pp >= 0) o_products();
            __syncthreads();
            o_reads(t0 + jj, jj, sb);
        }
    }
    if (pp >= 0) o_products();
    // the final state back to the caller
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        st[(long)(r0 + 2 * p) * D + col] = Sp[p][0];
        st[(long)(r0 + 2 * p + 1) * D + col] = Sp[p][1];
    }
}

// The checkpoint pass of the register-resident backward: the forward's state
// update (as r_fast_kernel, same roundings) with no outputs but the state
// before every SEGF-th token, stored column-major to ck.  Each lane's column
// needs only its own rows of k and c k, so a segment runs without barriers
// from staged rows (two barriers per segment, the next segment's reads in
// flight meanwhile).
template <int D, int NS, int LPC>
__global__ void __launch_bounds__((rfast_threads<D, NS, LPC>())) r_ckpt_kernel(
    const bf16* __restrict__ k, const bf16* __restrict__ v, const float* __restrict__ coef,
    const bf16* __restrict__ state, bf16* __restrict__ ck, int H, long T) {
    constexpr int NC = D / NS, NT = rfast_threads<D, NS, LPC>();
    constexpr int RPL = D / LPC, NP = RPL / 2;
    static_assert(RPL % 8 == 0 && (D == 64 || D == 128) && NC % 32 == 0 && NT % 64 == 0 &&
                      NT <= 1024,
                  "d = 64 or 128, 32-column multiples per workgroup");
    __shared__ __attribute__((aligned(16))) SegLds<D, NC, false, true, true, false> sm;
    const int tid = threadIdx.x;
    const int bh = blockIdx.x / NS, cb = blockIdx.x % NS;
    const int col = cb * NC + tid / LPC, lcol = tid / LPC, part = tid % LPC, r0 = part * RPL;
    const int b = bh / H, h = bh % H;
    const long dd = (long)D * D, nsegf = (T + SEGF - 1) / SEGF;
    const long tstride = (long)H * D;
    const long base0 = (long)b * T * tstride + (long)h * D;
    const float* cbh = coef + (long)bh * T;
    const bf16* st = state + (long)bh * dd;

    bf16x2 S[NP];  // rows r0 + 2p (low half) and r0 + 2p + 1 (high half)
#pragma unroll
    for (int p = 0; p < NP; ++p)
        S[p] = bf16x2{st[(long)(r0 + 2 * p) * D + col], st[(long)(r0 + 2 * p + 1) * D + col]};
    SegRows<D, NC, NT, false, true, true, false> rows;
    rows.load(k, nullptr, v, cbh, nullptr, base0, tstride, 0, (int)(T < SEGF ? T : SEGF), cb * NC,
              tid);
    for (long seg = 0; seg < nsegf; ++seg) {
        const long t0 = seg * SEGF;
        const int n = (int)(T - t0 < SEGF ? T - t0 : SEGF);
        rows.store(sm, n, tid);
        __syncthreads();
        if (seg + 1 < nsegf) {
            const long t2 = t0 + SEGF;
            rows.load(k, nullptr, v, cbh, nullptr, base0, tstride, t2,
                      (int)(T - t2 < SEGF ? T - t2 : SEGF), cb * NC, tid);
        }
        // the state before token t0, column-major [c][row]
        bf16* dst = ck + ((long)bh * nsegf + seg) * dd + (long)col * D + r0;
#pragma unroll
        for (int q = 0; q < NP / 4; ++q)
            *reinterpret_cast<bf16x8*>(dst + 8 * q) =
                bf16x8{S[4 * q][0], S[4 * q][1], S[4 * q + 1][0], S[4 * q + 1][1],
                       S[4 * q + 2][0], S[4 * q + 2][1], S[4 * q + 3][0], S[4 * q + 3][1]};
        for (int j = 0; j < n; ++j) {
            bf16x8 kq[NP / 4];
            mf::floatx4 cq[RPL / 4];
#pragma unroll
            for (int q = 0; q < NP / 4; ++q)
                kq[q] = *reinterpret_cast<const bf16x8*>(&sm.kb[j][r0 + 8 * q]);
#pragma unroll
            for (int q = 0; q < RPL / 4; ++q)
                cq[q] = *reinterpret_cast<const mf::floatx4*>(&sm.ckf[j][r0 + 4 * q]);
            const float vt = to_f(sm.vb[j][lcol]);
            float ua[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const bf16x2 kp = bf16x2{kq[p / 4][2 * (p % 4)], kq[p / 4][2 * (p % 4) + 1]};
                ua[p % 4] = __builtin_amdgcn_fdot2_f32_bf16(kp, S[p], ua[p % 4], false);
            }
            const float u = quad_sum<LPC>((ua[0] + ua[1]) + (ua[2] + ua[3]));
            const float rc = vt - u;
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const float lo = fmaf(cq[p / 2][2 * (p % 2)], rc, (float)S[p][0]);
                const float hi = fmaf(cq[p / 2][2 * (p % 2) + 1], rc, (float)S[p][1]);
                S[p] = bf16x2{(bf16)lo, (bf16)hi};
            }
        }
        __syncthreads();  // the segment's rows read
    }
}

// ---------------------------------------------------------------------------
// backward, register-resident (d = 64 or 128)
// ---------------------------------------------------------------------------
// The reference BPTT (efla.cu:355-453) per token, last to first, with
// G = dL/dS (after the token) in fp32 registers in the forward's column-owner
// layout.  With g = G + dO k^T, u = S^T k, w2 = v - u, sw = g^T k, w1 = c sw:
//   grad_v = w1,   G <- g - k w1^T
//   grad_k = 2 grad_lambda k + S_n^T dO + sum_c (c g[:, c] w2_c - S[:, c] w1_c)
//   grad_lambda = dc/dlambda * sum_c w2_c sw_c       (= sum_row k_row (g w2)_row)
// where S / S_n are the states before / after the token.  Column sums are
// lane-local (plus the lanes of the column); the row sum goes through LDS as
// bf16 high and low parts of each fp32 summand (about 16 bits kept) and
// 16x16x32 MFMAs against ones.
// Segments of SEGF tokens are taken last to first.  A segment's k, dO, c and
// dc/dlambda (and c k in fp32 and this workgroup's v columns where LDS allows:
// the split kernels) are staged in LDS by the whole workgroup at once, their
// global reads issued during the previous segment's reverse pass; the segment
// is then rebuilt from its checkpoint (ck, column-major) with the forward step
// without barriers (each lane's column needs only its own rows), every state
// stored column-major to the workspace (hist), which the same lanes read back
// in the reverse pass (one barrier per token, for the row sum).
template <int D, int NS>
struct RBwdSmem {
    static constexpr bool CKS = NS > 1;  // c k and v staged; else formed per row / read per lane
    bf16 Mh[2][(D / NS) * (D + 8)];      // the row sum's summands [c][row], high bf16 part
    bf16 Ml[2][(D / NS) * (D + 8)];      // low part
    SegLds<D, D / NS, true, CKS, CKS, true> seg;
    float gkv[2][D / NS];                // S_n^T dO per column
    float red[2][16];                    // grad_c partials per wave
    // NS > 1: this workgroup's fp32 grad_k row sums of a segment [token][row],
    // added into the output buffer once per segment (by segment parity)
    float gks[NS > 1 ? 2 : 1][NS > 1 ? SEGF : 1][NS > 1 ? D : 1];
};

template <int D, int NS, int LPC>
__global__ void __launch_bounds__((rfast_threads<D, NS, LPC>())) r_bwd_fast_kernel(
    const bf16* __restrict__ dO, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ coef, const float* __restrict__ dcoef, const bf16* __restrict__ ck,
    bf16* __restrict__ hist_all, bf16* __restrict__ grad_k, float* __restrict__ part_gk,
    bf16* __restrict__ grad_v, bf16* __restrict__ grad_state, int H, long T) {
    constexpr int NC = D / NS, NT = rfast_threads<D, NS, LPC>(), NW = NT / 64;
    constexpr int RPL = D / LPC, NP = RPL / 2, LDS = D + 8;
    constexpr int MT = D / 16 / NW, NK = NC / 32;
    constexpr bool CKS = RBwdSmem<D, NS>::CKS;
    static_assert(RPL % 8 == 0 && (D == 64 || D == 128) && NC % 32 == 0 && NT % 64 == 0 &&
                      NT <= 1024 && D % (16 * NW) == 0 && LPC % 4 == 0 && NW <= 16,
                  "d = 64 or 128, 32-column multiples per workgroup, 4 or 8 lanes per column");
    __shared__ __attribute__((aligned(16))) RBwdSmem<D, NS> sm;
    const int tid = threadIdx.x, w = mf::wave(), l = mf::lane();
    const int bh = blockIdx.x / NS, cb = blockIdx.x % NS;
    const int col = cb * NC + tid / LPC, lcol = tid / LPC, part = tid % LPC, r0 = part * RPL;
    const int g4 = l >> 4, j16 = l & 15;
    const int b = bh / H, h = bh % H;
    const long dd = (long)D * D, nsegf = (T + SEGF - 1) / SEGF;
    const long tstride = (long)H * D;
    const long base0 = (long)b * T * tstride + (long)h * D;
    const float* cbh = coef + (long)bh * T;
    const float* dcbh = dcoef + (long)bh * T;
    bf16* hist = hist_all + (long)bh * (SEGF + 1) * dd;
    auto col_ptr = [&](bf16* basep, long jj) { return basep + jj * dd + (long)col * D + r0; };
    auto load_col = [&](const bf16* src, bf16x2 (&dst)[NP]) {
#pragma unroll
        for (int i = 0; i < NP / 4; ++i) {
            const bf16x8 x = *reinterpret_cast<const bf16x8*>(src + 8 * i);
#pragma unroll
            for (int e = 0; e < 4; ++e) dst[4 * i + e] = bf16x2{x[2 * e], x[2 * e + 1]};
        }
    };
    auto pack8 = [&](const bf16x2 (&x)[NP], int i) {
        return bf16x8{x[4 * i][0], x[4 * i][1], x[4 * i + 1][0], x[4 * i + 1][1],
                      x[4 * i + 2][0], x[4 * i + 2][1], x[4 * i + 3][0], x[4 * i + 3][1]};
    };
    auto store_col = [&](bf16* dst, const bf16x2 (&x)[NP]) {
#pragma unroll
        for (int i = 0; i < NP / 4; ++i) *reinterpret_cast<bf16x8*>(dst + 8 * i) = pack8(x, i);
    };

    float G[RPL];
#pragma unroll
    for (int i = 0; i < RPL; ++i) G[i] = 0.f;
    const bf16x8 ones = bf16x8{(bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f,
                               (bf16)1.f, (bf16)1.f, (bf16)1.f, (bf16)1.f};

    SegRows<D, NC, NT, true, CKS, CKS, true> rows;
    {
        const long t0 = (nsegf - 1) * SEGF;
        rows.load(k, dO, v, cbh, dcbh, base0, tstride, t0, (int)(T - t0), cb * NC, tid);
    }
    for (long seg = nsegf - 1; seg >= 0; --seg) {
        const long t0 = seg * SEGF, t1 = t0 + SEGF < T ? t0 + SEGF : T;
        const int n = (int)(t1 - t0);
        // ---- the segment's rows into LDS (the previous segment's last
        // readers are done: barrier at the end of its reverse pass)
        rows.store(sm.seg, n, tid);
        // ---- rebuild: hist[jj] = the state before token t0 + jj
        bf16x2 S[NP];
        load_col(ck + ((long)bh * nsegf + seg) * dd + (long)col * D + r0, S);
        store_col(col_ptr(hist, 0), S);
        bf16 vreg[2];
        if constexpr (!CKS) {
            vreg[0] = v[base0 + t0 * tstride + col];
            if (n > 1) vreg[1] = v[base0 + (t0 + 1) * tstride + col];
        }
        __syncthreads();
        for (int j = 0; j < n; ++j) {
            float vt;
            if constexpr (CKS) {
                vt = to_f(sm.seg.vb[j][lcol]);
            } else {
                vt = to_f(vreg[j & 1]);
                if (j + 2 < n) vreg[j & 1] = v[base0 + (t0 + j + 2) * tstride + col];
            }
            bf16x8 kq[NP / 4];
#pragma unroll
            for (int i = 0; i < NP / 4; ++i)
                kq[i] = *reinterpret_cast<const bf16x8*>(&sm.seg.kb[j][r0 + 8 * i]);
            float ckr[RPL];
            if constexpr (CKS) {
#pragma unroll
                for (int i = 0; i < RPL / 4; ++i) {
                    const mf::floatx4 x =
                        *reinterpret_cast<const mf::floatx4*>(&sm.seg.ckf[j][r0 + 4 * i]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) ckr[4 * i + e] = x[e];
                }
            } else {
                const float cj = sm.seg.cc[j];
#pragma unroll
                for (int i = 0; i < RPL; ++i) ckr[i] = cj * (float)kq[i / 8][i % 8];
            }
            float ua[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const bf16x2 kp = bf16x2{kq[p / 4][2 * (p % 4)], kq[p / 4][2 * (p % 4) + 1]};
                ua[p % 4] = __builtin_amdgcn_fdot2_f32_bf16(kp, S[p], ua[p % 4], false);
            }
            const float u = quad_sum<LPC>((ua[0] + ua[1]) + (ua[2] + ua[3]));
            const float rc = vt - u;
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const float lo = fmaf(ckr[2 * p], rc, (float)S[p][0]);
                const float hi = fmaf(ckr[2 * p + 1], rc, (float)S[p][1]);
                S[p] = bf16x2{(bf16)lo, (bf16)hi};
            }
            store_col(col_ptr(hist, j + 1), S);
        }
        // ---- reverse over the segment
        {
            // per lane: (v_c and) the column of the state before the token, one ahead
            bf16 vR[2];
            bf16x2 SpR[2][NP], Sn[NP];
            auto load_lane = [&](int j, int slot) {
                if (j >= 0) {
                    if constexpr (!CKS) vR[slot] = v[base0 + (t0 + j) * tstride + col];
                    load_col(col_ptr(hist, j), SpR[slot]);
                }
            };
            load_col(col_ptr(hist, n), Sn);
            load_lane(n - 1, 0);
            // the next segment's rows: reads in flight during this reverse pass
            if (seg > 0)
                rows.load(k, dO, v, cbh, dcbh, base0, tstride, t0 - SEGF, SEGF, cb * NC, tid);
            // token t0 + j: its (v and) state in vR[s], SpR[s]
            auto rtoken = [&](int j, int s) {
                const int par = j & 1;
                load_lane(j - 1, s ^ 1);
                const bf16* kb = sm.seg.kb[j];
                const bf16* gb = sm.seg.gb[j];
                const float c = sm.seg.cc[j];
                const float kc = (float)kb[col];
                const float vt = CKS ? to_f(sm.seg.vb[j][lcol]) : to_f(vR[s]);
                // this lane's rows of k and dO (bf16), read once for both passes
                bf16x8 kq[RPL / 8], gq[RPL / 8];
#pragma unroll
                for (int i8 = 0; i8 < RPL / 8; ++i8) {
                    kq[i8] = *reinterpret_cast<const bf16x8*>(kb + r0 + 8 * i8);
                    gq[i8] = *reinterpret_cast<const bf16x8*>(gb + r0 + 8 * i8);
                }
                // pass 1, column sums: u = S^T k, gk = S_n^T dO (bf16 pairs),
                // sw = g^T k with g = G + dO k_c (fp32, left in G)
                float ua[2] = {0.f, 0.f}, ga[2] = {0.f, 0.f}, sa[4] = {0.f, 0.f, 0.f, 0.f};
                float kf[RPL];
#pragma unroll
                for (int i8 = 0; i8 < RPL / 8; ++i8) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int p = 4 * i8 + e;
                        ua[e & 1] = __builtin_amdgcn_fdot2_f32_bf16(
                            bf16x2{kq[i8][2 * e], kq[i8][2 * e + 1]}, SpR[s][p], ua[e & 1], false);
                        ga[e & 1] = __builtin_amdgcn_fdot2_f32_bf16(
                            bf16x2{gq[i8][2 * e], gq[i8][2 * e + 1]}, Sn[p], ga[e & 1], false);
                    }
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int ii = 8 * i8 + e;
                        kf[ii] = (float)kq[i8][e];
                        G[ii] = fmaf((float)gq[i8][e], kc, G[ii]);
                        sa[e & 3] = fmaf(G[ii], kf[ii], sa[e & 3]);
                    }
                }
                const float u = quad_sum<LPC>(ua[0] + ua[1]);
                const float gk = quad_sum<LPC>(ga[0] + ga[1]);
                const float sw = quad_sum<LPC>((sa[0] + sa[1]) + (sa[2] + sa[3]));
                const float w2 = vt - u, w1 = c * sw, cw2 = c * w2;
                // pass 2: the row sum's summands c g w2 - S w1 (bf16 high + low
                // parts); G <- g - k w1^T
                bf16* mh = sm.Mh[par] + lcol * LDS + r0;
                bf16* ml = sm.Ml[par] + lcol * LDS + r0;
#pragma unroll
                for (int i8 = 0; i8 < RPL / 8; ++i8) {
                    bf16x8 hv, lv;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int ii = 8 * i8 + e;
                        const float sp = (float)SpR[s][ii / 2][ii % 2];
                        const float m = fmaf(G[ii], cw2, -(sp * w1));
                        hv[e] = (bf16)m;
                        lv[e] = (bf16)(m - (float)hv[e]);
                        G[ii] = fmaf(-kf[ii], w1, G[ii]);
                    }
                    *reinterpret_cast<bf16x8*>(mh + 8 * i8) = hv;
                    *reinterpret_cast<bf16x8*>(ml + 8 * i8) = lv;
                }
                // grad_c = sum_c w2_c sw_c: one value per column, then per wave
                const float gc = wave_sum_q4(part == 0 ? w2 * sw : 0.f);
                if (part == 0) {
                    sm.gkv[par][lcol] = gk;
                    grad_v[base0 + (t0 + j) * tstride + col] = (bf16)w1;
                }
                if (l == 0) sm.red[par][w] = gc;
#pragma unroll
                for (int p = 0; p < NP; ++p) Sn[p] = SpR[s][p];  // the next token's S_n
                __syncthreads();
                // rows 16 (MT w + m) ..: q = sum_c M[row][c] by MFMA against ones
                // (this workgroup's columns; grad_lambda from its columns' grad_c)
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const int f0 = 16 * (MT * w + m);
                    mf::floatx4 acc = mf::zero4();
#pragma unroll
                    for (int q = 0; q < NK; ++q) {
                        acc = mf::mma(mf::frag_trc(l, sm.Mh[par], LDS, 32 * q, f0), ones, acc);
                        acc = mf::mma(mf::frag_trc(l, sm.Ml[par], LDS, 32 * q, f0), ones, acc);
                    }
                    // the 16 columns of acc are equal (B is ones); with the
                    // column split lanes 0..3 of each row group add one row each
                    // (one atomic instruction per wave on one 64-byte line)
                    if (NS == 1 ? j16 == 0 : j16 < 4) {
                        float gsum = 0.f;
#pragma unroll
                        for (int ww = 0; ww < NW; ++ww) gsum += sm.red[par][ww];
                        const float glam2 = 2.f * gsum * sm.seg.dcc[j];
                        const long o = base0 + (t0 + j) * tstride + f0 + 4 * g4;
                        if constexpr (NS == 1) {
                            mf::floatx4 gv4;
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const int row = f0 + 4 * g4 + i;
                                gv4[i] = fmaf(glam2, (float)kb[row], acc[i] + sm.gkv[par][row]);
                            }
                            *reinterpret_cast<bf16x4*>(grad_k + o) =
                                bf16x4{(bf16)gv4[0], (bf16)gv4[1], (bf16)gv4[2], (bf16)gv4[3]};
                        } else {
                            const int row = f0 + 4 * g4 + j16, lr = row - cb * NC;
                            const float sn = (lr >= 0 && lr < NC) ? sm.gkv[par][lr] : 0.f;
                            sm.gks[seg & 1][j][row] = fmaf(glam2, (float)kb[row], pick4(acc, j16) + sn);
                        }
                    }
                }
            };
            for (int j = n - 1; j >= 0; j -= 2) {
                rtoken(j, 0);
                if (j - 1 >= 0) rtoken(j - 1, 1);
            }
        }
        __syncthreads();  // the segment's staged data and last row sums read
        if constexpr (NS > 1) {
            // the segment's grad_k row sums into the shared fp32 buffer: whole
            // 256-byte rows of atomics, off the token chain (issued per token,
            // each atomic's round trip landed in the next token's wait for its
            // state loads, which share the in-order vector-memory counter).
            // Segment seg - 1 writes the other buffer; seg - 2 writes this one
            // only after the barriers of seg - 1's rebuild.
            const float* src = &sm.gks[seg & 1][0][0];
            for (int i = tid; i < n * D; i += NT) {
                const int jj = i / D, row = i - jj * D;
                unsafeAtomicAdd(part_gk + base0 + (t0 + jj) * tstride + row, src[i]);
            }
        }
    }
    // dL/dS_0 in the reference's [row][c] layout
    bf16* gs = grad_state + (long)bh * dd;
#pragma unroll
    for (int i = 0; i < RPL; ++i) gs[(long)(r0 + i) * D + col] = (bf16)G[i];
}

// out[i] = bf16(sum_s part[s * pstride + i]) over `ns` fp32 slices, four
// elements per thread, slices in order (the column-split kernels leave one
// slice holding the whole fp32 sum: ns = 1)
__global__ void __launch_bounds__(NTH) r_combine_kernel(const float* __restrict__ part,
                                                        long pstride, int ns,
                                                        bf16* __restrict__ out, long n4) {
    for (long i = (long)blockIdx.x * NTH + threadIdx.x; i < n4; i += (long)gridDim.x * NTH) {
        mf::floatx4 a = reinterpret_cast<const mf::floatx4*>(part)[i];
        for (int sl = 1; sl < ns; ++sl) {
            const mf::floatx4 b = reinterpret_cast<const mf::floatx4*>(part + sl * pstride)[i];
#pragma unroll
            for (int e = 0; e < 4; ++e) a[e] += b[e];
        }
        reinterpret_cast<bf16x4*>(out)[i] = bf16x4{(bf16)a[0], (bf16)a[1], (bf16)a[2], (bf16)a[3]};
    }
}

// Workgroups per (b, h) for the register-resident kernels: 2 (d = 64, 128)
// when B H would leave at least half of the CUs without one.
// (Four workgroups of 32 columns, two per CU, measured slower at B H = 128:
// forward 5.5 against 5.2 ms, backward 26.5 against 24.7 ms.)
inline int r_split(size_t nbh) {
    const int ncu = device_cu_count();
    return ncu > 0 && nbh * 2 <= (size_t)ncu ? 2 : 1;
}

template <int D, int NS, int LPC>
void r_launch_fwd(bool checkpoints, int sg, const void* k, const void* v, const float* coef,
                  void* state, void* out, float* part, long pstride, bf16* ck, int H, long T,
                  size_t nbh, hipStream_t stream) {
    const dim3 grid((unsigned)(nbh * NS)), block(rfast_threads<D, NS, LPC>());
    if (checkpoints)
        EFLA_LAUNCH("efla_r_checkpoint", (r_ckpt_kernel<D, NS, LPC>), grid, block, stream,
                    (const bf16*)k, (const bf16*)v, coef, (const bf16*)state, ck, H, T);
    else if (sg == 16)
        EFLA_LAUNCH("efla_r_forward", (r_fast_kernel<D, NS, LPC, 16>), grid, block, stream,
                    (const bf16*)k, (const bf16*)v, coef, (bf16*)state, (bf16*)out, part,
                    H, T);
    else if (sg == 64 && (NS > 1 || D == 64))  // the LDS of the other shapes holds 32 at most
        EFLA_LAUNCH("efla_r_forward", (r_fast_kernel<D, NS, LPC, (NS > 1 || D == 64) ? 64 : 32>),
                    grid, block, stream, (const bf16*)k, (const bf16*)v, coef, (bf16*)state,
                    (bf16*)out, part, H, T);
    else
        EFLA_LAUNCH("efla_r_forward", (r_fast_kernel<D, NS, LPC, 32>), grid, block, stream,
                    (const bf16*)k, (const bf16*)v, coef, (bf16*)state, (bf16*)out, part,
                    H, T);
}

template <int D, int NS, int LPC>
void r_launch_bwd(const void* dO, const void* k, const void* v, const float* coef,
                  const float* dcoef, const bf16* ck, bf16* hist, void* grad_k, float* part,
                  long pstride, void* grad_v, void* grad_state, int H, long T, size_t nbh,
                  hipStream_t stream) {
    EFLA_LAUNCH("efla_r_backward", (r_bwd_fast_kernel<D, NS, LPC>), dim3((unsigned)(nbh * NS)),
                dim3(rfast_threads<D, NS, LPC>()), stream, (const bf16*)dO, (const bf16*)k,
                (const bf16*)v, coef, dcoef, ck, hist, (bf16*)grad_k, part,
                (bf16*)grad_v, (bf16*)grad_state, H, T);
}

// the register-resident forward (checkpoints = false) or checkpoint pass for
// head_dim d and split ns
inline void r_fwd_fast(int d, int ns, bool checkpoints, int sg, const void* k, const void* v,
                       const float* coef, void* state, void* out, float* part, long pstride,
                       bf16* ck, int H, long T, size_t nbh, hipStream_t stream) {
    if (d == 128 && ns == 1)
        r_launch_fwd<128, 1, 4>(checkpoints, sg, k, v, coef, state, out, part, pstride, ck, H, T, nbh, stream);
    else if (d == 128)
        r_launch_fwd<128, 2, 8>(checkpoints, sg, k, v, coef, state, out, part, pstride, ck, H, T, nbh, stream);
    else if (ns == 1)
        r_launch_fwd<64, 1, 4>(checkpoints, sg, k, v, coef, state, out, part, pstride, ck, H, T, nbh, stream);
    else
        r_launch_fwd<64, 2, 8>(checkpoints, sg, k, v, coef, state, out, part, pstride, ck, H, T, nbh, stream);
}

// chunk_size as the forward's segment length: 16, 32 or 64 tokens staged in
// LDS at once (the largest not above it, at least 16; 0 picks 32)
inline int r_segment(size_t chunk_size) {
    if (chunk_size == 0) return SEGF;
    return chunk_size >= 64 ? 64 : chunk_size >= 32 ? 32 : 16;
}

inline void r_combine(const float* part, long pstride, int ns, void* out, size_t elems,
                      hipStream_t stream) {
    const long n4 = (long)(elems / 4);
    const long nb = (n4 + NTH - 1) / NTH;
    EFLA_LAUNCH("efla_r_combine", r_combine_kernel, dim3((unsigned)(nb < (1L << 20) ? nb : (1L << 20))),
                dim3(NTH), stream, part, pstride, ns, (bf16*)out, n4);
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
    // chunk_size (ignored by the reference, efla.cu:495) is the register-resident
    // forward's segment length hint; the results do not depend on it
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
    const dim3 grid((unsigned)nbh);
    // the register-resident path: d = 64 / 128, k and v aligned for d / 8-byte
    // row loads (the coefficient kernel's, the segment staging's) and output
    // for 8-byte row pieces, at most 2^35 tokens
    const bool fast = (head_dim == 128 || head_dim == 64) &&
                      (uintptr_t)k % (head_dim / 8) == 0 && (uintptr_t)v % (head_dim / 8) == 0 &&
                      (uintptr_t)output % 8 == 0 && nbh * seq_len <= ((size_t)1 << 35);
    if (fast) {
        // every token's coefficient first (the stream's workspace), then the
        // register-resident token loop; with the column split the fp32 row
        // sums (one zeroed buffer both halves add into) follow the
        // coefficients in the workspace
        const size_t ntok = nbh * seq_len;
        const int ns = r_split(nbh);
        const size_t off_p = (ntok * sizeof(float) + 255) & ~(size_t)255;
        const size_t need = ns > 1 ? off_p + elems * sizeof(float) : ntok * sizeof(float);
        void* ws = nullptr;
        WsLease lease;
        int rc = workspace_acquire(need, stream, &ws, lease);
        if (rc != kSuccess) return rc;
        float* part = ns > 1 ? (float*)((char*)ws + off_p) : nullptr;
        if (part) {
            rc = fill_zero(part, elems * sizeof(float), stream);
            if (rc != kSuccess) return rc;
        }
        const dim3 cg((unsigned)((ntok * 16 + NTH - 1) / NTH));
        if (head_dim == 128)
            EFLA_LAUNCH("efla_r_coeff", r_coeff_kernel<8>, cg, dim3(NTH), stream, (const bf16*)k,
                        (float*)ws, (float*)nullptr, (int)num_heads, (long)seq_len, beta,
                        (long)ntok);
        else
            EFLA_LAUNCH("efla_r_coeff", r_coeff_kernel<4>, cg, dim3(NTH), stream, (const bf16*)k,
                        (float*)ws, (float*)nullptr, (int)num_heads, (long)seq_len, beta,
                        (long)ntok);
        r_fwd_fast((int)head_dim, ns, false, r_segment(chunk_size), k, v, (const float*)ws, state,
                   output, part, (long)elems, nullptr, (int)num_heads, (long)seq_len, nbh, stream);
        if (ns > 1) r_combine(part, (long)elems, 1, output, elems, stream);
    } else {
        EFLA_LAUNCH("efla_r_forward", r_forward_kernel, grid, dim3(NTH), stream, (const bf16*)k,
                    (const bf16*)v, (bf16*)state, (bf16*)output, (int)num_heads, (long)seq_len,
                    (int)head_dim, beta);
    }
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
    // the register-resident path: d = 64 / 128, k, dO and v aligned for d / 8-byte
    // row loads (the coefficient kernel's, the segment staging's) and grad_k
    // for 8-byte row pieces, at most 2^35 tokens
    const size_t ra = head_dim / 8;
    const bool fast = (head_dim == 128 || head_dim == 64) && (uintptr_t)k % ra == 0 &&
                      (uintptr_t)grad_output % ra == 0 && (uintptr_t)v % ra == 0 &&
                      (uintptr_t)grad_k % 8 == 0 && nbh * seq_len <= ((size_t)1 << 35);
    if (fast) {
        // workspace: checkpoints every SEGF tokens | one segment's states |
        // c and dc/dlambda per token (all column-major states, bf16)
        const size_t nsegf = (seq_len + SEGF - 1) / SEGF, ntok = nbh * seq_len;
        size_t ck_elems, hist_elems;
        if (!mul_ok(gse, nsegf, &ck_elems) || !mul_ok(gse, SEGF + 1, &hist_elems))
            return kInvalidConfiguration;
        const size_t off_hist = (ck_elems * 2 + 255) & ~(size_t)255;
        const size_t off_c = (off_hist + hist_elems * 2 + 255) & ~(size_t)255;
        const size_t off_dc = (off_c + ntok * 4 + 255) & ~(size_t)255;
        // with the column split: grad_k's fp32 sums (one zeroed buffer)
        const int ns = r_split(nbh);
        size_t elems = 0;
        if (!mul_ok(ntok, head_dim, &elems)) return kInvalidConfiguration;
        const size_t off_p = (off_dc + ntok * 4 + 255) & ~(size_t)255;
        const size_t need = ns > 1 ? off_p + elems * 4 : off_dc + ntok * 4 + 256;
        void* ws = nullptr;
        WsLease lease;
        int rc = workspace_acquire(need, stream, &ws, lease);
        if (rc != kSuccess) return rc;
        bf16* ck = (bf16*)ws;
        bf16* hist = (bf16*)((char*)ws + off_hist);
        float* coef = (float*)((char*)ws + off_c);
        float* dcoef = (float*)((char*)ws + off_dc);
        float* part = ns > 1 ? (float*)((char*)ws + off_p) : nullptr;
        if (part) {
            rc = fill_zero(part, elems * 4, stream);
            if (rc != kSuccess) return rc;
        }
        const dim3 cg((unsigned)((ntok * 16 + NTH - 1) / NTH));
        if (head_dim == 128)
            EFLA_LAUNCH("efla_r_coeff", r_coeff_kernel<8>, cg, dim3(NTH), stream, (const bf16*)k,
                        coef, dcoef, (int)num_heads, (long)seq_len, beta, (long)ntok);
        else
            EFLA_LAUNCH("efla_r_coeff", r_coeff_kernel<4>, cg, dim3(NTH), stream, (const bf16*)k,
                        coef, dcoef, (int)num_heads, (long)seq_len, beta, (long)ntok);
        r_fwd_fast((int)head_dim, ns, true, SEGF, k, v, coef, (void*)state, nullptr, nullptr, 0, ck,
                   (int)num_heads, (long)seq_len, nbh, stream);
        const int H = (int)num_heads;
        const long T = (long)seq_len, ps = (long)elems;
        if (head_dim == 128 && ns == 1)
            r_launch_bwd<128, 1, 4>(grad_output, k, v, coef, dcoef, ck, hist, grad_k, part, ps,
                                    grad_v, grad_state, H, T, nbh, stream);
        else if (head_dim == 128)
            r_launch_bwd<128, 2, 8>(grad_output, k, v, coef, dcoef, ck, hist, grad_k, part, ps,
                                    grad_v, grad_state, H, T, nbh, stream);
        else if (ns == 1)
            r_launch_bwd<64, 1, 4>(grad_output, k, v, coef, dcoef, ck, hist, grad_k, part, ps,
                                   grad_v, grad_state, H, T, nbh, stream);
        else
            r_launch_bwd<64, 2, 8>(grad_output, k, v, coef, dcoef, ck, hist, grad_k, part, ps,
                                   grad_v, grad_state, H, T, nbh, stream);
        if (ns > 1) r_combine(part, ps, 1, grad_k, elems, stream);
        return (int)hipPeekAtLastError();
    }
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
