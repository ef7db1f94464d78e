// bf16 chunked EFLA kernels tuned for gfx950 (included by efla_q.hip after
// the SeqInfo helpers).  These keep operands in MFMA fragment registers
// instead of re-staging them, read LDS with 16-byte and transposing reads,
// write global memory in 8/16-byte pieces, and prefetch the next chunk while
// the current one computes.
//
// With b = c(beta, |k|^2), D = diag(b), T = (I + strict_lower(D K K^T))^{-1}
// the chunk's effective values are Vn = T D (V - K S) (= U - W S with the WY
// factors W = T D K, U = T D V, which are never materialised).
//
// prep_kernel   (grid: H x chunk slots)
//   b and T (fp32 solve) for one chunk; writes bf16 T [64][64] (zero above the
//   diagonal) and fp32 b [64].
// scan_o_kernel (grid: sequences x H x V/64, one 64-wide value slice each)
//   carries S[:, slice] (K x 64, fp32) through the chunks of one sequence in
//   MFMA accumulators (compute wave w owns value columns 16w..16w+15; four
//   more waves stage the next chunks' inputs in LDS) and per chunk
//     R = V - K S,  Vn = T D R,  o = Q S + tril(Q K^T) Vn,  S <- S + K^T Vn;
//   optionally writes each chunk's start state to `hist` (bf16 [chunk][head]
//   [v][f], as the backward reads it) so the backward need not recompute it.
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

constexpr int NT = 256;  // 4 waves

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
// bf16 row stride D + 16: 16-byte row reads (frag_nat, frag_row) and c-order
// transposing reads (frag_trc) run at the LDS's full rate on it (about 200 B
// per CU-cycle measured, against about 120 for stride D + 8 with D = 64);
// natural-order transposing reads (frag_tr: rows r and r + 8 in the same
// banks) run at about 120 on every 16-byte-aligned stride.
constexpr int ldb() {
    return D + 16;
}

// The per-chunk lower-triangular 64 x 64 bf16 matrices T and P live in the
// workspace packed: the ten lower 16 x 16 tiles (I >= J) in lower_tile order,
// each row-major (16 rows of 32 bytes), then a zero stub that loads of the
// upper tiles read, so the LDS copies stay whole 64 x 64 tiles while HBM
// moves 5184 instead of 8192 bytes per (chunk, head).
constexpr int TRI_ZERO = 10 * 256;         // element offset of the zero stub
constexpr int TRI_ELEMS = TRI_ZERO + 32;  // bf16 per (chunk, head): 81 64-byte lines

// Element offset of the 8-column piece f (0..7) of row `row` (the zero stub
// for pieces above the diagonal tiles).
__device__ __forceinline__ int tri_off(int row, int f) {
    const int I = row >> 4, J = f >> 1;
    return J <= I ? (I * (I + 1) / 2 + J) * 256 + (row & 15) * 16 + (f & 1) * 8 : TRI_ZERO;
}

// Writes row `row`, column tile J (16 values as two 8-value pieces) of a
// packed matrix; the upper tiles are not stored, and the thread holding row 0,
// tile 1 writes the zero stub instead.
__device__ __forceinline__ void tri_store_piece(bf16* __restrict__ base, int row, int J,
                                                const bf16x8& lo, const bf16x8& hi) {
    if (J <= (row >> 4)) {
        bf16* dst = base + tri_off(row, 2 * J);
        *reinterpret_cast<bf16x8*>(dst) = lo;
        *reinterpret_cast<bf16x8*>(dst + 8) = hi;
    } else if (row == 0 && J == 1) {
        *reinterpret_cast<bf16x8*>(base + TRI_ZERO) = bf16x8{};
        *reinterpret_cast<bf16x8*>(base + TRI_ZERO + 8) = bf16x8{};
    }
}

// Buffer stores whose out-of-range lanes the hardware drops.  A store written
// as `if (cond) *p = x` becomes a branch around the instruction, and the
// compiler's wait counts at the join assume the path without it: a later
// wait for a load issued before the store then also waits for the store (one
// in-order counter for loads and stores).  Every lane of a wave issuing the
// instruction, with the condition folded into the offset or into the
// resource's byte count, keeps the count the same on every path.
constexpr unsigned BUF_OOB = 0x40000000u;  // an offset past every resource used here
__device__ __forceinline__ __amdgpu_buffer_rsrc_t out_rsrc(const void* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}
__device__ __forceinline__ void bstore8(bf16x4 x, __amdgpu_buffer_rsrc_t r, unsigned off) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(mf::int2v, x), r, (int)off, 0, 0);
}
__device__ __forceinline__ void bstore16(bf16x8 x, __amdgpu_buffer_rsrc_t r, unsigned off) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(mf::int4v, x), r, (int)off, 0, 0);
}
// tri_store_piece through a resource over one packed matrix (no store when
// the resource holds 0 bytes)
__device__ __forceinline__ void tri_store_piece(__amdgpu_buffer_rsrc_t r, int row, int J,
                                                const bf16x8& lo, const bf16x8& hi) {
    const bool tile = J <= (row >> 4), stub = row == 0 && J == 1;
    const unsigned off = tile ? 2u * tri_off(row, 2 * J) : stub ? 2u * TRI_ZERO : BUF_OOB;
    bstore16(tile ? lo : bf16x8{}, r, off);
    bstore16(tile ? hi : bf16x8{}, r, off + 16);
}

// A packed matrix into the registers of a 64 x 64 tile loader, as
// TileRegs::load would hold the full matrix (upper pieces read as zeros).
template <int NT>
__device__ __forceinline__ void load_tri(mf::TileRegs<64, 64, NT>& r, const bf16* __restrict__ src,
                                         int thread = (int)threadIdx.x) {
    r.tid = thread;
    r.valid = 64;
    const int f = r.fg(), t = r.t0();
#pragma unroll
    for (int j = 0; j < r.TPT; ++j) r.x[j] = *reinterpret_cast<const bf16x8*>(src + tri_off(t + j, f));
}

constexpr int LD64 = ldb<64>();

// A packed lower-triangular matrix (tri_off) straight into a [64][LD64] LDS
// tile, as mf::dma_tile copies a full one: every 16-byte LDS chunk is written,
// the upper and pad chunks from the zero stub.
template <int NW>
__device__ __forceinline__ void dma_tri(bf16* lds, const bf16* src, int rot, int l) {
    constexpr int CPR = LD64 / 8, NI = 64 * CPR / 64;
    const int w = mf::wave();
    for (int i = (w + NW - rot % NW) % NW; i < NI; i += NW) {
        const int c = 64 * i + l, row = c / CPR, col = c - row * CPR;
        mf::dma16(src, (unsigned)(col < 8 ? tri_off(row, col) : TRI_ZERO) * 2u, lds + 512 * i);
    }
}

__device__ __forceinline__ void store4(bf16* p, floatx4 a) {
    *reinterpret_cast<bf16x4*>(p) = bf16x4{(bf16)a[0], (bf16)a[1], (bf16)a[2], (bf16)a[3]};
}

// Write a K x 64 state slice to hist[v][f] (row stride K) as bf16 from its
// operand fragments: sb[kb] holds keys 32 kb + 8 g .. 32 kb + 8 g + 7 of
// column vcol, one 16-byte store each.
template <int K>
__device__ __forceinline__ void store_state_frag(bf16* __restrict__ hist, const bf16x8* sb, int vcol) {
    bf16* p = hist + (long)vcol * K + 8 * (mf::lane() >> 4);
#pragma unroll
    for (int kb = 0; kb < K / 32; ++kb) *reinterpret_cast<bf16x8*>(p + 32 * kb) = sb[kb];
}
// the same through a resource over the K x V block (no store when it holds 0 bytes)
template <int K>
__device__ __forceinline__ void store_state_frag(__amdgpu_buffer_rsrc_t r, const bf16x8* sb, int vcol) {
    const unsigned o = 2u * (unsigned)(vcol * K + 8 * (mf::lane() >> 4));
#pragma unroll
    for (int kb = 0; kb < K / 32; ++kb) bstore16(sb[kb], r, o + 64u * kb);
}

// ---------------------------------------------------------------------------
// prep
// ---------------------------------------------------------------------------
// G = K K^T and T = (I + strict_lower(D G))^{-1} are kept as their ten lower
// 16x16 tiles, packed, fp32 (row stride 17 for G, 16 for T), both in the space
// k occupies until G is formed: 21 KB of LDS for K = 128, so seven workgroups
// fit on a CU (the kernel is a chain of short dependent phases and runs as
// fast as it has workgroups in flight).
constexpr int PT_LD = 17;  // G tiles
constexpr int PT_SZ = 16 * PT_LD;
constexpr int PTT_LD = 16;  // T tiles: 16-byte aligned rows for the bf16 write-out
constexpr int PTT_SZ = 16 * PTT_LD;

// packed offset of lower tile (I, J), I >= J, for tiles of `sz` floats
__device__ __forceinline__ int ptile(int I, int J, int sz = PT_SZ) {
    return (I * (I + 1) / 2 + J) * sz;
}

template <int K>
struct PrepSmem {
    union {
        bf16 Kr[64 * ldb<K>()];  // k, until K K^T is formed
        struct {
            float G[10 * PT_SZ];   // lower tiles of K K^T
            float T[10 * PTT_SZ];  // lower tiles of (I + A)^{-1}
        } f;
    } u;
    float lam[64];
    float b[64];
};

template <int K>
__global__ void __launch_bounds__(NT) prep_kernel(const bf16* __restrict__ k,
                                                  const bf16* __restrict__ beta, SeqInfo si,
                                                  int H, bf16* __restrict__ Tout,
                                                  float* __restrict__ bout,
                                                  float* __restrict__ dcout, long ldk) {
    constexpr int LDK = ldb<K>();
    __shared__ __attribute__((aligned(16))) PrepSmem<K> sm;
    const int h = blockIdx.x, slot = blockIdx.y;  // heads fastest: one chunk's rows stay together
    long bos;
    int len;
    if (!locate_chunk(si, slot, bos, len)) return;
    const int w = mf::wave(), l = mf::lane(), g = l >> 4, r = l & 15;
    const long cid = (long)slot * H + h;
    // beta of token threadIdx.x, loaded with k so its latency is not paid twice
    const float bet = (threadIdx.x < 64 && (int)threadIdx.x < len)
                          ? (float)beta[(bos + threadIdx.x) * H + h] : 0.f;
    {
        mf::TileRegs<64, K, NT> kt;
        kt.load(k + bos * ldk + (long)h * K, ldk, len);
        kt.store_rows(sm.u.Kr, LDK);
#pragma unroll
        for (int j = 0; j < kt.TPT; ++j) {
            const float s = kt.row_sumsq(j);
            if (kt.fg() == 0) sm.lam[kt.t0() + j] = s;
        }
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const int t = threadIdx.x;
        float c = 0.f, dcl = 0.f, dcb = 0.f;
        if (t < len) efla_coeff(sm.lam[t], bet, c, dcl, dcb);
        sm.b[t] = c;
        bout[cid * 64 + t] = c;
        // dc/dlambda and dc/dbeta for the backward: [chunk][head][2][64]
        if (dcout) {
            dcout[cid * 128 + t] = dcl;
            dcout[cid * 128 + 64 + t] = dcb;
        }
    }
    // G = K K^T, lower tiles (wave w: tiles w, w + 4, w + 8), held in
    // registers until every wave is done with k, whose space G and T take
    floatx4 gacc[3];
#pragma unroll
    for (int u = 0; u < 3; ++u) {
        const int n = w + 4 * u;
        gacc[u] = zero4();
        if (n < 10) {
            int I, J;
            lower_tile(n, I, J);
#pragma unroll
            for (int k0 = 0; k0 < K; k0 += 32)
                gacc[u] = mma(frag_nat(sm.u.Kr, LDK, 16 * I, k0),
                              frag_nat(sm.u.Kr, LDK, 16 * J, k0), gacc[u]);
        }
    }
    __syncthreads();  // k is dead from here
#pragma unroll
    for (int u = 0; u < 3; ++u) {
        const int n = w + 4 * u;
        if (n < 10) {
            int I, J;
            lower_tile(n, I, J);
            float* Gt = sm.u.f.G + ptile(I, J);
#pragma unroll
            for (int i = 0; i < 4; ++i) Gt[(4 * g + i) * PT_LD + r] = gacc[u][i];
        }
    }
    __syncthreads();
    // diagonal 16x16 blocks of T by forward substitution (lane = column)
    if (l < 16) {
        const int base = 16 * w;
        const float* Gd = sm.u.f.G + ptile(w, w);
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < i; ++j) s += Gd[i * PT_LD + j] * x[j];
            x[i] = (i == l ? 1.f : 0.f) - sm.b[base + i] * s;
        }
        float* Td = sm.u.f.T + ptile(w, w, PTT_SZ);
#pragma unroll
        for (int i = 0; i < 16; ++i) Td[i * PTT_LD + l] = x[i];
    }
    __syncthreads();
    // off-diagonal blocks by distance d: T_IJ = -T_II sum_{m=J}^{I-1} A_Im T_mJ
    for (int d = 1; d < 4; ++d) {
        if (w < 4 - d) {
            const int I = w + d, J = w;
            const float bi = sm.b[16 * I + r];
            floatx4 y = zero4();
            for (int m = 16 * J; m < 16 * I; m += 4) {
                const int mb = m >> 4, mo = (m & 15) + g;
                y = mma_f32(bi * sm.u.f.G[ptile(I, mb) + r * PT_LD + mo],
                            sm.u.f.T[ptile(mb, J, PTT_SZ) + mo * PTT_LD + r], y);
            }
            const float* Tii = sm.u.f.T + ptile(I, I, PTT_SZ) + r * PTT_LD + 4 * g;
            floatx4 t = zero4();
#pragma unroll
            for (int i = 0; i < 4; ++i) t = mma_f32(Tii[i], y[i], t);
            float* Tij = sm.u.f.T + ptile(I, J, PTT_SZ);
#pragma unroll
            for (int i = 0; i < 4; ++i) Tij[(4 * g + i) * PTT_LD + r] = -t[i];
        }
        __syncthreads();
    }
    // bf16 T [t][t'], zero above the diagonal: thread -> row tr, column tile J
    {
        const int tr = threadIdx.x >> 2, J = threadIdx.x & 3, I = tr >> 4, i = tr & 15;
        bf16x8 lo, hi;
        if (J <= I) {
            const floatx4* src =
                reinterpret_cast<const floatx4*>(sm.u.f.T + ptile(I, J, PTT_SZ) + i * PTT_LD);
            float v[16];
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const floatx4 f = src[q4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[4 * q4 + e] = f[e];
            }
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                lo[c] = (bf16)(J < I || c <= i ? v[c] : 0.f);
                hi[c] = (bf16)(J < I || 8 + c <= i ? v[8 + c] : 0.f);
            }
        } else {
#pragma unroll
            for (int c = 0; c < 8; ++c) lo[c] = hi[c] = (bf16)0.f;
        }
        tri_store_piece(Tout + cid * TRI_ELEMS, tr, J, lo, hi);
    }
}

// ---------------------------------------------------------------------------
// forward scan + output
// ---------------------------------------------------------------------------
constexpr int VS = 64;  // value slice per workgroup

template <int K>
struct ScanBuf {
    bf16 Q[64 * ldb<K>()];
    bf16 Kr[64 * ldb<K>()];
    bf16 Vs[64 * ldb<VS>()];  // v[:, slice]
    bf16 T[64 * ldb<64>()];   // bf16 T [t][t']
    float b[64];
};

template <int K>
struct ScanSmem {
    ScanBuf<K> buf[2];       // chunk n in buf[n & 1]; chunk n + 1 is stored meanwhile
    bf16 P[64 * ldb<64>()];  // tril(Q K^T) [t][t'] (upper tiles stay zero)
};

// Workgroup -> (sequence * H + head, value slice).  When the head count
// allows, the slices of one head get ids that are equal modulo 8 so they run
// on the same XCD and share its L2 for the Q / K / T tiles they all read.
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

// Per-chunk inputs of the scans, loaded one chunk ahead into registers.
template <int K, bool WITH_Q, bool VALUES>
struct ChunkRegs {
    mf::TileRegs<64, K, NT> rq, rk;
    mf::TileRegs<64, VS, NT> rv;  // v (VALUES) or dO slice
    mf::TileRegs<64, 64, NT> rt;
    float b;                      // b of token thread & 63
    int thread;                   // index among the NT threads that load and stage
    __device__ __forceinline__ void load(const bf16* q, const bf16* k, const bf16* vsl,
                                         const bf16* Tc, const float* bc, long bos, int len,
                                         int h, int V, int v0, long cid, long lq, long lk,
                                         long lv, int th = (int)threadIdx.x) {
        thread = th;
        if (WITH_Q) rq.load(q + bos * lq + (long)h * K, lq, len, th);
        rk.load(k + bos * lk + (long)h * K, lk, len, th);
        rv.load(vsl + bos * lv + (long)h * V + v0, lv, len, th);
        load_tri(rt, Tc + cid * TRI_ELEMS, th);
        b = bc[cid * 64 + (th & 63)];  // every lane: no branch around the load
    }
    template <typename Buf>
    __device__ __forceinline__ void stage(Buf& bf) {
        if constexpr (WITH_Q) rq.store_rows(bf.Q, ldb<K>());
        rk.store_rows(bf.Kr, ldb<K>());
        rv.store_rows(bf.Vs, ldb<VS>());
        rt.store_rows(bf.T, ldb<64>());
        bf.b[thread & 63] = b;  // every lane (the same values): no branch around the write
    }
};

// State layout in registers: S[fb] is a C tile whose row r = 4g + i is key
// index pim(fb, r) and whose column is value v0 + 16 w + (lane & 15).
// Token tiles (R, Vn) use the same map for their rows: tile tb row 4g + i is
// token pim(tb, 4g + i).
// Vn = T D (V - K S) for the chunk staged in `cb` (Kr, Vs, T, b); S is given as
// natural-order B fragments sb[kb] (k = key index) of this wave's 16 value
// columns.  Vn tile tb row 4g + i is token pim(tb, 4g + i).
template <int K, typename Buf>
__device__ __forceinline__ void chunk_vn(const Buf& cb, int w, const bf16x8* sb, floatx4* vn) {
    constexpr int LDK = ldb<K>(), LDV = ldb<VS>(), LDT = ldb<64>();
    const int l = mf::lane(), g = l >> 4, r = l & 15;
    floatx4 R[4];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
        const bf16x4 u = mf::tr_rows4(cb.Vs, LDV, 32 * (tb >> 1) + 4 * (tb & 1), 16 * w, 4);
        floatx4 acc = floatx4{(float)u[0], (float)u[1], (float)u[2], (float)u[3]};
        const int row = pim(tb, r);
#pragma unroll
        for (int kb = 0; kb < K / 32; ++kb)
            acc = mma(mf::frag_row(cb.Kr, LDK, row, 32 * kb), mf::neg(sb[kb]), acc);
        const floatx4 bb = *reinterpret_cast<const floatx4*>(cb.b + pim(tb, 4 * g));
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] *= bb[i];  // D R
        R[tb] = acc;
    }
    const bf16x8 dr0 = frag_from_c(R[0], R[1]), dr1 = frag_from_c(R[2], R[3]);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
        const int row = pim(tb, r);
        vn[tb] = mma(mf::frag_row(cb.T, LDT, row, 0), dr0, zero4());
        if (tb >= 2) vn[tb] = mma(mf::frag_row(cb.T, LDT, row, 32), dr1, vn[tb]);
    }
}

// Scan workgroups with copy waves: waves 0..3 compute (NT threads), waves
// 4..7 load the inputs of the next chunks into registers and write them to
// the chunk's LDS buffer while the compute waves work on the current one, so
// no compute wave waits for a load or spends time staging.  Both kinds pass
// the same barriers per chunk.  Two waves per SIMD: the kernel's registers
// stay at 256 per lane or fewer (launch bounds).  Copies straight into LDS
// (global_load_lds) by the copy waves measured slower than the register path.
constexpr int NTS = 2 * NT;
constexpr int NCW = NT / 64;  // copy waves

template <int K, int V>
__global__ void __launch_bounds__(NTS) scan_o_kernel(const bf16* __restrict__ q,
                                                     const bf16* __restrict__ k,
                                                     const bf16* __restrict__ v,
                                                     const bf16* __restrict__ Tc,
                                                     const float* __restrict__ bc, SeqInfo si,
                                                     int H, const float* __restrict__ S0,
                                                     float* __restrict__ ST,
                                                     bf16* __restrict__ o,
                                                     bf16* __restrict__ hist,
                                                     bf16* __restrict__ pout, TokLd ld) {
    constexpr int LDK = ldb<K>(), LDP = ldb<64>(), NVS = V / VS;
    __shared__ __attribute__((aligned(16))) ScanSmem<K> sm;
    const int w = mf::wave(), l = mf::lane(), g = l >> 4, r = l & 15;
    int bh, vsl;
    scan_map(blockIdx.x, si.N * H, NVS, bh, vsl);
    bh = scan_seq_head(si, bh, H);
    const int seq = bh / H, h = bh % H, v0 = vsl * VS;
    long sbos, slen;
    int slot0;
    seq_bounds(si, seq, sbos, slen, slot0);
    const int nch = (int)((slen + 63) / 64);
    if (w >= NCW) {
        // copy waves: three register sets, ra, rb and rc, each a chunk ahead
        // of the one before; chunk n + 1 is written to buf[(n + 1) & 1] during
        // chunk n, while the loads of chunks n + 2 and n + 3 are in flight
        const int ct = (int)threadIdx.x - NT;
        // chunk n's loads (clamped to the last chunk, so every iteration
        // issues the same loads and the staging's waits stay exact)
        auto load = [&](ChunkRegs<K, true, true>& R, int n) {
            n = min(n, nch - 1);
            const long bos = sbos + (long)n * 64;
            const int len = (int)min((long)64, slen - (long)n * 64);
            R.load(q, k, v, Tc, bc, bos, len, h, V, v0, (long)(slot0 + n) * H + h, ld.q, ld.k,
                   ld.v, ct);
        };
        ChunkRegs<K, true, true> ra, rb, rc;
        if (nch > 0) {
            load(ra, 0);
            ra.stage(sm.buf[0]);
            load(ra, 1);
            load(rb, 2);
            load(rc, 3);
        }
        for (int n = 0; n < nch; n += 3) {  // ra holds chunk n + 1, rb n + 2, rc n + 3
            __syncthreads();  // chunk n staged; everyone is done with chunk n - 1
            if (n + 1 < nch) ra.stage(sm.buf[(n + 1) & 1]);
            load(ra, n + 4);
            __syncthreads();  // the compute waves' P complete
            if (n + 1 >= nch) break;
            __syncthreads();  // chunk n + 1 staged
            if (n + 2 < nch) rb.stage(sm.buf[n & 1]);
            load(rb, n + 5);
            __syncthreads();
            if (n + 2 >= nch) break;
            __syncthreads();  // chunk n + 2 staged
            if (n + 3 < nch) rc.stage(sm.buf[(n + 1) & 1]);
            load(rc, n + 6);
            __syncthreads();
        }
        return;
    }
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
        // retire these loads here: left pending, their waits land inside the
        // chunk loop as vmcnt(0), which every chunk would then pay for the
        // previous chunk's stores
        mf::dma_wait();
    }
    for (int i = threadIdx.x; i < 64 * LDP; i += NT) sm.P[i] = (bf16)0.f;

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
        store_state_frag<K>(out_rsrc(hist ? hist + ((long)(slot0 + n) * H + h) * V * K : o,
                                     hist ? 2u * V * K : 0u),
                            sb, vcol);
        floatx4 vn[4];
        chunk_vn<K>(cb, w, sb, vn);
        __syncthreads();  // P complete
        {
            // hand P to the backward (packed lower tiles; slice 0 only)
            const int tr = threadIdx.x >> 2, J = threadIdx.x & 3;
            const bool put = pout && vsl == 0;
            tri_store_piece(out_rsrc(put ? pout + ((long)(slot0 + n) * H + h) * TRI_ELEMS : o,
                                     put ? 2u * TRI_ELEMS : 0u),
                            tr, J, *reinterpret_cast<const bf16x8*>(sm.P + tr * LDP + 16 * J),
                            *reinterpret_cast<const bf16x8*>(sm.P + tr * LDP + 16 * J + 8));
        }
        const bf16x8 vb0 = frag_from_c(vn[0], vn[1]), vb1 = frag_from_c(vn[2], vn[3]);
        // o^T = S^T Q^T + Vn^T P^T: tile tb holds (value 16w + 4g + i, token 16tb + r)
        // the chunk's output rows; lanes of rows past the sequence's end fall
        // outside the resource
        const __amdgpu_buffer_rsrc_t orr = out_rsrc(o + bos * H * V, 2u * (unsigned)len * H * V);
        const unsigned ocol = 2u * (unsigned)(h * V + v0 + 16 * w + 4 * g);
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            floatx4 acc = zero4();
#pragma unroll
            for (int kb = 0; kb < K / 32; ++kb)
                acc = mma(sb[kb], frag_nat(cb.Q, LDK, 16 * tb, 32 * kb), acc);
            acc = mma(vb0, frag_nat(sm.P, LDP, 16 * tb, 0), acc);
            if (tb >= 2) acc = mma(vb1, frag_nat(sm.P, LDP, 16 * tb, 32), acc);
            const int t = 16 * tb + r;
            bstore8(bf16x4{(bf16)acc[0], (bf16)acc[1], (bf16)acc[2], (bf16)acc[3]}, orr,
                    2u * (unsigned)(t * H * V) + ocol);
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
