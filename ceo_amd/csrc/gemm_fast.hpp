// Large-tile bf16 / fp16 GEMM for gfx950 (included by gemm.hip).
//
// D[m, n] = epilogue( sum_k opA(m, k) opB(k, n) ), fp32 accumulation, where
// each operand is a matrix whose element (line, k) -- line = m for A, n for
// B -- sits at base[line * ld + k] ("k-contiguous", KC) or base[k * ld + line]
// ("line-contiguous", LC).  The four combinations cover the forward product
// (A KC, B LC), dA = dC B^T (both KC) and dB = A^T dC (both LC).
//
// Workgroup tile 256 x 256 x 64.  The library launches eight waves (two per
// SIMD), each owning 128 x 64 of the output as 4 x 2 tiles of
// v_mfma_f32_32x32x16; the kernel also compiles for four waves of 128 x 128
// (4 x 4 tiles).
// The product is formed transposed, C^T = B^T A^T: B's fragments are the MFMA
// A operand (rows n) and A's the B operand (columns m), so each lane ends up
// holding 4 consecutive n of one output row m and writes 8-byte row pieces.
// Per k-iteration each operand tile (256 lines x 64 k, 32 KB) is copied
// straight from global memory into LDS (global_load_lds_dwordx4, 16 bytes per
// lane, no VGPR staging) one iteration ahead, double-buffered; all of an
// iteration's copies are issued at its start, and the MFMA operand fragments
// are double-buffered in registers with the LDS reads of k step ks + 1
// interleaved between the MFMAs of k step ks.  Both LDS
// layouts are XOR-swizzled in 16-byte chunks so the fragment reads are free
// of bank conflicts:
//   KC tile [line][k]  (128 B rows):  chunk c of line L at c ^ ((L >> 1) & 7)
//     read with one 16-byte ds_read per lane (lanes 0-15 = 16 lines, one chunk)
//   LC tile [k][line]  (512 B rows):  chunk c of row k at c ^ (4 (k & 3))
//     read with two ds_read_b64_tr_b16 per lane (4 k rows x 32 lines per half wave)
// A k-tail (K not a multiple of 64) runs one last iteration through registers
// with the missing k zeroed.  Rows and columns past M or N are clamped on load
// (they only reach outputs that are not stored).
#pragma once
#include "gelu.hpp"
#include "mfma.hpp"

namespace efla {
namespace gf {

using mf::bf16;
using mf::bf16x4;
using mf::bf16x8;
typedef _Float16 f16;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short short4v;
typedef __attribute__((address_space(3))) short4v lds_short4v;

constexpr int BM = 256, BN = 256, BK = 64, NT = 256;
constexpr int TILE_BYTES = 256 * 64 * 2;  // one operand tile

template <typename T>
__device__ __forceinline__ floatx16 mma32(bf16x8 a, bf16x8 b, floatx16 c) {
    if constexpr (__is_same(T, f16))
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                       __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// --- LDS addressing (bytes within one operand tile) ------------------------
__device__ __forceinline__ unsigned kc_off(int line, int chunk) {
    return (unsigned)(line * 128 + ((chunk ^ ((line >> 1) & 7)) << 4));
}
__device__ __forceinline__ unsigned lc_off(int krow, int line) {  // line = element column
    return (unsigned)(krow * 512 + (((line >> 3) ^ ((krow & 3) << 2)) << 4) + ((line & 7) << 1));
}

// One 32-line x 16-k MFMA operand (lane l: line l & 31, k = 8 (l >> 5) .. + 7)
// from a tile, k step ks (0..3), lines line0 .. line0 + 31.
template <bool KC>
__device__ __forceinline__ bf16x8 frag(const char* tile, int line0, int ks, int l) {
    if constexpr (KC) {
        return *reinterpret_cast<const bf16x8*>(tile + kc_off(line0 + (l & 31), 2 * ks + (l >> 5)));
    } else {
        // group G = l >> 4: lines line0 + 16 (G & 1) + j, k rows 16 ks + 8 (G >> 1) + 0..7;
        // lane 16G + 4a + b addresses k row (.. + a), lines (.. + 4b .. + 4b + 3)
        const int G = l >> 4, a = (l & 15) >> 2, b = l & 3;
        const int kr = 16 * ks + 8 * (G >> 1) + a;
        const int ln = line0 + 16 * (G & 1) + 4 * b;
        const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(tile + lc_off(kr, ln)));
        const short4v hi =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(tile + lc_off(kr + 4, ln)));
        const bf16x4 x = __builtin_bit_cast(bf16x4, lo), y = __builtin_bit_cast(bf16x4, hi);
        return bf16x8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
    }
}

// --- operand tile copies ----------------------------------------------------
// An operand: element (line, k) at base[line * ld + k] (KC) or base[k * ld + line].
struct Opnd {
    const char* base;  // bytes
    long ld;           // elements
    int nlines;        // M or N
};

// Direct copy of the tile (lines line0.., k k0..k0+63) into `tile` (LDS): 32
// instructions of 64 16-byte chunks, 8 per wave.  The global side is
// permuted so the LDS side lands swizzled.  Offsets are 32-bit from a per-tile
// scalar base (the host checks 256 * ld * 2 < 2^31).
// Instruction q (of the tile's 32) goes to wave q % NW; a call issues this
// wave's instructions numbered i0 .. i1 - 1 among its own.
template <bool KC, int NW>
__device__ __forceinline__ void copy_tile(const Opnd& op, int line0, long k0, char* tile, int w,
                                          int l, int i0 = 0, int i1 = 32 / NW) {
    const char* base = KC ? op.base + ((long)line0 * op.ld + k0) * 2
                          : op.base + (k0 * op.ld + line0) * 2;
#pragma unroll
    for (int i = i0; i < i1; ++i) {
        const int q = NW * i + w;
        const int P = 64 * q + l;  // physical 16-byte chunk of the tile
        unsigned off;
        if constexpr (KC) {
            const int line = P >> 3, c = (P & 7) ^ ((line >> 1) & 7);
            const int gl = min(line, op.nlines - 1 - line0);
            off = (unsigned)(gl * op.ld + 8 * c) * 2u;
        } else {
            const int kr = P >> 5, c = (P & 31) ^ ((kr & 3) << 2);
            const int gc = min(8 * c, op.nlines - 8 - line0);  // nlines % 8 == 0
            off = (unsigned)(kr * op.ld + gc) * 2u;
        }
        mf::dma16(base, off, tile + 1024 * q);
    }
}

// The k-tail tile through registers: k >= K reads as zero (K % 8 == 0).
template <bool KC, int NTH>
__device__ __forceinline__ void copy_tile_tail(const Opnd& op, int line0, long k0, long K,
                                               char* tile, int tid) {
#pragma unroll 4
    for (int i = 0; i < 2048 / NTH; ++i) {
        const int P = NTH * i + tid;
        bf16x8 x{};
        unsigned dst;
        if constexpr (KC) {
            const int line = P >> 3, c = P & 7;
            const int gl = min(line0 + line, op.nlines - 1);
            if (k0 + 8 * c < K)
                x = *reinterpret_cast<const bf16x8*>(op.base + ((long)gl * op.ld + k0 + 8 * c) * 2);
            dst = kc_off(line, c);
        } else {
            const int kr = P >> 5, c = P & 31;
            const int gc = min(line0 + 8 * c, op.nlines - 8);
            if (k0 + kr < K)
                x = *reinterpret_cast<const bf16x8*>(op.base + ((k0 + kr) * op.ld + gc) * 2);
            dst = (unsigned)(kr * 512 + ((c ^ ((kr & 3) << 2)) << 4));
        }
        *reinterpret_cast<bf16x8*>(tile + dst) = x;
    }
}

// --- epilogues ---------------------------------------------------------------
// Called once per 4 consecutive outputs D[m][n .. n+3] (n % 4 == 0, all inside
// the matrix) with their fp32 sums.
// PLAIN: alpha acc (+ bias); RESID: that + beta C; GELU_AUX: pre = acc (+ bias)
// and GELU(pre); DGELU: bf16(acc) GELU'(pre); PARTIAL: fp32 split-K partials.
enum EpiKind { EPI_PLAIN = 0, EPI_GELU_AUX = 1, EPI_DGELU = 2, EPI_PARTIAL = 3, EPI_RESID = 4 };

template <typename T>
struct EpiArgs {
    T* d;
    long ldd;
    const T* bias;  // [n] or NULL
    const T* c;     // residual, read when beta != 0
    long ldc;
    float alpha, beta;
    T* aux;  // GELU_AUX: pre-activation out; DGELU: pre-activation in
    long ldaux;
    float* part;   // PARTIAL: fp32 partial sums [split][M][N]
    float* cpart;  // DGELU: column sums of the output, one fp32 row per 128 output
                   // rows ([M / 128][N]), or NULL
};

template <typename T>
__device__ __forceinline__ void load4(const T* p, float* v) {
    typedef __attribute__((__vector_size__(4 * sizeof(T)))) T t4;
    const t4 x = *reinterpret_cast<const t4*>(p);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = (float)x[e];
}
template <typename T>
__device__ __forceinline__ void store4(T* p, const float* v) {
    typedef __attribute__((__vector_size__(4 * sizeof(T)))) T t4;
    *reinterpret_cast<t4*>(p) = t4{(T)v[0], (T)v[1], (T)v[2], (T)v[3]};
}

template <typename T, int EPI>
__device__ __forceinline__ void epilogue4(const EpiArgs<T>& ea, long m, long n, const float* acc) {
    if constexpr (EPI == EPI_PARTIAL) return;  // handled by the kernel
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = ea.alpha * acc[e];
    if (ea.bias) {
        float b[4];
        load4(ea.bias + n, b);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += b[e];
    }
    if constexpr (EPI == EPI_GELU_AUX) {
        store4(ea.aux + m * ea.ldaux + n, v);  // pre-activation for the backward
        float r[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = gelu::gelu_f<true>((float)(T)v[e]);
        store4(ea.d + m * ea.ldd + n, r);
        return;
    }
    if constexpr (EPI == EPI_DGELU) {
        float u[4];
        load4(ea.aux + m * ea.ldaux + n, u);
        float r[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = (float)(T)v[e] * gelu::gelu_df<true>(u[e]);
        store4(ea.d + m * ea.ldd + n, r);
        return;
    }
    if (ea.beta != 0.f) {
        float c[4];
        load4(ea.c + m * ea.ldc + n, c);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += ea.beta * c[e];
    }
    store4(ea.d + m * ea.ldd + n, v);
}

// --- epilogue staged through LDS ---------------------------------------------
// Each wave finishes its own 128 x (32 TNI) block of the output through a
// private slice of the free LDS buffer (32 rows x 32 TNI columns of fp32,
// 4 KB TNI), one 32-row m tile at a time: it writes alpha acc there in the
// MFMA layout, reads it back as 8-element row pieces and finishes the
// epilogue on them -- bias, residual, GELU and its derivative, with the
// residual and pre-activation read, and the outputs written, as whole
// 16-byte (32-byte for fp32 partials) pieces, eight or more lanes to a row
// (an MFMA result tile instead holds 8-byte pieces of 32 rows per store
// instruction).  No workgroup barrier is needed until the buffer is handed
// back.  Slice layout [32][32 TNI] fp32, 16-byte chunk c of row r at
// c ^ (r & 15): conflict-free for the MFMA-layout writes (32 rows, one chunk)
// and the row-wise reads.
template <int TNI>
__device__ __forceinline__ unsigned ep_off(int row, int col) {  // col % 4 == 0
    return (unsigned)(row * (128 * TNI) + (((col >> 2) ^ (row & 15)) << 4));
}

template <typename T, int EPI, int TNI, bool AHEAD>
__device__ __forceinline__ void epilogue_wave(const EpiArgs<T>& ea, const floatx16 (&acc)[TNI][4],
                                              int split, long mw, long nw, long M, long N, int l,
                                              char* wp) {
    constexpr int WC = 32 * TNI;  // columns of the wave's block
    constexpr int NP = WC / 16;   // 8-element pieces per lane and 32-row pass
    typedef __attribute__((__vector_size__(8 * sizeof(T)))) T t8;
    // DGELU with column sums: this lane's 8 columns (piece c8 = l % (WC / 8)
    // of every row it finishes) summed over its rows
    float csum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    // A lane's pieces keep their columns from pass to pass (piece s: row
    // (64 s + l) / (WC / 8) of the pass, columns 8 ((64 s + l) % (WC / 8))).
    // The pre-activation (DGELU) or residual (RESID) pieces are read ahead of
    // their use: with AHEAD those of pass j + 1 while pass j is finished, once
    // pass j's accumulators are in LDS (their registers are free by then);
    // otherwise (the kernels whose main loop leaves too few registers) those
    // of pass j, as soon as its accumulators are in LDS.
    constexpr bool IN = EPI == EPI_DGELU || EPI == EPI_RESID;
    const bool rd = IN && (EPI == EPI_DGELU || ea.beta != 0.f);
    const T* src = EPI == EPI_DGELU ? ea.aux : ea.c;
    const long lds = EPI == EPI_DGELU ? ea.ldaux : ea.ldc;
    auto piece = [&](int s, int& row, long& n) {
        const int p = 64 * s + l;
        row = p / (WC / 8);
        n = nw + 8 * (p % (WC / 8));
    };
    auto fetch = [&](int j, t8 (&dst)[NP]) {
#pragma unroll
        for (int s = 0; s < NP; ++s) {
            int row;
            long n;
            piece(s, row, n);
            const long m = mw + 32 * j + row;
            dst[s] = (m < M && n < N) ? *reinterpret_cast<const t8*>(src + m * lds + n) : t8{};
        }
    };
    t8 inp[2][NP];
    if (AHEAD && rd && mw < M) fetch(0, inp[0]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const long r0 = mw + 32 * j;
        if (r0 >= M) break;  // uniform over the wave
#pragma unroll
        for (int i = 0; i < TNI; ++i)
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const int col = 32 * i + 8 * qd + 4 * (l >> 5);
                mf::floatx4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    v[e] = (EPI == EPI_PARTIAL ? 1.f : ea.alpha) * acc[i][j][4 * qd + e];
                *reinterpret_cast<mf::floatx4*>(wp + ep_off<TNI>(l & 31, col)) = v;
            }
        if (AHEAD && rd && j + 1 < 4 && r0 + 32 < M) fetch(j + 1, inp[(j + 1) & 1]);
        if (!AHEAD && rd) fetch(j, inp[j & 1]);
#pragma unroll
        for (int s = 0; s < NP; ++s) {
            int row;
            long n;
            piece(s, row, n);
            const int c8 = (int)(n - nw) / 8;
            const long m = r0 + row;
            const mf::floatx4 v0 =
                *reinterpret_cast<const mf::floatx4*>(wp + ep_off<TNI>(row, 8 * c8));
            const mf::floatx4 v1 =
                *reinterpret_cast<const mf::floatx4*>(wp + ep_off<TNI>(row, 8 * c8 + 4));
            if (m >= M || n >= N) continue;
            if constexpr (EPI == EPI_PARTIAL) {
                float* dst = ea.part + ((long)split * M + m) * N + n;
                *reinterpret_cast<mf::floatx4*>(dst) = v0;
                *reinterpret_cast<mf::floatx4*>(dst + 4) = v1;
                continue;
            }
            float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
            if (ea.bias) {
                const t8 bb = *reinterpret_cast<const t8*>(ea.bias + n);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] += (float)bb[e];
            }
            t8 y;
            if constexpr (EPI == EPI_GELU_AUX) {
                t8 pre;
#pragma unroll
                for (int e = 0; e < 8; ++e) pre[e] = (T)v[e];
                *reinterpret_cast<t8*>(ea.aux + m * ea.ldaux + n) = pre;
#pragma unroll
                for (int e = 0; e < 8; ++e) y[e] = (T)gelu::gelu_f<true>((float)pre[e]);
            } else if constexpr (EPI == EPI_DGELU) {
                const t8 u = inp[j & 1][s];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    y[e] = (T)((float)(T)v[e] * gelu::gelu_df<true>((float)u[e]));
                    csum[e] += (float)y[e];
                }
            } else if constexpr (EPI == EPI_RESID) {
                if (rd) {
                    const t8 cc = inp[j & 1][s];
#pragma unroll
                    for (int e = 0; e < 8; ++e) y[e] = (T)(v[e] + ea.beta * (float)cc[e]);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) y[e] = (T)v[e];
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) y[e] = (T)v[e];
            }
            *reinterpret_cast<t8*>(ea.d + m * ea.ldd + n) = y;
        }
    }
    if constexpr (EPI == EPI_DGELU) {
        if (ea.cpart && mw < M) {
            // the lanes sharing a piece index hold different rows: sum them
            // (fixed order), then one fp32 row of the wave's 128 rows
#pragma unroll
            for (int e = 0; e < 8; ++e)
#pragma unroll
                for (int off = WC / 8; off < 64; off <<= 1) csum[e] += __shfl_xor(csum[e], off);
            const long n = nw + 8 * l;
            if (l < WC / 8 && n < N) {
                float* dst = ea.cpart + (mw / 128) * N + n;
                *reinterpret_cast<mf::floatx4*>(dst) = mf::floatx4{csum[0], csum[1], csum[2], csum[3]};
                *reinterpret_cast<mf::floatx4*>(dst + 4) =
                    mf::floatx4{csum[4], csum[5], csum[6], csum[7]};
            }
        }
    }
}

// --- the kernel --------------------------------------------------------------
// NW waves: 2 along m, NW / 2 along n; a wave owns 128 (m) x 512 / NW (n) of
// the output (4 x 4 tiles of 32 x 32 for NW = 4, 4 x 2 for NW = 8, which puts
// two waves on each SIMD).
//
// Persistent: workgroup b takes work items b, b + gridDim.x, ... (an item is
// an output tile, or a (tile, k-split) pair with ksplit > 1).  The LDS double
// buffer runs across items: the last k-iteration of an item copies the next
// item's first k-block, so an item starts with its first block in place and
// the previous item's epilogue stores drain behind the next main loop.
//
// ksplit > 1 (EPI_PARTIAL): the contraction is cut into ksplit ranges of
// kper (a multiple of 64) and item (tile, split) writes its fp32 partial tile
// to ea.part; gemm_splitk_reduce adds them up in split order.
struct Item {
    int m0, n0, split;
    long kbeg, klen;
};

template <typename T, bool AKC, bool BKC, int EPI, int NW>
__global__ void __launch_bounds__(64 * NW) gemm_fast_kernel(Opnd A, Opnd B, long M, long N,
                                                            long K, EpiArgs<T> ea, int ksplit,
                                                            long kper) {
    constexpr int NTH = 64 * NW;
    constexpr int TNI = 8 / NW * 2;  // 32-wide n tiles per wave: 4 (NW = 4) or 2 (NW = 8)
    // two buffers of [A tile | B tile]; the epilogue stages the output through
    // the one the next item's first k-block is not in
    __shared__ __attribute__((aligned(1024))) char smem[4 * TILE_BYTES];
    const long tm_n = (M + BM - 1) / BM, tn_n = (N + BN - 1) / BN;
    const long ntiles = tm_n * tn_n;
    const long nitems = ntiles * ksplit;
    // item -> tile: XCD-banded (the items of workgroup b, all on one XCD, form
    // a contiguous band), then groups of 8 tile rows so an XCD re-reads a band
    // of A and of B
    auto decode = [&](long it, Item& I) {
        long id = it;
        if (nitems % 8 == 0) id = (id % 8) * (nitems / 8) + id / 8;
        I.split = (int)(id % ksplit);
        const long pid = id / ksplit;
        constexpr long GROUP = 8;
        const long group_span = GROUP * tn_n;
        const long gi = pid / group_span;
        const long first_m = gi * GROUP;
        const long gsize = (tm_n - first_m) < GROUP ? (tm_n - first_m) : GROUP;
        I.m0 = (int)((first_m + (pid % group_span) % gsize) * BM);
        I.n0 = (int)(((pid % group_span) / gsize) * BN);
        I.kbeg = (long)I.split * kper;
        I.klen = (K - I.kbeg) < kper ? (K - I.kbeg) : kper;
    };

    const int w = mf::wave(), l = mf::lane();
    const int wm = (w & 1) * 128, wn = (w >> 1) * (32 * TNI);  // this wave's block
    // buffer b: A at smem + 2b * TILE_BYTES, B right after it
    auto As = [&](int b) { return smem + 2 * b * TILE_BYTES; };
    auto Bs = [&](int b) { return smem + (2 * b + 1) * TILE_BYTES; };

    long it = blockIdx.x;
    if (it >= nitems) return;  // uniform over the workgroup
    Item cur;
    decode(it, cur);
    // the first item's first k-block
    if (cur.klen >= BK) {
        copy_tile<AKC, NW>(A, cur.m0, cur.kbeg, As(0), w, l);
        copy_tile<BKC, NW>(B, cur.n0, cur.kbeg, Bs(0), w, l);
    } else {
        copy_tile_tail<AKC, NTH>(A, cur.m0, cur.kbeg, K, As(0), threadIdx.x);
        copy_tile_tail<BKC, NTH>(B, cur.n0, cur.kbeg, K, Bs(0), threadIdx.x);
    }
    mf::dma_wait();
    __syncthreads();
    int buf = 0;
    for (;;) {
        const long nitn = it + gridDim.x;
        const bool more = nitn < nitems;
        Item nxt = cur;
        if (more) decode(nitn, nxt);
        floatx16 acc[TNI][4];  // [n tile][m tile]
#pragma unroll
        for (int i = 0; i < TNI; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
        const long nfull = cur.klen / BK;  // whole k-iterations (direct copies)
        const long niter = (cur.klen + BK - 1) / BK;
        // on an edge tile a wave whose rows are all past M, or columns all
        // past N, holds no output: it only copies (the N = 3088 projection's
        // last tile column is 16 wide and 6 of its 8 waves sit idle)
        const bool act = cur.m0 + wm < M && cur.n0 + wn < N;
        for (long kt = 0; kt < niter; ++kt) {
            // what the other buffer receives: this item's next k-block, or
            // the next item's first; whole blocks by direct copies, a k-tail
            // block through registers
            const bool own = kt + 1 < niter;
            const bool fetch = own || more;
            const Item& src = own ? cur : nxt;
            const long k0 = own ? cur.kbeg + (kt + 1) * BK : nxt.kbeg;
            const bool direct = own ? kt + 1 < nfull : nxt.klen >= BK;
            if (fetch && !direct) {
                copy_tile_tail<AKC, NTH>(A, src.m0, k0, K, As(buf ^ 1), threadIdx.x);
                copy_tile_tail<BKC, NTH>(B, src.n0, k0, K, Bs(buf ^ 1), threadIdx.x);
            }
            const char* at = As(buf);
            const char* bt = Bs(buf);
            // fragments double-buffered in registers: k step ks + 1 is read
            // while the MFMAs of k step ks run
            bf16x8 fb[2][TNI], fa[2][4];
            // the iteration's reads, copies and MFMAs issue at raised wave
            // priority, the wait for the next block at the normal one: a wave
            // still computing wins the SIMD's issue slots over its partner
            // that has reached the end of the iteration (-1 to -4 % on the
            // config-4 products, measured)
            __builtin_amdgcn_s_setprio(1);
            if (act) {
#pragma unroll
                for (int i = 0; i < TNI; ++i) fb[0][i] = frag<BKC>(bt, wn + 32 * i, 0, l);
#pragma unroll
                for (int j = 0; j < 4; ++j) fa[0][j] = frag<AKC>(at, wm + 32 * j, 0, l);
            }
            // the next block's copies all go out now, a whole iteration ahead
            // of the wait (the buffer they fill was last read in the previous
            // iteration, which every wave has finished)
            if (fetch && direct) {
                copy_tile<AKC, NW>(A, src.m0, k0, As(buf ^ 1), w, l);
                copy_tile<BKC, NW>(B, src.n0, k0, Bs(buf ^ 1), w, l);
            }
            if (act) {
#pragma unroll
                for (int ks = 0; ks < BK / 16; ++ks) {
                    const int c = ks & 1;
                    if (ks + 1 < BK / 16) {
#pragma unroll
                        for (int i = 0; i < TNI; ++i)
                            fb[c ^ 1][i] = frag<BKC>(bt, wn + 32 * i, ks + 1, l);
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            fa[c ^ 1][j] = frag<AKC>(at, wm + 32 * j, ks + 1, l);
                    }
#pragma unroll
                    for (int i = 0; i < TNI; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            acc[i][j] = mma32<T>(fb[c][i], fa[c][j], acc[i][j]);
                    if (ks + 1 < BK / 16) {
                        // one LDS read between consecutive MFMAs
                        constexpr int NR = TNI * (BKC ? 1 : 2) + 4 * (AKC ? 1 : 2);
                        constexpr int NM = 4 * TNI;
                        constexpr int R = NR < NM ? NR : NM;
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                        }
                        if constexpr (NM > R) __builtin_amdgcn_sched_group_barrier(0x008, NM - R, 0);
                        if constexpr (NR > R) __builtin_amdgcn_sched_group_barrier(0x100, NR - R, 0);
                    }
                }
            }
            __builtin_amdgcn_s_setprio(0);
            mf::dma_wait();
            __syncthreads();
            buf ^= 1;
        }
        // lane l holds, for tile (i, j), output row m = m0 + wm + 32 j + (l & 31)
        // and columns n = n0 + wn + 32 i + 8 q + 4 (l >> 5) + e in acc[i][j][4 q + e].
        // The lane index is re-derived per item (mf::tid_in): the epilogue's
        // lane-dependent addresses are then not hoisted out of the item loop,
        // where they would stay live across the main loop.
        {
            const int le = mf::tid_in((int)it) & 63;
            char* wp = smem + 2 * (buf ^ 1) * TILE_BYTES + (4096 * TNI) * w;
            epilogue_wave<T, EPI, TNI, AKC && BKC>(ea, acc, cur.split, (long)cur.m0 + wm,
                                                    (long)cur.n0 + wn, M, N, le, wp);
        }
        __syncthreads();  // the next item's first copies refill the buffer
        if (!more) break;
        it = nitn;
        cur = nxt;
    }
}

// D = epilogue(sum over splits of the fp32 partials), 4 outputs per thread,
// the splits added in order (so the result does not depend on scheduling).
template <typename T>
__global__ void __launch_bounds__(256) gemm_splitk_reduce(EpiArgs<T> ea, long M, long N,
                                                          int ksplit) {
    const long nq = N / 4, total = M * nq;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
        const long m = i / nq, n = 4 * (i - m * nq);
        mf::floatx4 s = *reinterpret_cast<const mf::floatx4*>(ea.part + m * N + n);
        for (int k = 1; k < ksplit; ++k)
            s += *reinterpret_cast<const mf::floatx4*>(ea.part + ((long)k * M + m) * N + n);
        const float v[4] = {s[0], s[1], s[2], s[3]};
        epilogue4<T, EPI_PLAIN>(ea, m, n, v);
    }
}

}  // namespace gf
}  // namespace efla
