// bf16 MFMA building blocks for gfx950 (v_mfma_f32_16x16x32_bf16, wave64).
//
// Lane layouts of one 16x16x32 instruction (g = lane >> 4, r = lane & 15):
//   A (16 x 32):  lane holds row r, 8 k values in slots s = 0..7
//   B (32 x 16):  lane holds col r, 8 k values in slots s = 0..7
//   C (16 x 16):  lane holds col r, rows 4g + i (i = 0..3) as a floatx4
// The instruction sums over the slots, so any bijection (g, s) -> k works as
// long as A and B use the same one.  Two orders are used here:
//   natural : k = 8g + s                      (one 16-byte read per lane)
//   c-order : k = 4g + s        for s < 4,
//             k = 16 + 4g + s-4 for s >= 4    (two 8-byte reads per lane)
// The c-order is what a lane already holds when the k range is the rows of
// two stacked C tiles (rows 0..15 and 16..31): a product whose contraction
// runs over the rows of an earlier result then takes that result straight from
// registers (frag_from_c) and reads only its other operand from memory.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace efla {
namespace mf {

typedef __bf16 bf16;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4;
typedef __attribute__((__vector_size__(16))) int int4v;
typedef __attribute__((__vector_size__(8))) int int2v;

__device__ __forceinline__ int lane() { return threadIdx.x & 63; }
// threadIdx.x as a value that depends on `epoch` (an empty asm ties them): in a
// loop, lane-dependent address arithmetic derived from it is recomputed each
// iteration instead of being hoisted out of the loop and held live across it.
// The asm has no side effects, so repeated uses within an iteration still merge.
__device__ __forceinline__ int tid_in(int epoch) {
    int x = (int)threadIdx.x;
    asm("" : "+v"(x) : "s"(epoch));
    return x;
}
// wave index as a scalar (wave-uniform branches and addresses stay in SGPRs)
__device__ __forceinline__ int wave() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ __forceinline__ floatx4 zero4() { return floatx4{0.f, 0.f, 0.f, 0.f}; }

__device__ __forceinline__ floatx4 mma(bf16x8 a, bf16x8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// fp32 16x16x4: A lane (row r, k = g), B lane (col r, k = g), C as above.
__device__ __forceinline__ floatx4 mma_f32(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Operand fragment from a [line][k] bf16 array (line = A row or B column),
// natural k order, lines line0 .. line0+15, k range k0 .. k0+31.
__device__ __forceinline__ bf16x8 frag_nat(int l, const bf16* base, int ld, int line0, int k0) {
    return *reinterpret_cast<const bf16x8*>(base + (line0 + (l & 15)) * ld + k0 + 8 * (l >> 4));
}
__device__ __forceinline__ bf16x8 frag_nat(const bf16* base, int ld, int line0, int k0) {
    return frag_nat(lane(), base, ld, line0, k0);
}

// Same, c-order.
__device__ __forceinline__ bf16x8 frag_cc(const bf16* base, int ld, int line0, int k0) {
    const int l = lane();
    const bf16* p = base + (line0 + (l & 15)) * ld + k0 + 4 * (l >> 4);
    const bf16x4 lo = *reinterpret_cast<const bf16x4*>(p);
    const bf16x4 hi = *reinterpret_cast<const bf16x4*>(p + 16);
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// c-order fragment from two C tiles held in registers (rows 0..15 -> c0,
// rows 16..31 -> c1 of the k range), optionally negated.
__device__ __forceinline__ bf16x8 frag_from_c(floatx4 c0, floatx4 c1) {
    return bf16x8{(bf16)c0[0], (bf16)c0[1], (bf16)c0[2], (bf16)c0[3],
                  (bf16)c1[0], (bf16)c1[1], (bf16)c1[2], (bf16)c1[3]};
}

__device__ __forceinline__ bf16x8 neg(bf16x8 x) {
    int4v v = __builtin_bit_cast(int4v, x);
    v ^= int4v{(int)0x80008000, (int)0x80008000, (int)0x80008000, (int)0x80008000};
    return __builtin_bit_cast(bf16x8, v);
}

// Load a C-layout tile (rows row0 + 4g + i, column col0 + r) of a [row][col]
// bf16 array stored transposed as [col][row] (one 8-byte read per lane).
__device__ __forceinline__ floatx4 load_c_t(const bf16* baseT, int ldt, int row0, int col0) {
    const int l = lane();
    const bf16x4 x =
        *reinterpret_cast<const bf16x4*>(baseT + (col0 + (l & 15)) * ldt + row0 + 4 * (l >> 4));
    return floatx4{(float)x[0], (float)x[1], (float)x[2], (float)x[3]};
}

// Store a C tile as bf16 into a [row][col] array (4 two-byte stores).
__device__ __forceinline__ void store_c(bf16* base, int ld, int row0, int col0, floatx4 c) {
    const int l = lane();
    bf16* p = base + (row0 + 4 * (l >> 4)) * ld + col0 + (l & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i * ld] = (bf16)c[i];
}

// Store a C tile as bf16 into its transposed [col][row] array (one 8-byte store).
__device__ __forceinline__ void store_c_t(bf16* baseT, int ldt, int row0, int col0, floatx4 c) {
    const int l = lane();
    *reinterpret_cast<bf16x4*>(baseT + (col0 + (l & 15)) * ldt + row0 + 4 * (l >> 4)) =
        bf16x4{(bf16)c[0], (bf16)c[1], (bf16)c[2], (bf16)c[3]};
}

// ---------------------------------------------------------------------------
// Transposing LDS reads (ds_read_b64_tr_b16).  Within each group of 16 lanes,
// lane 16g + 4a + b supplies the address of 4 consecutive bf16 (8 bytes); the
// instruction returns to lane 16g + j the j & 3'th element of the addresses of
// lanes 16g + 4i + (j >> 2), i = 0..3.  With lane 16g + 4a + b pointing at
// row (r0 + a), column (c0 + b * cs), lane 16g + j receives rows r0 .. r0+3
// of column c0 + (j >> 2) * cs + (j & 3): a column slice of a row-major tile.
// (Layout checked on gfx950 with an in-bounds probe.)
// ---------------------------------------------------------------------------
typedef short short4v __attribute__((__vector_size__(8)));
typedef __attribute__((address_space(3))) short4v lds_short4v;

__device__ __forceinline__ bf16x4 ds_tr16(const bf16* p) {
    const short4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)p);
    return __builtin_bit_cast(bf16x4, v);
}

// Lane (g, j) gets rows k0 + 8g + i (i = 0..3) of column
// c0 + (j >> 2) * cs + (j & 3) of a row-major tile with row stride ld.
__device__ __forceinline__ bf16x4 tr_rows4(int l, const bf16* base, int ld, int k0, int c0, int cs) {
    const int g = l >> 4, a = (l & 15) >> 2, b = l & 3;
    return ds_tr16(base + (k0 + 8 * g + a) * ld + c0 + b * cs);
}
__device__ __forceinline__ bf16x4 tr_rows4(const bf16* base, int ld, int k0, int c0, int cs) {
    return tr_rows4(lane(), base, ld, k0, c0, cs);
}

// Operand fragment whose k runs along the ROWS of a row-major [k][line] tile:
// lane (g, j) gets line c0 + (j >> 2) * cs + (j & 3), k = k0 + 8g + s
// (natural order).  cs = 4 gives lines c0 .. c0+15 in order.
__device__ __forceinline__ bf16x8 frag_tr(int l, const bf16* base, int ld, int k0, int c0,
                                         int cs = 4) {
    const bf16x4 lo = tr_rows4(l, base, ld, k0, c0, cs);
    const bf16x4 hi = tr_rows4(l, base, ld, k0 + 4, c0, cs);
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
__device__ __forceinline__ bf16x8 frag_tr(const bf16* base, int ld, int k0, int c0, int cs = 4) {
    return frag_tr(lane(), base, ld, k0, c0, cs);
}

// frag_tr with the k rows in c-order: lane (g, j) gets k = k0 + 4g + i in
// slots 0-3 and k0 + 16 + 4g + i in slots 4-7 (as frag_cc / frag_from_c).  It
// pairs only with another c-order operand of the same k range, typically a
// second frag_trc.  Measured on gfx950 with SQ_LDS_BANK_CONFLICT: its two
// transposing reads take 2 LDS cycles each, against 4 for frag_tr, whose rows
// r and r + 8 fall in the same banks for every row stride that keeps 16-byte
// alignment.
__device__ __forceinline__ bf16x8 frag_trc(int l, const bf16* base, int ld, int k0, int c0,
                                          int cs = 4) {
    const int g = l >> 4, a = (l & 15) >> 2, b = l & 3;
    const bf16x4 lo = ds_tr16(base + (k0 + 4 * g + a) * ld + c0 + b * cs);
    const bf16x4 hi = ds_tr16(base + (k0 + 16 + 4 * g + a) * ld + c0 + b * cs);
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
__device__ __forceinline__ bf16x8 frag_trc(const bf16* base, int ld, int k0, int c0, int cs = 4) {
    return frag_trc(lane(), base, ld, k0, c0, cs);
}

// frag_nat with an explicit row for this lane (row permutations).
__device__ __forceinline__ bf16x8 frag_row(int l, const bf16* base, int ld, int row, int k0) {
    return *reinterpret_cast<const bf16x8*>(base + row * ld + k0 + 8 * (l >> 4));
}
__device__ __forceinline__ bf16x8 frag_row(const bf16* base, int ld, int row, int k0) {
    return frag_row(lane(), base, ld, row, k0);
}

// Natural-order fragment from two C tiles: lanes of group g hold rows 4g..4g+3
// of each tile; the caller's row numbering makes tile h row 4g+i stand for
// k = 8g + 4h + i (see the row maps in the kernels).
__device__ __forceinline__ bf16x8 frag_c2(floatx4 c0, floatx4 c1) { return frag_from_c(c0, c1); }

// ---------------------------------------------------------------------------
// Cooperative tile loads (all NT threads).  A tile is ROWS token rows of D
// bf16 values; source row t starts at src + t * ld (elements); rows >= valid
// read as zero.  Each thread owns 16-byte column group fg = tid % (D/8) of
// TPT = ROWS*D/(8*NT) consecutive rows, so a row is read by D/8 adjacent lanes.
// ---------------------------------------------------------------------------
template <int ROWS, int D, int NT>
struct TileRegs {
    static constexpr int FG = D / 8;
    static constexpr int TPT = ROWS * FG / NT;
    static_assert(TPT >= 1 && ROWS * FG == TPT * NT, "tile does not split evenly");
    bf16x8 x[TPT];
    int valid;
    int tid;  // this thread's index in the workgroup (set by load)

    __device__ __forceinline__ int fg() const { return tid % FG; }
    __device__ __forceinline__ int t0() const { return (tid / FG) * TPT; }

    // valid >= 1.  Rows past `valid` re-read the last valid row, so every load
    // is issued unconditionally and stays in bounds; they are zeroed by
    // mask(), which the store functions call.  Nothing here consumes the loaded
    // registers, so the loads stay in flight until the tile is stored (a
    // prefetch overlaps whatever runs in between).
    // `src` is uniform across the workgroup and ROWS * ld * 2 < 2^32 (the
    // host validates H * max(d_k, d_v) < 2^24), so each row is a 32-bit byte
    // offset from a scalar base (global_load ... v_off, s_base).
    __device__ __forceinline__ void load(const bf16* __restrict__ src, long ld, int nvalid,
                                         int thread = (int)threadIdx.x) {
        tid = thread;
        const int f = fg(), t = t0();
        valid = nvalid;
        const char* base = reinterpret_cast<const char*>(src);
#pragma unroll
        for (int j = 0; j < TPT; ++j) {
            const int tt = min(t + j, nvalid - 1);
            const unsigned off = (unsigned)(tt * (int)ld + 8 * f) * 2u;
            x[j] = *reinterpret_cast<const bf16x8*>(base + off);
        }
    }
    __device__ __forceinline__ void mask() {
        if (__builtin_amdgcn_readfirstlane(valid) >= ROWS) return;  // full tile
        const int t = t0();
#pragma unroll
        for (int j = 0; j < TPT; ++j)
            if (t + j >= valid) x[j] = bf16x8{};
    }
    // row-major [t][d] copy, row stride ldr
    __device__ __forceinline__ void store_rows(bf16* dst, int ldr) {
        mask();
        const int f = fg(), t = t0();
#pragma unroll
        for (int j = 0; j < TPT; ++j) *reinterpret_cast<bf16x8*>(dst + (t + j) * ldr + 8 * f) = x[j];
    }
    // row-major copy into column halves of 64: element (t, c) at
    // dst + (c / 64) * half + t * ldr + c % 64
    __device__ __forceinline__ void store_rows_split(bf16* dst, int ldr, int half) {
        mask();
        const int f = fg(), t = t0();
#pragma unroll
        for (int j = 0; j < TPT; ++j)
            *reinterpret_cast<bf16x8*>(dst + (8 * f >> 6) * half + (t + j) * ldr + (8 * f & 63)) = x[j];
    }
    // transposed [d][t] copy, row stride ldt (TPT consecutive tokens per write)
    __device__ __forceinline__ void store_cols(bf16* dst, int ldt) {
        mask();
        const int f = fg(), t = t0();
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            bf16* p = dst + (8 * f + i) * ldt + t;
            if constexpr (TPT == 8) {
                *reinterpret_cast<bf16x8*>(p) = bf16x8{x[0][i], x[1][i], x[2][i], x[3][i],
                                                       x[4][i], x[5][i], x[6][i], x[7][i]};
            } else if constexpr (TPT == 4) {
                *reinterpret_cast<bf16x4*>(p) = bf16x4{x[0][i], x[1][i], x[2][i], x[3][i]};
            } else if constexpr (TPT == 2) {
                typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
                *reinterpret_cast<bf16x2*>(p) = bf16x2{x[0][i], x[1][i]};
            } else {
#pragma unroll
                for (int j = 0; j < TPT; ++j) p[j] = x[j][i];
            }
        }
    }
    // sum of squares of the row values this thread holds, reduced over the
    // FG lanes that share a row: every lane gets the sum for row t0() + j
    __device__ __forceinline__ float row_sumsq(int j) {
        mask();
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) s += (float)x[j][i] * (float)x[j][i];
#pragma unroll
        for (int off = 1; off < FG; off <<= 1) s += __shfl_xor(s, off);
        return s;
    }
};

// Cooperative store of a [ROWS][D] bf16 LDS tile (row stride lds) to global
// rows (stride ld) with 16-byte vectors; rows >= valid are skipped.
template <int ROWS, int D, int NT>
__device__ __forceinline__ void store_tile(bf16* __restrict__ dst, long ld, const bf16* src,
                                           int lds, int valid) {
    constexpr int FG = D / 8;
    for (int i = threadIdx.x; i < ROWS * FG; i += NT) {
        const int t = i / FG, f = i % FG;
        if (t < valid)
            *reinterpret_cast<int4v*>(dst + (long)t * ld + 8 * f) =
                *reinterpret_cast<const int4v*>(src + t * lds + 8 * f);
    }
}

// --- direct global -> LDS copies ---------------------------------------------
// global_load_lds_dwordx4: lane i of the wave writes 16 bytes at LDS address
// m0 + 16 i, without staging through VGPRs.  It is issued from inline asm so
// the compiler does not make later, unrelated LDS reads wait for it (the
// builtin form makes every following ds_read wait for vmcnt(0)); the caller
// runs dma_wait() and a workgroup barrier before anyone reads the destination,
// and keeps the destination unread and unwritten while the copy is in flight.
// The compiler inserts no hazard wait states in front of inline asm, so the asm
// starts with its own: gfx9 needs 5 after a VALU write of an SGPR the VMEM
// instruction reads (the base, when it was made uniform by v_readfirstlane)
// and 1 after the write of m0.
__device__ __forceinline__ void dma16(const void* base, unsigned off, const void* lds) {
    const unsigned m0 =
        (unsigned)(uintptr_t)(__attribute__((address_space(3))) const void*)lds;
    asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(m0)
                 : "memory");
}
// this wave's vector memory operations (loads, stores and LDS copies) done
__device__ __forceinline__ void dma_wait() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// ROWS x D bf16 tile from global rows of stride ld (elements) into LDS rows of
// stride LDR > D: one wave instruction fills 64 consecutive 16-byte LDS
// chunks, so a row's pad chunks are copied too (they re-read the row's first
// 16 bytes and are never read back).  The NW waves of the workgroup take the
// instructions in turn, starting with wave `rot % NW`; l is the lane.  Rows past `nvalid`
// re-read the last valid row, so every access stays inside the source rows;
// the caller zeroes those rows where they matter.  `src` is uniform and
// ROWS * ld * 2 < 2^32 (as for TileRegs), so offsets are 32-bit.
template <int ROWS, int D, int LDR, int NW>
__device__ __forceinline__ void dma_tile(bf16* lds, const bf16* src, long ld, int nvalid, int rot,
                                         int l) {
    constexpr int CPR = LDR / 8, NI = ROWS * CPR / 64;
    static_assert(LDR % 8 == 0 && LDR > D && D % 8 == 0 && (ROWS * CPR) % 64 == 0,
                  "tile does not split into 64-chunk instructions");
    const int w = wave();
    for (int i = (w + NW - rot % NW) % NW; i < NI; i += NW) {
        const int c = 64 * i + l, row = c / CPR, col = c - row * CPR;
        const int rr = min(row, nvalid - 1);
        const unsigned off = (unsigned)(rr * (int)ld + (col < D / 8 ? 8 * col : 0)) * 2u;
        dma16(src, off, lds + 512 * i);
    }
}

}  // namespace mf
}  // namespace efla
