// Shared device helpers for the gfx950 EFLA library: element types, MFMA
// fragments, tile "views" over LDS / global memory, and a workgroup-level
// 16x16-tiled GEMM built on v_mfma_f32_16x16x32_bf16 (bf16 operands) and
// v_mfma_f32_16x16x4_f32 (fp32 operands).
//
// MFMA lane layouts (checked on gfx950 with an in-bounds probe):
//   A (16 x KS):  lane l holds row (l & 15), k = KPL*(l >> 4) + [0, KPL)
//   B (KS x 16):  lane l holds col (l & 15), k = KPL*(l >> 4) + [0, KPL)
//   C (16 x 16):  lane l holds col (l & 15), rows 4*(l >> 4) + [0, 4)
// with KS = 32, KPL = 8 for bf16 / fp16 and KS = 4, KPL = 1 for fp32.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace efla {

typedef __bf16 bf16;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4;
typedef _Float16 f16;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;

constexpr int kWave = 64;

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f(f16 x) { return (float)x; }

template <typename T>
__device__ __forceinline__ T from_f(float x);
template <>
__device__ __forceinline__ float from_f<float>(float x) { return x; }
template <>
__device__ __forceinline__ bf16 from_f<bf16>(float x) { return (bf16)x; }
template <>
__device__ __forceinline__ f16 from_f<f16>(float x) { return (f16)x; }

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x / kWave; }

// ---------------------------------------------------------------------------
// MFMA traits per operand type
// ---------------------------------------------------------------------------
template <typename MT>
struct Mfma;

template <>
struct Mfma<bf16> {
    static constexpr int KS = 32;   // k extent of one instruction
    static constexpr int KPL = 8;   // k values per lane
    typedef bf16x8 frag;
    static __device__ __forceinline__ floatx4 mma(frag a, frag b, floatx4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Mfma<f16> {
    static constexpr int KS = 32;
    static constexpr int KPL = 8;
    typedef f16x8 frag;
    static __device__ __forceinline__ floatx4 mma(frag a, frag b, floatx4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Mfma<float> {
    static constexpr int KS = 4;
    static constexpr int KPL = 1;
    typedef float frag;
    static __device__ __forceinline__ floatx4 mma(frag a, frag b, floatx4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
};

// ---------------------------------------------------------------------------
// A view describes one MFMA operand as a (line, k) matrix: for A the lines are
// output rows, for B the lines are output columns; k is the contraction index.
//   element(line, k) = base[line * ls + k * ks] * lscale[line] * kscale[k]
// KC marks ks == 1 (k-contiguous), which allows one vector load per fragment.
// ---------------------------------------------------------------------------
template <typename T, bool KC>
struct View {
    const T* base;
    int ls;
    int ks;
    const float* lscale;  // optional per-line factor (nullptr = 1)
    const float* kscale;  // optional per-k factor (nullptr = 1)
};

template <typename T>
__device__ __forceinline__ View<T, true> view_k(const T* base, int ls,
                                                const float* lscale = nullptr,
                                                const float* kscale = nullptr) {
    return View<T, true>{base, ls, 1, lscale, kscale};
}
template <typename T>
__device__ __forceinline__ View<T, false> view_t(const T* base, int ks,
                                                 const float* lscale = nullptr,
                                                 const float* kscale = nullptr) {
    // transposed storage: element(line, k) = base[k * ks + line]
    return View<T, false>{base, 1, ks, lscale, kscale};
}

template <typename MT, typename T, bool KC>
__device__ __forceinline__ typename Mfma<MT>::frag load_frag(const View<T, KC>& v, int line0,
                                                             int k0, int lane) {
    typedef typename Mfma<MT>::frag F;
    const int line = line0 + (lane & 15);
    const int kb = k0 + Mfma<MT>::KPL * (lane >> 4);
    const float ls = v.lscale ? v.lscale[line] : 1.0f;
    F f;
    if constexpr (Mfma<MT>::KPL == 1) {
        float x = to_f(v.base[line * v.ls + kb * v.ks]) * ls;
        if (v.kscale) x *= v.kscale[kb];
        f = x;
    } else if constexpr (KC && __is_same(T, MT)) {
        // 8 contiguous 2-byte elements = one 16-byte load
        const F raw = *reinterpret_cast<const F*>(v.base + line * v.ls + kb);
        if (v.lscale == nullptr && v.kscale == nullptr) {
            f = raw;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float x = (float)raw[i] * ls;
                if (v.kscale) x *= v.kscale[kb + i];
                f[i] = from_f<MT>(x);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float x = to_f(v.base[line * v.ls + (kb + i) * v.ks]) * ls;
            if (v.kscale) x *= v.kscale[kb + i];
            f[i] = from_f<MT>(x);
        }
    }
    return f;
}

// acc += A(line0.., 0..KD) * B(0..KD, col0..) for one 16x16 tile.
template <typename MT, int KD, typename VA, typename VB>
__device__ __forceinline__ floatx4 tile_mma(floatx4 acc, const VA& a, int row0, const VB& b,
                                            int col0, int lane) {
#pragma unroll 4
    for (int k = 0; k < KD; k += Mfma<MT>::KS) {
        const auto fa = load_frag<MT>(a, row0, k, lane);
        const auto fb = load_frag<MT>(b, col0, k, lane);
        acc = Mfma<MT>::mma(fa, fb, acc);
    }
    return acc;
}

// Workgroup GEMM over 16x16 tiles: C(M x N) = A(M x KD) * B(KD x N).  Tiles
// are dealt round-robin to the NW waves; `skip(tm, tn)` drops whole tiles (for
// triangular products) and `epi(row, col, acc)` receives each finished tile,
// where lane holds C[row + i][col] for i = 0..3.
template <typename MT, int M, int N, int KD, int NW, typename VA, typename VB, typename Skip,
          typename Epi>
__device__ __forceinline__ void block_gemm(const VA& a, const VB& b, Skip skip, Epi epi) {
    const int lane = lane_id();
    const int w = wave_id();
    constexpr int TN = N / 16;
    constexpr int NT = (M / 16) * TN;
    for (int t = w; t < NT; t += NW) {
        const int tm = t / TN, tn = t % TN;
        if (skip(tm, tn)) continue;
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        acc = tile_mma<MT, KD>(acc, a, tm * 16, b, tn * 16, lane);
        epi(tm * 16 + 4 * (lane >> 4), tn * 16 + (lane & 15), acc);
    }
}

struct NoSkip {
    __device__ __forceinline__ bool operator()(int, int) const { return false; }
};
// keep tiles with tm >= tn (lower triangle incl. diagonal tiles)
struct SkipUpper {
    __device__ __forceinline__ bool operator()(int tm, int tn) const { return tn > tm; }
};
// keep tiles with tm <= tn
struct SkipLower {
    __device__ __forceinline__ bool operator()(int tm, int tn) const { return tn < tm; }
};

// ---------------------------------------------------------------------------
// Cooperative tile movement (all threads of the workgroup take part)
// ---------------------------------------------------------------------------
// dst[r * dld + c] = src[r * sld + c] for r < rows_valid, zero for
// rows_valid <= r < ROWS; COLS elements per row.  16-byte vectors where the
// element type allows.
template <typename T, int ROWS, int COLS, int NT>
__device__ __forceinline__ void load_rows(T* dst, int dld, const T* __restrict__ src, long sld,
                                          int rows_valid) {
    constexpr int VEC = 16 / sizeof(T);
    constexpr int VPR = COLS / VEC;
    typedef __attribute__((__vector_size__(16))) int i4;
    for (int i = threadIdx.x; i < ROWS * VPR; i += NT) {
        const int r = i / VPR, c = (i % VPR) * VEC;
        i4 val = {0, 0, 0, 0};
        if (r < rows_valid) val = *reinterpret_cast<const i4*>(src + r * sld + c);
        *reinterpret_cast<i4*>(dst + r * dld + c) = val;
    }
}

// Same source, stored transposed: dst[c * dld + r].
template <typename T, int ROWS, int COLS, int NT>
__device__ __forceinline__ void load_rows_t(T* dst, int dld, const T* __restrict__ src, long sld,
                                            int rows_valid) {
    constexpr int VEC = 16 / sizeof(T);
    constexpr int VPR = COLS / VEC;
    typedef __attribute__((__vector_size__(16))) int i4;
    for (int i = threadIdx.x; i < ROWS * VPR; i += NT) {
        const int r = i / VPR, c = (i % VPR) * VEC;
        i4 val = {0, 0, 0, 0};
        if (r < rows_valid) val = *reinterpret_cast<const i4*>(src + r * sld + c);
        const T* e = reinterpret_cast<const T*>(&val);
#pragma unroll
        for (int j = 0; j < VEC; ++j) dst[(c + j) * dld + r] = e[j];
    }
}

// Store the 4 values of a C fragment (rows row..row+3, column col) to a
// row-major destination with row stride ld; rows >= rows_valid are dropped.
template <typename T>
__device__ __forceinline__ void store_frag(T* dst, long ld, int row, int col, floatx4 acc,
                                           int rows_valid) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (row + i < rows_valid) dst[(long)(row + i) * ld + col] = from_f<T>(acc[i]);
}

// Store a C fragment transposed: dst[col * ld + row + i] (4 contiguous values).
template <typename T>
__device__ __forceinline__ void store_frag_t(T* dst, int ld, int row, int col, floatx4 acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[col * ld + row + i] = from_f<T>(acc[i]);
}

}  // namespace efla
