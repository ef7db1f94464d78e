// Row-major GEMM for gfx950, replacing the reference's cuBLAS calls
// (kernels/cuda/gemm.cu:182-234, 303-548).  Every product runs on the
// hand-written MFMA kernels of this library; no vendor BLAS is linked.
//
//   forward:  C[m,n] = sum_k A[m,k] B[k,n] (+ bias[n])     any of fp32/fp16/bf16
//   backward: dA = dC B^T, dB = A^T dC, dbias = column sums of dC   (bf16)
//
// Matching bf16 / fp16 operands take the large-tile kernel of gemm_fast.hpp
// (256 x 256 workgroup tiles of v_mfma_f32_32x32x16, operands copied straight
// into LDS, persistent grid in XCD bands, split-K for short grids, fused
// bias / residual / GELU epilogues) wherever its shape and alignment checks
// pass (fast_ok).  Everything else -- fp32 and mixed dtypes, odd strides,
// shapes it does not take, and efla_rt_set_gemm_backend(1) -- runs the generic
// kernel below.
//
// The generic kernel covers all three products with one template.  Operands
// are described as (m,k) and (k,n) matrices whose contiguous index is either k
// ("K-major") or the other one; tiles are staged in LDS k-contiguous so MFMA
// fragments are single 16-byte reads, transposing on the way in when the
// source is not K-major.  Workgroup tile 128x128x32, 4 waves each owning 64x64
// (16 MFMA 16x16 tiles), one-stage register prefetch of the next k-tile, fp32
// accumulation, bias fused into the epilogue (the reference adds it in a
// second pass with a second rounding).  Tiles are ordered in groups of 8 rows
// of tiles, and consecutive tile ids are spread so that each XCD works on a
// contiguous band of C (its own L2 then holds the A rows / B columns it
// re-reads).  Matching dtypes run on bf16 / fp16 MFMA; mixed dtypes on fp32
// MFMA after conversion.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>

#include "../../include/efla_hip.h"
#include "../../include/efla_runtime.h"
#include "common.hpp"
#include "gemm_fast.hpp"
#include "internal.hpp"

namespace efla {
namespace gm {

constexpr int NTH = 256, BM = 128, BN = 128, BK = 32;

template <typename MT>
constexpr int lpad() {
    return 16 / (int)sizeof(MT);
}

// Loads a (LINES x BK) operand tile into registers as 8-element runs.
//   KM:  element(line, k) = src[line * ld + k]   (runs along k)
//   !KM: element(line, k) = src[k * ld + line]   (runs along line)
// Out-of-range elements read as zero.
template <typename T, int LINES, bool KM>
struct TileLoader {
    static constexpr int RUNS = LINES * BK / 8 / NTH;  // runs per thread
    float v[RUNS][8];
    __device__ __forceinline__ void load(const T* __restrict__ src, long ld, long line0,
                                         long k0, long nlines, long nk, bool vec_ok) {
#pragma unroll
        for (int r = 0; r < RUNS; ++r) {
            const int id = threadIdx.x + r * NTH;
            int line, kk;
            if (KM) {
                line = id / (BK / 8);
                kk = (id % (BK / 8)) * 8;
            } else {
                kk = id / (LINES / 8);
                line = (id % (LINES / 8)) * 8;
            }
            const long gl = line0 + line, gk = k0 + kk;
            const T* p = KM ? src + gl * ld + gk : src + gk * ld + gl;
            const bool full = KM ? (gl < nlines && gk + 8 <= nk) : (gk < nk && gl + 8 <= nlines);
            if (vec_ok && full) {
                if constexpr (sizeof(T) == 2) {
                    typedef __attribute__((__vector_size__(16))) short s8;
                    const s8 raw = *reinterpret_cast<const s8*>(p);
                    const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
                    for (int i = 0; i < 8; ++i) v[r][i] = to_f(e[i]);
                } else {
                    const floatx4 a = *reinterpret_cast<const floatx4*>(p);
                    const floatx4 b = *reinterpret_cast<const floatx4*>(p + 4);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        v[r][i] = to_f(a[i]);
                        v[r][4 + i] = to_f(b[i]);
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const long l2 = KM ? gl : gl + i;
                    const long k2 = KM ? gk + i : gk;
                    v[r][i] = (l2 < nlines && k2 < nk) ? to_f(KM ? src[l2 * ld + k2]
                                                                 : src[k2 * ld + l2])
                                                       : 0.f;
                }
            }
        }
    }
    // store into LDS tile dst[line * LD + k] (element type MT)
    template <typename MT, int LD>
    __device__ __forceinline__ void store(MT* dst) const {
#pragma unroll
        for (int r = 0; r < RUNS; ++r) {
            const int id = threadIdx.x + r * NTH;
            if (KM) {
                const int line = id / (BK / 8), kk = (id % (BK / 8)) * 8;
#pragma unroll
                for (int i = 0; i < 8; ++i) dst[line * LD + kk + i] = from_f<MT>(v[r][i]);
            } else {
                const int kk = id / (LINES / 8), line = (id % (LINES / 8)) * 8;
#pragma unroll
                for (int i = 0; i < 8; ++i) dst[(line + i) * LD + kk] = from_f<MT>(v[r][i]);
            }
        }
    }
};

// C[m, n] = alpha sum_k opA(m, k) opB(k, n) (+ bias[n]) (+ beta R[m, n]);
// ldc is C's row stride, ldr R's (R is read only when beta != 0 and may be C).
//   opA(m, k) = AKM ? A[m*lda + k] : A[k*lda + m]
//   opB(k, n) = BKM ? B[n*ldb + k] : B[k*ldb + n]
template <typename TA, typename TB, typename TC, typename MT, bool AKM, bool BKM>
__global__ void __launch_bounds__(NTH) gemm_kernel(const TA* __restrict__ A,
                                                   const TB* __restrict__ B,
                                                   const TC* __restrict__ bias, TC* C, long M,
                                                   long N, long K, long lda, long ldb, long ldc,
                                                   int vec_a, int vec_b, float alpha,
                                                   float beta, const TC* R, long ldr) {
    constexpr int LD = BK + lpad<MT>();
    __shared__ __attribute__((aligned(16))) MT As[BM * LD];
    __shared__ __attribute__((aligned(16))) MT Bs[BN * LD];
    // tile order: XCD-banded, then grouped by 8 tile rows
    const long tm_n = (M + BM - 1) / BM, tn_n = (N + BN - 1) / BN;
    const long ntiles = tm_n * tn_n;
    long pid = blockIdx.x;
    if (ntiles % 8 == 0) pid = (pid % 8) * (ntiles / 8) + pid / 8;
    constexpr long GROUP = 8;
    const long group_span = GROUP * tn_n;
    const long g = pid / group_span;
    const long first_m = g * GROUP;
    const long gsize = (tm_n - first_m) < GROUP ? (tm_n - first_m) : GROUP;
    const long tm = first_m + (pid % group_span) % gsize;
    const long tn = (pid % group_span) / gsize;
    const long m0 = tm * BM, n0 = tn * BN;

    const int w = wave_id(), lane = lane_id();
    const int wm = (w >> 1) * 64, wn = (w & 1) * 64;
    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    TileLoader<TA, BM, AKM> la;
    TileLoader<TB, BN, BKM> lb;
    const long nk = (K + BK - 1) / BK;
    la.load(A, lda, m0, 0, M, K, vec_a);
    lb.load(B, ldb, n0, 0, N, K, vec_b);
    for (long kt = 0; kt < nk; ++kt) {
        la.template store<MT, LD>(As);
        lb.template store<MT, LD>(Bs);
        __syncthreads();
        if (kt + 1 < nk) {
            la.load(A, lda, m0, (kt + 1) * BK, M, K, vec_a);
            lb.load(B, ldb, n0, (kt + 1) * BK, N, K, vec_b);
        }
#pragma unroll
        for (int ks = 0; ks < BK; ks += Mfma<MT>::KS) {
            typename Mfma<MT>::frag fa[4], fb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                fa[i] = load_frag<MT>(view_k((const MT*)As, LD), wm + 16 * i, ks, lane);
                fb[i] = load_frag<MT>(view_k((const MT*)Bs, LD), wn + 16 * i, ks, lane);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = Mfma<MT>::mma(fa[i], fb[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const long r = m0 + wm + 16 * i + 4 * (lane >> 4);
            const long c = n0 + wn + 16 * j + (lane & 15);
            if (c >= N) continue;
            const float bb = bias ? to_f(bias[c]) : 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (r + e < M) {
                    float v = alpha * acc[i][j][e] + bb;
                    if (beta != 0.f) v += beta * to_f(R[(r + e) * ldr + c]);
                    C[(r + e) * ldc + c] = from_f<TC>(v);
                }
        }
}

// grad_bias[n] = sum_m dC[m, n]: each workgroup owns 64 columns; its 4 waves
// stride over rows, 64 lanes over columns, then combine in LDS.
__global__ void __launch_bounds__(NTH) colsum_kernel(const bf16* __restrict__ x,
                                                     bf16* __restrict__ y, long M, long N) {
    __shared__ float part[4][64];
    const long c = (long)blockIdx.x * 64 + lane_id();
    float s = 0.f;
    if (c < N)
        for (long r = wave_id(); r < M; r += 4) s += (float)x[r * N + c];
    part[wave_id()][lane_id()] = s;
    __syncthreads();
    if (threadIdx.x < 64 && c < N)
        y[c] = (bf16)(part[0][threadIdx.x] + part[1][threadIdx.x] + part[2][threadIdx.x] +
                      part[3][threadIdx.x]);
}

// Column sums at full width: workgroup (blockIdx.x, blockIdx.y) sums columns
// 128 x .. 128 x + 127 over rows y, y + RS, y + 2 RS, ... (16 row groups of 16
// lanes, 8 bf16 columns each with 16-byte loads) into part[y][col]; a second
// kernel adds the RS partial rows in a fixed order.  N % 8 == 0, x aligned.
constexpr int CS_RS = 32;  // row splits
__global__ void __launch_bounds__(NTH) colsum_part_kernel(const bf16* __restrict__ x,
                                                          float* __restrict__ part, long M,
                                                          long N) {
    __shared__ float acc[16][128 + 4];
    const int q = threadIdx.x & 15, rg = threadIdx.x >> 4;
    const long c0 = (long)blockIdx.x * 128 + 8 * q;
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (c0 < N) {
        // 8 rows' loads in flight before any is added (rows past the end
        // load the last row and count as zero); the sum stays in row order
        constexpr int U = 8;
        constexpr long STEP = 16L * CS_RS;
        for (long r0 = (long)blockIdx.y + (long)rg * CS_RS; r0 < M; r0 += STEP * U) {
            bf16x8 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const long r = r0 + STEP * u < M ? r0 + STEP * u : M - 1;
                v[u] = *reinterpret_cast<const bf16x8*>(x + r * N + c0);
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (r0 + STEP * u < M)
#pragma unroll
                    for (int i = 0; i < 8; ++i) s[i] += (float)v[u][i];
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[rg][8 * q + i] = s[i];
    __syncthreads();
    if (threadIdx.x < 128) {
        const long c = (long)blockIdx.x * 128 + threadIdx.x;
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < 16; ++k) t += acc[k][threadIdx.x];
        if (c < N) part[(long)blockIdx.y * N + c] = t;
    }
}

__global__ void __launch_bounds__(NTH) colsum_final_kernel(const float* __restrict__ part,
                                                           bf16* __restrict__ y, long N) {
    const long c = (long)blockIdx.x * NTH + threadIdx.x;
    if (c >= N) return;
    float t = 0.f;
#pragma unroll 8
    for (int k = 0; k < CS_RS; ++k) t += part[(long)k * N + c];
    y[c] = (bf16)t;
}

// y[c] = sum over the rows of part (fp32 [rows][N]) as bf16, in a fixed order:
// row group g (of 16) adds rows g, g + 16, ..., then the 16 groups in turn.
// Workgroup: 16 row groups x 16 lanes of 4 columns (16-byte loads, all of a
// lane's rows in flight for the few hundred rows this takes); grid over
// 64-column blocks.
__global__ void __launch_bounds__(NTH) colsum_rows_kernel(const float* __restrict__ part,
                                                          long rows, bf16* __restrict__ y,
                                                          long N) {
    __shared__ float acc[16][64 + 1];
    const int q = threadIdx.x & 15, rg = threadIdx.x >> 4;
    const long c0 = (long)blockIdx.x * 64 + 4 * q;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    if (N % 4 == 0 && c0 + 4 <= N) {
        // 8 rows' loads in flight before any is added (rows past the end
        // load the last row and count as zero); the sum stays in row order
        constexpr int U = 8;
        for (long r0 = rg; r0 < rows; r0 += 16 * U) {
            floatx4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const long r = r0 + 16 * u < rows ? r0 + 16 * u : rows - 1;
                v[u] = *reinterpret_cast<const floatx4*>(part + r * N + c0);
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (r0 + 16 * u < rows)
#pragma unroll
                    for (int i = 0; i < 4; ++i) s[i] += v[u][i];
        }
    } else {
        for (long r = rg; r < rows; r += 16)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (c0 + i < N) s[i] += part[r * N + c0 + i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[rg][4 * q + i] = s[i];
    __syncthreads();
    const long c = (long)blockIdx.x * 64 + threadIdx.x;
    if (threadIdx.x < 64 && c < N) {
        float t = 0.f;
#pragma unroll
        for (int g = 0; g < 16; ++g) t += acc[g][threadIdx.x];
        y[c] = (bf16)t;
    }
}

// k == 0: C = bias (broadcast) or 0
template <typename TC>
__global__ void __launch_bounds__(NTH) bias_fill_kernel(TC* __restrict__ C,
                                                        const TC* __restrict__ bias, long M,
                                                        long N) {
    const long total = M * N, stride = (long)gridDim.x * blockDim.x;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride)
        C[i] = bias ? bias[i % N] : from_f<TC>(0.f);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// y[c] = sum_r x[r][c] (bf16 [M][N] -> bf16 [N], fp32 sums in a fixed order)
static int colsum_bf16(const bf16* x, long M, long N, bf16* y, hipStream_t stream) {
    void* ws = nullptr;
    WsLease lease;
    if (N % 8 == 0 && aligned16(x) &&
        workspace_acquire((size_t)CS_RS * N * sizeof(float), stream, &ws, lease) == kSuccess) {
        EFLA_LAUNCH("gemm_bwd_dbias", colsum_part_kernel, dim3((unsigned)((N + 127) / 128), CS_RS),
                    dim3(NTH), stream, x, (float*)ws, M, N);
        EFLA_LAUNCH("gemm_bwd_dbias_final", colsum_final_kernel,
                    dim3((unsigned)((N + NTH - 1) / NTH)), dim3(NTH), stream, (const float*)ws, y,
                    N);
    } else {
        EFLA_LAUNCH("gemm_bwd_dbias", colsum_kernel, dim3((unsigned)((N + 63) / 64)), dim3(NTH),
                    stream, x, y, M, N);
    }
    return (int)hipPeekAtLastError();
}


template <typename TA, typename TB, typename TC, typename MT, bool AKM, bool BKM>
static int launch(const void* a, const void* b, const void* bias, void* c, long M, long N,
                  long K, long lda, long ldb, long ldc, const char* name, hipStream_t st,
                  float alpha = 1.f, float beta = 0.f, const void* r = nullptr, long ldr = 0) {
    const long tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (tiles > 0x7FFFFFFFL) return kInvalidConfiguration;
    // 16-byte runs need an aligned base and a row stride that keeps them aligned
    const int va = aligned16(a) && (lda * (long)sizeof(TA)) % 16 == 0;
    const int vb = aligned16(b) && (ldb * (long)sizeof(TB)) % 16 == 0;
    EFLA_LAUNCH(name, (gemm_kernel<TA, TB, TC, MT, AKM, BKM>), dim3((unsigned)tiles), dim3(NTH),
                st, (const TA*)a, (const TB*)b, (const TC*)bias, (TC*)c, M, N, K, lda, ldb, ldc,
                va, vb, alpha, beta, (const TC*)r, ldr);
    return (int)hipPeekAtLastError();
}

template <typename TA, typename TB, typename TC>
static int fwd_typed(const void* a, const void* b, const void* bias, void* c, long M, long K,
                     long N, hipStream_t st) {
    if constexpr (__is_same(TA, TB) && !__is_same(TA, float))
        return launch<TA, TB, TC, TA, true, false>(a, b, bias, c, M, N, K, K, N, N,
                                                   "gemm_fwd", st);
    else
        return launch<TA, TB, TC, float, true, false>(a, b, bias, c, M, N, K, K, N, N,
                                                      "gemm_fwd", st);
}

template <typename TA, typename TB>
static int fwd_c(int dc, const void* a, const void* b, const void* bias, void* c, long M,
                 long K, long N, hipStream_t st) {
    switch (dc) {
        case kDtypeF32: return fwd_typed<TA, TB, float>(a, b, bias, c, M, K, N, st);
        case kDtypeF16: return fwd_typed<TA, TB, f16>(a, b, bias, c, M, K, N, st);
        case kDtypeBF16: return fwd_typed<TA, TB, bf16>(a, b, bias, c, M, K, N, st);
    }
    return kInvalidValue;
}

template <typename TA>
static int fwd_b(int db, int dc, const void* a, const void* b, const void* bias, void* c,
                 long M, long K, long N, hipStream_t st) {
    switch (db) {
        case kDtypeF32: return fwd_c<TA, float>(dc, a, b, bias, c, M, K, N, st);
        case kDtypeF16: return fwd_c<TA, f16>(dc, a, b, bias, c, M, K, N, st);
        case kDtypeBF16: return fwd_c<TA, bf16>(dc, a, b, bias, c, M, K, N, st);
    }
    return kInvalidValue;
}

static size_t dsize(int dt) {
    switch (dt) {
        case kDtypeF32: return 4;
        case kDtypeF16: return 2;
        case kDtypeBF16: return 2;
    }
    return 0;
}

template <typename TC>
static int launch_bias_fill(void* c, const void* bias, long M, long N, hipStream_t st) {
    long g = (M * N + NTH - 1) / NTH;
    if (g > 8192) g = 8192;
    EFLA_LAUNCH("gemm_bias_fill", bias_fill_kernel<TC>, dim3((unsigned)g), dim3(NTH), st, (TC*)c,
                (const TC*)bias, M, N);
    return (int)hipPeekAtLastError();
}

// ---------------------------------------------------------------------------
// large-tile kernel (gemm_fast.hpp)
// ---------------------------------------------------------------------------
// An operand of the large-tile kernel: element (line, k) at p[line * ld + k]
// (k-contiguous) or p[k * ld + line].
struct FastOp {
    const void* p;
    long ld;
    bool kc;
};

static bool aligned_to(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Whether the large-tile kernel takes the problem: whole 16-byte rows and
// chunks along k (K % 8), along every line-contiguous operand's lines and
// along the output's columns (N % 8); 16-byte aligned operands and outputs
// (the epilogue moves 16-byte row pieces); 32-bit in-tile offsets
// (256 * ld * 2 < 2^31).
static bool fast_ok(long M, long N, long K, const FastOp& a, const FastOp& b, const void* d,
                    long ldd, const void* bias, const void* c, long ldc, const void* aux,
                    long ldaux) {
    const long lim = (long)1 << 22;
    if (M < 1 || N < 1 || K < 1 || M > INT32_MAX / 2 || N > INT32_MAX / 2) return false;
    if (K % 8 || N % 8 || (!a.kc && M % 8)) return false;
    for (long ld : {a.ld, b.ld, ldd})
        if (ld % 8 || ld >= lim) return false;
    if (!aligned_to(a.p, 16) || !aligned_to(b.p, 16) || !aligned_to(d, 16)) return false;
    if (bias && !aligned_to(bias, 16)) return false;
    if (c && (ldc % 8 || ldc >= lim || !aligned_to(c, 16))) return false;
    if (aux && (ldaux % 8 || ldaux >= lim || !aligned_to(aux, 16))) return false;
    return true;
}

template <typename T, int EPI, int NW>
static void fast_kernel_launch_nw(const FastOp& a, const FastOp& b, const gf::Opnd& A,
                                  const gf::Opnd& B, long M, long N, long K,
                                  const gf::EpiArgs<T>& ea, int ksplit, long kper, long tiles,
                                  const char* name, hipStream_t st) {
    // persistent: at most one workgroup per CU (the LDS allows no more)
    const long cus = device_cu_count() > 0 ? device_cu_count() : 256;
    const long items = tiles * ksplit;
    const dim3 grid((unsigned)(items < cus ? items : cus)), block(64 * NW);
    if (a.kc && b.kc)
        EFLA_LAUNCH(name, (gf::gemm_fast_kernel<T, true, true, EPI, NW>), grid, block, st, A, B,
                    M, N, K, ea, ksplit, kper);
    else if (a.kc)
        EFLA_LAUNCH(name, (gf::gemm_fast_kernel<T, true, false, EPI, NW>), grid, block, st, A, B,
                    M, N, K, ea, ksplit, kper);
    else if (b.kc)
        EFLA_LAUNCH(name, (gf::gemm_fast_kernel<T, false, true, EPI, NW>), grid, block, st, A, B,
                    M, N, K, ea, ksplit, kper);
    else
        EFLA_LAUNCH(name, (gf::gemm_fast_kernel<T, false, false, EPI, NW>), grid, block, st, A,
                    B, M, N, K, ea, ksplit, kper);
}

// 8 waves (two per SIMD) measured faster than 4 at every config-4 shape
template <typename T, int EPI>
static void fast_kernel_launch(const FastOp& a, const FastOp& b, const gf::Opnd& A,
                               const gf::Opnd& B, long M, long N, long K,
                               const gf::EpiArgs<T>& ea, int ksplit, long kper, long tiles,
                               const char* name, hipStream_t st) {
    fast_kernel_launch_nw<T, EPI, 8>(a, b, A, B, M, N, K, ea, ksplit, kper, tiles, name, st);
}

// Large-tile product.  Problems with fewer output tiles than the GPU has CUs
// and a long contraction are split along k: fp32
// partial tiles go to the stream's cached workspace and a second kernel adds
// them in split order and runs the epilogue (plain epilogues only).
template <typename T, int EPI>
static int fast_launch(const FastOp& a, const FastOp& b, long M, long N, long K,
                       const gf::EpiArgs<T>& ea, const char* name, hipStream_t st) {
    const gf::Opnd A{(const char*)a.p, a.ld, (int)M}, B{(const char*)b.p, b.ld, (int)N};
    const long tiles = ((M + gf::BM - 1) / gf::BM) * ((N + gf::BN - 1) / gf::BN);
    if (tiles > 0x7FFFFFFFL / 64) return kInvalidConfiguration;
    int ksplit = 1;
    const long cus = device_cu_count() > 0 ? device_cu_count() : 256;
    if ((EPI == gf::EPI_PLAIN || EPI == gf::EPI_RESID) && tiles < cus) {
        const long want = cus / tiles;       // splits that fill every CU once
        const long most = K / (4 * gf::BK);  // at least 4 k-iterations each
        ksplit = (int)std::max(1L, std::min({want, most, 32L}));
    }
    if (ksplit == 1) {
        fast_kernel_launch<T, EPI>(a, b, A, B, M, N, K, ea, 1, K, tiles, name, st);
        return (int)hipPeekAtLastError();
    }
    const long kper = ((K + ksplit - 1) / ksplit + gf::BK - 1) / gf::BK * gf::BK;
    ksplit = (int)((K + kper - 1) / kper);
    void* ws = nullptr;
    WsLease lease;
    EFLA_CHECK((hipError_t)workspace_acquire((size_t)ksplit * M * N * sizeof(float), st, &ws,
                                             lease));
    gf::EpiArgs<T> ep = ea;
    ep.part = (float*)ws;
    fast_kernel_launch<T, gf::EPI_PARTIAL>(a, b, A, B, M, N, K, ep, ksplit, kper, tiles, name,
                                           st);
    long g = (M * (N / 4) + 255) / 256;
    if (g > 4096) g = 4096;
    EFLA_LAUNCH("gemm_splitk_reduce", gf::gemm_splitk_reduce<T>, dim3((unsigned)g), dim3(256), st,
                ep, M, N, ksplit);
    return (int)hipPeekAtLastError();
}

template <typename T>
static gf::EpiArgs<T> epi(void* d, long ldd, const void* bias = nullptr, float alpha = 1.f,
                          float beta = 0.f, const void* c = nullptr, long ldc = 0,
                          void* aux = nullptr, long ldaux = 0) {
    return gf::EpiArgs<T>{(T*)d, ldd, (const T*)bias, (const T*)c, ldc, alpha, beta, (T*)aux,
                          ldaux, nullptr, nullptr};
}

// 0: the hand-written kernels (large-tile where it takes the problem, else the
// generic one); 1: the generic hand-written kernel only
static std::mutex g_backend_mu;
static int g_backend = 0;

}  // namespace gm

int colsum_bf16_rows(const bf16* x, long M, long N, bf16* y, hipStream_t stream) {
    return gm::colsum_bf16(x, M, N, y, stream);
}

}  // namespace efla

using namespace efla;
using namespace efla::gm;

static int backend() {
    std::lock_guard<std::mutex> lk(g_backend_mu);
    return g_backend;
}

extern "C" int efla_rt_set_gemm_backend(int backend) {
    if (backend < 0 || backend > 1) return kInvalidValue;
    std::lock_guard<std::mutex> lk(g_backend_mu);
    g_backend = backend;
    return kSuccess;
}

extern "C" int gemm_forward_hip(const void* a, const void* b, const void* bias, void* c,
                                size_t m, size_t k, size_t n, int dtype_a, int dtype_b,
                                int dtype_c, hipStream_t stream) {
    if (!a || !b || !c) return kInvalidValue;
    if (!dsize(dtype_a) || !dsize(dtype_b) || !dsize(dtype_c)) return kInvalidValue;
    size_t mn;
    if (!mul_ok(m, n, &mn)) return kInvalidValue;
    if (m == 0 || n == 0) return kSuccess;
    if (m > ((size_t)1 << 40) || n > ((size_t)1 << 40) || k > ((size_t)1 << 40))
        return kInvalidValue;
    if (k == 0) {
        switch (dtype_c) {
            case kDtypeF32: return launch_bias_fill<float>(c, bias, (long)m, (long)n, stream);
            case kDtypeF16: return launch_bias_fill<f16>(c, bias, (long)m, (long)n, stream);
            default: return launch_bias_fill<bf16>(c, bias, (long)m, (long)n, stream);
        }
    }
    if (dtype_a == dtype_b && dtype_b == dtype_c) {
        // C[m, n] = A[m, k] B[k, n]: A k-contiguous, B line (n) contiguous
        const FastOp fa{a, (long)k, true}, fb{b, (long)n, false};
        if (dtype_a != kDtypeF32 && backend() != 1 &&
            fast_ok((long)m, (long)n, (long)k, fa, fb, c, (long)n, bias, nullptr, 0, nullptr, 0)) {
            if (dtype_a == kDtypeBF16)
                return fast_launch<bf16, gf::EPI_PLAIN>(fa, fb, (long)m, (long)n, (long)k,
                                                        epi<bf16>(c, (long)n, bias), "gemm_fwd",
                                                        stream);
            return fast_launch<f16, gf::EPI_PLAIN>(fa, fb, (long)m, (long)n, (long)k,
                                                   epi<f16>(c, (long)n, bias), "gemm_fwd",
                                                   stream);
        }
    }
    switch (dtype_a) {
        case kDtypeF32:
            return fwd_b<float>(dtype_b, dtype_c, a, b, bias, c, (long)m, (long)k, (long)n, stream);
        case kDtypeF16:
            return fwd_b<f16>(dtype_b, dtype_c, a, b, bias, c, (long)m, (long)k, (long)n, stream);
        case kDtypeBF16:
            return fwd_b<bf16>(dtype_b, dtype_c, a, b, bias, c, (long)m, (long)k, (long)n, stream);
    }
    return kInvalidValue;
}

extern "C" int gemm_backward_hip(const void* grad_c, const void* a, const void* b, void* grad_a,
                                 void* grad_b, void* grad_bias, size_t m, size_t k, size_t n,
                                 hipStream_t stream) {
    size_t ea, eb;
    if (!mul_ok(m, k, &ea) || !mul_ok(k, n, &eb)) return kInvalidValue;
    const bool need_a = grad_a != nullptr, need_b = grad_b != nullptr,
               need_bias = grad_bias != nullptr;
    if (!need_a && !need_b && !need_bias) return kSuccess;
    // validation and zero-fills in the reference's order (gemm.cu:424-466)
    if (need_a) {
        if (m == 0 || k == 0 || n == 0) {
            EFLA_CHECK((hipError_t)fill_zero(grad_a, ea * 2, stream));
        } else if (!grad_c || !b) {
            return kInvalidValue;
        }
    }
    if (need_b) {
        if (k == 0 || n == 0 || m == 0) {
            EFLA_CHECK((hipError_t)fill_zero(grad_b, eb * 2, stream));
        } else if (!a || !grad_c) {
            return kInvalidValue;
        }
    }
    if (need_bias) {
        if (n == 0) return kSuccess;
        if (m == 0) {
            EFLA_CHECK((hipError_t)fill_zero(grad_bias, n * 2, stream));
        } else if (!grad_c) {
            return kInvalidValue;
        }
    }
    const long M = (long)m, K = (long)k, N = (long)n;
    if (need_a && m && k && n) {
        // dA[m, k] = sum_n dC[m, n] B[k, n]; column-major dA^T = op_T(B') dC^T
        // with B' = B as (n x k, ld n) and dC^T as (n x m, ld n)
        int rc = -1;
        // dA = dC B^T: contraction over n, both operands n-contiguous
        const FastOp fa{grad_c, N, true}, fb{b, N, true};
        if (backend() != 1 &&
            fast_ok(M, K, N, fa, fb, grad_a, K, nullptr, nullptr, 0, nullptr, 0))
            rc = fast_launch<bf16, gf::EPI_PLAIN>(fa, fb, M, K, N, epi<bf16>(grad_a, K),
                                                  "gemm_bwd_da", stream);
        if (rc < 0)
            rc = launch<bf16, bf16, bf16, bf16, true, true>(grad_c, b, nullptr, grad_a, M, K, N,
                                                            N, N, K, "gemm_bwd_da", stream);
        if (rc != kSuccess) return rc;
    }
    if (need_b && m && k && n) {
        // dB[k, n] = sum_m A[m, k] dC[m, n]; column-major dB^T = dC^T op_T(A')
        // with dC^T as (n x m, ld n) and A' = A as (k x m, ld k)
        int rc = -1;
        // dB = A^T dC: contraction over m, A k- (line-) contiguous, dC n-contiguous
        const FastOp fa{a, K, false}, fb{grad_c, N, false};
        if (backend() != 1 &&
            fast_ok(K, N, M, fa, fb, grad_b, N, nullptr, nullptr, 0, nullptr, 0))
            rc = fast_launch<bf16, gf::EPI_PLAIN>(fa, fb, K, N, M, epi<bf16>(grad_b, N),
                                                  "gemm_bwd_db", stream);
        if (rc < 0)
            rc = launch<bf16, bf16, bf16, bf16, false, false>(a, grad_c, nullptr, grad_b, K, N, M,
                                                              K, N, N, "gemm_bwd_db", stream);
        if (rc != kSuccess) return rc;
    }
    if (need_bias && m && n) {
        const int rc = colsum_bf16((const bf16*)grad_c, M, N, (bf16*)grad_bias, stream);
        if (rc != kSuccess) return rc;
    }
    return (int)hipPeekAtLastError();
}

// gemm_ex on the generic kernel: any shape, strides and transposes.
template <typename T>
static int ex_generic(int ta, int tb, size_t m, size_t n, size_t k, float alpha, const void* a,
                      size_t lda, const void* b, size_t ldb, const void* bias, float beta,
                      const void* c, size_t ldc, void* d, size_t ldd, hipStream_t st) {
    typedef typename std::conditional<__is_same(T, float), float, T>::type MT;
    const long M = (long)m, N = (long)n, K = (long)k;
#define EX_CASE(AK, BK)                                                                          \
    return launch<T, T, T, MT, AK, BK>(a, b, bias, d, M, N, K, (long)lda, (long)ldb, (long)ldd, \
                                       "gemm_ex", st, alpha, beta, c, (long)ldc)
    if (!ta && !tb) EX_CASE(true, false);
    if (!ta && tb) EX_CASE(true, true);
    if (ta && !tb) EX_CASE(false, false);
    EX_CASE(false, true);
#undef EX_CASE
}

extern "C" int gemm_ex_hip(int trans_a, int trans_b, size_t m, size_t n, size_t k, float alpha,
                           const void* a, size_t lda, const void* b, size_t ldb,
                           const void* bias, float beta, const void* c, size_t ldc, void* d,
                           size_t ldd, int dtype, hipStream_t stream) {
    if ((trans_a != 0 && trans_a != 1) || (trans_b != 0 && trans_b != 1) || !dsize(dtype))
        return kInvalidValue;
    if (m == 0 || n == 0) return kSuccess;
    if (!d || (k > 0 && (!a || !b)) || (beta != 0.f && !c)) return kInvalidValue;
    const size_t lim = (size_t)1 << 40;
    if (m > lim || n > lim || k > lim || lda > lim || ldb > lim || ldc > lim || ldd > lim)
        return kInvalidValue;
    // row strides: op(A) is m x k (A stored m x k, or k x m when transposed),
    // etc.; with k == 0 neither A nor B is read, nor are their strides
    if ((k > 0 && (lda < (trans_a ? m : k) || ldb < (trans_b ? k : n))) || ldd < n ||
        (beta != 0.f && ldc < n))
        return kInvalidValue;
    // op(A) is A (k-contiguous) or A^T of a stored k x m (m-contiguous); op(B)
    // is B of a stored k x n (n-contiguous) or B^T of a stored n x k
    const FastOp fa{a, (long)lda, trans_a == 0}, fb{b, (long)ldb, trans_b != 0};
    const void* cc = beta != 0.f ? c : nullptr;
    if (dtype != kDtypeF32 && backend() != 1 &&
        fast_ok((long)m, (long)n, (long)k, fa, fb, d, (long)ldd, bias, cc, (long)ldc, nullptr, 0)) {
        if (cc) {
            if (dtype == kDtypeBF16)
                return fast_launch<bf16, gf::EPI_RESID>(
                    fa, fb, (long)m, (long)n, (long)k,
                    epi<bf16>(d, (long)ldd, bias, alpha, beta, cc, (long)ldc), "gemm_ex", stream);
            return fast_launch<f16, gf::EPI_RESID>(
                fa, fb, (long)m, (long)n, (long)k,
                epi<f16>(d, (long)ldd, bias, alpha, beta, cc, (long)ldc), "gemm_ex", stream);
        }
        if (dtype == kDtypeBF16)
            return fast_launch<bf16, gf::EPI_PLAIN>(fa, fb, (long)m, (long)n, (long)k,
                                                    epi<bf16>(d, (long)ldd, bias, alpha),
                                                    "gemm_ex", stream);
        return fast_launch<f16, gf::EPI_PLAIN>(fa, fb, (long)m, (long)n, (long)k,
                                               epi<f16>(d, (long)ldd, bias, alpha), "gemm_ex",
                                               stream);
    }
    switch (dtype) {
        case kDtypeBF16: return ex_generic<bf16>(trans_a, trans_b, m, n, k, alpha, a, lda, b, ldb,
                                                 bias, beta, cc, ldc, d, ldd, stream);
        case kDtypeF16: return ex_generic<f16>(trans_a, trans_b, m, n, k, alpha, a, lda, b, ldb,
                                               bias, beta, cc, ldc, d, ldd, stream);
        default: return ex_generic<float>(trans_a, trans_b, m, n, k, alpha, a, lda, b, ldb, bias,
                                          beta, cc, ldc, d, ldd, stream);
    }
}

// ---------------------------------------------------------------------------
// GEMMs with the MLP's GELU fused into the epilogue
// ---------------------------------------------------------------------------
extern "C" int gelu_forward_hip(const void* input, void* output, size_t numel, bool approximate,
                                hipStream_t stream);
extern "C" int gelu_backward_hip(const void* grad_output, const void* input, void* grad_input,
                                 size_t numel, bool approximate, hipStream_t stream);

extern "C" int gemm_gelu_forward_hip(const void* a, const void* b, const void* bias, void* pre,
                                     void* out, size_t m, size_t k, size_t n,
                                     hipStream_t stream) {
    if (!a || !b || !pre || !out) return kInvalidValue;
    size_t mn;
    if (!mul_ok(m, n, &mn)) return kInvalidValue;
    if (m == 0 || n == 0) return kSuccess;
    if (m > ((size_t)1 << 40) || n > ((size_t)1 << 40) || k > ((size_t)1 << 40))
        return kInvalidValue;
    const FastOp fa{a, (long)k, true}, fb{b, (long)n, false};
    if (k > 0 && backend() == 0 &&
        fast_ok((long)m, (long)n, (long)k, fa, fb, out, (long)n, bias, nullptr, 0, pre,
                (long)n))
        return fast_launch<bf16, gf::EPI_GELU_AUX>(
            fa, fb, (long)m, (long)n, (long)k,
            epi<bf16>(out, (long)n, bias, 1.f, 0.f, nullptr, 0, pre, (long)n), "gemm_gelu_fwd",
            stream);
    // the product, then GELU over it (the same functions, so the same bits)
    const int rc = gemm_forward_hip(a, b, bias, pre, m, k, n, kDtypeBF16, kDtypeBF16, kDtypeBF16,
                                    stream);
    if (rc != kSuccess) return rc;
    return gelu_forward_hip(pre, out, mn, true, stream);
}

extern "C" int gemm_gelu_backward_hip(const void* grad_c, const void* a, const void* b,
                                      const void* pre, void* grad_pre, void* grad_b,
                                      void* grad_bias, void* grad_pre_bias, size_t m, size_t k,
                                      size_t n, hipStream_t stream) {
    size_t mk;
    if (!mul_ok(m, k, &mk)) return kInvalidValue;
    if (grad_pre_bias && !grad_pre) return kInvalidValue;  // the sums are of grad_pre
    if (grad_pre) {
        if (m == 0 || k == 0) {
            // nothing to contract or no rows: gemm_backward_hip's zero fill
            int rc = gemm_backward_hip(grad_c, a, b, grad_pre, nullptr, nullptr, m, k, n, stream);
            if (rc != kSuccess) return rc;
            if (grad_pre_bias && k) {
                rc = fill_zero(grad_pre_bias, k * 2, stream);
                if (rc != kSuccess) return rc;
            }
        } else {
            if (!grad_c || !b || !pre) return kInvalidValue;
            // grad_pre = (grad_c b^T) * GELU'(pre): contraction over n, both n-contiguous
            const FastOp fa{grad_c, (long)n, true}, fb{b, (long)n, true};
            if (n > 0 && backend() == 0 &&
                fast_ok((long)m, (long)k, (long)n, fa, fb, grad_pre, (long)k, nullptr, nullptr,
                        0, pre, (long)k)) {
                gf::EpiArgs<bf16> ea = epi<bf16>(grad_pre, (long)k, nullptr, 1.f, 0.f, nullptr, 0,
                                                 (void*)pre, (long)k);
                // grad_pre's column sums from the epilogue: one fp32 row per
                // 128 output rows, then their sum
                void* ws = nullptr;
                WsLease lease;
                const long prow = ((long)m + 127) / 128;
                if (grad_pre_bias) {
                    EFLA_CHECK((hipError_t)workspace_acquire((size_t)prow * k * sizeof(float),
                                                             stream, &ws, lease));
                    ea.cpart = (float*)ws;
                }
                int rc = fast_launch<bf16, gf::EPI_DGELU>(fa, fb, (long)m, (long)k, (long)n, ea,
                                                          "gemm_gelu_bwd_da", stream);
                if (rc != kSuccess) return rc;
                if (grad_pre_bias)
                    EFLA_LAUNCH("gemm_gelu_bwd_dbias", colsum_rows_kernel,
                                dim3((unsigned)((k + 63) / 64)), dim3(NTH), stream,
                                (const float*)ws, prow, (bf16*)grad_pre_bias, (long)k);
            } else {
                int rc = gemm_backward_hip(grad_c, a, b, grad_pre, nullptr, nullptr, m, k, n,
                                           stream);
                if (rc != kSuccess) return rc;
                rc = gelu_backward_hip(grad_pre, pre, grad_pre, mk, true, stream);
                if (rc != kSuccess) return rc;
                if (grad_pre_bias) {
                    rc = colsum_bf16((const bf16*)grad_pre, (long)m, (long)k,
                                     (bf16*)grad_pre_bias, stream);
                    if (rc != kSuccess) return rc;
                }
            }
        }
    }
    if (!grad_b && !grad_bias) return (int)hipPeekAtLastError();
    return gemm_backward_hip(grad_c, a, b, nullptr, grad_b, grad_bias, m, k, n, stream);
}
