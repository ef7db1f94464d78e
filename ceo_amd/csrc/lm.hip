// Token embedding and cross-entropy for gfx950: the two ends of the config-4
// language-model step around EFLA.
//
// Embedding (replaces embedding_forward_cuda, kernels.h:366-373, declared but
// not implemented in the reference; semantics of Embedding.forward,
// layers.zig:658-686): out[i, :] = weight[idx[i], :], bf16 rows copied with
// 16-byte accesses, one wave per row.  The reference entry has no vocabulary
// size and so cannot range-check; embedding_forward_checked_hip takes it and
// zero-fills rows whose id is out of range.  The backward (no reference
// counterpart) adds each gradient row into an fp32 weight gradient with vector
// float atomics (summation order between duplicate ids is not fixed).
//
// Cross-entropy (replaces cross_entropy_{forward,backward}_cuda,
// kernels.h:248-270, declared only; semantics of crossEntropyForwardCpu,
// nn_kernels.zig:200-246): per row i with lse = log sum_j exp(z_ij),
//   loss[i] = ((1 - eps) (lse - z_i,t) + eps log V) / B
// (the CPU reference's label smoothing adds the constant eps log V), and
//   dL/dz_ij = grad_loss[i] (1 - eps) (softmax_ij - [j = t_i]) / B.
// One workgroup per row; when the row fits (V <= 8192 * NV for the compiled
// NV, V % 8 == 0, aligned rows) it is held in registers, so the forward reads
// the logits once and the backward reads them once and writes the gradient
// once; cross_entropy_forward_backward_hip (no reference counterpart) does
// both from one read, optionally in place.  Other rows take a looped two-pass
// path.  A target outside [0, V) gives loss NaN and a zero gradient row.
#include <hip/hip_runtime.h>
#include <math.h>

#include "../../include/efla_hip.h"
#include "common.hpp"
#include "internal.hpp"

namespace efla {
namespace lm {

// ---------------------------------------------------------------------------
// embedding
// ---------------------------------------------------------------------------
constexpr int ENT = 256;  // 4 rows per workgroup, one per wave

// vocab < 0: no range check (the reference entry)
__global__ void __launch_bounds__(ENT) emb_fwd_kernel(const int32_t* __restrict__ idx,
                                                      const bf16* __restrict__ w,
                                                      bf16* __restrict__ out, long n, long D,
                                                      long vocab, int vec) {
    const long row = (long)blockIdx.x * (ENT / kWave) + wave_id();
    if (row >= n) return;
    const int lane = lane_id();
    const long id = idx[row];
    const bool ok = vocab < 0 || (id >= 0 && id < vocab);
    const bf16* src = w + id * D;
    bf16* dst = out + row * D;
    if (!ok) {  // checked entry, id out of range: a zero row, nothing read
        for (long c = lane; c < D; c += kWave) dst[c] = (bf16)0.f;
    } else if (vec) {
        for (long c = lane; c < D / 8; c += kWave)
            reinterpret_cast<bf16x8*>(dst)[c] = reinterpret_cast<const bf16x8*>(src)[c];
    } else {
        for (long c = lane; c < D; c += kWave) dst[c] = src[c];
    }
}

__global__ void __launch_bounds__(ENT) emb_bwd_kernel(const bf16* __restrict__ dy,
                                                      const int32_t* __restrict__ idx,
                                                      float* __restrict__ dw, long n, long D,
                                                      long vocab) {
    const long row = (long)blockIdx.x * (ENT / kWave) + wave_id();
    if (row >= n) return;
    const long id = idx[row];
    if (id < 0 || id >= vocab) return;
    const bf16* g = dy + row * D;
    float* d = dw + id * D;
    for (long c = lane_id(); c < D; c += kWave) unsafeAtomicAdd(d + c, (float)g[c]);
}

// ---------------------------------------------------------------------------
// cross-entropy
// ---------------------------------------------------------------------------
constexpr int CNT = 1024;          // threads per row
constexpr int CW = CNT / kWave;    // waves per row
constexpr float kLog2e = 1.4426950408889634f;

// (max, sum of exp(x - max)) pairs, combined
__device__ __forceinline__ void ms_add(float& m, float& s, float m2, float s2) {
    const float mn = fmaxf(m, m2);
    if (mn == -INFINITY) return;  // both empty
    s = s * __builtin_amdgcn_exp2f((m - mn) * kLog2e) + s2 * __builtin_amdgcn_exp2f((m2 - mn) * kLog2e);
    m = mn;
}

// Workgroup reduction of (m, s); every thread gets the result.
__device__ __forceinline__ void ms_reduce(float& m, float& s, float* sm_m, float* sm_s) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float m2 = __shfl_xor(m, off), s2 = __shfl_xor(s, off);
        ms_add(m, s, m2, s2);
    }
    if (lane_id() == 0) {
        sm_m[wave_id()] = m;
        sm_s[wave_id()] = s;
    }
    __syncthreads();
    m = sm_m[0];
    s = sm_s[0];
#pragma unroll
    for (int k = 1; k < CW; ++k) ms_add(m, s, sm_m[k], sm_s[k]);
    __syncthreads();
}

__device__ __forceinline__ void ms_push(float& m, float& s, float x) {
    if (x > m) {
        s = s * __builtin_amdgcn_exp2f((m - x) * kLog2e) + 1.f;
        m = x;
    } else if (x != -INFINITY) {  // a -inf logit adds nothing (and -inf - -inf is NaN)
        s += __builtin_amdgcn_exp2f((x - m) * kLog2e);
    }
}

// NV = 16-byte vectors per thread held in registers (0: looped path).
// MODE: CE_FWD loss only; CE_BWD gradient only; CE_BOTH both from one read of
// the row (grad_loss NULL: 1 for every row; grad may be the logits themselves:
// every element is read before any is written, by the thread that writes it).
enum { CE_FWD = 0, CE_BWD = 1, CE_BOTH = 2 };
template <int NV, int MODE>
__global__ void __launch_bounds__(CNT) ce_kernel(const bf16* logits,
                                                 const int32_t* __restrict__ targets,
                                                 const float* __restrict__ grad_loss,
                                                 float* __restrict__ loss,
                                                 bf16* grad, long B, long V,
                                                 float eps) {
    __shared__ float sm_m[CW], sm_s[CW];
    const long row = blockIdx.x;
    const bf16* z = logits + row * V;
    const long t = targets[row];
    const bool tok = t >= 0 && t < V;
    // the target's logit, read before anything of the row can be overwritten
    const float zt = (MODE != CE_BWD && threadIdx.x == 0 && tok) ? (float)z[t] : 0.f;
    float m = -INFINITY, s = 0.f;
    bf16x8 xv[NV > 0 ? NV : 1];
    if constexpr (NV > 0) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const long c = (long)j * CNT + threadIdx.x;
            if (c < V / 8) {
                xv[j] = reinterpret_cast<const bf16x8*>(z)[c];
#pragma unroll
                for (int i = 0; i < 8; ++i) ms_push(m, s, (float)xv[j][i]);
            }
        }
    } else {
        for (long c = threadIdx.x; c < V; c += CNT) ms_push(m, s, (float)z[c]);
    }
    ms_reduce(m, s, sm_m, sm_s);
    const float lse = m + __logf(s);
    const float inv_b = 1.0f / (float)B;
    if constexpr (MODE != CE_BWD) {
        if (threadIdx.x == 0) {
            const float l = (1.f - eps) * (lse - zt) + eps * logf((float)V);
            loss[row] = tok ? l * inv_b : NAN;
        }
    }
    if constexpr (MODE != CE_FWD) {
        // softmax_j = exp(z_j - lse); dz_j = coef (softmax_j - [j = t])
        const float gl = (MODE == CE_BOTH && !grad_loss) ? 1.f : grad_loss[row];
        const float coef = tok ? gl * (1.f - eps) * inv_b : 0.f;
        bf16* g = grad + row * V;
        if constexpr (NV > 0) {
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const long c = (long)j * CNT + threadIdx.x;
                if (c < V / 8) {
                    bf16x8 o;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const float p = __builtin_amdgcn_exp2f(((float)xv[j][i] - lse) * kLog2e);
                        const float hot = (c * 8 + i == t) ? 1.f : 0.f;
                        o[i] = (bf16)(coef * (p - hot));
                    }
                    reinterpret_cast<bf16x8*>(g)[c] = o;
                }
            }
        } else {
            for (long c = threadIdx.x; c < V; c += CNT) {
                const float p = __builtin_amdgcn_exp2f(((float)z[c] - lse) * kLog2e);
                g[c] = (bf16)(coef * (p - (c == t ? 1.f : 0.f)));
            }
        }
    }
}

template <int MODE>
static int ce_launch(const bf16* z, const int32_t* t, const float* gl, float* loss, bf16* g,
                     long B, long V, float eps, hipStream_t st) {
    const bool vec =
        V % 8 == 0 && ((uintptr_t)z & 15) == 0 && (MODE == CE_FWD || ((uintptr_t)g & 15) == 0);
    const long nvec = (V / 8 + CNT - 1) / CNT;  // vectors per thread
    const char* name = MODE == CE_FWD   ? "cross_entropy_fwd"
                       : MODE == CE_BWD ? "cross_entropy_bwd"
                                        : "cross_entropy_fwd_bwd";
    const dim3 grid((unsigned)B), block(CNT);
#define CE_CASE(nv)                                                                         \
    if (vec && nvec <= nv) {                                                                \
        EFLA_LAUNCH(name, (ce_kernel<nv, MODE>), grid, block, st, z, t, gl, loss, g, B, V, eps); \
        return (int)hipPeekAtLastError();                                                   \
    }
    CE_CASE(1) CE_CASE(2) CE_CASE(4) CE_CASE(8)
#undef CE_CASE
    EFLA_LAUNCH(name, (ce_kernel<0, MODE>), grid, block, st, z, t, gl, loss, g, B, V, eps);
    return (int)hipPeekAtLastError();
}

static int ce_check(const void* logits, const int32_t* targets, size_t batch, size_t vocab,
                    float eps) {
    if (batch == 0) return kSuccess;
    if (!logits || !targets || vocab == 0) return kInvalidValue;
    if (!(eps >= 0.f && eps < 1.f)) return kInvalidValue;
    if (batch > 0x7FFFFFFFull || vocab > ((size_t)1 << 31)) return kInvalidConfiguration;
    size_t n;
    if (!mul_ok(batch, vocab, &n)) return kInvalidConfiguration;
    return kSuccess;
}

static int emb_launch(const int32_t* indices, const void* weight, void* output, size_t n,
                      size_t D, long vocab, hipStream_t st) {
    if (n == 0) return kSuccess;
    if (!indices || !weight || !output || D == 0) return kInvalidValue;
    size_t e;
    if (!mul_ok(n, D, &e) || n > ((size_t)1 << 36)) return kInvalidConfiguration;
    const int vec = D % 8 == 0 && (((uintptr_t)weight | (uintptr_t)output) & 15) == 0;
    const size_t grid = (n + ENT / kWave - 1) / (ENT / kWave);
    EFLA_LAUNCH("embedding_fwd", emb_fwd_kernel, dim3((unsigned)grid), dim3(ENT), st, indices,
                (const bf16*)weight, (bf16*)output, (long)n, (long)D, vocab, vec);
    return (int)hipPeekAtLastError();
}

}  // namespace lm
}  // namespace efla

using namespace efla;

extern "C" int embedding_forward_hip(const int32_t* indices, const void* weight, void* output,
                                     size_t num_indices, size_t embedding_dim,
                                     hipStream_t stream) {
    return lm::emb_launch(indices, weight, output, num_indices, embedding_dim, -1, stream);
}

extern "C" int embedding_forward_checked_hip(const int32_t* indices, const void* weight,
                                             void* output, size_t num_indices,
                                             size_t num_embeddings, size_t embedding_dim,
                                             hipStream_t stream) {
    if (num_embeddings == 0 && num_indices != 0) return kInvalidValue;
    return lm::emb_launch(indices, weight, output, num_indices, embedding_dim,
                          (long)num_embeddings, stream);
}

extern "C" int embedding_backward_hip(const void* grad_output, const int32_t* indices,
                                      float* grad_weight, size_t num_indices,
                                      size_t num_embeddings, size_t embedding_dim,
                                      hipStream_t stream) {
    if (num_indices == 0) return kSuccess;
    if (!grad_output || !indices || !grad_weight || embedding_dim == 0 || num_embeddings == 0)
        return kInvalidValue;
    size_t e;
    if (!mul_ok(num_indices, embedding_dim, &e) || !mul_ok(num_embeddings, embedding_dim, &e) ||
        num_indices > ((size_t)1 << 36))
        return kInvalidConfiguration;
    const size_t grid = (num_indices + lm::ENT / kWave - 1) / (lm::ENT / kWave);
    EFLA_LAUNCH("embedding_bwd", lm::emb_bwd_kernel, dim3((unsigned)grid), dim3(lm::ENT), stream,
                (const bf16*)grad_output, indices, grad_weight, (long)num_indices,
                (long)embedding_dim, (long)num_embeddings);
    return (int)hipPeekAtLastError();
}

extern "C" int cross_entropy_forward_hip(const void* logits, const int32_t* targets, void* loss,
                                         size_t batch_size, size_t vocab_size,
                                         float label_smoothing, hipStream_t stream) {
    int rc = lm::ce_check(logits, targets, batch_size, vocab_size, label_smoothing);
    if (rc != kSuccess || batch_size == 0) return rc;
    if (!loss) return kInvalidValue;
    return lm::ce_launch<lm::CE_FWD>((const bf16*)logits, targets, nullptr, (float*)loss, nullptr,
                                (long)batch_size, (long)vocab_size, label_smoothing, stream);
}

extern "C" int cross_entropy_backward_hip(const void* grad_loss, const void* logits,
                                          const int32_t* targets, void* grad_logits,
                                          size_t batch_size, size_t vocab_size,
                                          float label_smoothing, hipStream_t stream) {
    int rc = lm::ce_check(logits, targets, batch_size, vocab_size, label_smoothing);
    if (rc != kSuccess || batch_size == 0) return rc;
    if (!grad_loss || !grad_logits) return kInvalidValue;
    return lm::ce_launch<lm::CE_BWD>((const bf16*)logits, targets, (const float*)grad_loss,
                                     nullptr, (bf16*)grad_logits, (long)batch_size,
                                     (long)vocab_size, label_smoothing, stream);
}

extern "C" int cross_entropy_forward_backward_hip(const void* logits, const int32_t* targets,
                                                  const float* grad_loss, float* loss,
                                                  void* grad_logits, size_t batch_size,
                                                  size_t vocab_size, float label_smoothing,
                                                  hipStream_t stream) {
    int rc = lm::ce_check(logits, targets, batch_size, vocab_size, label_smoothing);
    if (rc != kSuccess || batch_size == 0) return rc;
    if (!loss || !grad_logits) return kInvalidValue;
    return lm::ce_launch<lm::CE_BOTH>((const bf16*)logits, targets, grad_loss, loss,
                                      (bf16*)grad_logits, (long)batch_size, (long)vocab_size,
                                      label_smoothing, stream);
}
