// Affine combine of EFLA chunk states: the composition the reference's
// efla_chunked_scan_cuda (efla.cu:711-748) and the empty
// ChunkedScan.prefixScan (src/model/efla.zig:473-484) stand in for.
//
// Over a segment of tokens the state recurrence
//   S_t = (I - c_t k_t k_t^T) S_{t-1} + c_t k_t v_t^T
// is affine in the incoming state: S_out = A S_in + B, with A = prod_t
// (I - c_t k_t k_t^T) (d_k x d_k) and B the segment's final state from zero
// (d_k x d_v).  Segments therefore combine by
//   S_i = A_i S_{i-1} + B_i,
// which this entry applies in place over an array of segment states, in the
// reference's calling form (a host array of per-chunk device pointers, one
// launch per step).  A segment's A is what the chunked forward returns as its
// final state when started from S_0 = I with v = 0 (d_v = d_k).
//
// fp32 throughout.  One workgroup per (state, 64-column block of S_i): the
// previous state's column block sits in LDS, each thread accumulates 16
// outputs over the d_k contraction reading rows of A through the L1.
#include <hip/hip_runtime.h>

#include "../../include/efla_hip.h"
#include "common.hpp"
#include "internal.hpp"

namespace efla {
namespace sscan {

constexpr int NTH = 256;
constexpr int CB = 64;     // columns of S per workgroup
constexpr int MAXK = 256;

// S_cur[h] = A[h] S_prev[h] + S_cur[h] for columns cb*64 .. +63
__global__ void __launch_bounds__(NTH) combine_kernel(const float* __restrict__ A,
                                                      const float* __restrict__ S_prev,
                                                      float* __restrict__ S_cur, int K, int V) {
    __shared__ float sp[MAXK][CB + 1];
    const long h = blockIdx.x;
    const int c0 = blockIdx.y * CB;
    const int nc = min(CB, V - c0);
    const float* Ah = A + h * K * K;
    const float* Ph = S_prev + h * (long)K * V;
    float* Ch = S_cur + h * (long)K * V;
    for (int i = threadIdx.x; i < K * CB; i += NTH) {
        const int r = i / CB, c = i % CB;
        sp[r][c] = c < nc ? Ph[(long)r * V + c0 + c] : 0.f;
    }
    __syncthreads();
    // thread -> column c = tid % 64, rows r = tid / 64 + 4 j
    const int c = threadIdx.x % CB;
    for (int r0 = threadIdx.x / CB; r0 < K; r0 += 4 * 16) {
        float acc[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[j] = 0.f;
        for (int k = 0; k < K; ++k) {
            const float p = sp[k][c];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int r = r0 + 4 * j;
                if (r < K) acc[j] += Ah[(long)r * K + k] * p;
            }
        }
        if (c < nc) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int r = r0 + 4 * j;
                if (r < K) Ch[(long)r * V + c0 + c] += acc[j];
            }
        }
    }
}

}  // namespace sscan
}  // namespace efla

using namespace efla;

extern "C" int efla_affine_state_scan_hip(const float* const* transitions, float* const* states,
                                          size_t num_chunks, size_t num_states,
                                          size_t head_dim_k, size_t head_dim_v,
                                          hipStream_t stream) {
    if (num_chunks == 0 || num_states == 0 || head_dim_k == 0 || head_dim_v == 0)
        return kInvalidValue;
    if (!transitions || !states) return kInvalidValue;
    if (head_dim_k > (size_t)sscan::MAXK || num_states > 0x7FFFFFFFull ||
        head_dim_v > ((size_t)1 << 20))
        return kInvalidConfiguration;
    for (size_t i = 0; i < num_chunks; ++i) {
        if (!states[i]) return kInvalidValue;
        if (i > 0 && !transitions[i]) return kInvalidValue;
    }
    const dim3 grid((unsigned)num_states, (unsigned)((head_dim_v + sscan::CB - 1) / sscan::CB));
    for (size_t i = 1; i < num_chunks; ++i) {
        EFLA_LAUNCH("efla_affine_state_scan", sscan::combine_kernel, grid, dim3(sscan::NTH),
                    stream, transitions[i], (const float*)states[i - 1], states[i],
                    (int)head_dim_k, (int)head_dim_v);
        const hipError_t e = hipPeekAtLastError();
        if (e != hipSuccess) return (int)e;
    }
    return kSuccess;
}
