// Fixed-order sum of per-workgroup partials: out[c] += sum_b part[b * n + c].
// Workgroup of 256: 16 row groups x 16 lanes of 4 columns (16-byte loads when
// n is a multiple of 4), one 64-column block per workgroup; the 16 row-group
// sums are added in LDS in row-group order, so the result does not depend on
// scheduling.  Internal linkage: each source file that launches it has its
// own copy.
#pragma once
#include <hip/hip_runtime.h>

#include "common.hpp"

namespace efla {

static __global__ void __launch_bounds__(256) partial_colsum_add_kernel(const float* __restrict__ part,
                                                                 int nblk, long n,
                                                                 float* __restrict__ out) {
    __shared__ float acc[16][64 + 1];
    const int q = threadIdx.x & 15, rg = threadIdx.x >> 4;
    const long c0 = (long)blockIdx.x * 64 + 4 * q;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    if (n % 4 == 0 && c0 + 4 <= n) {
#pragma unroll 4
        for (int b = rg; b < nblk; b += 16) {
            const floatx4 v = *reinterpret_cast<const floatx4*>(part + (long)b * n + c0);
#pragma unroll
            for (int i = 0; i < 4; ++i) s[i] += v[i];
        }
    } else {
        for (int b = rg; b < nblk; b += 16)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (c0 + i < n) s[i] += part[(long)b * n + c0 + i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[rg][4 * q + i] = s[i];
    __syncthreads();
    if (threadIdx.x < 64) {
        const long c = (long)blockIdx.x * 64 + threadIdx.x;
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < 16; ++k) t += acc[k][threadIdx.x];
        if (c < n) out[c] += t;
    }
}

inline dim3 partial_colsum_grid(long n) { return dim3((unsigned)((n + 63) / 64)); }

}  // namespace efla
