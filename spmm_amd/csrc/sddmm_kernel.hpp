// sddmm_kernel.hpp -- kernels of the PyTorch op's backward pass (gfx950).
//
// For C = A * B with A in CSR, the gradients are
//   dL/dB      = A^T * dL/dC         (an SpMM with the transposed plan), and
//   dL/dA[j]   = <dL/dC[row(j), :], B[col(j), :]>   for every nonzero j,
// the second being a sampled dense-dense product (SDDMM) over A's pattern.
// No counterpart in the reference, which has no backward pass.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "row_kernel.hpp"

namespace tca {

constexpr int kSddmmRowsPerBlock = 4;  // one wavefront per row
constexpr int kSddmmCols = 8;          // columns per lane per chunk (chunk = 512 columns)

// out[j] = sum_n G[r, n] * B[colidx[j], n] for the nonzeros j of row r.  The
// row of G is held in registers chunk by chunk; each nonzero's partial sums
// are reduced across the wavefront with xor shuffles in a fixed order and
// chunks are added in column order, so the result does not depend on the
// schedule.
template <typename T>
__global__ __launch_bounds__(64 * kSddmmRowsPerBlock) void sddmm_kernel(const int* __restrict__ rowptr,
                                                                        const int* __restrict__ colidx, int M, int N,
                                                                        const float* __restrict__ G,
                                                                        const T* __restrict__ B,
                                                                        float* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * kSddmmRowsPerBlock + (threadIdx.x >> 6);
    if (r >= M) return;
    const int j0 = rowptr[r], j1 = rowptr[r + 1];
    if (j0 == j1) return;
    const float* g_row = G + static_cast<size_t>(r) * N;
    for (int n0 = 0; n0 < N; n0 += 64 * kSddmmCols) {
        float g[kSddmmCols];
#pragma unroll
        for (int q = 0; q < kSddmmCols; q++) {
            const int c = n0 + 64 * q + lane;
            g[q] = c < N ? g_row[c] : 0.f;
        }
        for (int j = j0; j < j1; j++) {
            const T* b_row = B + static_cast<size_t>(colidx[j]) * N;
            float s = 0.f;
#pragma unroll
            for (int q = 0; q < kSddmmCols; q++) {
                const int c = n0 + 64 * q + lane;
                if (c < N) s += g[q] * to_f32(b_row[c]);
            }
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) s += __shfl_xor(s, d, 64);
            if (lane == 0) out[j] = n0 == 0 ? s : out[j] + s;
        }
    }
}

// out[i] = value perm[i] of `val`, widened to fp32 (A's values in the order
// of the transpose).
template <typename T>
__global__ __launch_bounds__(256) void gather_values_kernel(const int* __restrict__ perm, int n,
                                                            const T* __restrict__ val, float* __restrict__ out) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = to_f32(val[perm[i]]);
}

}  // namespace tca
