// device_planner.hpp -- the row kernel's task list built on the GPU from a
// device-resident CSR (tca_spmm_plan_create_device), with no host copy of
// the structure.  It reproduces plan_rows (planner.cpp) exactly: rows are
// ordered longest first with ties by row id (a stable descending radix sort
// of the row lengths), and each row's place in that order fixes its tasks:
//   [0, 4 W)              the 4 quarters of the W wide rows,
//   [4 W, 4 W + S)        the segments of the long rows (S in all),
//   [4 W + S, .. + R)     one task per medium row,
//   then                  groups of `slots` consecutive short rows.
// Long rows come first in the order, then wide, medium and short rows, so
// the category boundaries are three positions in the sorted lengths.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "planner.hpp"

namespace tca {

// CSR checks of tca_csr_validate: rowptr[0] == 0, rowptr[M] == nnz,
// non-decreasing, columns in [0, K) and strictly ascending within a row.
// err bit 1: row offsets, bit 2: a column.  `start` marks the first entry of
// every non-empty row (nnz + 1 bytes, zeroed by the caller).
__global__ void dp_check_rows_kernel(const int* __restrict__ rowptr, int M, int nnz, uint8_t* __restrict__ start,
                                     int* __restrict__ err) {
    for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < M; r += gridDim.x * blockDim.x) {
        const int b = rowptr[r], e = rowptr[r + 1];
        if ((r == 0 && b != 0) || (r == M - 1 && e != nnz) || b > e || b < 0 || e > nnz) {
            atomicOr(err, 1);
            continue;
        }
        if (b < e) start[b] = 1;
    }
}

__global__ void dp_check_cols_kernel(const int* __restrict__ colidx, int nnz, int K, const uint8_t* __restrict__ start,
                                     int* __restrict__ err) {
    for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < nnz; j += gridDim.x * blockDim.x) {
        const int c = colidx[j];
        if (c < 0 || c >= K || (j + 1 < nnz && !start[j + 1] && colidx[j + 1] <= c)) atomicOr(err, 2);
    }
}

// keys = row lengths, vals = row ids (the radix sort's input)
__global__ void dp_lengths_kernel(const int* __restrict__ rowptr, int M, uint32_t* __restrict__ keys,
                                  int* __restrict__ rows) {
    for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < M; r += gridDim.x * blockDim.x) {
        keys[r] = static_cast<uint32_t>(rowptr[r + 1] - rowptr[r]);
        rows[r] = r;
    }
}

// Boundaries in the descending lengths: out[0] = rows longer than wide_len,
// out[1] = longer than row_len, out[2] = longer than multi_max.
__global__ void dp_bounds_kernel(const uint32_t* __restrict__ len, int M, int wide_len, int row_len, int multi_max,
                                 int* __restrict__ out) {
    const int th[3] = {wide_len, row_len, multi_max};
    const int k = threadIdx.x;
    if (k >= 3) return;
    if (th[k] < 0) {
        out[k] = M;
        return;
    }
    int lo = 0, hi = M;  // first index whose length <= th[k]
    while (lo < hi) {
        const int mid = lo + (hi - lo) / 2;
        if (static_cast<int64_t>(len[mid]) > th[k]) lo = mid + 1;
        else hi = mid;
    }
    out[k] = lo;
}

// segments of each long row (n_long of them, the first in the order)
__global__ void dp_nseg_kernel(const uint32_t* __restrict__ len, int n_long, int seg_len, int* __restrict__ nseg) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n_long; i += gridDim.x * blockDim.x)
        nseg[i] = (static_cast<int>(len[i]) + seg_len - 1) / seg_len;
}

struct DpEmitArgs {
    const int* rowptr;
    const uint32_t* len;  // sorted lengths
    const int* rows;      // rows in that order
    const int* segoff;    // first segment slot of each long row (exclusive sum)
    int4* tasks;
    int* perm;
    int4* longrows;
    int M, n_long, end_wide, end_row, slots, seg_total;
};

// Every row of the order writes its own tasks (see the file comment).
__global__ void dp_emit_kernel(DpEmitArgs a) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < a.M; i += gridDim.x * blockDim.x) {
        const int r = a.rows[i];
        const int beg = a.rowptr[r];
        const int64_t L = a.len[i];
        const int n_wide = a.end_wide - a.n_long;
        if (i < a.n_long) {
            const int off = a.segoff[i];
            const int nseg = a.segoff[i + 1] - off;
            a.longrows[i] = make_int4(r, off, nseg, 0);
            for (int s = 0; s < nseg; s++) {
                const int b = beg + static_cast<int>(L * s / nseg);
                const int e = beg + static_cast<int>(L * (s + 1) / nseg);
                a.tasks[4 * n_wide + off + s] = make_int4(i, b, e, kTaskSeg | ((off + s) << 2));
            }
        } else if (i < a.end_wide) {
            const int w = i - a.n_long;
            for (int q = 0; q < 4; q++)
                a.tasks[4 * w + q] = make_int4(r, beg + static_cast<int>(L * q / 4), beg + static_cast<int>(L * (q + 1) / 4),
                                               kTaskWide | (q << 2));
        } else if (i < a.end_row) {
            a.tasks[4 * n_wide + a.seg_total + (i - a.end_wide)] = make_int4(r, beg, beg + static_cast<int>(L), kTaskRow);
        } else {
            const int k = i - a.end_row;
            a.perm[k] = r;
            if (k % a.slots == 0) {
                const int g = k / a.slots;
                const int cnt = min(a.slots, a.M - i);
                a.tasks[4 * n_wide + a.seg_total + (a.end_row - a.end_wide) + g] =
                    make_int4(k, cnt, static_cast<int>(L), kTaskMulti);
            }
        }
    }
}

}  // namespace tca
