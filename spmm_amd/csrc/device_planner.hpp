// device_planner.hpp -- the row kernel's task list built on the GPU from a
// device-resident CSR (tca_spmm_plan_create_device), with no host copy of
// the structure.  It reproduces plan_rows (planner.cpp) exactly: rows are
// ordered longest first with ties by row id (a stable descending radix sort
// of the row lengths), and each row's place in that order fixes its tasks:
//   [0, 4 W)              the 4 quarters of the W wide rows,
//   [4 W, 4 W + S)        the segments of the long rows (S in all),
//   [4 W + S, .. + R)     one task per medium row,
//   then                  groups of multi_group_rows(slots) consecutive short
//                         rows, and groups of kZeroRows empty rows.
// Long rows come first in the order, then wide, medium and short rows, so
// the category boundaries are three positions in the sorted lengths.  The
// sort keys are length + 1, and 0 for the rows of the windows routed to the
// matrix cores, which so sort last and are left out (the first Mp rows of
// the order are planned).
//
// MFMA windows (plan_mfma in planner.cpp, the same routing through
// route_windows) from per-window statistics computed here: the column union
// of each 128-row window as a bitmap, its size and the exclusive popcount
// prefix of its words (a column's condensed position is the prefix of its
// word plus the set bits below it in the word), and the nonzeros of every
// 32-column condensed step.  For the routed windows the dense-tile
// positions of the nonzeros (natural column order, or condensed) and the B
// row offsets of the condensed columns are written here too.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "planner.hpp"
#include "mfma_common.hpp"

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

// keys = row lengths + 1 (0 for rows of routed windows: wmap[r / 128] >= 0,
// and for rows of taken panels: in_panel[r] != 0), vals = row ids (the radix
// sort's input).  wmap and in_panel may be NULL.
__global__ void dp_lengths_kernel(const int* __restrict__ rowptr, int M, const int* __restrict__ wmap,
                                  const uint8_t* __restrict__ in_panel, uint32_t* __restrict__ keys,
                                  int* __restrict__ rows) {
    for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < M; r += gridDim.x * blockDim.x) {
        const bool tiles = (wmap && wmap[r / kDmaWinRows] >= 0) || (in_panel && in_panel[r]);
        keys[r] = tiles ? 0u : static_cast<uint32_t>(rowptr[r + 1] - rowptr[r]) + 1u;
        rows[r] = r;
    }
}

// Boundaries in the first M descending keys (length + 1): out[0] = rows
// longer than wide_len, out[1] = longer than row_len, out[2] = longer than
// max(multi_max, 0), out[3] = non-empty rows.
__global__ void dp_bounds_kernel(const uint32_t* __restrict__ len, int M, int wide_len, int row_len, int multi_max,
                                 int* __restrict__ out) {
    const int th[4] = {wide_len, row_len, max(multi_max, 0), 0};
    const int k = threadIdx.x;
    if (k >= 4) return;
    int lo = 0, hi = M;  // first index whose length <= th[k]
    while (lo < hi) {
        const int mid = lo + (hi - lo) / 2;
        if (static_cast<int64_t>(len[mid]) - 1 > th[k]) lo = mid + 1;
        else hi = mid;
    }
    out[k] = lo;
}

// segments of each long row (n_long of them, the first in the order)
__global__ void dp_nseg_kernel(const uint32_t* __restrict__ len, int n_long, int seg_len, int* __restrict__ nseg) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n_long; i += gridDim.x * blockDim.x)
        nseg[i] = (static_cast<int>(len[i]) - 1 + seg_len - 1) / seg_len;
}

struct DpEmitArgs {
    const int* rowptr;
    const uint32_t* len;  // sorted keys (length + 1)
    const int* rows;      // rows in that order
    const int* segoff;    // first segment slot of each long row (exclusive sum)
    int4* tasks;
    int* perm;
    int4* longrows;
    int M, n_long, end_wide, end_row, end_nz, group, seg_total;  // M: the rows planned (Mp); group: rows per multi task
};

// Every row of the order writes its own tasks (see the file comment).
__global__ void dp_emit_kernel(DpEmitArgs a) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < a.M; i += gridDim.x * blockDim.x) {
        const int r = a.rows[i];
        const int beg = a.rowptr[r];
        const int64_t L = static_cast<int64_t>(a.len[i]) - 1;
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
            // short rows in groups of `group`, then empty rows in groups of kZeroRows
            const int k = i - a.end_row;
            a.perm[k] = r;
            const int base = 4 * n_wide + a.seg_total + (a.end_row - a.end_wide);
            if (i < a.end_nz) {
                if (k % a.group == 0)
                    a.tasks[base + k / a.group] = make_int4(k, min(a.group, a.end_nz - i), static_cast<int>(L), kTaskMulti);
            } else {
                const int k0 = i - a.end_nz;
                if (k0 % kZeroRows == 0)
                    a.tasks[base + (a.end_nz - a.end_row + a.group - 1) / a.group + k0 / kZeroRows] =
                        make_int4(k, min(kZeroRows, a.M - i), 0, kTaskMulti);
            }
        }
    }
}

// ---------------- launch order of the segments (order_row_tasks) ----------------

// Key of segment task i: the column of its middle nonzero (the host's sort key).
__global__ void dp_segkey_kernel(const int4* __restrict__ tasks, int first, int ns, const int* __restrict__ colidx,
                                 uint32_t* __restrict__ key, int* __restrict__ idx) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < ns; i += gridDim.x * blockDim.x) {
        const int4 t = tasks[first + i];
        key[i] = static_cast<uint32_t>(colidx[t.y + (t.z - t.y) / 2]);
        idx[i] = first + i;
    }
}

// Slots outside the segment queues: wide tasks in place ([0, nw)), idle
// slots where the queues' blocks go ([nw, 4 b_end)), then the row and multi
// tasks in order, idle slots to a whole workgroup.
__global__ void dp_order_fill_kernel(int* __restrict__ order, int n_slots, int nw, int ns, int rest, int b_end) {
    for (int k = blockIdx.x * blockDim.x + threadIdx.x; k < n_slots; k += gridDim.x * blockDim.x) {
        int v = -1;
        if (k < nw) v = k;
        else if (k >= 4 * b_end && k - 4 * b_end < rest) v = nw + ns + (k - 4 * b_end);
        order[k] = v;
    }
}

// Segment j of the column order: queue x holds [ns x / 8, ns (x + 1) / 8);
// its k-th entry goes to slot k % 4 of the (k / 4)-th workgroup on XCD x
// after the wide rows' workgroups (workgroup b runs on XCD b % 8).
__global__ void dp_order_seg_kernel(const int* __restrict__ sorted_idx, int ns, int b0, int* __restrict__ order) {
    for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < ns; j += gridDim.x * blockDim.x) {
        int x = kXcds - 1;
        while (static_cast<int64_t>(ns) * x / kXcds > j) x--;
        const int k = j - static_cast<int>(static_cast<int64_t>(ns) * x / kXcds);
        const int b = b0 + ((x - b0) % kXcds + kXcds) % kXcds + kXcds * (k / 4);
        order[4 * b + k % 4] = sorted_idx[j];
    }
}

// ---------------- MFMA windows ----------------

// Column-union bitmaps: bit c % 32 of bm[w * kw + c / 32] for every column c
// of window w (rows 128 w .. 128 w + 127).  One wavefront per row.
__global__ void dm_bitmap_kernel(const int* __restrict__ rowptr, const int* __restrict__ colidx, int M, int kw,
                                 uint32_t* __restrict__ bm) {
    const int lane = threadIdx.x & 63;
    const int waves = (gridDim.x * blockDim.x) >> 6;
    for (int r = (blockIdx.x * blockDim.x + threadIdx.x) >> 6; r < M; r += waves) {
        uint32_t* const b = bm + static_cast<size_t>(r / kDmaWinRows) * kw;
        for (int j = rowptr[r] + lane; j < rowptr[r + 1]; j += 64) {
            const int c = colidx[j];
            atomicOr(b + (c >> 5), 1u << (c & 31));
        }
    }
}

// One workgroup (256 threads) per window: wrow[w] = rowptr[128 w] (and
// wrow[nw] = rowptr[M]), wordpre = exclusive popcount prefix of the window's
// words, ucount[w] = the union size.
__global__ __launch_bounds__(256) void dm_union_kernel(const int* __restrict__ rowptr, int M, int nw, int kw,
                                                       const uint32_t* __restrict__ bm, int* __restrict__ wordpre,
                                                       int* __restrict__ ucount, int* __restrict__ wrow) {
    const int w = blockIdx.x;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    __shared__ int part[4];
    __shared__ int carry;
    if (t == 0) {
        carry = 0;
        wrow[w] = rowptr[w * kDmaWinRows];
        if (w == nw - 1) wrow[nw] = rowptr[M];
    }
    __syncthreads();
    const size_t wb = static_cast<size_t>(w) * kw;
    for (int base = 0; base < kw; base += 256) {
        const int i = base + t;
        const int v = i < kw ? __popc(bm[wb + i]) : 0;
        int x = v;  // inclusive scan within the wavefront
        for (int d = 1; d < 64; d <<= 1) {
            const int y = __shfl_up(x, d, 64);
            if (lane >= d) x += y;
        }
        if (lane == 63) part[wv] = x;
        __syncthreads();
        int off = carry;
        for (int k = 0; k < wv; k++) off += part[k];
        if (i < kw) wordpre[wb + i] = off + x - v;
        __syncthreads();
        if (t == 255) carry = off + x;
        __syncthreads();
    }
    if (t == 0) ucount[w] = carry;
}

// condensed position of column c in the window whose words start at wb
__device__ inline int dm_cpos(const uint32_t* __restrict__ bm, const int* __restrict__ wordpre, size_t wb, int c) {
    const uint32_t word = bm[wb + (c >> 5)];
    return wordpre[wb + (c >> 5)] + __popc(word & ((1u << (c & 31)) - 1u));
}

// Nonzeros per condensed step: cnt[w * kw + cpos / 32] (a window has at most
// kw steps).  One wavefront per row.
__global__ void dm_stepcount_kernel(const int* __restrict__ rowptr, const int* __restrict__ colidx, int M, int kw,
                                    const uint32_t* __restrict__ bm, const int* __restrict__ wordpre,
                                    int* __restrict__ cnt) {
    const int lane = threadIdx.x & 63;
    const int waves = (gridDim.x * blockDim.x) >> 6;
    for (int r = (blockIdx.x * blockDim.x + threadIdx.x) >> 6; r < M; r += waves) {
        const size_t wb = static_cast<size_t>(r / kDmaWinRows) * kw;
        for (int j = rowptr[r] + lane; j < rowptr[r + 1]; j += 64)
            atomicAdd(cnt + wb + (dm_cpos(bm, wordpre, wb, colidx[j]) >> 5), 1);
    }
}

// Most nonzeros in one step of each window (one workgroup per window).
__global__ __launch_bounds__(256) void dm_stepmax_kernel(const int* __restrict__ cnt, int kw,
                                                         const int* __restrict__ ucount, int* __restrict__ maxper) {
    const int w = blockIdx.x, t = threadIdx.x;
    const int steps = (ucount[w] + 31) / 32;
    int m = 0;
    for (int s = t; s < steps; s += 256) m = max(m, cnt[static_cast<size_t>(w) * kw + s]);
    __shared__ int red[256];
    red[t] = m;
    __syncthreads();
    for (int d = 128; d > 0; d >>= 1) {
        if (t < d) red[t] = max(red[t], red[t + d]);
        __syncthreads();
    }
    if (t == 0) maxper[w] = red[0];
}

struct DmEntryArgs {
    const int* rowptr;
    const int* colidx;
    const uint32_t* bm;
    const int* wordpre;
    const int* wmap;    // [window] routed index, -1 for none
    const int* wgbase;  // [routed index] first global step
    uint32_t* keys;     // [nonzero] half index in the dense tiles, 0xffffffff outside routed windows
    int* vals;          // [nonzero] its index
    int M, kw;
    int natural;        // windows span all of K in column order
};

// Dense-tile position of every nonzero (the dense pack's list, sorted
// afterwards).  One wavefront per row.
__global__ void dm_entries_kernel(DmEntryArgs a) {
    const int lane = threadIdx.x & 63;
    const int waves = (gridDim.x * blockDim.x) >> 6;
    for (int r = (blockIdx.x * blockDim.x + threadIdx.x) >> 6; r < a.M; r += waves) {
        const int w = r / kDmaWinRows;
        const int t = a.wmap[w];
        const size_t wb = static_cast<size_t>(w) * a.kw;
        for (int j = a.rowptr[r] + lane; j < a.rowptr[r + 1]; j += 64) {
            uint32_t key = 0xffffffffu;
            if (t >= 0) {
                const int c = a.colidx[j];
                const int pc = a.natural ? c : dm_cpos(a.bm, a.wordpre, wb, c);
                const uint32_t g = static_cast<uint32_t>(a.wgbase[t] + (pc >> 5));
                key = g * static_cast<uint32_t>(kDmaATile) + static_cast<uint32_t>(a_cell(r - w * kDmaWinRows, pc & 31));
            }
            a.keys[j] = key;
            a.vals[j] = j;
        }
    }
}

// B row byte offsets (row * N * 2) of the condensed columns of the routed
// windows, step by step; ucols is prefilled with 0xff bytes (padding).
__global__ void dm_ucols_kernel(int nw, int kw, const uint32_t* __restrict__ bm, const int* __restrict__ wordpre,
                                const int* __restrict__ wmap, const int* __restrict__ wgbase, int N,
                                uint32_t* __restrict__ ucols) {
    const int64_t total = static_cast<int64_t>(nw) * kw;
    for (int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < total;
         q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int w = static_cast<int>(q / kw), i = static_cast<int>(q % kw);
        const int t = wmap[w];
        if (t < 0) continue;
        uint32_t word = bm[q];
        int pos = wordpre[q];
        uint32_t* const out = ucols + static_cast<size_t>(wgbase[t]) * 32;
        while (word) {
            const int b = __ffs(word) - 1;
            word &= word - 1;
            out[pos++] = static_cast<uint32_t>(32 * i + b) * static_cast<uint32_t>(N) * 2u;
        }
    }
}

// Compaction of the dense tiles (the host planner's rule, tca_spmm.hip):
// per global step, bit L of mask[step * 8 + b] is set when fragment cell
// (row block b, lane L) holds an entry.  `pos` are the sorted dense-tile half
// indices of the routed nonzeros (step * kDmaATile + a_cell).
__global__ void dm_cmask_kernel(const uint32_t* __restrict__ pos, int n, unsigned long long* __restrict__ mask) {
    for (int x = blockIdx.x * blockDim.x + threadIdx.x; x < n; x += gridDim.x * blockDim.x) {
        const uint32_t g = pos[x] / kDmaATile, c = (pos[x] % kDmaATile) / 8;
        atomicOr(&mask[static_cast<size_t>(g) * 8 + c / 64], 1ull << (c % 64));
    }
}

// flag |= 1 when a step has more non-empty cells than a compacted step holds
// (cells - 1: the last cell stays zero for the empty lanes).
__global__ void dm_cfit_kernel(const unsigned long long* __restrict__ mask, int64_t steps, int cells,
                               int* __restrict__ flag) {
    for (int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; g < steps;
         g += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        int tot = 0;
#pragma unroll
        for (int b = 0; b < 8; b++) tot += __popcll(mask[g * 8 + b]);
        if (tot > cells - 1) atomicOr(flag, 1);
    }
}

// Compacted position of every entry, in place: the step's base, the rank of
// its cell among the step's non-empty cells (in cell order), the half within
// the cell.  Ranks grow with the cell, so the positions stay sorted.
__global__ void dm_cpos_kernel(uint32_t* __restrict__ pos, int n, const unsigned long long* __restrict__ mask,
                               int cells) {
    for (int x = blockIdx.x * blockDim.x + threadIdx.x; x < n; x += gridDim.x * blockDim.x) {
        const uint32_t g = pos[x] / kDmaATile, h = pos[x] % kDmaATile, c = h / 8;
        const unsigned long long* m = mask + static_cast<size_t>(g) * 8;
        uint32_t rank = 0;
        for (uint32_t b = 0; b < c / 64; b++) rank += static_cast<uint32_t>(__popcll(m[b]));
        rank += static_cast<uint32_t>(__popcll(m[c / 64] & ((1ull << (c % 64)) - 1ull)));
        pos[x] = g * static_cast<uint32_t>(cells * 8) + rank * 8u + h % 8;
    }
}

}  // namespace tca
