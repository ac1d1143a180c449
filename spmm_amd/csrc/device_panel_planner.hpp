// device_panel_planner.hpp -- the row panels of the panel kernel planned on
// the GPU (tca_spmm_plan_create_device), equal entry for entry to the host's
// plan_panels (planner.cpp).
//
// Candidate panel q holds rows q R .. q R + R - 1 of the longest-first order
// (the device row planner's stable descending sort of the row lengths,
// restricted to rows with nonzeros outside MFMA windows); its k-th row goes
// to slot ((k % G) / 4 * rpg + k / G) * 4 + k % 4 (G = waves * 4), as on the
// host.
//   dpp_union_kernel  one workgroup per candidate: the sorted column union
//                     through a bitmap in LDS (column chunks of 2^19 starting
//                     at the smallest column not yet seen), the union's
//                     columns, each nonzero's position in the union, the
//                     panel's nonzeros and union size.  The host then decides
//                     which candidates are taken (reuse rule of plan_panels).
//   tile cuts         the greedy cut of plan_panels (a tile ends before
//                     the column where some slot would get its 17th nonzero,
//                     or at P columns) through a suffix minimum over union
//                     positions (dpp_m_kernel, dpp_walk_kernel); then per
//                     tile its union positions and staged rows
//                     (dpp_tile_fill_kernel) and per nonzero its position,
//                     its run's count and the units' cursors
//                     (dpp_runs_kernel).
//   dpp_units_kernel  one wavefront per taken panel: the unit cuts (tiles
//                     split at multiples of nnz / units), as on the host.
// The host does the exclusive sums over panels (small arrays) and the XCD
// launch order of the units (order_unit_spans) from each unit's first and
// last staged column.
#pragma once

#include <hip/hip_runtime.h>
#include <limits.h>
#include <stdint.h>

#include "planner.hpp"

namespace tca {

constexpr int kDppChunkWords = 16384;  // bitmap words per column chunk (2^19 columns, 64 KiB of LDS)
constexpr int kDppThreads = 1024;      // union kernel
constexpr int kDppUnroll = 16;         // union kernel: loads of 64 columns in flight per wavefront
constexpr int kDppR = kPanelWaves * 4 * kPanelRpg;
constexpr int kDppG = kPanelWaves * 4;
constexpr int kDppCntDwords = kPanelWaves * kPanelCntRows;  // count dwords of one tile

// Row k of a panel -> its slot, and back.
__host__ __device__ inline int dpp_slot_of(int k) {
    const int gi = k % kDppG, i = k / kDppG;
    return ((gi >> 2) * kPanelRpg + i) * 4 + (gi & 3);
}
__host__ __device__ inline int dpp_k_of(int s) {
    const int wave = s / (4 * kPanelRpg), i = (s / 4) % kPanelRpg, g = s % 4;
    return i * kDppG + wave * 4 + g;
}

// Block-wide min / sum / exclusive sum (every thread of the block calls
// them; `red` holds one int per wavefront).
template <int kThreads>
__device__ inline int dpp_block_min(int v, int* red) {
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    int r = red[0];
    for (int i = 1; i < kThreads / 64; i++) r = min(r, red[i]);
    return r;
}
template <int kThreads>
__device__ inline int dpp_block_sum(int v, int* red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    int r = 0;
    for (int i = 0; i < kThreads / 64; i++) r += red[i];
    return r;
}
template <int kThreads>
__device__ inline int dpp_block_exscan(int v, int* red, int* total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int x = v;  // inclusive scan within the wavefront
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    __syncthreads();
    if (lane == 63) red[w] = x;
    __syncthreads();
    int before = 0, all = 0;
    for (int i = 0; i < kThreads / 64; i++) {
        if (i < w) before += red[i];
        all += red[i];
    }
    *total = all;
    return before + x - v;
}

struct DppUnionArgs {
    const int* rowptr;
    const int* colidx;
    const int* rows;    // rows in the longest-first order
    const int* lenpre;  // [k]: sum of the lengths of the order's first k rows (union scratch base)
    int n_nz;           // rows with nonzeros: the first n_nz of the order
    int* ucols;         // [lenpre[q R] + u]: column u of candidate q's sorted union
    int* upos;          // [CSR index]: the nonzero's position in its panel's union
    int* ucount;        // [q]: union size
    int* pnnz;          // [q]: nonzeros
};

__global__ __launch_bounds__(kDppThreads) void dpp_union_kernel(DppUnionArgs a) {
    __shared__ uint32_t bm[kDppChunkWords];
    __shared__ int wpre[kDppChunkWords];
    __shared__ int cur[kDppR], nxt[kDppR], ends[kDppR];
    __shared__ int red[kDppThreads / 64];
    const int q = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int first = q * kDppR;
    const int cnt = min(kDppR, a.n_nz - first);
    int mylen = 0;
    for (int k = tid; k < cnt; k += kDppThreads) {
        const int r = a.rows[first + k];
        cur[k] = a.rowptr[r];
        ends[k] = a.rowptr[r + 1];
        mylen += ends[k] - cur[k];
    }
    const int nnzq = dpp_block_sum<kDppThreads>(mylen, red);  // (its barriers also publish cur / ends)
    const int ub = a.lenpre[first];
    int total = 0;
    for (;;) {
        // the chunk starts at the smallest column not yet seen
        int mn = INT_MAX;
        for (int k = tid; k < cnt; k += kDppThreads)
            if (cur[k] < ends[k]) mn = min(mn, a.colidx[cur[k]]);
        mn = dpp_block_min<kDppThreads>(mn, red);
        if (mn == INT_MAX) break;
        const int64_t c0 = mn, c1 = c0 + 32 * kDppChunkWords;
        for (int w = tid; w < kDppChunkWords; w += kDppThreads) bm[w] = 0u;
        __syncthreads();
        // one wavefront per row: its nonzeros below c1 (a prefix of what is
        // left: columns ascend), kDppUnroll loads of 64 in flight per step
        for (int k = wave; k < cnt; k += kDppThreads / 64) {
            int j = cur[k];
            const int e = ends[k];
            for (;;) {
                int c[kDppUnroll];
#pragma unroll
                for (int u = 0; u < kDppUnroll; u++) {
                    const int jj = j + u * 64 + lane;
                    c[u] = jj < e ? a.colidx[jj] : INT_MAX;
                }
                int n = 0;
#pragma unroll
                for (int u = 0; u < kDppUnroll; u++) {
                    const bool ok = c[u] < c1;  // (INT_MAX past the row: c1 <= INT_MAX, K < 2^31 - 2^19 checked by the host)
                    if (ok) {
                        const int x = static_cast<int>(c[u] - c0);
                        atomicOr(&bm[x >> 5], 1u << (x & 31));
                    }
                    n += __popcll(__ballot(ok));
                }
                j += n;
                if (n < 64 * kDppUnroll) break;
            }
            if (lane == 0) nxt[k] = j;
        }
        __syncthreads();
        // exclusive popcount prefix of the words (16 per thread) and the union's columns
        constexpr int kPer = kDppChunkWords / kDppThreads;
        int loc = 0;
        for (int i = 0; i < kPer; i++) loc += __popc(bm[tid * kPer + i]);
        int chunk_total = 0;
        int run = total + dpp_block_exscan<kDppThreads>(loc, red, &chunk_total);
        for (int i = 0; i < kPer; i++) {
            const int w = tid * kPer + i;
            const uint32_t bits = bm[w];
            wpre[w] = run;
            uint32_t m = bits;
            int r = run;
            while (m) {
                const int b = __ffs(m) - 1;
                a.ucols[ub + r] = static_cast<int>(c0) + w * 32 + b;
                r++;
                m &= m - 1u;
            }
            run += __popc(bits);
        }
        __syncthreads();
        // union positions of this chunk's nonzeros
        for (int k = wave; k < cnt; k += kDppThreads / 64) {
            const int e = nxt[k];
            for (int j0 = cur[k]; j0 < e; j0 += 64 * kDppUnroll) {
                int c[kDppUnroll];
#pragma unroll
                for (int u = 0; u < kDppUnroll; u++) {
                    const int j = j0 + u * 64 + lane;
                    c[u] = j < e ? a.colidx[j] - static_cast<int>(c0) : 0;
                }
#pragma unroll
                for (int u = 0; u < kDppUnroll; u++) {
                    const int j = j0 + u * 64 + lane;
                    const int x = c[u];
                    if (j < e) a.upos[j] = wpre[x >> 5] + __popc(bm[x >> 5] & ((1u << (x & 31)) - 1u));
                }
            }
        }
        total += chunk_total;
        __syncthreads();
        for (int k = tid; k < cnt; k += kDppThreads) cur[k] = nxt[k];
        __syncthreads();
    }
    if (tid == 0) {
        a.ucount[q] = total;
        a.pnnz[q] = nnzq;
    }
}

// Rows of the taken panels: flag = 1 (they leave the row kernel's plan).
__global__ void dpp_mark_kernel(const int* __restrict__ rows, int n_nz, const int* __restrict__ take_q, int n_take,
                                uint8_t* __restrict__ in_panel) {
    const int pid = blockIdx.x;
    if (pid >= n_take) return;
    const int first = take_q[pid] * kDppR;
    const int cnt = min(kDppR, n_nz - first);
    for (int k = threadIdx.x; k < cnt; k += blockDim.x) in_panel[rows[first + k]] = 1;
}


// ---- tile cuts: b(a) = min(a + P, |U|, f(a)) with f(a) the smallest
// upos[j + kPanelMaxRun] over nonzeros j (of any slot) with upos[j] >= a.
// Within a slot upos ascends, so its first nonzero at or after a gives its
// smallest value and f(a) is a suffix minimum over union positions of
// m[u] = min over the nonzeros j at position u of upos[j + kPanelMaxRun]
// (no value past a row's end).  plan_panels cuts a tile where some slot
// would get its (kPanelMaxRun + 1)-th nonzero or where the tile has P
// columns: the same b.

struct DppPanelArgs {
    const int* rowptr;
    const int* rows;     // longest-first order
    const int* lenpre;   // union scratch bases (by order position)
    const int* ucols;
    const int* upos;     // [CSR index]
    const int* ucount;   // [candidate]
    const int* take_q;   // [pid]: candidate of taken panel pid
    const int* ubase;    // [pid]: base of the panel's union-position arrays (m, tile_of)
    const int* tbase;    // [pid]: base of the panel's tile scratch (|U| + 1 entries)
    const int* tile0;    // [pid]: global index of the panel's first tile (after the walk)
    int n_nz, P, n_take;
    uint32_t row_bytes;  // B row stride: N * element size
    int* m;              // [ubase + u]: m, then f
    int* cuts;           // [tbase + t]: first union position of tile t (cuts[nt] = |U|)
    int* ntiles;         // [pid]
    int* tile_of;        // [ubase + u]: tile of union position u
    int* tn;             // [tbase + t]: nonzeros of tile t
    uint8_t* cntb;       // [tile * kDppCntDwords * 4 + byte]: the plan's count bytes
    uint32_t* boff;      // [tile * P + j]
    uint8_t* pos;        // [CSR index]
    int* ucut;           // [tbase + k]: first tile of unit k (k <= units)
    int* nunits;         // [pid]
    // emission of units (phase b)
    const int4* poff;    // [pid]: {first tile, first unit, first segment (-1: not split), first long row}
    int* prows;          // [pid * R + slot]
    int4* units;
    int* ustart;         // [unit * R + slot]
    int* panel_units;    // [pid]
    int4* longrows;      // the panels' long rows (after the row kernel's)
    int64_t* ulo;        // [unit]: first staged column
    int64_t* uhi;        // [unit]: last staged column
};

// Row k of taken panel pid for wavefront w of a grid of (panels x R / 4)
// workgroups of four wavefronts: its row, CSR range and slot (row -1: none).
__device__ inline void dpp_row_of(const DppPanelArgs& a, int* pid, int* k, int* row, int* rs, int* re) {
    const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
    *pid = w / kDppR;
    *k = w % kDppR;
    *row = -1;
    *rs = *re = 0;
    if (*pid >= a.n_take) return;
    const int first = a.take_q[*pid] * kDppR;
    if (*k >= min(kDppR, a.n_nz - first)) return;
    *row = a.rows[first + *k];
    *rs = a.rowptr[*row];
    *re = a.rowptr[*row + 1];
}

// m[u] = min over the nonzeros at u of upos[j + kPanelMaxRun]; m starts at
// 0x7f7f7f7f (larger than any position).
__global__ __launch_bounds__(256) void dpp_m_kernel(DppPanelArgs a) {
    int pid, k, row, rs, re;
    dpp_row_of(a, &pid, &k, &row, &rs, &re);
    if (row < 0) return;
    const int ub = a.ubase[pid];
    const int lane = threadIdx.x & 63;
    constexpr int kU = 8;  // chunks of 64 nonzeros in flight
    for (int j0 = rs; j0 < re; j0 += 64 * kU) {
        int u[kU], h[kU];
#pragma unroll
        for (int x = 0; x < kU; x++) {
            const int j = j0 + 64 * x + lane;
            u[x] = j < re ? a.upos[j] : -1;
            h[x] = j + kPanelMaxRun < re ? a.upos[j + kPanelMaxRun] : INT_MAX;
        }
#pragma unroll
        for (int x = 0; x < kU; x++)
            if (u[x] >= 0 && h[x] != INT_MAX) atomicMin(&a.m[ub + u[x]], h[x]);
    }
}

// Per panel (1024 threads): f = suffix minimum of m (in place), then the
// walk a -> b(a) over chunks of f staged in LDS; cuts and the tile count.
constexpr int kDppWalkChunk = 32768;  // f entries per LDS chunk (128 KiB)
__global__ __launch_bounds__(1024) void dpp_walk_kernel(DppPanelArgs a) {
    __shared__ int fch[kDppWalkChunk];
    __shared__ int red[16];
    __shared__ int s_a, s_nt;
    const int pid = blockIdx.x, tid = threadIdx.x;
    const int U = a.ucount[a.take_q[pid]];
    int* f = a.m + a.ubase[pid];
    // suffix minimum, chunks of 4096 from the right (4 per thread)
    int carry = INT_MAX;
    for (int hi = U; hi > 0; hi -= 4096) {
        const int lo = max(0, hi - 4096);
        int v[4];
        int mn = INT_MAX;
#pragma unroll
        for (int x = 3; x >= 0; x--) {  // thread tid holds lo + 4 tid .. + 3
            const int u = lo + 4 * tid + x;
            v[x] = u < hi ? f[u] : INT_MAX;
            mn = min(mn, v[x]);
            v[x] = mn;  // suffix min within the thread's four
        }
        // minimum of the threads after this one: reverse scan over the block
        int x = mn;
        const int lane = tid & 63, w = tid >> 6;
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_down(x, o);
            if (lane + o < 64) x = min(x, y);
        }
        __syncthreads();
        if (lane == 0) red[w] = x;  // minimum of wavefront w from lane 0 on
        __syncthreads();
        int after = carry;  // everything right of this thread
        for (int i = w + 1; i < 16; i++) after = min(after, red[i]);
        const int nextx = __shfl_down(x, 1);
        if (lane < 63) after = min(after, nextx);
#pragma unroll
        for (int y = 0; y < 4; y++) {
            const int u = lo + 4 * tid + y;
            if (u < hi) f[u] = min(v[y], after);
        }
        int chunk_min = INT_MAX;
        for (int i = 0; i < 16; i++) chunk_min = min(chunk_min, red[i]);
        carry = min(carry, chunk_min);
        __syncthreads();
    }
    // (the walk reads f back: agent-scope fence so no stale cached line of m is read)
    __threadfence();
    __syncthreads();
    // the walk: thread 0 follows b(a) through the chunk of f in LDS; all
    // threads restage f at the next chunk when the walk leaves it
    const int tb = a.tbase[pid];
    if (tid == 0) {
        s_a = 0;
        s_nt = 0;
    }
    __syncthreads();
    while (s_a < U) {
        const int base = s_a;
        const int lim = min(U, base + kDppWalkChunk);
        for (int u = base + tid; u < lim; u += 1024) fch[u - base] = f[u];
        __syncthreads();
        if (tid == 0) {
            int x = s_a, nt = s_nt;
            while (x < lim) {
                a.cuts[tb + nt] = x;
                x = min(min(x + a.P, U), fch[x - base]);
                nt++;
            }
            s_a = x;
            s_nt = nt;
        }
        __syncthreads();
    }
    if (tid == 0) {
        a.cuts[tb + s_nt] = U;
        a.ntiles[pid] = s_nt;
    }
}

// Per tile (one workgroup of 256): tile_of over its union positions, its
// staged rows (positions past its width repeat its last column).  Tile
// `g` of all panels: its panel by binary search over tile0.
__device__ inline int dpp_panel_of_tile(const DppPanelArgs& a, int g) {
    int lo = 0, hi = a.n_take - 1;  // last pid with tile0 <= g
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (a.tile0[mid] <= g) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}
__global__ __launch_bounds__(256) void dpp_tile_fill_kernel(DppPanelArgs a) {
    const int g = blockIdx.x;
    const int pid = dpp_panel_of_tile(a, g);
    const int t = g - a.tile0[pid];
    const int tb = a.tbase[pid], ub = a.ubase[pid];
    const int lu = a.lenpre[a.take_q[pid] * kDppR];
    const int c0 = a.cuts[tb + t], c1 = a.cuts[tb + t + 1];
    const int x = threadIdx.x;
    if (c0 + x < c1) a.tile_of[ub + c0 + x] = t;
    if (x < a.P) a.boff[static_cast<size_t>(g) * a.P + x] =
        static_cast<uint32_t>(a.ucols[lu + min(c0 + x, c1 - 1)]) * a.row_bytes;
}

// Per nonzero (one wavefront per row): position in its tile, and at the
// end of each run (the row's nonzeros in one tile) its count byte and the
// tile's nonzeros.  kUstart: instead, at the start of each run, the row's
// cursor for every unit that starts after the row's previous run's tile
// and at or before this run's tile.
template <bool kUstart>
__global__ __launch_bounds__(256) void dpp_runs_kernel(DppPanelArgs a) {
    int pid, k, row, rs, re;
    dpp_row_of(a, &pid, &k, &row, &rs, &re);
    if (row < 0) return;
    const int lane = threadIdx.x & 63;
    const int ub = a.ubase[pid], tb = a.tbase[pid], t0 = a.tile0[pid];
    const int s = dpp_slot_of(k);
    const int cw = s / (4 * kPanelRpg), ci = (s / 4) % kPanelRpg, cg = s % 4;
    int4 po = make_int4(0, 0, 0, 0);
    int nu = 0;
    if constexpr (kUstart) {
        po = a.poff[pid];
        nu = a.nunits[pid];
    }
    int run_start = rs;  // start of the run in progress (carried across chunks)
    int prev_tile = -1;  // tile of the nonzero before the chunk
    constexpr int kU = 8;  // chunks of 64 nonzeros in flight
    for (int jb = rs; jb < re; jb += 64 * kU) {
        int u[kU], t[kU];
#pragma unroll
        for (int x = 0; x < kU; x++) {
            const int j = jb + 64 * x + lane;
            u[x] = j < re ? a.upos[j] : 0;
        }
#pragma unroll
        for (int x = 0; x < kU; x++) {
            const int j = jb + 64 * x + lane;
            t[x] = j < re ? a.tile_of[ub + u[x]] : INT_MAX;
        }
        const int jlast = jb + 64 * kU;  // the nonzero after these chunks
        const int tafter = jlast < re ? a.tile_of[ub + a.upos[jlast]] : INT_MAX;
#pragma unroll
        for (int x = 0; x < kU; x++) {
            const int j0 = jb + 64 * x;
            if (j0 >= re) break;
            const int j = j0 + lane;
            const bool in = j < re;
            int tnext = __shfl_down(t[x], 1);
            const int tn0 = __shfl(t[x + 1 < kU ? x + 1 : x], 0);  // (every lane active in the shuffle)
            if (lane == 63) tnext = x + 1 < kU ? tn0 : tafter;
            if (j + 1 >= re) tnext = INT_MAX;
            int tprev = __shfl_up(t[x], 1);
            if (lane == 0) tprev = prev_tile;
            const bool first = in && t[x] != tprev;
            const bool last = in && t[x] != tnext;
            const uint64_t fm = __ballot(first);
            if constexpr (!kUstart) {
                if (in) a.pos[j] = static_cast<uint8_t>(u[x] - a.cuts[tb + t[x]] + 1);
                if (last) {
                    const uint64_t upto = fm & (lane == 63 ? ~uint64_t(0) : ((uint64_t(2) << lane) - 1));
                    const int start = upto ? j0 + 63 - __clzll(upto) : run_start;
                    const int n = j - start + 1;
                    a.cntb[(static_cast<size_t>(t0) + t[x]) * (kDppCntDwords * 4) + (cw * kPanelCntRows + ci) * 4 + cg] =
                        static_cast<uint8_t>(n);
                    atomicAdd(&a.tn[tb + t[x]], n);
                }
            } else if (first) {
                // units whose first tile lies in (tprev, t]: this run's start is their
                // cursor (unit starts ascend: the first one after tprev by binary search)
                int lo = 0, hi = nu;
                while (lo < hi) {
                    const int mid = (lo + hi) / 2;
                    if (a.ucut[tb + mid] > tprev) hi = mid;
                    else lo = mid + 1;
                }
                for (int q = lo; q < nu && a.ucut[tb + q] <= t[x]; q++)
                    a.ustart[(static_cast<size_t>(po.y) + q) * kDppR + s] = j;
            }
            if (fm) run_start = j0 + 63 - __clzll(fm);
            prev_tile = __shfl(t[x], 63);
        }
    }
}

// Per tile: the longest of each (wavefront, entry)'s four group counts.
__global__ void dpp_cnt_max_kernel(uint8_t* __restrict__ cntb, int64_t n_tiles) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;  // (tile, wave, entry)
    if (i >= n_tiles * kPanelWaves * kPanelRpg) return;
    const int64_t t = i / (kPanelWaves * kPanelRpg);
    const int r = static_cast<int>(i % (kPanelWaves * kPanelRpg)), cw = r / kPanelRpg, ci = r % kPanelRpg;
    uint8_t* tile = cntb + t * (kDppCntDwords * 4);
    const uint8_t* c4 = tile + (cw * kPanelCntRows + ci) * 4;
    const uint8_t mx = max(max(c4[0], c4[1]), max(c4[2], c4[3]));
    tile[(cw * kPanelCntRows + kPanelMaxDword + ci / 4) * 4 + ci % 4] = mx;
}

// Unit cuts of each taken panel (plan_panels: nu = max(1, min(tiles,
// ceil(nnz / unit_nnz))); a cut after tile t when the nonzeros so far reach
// nnz * k / nu, at most one per tile, none after the last).  One wavefront
// per panel: tile counts arrive 64 at a time, the rule walks them in order.
__global__ void dpp_units_kernel(const int* __restrict__ take_q, int n_take, const int* __restrict__ pnnz,
                                 const int* __restrict__ tbase, const int* __restrict__ ntiles,
                                 const int* __restrict__ tn, int64_t unit_nnz, int* __restrict__ cuts,
                                 int* __restrict__ nunits) {
    const int pid = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (pid >= n_take) return;
    const int nt = ntiles[pid], tb = tbase[pid];
    const int64_t nnz = pnnz[take_q[pid]];
    const int64_t nu = max(int64_t(1), min(static_cast<int64_t>(nt), (nnz + unit_nnz - 1) / unit_nnz));
    int ncut = 1;
    int64_t acc = 0;
    if (lane == 0) cuts[tb] = 0;
    for (int t0 = 0; t0 < nt; t0 += 64) {
        const int mine = t0 + lane < nt ? tn[tb + t0 + lane] : 0;
        const int m = min(64, nt - t0);
        for (int x = 0; x < m; x++) {
            const int t = t0 + x;
            acc += __shfl(mine, x);
            const int64_t want = nnz * ncut / nu;
            if (acc >= want && ncut < nu && t + 1 < nt) {
                if (lane == 0) cuts[tb + ncut] = t + 1;
                ncut++;
            }
        }
    }
    if (lane == 0) {
        cuts[tb + ncut] = nt;
        nunits[pid] = ncut;
    }
}

// Per taken panel (256 threads): its rows, unit count, units (with their
// first and last staged columns), the split panels' long rows, and every
// unit's cursors at the rows' ends (dpp_runs_kernel<true> then writes the
// cursors of the rows with nonzeros at or after a unit's first tile).
__global__ __launch_bounds__(256) void dpp_emit_units_kernel(DppPanelArgs a) {
    __shared__ int red[4];
    const int pid = blockIdx.x, s = threadIdx.x;
    const int q = a.take_q[pid];
    const int first = q * kDppR;
    const int rows_in = min(kDppR, a.n_nz - first);
    const int4 po = a.poff[pid];
    const int nu = a.nunits[pid];
    const int tb = a.tbase[pid];
    const int lu = a.lenpre[first];
    int row = -1, re = 0;
    if (s < kDppR) {
        const int k = dpp_k_of(s);
        if (k < rows_in) {
            row = a.rows[first + k];
            re = a.rowptr[row + 1];
        }
        a.prows[static_cast<size_t>(pid) * kDppR + s] = row;
    }
    if (s == 0) a.panel_units[pid] = nu;
    int tot = 0;
    const int rank = dpp_block_exscan<256>(row >= 0 ? 1 : 0, red, &tot);
    if (nu > 1 && row >= 0) a.longrows[po.w + rank] = make_int4(row, po.z + s * nu, nu, 0);
    for (int k = 0; k < nu; k++) {
        const size_t un = static_cast<size_t>(po.y) + k;
        if (s < kDppR) a.ustart[un * kDppR + s] = row >= 0 ? re : 0;
        if (s == 0) {
            const int ft = a.ucut[tb + k], lt = a.ucut[tb + k + 1];  // tiles [ft, lt)
            a.units[un] = make_int4(pid, po.x + ft, lt - ft, nu > 1 ? po.z + k : -1);
            a.ulo[un] = a.ucols[lu + a.cuts[tb + ft]];
            a.uhi[un] = a.ucols[lu + a.cuts[tb + lt] - 1];
        }
    }
}

// Sorted lengths (keys: length + 1) -> lengths, for the exclusive sum.
__global__ void dpp_len_kernel(const uint32_t* __restrict__ keys, int n, int* __restrict__ len) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        len[i] = keys[i] > 0 ? static_cast<int>(keys[i]) - 1 : 0;
}

}  // namespace tca
