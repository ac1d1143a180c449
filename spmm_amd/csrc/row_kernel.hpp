// row_kernel.hpp -- the wavefront-per-row SpMM kernels for gfx950 (VALU path).
//
// One 64-lane wavefront per task.  The lanes form S = 64 / G slots of G
// lanes; the G lanes of a slot cover one chunk of a B row with 16-byte loads
// (E values each), so a wavefront reads S B rows per load instruction, fully
// coalesced.  Per task kind:
//   row   -- the S slots take every S-th nonzero of one row, 8 loads in flight
//            per lane; the slots' fp32 partial rows are then summed with
//            xor shuffles (identical order on every run) and written once.
//   multi -- each slot walks its own short row (rows grouped by length);
//            a group of empty rows (z == 0) only clears their C rows.
//   seg   -- like row over one segment of a long row; the segment's partial
//            row goes to plan scratch and seg_finalize_kernel, launched next
//            on the same stream, adds the segments in a fixed order.
// Every row of C is written exactly once, so results do not depend on the
// schedule, and C needs no zeroing.
//
// All operand loads are raw buffer loads: a masked lane uses an offset past
// the buffer's size, which the hardware returns as zeros without a fault, so
// the loads carry no branches and all eight stay in flight.
//
// Functionally replaces reference multirow_per_tb / multitb_per_row
// (src/our_spmm.cu:24-295), which stage B through shared memory and use one
// eighth of each m16n8k8 MMA.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tca {

struct bf16_t {
    uint16_t b;
};

__device__ __forceinline__ float to_f32(_Float16 x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return __uint_as_float(static_cast<uint32_t>(x.b) << 16); }

template <typename T, int E>
struct alignas(E * sizeof(T)) Pack {
    T v[E];
};

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kRowWaves = 4;   // wavefronts per workgroup (independent tasks)
constexpr int kRowUnroll = 8;  // B loads in flight per lane
constexpr uint32_t kOob = 0xfffffff0u;  // buffer offset past any buffer this library builds

// Raw buffer resource over `bytes` bytes at `base` (gfx9 word 3: 32-bit data format).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// E elements of T at byte offset `off` of buffer r (zeros when off is out of range).
template <typename T, int E>
__device__ __forceinline__ Pack<T, E> load_pack(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    using P = Pack<T, E>;
    constexpr int bytes = E * static_cast<int>(sizeof(T));
    if constexpr (bytes == 16) {
        return __builtin_bit_cast(P, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
    } else if constexpr (bytes == 8) {
        return __builtin_bit_cast(P, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
    } else if constexpr (bytes == 4) {
        return __builtin_bit_cast(P, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
    } else {
        return __builtin_bit_cast(P, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
    }
}

template <typename T>
__device__ __forceinline__ float load_val(__amdgpu_buffer_rsrc_t r, uint32_t idx, bool ok) {
    const uint32_t off = ok ? idx * static_cast<uint32_t>(sizeof(T)) : kOob;
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
    } else {
        return to_f32(__builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0)));
    }
}

__device__ __forceinline__ int load_idx(__amdgpu_buffer_rsrc_t r, uint32_t idx, bool ok) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, ok ? idx * 4u : kOob, 0, 0);
}

// Stores E consecutive fp32 values (16-byte stores when E >= 4), streaming.
template <int E>
__device__ __forceinline__ void store_row(float* dst, const float (&v)[E]) {
    if constexpr (E >= 4) {
#pragma unroll
        for (int i = 0; i < E; i += 4)
            __builtin_nontemporal_store(f32x4{v[i], v[i + 1], v[i + 2], v[i + 3]}, reinterpret_cast<f32x4*>(dst + i));
    } else if constexpr (E == 2) {
        __builtin_nontemporal_store(f32x2{v[0], v[1]}, reinterpret_cast<f32x2*>(dst));
    } else {
        __builtin_nontemporal_store(v[0], dst);
    }
}

// C stores of lanes holding 32 bytes (E = 8: fp16 / bf16 B): lane g of a
// slot holds 16-byte pieces 2g and 2g + 1 of the slot's chunk row, so two
// plain store instructions would each fill half of every 128-byte line.
// Instead the pieces are exchanged inside the slot (every lane active):
// lane g receives piece g (from lane g / 2) for the first store and piece
// g + cl (from lane (g + cl) / 2) for the second, so each store instruction
// writes whole lines.  cl: lanes of the slot holding data.
struct LinePieces {
    f32x4 p0, p1;  // pieces g and g + cl of the chunk row
};
template <int E>
__device__ __forceinline__ LinePieces line_pieces(const float (&v)[E], int lane, int g, int cl) {
    static_assert(E == 8, "32-byte lanes");
    const int base = lane - g;  // first lane of the slot
    const int s1 = base + g / 2, s2 = base + (g + cl) / 2;
    const bool odd1 = (g & 1) != 0, odd2 = ((g + cl) & 1) != 0;
    LinePieces r;
    float a[4], b[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float lo1 = __shfl(v[e], s1), hi1 = __shfl(v[e + 4], s1);
        const float lo2 = __shfl(v[e], s2), hi2 = __shfl(v[e + 4], s2);
        a[e] = odd1 ? hi1 : lo1;
        b[e] = odd2 ? hi2 : lo2;
    }
    r.p0 = f32x4{a[0], a[1], a[2], a[3]};
    r.p1 = f32x4{b[0], b[1], b[2], b[3]};
    return r;
}
// Stores pieces g and g + cl of a chunk row starting at `row` (column
// chunk_col of the row); pieces past n_cols are not written.
__device__ __forceinline__ void store_line_pieces(float* row, int chunk_col, int n_cols, int g, int cl,
                                                  const LinePieces& p) {
    if (chunk_col + 4 * g < n_cols)
        __builtin_nontemporal_store(p.p0, reinterpret_cast<f32x4*>(row + chunk_col + 4 * g));
    if (chunk_col + 4 * (g + cl) < n_cols)
        __builtin_nontemporal_store(p.p1, reinterpret_cast<f32x4*>(row + chunk_col + 4 * (g + cl)));
}

template <typename T, int E>
__device__ __forceinline__ void fma_pack(float (&acc)[E], float a, const Pack<T, E>& b) {
#pragma unroll
    for (int e = 0; e < E; e++) acc[e] = __builtin_fmaf(a, to_f32(b.v[e]), acc[e]);
}

struct RowArgs {
    const int4* tasks;
    const int* order;  // [wavefront slot]: task, -1 idle; null: slot = task
    int ntasks;
    const int* rowptr;
    const int* perm;
    float* partials;
    float* C;
    int N;
    int logG;         // log2 of lanes per slot
    int chunk_lanes;  // lanes per slot that hold data
    int col_chunks;   // blockIdx.x = task group * col_chunks + chunk
    const void* colidx;  // buffer bases and sizes in bytes
    const void* val;
    const void* B;
    uint32_t colidx_bytes, val_bytes, B_bytes;
};

// Slots split the nonzeros [beg, end) of one row; lane (slot, g) accumulates
// columns [col, col + E).  Column indices and values are fetched 64 at a
// time with one coalesced load and handed to the slots with ds_bpermute (or
// v_readlane when one slot spans the whole wavefront).
template <typename T, int E, bool kOneSlot>
__device__ __forceinline__ void accumulate_span(float (&acc)[E], int beg, int end, const RowArgs& a,
                                                __amdgpu_buffer_rsrc_t rcol, __amdgpu_buffer_rsrc_t rval,
                                                __amdgpu_buffer_rsrc_t rB, int col, bool colok, int lane, int slot,
                                                int logS) {
    const uint32_t rowbytes = static_cast<uint32_t>(a.N) * sizeof(T);
    const uint32_t colbytes = static_cast<uint32_t>(col) * sizeof(T);
    // Indices and values of the first chunk of 64; each chunk's loop below
    // first issues the loads of the next chunk, so they travel while the B
    // rows of this one are gathered.
    int myc = load_idx(rcol, beg + lane, beg + lane < end);
    float mya = load_val<T>(rval, beg + lane, beg + lane < end);
    for (int base = beg; base < end; base += 64) {
        const int n = min(64, end - base);
        const int nb = base + 64;
        const int nmyc = load_idx(rcol, nb + lane, nb + lane < end);
        const float nmya = load_val<T>(rval, nb + lane, nb + lane < end);
        const int rounds = (n + (1 << logS) - 1) >> logS;
        for (int r = 0; r < rounds; r += kRowUnroll) {
            Pack<T, E> bv[kRowUnroll];
            float av[kRowUnroll];
#pragma unroll
            for (int u = 0; u < kRowUnroll; u++) {
                int c;
                bool ok;
                if constexpr (kOneSlot) {
                    const int idx = r + u;  // wave-uniform
                    c = __builtin_amdgcn_readlane(myc, idx & 63);
                    av[u] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mya), idx & 63));
                    ok = idx < n && colok;
                } else {
                    const int idx = ((r + u) << logS) + slot;
                    c = __shfl(myc, idx & 63);
                    av[u] = __shfl(mya, idx & 63);
                    ok = idx < n && colok;
                }
                bv[u] = load_pack<T, E>(rB, ok ? static_cast<uint32_t>(c) * rowbytes + colbytes : kOob);
            }
#pragma unroll
            for (int u = 0; u < kRowUnroll; u++) fma_pack<T, E>(acc, av[u], bv[u]);
        }
        myc = nmyc;
        mya = nmya;
    }
}

template <typename T, int E>
__global__ __launch_bounds__(256) void row_kernel(RowArgs a) {
    __shared__ float red[kRowWaves][64 * E];  // wide rows: one partial row chunk per wavefront
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    // Consecutive workgroups take consecutive column chunks: the hardware
    // deals workgroups to the 8 XCDs round robin, so with 8 (or 4, 2) chunks
    // every XCD reads one fixed slice of B and keeps it in its own L2.
    const int chunk = blockIdx.x % a.col_chunks;
    const int sid = (blockIdx.x / a.col_chunks) * kRowWaves + wave;
    const int tid = a.order ? a.order[sid] : sid;
    if (tid < 0 || tid >= a.ntasks) return;
    const __amdgpu_buffer_rsrc_t rcol = make_rsrc(a.colidx, a.colidx_bytes);
    const __amdgpu_buffer_rsrc_t rval = make_rsrc(a.val, a.val_bytes);
    const __amdgpu_buffer_rsrc_t rB = make_rsrc(a.B, a.B_bytes);
    const int logS = 6 - a.logG;
    const int slot = lane >> a.logG;
    const int g = lane & ((1 << a.logG) - 1);
    const int col = (chunk * a.chunk_lanes + g) * E;
    const bool colok = g < a.chunk_lanes && col < a.N;
    const int4 t = a.tasks[tid];
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; e++) acc[e] = 0.f;

    if (t.w == 1 && t.z == 0) {  // zero task: clear the C rows of up to kZeroRows empty rows
        // A task's rows ascend (the planners keep the empty rows of the
        // longest-first order in row order), so when its first and last
        // differ by its count less one they are consecutive and, with one
        // column chunk, their C rows are one contiguous range: cleared 16
        // bytes per lane, 1 KiB per store instruction.
        if (a.col_chunks == 1 && (a.N & 3) == 0) {
            const int r0 = a.perm[t.x];
            if (a.perm[t.x + t.y - 1] - r0 == t.y - 1) {
                f32x4* const base = reinterpret_cast<f32x4*>(a.C + static_cast<size_t>(r0) * a.N);
                const int n4 = t.y * (a.N >> 2);
                const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                for (int o = lane; o < n4; o += 64) __builtin_nontemporal_store(z, base + o);
                return;
            }
        }
        const int step = 1 << logS;
        if constexpr (E == 8) {
            // 32 bytes per lane: lane g clears 16-byte pieces g and g + chunk
            // lanes of the chunk, so each store instruction covers whole
            // 128-byte lines (store_row's two halves per lane would leave
            // every line half written by each instruction)
            const int c0 = chunk * a.chunk_lanes * 8;
            const f32x4 z = {0.f, 0.f, 0.f, 0.f};
            if (g < a.chunk_lanes)
                for (int r = slot; r < t.y; r += step) {
                    float* dst = a.C + static_cast<size_t>(a.perm[t.x + r]) * a.N + c0;
                    if (c0 + 4 * g < a.N) __builtin_nontemporal_store(z, reinterpret_cast<f32x4*>(dst + 4 * g));
                    if (c0 + 4 * (g + a.chunk_lanes) < a.N)
                        __builtin_nontemporal_store(z, reinterpret_cast<f32x4*>(dst + 4 * (g + a.chunk_lanes)));
                }
        } else if (colok) {
            for (int r = slot; r < t.y; r += step)
                store_row<E>(a.C + static_cast<size_t>(a.perm[t.x + r]) * a.N + col, acc);
        }
        return;
    }
    if (t.w == 1) {  // multi: in pass p0 (of S rows), slot s walks row perm[t.x + p0 + s]
        // The next pass's row and CSR range are loaded before this pass's
        // gathers, so they arrive during them.  Every pass runs t.z steps
        // (the group's first and longest row).
        const int S = 1 << logS;
        int row = -1, beg = 0, len = 0;
        if (slot < t.y) {
            row = a.perm[t.x + slot];
            beg = a.rowptr[row];
            len = a.rowptr[row + 1] - beg;
        }
        const uint32_t rowbytes = static_cast<uint32_t>(a.N) * sizeof(T);
        const uint32_t colbytes = static_cast<uint32_t>(col) * sizeof(T);
        for (int p0 = 0; p0 < t.y; p0 += S) {
            int nrow = -1, nbeg = 0, nlen = 0;
            if (p0 + S + slot < t.y) {
                nrow = a.perm[t.x + p0 + S + slot];
                nbeg = a.rowptr[nrow];
                nlen = a.rowptr[nrow + 1] - nbeg;
            }
#pragma unroll
            for (int e = 0; e < E; e++) acc[e] = 0.f;
            for (int j = 0; j < t.z; j += kRowUnroll) {
                Pack<T, E> bv[kRowUnroll];
                float av[kRowUnroll];
                int c[kRowUnroll];
#pragma unroll
                for (int u = 0; u < kRowUnroll; u++) {
                    c[u] = load_idx(rcol, beg + j + u, j + u < len);
                    av[u] = load_val<T>(rval, beg + j + u, j + u < len);
                }
#pragma unroll
                for (int u = 0; u < kRowUnroll; u++)
                    bv[u] = load_pack<T, E>(rB, j + u < len && colok ? static_cast<uint32_t>(c[u]) * rowbytes + colbytes
                                                                     : kOob);
#pragma unroll
                for (int u = 0; u < kRowUnroll; u++) fma_pack<T, E>(acc, av[u], bv[u]);
            }
            if constexpr (E == 8) {
                const LinePieces lp = line_pieces<E>(acc, lane, g, a.chunk_lanes);
                if (row >= 0 && g < a.chunk_lanes)
                    store_line_pieces(a.C + static_cast<size_t>(row) * a.N, chunk * a.chunk_lanes * 8, a.N, g,
                                      a.chunk_lanes, lp);
            } else {
                if (row >= 0 && colok) store_row<E>(a.C + static_cast<size_t>(row) * a.N + col, acc);
            }
            row = nrow;
            beg = nbeg;
            len = nlen;
        }
        return;
    }

    // row / seg: all slots on one span
    if (a.logG == 6)
        accumulate_span<T, E, true>(acc, t.y, t.z, a, rcol, rval, rB, col, colok, lane, slot, logS);
    else
        accumulate_span<T, E, false>(acc, t.y, t.z, a, rcol, rval, rB, col, colok, lane, slot, logS);
    for (int off = 1 << a.logG; off < 64; off <<= 1)
#pragma unroll
        for (int e = 0; e < E; e++) acc[e] += __shfl_xor(acc[e], off);
    if ((t.w & 3) == 3) {
        // wide row: the four quarters meet in LDS and wavefront 0 adds them in
        // quarter order.  Every wavefront of this workgroup holds a quarter of
        // the same row (the plan places wide groups 4-aligned), so all four
        // reach the barrier.
        if (slot == 0)
#pragma unroll
            for (int e = 0; e < E; e++) red[wave][g * E + e] = acc[e];
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int e = 0; e < E; e++)
            acc[e] = ((red[0][g * E + e] + red[1][g * E + e]) + red[2][g * E + e]) + red[3][g * E + e];
        if constexpr (E == 8) {
            const LinePieces lp = line_pieces<E>(acc, lane, g, a.chunk_lanes);
            if (slot == 0 && g < a.chunk_lanes)
                store_line_pieces(a.C + static_cast<size_t>(t.x) * a.N, chunk * a.chunk_lanes * 8, a.N, g, a.chunk_lanes,
                                  lp);
        } else {
            if (slot == 0 && colok) store_row<E>(a.C + static_cast<size_t>(t.x) * a.N + col, acc);
        }
        return;
    }
    float* const dst_row = t.w == 0 ? a.C + static_cast<size_t>(t.x) * a.N
                                    : a.partials + static_cast<size_t>(t.w >> 2) * a.N;  // seg: partial row of slot t.w >> 2
    if constexpr (E == 8) {
        const LinePieces lp = line_pieces<E>(acc, lane, g, a.chunk_lanes);
        if (slot == 0 && g < a.chunk_lanes) store_line_pieces(dst_row, chunk * a.chunk_lanes * 8, a.N, g, a.chunk_lanes, lp);
    } else {
        if (slot == 0 && colok) store_row<E>(dst_row + col, acc);
    }
}

// Lanes of seg_finalize_kernel per partial row: four columns each, a power
// of two up to 64 covering N; the 256 threads of a workgroup form 256 / L
// groups of L lanes.
__host__ __device__ inline int fin_lanes(int N) {
    const int q = (N + 3) / 4;
    int l = 1;
    while (l < q && l < 64) l <<= 1;
    return l;
}

// C[row, :] = sum of the row's partial rows (segments or panel units).  One
// workgroup per (long row, 4L columns): group j of the 256 / L groups adds
// the j-th contiguous block of the partial rows in order, eight loads in
// flight, and group 0 adds the blocks' sums in block order.  The order is
// fixed by N and the number of partial rows, so results do not depend on
// the schedule.
__global__ __launch_bounds__(256) void seg_finalize_kernel(const int4* __restrict__ longrows,
                                                           const float* __restrict__ partials, float* __restrict__ C,
                                                           int N) {
    __shared__ f32x4 red[256];
    const int4 lr = longrows[blockIdx.x];  // {row, first partial row, partial rows, 0}
    const int L = fin_lanes(N), P = 256 / L;
    const int grp = threadIdx.x / L, l = threadIdx.x % L;
    const int col = (blockIdx.y * L + l) * 4;
    const int k0 = static_cast<int>(static_cast<int64_t>(lr.z) * grp / P);
    const int k1 = static_cast<int>(static_cast<int64_t>(lr.z) * (grp + 1) / P);
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    if (col < N) {
        if ((N & 3) == 0) {  // rows 16-byte aligned
            const f32x4* src = reinterpret_cast<const f32x4*>(partials + static_cast<size_t>(lr.y) * N + col);
            const size_t stride = static_cast<size_t>(N) / 4;
            int k = k0;
            for (; k + 8 <= k1; k += 8) {
                f32x4 v[8];
#pragma unroll
                for (int u = 0; u < 8; u++) v[u] = src[(k + u) * stride];
#pragma unroll
                for (int u = 0; u < 8; u++) s += v[u];
            }
            for (; k < k1; k++) s += src[k * stride];
        } else {  // this thread's columns [col, col + 4) only
            const float* src = partials + static_cast<size_t>(lr.y) * N + col;
            for (int k = k0; k < k1; k++) {
                const float* r = src + static_cast<size_t>(k) * N;
                s.x += r[0];
                if (col + 1 < N) s.y += r[1];
                if (col + 2 < N) s.z += r[2];
                if (col + 3 < N) s.w += r[3];
            }
        }
    }
    red[threadIdx.x] = s;
    __syncthreads();
    if (grp != 0 || col >= N) return;
    f32x4 t = red[l];
    for (int j = 1; j < P; j++) t += red[j * L + l];
    float* dst = C + static_cast<size_t>(lr.x) * N + col;
    if ((N & 3) == 0) {
        *reinterpret_cast<f32x4*>(dst) = t;
    } else {
        dst[0] = t.x;
        if (col + 1 < N) dst[1] = t.y;
        if (col + 2 < N) dst[2] = t.z;
        if (col + 3 < N) dst[3] = t.w;
    }
}

}  // namespace tca
