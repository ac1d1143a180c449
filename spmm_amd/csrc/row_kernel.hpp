// row_kernel.hpp -- the wavefront-per-row SpMM kernel for gfx950 (VALU path).
//
// One 64-lane wavefront per task.  The lanes form S = 64 / G slots of G
// lanes; the G lanes of a slot cover one chunk of a B row with 16-byte loads
// (E values each), so a wavefront reads S B rows per load instruction, fully
// coalesced.  Per task kind:
//   row   -- the S slots take every S-th nonzero of one row, 8 loads in flight
//            per lane; the slots' fp32 partial rows are then summed with
//            xor shuffles (identical order on every run) and written once.
//   multi -- each slot walks its own short row (rows grouped by length).
//   seg   -- like row over one segment of a long row; the segment's partial
//            row goes to plan scratch and the last segment to finish (atomic
//            ticket) adds all segments in segment order and writes C.
// Every row of C is written exactly once, so results do not depend on the
// schedule, and C needs no zeroing.
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

// Stores E consecutive fp32 values (16-byte stores when E >= 4).
template <int E>
__device__ __forceinline__ void store_row(float* dst, const float (&v)[E]) {
    if constexpr (E >= 4) {
#pragma unroll
        for (int i = 0; i < E; i += 4)
            __builtin_nontemporal_store(f32x4{v[i], v[i + 1], v[i + 2], v[i + 3]},
                                        reinterpret_cast<f32x4*>(dst + i));
    } else if constexpr (E == 2) {
        __builtin_nontemporal_store(f32x2{v[0], v[1]}, reinterpret_cast<f32x2*>(dst));
    } else {
        __builtin_nontemporal_store(v[0], dst);
    }
}

template <typename T, int E>
__device__ __forceinline__ void fma_pack(float (&acc)[E], float a, const Pack<T, E>& b) {
#pragma unroll
    for (int e = 0; e < E; e++) acc[e] = __builtin_fmaf(a, to_f32(b.v[e]), acc[e]);
}

// Slots split the nonzeros [beg, end) of one row; lane (slot, g) accumulates
// columns [col, col + E).  Column indices and values are fetched 64 at a time
// with one coalesced load and handed to the slots with ds_bpermute (or
// v_readlane when one slot spans the whole wavefront).
template <typename T, int E, bool kOneSlot>
__device__ __forceinline__ void accumulate_span(float (&acc)[E], int beg, int end, const int* __restrict__ colidx,
                                                const T* __restrict__ val, const T* __restrict__ B, int N, int col,
                                                bool colok, int lane, int slot, int logS) {
    for (int base = beg; base < end; base += 64) {
        const int n = min(64, end - base);
        int myc = 0;
        float mya = 0.f;
        if (lane < n) {
            myc = __builtin_nontemporal_load(colidx + base + lane);
            mya = to_f32(val[base + lane]);
        }
        const int rounds = (n + (1 << logS) - 1) >> logS;
        for (int r = 0; r < rounds; r += kRowUnroll) {
            Pack<T, E> bv[kRowUnroll];
            float av[kRowUnroll];
#pragma unroll
            for (int u = 0; u < kRowUnroll; u++) {
                int c;
                float a;
                bool ok;
                if constexpr (kOneSlot) {
                    const int idx = r + u;  // wave-uniform
                    c = __builtin_amdgcn_readlane(myc, idx & 63);
                    a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mya), idx & 63));
                    ok = idx < n && colok;
                } else {
                    const int idx = ((r + u) << logS) + slot;
                    c = __shfl(myc, idx & 63);
                    a = __shfl(mya, idx & 63);
                    ok = idx < n && colok;
                }
                av[u] = ok ? a : 0.f;
                if (ok)
                    bv[u] = *reinterpret_cast<const Pack<T, E>*>(B + static_cast<size_t>(c) * N + col);
                else
#pragma unroll
                    for (int e = 0; e < E; e++) bv[u].v[e] = T{};
            }
#pragma unroll
            for (int u = 0; u < kRowUnroll; u++) fma_pack<T, E>(acc, av[u], bv[u]);
        }
    }
}

template <typename T, int E>
__global__ __launch_bounds__(256) void row_kernel(const int4* __restrict__ tasks, int ntasks,
                                                  const int* __restrict__ rowptr, const int* __restrict__ colidx,
                                                  const T* __restrict__ val, const T* __restrict__ B,
                                                  float* __restrict__ C, int N, int logG,
                                                  const int* __restrict__ perm, const int4* __restrict__ longrows,
                                                  float* __restrict__ partials, int* __restrict__ tickets) {
    const int lane = threadIdx.x & 63;
    const int tid = blockIdx.x * kRowWaves + (threadIdx.x >> 6);
    if (tid >= ntasks) return;
    const int logS = 6 - logG;
    const int slot = lane >> logG;
    const int col = blockIdx.y * (64 * E) + (lane & ((1 << logG) - 1)) * E;
    const bool colok = col < N;
    const int4 t = tasks[tid];
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; e++) acc[e] = 0.f;

    if (t.w == 1) {  // multi: slot s walks row perm[t.x + s]
        int row = -1, beg = 0, len = 0;
        if (slot < t.y) {
            row = perm[t.x + slot];
            beg = rowptr[row];
            len = rowptr[row + 1] - beg;
        }
        for (int j = 0; j < t.z; j += kRowUnroll) {
            Pack<T, E> bv[kRowUnroll];
            float av[kRowUnroll];
#pragma unroll
            for (int u = 0; u < kRowUnroll; u++) {
                const bool ok = j + u < len && colok;
                av[u] = 0.f;
#pragma unroll
                for (int e = 0; e < E; e++) bv[u].v[e] = T{};
                if (ok) {
                    const int c = colidx[beg + j + u];
                    av[u] = to_f32(val[beg + j + u]);
                    bv[u] = *reinterpret_cast<const Pack<T, E>*>(B + static_cast<size_t>(c) * N + col);
                }
            }
#pragma unroll
            for (int u = 0; u < kRowUnroll; u++) fma_pack<T, E>(acc, av[u], bv[u]);
        }
        if (row >= 0 && colok) store_row<E>(C + static_cast<size_t>(row) * N + col, acc);
        return;
    }

    // row / seg: all slots on one span
    if (logG == 6)
        accumulate_span<T, E, true>(acc, t.y, t.z, colidx, val, B, N, col, colok, lane, slot, logS);
    else
        accumulate_span<T, E, false>(acc, t.y, t.z, colidx, val, B, N, col, colok, lane, slot, logS);
    for (int off = 1 << logG; off < 64; off <<= 1)
#pragma unroll
        for (int e = 0; e < E; e++) acc[e] += __shfl_xor(acc[e], off);

    if (t.w == 0) {
        if (slot == 0 && colok) store_row<E>(C + static_cast<size_t>(t.x) * N + col, acc);
        return;
    }

    // seg: publish this segment, take a ticket; the last one sums in order.
    const int seg = t.w >> 2;
    const int4 lr = longrows[t.x];  // {row, first segment, segments, 0}
    if (slot == 0 && colok) {
        float* dst = partials + static_cast<size_t>(seg) * N + col;
#pragma unroll
        for (int e = 0; e < E; e++) dst[e] = acc[e];
    }
    __threadfence();
    int* ticket = tickets + static_cast<size_t>(t.x) * gridDim.y + blockIdx.y;
    int prev = 0;
    if (lane == 0) prev = atomicAdd(ticket, 1);
    prev = __shfl(prev, 0);
    if (prev != lr.z - 1) return;
    __threadfence();
    // Slot s adds segments s, s + S, ...; then the slots are combined as above.
#pragma unroll
    for (int e = 0; e < E; e++) acc[e] = 0.f;
    if (colok)
        for (int s = slot; s < lr.z; s += (1 << logS)) {
            const float* src = partials + static_cast<size_t>(lr.y + s) * N + col;
#pragma unroll
            for (int e = 0; e < E; e++) acc[e] += src[e];
        }
    for (int off = 1 << logG; off < 64; off <<= 1)
#pragma unroll
        for (int e = 0; e < E; e++) acc[e] += __shfl_xor(acc[e], off);
    if (slot == 0 && colok) store_row<E>(C + static_cast<size_t>(lr.x) * N + col, acc);
    if (lane == 0) *ticket = 0;  // ready for the next launch
}

}  // namespace tca
