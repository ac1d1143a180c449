// mfma_common.hpp -- what the matrix-core tile kernels share: the condensed
// step and tile geometry, the fragment-order A-tile cell, the kernel argument
// block, the per-run pack kernel and the global -> LDS transfer helpers.
//
// A row window of 128 rows is condensed: U = the sorted union of its nonzero
// columns, padded to a multiple of 32.  The window's sub-matrix A_w
// (128 x |U|) is multiplied as tiles, C[rows, cols] = A_w * B[U, cols], one
// 32-wide step of U at a time, on v_mfma_f32_16x16x32_{f16,bf16}; a workgroup
// owns one window and one 64-column block of C.  The kernels differ in how a
// step's A tile reaches LDS (mfma_pair_kernel.hpp: scattered entries;
// mfma_dense_kernel.hpp: dense tiles built per run; mfma_compact_kernel.hpp:
// the non-empty cells of the dense tiles), the B tile is always gathered by
// global -> LDS transfers.
//
// No counterpart in the reference's structure: the reference feeds one
// nonzero column at a time through m16n8k8 and keeps 1/8 of each MMA
// (src/our_spmm.cu:112-136); here the contraction runs over the window's
// condensed columns, so every MFMA output is used.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "planner.hpp"
#include "row_kernel.hpp"

namespace tca {

constexpr int kStepK = 32;                            // condensed columns per step (MFMA K)
constexpr int kDmaWinRows = 128;                      // rows per window (8 row blocks of 16)
constexpr int kDmaTileCols = 64;                      // columns of C per workgroup
constexpr int kDmaBRow = kDmaTileCols;                // halves per B-tile row in LDS (128 bytes)
constexpr int kDmaATile = kDmaWinRows * kStepK;       // halves of one A tile (fragment order)
constexpr int kDmaMaxStepEntries = 2 * 256;           // nonzeros a step of the paired kernel may hold

// A-tile cell of (row, step column) in MFMA fragment order: row block,
// 8-column group, row, column (each fragment read is one contiguous 1 KiB).
__host__ __device__ inline int a_cell(int r, int k) {
    return (r >> 4) * 512 + (k >> 3) * 128 + (r & 15) * 8 + (k & 7);
}
constexpr uint32_t kNoEntry = 0xffffffffu;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef int i32x4v __attribute__((ext_vector_type(4)));
typedef int i32x2v __attribute__((ext_vector_type(2)));

struct MfmaArgs {
    const int4* windows;     // {first row, steps, first global step, first nonzero}
    const uint32_t* ucols;   // [global step][32] byte offset of the B row of each condensed column
                             // (row * N * 2), 0xffffffff = padding
    const int* eoff;         // [global step + 1] entry range of each step
    const uint32_t* packed;  // per entry: A-tile cell | value bits << 16 (written each run by
                             // mfma_pack_kernel), placed per step as the paired kernel reads them
    const void* B;
    float* C;
    int M, N;
    int col_blocks;          // blockIdx.x = window * col_blocks + column block
    uint32_t B_bytes, packed_bytes, ucols_bytes, eoff_bytes;
    const void* zeros;       // 16 zero bytes (source of padding B pieces)
    const i32x2v* emeta;     // [global step] {first word of the packed block, groups of 64 entries} (paired kernel)
    const void* adense;      // [global step] dense A tile, 8 KiB in fragment order (dense kernel)
    int n_windows;           // windows (dense kernel: its workgroup -> window mapping)
    int K;                   // rows of B (dense kernel, windows in natural column order)
    const uint64_t* amask;   // [global step][8] non-empty cells of each row block (compact dense kernel)
};

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// Per run: pair each MFMA entry's A-tile cell with its value, in the packed
// array's word order, so the tile kernel loads one coalesced word per entry
// (the values are read once here instead of once per column block).  Word x
// gets cell[x] | val[src[x]] << 16; words that hold no entry (src[x] < 0)
// keep their plan-time content: cell[x] with value bits 0, or kNoEntry where
// cell[x] is 0xffff.  Four words per thread: the loads of src and cell and
// the stores are coalesced, only the value loads gather (from the CSR range
// of one window at a time).
__global__ __launch_bounds__(256) void mfma_pack_kernel(const int* __restrict__ src, const uint16_t* __restrict__ cell,
                                                        int n, const uint16_t* __restrict__ val,
                                                        uint32_t* __restrict__ packed) {
    const int x = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (x >= n) return;
    auto word = [&](int s, uint32_t c) -> uint32_t {
        const uint32_t hi = s >= 0 ? static_cast<uint32_t>(val[s]) : (c == 0xffffu ? 0xffffu : 0u);
        return c | (hi << 16);
    };
    if (x + 4 <= n) {
        const int4 s = *reinterpret_cast<const int4*>(src + x);
        const uint2 c = *reinterpret_cast<const uint2*>(cell + x);
        *reinterpret_cast<uint4*>(packed + x) = uint4{word(s.x, c.x & 0xffffu), word(s.y, c.x >> 16),
                                                       word(s.z, c.y & 0xffffu), word(s.w, c.y >> 16)};
    } else {
        for (int k = x; k < n; k++) packed[k] = word(src[k], cell[k]);
    }
}

// XOR permutation of the 16-byte pieces of a 128-byte B-tile row: with it the
// ds_read_b64_tr_b16 fragment reads (two passes of 32 lanes, 8 rows x 32
// bytes each) touch every LDS bank once.
__host__ __device__ constexpr int bswz64(int r) { return 2 * (((r >> 1) & 1) | ((r >> 2) & 2)); }

// One global -> LDS transfer per lane: 16 bytes from `g` to LDS byte address
// m0 + 16 * lane.  M0 is set by the compiler through the "{m0}" operand; the
// s_nop covers the M0 -> LDS-transfer hazard.  The compiler does not see the
// transfer: the kernel orders it with explicit vmcnt waits.
__device__ __forceinline__ void dma_x4(const void* g, uint32_t m0) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(m0) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <typename P>
__device__ __forceinline__ uint32_t lds_addr(P* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)p));
}

}  // namespace tca
