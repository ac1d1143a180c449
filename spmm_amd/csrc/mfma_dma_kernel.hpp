// mfma_dma_kernel.hpp -- condensed-tile SpMM on gfx950 matrix cores, K-split
// across the consumer wavefronts, operands staged by global -> LDS transfers.
//
// A workgroup owns a 128-row window of A and a 64-column block of C and
// walks the window's steps (32 condensed columns of A = 32 gathered rows of
// B).  Tall, narrow tiles halve the gathered B bytes per output against the
// 64 x 128 tiles of mfma_tile_kernel (mfma_kernel.hpp): the column union of
// 128 rows is barely larger than that of 64 rows on the matrices this path
// serves, so each gathered B row feeds twice the rows.
//   * consumer wavefront w (one per SIMD) takes step 4 i + w of iteration i:
//     8 row blocks x 4 column blocks = 32 v_mfma_f32_16x16x32 into 128
//     accumulators.  Each step's A and B tiles are read from LDS by one
//     wavefront only; the four partial 128 x 64 tiles are added through LDS
//     once at the end;
//   * each consumer builds its own A tiles: it reads its step's packed entries
//     from LDS and scatters them into a private, double-buffered A tile;
//   * producer wavefronts only issue global_load_lds_dwordx4 transfers (lane
//     L of one instruction writes 16 bytes at M0 + 16 L): per step one 1 KiB
//     instruction of B rows per producer and 256 entry words per instruction.
//     Their plan metadata (B row offsets) comes through scalar loads one
//     iteration ahead, so the only vector-memory operations of a producer
//     are its transfers: each iteration issues the same number N of them,
//     and s_waitcnt vmcnt(N) after issuing retires exactly the previous
//     iteration's transfers.  (An LDS transfer costs a producer wavefront
//     ~100 cycles to issue whatever its width, so the kernel issues as few
//     and as wide ones as it can.)
// Pipeline, iteration i (one barrier each):
//   producers: issue B(i + 2), entries(i + 3); wait for B(i + 1), entries(i + 2)
//   consumers: MFMAs of step 4 i + w with A(i) and B(i); build A(i + 1)
// Rings: B 3 slots, entries 3 slots, A 2 slots per consumer.
// Packed entries of global step g sit at g * 256 * kSlots (unused words
// kNoEntry), so a step's entries are one or two aligned 1 KiB transfers.
// Every transfer address is in bounds: padding columns, steps past the
// window and columns past N read 16 zero bytes (MfmaArgs::zeros), which also
// stand for the entries of steps past the window (cell 0, value 0).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mfma_kernel.hpp"

namespace tca {

constexpr int kDmaSteps = 4;     // steps per iteration = consumer wavefronts
constexpr int kDmaBRing = 3;     // B tile slots (iterations)
constexpr int kDmaERing = 3;     // packed-entry slots (iterations)
constexpr int kDmaARing = 2;     // A tile slots per consumer
constexpr int kDmaWinRows = 128;  // rows per window (8 row blocks of 16)
constexpr int kDmaTileCols = 64;  // columns of C per workgroup
constexpr int kDmaBRow = kDmaTileCols;               // halves per B-tile row in LDS (128 bytes)
constexpr int kDmaATile = kDmaWinRows * kStepK;      // halves of one A tile (fragment order)
constexpr int kDmaAElems = kDmaATile + 64;           // A tile + one dummy cell per lane

// XOR permutation of the 16-byte pieces of a 128-byte B-tile row: with it the
// ds_read_b64_tr_b16 fragment reads (two passes of 32 lanes, 8 rows x 32
// bytes each) touch every LDS bank once.
__host__ __device__ constexpr int bswz64(int r) { return 2 * (((r >> 1) & 1) | ((r >> 2) & 2)); }

template <int kSlots>
constexpr int mfma_dma_lds_bytes() {
    constexpr int main = kDmaBRing * kDmaSteps * kStepK * kDmaBRow * 2 + kDmaERing * kDmaSteps * 256 * kSlots * 4 +
                         kDmaSteps * kDmaARing * kDmaAElems * 2;
    constexpr int red = kDmaSteps * 32 * 64 * 16;  // four partial 128 x 64 fp32 tiles
    return main > red ? main : red;
}

// One global -> LDS transfer per lane: 16 bytes from `g` to LDS byte address
// m0 + 16 * lane.  M0 is set by the compiler through the "{m0}" operand; the
// s_nop covers the M0 -> LDS-transfer hazard.
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

template <bool kBf16, int kSlots>
__global__ __launch_bounds__(kMfmaThreads) void mfma_dma_kernel(MfmaArgs a) {
    static_assert(kSlots == 1 || kSlots == 2, "entry slots per step (x 256)");
    constexpr int KS = kDmaSteps, NB = kDmaBRing, NE = kDmaERing, NA = kDmaARing;
    constexpr int kBElems = kStepK * kDmaBRow;  // halves per B tile (4 KiB)
    constexpr int kEWords = 256 * kSlots;       // entry words per step
    constexpr int kBBytes = NB * KS * kBElems * 2;
    constexpr int kEBytes = NE * KS * kEWords * 4;
    // Transfers per producer wavefront and iteration: one B instruction per
    // step, kSlots entry instructions for one step.
    constexpr int kOps = KS + kSlots;
    __shared__ __attribute__((aligned(16))) char smem[mfma_dma_lds_bytes<kSlots>()];
    auto Bs = reinterpret_cast<uint16_t(*)[KS][kBElems]>(smem);                         // [NB][KS][kBElems]
    auto Es = reinterpret_cast<uint32_t(*)[KS][kEWords]>(smem + kBBytes);                // [NE][KS][kEWords]
    auto As = reinterpret_cast<uint16_t(*)[NA][kDmaAElems]>(smem + kBBytes + kEBytes);  // [KS][NA][..]

    const int t = threadIdx.x;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);  // wavefront (uniform)
    const int lane = t & 63;
    const int cb = blockIdx.x % a.col_blocks;
    const int4 win = a.windows[blockIdx.x / a.col_blocks];
    const int row0 = win.x, nsteps = win.y, sbase = win.z;
    __builtin_assume(nsteps >= 1);
    const int c0 = cb * kDmaTileCols;
    const int niters = (nsteps + KS - 1) / KS;

    for (int i = t * 8; i < KS * NA * kDmaAElems; i += kMfmaThreads * 8)
        *reinterpret_cast<i32x4v*>(&As[0][0][0] + i) = i32x4v{0, 0, 0, 0};
    __syncthreads();

    f32x4 acc[8][4];
#pragma unroll
    for (int b = 0; b < 8; b++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[b][c] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (wv < KS) {
        // ================= consumer w: step 4 i + w of every iteration =================
        const int w = wv;
        const int li = lane & 15, lh = lane >> 4;
        const int br = 8 * lh + (li >> 2);
        const int bx = bswz64(br), bh = (li & 3) >> 1;
        const int b_row = br * kDmaBRow + 4 * (li & 1);
        const int pad = kDmaATile + lane;
        int pos_prev[4 * kSlots], pos_cur[4 * kSlots];
#pragma unroll
        for (int k = 0; k < 4 * kSlots; k++) pos_prev[k] = pos_cur[k] = pad;
        int bslot = 0;  // B ring slot of iteration i
        int eslot = 1;  // entry ring slot of iteration i + 1
        for (int i = -3; i < niters; i++) {
            uint32_t ent[4 * kSlots];
            if (i + 1 >= 0) {
                // entries of A(i + 1): lane reads words 4 lane .. 4 lane + 3 of each 256
#pragma unroll
                for (int k = 0; k < kSlots; k++) {
                    const i32x4v e4 = *reinterpret_cast<const i32x4v*>(&Es[eslot][w][256 * k + 4 * lane]);
#pragma unroll
                    for (int q = 0; q < 4; q++) ent[4 * k + q] = static_cast<uint32_t>(e4[q]);
                }
            }
            // Fragments of step 4 i + w are all read first (the MFMAs then run
            // back to back); the A(i + 1) scatter goes between MFMA groups.
            const bool active = i >= 0 && KS * i + w < nsteps;
            const bool build = i + 1 >= 0;
            i32x4v af[8], bq[4];
            if (active) {
                const uint16_t* Ab = &As[w][i & 1][8 * lane];
                const uint16_t* Bb = &Bs[bslot][w][b_row];
#pragma unroll
                for (int b = 0; b < 8; b++) af[b] = *reinterpret_cast<const i32x4v*>(Ab + 512 * b);
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const uint16_t* Bp = Bb + 8 * ((2 * c + bh) ^ bx);
                    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp));
                    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp + 4 * kDmaBRow));
                    bq[c] = i32x4v{__builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 0, 1)),
                                   __builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 2, 3)),
                                   __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 0, 1)),
                                   __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 2, 3))};
                }
            }
            auto mfmas = [&](int c) {
#pragma unroll
                for (int b = 0; b < 8; b++) {
                    if constexpr (kBf16)
                        acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8, af[b]), __builtin_bit_cast(bf16x8, bq[c]), acc[b][c], 0, 0, 0);
                    else
                        acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(f16x8, af[b]), __builtin_bit_cast(f16x8, bq[c]), acc[b][c], 0, 0, 0);
                }
            };
            // A(i + 1) goes to slot (i + 1) & 1 after A(i - 1)'s cells there are cleared
            uint16_t* Aw = &As[w][(i + 1) & 1][0];
            if (active) mfmas(0);
            __builtin_amdgcn_sched_barrier(0);
            if (build) {
#pragma unroll
                for (int k = 0; k < 4 * kSlots; k++) Aw[pos_prev[k]] = 0;
            }
            __builtin_amdgcn_sched_barrier(0);
            if (active) mfmas(1);
            __builtin_amdgcn_sched_barrier(0);
            if (build) {
#pragma unroll
                for (int k = 0; k < 4 * kSlots; k++) {
                    const uint32_t e = ent[k];
                    const bool ok = e != kNoEntry;
                    const int pos = ok ? static_cast<int>(e & 0xffffu) : pad;
                    Aw[pos] = ok ? static_cast<uint16_t>(e >> 16) : uint16_t(0);
                    pos_prev[k] = pos_cur[k];
                    pos_cur[k] = pos;
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (active) {
                mfmas(2);
                mfmas(3);
            }
            __syncthreads();
            if (i >= 0) bslot = bslot == NB - 1 ? 0 : bslot + 1;
            eslot = eslot == NE - 1 ? 0 : eslot + 1;
        }
    } else {
        // ================= producer: transfers only =================
        const int pw = wv - KS;
        const char* Bg = static_cast<const char*>(a.B);
        const char* Zg = static_cast<const char*>(a.zeros);
        // B transfer role: rows 8 pw .. 8 pw + 7 of every step; this lane fills
        // row 8 pw + lane / 8, physical piece lane % 8 (logical piece
        // (lane % 8) ^ bswz64(row)).
        const int g8 = lane >> 3;
        int bcol;
        {
            const int row = 8 * pw + g8;
            const int col = c0 + 8 * ((lane & 7) ^ bswz64(row));
            bcol = col < a.N ? col * 2 : -1;
        }
        // B row offsets of rows 8 pw .. 8 pw + 7 for the steps of B(ib), by
        // scalar loads (constant address space: uniform loads from it are
        // scalar loads, which keeps vmcnt counting the transfers alone).
        typedef __attribute__((address_space(4))) const uint32_t* cu32p;
        const cu32p ucols_c = (cu32p)(a.ucols);
        uint32_t mu[KS][8];
        auto load_meta = [&](int ib) {
#pragma unroll
            for (int sp = 0; sp < KS; sp++) {
                const int j = min(max(KS * ib + sp, 0), nsteps - 1);
                const cu32p up = ucols_c + static_cast<size_t>(sbase + j) * kStepK + 8 * pw;
#pragma unroll
                for (int r = 0; r < 8; r++) mu[sp][r] = up[r];
            }
        };
        int bslot = 0;  // ring slot of B(i + 2)
        int eslot = 0;  // ring slot of entries(i + 3)
        load_meta(-1);
        for (int i = -3; i < niters; i++) {
            if (i + 2 >= 0) {
#pragma unroll
                for (int sp = 0; sp < KS; sp++) {
                    const bool in = KS * (i + 2) + sp < nsteps;
                    // this lane's row offset: a select tree over the step's
                    // eight values (held as values, so the selects stay
                    // v_cndmask instead of an indexed private array)
                    uint32_t m[8];
#pragma unroll
                    for (int r = 0; r < 8; r++) m[r] = __builtin_amdgcn_readfirstlane(mu[sp][r]);
                    const uint32_t u01 = (g8 & 1) ? m[1] : m[0], u23 = (g8 & 1) ? m[3] : m[2];
                    const uint32_t u45 = (g8 & 1) ? m[5] : m[4], u67 = (g8 & 1) ? m[7] : m[6];
                    const uint32_t u03 = (g8 & 2) ? u23 : u01, u47 = (g8 & 2) ? u67 : u45;
                    const uint32_t uo = (g8 & 4) ? u47 : u03;
                    const char* src = (in && uo != kNoEntry && bcol >= 0) ? Bg + uo + bcol : Zg;
                    dma_x4(src, lds_addr(&Bs[bslot][sp][kDmaBRow * 8 * pw]));
                }
            }
            {
                // entries of step 4 (i + 3) + pw
                const int j = KS * (i + 3) + pw;
                const uint32_t* ep = a.packed + static_cast<size_t>(sbase + j) * kEWords + 4 * lane;
#pragma unroll
                for (int k = 0; k < kSlots; k++)
                    dma_x4(j < nsteps ? static_cast<const void*>(ep + 256 * k) : static_cast<const void*>(Zg),
                           lds_addr(&Es[eslot][pw][256 * k]));
            }
            // next iteration's metadata (after the transfers that used this one)
            load_meta(i + 3);
            wait_vmcnt<kOps>();  // everything issued before this iteration has landed
            __syncthreads();
            if (i + 2 >= 0) bslot = bslot == NB - 1 ? 0 : bslot + 1;
            eslot = eslot == NE - 1 ? 0 : eslot + 1;
        }
        wait_vmcnt<0>();
    }

    // ================= add the four partial tiles, store C =================
    __syncthreads();  // rings are dead: the region holds the partial tiles now
    f32x4* Red = reinterpret_cast<f32x4*>(smem);  // [consumer][row block * 4 + column block][lane]
    if (wv < KS) {
#pragma unroll
        for (int b = 0; b < 8; b++)
#pragma unroll
            for (int c = 0; c < 4; c++) Red[(wv * 32 + b * 4 + c) * 64 + lane] = acc[b][c];
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < 4; m++) {
        const int gi = t + kMfmaThreads * m;  // (block, lane) pair
        const int blk = gi >> 6, l = gi & 63;
        const f32x4 s = ((Red[blk * 64 + l] + Red[(32 + blk) * 64 + l]) + Red[(64 + blk) * 64 + l]) +
                        Red[(96 + blk) * 64 + l];
        const int col = c0 + 16 * (blk & 3) + (l & 15);
        if (col >= a.N) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = row0 + 16 * (blk >> 2) + 4 * (l >> 4) + r;
            if (row < a.M) __builtin_nontemporal_store(s[r], a.C + static_cast<size_t>(row) * a.N + col);
        }
    }
}

}  // namespace tca
