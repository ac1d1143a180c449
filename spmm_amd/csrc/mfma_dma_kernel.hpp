// mfma_dma_kernel.hpp -- condensed-tile SpMM on gfx950 matrix cores, K-split
// across the consumer wavefronts, B tiles staged by global -> LDS transfers.
//
// A workgroup owns a 128-row window of A and a 64-column block of C and
// walks the window's steps (32 condensed columns of A = 32 gathered rows of
// B).  Tall, narrow tiles halve the gathered B bytes per output against the
// 64 x 128 tiles of mfma_tile_kernel (mfma_kernel.hpp): the column union of
// 128 rows is barely larger than that of 64 rows on the matrices this path
// serves, so each gathered B row feeds twice the rows.
//
// Roles (8 wavefronts, one consumer and one producer per SIMD):
//   * consumer wavefront w takes step 4 i + w of iteration i.  It loads the
//     packed entries of its next step with ordinary global loads one
//     iteration ahead, scatters them into its private, double-buffered A
//     tile (before its MFMAs: VALU or LDS instructions placed between a
//     wavefront's back-to-back MFMAs wait for the MFMA in flight), reads its
//     A and B fragments and runs 8 row blocks x 4 column blocks = 32
//     v_mfma_f32_16x16x32 into 128 accumulators.  The four partial
//     128 x 64 tiles are added through LDS once at the end;
//   * producer wavefront p issues only global_load_lds_dwordx4 transfers (lane
//     L of one instruction writes 16 bytes at M0 + 16 L): rows 8 p .. 8 p + 7
//     of every step's B tile.  It executes no LDS instruction at all: an LDS
//     instruction of a wavefront waits until that wavefront's earlier LDS
//     transfers have landed (measured on the MI355X: ~360 cycles with 8 in
//     flight against ~60 without, and no wait behind another wavefront's
//     transfers), which would put the gather latency on the critical path.
//     Its B row offsets come through scalar loads issued after the transfers
//     that use the previous ones, and each iteration issues the same four
//     transfers, so one s_waitcnt vmcnt(N) retires exactly what is due.
// Pipeline, iteration i (one barrier each), lookahead LB = 3:
//   producers: issue B(i + 3); load the row offsets of B(i + 5); wait until
//              B(i + 1) has landed (B(i + 2), B(i + 3) stay in flight)
//   consumers: load the entries of A(i + 2); read A(i), B(i) fragments;
//              build A(i + 1) from the entries loaded in iteration i - 1;
//              MFMAs of step 4 i + w
// Rings: B 4 slots, A 2 slots per step of an iteration.
// The packed block of global step g sits at g * 256 * kSlots words (unused
// words kNoEntry).  Every transfer address is in bounds: padding columns,
// steps past the window and columns past N read 16 zero bytes
// (MfmaArgs::zeros).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mfma_kernel.hpp"

namespace tca {

constexpr int kDmaSteps = 4;      // steps per iteration = consumer wavefronts
constexpr int kDmaWinRows = 128;  // rows per window (8 row blocks of 16)
constexpr int kDmaTileCols = 64;  // columns of C per workgroup
constexpr int kDmaBRow = kDmaTileCols;           // halves per B-tile row in LDS (128 bytes)
constexpr int kDmaATile = kDmaWinRows * kStepK;  // halves of one A tile (fragment order)
constexpr int kDmaAElems = kDmaATile + 64;       // A tile + one dummy cell per lane
constexpr int kDmaLB = 3;                        // B lookahead (iterations)
constexpr int kDmaNB = kDmaLB + 1;               // B ring slots
constexpr int kDmaNA = 2;                        // A slots per step of an iteration
// Transfers a producer issues per iteration (one per step) and its wait
// count: B(i + 1) must land in iteration i while B(i + 2), B(i + 3) may not.
constexpr int kDmaOps = kDmaSteps;
constexpr int kDmaWait = (kDmaLB - 1) * kDmaOps;
// Nonzeros a step may hold under the LDS-DMA kernel (two 256-word slots).
constexpr int kDmaMaxStepEntries = 2 * 256;

// XOR permutation of the 16-byte pieces of a 128-byte B-tile row: with it the
// ds_read_b64_tr_b16 fragment reads (two passes of 32 lanes, 8 rows x 32
// bytes each) touch every LDS bank once.
__host__ __device__ constexpr int bswz64(int r) { return 2 * (((r >> 1) & 1) | ((r >> 2) & 2)); }

constexpr int mfma_dma_lds_bytes() {
    constexpr int main = kDmaNB * kDmaSteps * kStepK * kDmaBRow * 2 + kDmaSteps * kDmaNA * kDmaAElems * 2;
    constexpr int red = kDmaSteps * 32 * 64 * 16;  // four partial 128 x 64 fp32 tiles
    static_assert(main <= 160 * 1024 && red <= 160 * 1024, "LDS budget");
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
    constexpr int KS = kDmaSteps, NB = kDmaNB, NA = kDmaNA, LB = kDmaLB;
    constexpr int kBElems = kStepK * kDmaBRow;  // halves per B tile (4 KiB)
    constexpr int kEWords = 256 * kSlots;       // words of a step's packed block
    constexpr int kBBytes = NB * KS * kBElems * 2;
    __shared__ __attribute__((aligned(16))) char smem[mfma_dma_lds_bytes()];
    auto Bs = reinterpret_cast<uint16_t(*)[KS][kBElems]>(smem);                // [NB][KS][kBElems]
    auto As = reinterpret_cast<uint16_t(*)[NA][kDmaAElems]>(smem + kBBytes);  // [KS][NA][..]

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
        // packed entries of step 4 n + w; the load always reads a step of the
        // window and `valid` says whether they count (the select happens where
        // they are used, so the load is not waited for earlier).  Lane reads
        // words 4 lane .. 4 lane + 3 of each 256.
        auto load_entries = [&](int n, i32x4v* e4, bool& valid) {
            const int j = KS * n + w;
            valid = j >= 0 && j < nsteps;
            const int jc = valid ? j : 0;
            const i32x4v* ep =
                reinterpret_cast<const i32x4v*>(a.packed + static_cast<size_t>(sbase + jc) * kEWords) + lane;
#pragma unroll
            for (int k = 0; k < kSlots; k++) e4[k] = ep[64 * k];
        };
        int bslot = 0;  // B ring slot of iteration i: B(n) sits in slot n % NB
        // One iteration; `cur` holds the entries of A(i + 1) (loaded in
        // iteration i - 1), `nxt` receives those of A(i + 2).  The loop below
        // alternates the two buffers instead of copying, so the compiler waits
        // for a load only where its data is used.
        auto iteration = [&](const int i, const i32x4v* cur, bool cur_valid, i32x4v* nxt, bool& nxt_valid) {
            load_entries(i + 2, nxt, nxt_valid);
            const bool active = i >= 0 && KS * i + w < nsteps;
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
            if (i + 1 >= 0) {
                // A(i + 1) into slot (i + 1) & 1 after A(i - 1)'s cells there are cleared
                uint16_t* Aw = &As[w][(i + 1) & 1][0];
#pragma unroll
                for (int k = 0; k < 4 * kSlots; k++) Aw[pos_prev[k]] = 0;
#pragma unroll
                for (int k = 0; k < 4 * kSlots; k++) {
                    const uint32_t e = cur_valid ? static_cast<uint32_t>(cur[k / 4][k % 4]) : kNoEntry;
                    const bool ok = e != kNoEntry;
                    const int pos = ok ? static_cast<int>(e & 0xffffu) : pad;
                    Aw[pos] = ok ? static_cast<uint16_t>(e >> 16) : uint16_t(0);
                    pos_prev[k] = pos_cur[k];
                    pos_cur[k] = pos;
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (active) {
#pragma unroll
                for (int c = 0; c < 4; c++)
#pragma unroll
                    for (int b = 0; b < 8; b++) {
                        if constexpr (kBf16)
                            acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                __builtin_bit_cast(bf16x8, af[b]), __builtin_bit_cast(bf16x8, bq[c]), acc[b][c], 0, 0, 0);
                        else
                            acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                __builtin_bit_cast(f16x8, af[b]), __builtin_bit_cast(f16x8, bq[c]), acc[b][c], 0, 0, 0);
                    }
            }
            __syncthreads();
            if (i >= 0) bslot = bslot == NB - 1 ? 0 : bslot + 1;
        };
        i32x4v ent0[kSlots], ent1[kSlots];
        bool val0, val1;
        load_entries(1 - LB, ent0, val0);  // entries of A(i + 1) for the first iteration i = -LB
        int i = -LB;
        for (; i + 1 < niters; i += 2) {
            iteration(i, ent0, val0, ent1, val1);
            iteration(i + 1, ent1, val1, ent0, val0);
        }
        if (i < niters) iteration(i, ent0, val0, ent1, val1);
    } else {
        // ================= producer: B transfers only =================
        const int pw = wv - KS;
        const char* Bg = static_cast<const char*>(a.B);
        const char* Zg = static_cast<const char*>(a.zeros);
        // This lane fills row 8 pw + lane / 8 of every step's B tile, physical
        // piece lane % 8 (logical piece (lane % 8) ^ bswz64(row)).
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
        auto load_meta = [&](int ib, uint32_t (&mu)[KS][8]) {
#pragma unroll
            for (int sp = 0; sp < KS; sp++) {
                const int j = min(max(KS * ib + sp, 0), nsteps - 1);
                const cu32p up = ucols_c + static_cast<size_t>(sbase + j) * kStepK + 8 * pw;
#pragma unroll
                for (int r = 0; r < 8; r++) mu[sp][r] = up[r];
            }
        };
        // iteration i: B(i + LB) from `mu`, whose registers then receive the
        // offsets of B(i + LB + 2) (two buffers, so the scalar loads have a
        // whole iteration before their first use)
        auto iteration = [&](const int i, int& bslot, uint32_t (&mu)[KS][8]) {
#pragma unroll
            for (int sp = 0; sp < KS; sp++) {
                // rows 8 pw .. 8 pw + 7 of B(i + LB), step sp
                const bool in = KS * (i + LB) + sp < nsteps;
                // this lane's row offset: a select tree over the step's eight
                // values (held as values, so the selects stay v_cndmask
                // instead of an indexed private array)
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
            bslot = bslot == NB - 1 ? 0 : bslot + 1;
            load_meta(i + LB + 2, mu);
            wait_vmcnt<kDmaWait>();  // B(i + 1) has landed
            // A plain barrier: this wavefront has no LDS instruction to order,
            // and waiting for its scalar loads here would stall the barrier.
            __builtin_amdgcn_s_barrier();
        };
        int bslot = 0;  // ring slot of B(i + LB): B(n) sits in slot n % NB
        uint32_t mu0[KS][8], mu1[KS][8];
        load_meta(0, mu0);
        load_meta(1, mu1);
        int i = -LB;
        for (; i + 1 < niters; i += 2) {
            iteration(i, bslot, mu0);
            iteration(i + 1, bslot, mu1);
        }
        if (i < niters) iteration(i, bslot, mu0);
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
