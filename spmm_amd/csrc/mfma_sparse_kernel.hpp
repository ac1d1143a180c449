// mfma_sparse_kernel.hpp -- condensed-tile SpMM on gfx950's sparse matrix
// cores (v_smfmac_f32_16x16x64_{f16,bf16}).
//
// The planner (plan_mfma24) reorders each 128-row window's condensed
// columns so that every aligned group of 4 holds at most two nonzeros of
// any row; the window's A is then exactly 2:4 and is kept compressed: per
// step of 64 condensed columns, 8 KiB of values ([row block 8][lane 64][8
// halves], the v_smfmac A operand of each lane) and 2 KiB of index words
// ([row block][lane], both 16-bit halves).  The index words are fixed per
// plan; dense_pack_kernel writes this run's values into the (otherwise
// zero) value tiles.  Against dense condensed tiles this halves the A bytes
// and the matrix-core instructions per step.
//
// A workgroup owns a window x 64 columns of C.  Consumer wavefront w takes
// step 2 i + (w & 1) of iteration i for rows 64 (w >> 1) .. + 63 (4 row
// blocks x 4 column blocks = 16 v_smfmac): during the smfmacs of tile i it
// reads the fragments of tile i + 1 (4 A, 4 index words, 16 transposing B
// reads; B of a 64-row step is two dense 32-row fragments per column
// block).  Producer wavefront p issues only global_load_lds_dwordx4
// transfers for step p / 2 of a tile: A row blocks 4 (p % 2) .. + 3, half
// p % 2 of the index words, B rows 32 (p % 2) .. + 31 — 9 transfers per
// iteration, four iterations ahead, into a 4-slot ring of 36 KiB tiles; it
// waits until tile i + 2 has landed (vmcnt(18)) before each barrier.  The
// two K halves are added through LDS at the end in a fixed order.
// All columns of a window run on one XCD (workgroup x on XCD x mod 8).
// Every transfer address is in bounds: steps past the window reread its last
// step (not used), padding columns and columns past N read zeros.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mfma_dense_kernel.hpp"
#include "sparse24_kernel.hpp"

namespace tca {

constexpr int kSpSteps = 2;                   // steps per iteration (K split of the consumers)
constexpr int kSpThreads = 512;               // 4 consumer + 4 producer wavefronts
constexpr int kSpStepK = 64;                  // condensed columns per step
constexpr int kSpATile = 8 * 1024;            // compressed A values of one step
constexpr int kSpITile = 2 * 1024;            // index words of one step
constexpr int kSpBTile = 64 * kDmaBRow * 2;   // B of one step: 64 rows x 64 halves
constexpr int kSpStepBytes = kSpATile + kSpITile + kSpBTile;
constexpr int kSpSlotBytes = kSpSteps * kSpStepBytes;
constexpr int kSpSlots = 4;
constexpr int kSpLB = 4;                      // transfer lookahead (iterations)
constexpr int kSpOps = 9;                     // transfers per producer and iteration
constexpr int kSpWait = (kSpLB - 2) * kSpOps; // tile i + 2 lands in iteration i

constexpr int mfma_sparse_lds_bytes() {
    constexpr int main = kSpSlots * kSpSlotBytes;
    static_assert(main <= 160 * 1024, "LDS budget");
    return main;
}

template <bool kBf16>
__global__ __launch_bounds__(kSpThreads) void mfma_sparse_kernel(MfmaArgs a) {
    constexpr int LB = kSpLB, NS = kSpSlots;
    __shared__ __attribute__((aligned(16))) char smem[mfma_sparse_lds_bytes()];

    const int total = a.n_windows * a.col_blocks;
    const int per = (total + kXcds - 1) / kXcds;
    const int f = static_cast<int>(blockIdx.x % kXcds) * per + static_cast<int>(blockIdx.x / kXcds);
    if (f >= total) return;  // whole workgroup, before any barrier
    const int t = threadIdx.x;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int lane = t & 63;
    const int cb = f % a.col_blocks;
    const int4 win = a.windows[f / a.col_blocks];
    const int row0 = win.x, nsteps = win.y, sbase = win.z;
    __builtin_assume(nsteps >= 1);
    const int c0 = cb * kDmaTileCols;
    const int niters = (nsteps + kSpSteps - 1) / kSpSteps;

    f32x4 acc[4][4];
#pragma unroll
    for (int b = 0; b < 4; b++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[b][c] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int kpar = wv & 1, rh = (wv >> 1) & 1;
    if (wv < 4) {
        // ================= consumer: fragments and sparse MFMAs =================
        const int li = lane & 15, lh = lane >> 4;
        const int br = 8 * lh + (li >> 2);
        const int bx = bswz64(br), bh = (li & 3) >> 1;
        struct Frag {
            i32x4v a[4];
            int ix[4];
            i32x4v b[2][4];
        };
        auto read = [&](const int sl, Frag& fr) {
            const char* st = smem + sl * kSpSlotBytes + kpar * kSpStepBytes;
#pragma unroll
            for (int q = 0; q < 4; q++)
                fr.a[q] = *reinterpret_cast<const i32x4v*>(st + (4 * rh + q) * 1024 + 16 * lane);
#pragma unroll
            for (int q = 0; q < 4; q++)
                fr.ix[q] = *reinterpret_cast<const int*>(st + kSpATile + (4 * rh + q) * 256 + 4 * lane);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint16_t* Bfr = reinterpret_cast<const uint16_t*>(st + kSpATile + kSpITile + h * 32 * kDmaBRow * 2) +
                                      br * kDmaBRow + 4 * (li & 1);
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const uint16_t* Bp = Bfr + 8 * ((2 * c + bh) ^ bx);
                    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp));
                    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp + 4 * kDmaBRow));
                    fr.b[h][c] = i32x4v{__builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 0, 1)),
                                        __builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 2, 3)),
                                        __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 0, 1)),
                                        __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 2, 3))};
                }
            }
        };
        typedef int i32x8v __attribute__((ext_vector_type(8)));
        // iteration i: smfmacs of tile i from `cf`, fragments of tile i + 1 into `nf`
        auto iteration = [&](const int i, const Frag& cf, Frag& nf) {
            if (i >= 0) {
                if (kSpSteps * i + kpar < nsteps) {
                    read((i + 1) % NS, nf);
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const i32x8v b8 = __builtin_shufflevector(cf.b[0][c], cf.b[1][c], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            if constexpr (kBf16)
                                acc[q][c] = __builtin_amdgcn_smfmac_f32_16x16x64_bf16(
                                    __builtin_bit_cast(bf16x8, cf.a[q]), __builtin_bit_cast(bf16x16, b8), acc[q][c],
                                    cf.ix[q], 0, 0);
                            else
                                acc[q][c] = __builtin_amdgcn_smfmac_f32_16x16x64_f16(
                                    __builtin_bit_cast(f16x8, cf.a[q]), __builtin_bit_cast(f16x16, b8), acc[q][c],
                                    cf.ix[q], 0, 0);
                        }
                    }
                    // 24 fragment reads among the 16 smfmacs
#pragma unroll
                    for (int g = 0; g < 8; g++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    }
                }
            } else if (i == -1) {
                read(0, nf);
            }
            __syncthreads();
        };
        Frag f0, f1;
        int i = -LB;
        for (; i + 1 < niters; i += 2) {
            iteration(i, f0, f1);
            iteration(i + 1, f1, f0);
        }
        if (i < niters) iteration(i, f0, f1);
    } else {
        // ================= producer p: transfers only =================
        const int pw = wv - 4;
        const int sp = pw >> 1, hp = pw & 1;  // step of the tile, half (A row blocks, index words, B rows)
        const char* const Ag = static_cast<const char*>(a.adense);
        const char* const Ig = reinterpret_cast<const char*>(a.packed);  // index words
        const char* const Bg = static_cast<const char*>(a.B);
        const char* const Zg = static_cast<const char*>(a.zeros);
        const int g8 = lane >> 3;
        // B row 8 d + g8 of half hp (d = 0..3): physical piece lane % 8 holds
        // logical piece (lane % 8) ^ bswz64(row within the 32-row half)
        int bcol[4];
#pragma unroll
        for (int d = 0; d < 4; d++) {
            const int col = c0 + 8 * ((lane & 7) ^ bswz64(8 * d + g8));
            bcol[d] = col < a.N ? col * 2 : -1;
        }
        typedef __attribute__((address_space(4))) const uint32_t* cu32p;
        const cu32p ucols_c = (cu32p)(a.ucols);
        // B row offsets of rows 32 hp .. 32 hp + 31 of step sp of tile ib
        auto load_meta = [&](int ib, uint32_t (&mu)[4][8]) {
            const int j = min(max(kSpSteps * ib + sp, 0), nsteps - 1);
            const cu32p up = ucols_c + static_cast<size_t>(sbase + j) * kSpStepK + 32 * hp;
#pragma unroll
            for (int d = 0; d < 4; d++)
#pragma unroll
                for (int r = 0; r < 8; r++) mu[d][r] = up[8 * d + r];
        };
        auto iteration = [&](const int i, uint32_t (&mu)[4][8]) {
            const int n = i + LB;
            char* const st = smem + (n % NS) * kSpSlotBytes + sp * kSpStepBytes;
            const int j = kSpSteps * n + sp;
            const bool in = j < nsteps;
            const size_t gs = static_cast<size_t>(sbase + min(j, nsteps - 1));
            // A row blocks 4 hp .. 4 hp + 3 and half hp of the index words
            const char* asrc = Ag + gs * kSpATile + (4 * hp) * 1024 + 16 * lane;
#pragma unroll
            for (int q = 0; q < 4; q++) dma_x4(asrc + q * 1024, lds_addr(st + (4 * hp + q) * 1024));
            dma_x4(Ig + gs * kSpITile + hp * 1024 + 16 * lane, lds_addr(st + kSpATile + hp * 1024));
            // B rows 32 hp + 8 d + g8
            char* const bdst = st + kSpATile + kSpITile + hp * 32 * kDmaBRow * 2;
#pragma unroll
            for (int d = 0; d < 4; d++) {
                uint32_t m[8];
#pragma unroll
                for (int r = 0; r < 8; r++) m[r] = __builtin_amdgcn_readfirstlane(mu[d][r]);
                const uint32_t u01 = (g8 & 1) ? m[1] : m[0], u23 = (g8 & 1) ? m[3] : m[2];
                const uint32_t u45 = (g8 & 1) ? m[5] : m[4], u67 = (g8 & 1) ? m[7] : m[6];
                const uint32_t u03 = (g8 & 2) ? u23 : u01, u47 = (g8 & 2) ? u67 : u45;
                const uint32_t uo = (g8 & 4) ? u47 : u03;
                const char* bsrc = (in && uo != kNoEntry && bcol[d] >= 0) ? Bg + uo + bcol[d] : Zg;
                dma_x4(bsrc, lds_addr(bdst + 8 * d * (kDmaBRow * 2)));
            }
            load_meta(n + 2, mu);
            wait_vmcnt<kSpWait>();  // tile i + 2 has landed
            __builtin_amdgcn_s_barrier();
        };
        uint32_t mu0[4][8], mu1[4][8];
        load_meta(0, mu0);
        load_meta(1, mu1);
        int i = -LB;
        for (; i + 1 < niters; i += 2) {
            iteration(i, mu0);
            iteration(i + 1, mu1);
        }
        if (i < niters) iteration(i, mu0);
        wait_vmcnt<0>();
    }

    // ================= add the two K halves, store C =================
    __syncthreads();  // the ring is dead: the region holds the odd-step partial tiles
    f32x4* Red = reinterpret_cast<f32x4*>(smem);  // [row half][row block * 4 + column block][lane]
    if (wv < 4 && kpar == 1) {
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int c = 0; c < 4; c++) Red[(rh * 16 + q * 4 + c) * 64 + lane] = acc[q][c];
    }
    __syncthreads();
    if (wv < 4 && kpar == 0) {
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const f32x4 s = acc[q][c] + Red[(rh * 16 + q * 4 + c) * 64 + lane];
                const int col = c0 + 16 * c + (lane & 15);
                if (col >= a.N) continue;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = row0 + 64 * rh + 16 * q + 4 * (lane >> 4) + r;
                    if (row < a.M) __builtin_nontemporal_store(s[r], a.C + static_cast<size_t>(row) * a.N + col);
                }
            }
    }
}

}  // namespace tca
