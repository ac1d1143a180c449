// mfma_compact_kernel.hpp -- the dense-tile SpMM of mfma_dense_kernel.hpp
// with compacted A steps: a step keeps only its non-empty fragment cells.
//
// A step of the dense tiles is 8 row blocks x 64 lanes x 16 bytes (lane L of
// row block b: row 16 b + L % 16, columns 8 (L / 16) .. 8 (L / 16) + 7 of
// the step, the operand of one v_mfma_f32_16x16x32 lane).  At the densities
// the dense tiles serve (a few percent) about two cells in three are zero.
// The compact form keeps, per global step,
//   * amask[step][b]: bit L set when cell (b, L) holds an entry;
//   * a 4 KiB payload: the non-empty cells in (b, L) order, 16 bytes each,
//     at most 255 of them; cell 255 stays zero (plan time) and is what the
//     empty cells read.
// Cell (b, L) present sits at index sum_{b' < b} popcount(amask[b']) +
// popcount(amask[b] & ((1 << L) - 1)), i.e. a prefix of scalar popcounts
// plus v_mbcnt of the row block's mask.  The plan routes a matrix here only
// when every step fits; the pack kernel writes each run's values into the
// payloads (positions fixed by the plan, zero halves never written).
//
// Pipeline: that of the dense kernel (4 consumer wavefronts splitting the
// steps of an iteration, 4 producer wavefronts issuing only global -> LDS
// transfers, LB iterations of lookahead), with half the A bytes per step:
// producer p transfers 1 KiB chunk p of each step's payload and B rows
// 8 p .. 8 p + 7, 8 transfers per iteration.  The ring has LB + 1 slots, so a
// tile's slot stays valid during its own iteration: consumers keep only the
// A fragments double-buffered and read each B column block one block ahead
// of its MFMAs (fewer live registers than the dense kernel, whose four B
// blocks are read an iteration early).  The consumers load the masks of the
// step after next one iteration ahead (a vector load: lane b holds row
// block b's mask).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mfma_dense_kernel.hpp"

namespace tca {

constexpr int kCpCells = 256;                                 // payload cells per step (the last one zero)
constexpr int kCpATileBytes = kCpCells * 16;                  // 4 KiB per step
constexpr int kCpSlotBytes = kDnSteps * (kCpATileBytes + kDnBTileBytes);  // one tile of 4 steps
constexpr int kCpOps = 2 * kDnSteps;                          // transfers per producer and iteration

template <int LB>
constexpr int mfma_compact_lds_bytes() {
    constexpr int main = (LB + 1) * kCpSlotBytes;
    constexpr int red = kDnSteps * 32 * 64 * 16;  // four partial 128 x 64 fp32 tiles
    static_assert(main <= 160 * 1024 && red <= 160 * 1024, "LDS budget");
    return main > red ? main : red;
}

template <bool kBf16, bool kNatural, int LB>
__global__ __launch_bounds__(kDnThreads) void mfma_compact_kernel(MfmaArgs a) {
    static_assert(LB >= 3 && LB <= 4, "lookahead");
    constexpr int KS = kDnSteps, NS = LB + 1;
    __shared__ __attribute__((aligned(16))) char smem[mfma_compact_lds_bytes<LB>()];

    // all column blocks of a window on one XCD, as in the dense kernel
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
    const int niters = (nsteps + KS - 1) / KS;

    f32x4 acc[8][4];
#pragma unroll
    for (int b = 0; b < 8; b++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[b][c] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (wv < KS) {
        // ================= consumer w: fragments and MFMAs only =================
        const int w = wv;
        const int li = lane & 15, lh = lane >> 4;
        const int br = 8 * lh + (li >> 2);
        const int bx = bswz64(br), bh = (li & 3) >> 1;
        const char* const Afr = smem + w * kCpATileBytes;
        const uint16_t* const Bfr = reinterpret_cast<const uint16_t*>(smem + KS * kCpATileBytes + w * kDnBTileBytes) +
                                    br * kDmaBRow + 4 * (li & 1);
        const uint32_t zero_cell = kCpCells - 1;
        // Masks of this consumer's step of tile n (the window's last step past
        // its end): lane L holds the mask of row block L % 8.  A vector load,
        // so the barriers (which wait for this wavefront's LDS reads) never
        // wait for it; v_readlane takes each mask when it is used.
        const uint2* const mask_v = reinterpret_cast<const uint2*>(a.amask) + (lane & 7);
        auto load_masks = [&](const int n, uint2& mk) {
            const int j = min(KS * n + w, nsteps - 1);
            mk = mask_v[static_cast<size_t>(sbase + j) * 8];
        };
        auto mask_of = [&](const uint2& mk, const int b) {
            return (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(mk.y), b)))
                    << 32) |
                   static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(mk.x), b));
        };
        // A fragment of row block b of the tile in slot `sl` with mask m; `pre`
        // counts the cells of row blocks 0..b-1 and advances past block b
        auto read_a = [&](const int sl, const uint64_t m, uint32_t& pre) {
            const uint32_t at = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                          __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), pre));
            // the row block's mask is the lane predicate: present lanes take
            // their cell, the others the zero cell
            uint32_t idx;
            asm("v_cndmask_b32 %0, %1, %2, %3" : "=v"(idx) : "v"(zero_cell), "v"(at), "s"(m));
            pre += static_cast<uint32_t>(__builtin_popcountll(m));
            return *reinterpret_cast<const i32x4v*>(Afr + sl * kCpSlotBytes + 16 * idx);
        };
        // B fragment of column block c of the tile in slot `sl`
        auto read_b = [&](const int sl, const int c) {
            const uint16_t* Bp = Bfr + sl * (kCpSlotBytes / 2) + 8 * ((2 * c + bh) ^ bx);
            const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp));
            const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp + 4 * kDmaBRow));
            return i32x4v{__builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 0, 1)),
                          __builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 2, 3)),
                          __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 0, 1)),
                          __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 2, 3))};
        };
        // iteration i: MFMAs of tile i (A fragments `ca`, B column block 0 in
        // `cb0`, blocks 1..3 read from tile i's slot one block ahead); A
        // fragments of tile i + 1 into `na` with masks `mu`, its B block 0
        // into `nb0`; masks of tile i + 2 into `ml`.  Tile i's slot is
        // refilled only in iteration i + 1 (NS = LB + 1).
        auto iteration = [&](const int i, const i32x4v* ca, i32x4v* na, const i32x4v& cb0, i32x4v& nb0,
                             const uint2& mu, uint2& ml) {
            if (i >= 0) {
                if (KS * i + w < nsteps) {
                    const int sc = i % NS, sn = (i + 1) % NS;
                    load_masks(i + 2, ml);
                    uint32_t pre = 0;
                    i32x4v bc = cb0;
                    // column block c: its 8 MFMAs, with the reads of B block
                    // c + 1 (or the next tile's block 0) and of the next
                    // tile's A row blocks 2 c and 2 c + 1
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        i32x4v bn;
                        if (c < 3) bn = read_b(sc, c + 1);
                        else nb0 = read_b(sn, 0);
                        na[2 * c] = read_a(sn, mask_of(mu, 2 * c), pre);
                        na[2 * c + 1] = read_a(sn, mask_of(mu, 2 * c + 1), pre);
#pragma unroll
                        for (int b = 0; b < 8; b++) {
                            if constexpr (kBf16)
                                acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                    __builtin_bit_cast(bf16x8, ca[b]), __builtin_bit_cast(bf16x8, bc), acc[b][c], 0, 0, 0);
                            else
                                acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                    __builtin_bit_cast(f16x8, ca[b]), __builtin_bit_cast(f16x8, bc), acc[b][c], 0, 0, 0);
                        }
                        if (c < 3) bc = bn;
                    }
#pragma unroll
                    for (int g = 0; g < 16; g++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    }
                }
            } else if (i == -1) {
                uint32_t pre = 0;
#pragma unroll
                for (int b = 0; b < 8; b++) na[b] = read_a(0, mask_of(mu, b), pre);
                nb0 = read_b(0, 0);
                load_masks(1, ml);
            }
            __syncthreads();
        };
        i32x4v a0[8], a1[8], b00, b01;
        uint2 mA, mB;
        // the call at i = -1 is the first of its pair when LB is odd
        if constexpr (LB % 2) load_masks(0, mA);
        else load_masks(0, mB);
        int i = -LB;
        for (; i + 1 < niters; i += 2) {
            iteration(i, a0, a1, b00, b01, mA, mB);
            iteration(i + 1, a1, a0, b01, b00, mB, mA);
        }
        if (i < niters) iteration(i, a0, a1, b00, b01, mA, mB);
    } else {
        // ================= producer p: transfers only =================
        const int pw = wv - KS;
        const char* const Ag = static_cast<const char*>(a.adense);
        const char* const Bg = static_cast<const char*>(a.B);
        const char* const Zg = static_cast<const char*>(a.zeros);
        const int g8 = lane >> 3;
        int bcol;
        {
            const int row = 8 * pw + g8;
            const int col = c0 + 8 * ((lane & 7) ^ bswz64(row));
            bcol = col < a.N ? col * 2 : -1;
        }
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
        auto iteration = [&](const int i, uint32_t (&mu)[KS][8]) {
            const int n = i + LB;
            char* const slot = smem + (n % NS) * kCpSlotBytes;
#pragma unroll
            for (int sp = 0; sp < KS; sp++) {
                const int j = KS * n + sp;
                const bool in = j < nsteps;
                // payload chunk pw of the step (the window's last step past its end)
                const char* asrc = Ag + static_cast<size_t>(sbase + min(j, nsteps - 1)) * kCpATileBytes + pw * 1024 +
                                   16 * lane;
                dma_x4(asrc, lds_addr(slot + sp * kCpATileBytes + pw * 1024));
                uint32_t uo;
                if constexpr (kNatural) {
                    const int brow = kStepK * j + 8 * pw + g8;
                    uo = brow < a.K ? static_cast<uint32_t>(brow) * static_cast<uint32_t>(a.N) * 2u : kNoEntry;
                } else {
                    uint32_t m[8];
#pragma unroll
                    for (int r = 0; r < 8; r++) m[r] = __builtin_amdgcn_readfirstlane(mu[sp][r]);
                    const uint32_t u01 = (g8 & 1) ? m[1] : m[0], u23 = (g8 & 1) ? m[3] : m[2];
                    const uint32_t u45 = (g8 & 1) ? m[5] : m[4], u67 = (g8 & 1) ? m[7] : m[6];
                    const uint32_t u03 = (g8 & 2) ? u23 : u01, u47 = (g8 & 2) ? u67 : u45;
                    uo = (g8 & 4) ? u47 : u03;
                }
                const char* bsrc = (in && uo != kNoEntry && bcol >= 0) ? Bg + uo + bcol : Zg;
                dma_x4(bsrc, lds_addr(slot + KS * kCpATileBytes + sp * kDnBTileBytes + 8 * pw * (kDmaBRow * 2)));
            }
            if constexpr (!kNatural) load_meta(n + 2, mu);
            wait_vmcnt<(LB - 2) * kCpOps>();  // tile i + 2 has landed
            __builtin_amdgcn_s_barrier();
        };
        uint32_t mu0[KS][8], mu1[KS][8];
        if constexpr (!kNatural) {
            load_meta(0, mu0);
            load_meta(1, mu1);
        }
        int i = -LB;
        for (; i + 1 < niters; i += 2) {
            iteration(i, mu0);
            iteration(i + 1, mu1);
        }
        if (i < niters) iteration(i, mu0);
        wait_vmcnt<0>();
    }

    // ================= add the four partial tiles, store C =================
    __syncthreads();  // the ring is dead: the region holds the partial tiles now
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
        const int gi = t + kDnThreads * m;  // (block, lane) pair
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
