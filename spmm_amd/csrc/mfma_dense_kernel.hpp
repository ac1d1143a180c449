// mfma_dense_kernel.hpp -- condensed-tile SpMM on gfx950 matrix cores with
// dense A tiles: both operands reach LDS by global -> LDS transfers, so no
// wavefront writes LDS during the main loop.
//
// Tiles and steps are those of the paired kernel: a workgroup
// owns a 128-row window of A and a 64-column block of C, a step is 32
// condensed columns, an iteration is 4 steps, K-split over four consumers
// (step 4 i + w of iteration i goes to consumer w), partial tiles added
// through LDS at the end in a fixed order.  What differs is where A comes
// from: the plan keeps a dense copy of every condensed window (8 KiB per
// step: 128 rows x 32 halves in MFMA fragment order, zero where A has no
// entry), and dense_pack_kernel writes only this run's values into it (the
// zero cells never change).  The tile kernel then streams A like B:
//   * consumer wavefront w only reads fragments and issues MFMAs: during the
//     32 v_mfma_f32_16x16x32 of tile i it issues the 16 fragment reads of
//     tile i + 1 (8 contiguous 1 KiB A reads, 8 transposing B reads), one
//     read after every second MFMA, into a second register set;
//   * producer wavefront p issues only global_load_lds_dwordx4 transfers
//     (lane L of one instruction writes 16 bytes at M0 + 16 L): A fragments
//     2 p and 2 p + 1 and B rows 8 p .. 8 p + 7 of every step, three
//     iterations ahead, into a 3-slot ring.  It executes no LDS instruction:
//     an LDS instruction of a wavefront waits until that wavefront's earlier
//     transfers have landed.  Each iteration issues the same 12 transfers, so
//     one s_waitcnt vmcnt(12) retires exactly the tile that is due.
// Pipeline, iteration i (one barrier each), tile n = steps 4 n .. 4 n + 3:
//   producers: issue tile i + 3 into slot i % 3; load the B row offsets of
//              tile i + 5; wait until tile i + 2 has landed
//   consumers: MFMAs of tile i (registers); read fragments of tile i + 1
// Slot i % 3 held tile i, whose fragments the consumers read in iteration
// i - 1, before that iteration's barrier.
// Workgroups are dealt to the 8 XCDs round robin (workgroup x on XCD
// x mod 8); the kernel maps them so that all column blocks of a window run
// on one XCD, whose L2 then fetches the window's dense A tiles once.
// Every transfer address is in bounds: steps past the window reread its last
// step (not used), padding columns and columns past N read 16 zero bytes
// (MfmaArgs::zeros).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mfma_common.hpp"

namespace tca {

constexpr int kDnSteps = 4;                                   // steps per iteration = consumers
constexpr int kDnThreads = 512;                               // 4 consumer + 4 producer wavefronts
constexpr int kDnATileBytes = kDmaATile * 2;                  // 8 KiB per step
constexpr int kDnBTileBytes = kStepK * kDmaBRow * 2;          // 4 KiB per step
constexpr int kDnSlotBytes = kDnSteps * (kDnATileBytes + kDnBTileBytes);  // one tile of 4 steps
constexpr int kDnSlots = 3;                                   // ring slots
constexpr int kDnLB = 3;                                      // transfer lookahead (iterations)
constexpr int kDnOps = 3 * kDnSteps;                          // transfers per producer and iteration
constexpr int kDnWait = (kDnLB - 2) * kDnOps;                 // tile i + 2 lands in iteration i
constexpr size_t kDenseMaxBytes = size_t(2) << 30;            // dense tiles a plan may keep
constexpr double kNaturalCover = 0.85;  // windows covering this share of K keep all of K in column order

constexpr int mfma_dense_lds_bytes() {
    constexpr int main = kDnSlots * kDnSlotBytes;
    constexpr int red = kDnSteps * 32 * 64 * 16;  // four partial 128 x 64 fp32 tiles
    static_assert(main <= 160 * 1024 && red <= 160 * 1024, "LDS budget");
    return main > red ? main : red;
}

// Workgroups of the dense tile kernel: a multiple of the XCD count.
inline int mfma_dense_grid(int windows, int col_blocks) {
    const int per = (windows * col_blocks + kXcds - 1) / kXcds;
    return per * kXcds;
}

// Per run: this run's values into the plan's dense A tiles.  pos[x] is the
// half index of entry x in the dense tiles (entries sorted by it, so a
// wavefront's stores fall in few lines), src[x] its CSR index.
__global__ __launch_bounds__(256) void dense_pack_kernel(const int* __restrict__ src, const uint32_t* __restrict__ pos,
                                                         int n, const uint16_t* __restrict__ val,
                                                         uint16_t* __restrict__ adense) {
    const int x = blockIdx.x * 256 + threadIdx.x;
    if (x < n) adense[pos[x]] = val[src[x]];
}

// kNatural: the windows span all of K in column order (step j = columns
// 32 j .. 32 j + 31), so a B row's offset is its row number times the row
// pitch and the producers need no row-offset table.
template <bool kBf16, bool kNatural>
__global__ __launch_bounds__(kDnThreads) void mfma_dense_kernel(MfmaArgs a) {
    constexpr int KS = kDnSteps, LB = kDnLB, NS = kDnSlots;
    __shared__ __attribute__((aligned(16))) char smem[mfma_dense_lds_bytes()];

    // all column blocks of a window on one XCD (see above)
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
        const char* const Afr = smem + w * kDnATileBytes + 16 * lane;
        const uint16_t* const Bfr = reinterpret_cast<const uint16_t*>(smem + KS * kDnATileBytes + w * kDnBTileBytes) +
                                    br * kDmaBRow + 4 * (li & 1);
        // fragments of the tile in slot `sl`: f[0..7] A row blocks, f[8..11] B column blocks
        auto read = [&](const int sl, i32x4v* fr) {
            const char* Ab = Afr + sl * kDnSlotBytes;
#pragma unroll
            for (int b = 0; b < 8; b++) fr[b] = *reinterpret_cast<const i32x4v*>(Ab + 1024 * b);
            const uint16_t* Bb = Bfr + sl * (kDnSlotBytes / 2);
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint16_t* Bp = Bb + 8 * ((2 * c + bh) ^ bx);
                const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp));
                const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp + 4 * kDmaBRow));
                fr[8 + c] = i32x4v{__builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 0, 1)),
                                   __builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 2, 3)),
                                   __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 0, 1)),
                                   __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 2, 3))};
            }
        };
        // iteration i: MFMAs of tile i from `cf`, fragments of tile i + 1 into `nf`
        auto iteration = [&](const int i, const i32x4v* cf, i32x4v* nf) {
            if (i >= 0) {
                if (KS * i + w < nsteps) {
                    read((i + 1) % NS, nf);
#pragma unroll
                    for (int c = 0; c < 4; c++)
#pragma unroll
                        for (int b = 0; b < 8; b++) {
                            if constexpr (kBf16)
                                acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                    __builtin_bit_cast(bf16x8, cf[b]), __builtin_bit_cast(bf16x8, cf[8 + c]), acc[b][c],
                                    0, 0, 0);
                            else
                                acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                    __builtin_bit_cast(f16x8, cf[b]), __builtin_bit_cast(f16x8, cf[8 + c]), acc[b][c],
                                    0, 0, 0);
                        }
                    // one fragment read after every second MFMA
#pragma unroll
                    for (int g = 0; g < 16; g++) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    }
                }
            } else if (i == -1) {
                read(0, nf);
            }
            __syncthreads();
        };
        i32x4v f0[12], f1[12];
        int i = -LB;
        for (; i + 1 < niters; i += 2) {
            iteration(i, f0, f1);
            iteration(i + 1, f1, f0);
        }
        if (i < niters) iteration(i, f0, f1);
    } else {
        // ================= producer p: transfers only =================
        const int pw = wv - KS;
        const char* const Ag = static_cast<const char*>(a.adense);
        const char* const Bg = static_cast<const char*>(a.B);
        const char* const Zg = static_cast<const char*>(a.zeros);
        // This lane fills row 8 pw + lane / 8 of every step's B tile, physical
        // piece lane % 8 (logical piece (lane % 8) ^ bswz64(row)).
        const int g8 = lane >> 3;
        int bcol;
        {
            const int row = 8 * pw + g8;
            const int col = c0 + 8 * ((lane & 7) ^ bswz64(row));
            bcol = col < a.N ? col * 2 : -1;
        }
        // B row offsets of rows 8 pw .. 8 pw + 7 for the steps of tile ib, by
        // scalar loads (constant address space), so vmcnt counts the transfers alone.
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
        // iteration i: tile n = i + LB from `mu`, whose registers then receive
        // the offsets of tile n + 2 (two buffers, so the scalar loads have a
        // whole iteration before their first use)
        auto iteration = [&](const int i, uint32_t (&mu)[KS][8]) {
            const int n = i + LB;
            char* const slot = smem + (n % NS) * kDnSlotBytes;
#pragma unroll
            for (int sp = 0; sp < KS; sp++) {
                const int j = KS * n + sp;
                const bool in = j < nsteps;
                // A fragments 2 pw, 2 pw + 1 of the step (the window's last step past its end)
                const char* asrc = Ag + static_cast<size_t>(sbase + min(j, nsteps - 1)) * kDnATileBytes +
                                   2 * pw * 1024 + 16 * lane;
                char* const adst = slot + sp * kDnATileBytes + 2 * pw * 1024;
                dma_x4(asrc, lds_addr(adst));
                dma_x4(asrc + 1024, lds_addr(adst + 1024));
                // B rows 8 pw .. 8 pw + 7: this lane's row offset by a select tree
                // (natural order: the row is 32 j + 8 pw + lane / 8)
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
                dma_x4(bsrc, lds_addr(slot + KS * kDnATileBytes + sp * kDnBTileBytes + 8 * pw * (kDmaBRow * 2)));
            }
            if constexpr (!kNatural) load_meta(n + 2, mu);
            wait_vmcnt<kDnWait>();  // tile i + 2 has landed
            // A plain barrier: this wavefront has no LDS instruction to order.
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
