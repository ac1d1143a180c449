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
//     accumulators, nothing else (VALU or LDS instructions placed between a
//     wavefront's back-to-back MFMAs wait for the MFMA in flight).  Each
//     step's A and B tiles are read from LDS by one wavefront only; the four
//     partial 128 x 64 tiles are added through LDS once at the end;
//   * producer wavefront p issues global_load_lds_dwordx4 transfers (lane L
//     of one instruction writes 16 bytes at M0 + 16 L): the packed block of
//     step 4 i + p (its entries and, in the last 32 words, the byte offsets
//     of the step's 32 B rows) and its share (8 rows) of every step's B
//     tile.  The B row offsets of a step are read from its packed block in
//     LDS, one ds_read_b32 per lane and step, so a producer issues no other
//     memory operation and builds each address with a few VALU operations.
//     It also builds the A tile of step 4 i + p from the entries it
//     transferred itself (each lane reads back its own 16 bytes, so its own
//     vmcnt wait is the only synchronisation) into that consumer's
//     double-buffered A slot.  Each iteration issues the same transfers in
//     the same order, and one s_waitcnt vmcnt(N) retires exactly what is due.
// Pipeline, iteration i (one barrier each), lookahead LB = 3 (one entry slot
// per thread) or 2 (two), LE = LB + 2:
//   producers: issue blocks(i + LE), then B(i + LB) (row offsets from
//              blocks(i + LB)); build A(i + 1) from blocks(i + 1); wait
//              until blocks(i + LE - 1) and B(i + 1) have landed
//   consumers: MFMAs of step 4 i + w with A(i) and B(i)
// Rings: B LB + 1 slots, blocks LE slots, A 2 slots per step of an iteration.
// The packed block of global step g sits at g * 256 * kSlots words: up to
// 256 * kSlots - 32 entries (unused words kNoEntry), then the 32 B row
// offsets (kNoEntry for padding columns).
// Every transfer address is in bounds: padding columns, steps past the
// window and columns past N read 16 zero bytes (MfmaArgs::zeros), which also
// stand for the entries of steps past the window (cell 0, value 0).
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
constexpr int kDmaStepMeta = kStepK;             // B row offsets at the end of a step's packed block

// Pipeline shape by entry slots (256 words each) per step.
template <int kSlots>
struct MfmaDmaShape {
    static constexpr int kLB = kSlots == 1 ? 3 : 2;  // B lookahead (iterations)
    static constexpr int kLE = kLB + 2;              // packed-block lookahead
    static constexpr int kNB = kLB + 1;              // B ring slots
    static constexpr int kNE = kLE;                  // packed-block ring slots
    static constexpr int kNA = 2;                    // A slots per step of an iteration
    static constexpr int kEWords = 256 * kSlots;     // words of a step's packed block
};
// Nonzeros a step may hold under the LDS-DMA kernel (two slots).
constexpr int kDmaMaxStepEntries = 2 * 256 - kDmaStepMeta;

// XOR permutation of the 16-byte pieces of a 128-byte B-tile row: with it the
// ds_read_b64_tr_b16 fragment reads (two passes of 32 lanes, 8 rows x 32
// bytes each) touch every LDS bank once.
__host__ __device__ constexpr int bswz64(int r) { return 2 * (((r >> 1) & 1) | ((r >> 2) & 2)); }

template <int kSlots>
constexpr int mfma_dma_lds_bytes() {
    using SH = MfmaDmaShape<kSlots>;
    constexpr int main = SH::kNB * kDmaSteps * kStepK * kDmaBRow * 2 + SH::kNE * kDmaSteps * SH::kEWords * 4 +
                         kDmaSteps * SH::kNA * kDmaAElems * 2;
    constexpr int red = kDmaSteps * 32 * 64 * 16;  // four partial 128 x 64 fp32 tiles
    static_assert(main <= 160 * 1024, "LDS budget");
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
    using SH = MfmaDmaShape<kSlots>;
    constexpr int KS = kDmaSteps, NB = SH::kNB, NE = SH::kNE, NA = SH::kNA, LB = SH::kLB, LE = SH::kLE;
    constexpr int kBElems = kStepK * kDmaBRow;  // halves per B tile (4 KiB)
    constexpr int kEWords = SH::kEWords;        // words of a step's packed block
    constexpr int kMetaAt = kEWords - kDmaStepMeta;
    constexpr int kBBytes = NB * KS * kBElems * 2;
    constexpr int kEBytes = NE * KS * kEWords * 4;
    // Transfers per producer wavefront and iteration: kSlots for one packed
    // block, then one B instruction per step.  The wait of iteration i must
    // retire the block issued in iteration i - 1 and B(i + 1): with LB = 3 the
    // B instructions of iteration i - 1 may stay in flight, with LB = 2 they
    // are B(i + 1) themselves.
    constexpr int kOps = kSlots + KS;
    constexpr int kWait = LB == 3 ? KS + kOps : kOps;
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
        int bslot = 0;  // B ring slot of iteration i
        for (int i = -LE; i < niters; i++) {
            if (i >= 0 && KS * i + w < nsteps) {
                i32x4v af[8], bq[4];
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
        const int pad = kDmaATile + lane;
        int pos_prev[4 * kSlots], pos_cur[4 * kSlots];
#pragma unroll
        for (int k = 0; k < 4 * kSlots; k++) pos_prev[k] = pos_cur[k] = pad;
        // B(n) sits in ring slot n mod NB.  Every iteration issues the same
        // transfers, the first ones B(-2), B(-1) from the zero bytes, so that
        // one wait count holds from the first iteration on.
        int bslot = NB - 2;
        int eslot = 0;             // block ring slot of blocks(i + LE): blocks(n) sit in slot n % NE
        for (int i = -LE; i < niters; i++) {
            {
                // packed block of step 4 (i + LE) + p (issued first: see the wait below)
                const int j = KS * (i + LE) + pw;
                const uint32_t* ep = a.packed + static_cast<size_t>(sbase + j) * kEWords + 4 * lane;
#pragma unroll
                for (int k = 0; k < kSlots; k++)
                    dma_x4(j < nsteps ? static_cast<const void*>(ep + 256 * k) : static_cast<const void*>(Zg),
                           lds_addr(&Es[eslot][pw][256 * k]));
            }
            {
                // rows 8 p .. 8 p + 7 of B(i + LB); row offsets from blocks(i + LB),
                // which landed by every producer's wait of iteration i - 1
                const bool real = i + LB >= 0;
                const int em = eslot >= LE - LB ? eslot - (LE - LB) : eslot + LB;  // (i + LB) % NE
                uint32_t uo[KS];
#pragma unroll
                for (int sp = 0; sp < KS; sp++) uo[sp] = real ? Es[em][sp][kMetaAt + 8 * pw + g8] : kNoEntry;
#pragma unroll
                for (int sp = 0; sp < KS; sp++) {
                    const bool in = real && KS * (i + LB) + sp < nsteps;
                    const char* src = (in && uo[sp] != kNoEntry && bcol >= 0) ? Bg + uo[sp] + bcol : Zg;
                    dma_x4(src, lds_addr(&Bs[bslot][sp][kDmaBRow * 8 * pw]));
                }
                bslot = bslot == NB - 1 ? 0 : bslot + 1;
            }
            if (i + 1 >= 0) {
                // A(i + 1) of step 4 (i + 1) + p into consumer p's slot (i + 1) & 1,
                // after clearing A(i - 1)'s cells there.  Every lane reads back
                // the 16 bytes it transferred; the block's last 32 words (lanes
                // 56..63 of its last 256) are the B row offsets, not entries.
                const int er = eslot + 1 - (eslot + 1 >= NE ? NE : 0);  // (i + 1) % NE
                uint32_t ent[4 * kSlots];
#pragma unroll
                for (int k = 0; k < kSlots; k++) {
                    const i32x4v e4 = *reinterpret_cast<const i32x4v*>(&Es[er][pw][256 * k + 4 * lane]);
                    const bool meta = k == kSlots - 1 && lane >= 56;
#pragma unroll
                    for (int q = 0; q < 4; q++) ent[4 * k + q] = meta ? kNoEntry : static_cast<uint32_t>(e4[q]);
                }
                uint16_t* Aw = &As[pw][(i + 1) & 1][0];
#pragma unroll
                for (int k = 0; k < 4 * kSlots; k++) Aw[pos_prev[k]] = 0;
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
            wait_vmcnt<kWait>();
            __syncthreads();
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
