// mfma_pair_kernel.hpp -- condensed-tile SpMM on gfx950 matrix cores with one
// MFMA wavefront and one staging wavefront per SIMD.
//
// Tiles and steps of mfma_common.hpp: a workgroup owns a 128-row window of A
// and a 64-column block of C and walks the window's steps of 32 condensed
// columns, K-split over four consumers (step 4 i + w of iteration i goes to
// consumer w), partial tiles added through LDS at the end.  Who does what:
//   * consumer wavefront w only reads fragments and issues MFMAs.  During the
//     32 v_mfma_f32_16x16x32 of step i it issues the 16 fragment reads of its
//     step i + 1 (8 A reads of 16 bytes, 8 transposing B reads), interleaved
//     one read per two MFMAs, into a second register set;
//   * staging wavefront h = w (wavefronts 4..7) builds consumer w's tiles two
//     iterations ahead: it loads the step's B rows (4 x 16 bytes per lane) and
//     its packed entries with ordinary global loads, writes the B tile with
//     ds_write_b128 and scatters the entries into the A tile after clearing
//     the cells of the tile that held the slot before.
// On the MI355X a wavefront's own VALU and LDS instructions do not overlap its
// MFMAs (each adds its issue time), while another wavefront's on the same
// SIMD do, without slowing the MFMAs: this split puts all staging work beside
// the matrix pipe instead of in front of it.
//
// Packed entries (written by mfma_pack_kernel each run): step g's block
// starts at word emeta[g].x and holds whole chunks of 256 words; entry e of
// the step sits at word 256 (e / 256) + 4 (e % 64) + (e / 64) % 4 of it
// (pair_entry_word), so the 16-byte load q of lane L returns entries
// 256 q + 64 c + L (c = 0..3): component c of load q is group 4 q + c of 64
// entries, and only the emeta[g].y groups that the step has are scattered.
// Entry word = LDS byte address of the cell (slot 0 of the consumer's tile
// pair; bits 0..15) | value << 16.  Words past the step's count point at the
// lane's own dummy cell with value 0.
// B-row offsets (MfmaArgs::ucols) come permuted per step: word 4 r + k of the
// step's 32 is condensed column r + 8 k, so lane L loads its four rows
// L / 8 + 8 k with one 16-byte load.
//
// Pipeline, iteration i (one barrier each), tile n = step 4 n + w:
//   consumer w: MFMAs of tile i (registers); read fragments of tile i + 1
//   staging w:  write tile i + 2 into slot i & 1 (its data loaded in i - 2);
//               load the B-row offsets of tile i + 5, the data of tile i + 4,
//               the entry range of tile i + 6
// The loads are issued in an order where every wait the compiler places
// retires only loads at least one iteration old (vmcnt counts in order).
// LDS: A tiles [consumer][slot] at offset 0 (8320 bytes each: 4096 cells in
// fragment order + 64 dummy cells), B tiles [slot][consumer] after them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mfma_common.hpp"

namespace tca {

constexpr int kPairSteps = 4;                                   // steps per iteration = consumers
constexpr int kPairThreads = 512;                               // 4 consumers + 4 staging wavefronts
constexpr int kPairATileBytes = (kDmaATile + 64) * 2;           // A tile + one dummy cell per lane
constexpr int kPairABytes = kPairSteps * 2 * kPairATileBytes;   // A tiles, two slots per consumer
constexpr int kPairBTileBytes = kStepK * kDmaBRow * 2;          // 32 rows x 64 halves
constexpr int kPairBBytes = 2 * kPairSteps * kPairBTileBytes;   // B tiles, two slots per consumer
constexpr int kPairGroup = 64;                                  // entries per scatter instruction
constexpr int kPairChunk = 256;                                 // entries per 16-byte load of the 64 lanes

// Word of entry e inside its step's block.
__host__ __device__ constexpr int pair_entry_word(int e) {
    return kPairChunk * (e / kPairChunk) + 4 * (e % kPairGroup) + (e / kPairGroup) % 4;
}

// Entry address of fragment-order cell `cell` (or dummy cell 4096 + lane) of
// consumer `w`'s tile pair, slot 0.
__host__ __device__ constexpr uint32_t pair_cell_addr(int w, int cell) {
    return static_cast<uint32_t>(w * 2 * kPairATileBytes + 2 * cell);
}
static_assert(pair_cell_addr(kPairSteps - 1, kDmaATile + 63) < 65536u, "entry addresses fit 16 bits");

constexpr int mfma_pair_lds_bytes() {
    constexpr int main = kPairABytes + kPairBBytes;
    constexpr int red = kPairSteps * 32 * 64 * 16;  // four partial 128 x 64 fp32 tiles
    static_assert(main <= 160 * 1024 && red <= 160 * 1024, "LDS budget");
    return main > red ? main : red;
}

// G = groups of 64 entries a step may hold (4 or 8).
template <bool kBf16, int G>
__global__ __launch_bounds__(kPairThreads) void mfma_pair_kernel(MfmaArgs a) {
    static_assert(G == 4 || G == 8, "entry groups per step (one or two 16-byte loads)");
    constexpr int KS = kPairSteps;
    __shared__ __attribute__((aligned(16))) char smem[mfma_pair_lds_bytes()];

    const int t = threadIdx.x;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int lane = t & 63;
    const int cb = blockIdx.x % a.col_blocks;
    const int4 win = a.windows[blockIdx.x / a.col_blocks];
    const int row0 = win.x, nsteps = win.y, sbase = win.z;
    __builtin_assume(nsteps >= 1);
    const int c0 = cb * kDmaTileCols;
    const int niters = (nsteps + KS - 1) / KS;

    for (int i = t * 16; i < kPairABytes; i += kPairThreads * 16)
        *reinterpret_cast<i32x4v*>(smem + i) = i32x4v{0, 0, 0, 0};
    __syncthreads();

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
        const char* const Afr = smem + w * 2 * kPairATileBytes + 16 * lane;
        const uint16_t* const Bfr =
            reinterpret_cast<const uint16_t*>(smem + kPairABytes + w * kPairBTileBytes) + br * kDmaBRow + 4 * (li & 1);
        // fragments of the tile in `slot`: f[0..7] A row blocks, f[8..11] B column blocks
        auto read = [&](const int slot, i32x4v* f) {
            const char* Ab = Afr + slot * kPairATileBytes;
#pragma unroll
            for (int b = 0; b < 8; b++) f[b] = *reinterpret_cast<const i32x4v*>(Ab + 1024 * b);
            const uint16_t* Bb = Bfr + slot * (KS * kPairBTileBytes / 2);
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint16_t* Bp = Bb + 8 * ((2 * c + bh) ^ bx);
                const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp));
                const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp + 4 * kDmaBRow));
                f[8 + c] = i32x4v{__builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 0, 1)),
                                  __builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 2, 3)),
                                  __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 0, 1)),
                                  __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 2, 3))};
            }
        };
        // iteration i: MFMAs of tile i from `cf`, fragments of tile i + 1
        // (slot `nslot` = (i + 1) & 1) into `nf`
        auto iteration = [&](const int i, const int nslot, const i32x4v* cf, i32x4v* nf) {
            if (i >= 0) {
                if (KS * i + w < nsteps) {
                    read(nslot, nf);
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
        int i = -4;
        for (; i + 1 < niters; i += 2) {
            iteration(i, 1, f0, f1);
            iteration(i + 1, 0, f1, f0);
        }
        if (i < niters) iteration(i, 1, f0, f1);
    } else {
        // ================= staging wavefront for consumer w =================
        const int w = wv - KS;
        const char* const Bg = static_cast<const char*>(a.B);
        const char* const Zg = static_cast<const char*>(a.zeros);
        // Lane L stages rows L / 8 + 8 k (k = 0..3) of every B tile, physical
        // piece L % 8, which holds logical piece (L % 8) ^ bswz64(row).
        // bswz64 reads row bits 1 and 3, so rows L / 8 + 8 k of even and of
        // odd k take different pieces.
        const int g8 = lane >> 3;
        int bcol[2];
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int col = c0 + 8 * ((lane & 7) ^ bswz64(g8 + 8 * k));
            bcol[k] = col < a.N ? col * 2 : -1;
        }
        char* const Bst = smem + kPairABytes + w * kPairBTileBytes + g8 * (kDmaBRow * 2) + (lane & 7) * 16;
        const uint32_t* const packed = a.packed;

        // loads of tile n clamp to a step of the window (tiles past its end are never written)
        auto gstep = [&](int n) { return sbase + min(KS * n + w, nsteps - 1); };
        auto load_meta = [&](int n, i32x2v& m) { m = a.emeta[gstep(n)]; };
        auto load_ucols = [&](int n, i32x4v& u) {
            u = *reinterpret_cast<const i32x4v*>(a.ucols + static_cast<size_t>(gstep(n)) * kStepK + 4 * g8);
        };
        auto load_data = [&](int n, const i32x2v m, const i32x4v u, i32x4v* bv, i32x4v* ev, int& ng) {
            const bool valid = KS * n + w < nsteps;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int bc = bcol[k & 1];
                const uint32_t uk = static_cast<uint32_t>(u[k]);
                const char* src = (valid && uk != kNoEntry && bc >= 0) ? Bg + uk + bc : Zg;
                bv[k] = *reinterpret_cast<const i32x4v*>(src);
            }
            const int e0 = __builtin_amdgcn_readfirstlane(m.x);
            ng = __builtin_amdgcn_readfirstlane(m.y);
            const int nq = (ng + 3) / 4;
            const i32x4v* ep = reinterpret_cast<const i32x4v*>(packed + e0) + lane;
#pragma unroll
            for (int q = 0; q < G / 4; q++) ev[q] = ep[(kPairChunk / 4) * min(q, nq - 1)];
        };
        // tile n into slot `slot` (= n & 1): B tile, clear the cells of the
        // slot's previous tile, scatter the entries
        auto write_tile = [&](int n, const int slot, const i32x4v* bv, const i32x4v* ev, int ng, uint32_t* clr,
                              int& cng) {
            if (n < 0 || KS * n + w >= nsteps) return;
            char* const Bt = Bst + slot * KS * kPairBTileBytes;
#pragma unroll
            for (int k = 0; k < 4; k++) *reinterpret_cast<i32x4v*>(Bt + 8 * (kDmaBRow * 2) * k) = bv[k];
            char* const As = smem + slot * kPairATileBytes;
#pragma unroll
            for (int k = 0; k < G; k++)
                if (k < cng) *reinterpret_cast<uint16_t*>(As + clr[k]) = 0;
#pragma unroll
            for (int k = 0; k < G; k++)
                if (k < ng) {
                    const uint32_t e = static_cast<uint32_t>(ev[k / 4][k % 4]);
                    const uint32_t ad = e & 0xffffu;
                    *reinterpret_cast<uint16_t*>(As + ad) = static_cast<uint16_t>(e >> 16);
                    clr[k] = ad;
                }
            cng = ng;
        };
        // buffers by tile parity: data (bv, ev, ng), entry range m, B-row
        // offsets u; clear lists by slot
        i32x4v bv0[4], bv1[4], ev0[G / 4], ev1[G / 4], u0, u1;
        i32x2v m0, m1;
        uint32_t clr0[G], clr1[G];
        int ng0 = 0, ng1 = 0, cng0 = 0, cng1 = 0;
        // iteration i: everything of parity p = i & 1 except the B-row offsets
        // loaded for tile i + 5 (parity 1 - p)
        auto iteration = [&](const int i, const int p, i32x4v* bv, i32x4v* ev, int& ng, i32x2v& m, const i32x4v& u,
                             i32x4v& u_next, uint32_t* clr, int& cng) {
            write_tile(i + 2, p, bv, ev, ng, clr, cng);
            load_ucols(i + 5, u_next);
            load_data(i + 4, m, u, bv, ev, ng);
            load_meta(i + 6, m);
            __syncthreads();
        };
        load_ucols(0, u0);
        load_meta(0, m0);
        load_meta(1, m1);
        int i = -4;
        for (; i + 1 < niters; i += 2) {
            iteration(i, 0, bv0, ev0, ng0, m0, u0, u1, clr0, cng0);
            iteration(i + 1, 1, bv1, ev1, ng1, m1, u1, u0, clr1, cng1);
        }
        if (i < niters) iteration(i, 0, bv0, ev0, ng0, m0, u0, u1, clr0, cng0);
    }

    // ================= add the four partial tiles, store C =================
    __syncthreads();  // tiles are dead: the region holds the partial tiles now
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
        const int gi = t + kPairThreads * m;  // (block, lane) pair
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
