// bell_kernel.hpp -- SpMM C = A * B over a Blocked-ELL A on gfx950 matrix
// cores (fp16 / bf16 inputs, fp32 accumulation and output).
//
// Blocked-ELL is the format the reference hands to cusparseSpMM for its
// block baseline (src/spmm_cusparse.cu:201-342; layout in tca_host.h):
// every block is a dense BS x BS tile, so the format feeds the matrix cores
// with no condensing.  A workgroup owns one block row (BS rows) and 256
// columns of C; wavefront w owns columns 64 w .. 64 w + 63.  Per ELL block e
// of the block row:
//   * the BS rows of B it multiplies (block column colind[e] * BS ..) x the
//     workgroup's 256 columns are staged in LDS, double-buffered: every
//     thread loads BS / 8 pieces of 16 bytes (coalesced, 512 bytes per row)
//     one block ahead and writes them after the MFMAs of the current block.
//     The LDS tile is [32-row step][64-column block][32 rows][64 halves]
//     with the 16-byte pieces of each 128-byte row XOR-permuted by bswz64,
//     so the transposing fragment reads (ds_read_b64_tr_b16) are
//     conflict-free, exactly as in the condensed-tile kernels;
//   * the A fragments come straight from global memory: lane l of fragment
//     (row block rf, step ks) needs row 16 rf + l % 16, columns
//     32 ks + 8 (l / 16) .. + 7 of the block, 16 contiguous bytes of the
//     row-major ELL values, loaded one block ahead;
//   * v_mfma_f32_16x16x32_{f16,bf16}: (BS / 16) row blocks x 4 column
//     blocks x (BS / 32) steps per wavefront.
// Blocks are added in ELL order, so every output is one MFMA chain in a
// fixed order (deterministic).  B rows past K and columns past N load as
// zeros (buffer range checks); rows past M and columns past N are not
// stored.  Padding blocks (colind -1) end the block row's list.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mfma_common.hpp"

namespace tca {

constexpr int kBellThreads = 256;  // 4 wavefronts
constexpr int kBellCols = 256;     // columns of C per workgroup

struct BellArgs {
    const int* colind;   // [block rows][ell_blocks] block column, -1 = padding
    const void* values;  // [block rows * BS][ell_blocks * BS] row-major
    const void* B;       // K x N row-major
    float* C;            // M x N row-major
    int M, N, ell_blocks;
    int col_groups;      // workgroups per block row: blockIdx.x = block row * col_groups + group
    uint32_t B_bytes;    // K * N * 2
};

template <int BS>
constexpr int bell_lds_bytes() {
    return 2 * BS * kBellCols * 2;
}

template <bool kBf16, int BS>
__global__ __launch_bounds__(kBellThreads) void bell_mfma_kernel(BellArgs a) {
    static_assert(BS == 32 || BS == 64, "block size");
    constexpr int KS = BS / 32;               // 32-deep MFMA steps per block
    constexpr int RF = BS / 16;               // 16-row fragments per block row
    constexpr int PIECES = BS / 8;            // 16-byte B pieces per thread and block
    constexpr int kTile = BS * kBellCols;     // halves of one staged B tile
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][kTile];

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int brow = blockIdx.x / a.col_groups;
    const int c0 = (blockIdx.x % a.col_groups) * kBellCols;
    const int ecols = a.ell_blocks * BS;
    const int* const cind = a.colind + static_cast<size_t>(brow) * a.ell_blocks;
    const char* const Av = static_cast<const char*>(a.values);
    const __amdgpu_buffer_rsrc_t rB = make_rsrc(a.B, a.B_bytes);
    const uint32_t rowbytes = static_cast<uint32_t>(a.N) * 2u;

    // number of blocks in this block row (the list is a prefix, -1 after it)
    int nblk = 0;
    while (nblk < a.ell_blocks && cind[nblk] >= 0) nblk++;

    // B pieces of this thread: piece p = t + 256 q covers row p / 32 of the
    // block, bytes 16 (p % 32) .. of the workgroup's 512-byte row slice.
    auto load_b = [&](int e, i32x4v* bv) {
        const int r0 = cind[e] * BS;
#pragma unroll
        for (int q = 0; q < PIECES; q++) {
            const int p = t + kBellThreads * q;
            const int r = p >> 5, pc = p & 31;
            const int col = c0 + 8 * pc;
            const uint32_t off =
                col < a.N ? static_cast<uint32_t>(r0 + r) * rowbytes + static_cast<uint32_t>(col) * 2u : kOob;
            bv[q] = __builtin_bit_cast(i32x4v, __builtin_amdgcn_raw_buffer_load_b128(rB, off, 0, 0));
        }
    };
    auto store_b = [&](int buf, const i32x4v* bv) {
#pragma unroll
        for (int q = 0; q < PIECES; q++) {
            const int p = t + kBellThreads * q;
            const int r = p >> 5, pc = p & 31;
            const int ks = r >> 5, rr = r & 31, cb = pc >> 3, lp = pc & 7;
            uint16_t* dst = &Bs[buf][((ks * 4 + cb) * 32 + rr) * kDmaBRow + 8 * (lp ^ bswz64(rr))];
            *reinterpret_cast<i32x4v*>(dst) = bv[q];
        }
    };
    // A fragments of block e: [row block][step]
    auto load_a = [&](int e, i32x4v (&af)[RF][KS]) {
#pragma unroll
        for (int rf = 0; rf < RF; rf++)
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const size_t row = static_cast<size_t>(brow) * BS + rf * 16 + (lane & 15);
                const size_t col = static_cast<size_t>(e) * BS + ks * 32 + 8 * (lane >> 4);
                af[rf][ks] = *reinterpret_cast<const i32x4v*>(Av + (row * ecols + col) * 2);
            }
    };

    f32x4 acc[RF][4];
#pragma unroll
    for (int rf = 0; rf < RF; rf++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[rf][c] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int li = lane & 15, lh = lane >> 4;
    const int br = 8 * lh + (li >> 2);
    const int bx = bswz64(br), bh = (li & 3) >> 1;

    i32x4v bv[PIECES];
    i32x4v a0[RF][KS], a1[RF][KS];
    if (nblk > 0) {
        load_b(0, bv);
        load_a(0, a0);
        store_b(0, bv);
    }
    __syncthreads();
    // block e: MFMAs from LDS buffer e & 1 and A registers `ac`; loads of
    // block e + 1 into registers (B pieces, `an`), B stored after the MFMAs
    auto block = [&](int e, const i32x4v (&ac)[RF][KS], i32x4v (&an)[RF][KS]) {
        const bool more = e + 1 < nblk;
        if (more) {
            load_b(e + 1, bv);
            load_a(e + 1, an);
        }
        const uint16_t* Bb = &Bs[e & 1][0];
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const uint16_t* Bfr = Bb + ((ks * 4 + wv) * 32 + br) * kDmaBRow + 4 * (li & 1);
            i32x4v bq[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint16_t* Bp = Bfr + 8 * ((2 * c + bh) ^ bx);
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
                for (int rf = 0; rf < RF; rf++) {
                    if constexpr (kBf16)
                        acc[rf][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8, ac[rf][ks]), __builtin_bit_cast(bf16x8, bq[c]), acc[rf][c], 0, 0,
                            0);
                    else
                        acc[rf][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(f16x8, ac[rf][ks]), __builtin_bit_cast(f16x8, bq[c]), acc[rf][c], 0, 0,
                            0);
                }
        }
        // buffer (e + 1) & 1 was last read in block e - 1, before its barrier
        if (more) store_b((e + 1) & 1, bv);
        __syncthreads();
    };
    int e = 0;
    for (; e + 1 < nblk; e += 2) {
        block(e, a0, a1);
        block(e + 1, a1, a0);
    }
    if (e < nblk) block(e, a0, a1);

    // D layout: lane l holds rows 4 (l / 16) + r, column l % 16 of each 16 x 16 block
#pragma unroll
    for (int rf = 0; rf < RF; rf++)
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int col = c0 + 64 * wv + 16 * c + (lane & 15);
            if (col >= a.N) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = brow * BS + 16 * rf + 4 * (lane >> 4) + r;
                if (row < a.M) __builtin_nontemporal_store(acc[rf][c][r], a.C + static_cast<size_t>(row) * a.N + col);
            }
        }
}

}  // namespace tca
