// sparse24_kernel.hpp -- C = A * B with A in 2:4 structured sparsity on the
// gfx950 sparse matrix cores (v_smfmac_f32_16x16x64_{f16,bf16}), fp32
// accumulation and output.
//
// Replaces the reference's cuSPARSELt baseline
// (perform_cuSPARSELT_24sparsity, src/spmm_cusparse.cu:2-179).  A arrives
// compressed (tca_csr_to_24): vals [M][Kp/2], meta [M][Kp/16] uint16.
// Operand layout of v_smfmac_f32_16x16x64 (probed on the MI355X with one-hot
// inputs, 2048 cases):
//   * A: lane L holds row L % 16 and columns 16 (L / 16) .. + 15 as 4 groups
//     of 4; its 8 halves are the two kept values of each group (2 G, 2 G + 1);
//   * index: bits 4G .. 4G+1 and 4G+2 .. 4G+3 of the lane's word are the
//     positions of values 2 G and 2 G + 1 inside group G — exactly one meta
//     word of tca_csr_to_24 (placed in both 16-bit halves);
//   * B: lane n + 16 g holds column n, rows 8 g .. 8 g + 7 in halves 0..7 and
//     rows 32 + 8 g .. + 7 in halves 8..15: two fragments of the dense
//     v_mfma_f32_16x16x32 B operand, one per 32-row half of the 64-row step;
//   * D: as the dense 16x16 MFMA (lane l: column l % 16, rows 4 (l / 16) + r).
// A workgroup owns 64 rows and 256 columns of C; wavefront w owns columns
// 64 w .. 64 w + 63 (4 row blocks x 4 column blocks).  Per K step of 64:
// B rows (64 x 256) are staged in LDS, double-buffered, in the layout of the
// Blocked-ELL kernel (two 32-row halves, bswz64-permuted 128-byte rows, read
// with ds_read_b64_tr_b16); A's compressed fragment (16 bytes per lane) and
// meta word come straight from global memory one step ahead.  Steps are
// added in order (deterministic).  B rows past K load as zeros; rows past M
// read row M - 1 and are not stored.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mfma_common.hpp"

namespace tca {

typedef _Float16 f16x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x16 __attribute__((ext_vector_type(16)));

constexpr int kS24Threads = 256;  // 4 wavefronts
constexpr int kS24Cols = 256;     // columns of C per workgroup
constexpr int kS24Rows = 64;      // rows of C per workgroup

struct S24Args {
    const void* vals;       // [M][Kp / 2]
    const uint16_t* meta;   // [M][Kp / 16]
    const void* B;          // K x N row-major
    float* C;               // M x N row-major
    int M, N, Kp;
    int col_groups;         // blockIdx.x = row group * col_groups + column group
    uint32_t B_bytes;       // K * N * 2
};

template <bool kBf16>
__global__ __launch_bounds__(kS24Threads) void sparse24_kernel(S24Args a) {
    constexpr int KROWS = 64;                 // B rows per step
    constexpr int PIECES = KROWS / 8;         // 16-byte B pieces per thread and step
    constexpr int kTile = KROWS * kS24Cols;   // halves of one staged B tile
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][kTile];

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int row0 = (blockIdx.x / a.col_groups) * kS24Rows;
    const int c0 = (blockIdx.x % a.col_groups) * kS24Cols;
    const int steps = a.Kp / 64;
    const int vcols = a.Kp / 2, mcols = a.Kp / 16;
    const __amdgpu_buffer_rsrc_t rB = make_rsrc(a.B, a.B_bytes);
    const uint32_t rowbytes = static_cast<uint32_t>(a.N) * 2u;
    const uint16_t* const V = static_cast<const uint16_t*>(a.vals);

    auto load_b = [&](int s, i32x4v* bv) {
#pragma unroll
        for (int q = 0; q < PIECES; q++) {
            const int p = t + kS24Threads * q;
            const int r = p >> 5, pc = p & 31;
            const int col = c0 + 8 * pc;
            const uint32_t off =
                col < a.N ? static_cast<uint32_t>(64 * s + r) * rowbytes + static_cast<uint32_t>(col) * 2u : kOob;
            bv[q] = __builtin_bit_cast(i32x4v, __builtin_amdgcn_raw_buffer_load_b128(rB, off, 0, 0));
        }
    };
    auto store_b = [&](int buf, const i32x4v* bv) {
#pragma unroll
        for (int q = 0; q < PIECES; q++) {
            const int p = t + kS24Threads * q;
            const int r = p >> 5, pc = p & 31;
            const int h = r >> 5, rr = r & 31, cb = pc >> 3, lp = pc & 7;
            uint16_t* dst = &Bs[buf][((h * 4 + cb) * 32 + rr) * kDmaBRow + 8 * (lp ^ bswz64(rr))];
            *reinterpret_cast<i32x4v*>(dst) = bv[q];
        }
    };
    // compressed A fragments and index words of step s, per row block
    auto load_a = [&](int s, i32x4v (&af)[4], int (&ix)[4]) {
#pragma unroll
        for (int rb = 0; rb < 4; rb++) {
            const int row = min(row0 + 16 * rb + (lane & 15), a.M - 1);
            af[rb] = *reinterpret_cast<const i32x4v*>(V + static_cast<size_t>(row) * vcols + 32 * s + 8 * (lane >> 4));
            const uint32_t m = a.meta[static_cast<size_t>(row) * mcols + 4 * s + (lane >> 4)];
            ix[rb] = static_cast<int>(m | (m << 16));
        }
    };

    f32x4 acc[4][4];
#pragma unroll
    for (int rb = 0; rb < 4; rb++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[rb][c] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int li = lane & 15, lh = lane >> 4;
    const int br = 8 * lh + (li >> 2);
    const int bx = bswz64(br), bh = (li & 3) >> 1;

    i32x4v bv[PIECES];
    i32x4v a0[4], a1[4];
    int x0[4], x1[4];
    if (steps > 0) {
        load_b(0, bv);
        load_a(0, a0, x0);
        store_b(0, bv);
    }
    __syncthreads();
    auto step = [&](int s, const i32x4v (&ac)[4], const int (&xc)[4], i32x4v (&an)[4], int (&xn)[4]) {
        const bool more = s + 1 < steps;
        if (more) {
            load_b(s + 1, bv);
            load_a(s + 1, an, xn);
        }
        const uint16_t* Bb = &Bs[s & 1][0];
        // B operand of column block c: halves 0..7 from rows 0..31, 8..15 from rows 32..63
        i32x4v bq[2][4];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint16_t* Bfr = Bb + ((h * 4 + wv) * 32 + br) * kDmaBRow + 4 * (li & 1);
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint16_t* Bp = Bfr + 8 * ((2 * c + bh) ^ bx);
                const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp));
                const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp + 4 * kDmaBRow));
                bq[h][c] = i32x4v{__builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 0, 1)),
                                  __builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 2, 3)),
                                  __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 0, 1)),
                                  __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 2, 3))};
            }
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
            typedef int i32x8v __attribute__((ext_vector_type(8)));
            const i32x8v b8 = __builtin_shufflevector(bq[0][c], bq[1][c], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
            for (int rb = 0; rb < 4; rb++) {
                if constexpr (kBf16)
                    acc[rb][c] = __builtin_amdgcn_smfmac_f32_16x16x64_bf16(
                        __builtin_bit_cast(bf16x8, ac[rb]), __builtin_bit_cast(bf16x16, b8), acc[rb][c], xc[rb], 0, 0);
                else
                    acc[rb][c] = __builtin_amdgcn_smfmac_f32_16x16x64_f16(
                        __builtin_bit_cast(f16x8, ac[rb]), __builtin_bit_cast(f16x16, b8), acc[rb][c], xc[rb], 0, 0);
            }
        }
        if (more) store_b((s + 1) & 1, bv);
        __syncthreads();
    };
    int s = 0;
    for (; s + 1 < steps; s += 2) {
        step(s, a0, x0, a1, x1);
        step(s + 1, a1, x1, a0, x0);
    }
    if (s < steps) step(s, a0, x0, a1, x1);

#pragma unroll
    for (int rb = 0; rb < 4; rb++)
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int col = c0 + 64 * wv + 16 * c + (lane & 15);
            if (col >= a.N) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = row0 + 16 * rb + 4 * (lane >> 4) + r;
                if (row < a.M) __builtin_nontemporal_store(acc[rb][c][r], a.C + static_cast<size_t>(row) * a.N + col);
            }
        }
}

}  // namespace tca
