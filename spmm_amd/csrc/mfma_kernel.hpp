// mfma_kernel.hpp -- condensed-tile SpMM on gfx950 matrix cores (fp16 / bf16).
//
// A row window of 64 rows is condensed: U = the sorted union of its nonzero
// columns, padded to a multiple of 32.  The window's sub-matrix A_w (64 x |U|)
// is multiplied as tiles: C[rows, cols] = A_w * B[U, cols], one 32-wide step
// of U at a time, on v_mfma_f32_16x16x32_{f16,bf16}.
//
// Workgroup = 8 wavefronts = one window x 128 columns of C, specialised:
//   * 4 consumer wavefronts (one per SIMD): wavefront w owns columns
//     [32w, 32w + 32) for all 64 rows (4 row blocks x 2 column blocks = 8
//     MFMAs per step); they only read operand fragments from LDS and issue
//     MFMAs;
//   * 4 producer wavefronts (one per SIMD): all global loads (plan meta,
//     entries, values, gathered B rows) and all LDS staging.
// With one of each per SIMD, the texture path, the LDS and the matrix cores
// work at the same time instead of in turn.  An iteration handles a pair of
// steps (2i, 2i+1), each with its own LDS tiles:
//   * B tile: the 32 gathered B rows (32 x 128 halves) as 256-byte rows
//     whose 16-byte pieces are permuted per row (piece c of row r sits at
//     c ^ bswz(r)), so the 8 row pieces that one transposing read touches per
//     32 lanes fall in distinct banks; B operands come out with
//     ds_read_b64_tr_b16, which gives lane n column n of 4 consecutive rows;
//   * A tile (64 x 32 halves) in MFMA fragment order (row block, 8-column
//     group, row, column), so each fragment read is one contiguous 1 KiB; it
//     is built by scattering the step's nonzeros (plan entries: row, step
//     column, nonzero index) onto zeros, and the cells are cleared again
//     two pairs later.
// Both layouts were chosen with SQ_LDS_BANK_CONFLICT measurements on gfx950:
// padded row-major tiles doubled the LDS time of both operand reads.
//
// Producer pipeline (all loads are ordinary vector loads, so the compiler's
// in-order vmcnt accounting is exact):
//   * meta    -- B row indices and entry offsets of each chunk of kDepth
//                pairs are loaded one chunk ahead and kept in LDS;
//   * entries -- kDepth pairs ahead (a slot past the step's entries loads
//                the sentinel entry, so no select waits for the load);
//   * B rows and values -- kDataDepth pairs ahead;
//   * LDS     -- two pairs ahead the staged registers are written to LDS.
// Loads are issued oldest-consumer-last inside an iteration (meta, entries,
// B, values), so waiting for one retires only loads at least
// min(kDepth - kDataDepth, kDataDepth - 2) iterations old.  Staging rotates
// through register slots; the iteration loop is unrolled kDepth times so
// every slot index is a constant.  Consumers read the fragments of pair
// i + 1 during iteration i into a second register set, so their MFMAs start
// right after the barrier.  One barrier per iteration orders LDS: B tiles
// double-buffered, A tiles triple-buffered (write pair i+2, read i+1, clear
// i), meta chunks double-buffered.
//
// Every output element is produced by one MFMA chain over the window's
// steps in order, so results are deterministic.
//
// No counterpart in the reference's structure: the reference feeds one
// nonzero column at a time through m16n8k8 and keeps 1/8 of each MMA
// (src/our_spmm.cu:112-136); here the contraction runs over the window's
// condensed columns, so every MFMA output is used.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "row_kernel.hpp"

namespace tca {

constexpr int kWinRows = 64;    // rows per window (4 row blocks of 16)
constexpr int kTileCols = 128;  // columns of C per workgroup
constexpr int kStepK = 32;      // condensed columns per step (MFMA K)
constexpr int kMaxStepEntries = 1024;     // nonzeros per (window, step): at most 4 per thread
constexpr int kATile = kWinRows * kStepK;  // halves of one A tile (fragment order)
constexpr int kBRow = kTileCols;           // halves per B-tile row in LDS (256 bytes)

// A-tile cell of (row, step column): row block, 8-column group, row, column.
__device__ __forceinline__ int a_cell(int r, int k) {
    return (r >> 4) * 512 + (k >> 3) * 128 + (r & 15) * 8 + (k & 7);
}
// Piece permutation of B-tile row r (even, so a 32-byte pair of pieces stays together).
__device__ __forceinline__ int bswz(int r) { return 2 * ((r & 3) | ((r >> 1) & 4)); }
constexpr uint32_t kNoEntry = 0xffffffffu;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef int i32x4v __attribute__((ext_vector_type(4)));
typedef int i32x2v __attribute__((ext_vector_type(2)));

struct MfmaArgs {
    const int4* windows;     // {first row, steps, first global step, first nonzero}
    const int* ucols;        // [global step][32] B row per condensed column, -1 = padding
    const int* eoff;         // [global step + 1] entry range of each step
    const uint32_t* entries; // row (6 bits) | step column << 6 | (nonzero - first nonzero) << 11
    const void* val;
    const void* B;
    float* C;
    int M, N;
    int col_blocks;          // blockIdx.x = window * col_blocks + column block
    uint32_t val_bytes, B_bytes, entries_bytes, ucols_bytes, eoff_bytes;
    int sentinel;            // index of an entry equal to kNoEntry, loaded for empty slots
};

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// Pipeline shape per entry-slot count (entries per thread and step): the
// producer's register staging must leave room for two wavefronts per SIMD.
template <int kSlots>
struct MfmaDepth {
    static constexpr int kDepth = kSlots == 1 ? 16 : 8;  // unroll, meta chunk, entry lookahead (pairs)
    static constexpr int kDataDepth = kDepth / 2;        // B and value lookahead (pairs)
};

constexpr int kMfmaThreads = 512;  // 4 consumer + 4 producer wavefronts

template <bool kBf16, int kSlots>
__global__ __launch_bounds__(kMfmaThreads) void mfma_tile_kernel(MfmaArgs a) {
    constexpr int R = MfmaDepth<kSlots>::kDepth;
    constexpr int D = MfmaDepth<kSlots>::kDataDepth;
    static_assert(R <= 16 && R % 4 == 0 && D >= 3 && D < R && R % D == 0, "pipeline shape");
    constexpr int kAElems = kATile + 256;  // A tile + one dummy cell per producer thread
    constexpr int kBElems = kStepK * kBRow;
    constexpr int kMI = R / 4;             // meta B-row indices per producer thread
    __shared__ __attribute__((aligned(16))) uint16_t As[2][3][kAElems];  // [step parity][ring]
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][2][kBElems];  // [step parity][ring]
    __shared__ __attribute__((aligned(16))) int metaU[2][2 * R * kStepK];
    __shared__ int metaE[2][2 * R + 1];

    const int t = threadIdx.x;
    const int cb = blockIdx.x % a.col_blocks;
    const int4 win = a.windows[blockIdx.x / a.col_blocks];
    const int row0 = win.x, nsteps = win.y, sbase = win.z, nzbase = win.w;
    __builtin_assume(nsteps >= 1);
    const int c0 = cb * kTileCols;
    const int npairs = (nsteps + 1) / 2;
    // Block blk = iterations [(blk - 1)R, blk R); iteration i computes pair i.
    // Block 0 (the pipeline fill) is peeled off the loop so the loop is entered
    // with the same loads in flight as at its back edge.  Blocks run whole
    // (iterations past the last step only move zeros), so the loop has a
    // single exit and both roles pass the same barriers.
    const int nblocks = (npairs + R - 1) / R + 1;

    // Meta chunk c = pairs [cR, cR + R) = steps [2cR, 2cR + 2R): producer p
    // holds B row indices kMI p .. kMI p + kMI - 1 of the chunk and, for
    // p <= 2R, entry offset p.  Buffer loads: lanes past the window read
    // zeros without a branch.
    const int p = t - 256;  // producer thread index (valid for t >= 256)
    const __amdgpu_buffer_rsrc_t rU = make_rsrc(a.ucols, a.ucols_bytes);
    const __amdgpu_buffer_rsrc_t rE = make_rsrc(a.eoff, a.eoff_bytes);
    auto load_meta = [&](int c, int (&mu)[kMI], int& me) {
        const int s0 = 2 * c * R;
#pragma unroll
        for (int q = 0; q < kMI; q++) {
            const int idx = kMI * p + q;
            const uint32_t uo = static_cast<uint32_t>((sbase + s0) * kStepK + idx) * 4u;
            mu[q] = static_cast<int>(
                __builtin_amdgcn_raw_buffer_load_b32(rU, s0 + idx / kStepK < nsteps ? uo : kOob, 0, 0));
        }
        const uint32_t eo = static_cast<uint32_t>(sbase + s0 + p) * 4u;
        me = static_cast<int>(
            __builtin_amdgcn_raw_buffer_load_b32(rE, (p <= 2 * R && s0 + p <= nsteps) ? eo : kOob, 0, 0));
    };
    auto store_meta = [&](int buf, const int (&mu)[kMI], int me) {
#pragma unroll
        for (int q = 0; q < kMI; q++) metaU[buf][kMI * p + q] = mu[q];
        if (p <= 2 * R) metaE[buf][p] = me;
    };

    // Clear the A tiles; chunk 0 of the meta goes to LDS before the loop.
    for (int i = t * 8; i < 2 * 3 * kAElems; i += kMfmaThreads * 8)
        *reinterpret_cast<i32x4v*>(&As[0][0][0] + i) = i32x4v{0, 0, 0, 0};
    if (t >= 256) {
        int mu[kMI], me;
        load_meta(0, mu, me);
        store_meta(0, mu, me);
    }
    __syncthreads();

    if (t < 256) {
        // ================= consumer: fragments and MFMAs =================
        const int lane = t & 63;
        const int wave = t >> 6;  // column slice [32 wave, 32 wave + 32)
        f32x4 acc[4][2];
#pragma unroll
        for (int b = 0; b < 4; b++)
#pragma unroll
            for (int c = 0; c < 2; c++) acc[b][c] = f32x4{0.f, 0.f, 0.f, 0.f};
        i32x4v af[2][2][4], bfr[2][2][2];  // [iteration parity][step parity]
        // A: lane (i, h) = (lane % 16, lane / 16) holds row 16b + i, columns
        // 8h .. 8h+7 -- in fragment order that is the lane's own 16 bytes.
        // B: the transposing read of a 16-lane group h delivers rows 8h .. 8h+3
        // (then +4) of 16 columns; source lane 4j + m addresses row 8h + j,
        // columns 4m .. 4m+3 of the block.
        const int li = lane & 15, lh = lane >> 4;
        const int br = 8 * lh + (li >> 2);            // row of the low read; the high read is br + 4 (same bswz)
        const int bpc = 4 * wave + ((li & 3) >> 1);   // 16-byte piece of column block 0
        const int b_off0 = br * kBRow + 8 * (bpc ^ bswz(br)) + 4 * (li & 1);
        const int b_off1 = br * kBRow + 8 * ((bpc + 2) ^ bswz(br)) + 4 * (li & 1);
        auto run_block = [&](const int blk) {
#pragma unroll
            for (int u = 0; u < R; u++) {
                const int i = (blk - 1) * R + u;
                // MFMAs of steps 2i, 2i+1 on the fragments read last iteration.
                // Steps past the window have zero tiles and add exact zeros.
                if (i >= 0) {
#pragma unroll
                    for (int sp = 0; sp < 2; sp++)
#pragma unroll
                        for (int b = 0; b < 4; b++)
#pragma unroll
                            for (int c = 0; c < 2; c++) {
                                if constexpr (kBf16)
                                    acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                        __builtin_bit_cast(bf16x8, af[u & 1][sp][b]),
                                        __builtin_bit_cast(bf16x8, bfr[u & 1][sp][c]), acc[b][c], 0, 0, 0);
                                else
                                    acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                        __builtin_bit_cast(f16x8, af[u & 1][sp][b]),
                                        __builtin_bit_cast(f16x8, bfr[u & 1][sp][c]), acc[b][c], 0, 0, 0);
                            }
                }
                // Fragments of pair i + 1 (written by the producers last iteration).
                if (i + 1 >= 0) {
                    const int nx = (u + 1) & 1;
                    const int ar = (i + 1 + 3 * R) % 3;
#pragma unroll
                    for (int sp = 0; sp < 2; sp++) {
                        const uint16_t* Ab = &As[sp][ar][8 * lane];
#pragma unroll
                        for (int b = 0; b < 4; b++) af[nx][sp][b] = *reinterpret_cast<const i32x4v*>(Ab + 512 * b);
#pragma unroll
                        for (int c = 0; c < 2; c++) {
                            const uint16_t* Bp = &Bs[sp][(i + 1) & 1][c == 0 ? b_off0 : b_off1];
                            const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp));
                            const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp + 4 * kBRow));
                            bfr[nx][sp][c] = i32x4v{__builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 0, 1)),
                                                    __builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 2, 3)),
                                                    __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 0, 1)),
                                                    __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 2, 3))};
                        }
                    }
                }
                __syncthreads();
            }
        };
        run_block(0);
        for (int blk = 1; blk < nblocks; blk++) run_block(blk);
        // Lane (i, h) holds rows 4h .. 4h+3 of row block b, column i of column block c.
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const int col = c0 + 32 * wave + 16 * c + li;
            if (col >= a.N) continue;
#pragma unroll
            for (int b = 0; b < 4; b++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = row0 + 16 * b + 4 * lh + r;
                    if (row < a.M) __builtin_nontemporal_store(acc[b][c][r], a.C + static_cast<size_t>(row) * a.N + col);
                }
        }
    } else {
        // ================= producer: loads and LDS staging =================
        const __amdgpu_buffer_rsrc_t rB = make_rsrc(a.B, a.B_bytes);
        const __amdgpu_buffer_rsrc_t rval = make_rsrc(a.val, a.val_bytes);
        const __amdgpu_buffer_rsrc_t rent = make_rsrc(a.entries, a.entries_bytes);
        const uint32_t rowbytes = static_cast<uint32_t>(a.N) * 2u;
        // B staging role: row p / 8 of a step, 16-byte pieces p % 8 and p % 8 + 8
        // (columns c0 + 8q and c0 + 64 + 8q).
        const int brow = p >> 3;
        const int bq = p & 7;
        const bool bok0 = c0 + 8 * bq < a.N;
        const bool bok1 = c0 + 64 + 8 * bq < a.N;
        const uint32_t bcol = static_cast<uint32_t>(c0 + 8 * bq) * 2u;
        const int bw0 = brow * kBRow + 8 * (bq ^ bswz(brow));
        const int bw1 = brow * kBRow + 8 * ((bq + 8) ^ bswz(brow));
        // Every stage runs unconditionally (slots of steps outside the window
        // hold zeros / kNoEntry), so no load's register is conditionally consumed.
        i32x4v breg[2][D][2];          // [step parity][pair % D]: B pieces
        uint32_t ereg[2][R][kSlots];   // [step parity][pair % R]: entries
        uint16_t vreg[2][D][kSlots];   // [step parity][pair % D]: values
#pragma unroll
        for (int sp = 0; sp < 2; sp++) {
#pragma unroll
            for (int u = 0; u < D; u++) {
                breg[sp][u][0] = breg[sp][u][1] = i32x4v{0, 0, 0, 0};
#pragma unroll
                for (int k = 0; k < kSlots; k++) vreg[sp][u][k] = 0;
            }
#pragma unroll
            for (int u = 0; u < R; u++)
#pragma unroll
                for (int k = 0; k < kSlots; k++) ereg[sp][u][k] = kNoEntry;
        }
        // A cells scattered for pairs i and i + 1; an empty slot uses this
        // thread's own dummy cell past the tile, which no MFMA reads.
        const int pad = kATile + p;
        int pos_prev[2][kSlots], pos_cur[2][kSlots];
#pragma unroll
        for (int sp = 0; sp < 2; sp++)
#pragma unroll
            for (int k = 0; k < kSlots; k++) pos_prev[sp][k] = pos_cur[sp][k] = pad;
        int mu_next[kMI], me_next;

        auto run_block = [&](const int blk) {
            load_meta(blk + 1, mu_next, me_next);
#pragma unroll
            for (int u = 0; u < R; u++) {
                const int i = (blk - 1) * R + u;
                // ---- entries of pair i + R (meta chunk blk, position u)
#pragma unroll
                for (int sp = 0; sp < 2; sp++) {
                    const int eb = metaE[blk & 1][2 * u + sp];
                    const int ee = metaE[blk & 1][2 * u + sp + 1];
#pragma unroll
                    for (int k = 0; k < kSlots; k++) {
                        const int e = eb + p + 256 * k;
                        ereg[sp][u][k] = __builtin_amdgcn_raw_buffer_load_b32(
                            rent, static_cast<uint32_t>(e < ee ? e : a.sentinel) * 4u, 0, 0);
                    }
                }
                // ---- B pieces of pair i + D (meta chunk blk - 1 or blk)
#pragma unroll
                for (int sp = 0; sp < 2; sp++) {
                    const int pq = (u + D) % R;  // position in its chunk
                    const int mb = (u + D < R) ? ((blk - 1) & 1) : (blk & 1);
                    const int j = 2 * (i + D) + sp;  // step
                    const int ucol = (j >= 0 && j < nsteps) ? metaU[mb][(2 * pq + sp) * kStepK + brow] : -1;
                    const uint32_t boff = ucol >= 0 ? static_cast<uint32_t>(ucol) * rowbytes + bcol : kOob;
                    breg[sp][u % D][0] =
                        __builtin_amdgcn_raw_buffer_load_b128(rB, (ucol >= 0 && bok0) ? boff : kOob, 0, 0);
                    breg[sp][u % D][1] =
                        __builtin_amdgcn_raw_buffer_load_b128(rB, (ucol >= 0 && bok1) ? boff + 128u : kOob, 0, 0);
                }
                // ---- values of pair i + D (its entries were issued R - D iterations ago)
#pragma unroll
                for (int sp = 0; sp < 2; sp++) {
                    const int se = (u + D) % R;
#pragma unroll
                    for (int k = 0; k < kSlots; k++) {
                        const uint32_t e = ereg[sp][se][k];
                        const uint32_t off =
                            e != kNoEntry ? (static_cast<uint32_t>(nzbase) + (e >> 11)) * 2u : kOob;
                        vreg[sp][u % D][k] =
                            __builtin_bit_cast(uint16_t, __builtin_amdgcn_raw_buffer_load_b16(rval, off, 0, 0));
                    }
                }
                // ---- pair i + 2 to LDS (B ring i&1, A ring (i+2)%3); clear pair i's A cells
                {
                    const int a_wr = (i + 2 + 3 * R) % 3;
                    const int a_cl = (i + 3 * R) % 3;
                    const int sb = (u + 2) % D;
                    const int se = (u + 2) % R;
#pragma unroll
                    for (int sp = 0; sp < 2; sp++) {
                        uint16_t* bs = &Bs[sp][i & 1][0];
                        *reinterpret_cast<i32x4v*>(bs + bw0) = breg[sp][sb][0];
                        *reinterpret_cast<i32x4v*>(bs + bw1) = breg[sp][sb][1];
#pragma unroll
                        for (int k = 0; k < kSlots; k++) {
                            As[sp][a_cl][pos_prev[sp][k]] = 0;
                            // An empty slot's value loaded as zero (out-of-range offset).
                            const uint32_t e = ereg[sp][se][k];
                            const int cell = a_cell(static_cast<int>(e & 63u), static_cast<int>((e >> 6) & 31u));
                            const int m = -static_cast<int>(e != kNoEntry);
                            const int pos = (cell & m) | (pad & ~m);
                            As[sp][a_wr][pos] = vreg[sp][sb][k];
                            pos_prev[sp][k] = pos_cur[sp][k];
                            pos_cur[sp][k] = pos;
                        }
                    }
                }
                // ---- meta chunk blk + 1 to LDS at the end of block blk
                if (u == R - 1) store_meta((blk + 1) & 1, mu_next, me_next);
                __syncthreads();
            }
        };
        run_block(0);
        for (int blk = 1; blk < nblocks; blk++) run_block(blk);
    }
}

}  // namespace tca
