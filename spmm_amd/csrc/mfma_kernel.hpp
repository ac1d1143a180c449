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

#include <type_traits>

#include "row_kernel.hpp"

namespace tca {

constexpr int kWinRows = 64;    // rows per window (4 row blocks of 16)
constexpr int kTileCols = 128;  // columns of C per workgroup
constexpr int kStepK = 32;      // condensed columns per step (MFMA K)
constexpr int kMaxStepEntries = 1024;     // nonzeros per (window, step): at most 4 per thread
constexpr int kATile = kWinRows * kStepK;  // halves of one A tile (fragment order)
constexpr int kBRow = kTileCols;           // halves per B-tile row in LDS (256 bytes)

// A-tile cell of (row, step column): row block, 8-column group, row, column.
__host__ __device__ inline int a_cell(int r, int k) {
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
    const int4* windows;     // {first row, steps, first global step, first nonzero (unused here)}
    const uint32_t* ucols;   // [global step][32] byte offset of the B row of each condensed column
                             // (row * N * 2), 0xffffffff = padding
    const int* eoff;         // [global step + 1] entry range of each step
    const uint32_t* packed;  // per entry: a_cell(row, step column) | value bits << 16
                             // (written each run by mfma_pack_kernel), then one kNoEntry sentinel
    const void* B;
    float* C;
    int M, N;
    int col_blocks;          // blockIdx.x = window * col_blocks + column block
    uint32_t B_bytes, packed_bytes, ucols_bytes, eoff_bytes;
    int sentinel;            // index of the kNoEntry entry, loaded for empty slots
    const void* zeros;       // 16 zero bytes (source of padding B pieces, LDS-DMA and paired kernels)
    const i32x2v* emeta;     // [global step] {first word of the packed block, groups of 64 entries} (paired kernel)
    const void* adense;      // [global step] dense A tile, 8 KiB in fragment order (dense kernel)
    int n_windows;           // windows (dense kernel: its workgroup -> window mapping)
    int K;                   // rows of B (dense kernel, windows in natural column order)
    const uint64_t* amask;   // [global step][8] non-empty cells of each row block (compact dense kernel)
};

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// Pipeline shape per entry-slot count (entries per thread and step): the
// producer's register staging must leave room for two wavefronts per SIMD.
template <int kSlots>
struct MfmaDepth {
    static constexpr int kSteps = kSlots == 4 ? 2 : 4;  // steps per iteration (one barrier each)
    static constexpr int kDepth = 8;      // unroll and meta chunk (iterations)
    static constexpr int kDataDepth = 4;  // entry and B lookahead (iterations)
};

constexpr int kMfmaThreads = 512;  // 4 consumer + 4 producer wavefronts

// Per run: pair each MFMA entry's A-tile cell with its value, in the packed
// array's word order, so the tile kernels load one coalesced word per entry
// (the values are read once here instead of once per column block).  Word x
// gets cell[x] | val[src[x]] << 16; words that hold no entry (src[x] < 0)
// keep their plan-time content: cell[x] with value bits 0, or kNoEntry where
// cell[x] is 0xffff.  Four words per thread: the loads of src and cell and
// the stores are coalesced, only the value loads gather (from the CSR range
// of one window at a time).
__global__ __launch_bounds__(256) void mfma_pack_kernel(const int* __restrict__ src, const uint16_t* __restrict__ cell,
                                                        int n, const uint16_t* __restrict__ val,
                                                        uint32_t* __restrict__ packed) {
    const int x = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (x >= n) return;
    auto word = [&](int s, uint32_t c) -> uint32_t {
        const uint32_t hi = s >= 0 ? static_cast<uint32_t>(val[s]) : (c == 0xffffu ? 0xffffu : 0u);
        return c | (hi << 16);
    };
    if (x + 4 <= n) {
        const int4 s = *reinterpret_cast<const int4*>(src + x);
        const uint2 c = *reinterpret_cast<const uint2*>(cell + x);
        *reinterpret_cast<uint4*>(packed + x) = uint4{word(s.x, c.x & 0xffffu), word(s.y, c.x >> 16),
                                                       word(s.z, c.y & 0xffffu), word(s.w, c.y >> 16)};
    } else {
        for (int k = x; k < n; k++) packed[k] = word(src[k], cell[k]);
    }
}

// Static LDS of mfma_tile_kernel<*, kSlots> in bytes.
template <int kSlots>
constexpr int mfma_lds_bytes() {
    constexpr int KS = MfmaDepth<kSlots>::kSteps, R = MfmaDepth<kSlots>::kDepth;
    return KS * 3 * (kATile + 256) * 2 + KS * 2 * kStepK * kBRow * 2 + 2 * kStepK * (R * KS + 4) * 4 + 2 * (R * KS + 4) * 4;
}

template <bool kBf16, int kSlots>
__global__ __launch_bounds__(kMfmaThreads) void mfma_tile_kernel(MfmaArgs a) {
    constexpr int KS = MfmaDepth<kSlots>::kSteps;
    constexpr int R = MfmaDepth<kSlots>::kDepth;
    constexpr int D = MfmaDepth<kSlots>::kDataDepth;
    static_assert(D >= 2 && D < R && R % D == 0, "pipeline shape");
    constexpr int kAElems = kATile + 256;         // A tile + one dummy cell per producer thread
    constexpr int kBElems = kStepK * kBRow;
    constexpr int kChunkU = R * KS * kStepK;      // B row offsets per meta chunk
    static_assert(kChunkU % 256 == 0, "meta chunk split over the producers");
    constexpr int kMI = kChunkU / 256;            // ... per producer thread
    __shared__ __attribute__((aligned(16))) uint16_t As[KS][3][kAElems];  // [step in iteration][ring]
    __shared__ __attribute__((aligned(16))) uint16_t Bs[KS][2][kBElems];  // [step in iteration][ring]
    // Meta chunks are stored B-row-major ([row][step of the chunk], rows padded
    // by 4) so that one iteration's KS row offsets of a producer are one read.
    constexpr int kMetaRow = R * KS + 4;
    __shared__ __attribute__((aligned(16))) uint32_t metaU[2][kStepK * kMetaRow];
    __shared__ __attribute__((aligned(16))) int metaE[2][R * KS + 4];

    const int t = threadIdx.x;
    const int cb = blockIdx.x % a.col_blocks;
    const int4 win = a.windows[blockIdx.x / a.col_blocks];
    const int row0 = win.x, nsteps = win.y, sbase = win.z;
    __builtin_assume(nsteps >= 1);
    const int c0 = cb * kTileCols;
    const int niters = (nsteps + KS - 1) / KS;
    // Block blk = iterations [(blk - 1)R, blk R); iteration i computes steps
    // [KS i, KS i + KS).  Block 0 (the pipeline fill; only its last D iterations
    // run) is peeled off the loop so the loop is entered with the same loads in
    // flight as at its back edge.
    // Blocks run whole (iterations past the last step only move zeros), so the
    // loop has a single exit and both roles pass the same barriers.
    const int nblocks = (niters + R - 1) / R + 1;

    // Meta chunk c = iterations [cR, cR + R) = steps [KS cR, KS cR + KS R):
    // producer p holds B row offsets kMI p .. kMI p + kMI - 1 of the chunk and,
    // for p <= KS R, entry offset p.  Buffer loads: lanes past the window read
    // zeros without a branch (a zero row offset is never used: see ucol below).
    const int p = t - 256;  // producer thread index (valid for t >= 256)
    const __amdgpu_buffer_rsrc_t rU = make_rsrc(a.ucols, a.ucols_bytes);
    const __amdgpu_buffer_rsrc_t rE = make_rsrc(a.eoff, a.eoff_bytes);
    auto load_meta = [&](int c, uint32_t (&mu)[kMI], int& me) {
        const int s0 = KS * c * R;
#pragma unroll
        for (int q = 0; q < kMI; q++) {
            const int idx = kMI * p + q;
            const uint32_t uo = static_cast<uint32_t>((sbase + s0) * kStepK + idx) * 4u;
            mu[q] = __builtin_amdgcn_raw_buffer_load_b32(rU, s0 + idx / kStepK < nsteps ? uo : kOob, 0, 0);
        }
        const uint32_t eo = static_cast<uint32_t>(sbase + s0 + p) * 4u;
        me = static_cast<int>(
            __builtin_amdgcn_raw_buffer_load_b32(rE, (p <= KS * R && s0 + p <= nsteps) ? eo : kOob, 0, 0));
    };
    auto store_meta = [&](int buf, const uint32_t (&mu)[kMI], int me) {
#pragma unroll
        for (int q = 0; q < kMI; q++) {
            const int idx = kMI * p + q;  // chunk index: step idx / 32, B-tile row idx % 32
            metaU[buf][(idx % kStepK) * kMetaRow + idx / kStepK] = mu[q];
        }
        if (p <= KS * R) metaE[buf][p] = me;
    };

    // Clear the A tiles; chunk 0 of the meta goes to LDS before the loop.
    for (int i = t * 8; i < KS * 3 * kAElems; i += kMfmaThreads * 8)
        *reinterpret_cast<i32x4v*>(&As[0][0][0] + i) = i32x4v{0, 0, 0, 0};
    if (t >= 256) {
        uint32_t mu[kMI];
        int me;
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
        auto run_block = [&](const int blk, auto first) {
#pragma unroll
            for (int u = 0; u < R; u++) {
                if constexpr (decltype(first)::value)
                    if (u < R - D) continue;  // the fill needs only D iterations
                const int i = (blk - 1) * R + u;
                // Steps KS i .. KS i + KS - 1 in order (tiles written last
                // iteration); steps past the window have zero tiles and add
                // exact zeros, so only the pipeline fill skips them.
                if (i >= 0) {
                    const int ar = (i + 3 * R) % 3;
                    // Fragments of step sp + 1 are read while the MFMAs of step sp
                    // run (two register sets); scheduling barriers keep the
                    // compiler from sinking the reads below the MFMAs.
                    i32x4v af[2][4], bfr[2][2];
                    auto read_frags = [&](int sp, int set) {
                        const uint16_t* Ab = &As[sp][ar][8 * lane];
#pragma unroll
                        for (int b = 0; b < 4; b++) af[set][b] = *reinterpret_cast<const i32x4v*>(Ab + 512 * b);
#pragma unroll
                        for (int c = 0; c < 2; c++) {
                            const uint16_t* Bp = &Bs[sp][i & 1][c == 0 ? b_off0 : b_off1];
                            const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp));
                            const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp + 4 * kBRow));
                            bfr[set][c] = i32x4v{__builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 0, 1)),
                                                 __builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 2, 3)),
                                                 __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 0, 1)),
                                                 __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 2, 3))};
                        }
                    };
                    read_frags(0, 0);
#pragma unroll
                    for (int sp = 0; sp < KS; sp++) {
                        if (sp + 1 < KS) read_frags(sp + 1, (sp + 1) & 1);
                        __builtin_amdgcn_sched_barrier(0);
                        const int set = sp & 1;
#pragma unroll
                        for (int b = 0; b < 4; b++)
#pragma unroll
                            for (int c = 0; c < 2; c++) {
                                if constexpr (kBf16)
                                    acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                        __builtin_bit_cast(bf16x8, af[set][b]), __builtin_bit_cast(bf16x8, bfr[set][c]),
                                        acc[b][c], 0, 0, 0);
                                else
                                    acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                        __builtin_bit_cast(f16x8, af[set][b]), __builtin_bit_cast(f16x8, bfr[set][c]),
                                        acc[b][c], 0, 0, 0);
                            }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                __syncthreads();
            }
        };
        run_block(0, std::true_type{});
        for (int blk = 1; blk < nblocks; blk++) run_block(blk, std::false_type{});
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
        const __amdgpu_buffer_rsrc_t rent = make_rsrc(a.packed, a.packed_bytes);
        // B staging role: row p / 8 of a step, 16-byte pieces p % 8 and p % 8 + 8
        // (columns c0 + 8q and c0 + 64 + 8q).
        const int brow = p >> 3;
        const int bq = p & 7;
        const uint32_t bcol0 = c0 + 8 * bq < a.N ? static_cast<uint32_t>(c0 + 8 * bq) * 2u : kOob;
        const uint32_t bcol1 = c0 + 64 + 8 * bq < a.N ? static_cast<uint32_t>(c0 + 64 + 8 * bq) * 2u : kOob;
        const int bw0 = brow * kBRow + 8 * (bq ^ bswz(brow));
        const int bw1 = brow * kBRow + 8 * ((bq + 8) ^ bswz(brow));
        // Every stage runs unconditionally (slots of steps outside the window
        // hold zeros / kNoEntry), so no load's register is conditionally consumed.
        i32x4v breg[KS][D][2];          // [step in iteration][iteration % D]: B pieces
        uint32_t ereg[KS][D][kSlots];   // [step in iteration][iteration % D]: packed entries
#pragma unroll
        for (int sp = 0; sp < KS; sp++)
#pragma unroll
            for (int u = 0; u < D; u++) {
                breg[sp][u][0] = breg[sp][u][1] = i32x4v{0, 0, 0, 0};
#pragma unroll
                for (int k = 0; k < kSlots; k++) ereg[sp][u][k] = kNoEntry;
            }
        // A cells scattered for the previous and current iteration; an empty
        // slot uses this thread's own dummy cell past the tile, never read.
        const int pad = kATile + p;
        int pos_prev[KS][kSlots], pos_cur[KS][kSlots];
#pragma unroll
        for (int sp = 0; sp < KS; sp++)
#pragma unroll
            for (int k = 0; k < kSlots; k++) pos_prev[sp][k] = pos_cur[sp][k] = pad;
        uint32_t mu_next[kMI];
        int me_next;
        // Meta of the B / entry stage of iteration (blk, u): pairs of iteration
        // (blk - 1)R + u + D, in chunk blk - 1 or blk (both in LDS during block blk).
        using VecKS = int __attribute__((ext_vector_type(KS)));
        VecKS ev_n, uv_n;
        int el_n;
        auto read_meta = [&](int blk, int u) {
            const int pq = (u + D) % R;
            const int mb = (u + D < R) ? ((blk - 1) & 1) : (blk & 1);
            ev_n = *reinterpret_cast<const VecKS*>(&metaE[mb][KS * pq]);
            el_n = metaE[mb][KS * pq + KS];
            uv_n = *reinterpret_cast<const VecKS*>(&metaU[mb][brow * kMetaRow + KS * pq]);
        };
        read_meta(0, R - D);

        auto run_block = [&](const int blk, auto first) {
            load_meta(blk + 1, mu_next, me_next);
#pragma unroll
            for (int u = 0; u < R; u++) {
                if constexpr (decltype(first)::value)
                    if (u < R - D) continue;  // the fill needs only D iterations
                const int i = (blk - 1) * R + u;
                // ---- packed entries and B pieces of iteration i + D (meta chunk blk - 1 or
                // blk).  The iteration's KS entry ranges and KS B row offsets were read
                // from LDS during the previous iteration; the reads for the next
                // iteration are issued now and complete under this one.
                {
                    const VecKS ev = ev_n, uv = uv_n;
                    const int e_last = el_n;
                    if (u + 1 < R) read_meta(blk, u + 1);
                    else read_meta(blk + 1, 0);
#pragma unroll
                    for (int sp = 0; sp < KS; sp++) {
                        const int j = KS * (i + D) + sp;  // step
                        const bool in = j >= 0 && j < nsteps;
                        const int eb = in ? ev[sp] : 0;
                        const int ee = in ? (sp + 1 < KS ? ev[(sp + 1) % KS] : e_last) : 0;
#pragma unroll
                        for (int k = 0; k < kSlots; k++) {
                            const int e = eb + p + 256 * k;
                            ereg[sp][u % D][k] = __builtin_amdgcn_raw_buffer_load_b32(
                                rent, static_cast<uint32_t>(e < ee ? e : a.sentinel) * 4u, 0, 0);
                        }
                        // B row byte offset; 0xffffffff = padding column, or a step
                        // outside the window (chunk -1 of the pipeline fill included).
                        const uint32_t uo = in ? static_cast<uint32_t>(uv[sp]) : kNoEntry;
                        breg[sp][u % D][0] =
                            __builtin_amdgcn_raw_buffer_load_b128(rB, uo != kNoEntry ? uo + bcol0 : kOob, 0, 0);
                        breg[sp][u % D][1] =
                            __builtin_amdgcn_raw_buffer_load_b128(rB, uo != kNoEntry ? uo + bcol1 : kOob, 0, 0);
                    }
                }
                // ---- iteration i + 1 to LDS (B ring (i+1)&1, A ring (i+1)%3); clear iteration i-1's A cells
                {
                    const int a_wr = (i + 1 + 3 * R) % 3;
                    const int a_cl = (i + 2 + 3 * R) % 3;
                    const int sb = (u + 1) % D;
#pragma unroll
                    for (int sp = 0; sp < KS; sp++) {
                        uint16_t* bs = &Bs[sp][(i + 1) & 1][0];
                        *reinterpret_cast<i32x4v*>(bs + bw0) = breg[sp][sb][0];
                        *reinterpret_cast<i32x4v*>(bs + bw1) = breg[sp][sb][1];
#pragma unroll
                        for (int k = 0; k < kSlots; k++) {
                            As[sp][a_cl][pos_prev[sp][k]] = 0;
                            const uint32_t e = ereg[sp][sb][k];
                            const bool ok = e != kNoEntry;
                            const int pos = ok ? static_cast<int>(e & 0xffffu) : pad;
                            As[sp][a_wr][pos] = ok ? static_cast<uint16_t>(e >> 16) : uint16_t(0);
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
        run_block(0, std::true_type{});
        for (int blk = 1; blk < nblocks; blk++) run_block(blk, std::false_type{});
    }
}

}  // namespace tca
