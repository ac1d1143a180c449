// mfma_short_kernel.hpp -- one-launch matrix-core SpMM for short K (fp16 /
// bf16, K <= 640): every row of A, no plan-time tiles, no pack kernel.
//
// A workgroup owns a window of 64 rows (four 16-row blocks) and a 64-column
// block of C, and holds the whole window in LDS: its A rows dense over all
// of K (zeros, then its CSR entries scattered in, values read straight from
// the caller's array) and B[0..K, 64 columns].  Then each of the 8
// wavefronts takes two row blocks and one 16-column block and walks K in
// steps of 32 with v_mfma_f32_16x16x32_{f16,bf16}.  With K = 512 that is
// 128 KiB of LDS and 16 steps; 2048 rows and N = 256 give 128 workgroups.
// Wide windows and few workgroups on purpose: a window's B block costs the
// same whatever its height (64 rows halve the B bytes per row against 32),
// and the GPU starts a launch's workgroups over ~1.5 us (measured with
// s_memrealtime: 256 workgroups of 32 rows started over 1.6 - 4 us), so
// half as many start sooner.
//
// The plan keeps, per nonzero, its half index in the window's A tiles
// (soff: step * 2048 + a_cell(row in window, column in step), < 40960) and
// per window its first nonzero (windows' starts, in the kernel arguments
// when there are at most kShArgWindows windows): what the kernel loads does
// not depend on anything it loads, so every load is in flight at once.
// Per workgroup, in order, all loads ordinary vector loads (so the
// compiler's vmcnt waits are exact; a global -> LDS transfer would make it
// wait for every transfer before any LDS access):
//   1. the window's nonzero range (kernel arguments or one scalar load);
//   2. B[0..K, 64 columns] into registers, 16 bytes per thread per two
//      steps, and the window's nonzeros (soff, value), 8 per thread per
//      round -- in flight together, one round trip;
//   3. all threads zero the A tiles; B is written to LDS as it lands;
//   4. barrier (zeros done), the nonzeros stored at their soff (windows
//      with more than 4096 nonzeros take more rounds), barrier;
//   5. MFMAs: wavefront w, row blocks 2 (w / 4) and 2 (w / 4) + 1, column
//      block w % 4, fragments read 4 steps ahead; C stored from the
//      accumulators.
// Layouts are those of mfma_common.hpp: per step, the A tile in MFMA
// fragment order (a_cell; 1 KiB per row block, each fragment read one
// contiguous 16 bytes per lane) and the B tile as 32 rows of 128 bytes with
// the bswz64 piece permutation, read with ds_read_tr16_b64.  B rows past K
// and columns past N are read from 16 zero bytes.
//
// Every output element is one MFMA chain over the steps in order, so
// results are deterministic.  No counterpart in the reference, which feeds
// one nonzero column at a time through m16n8k8 (src/our_spmm.cu:112-136).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mfma_common.hpp"

namespace tca {

constexpr int kShThreads = 512;                        // 8 wavefronts: 2 row-block pairs x 4 column blocks
constexpr int kShRows = 64;                            // rows per window (4 row blocks)
constexpr int kShMaxSteps = 20;                        // K <= 640
constexpr int kShATileBytes = 4 * 1024;                // per step: 4 row blocks in fragment order
constexpr int kShBTileBytes = kStepK * kDmaBRow * 2;   // per step: 32 rows x 64 halves
constexpr int kShLook = 4;                             // steps of fragments read ahead of the MFMAs
constexpr int kShBatch = 8;                            // nonzeros per thread per scatter round
constexpr int kShArgWindows = 255;                     // window starts passed in the kernel arguments

constexpr int kShLdsBytes = kShMaxSteps * (kShATileBytes + kShBTileBytes);  // 160 KiB

struct ShortArgs {
    const int32_t* wstart;  // [nwin + 1] first nonzero of each window (used when nwin > kShArgWindows)
    const uint16_t* soff;   // [nnz] half index of each nonzero in its window's A tiles
    const uint16_t* val;    // [nnz] fp16 / bf16 bits
    const void* B;          // [K][N]
    float* C;               // [M][N]
    const void* zeros;      // 16 zero bytes
    int M, K, N;
    int nwin;               // windows of 64 rows: ceil(M / 64)
    int col_blocks;         // ceil(N / 64)
    int steps;              // ceil(K / 32)
    int wstart_arg[kShArgWindows + 1];  // window starts, when nwin <= kShArgWindows
};

// Workgroups: a multiple of the XCD count (see the mapping in the kernel).
inline int mfma_short_grid(int nwin, int col_blocks) {
    const int per = (nwin * col_blocks + kXcds - 1) / kXcds;
    return per * kXcds;
}

template <bool kBf16>
__global__ __launch_bounds__(kShThreads) void mfma_short_kernel(ShortArgs a) {
    __shared__ __attribute__((aligned(16))) char smem[kShLdsBytes];
    // Column-block-major order, a contiguous range per XCD (workgroup x runs
    // on XCD x % 8): the workgroups of one XCD share B's column blocks in its L2.
    const int total = a.nwin * a.col_blocks;
    const int per = (total + kXcds - 1) / kXcds;
    const int v = static_cast<int>(blockIdx.x % kXcds) * per + static_cast<int>(blockIdx.x / kXcds);
    if (v >= total) return;  // whole workgroup, before any barrier
    const int cb = v / a.nwin;
    const int row0 = (v % a.nwin) * kShRows;
    const int c0 = cb * kDmaTileCols;
    const int steps = a.steps;
    const int t = threadIdx.x;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int lane = t & 63;
    char* const Abase = smem;
    char* const Bbase = smem + steps * kShATileBytes;

    // 1. the window's nonzeros [e0, e1)
    const int w = v % a.nwin;
    const int e0 = a.nwin <= kShArgWindows ? a.wstart_arg[w] : a.wstart[w];
    const int e1 = a.nwin <= kShArgWindows ? a.wstart_arg[w + 1] : a.wstart[w + 1];

    // 2. B: thread t holds, of step tiles 2 j + t / 256, row (t % 256) / 8
    //    and physical piece t % 8 (logical piece (t % 8) ^ bswz64(row))
    const int bsp = t >> 8;
    const int br0 = (t & 255) >> 3;
    const int bcol = c0 + 8 * ((t & 7) ^ bswz64(br0));
    const char* const Bg = static_cast<const char*>(a.B);
    i32x4v bq[kShMaxSteps / 2];
#pragma unroll
    for (int j = 0; j < kShMaxSteps / 2; j++) {
        const int s = 2 * j + bsp;
        const int k = kStepK * s + br0;
        bq[j] = (s < steps && k < a.K && bcol < a.N)
                    ? *reinterpret_cast<const i32x4v*>(Bg + (static_cast<size_t>(k) * a.N + bcol) * 2)
                    : i32x4v{0, 0, 0, 0};
    }
    //    ... and the first round of the window's nonzeros
    int so[kShBatch];
    uint16_t sv[kShBatch];
    auto load_round = [&](int base) {
#pragma unroll
        for (int i = 0; i < kShBatch; i++) {
            const int e = base + i * kShThreads + t;
            const bool in = e < e1;
            so[i] = in ? static_cast<int>(a.soff[e]) : -1;
            sv[i] = in ? a.val[e] : uint16_t(0);
        }
    };
    load_round(e0);

    // 3. zero the A tiles; B into LDS
    for (int o = 16 * t; o < steps * kShATileBytes; o += 16 * kShThreads)
        *reinterpret_cast<i32x4v*>(Abase + o) = i32x4v{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < kShMaxSteps / 2; j++)
        if (2 * j + bsp < steps) *reinterpret_cast<i32x4v*>(Bbase + (2 * j + bsp) * kShBTileBytes + 16 * (t & 255)) = bq[j];

    // 4. scatter
    uint16_t* const A16 = reinterpret_cast<uint16_t*>(Abase);
    __syncthreads();  // the zeros are written
    for (int base = e0;;) {
#pragma unroll
        for (int i = 0; i < kShBatch; i++)
            if (so[i] >= 0) A16[so[i]] = sv[i];
        base += kShBatch * kShThreads;
        if (base >= e1) break;  // uniform
        load_round(base);
    }
    __syncthreads();  // A and B complete

    // 5. MFMAs: row blocks 2 (wv / 4) + 0/1, column block wv % 4, steps in order
    const int cbk = wv & 3, rb0 = 2 * (wv >> 2);
    const int li = lane & 15, lh = lane >> 4;
    const int br = 8 * lh + (li >> 2);
    const int bx = bswz64(br), bh = (li & 3) >> 1;
    const char* const Afr = Abase + rb0 * 1024 + 16 * lane;
    const uint16_t* const Bfr = reinterpret_cast<const uint16_t*>(Bbase) + br * kDmaBRow + 4 * (li & 1) +
                                8 * ((2 * cbk + bh) ^ bx);
    auto read = [&](int s, i32x4v (&fr)[3]) {
        const char* Ab = Afr + s * kShATileBytes;
        fr[0] = *reinterpret_cast<const i32x4v*>(Ab);
        fr[1] = *reinterpret_cast<const i32x4v*>(Ab + 1024);
        const uint16_t* Bp = Bfr + s * (kShBTileBytes / 2);
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp + 4 * kDmaBRow));
        fr[2] = i32x4v{__builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 0, 1)),
                       __builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 2, 3)),
                       __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 0, 1)),
                       __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 2, 3))};
    };
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    auto mma = [&](const i32x4v (&fr)[3]) {
#pragma unroll
        for (int b = 0; b < 2; b++) {
            if constexpr (kBf16)
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, fr[b]),
                                                                 __builtin_bit_cast(bf16x8, fr[2]), acc[b], 0, 0, 0);
            else
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, fr[b]),
                                                                __builtin_bit_cast(f16x8, fr[2]), acc[b], 0, 0, 0);
        }
    };
    // fragments kShLook steps ahead of the MFMA chain (a ring of registers;
    // the loops unroll fully, so every ring index is a constant)
    i32x4v fr[kShLook][3];
#pragma unroll
    for (int s = 0; s < kShLook; s++)
        if (s < steps) read(s, fr[s]);
#pragma unroll
    for (int s = 0; s < kShMaxSteps; s++) {
        if (s < steps) {
            mma(fr[s % kShLook]);
            if (s + kShLook < steps) read(s + kShLook, fr[s % kShLook]);
        }
    }

    // C: row block rb0 + b, column block cbk; lane holds rows 4 (lane / 16) + r
    const int col = c0 + 16 * cbk + li;
    if (col < a.N) {
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = row0 + 16 * (rb0 + b) + 4 * lh + r;
                if (row < a.M) __builtin_nontemporal_store(acc[b][r], a.C + static_cast<size_t>(row) * a.N + col);
            }
    }
}

}  // namespace tca
