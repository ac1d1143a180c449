// mfma_kernel.hpp -- condensed-tile SpMM on gfx950 matrix cores (fp16 / bf16).
//
// A row window of 64 rows is condensed: U = the sorted union of its nonzero
// columns, padded to a multiple of 32.  The window's sub-matrix A_w (64 x |U|)
// is then dense enough to be multiplied as tiles: C[rows, cols] = A_w *
// B[U, cols], one 32-wide step of U at a time, on v_mfma_f32_16x16x32_{f16,bf16}.
//
// Workgroup = 4 wavefronts = one window x 128 columns of C.  Wavefront w owns
// rows [16w, 16w + 16) of the window and all 8 column blocks of 16, so each A
// operand feeds 8 MFMAs.  Per step:
//   * the 32 gathered B rows (32 x 128 halves) are staged in LDS row-major;
//     B operands come out of LDS with ds_read_b64_tr_b16, which transposes
//     4 x 16 blocks so lane n receives column n for 4 consecutive rows;
//   * the A tile (64 x 32 halves) is built in LDS by scattering the step's
//     nonzeros (plan entries: row, step column, value index) onto zeros;
//     each thread clears what it scattered once the tile has been consumed;
//   * three LDS buffers rotate (write step s+1, clear step s-1, read step s),
//     so one barrier per step orders everything; global loads run two steps
//     ahead.
// Every output element is produced by one MFMA chain over the steps in
// order, so results are deterministic.
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
constexpr int kMaxStepEntries = 1024;  // nonzeros per (window, step): 4 per thread
constexpr int kAStride = kStepK + 8;      // halves per A-tile row in LDS (80 bytes)
constexpr int kBStride = kTileCols + 8;   // halves per B-tile row in LDS (272 bytes)

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef int i32x4v __attribute__((ext_vector_type(4)));

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
    uint32_t val_bytes, B_bytes;
};

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

template <bool kBf16>
__global__ __launch_bounds__(256) void mfma_tile_kernel(MfmaArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t As[3][kWinRows * kAStride];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[3][kStepK * kBStride];

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int cb = blockIdx.x % a.col_blocks;
    const int4 win = a.windows[blockIdx.x / a.col_blocks];
    const int row0 = win.x, nsteps = win.y, sbase = win.z, nzbase = win.w;
    const int c0 = cb * kTileCols;
    const __amdgpu_buffer_rsrc_t rB = make_rsrc(a.B, a.B_bytes);
    const __amdgpu_buffer_rsrc_t rval = make_rsrc(a.val, a.val_bytes);
    const uint32_t rowbytes = static_cast<uint32_t>(a.N) * 2u;

    // Clear the three A tiles once.
    for (int i = t * 8; i < 3 * kWinRows * kAStride; i += 256 * 8)
        *reinterpret_cast<i32x4v*>(&As[0][0] + i) = i32x4v{0, 0, 0, 0};

    // B staging role: thread t copies row t/8 of the step, columns
    // c0 + 16*(t%8) .. +16 (two 16-byte loads).
    const int brow = t >> 3;
    const int bcol = (t & 7) * 16;
    const bool bcol_ok0 = c0 + bcol < a.N;
    const bool bcol_ok1 = c0 + bcol + 8 < a.N;

    // Prefetch state: "u" = B row index for a step, "e" = entries.
    int u_next = -1;                 // ucols of step s+2 (loaded one iteration ahead)
    int eb_next = 0, ee_next = 0;    // entry range of step s+2
    uint32_t ent_next[4];
    i32x4v bv[2];                    // B data of step s+1 (to be written to LDS)
    uint32_t ent_w[4];               // entries of step s+1
    float unused = 0.f;
    (void)unused;
    uint16_t valw[4];                // values of step s+1
    uint32_t pos_prev[4];            // LDS positions scattered for step s-1 (cleared after use)
    uint32_t pos_cur[4];             // ... for step s
    int n_prev = 0, n_cur = 0;

    auto load_meta = [&](int s, int& u, int& eb, int& ee, uint32_t (&ent)[4]) {
        u = -1;
        eb = ee = 0;
        if (s < nsteps) {
            u = a.ucols[(sbase + s) * kStepK + brow];
            eb = a.eoff[sbase + s];
            ee = a.eoff[sbase + s + 1];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int e = eb + t + 256 * k;
                ent[k] = e < ee ? a.entries[e] : 0xffffffffu;
            }
        }
    };
    auto load_data = [&](int u, uint32_t (&ent)[4], i32x4v (&b)[2], uint16_t (&v)[4]) {
        const uint32_t base = u >= 0 ? static_cast<uint32_t>(u) * rowbytes + (c0 + bcol) * 2u : kOob;
        b[0] = __builtin_amdgcn_raw_buffer_load_b128(rB, (u >= 0 && bcol_ok0) ? base : kOob, 0, 0);
        b[1] = __builtin_amdgcn_raw_buffer_load_b128(rB, (u >= 0 && bcol_ok1) ? base + 16 : kOob, 0, 0);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const bool ok = ent[k] != 0xffffffffu;
            const uint32_t off = ok ? (static_cast<uint32_t>(nzbase) + (ent[k] >> 11)) * 2u : kOob;
            v[k] = __builtin_bit_cast(uint16_t, __builtin_amdgcn_raw_buffer_load_b16(rval, off, 0, 0));
        }
    };
    auto write_step = [&](int buf, const i32x4v (&b)[2], const uint32_t (&ent)[4], const uint16_t (&v)[4],
                          uint32_t (&pos)[4], int& npos) {
        *reinterpret_cast<i32x4v*>(&Bs[buf][brow * kBStride + bcol]) = b[0];
        *reinterpret_cast<i32x4v*>(&Bs[buf][brow * kBStride + bcol + 8]) = b[1];
        npos = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if (ent[k] != 0xffffffffu) {
                const uint32_t p = (ent[k] & 63u) * kAStride + ((ent[k] >> 6) & 31u);
                As[buf][p] = v[k];
                pos[k] = p;
                npos = k + 1;
            }
        }
    };

    // Prologue: step 0 -> buffer 0 now, step 1 data in registers, step 2 meta.
    int u0, eb0, ee0;
    uint32_t ent0[4];
    load_meta(0, u0, eb0, ee0, ent0);
    i32x4v b0[2];
    uint16_t v0[4];
    load_data(u0, ent0, b0, v0);
    int u1, eb1, ee1;
    load_meta(1, u1, eb1, ee1, ent_w);
    load_data(u1, ent_w, bv, valw);
    load_meta(2, u_next, eb_next, ee_next, ent_next);
    __syncthreads();  // A tiles cleared
    write_step(0, b0, ent0, v0, pos_cur, n_cur);
    (void)eb0; (void)ee0; (void)eb1; (void)ee1;
    __syncthreads();

    f32x4 acc[8];
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Lane roles in the MFMA: i = lane % 16, g = lane / 16.
    const int li = lane & 15, lg = lane >> 4;
    // ds_read_b64_tr_b16 source address: lane (within 16) 4*j + m reads row
    // 8g + j (+4), columns 4m .. 4m+3 of the column block.
    const int tr_row = 8 * lg + (li >> 2);
    const int tr_col = 4 * (li & 3);

    for (int s = 0; s < nsteps; s++) {
        const int cur = s % 3, nxt = (s + 1) % 3, prv = (s + 2) % 3;
        // (1) step s+1 data -> LDS buffer nxt (cleared when step s-2 ended)
        uint32_t pos_nxt[4];
        int n_nxt = 0;
        if (s + 1 < nsteps) write_step(nxt, bv, ent_w, valw, pos_nxt, n_nxt);
        // (2) clear the A entries of step s-1 (buffer prv; its reads ended at the last barrier)
        for (int k = 0; k < n_prev; k++)
            if (k < 4) As[prv][pos_prev[k]] = 0;
        // (3) loads for step s+2 (meta loaded last iteration), meta for step s+3
        if (s + 2 < nsteps) {
#pragma unroll
            for (int k = 0; k < 4; k++) ent_w[k] = ent_next[k];
            load_data(u_next, ent_w, bv, valw);
            load_meta(s + 3, u_next, eb_next, ee_next, ent_next);
        }
        // (4) MFMAs of step s from buffer cur
        const uint16_t* Ab = &As[cur][(16 * wave + li) * kAStride + 8 * lg];
        const i32x4v araw = *reinterpret_cast<const i32x4v*>(Ab);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint16_t* Bp0 = &Bs[cur][tr_row * kBStride + 16 * j + tr_col];
            const uint16_t* Bp1 = Bp0 + 4 * kBStride;
            const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp0));
            const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(Bp1));
            const i32x4v braw = {__builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 0, 1)),
                                 __builtin_bit_cast(int, __builtin_shufflevector(lo, lo, 2, 3)),
                                 __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 0, 1)),
                                 __builtin_bit_cast(int, __builtin_shufflevector(hi, hi, 2, 3))};
            if constexpr (kBf16)
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, araw),
                                                                 __builtin_bit_cast(bf16x8, braw), acc[j], 0, 0, 0);
            else
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, araw),
                                                                __builtin_bit_cast(f16x8, braw), acc[j], 0, 0, 0);
        }
        // rotate scatter bookkeeping: step s becomes "previous"
#pragma unroll
        for (int k = 0; k < 4; k++) pos_prev[k] = pos_cur[k];
        n_prev = n_cur;
#pragma unroll
        for (int k = 0; k < 4; k++) pos_cur[k] = pos_nxt[k];
        n_cur = n_nxt;
        __syncthreads();
    }

    // Lane (i, g) holds rows 4g .. 4g+3 of row block `wave`, column i of each block.
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int col = c0 + 16 * j + li;
        if (col >= a.N) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = row0 + 16 * wave + 4 * lg + r;
            if (row < a.M) __builtin_nontemporal_store(acc[j][r], a.C + static_cast<size_t>(row) * a.N + col);
        }
    }
}

}  // namespace tca
