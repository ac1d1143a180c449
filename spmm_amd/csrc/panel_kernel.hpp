// panel_kernel.hpp -- SpMM over row panels with B rows staged in LDS (VALU).
//
// A workgroup runs one unit of a row panel (planner.hpp, PanelPlan): the
// panel's rows are spread over the 16-lane groups of kPanelWaves consumer
// wavefronts (four groups per wavefront, rpg rows per group), and the unit's
// tiles -- ranges of the panel's sorted column union, P columns each -- are
// staged one after another into two LDS buffers by one producer wavefront.
// While the consumers multiply tile t, the producer's global -> LDS
// transfers bring tile t + 1; one barrier per tile separates the two.
//
// Consumers.  A 16-lane group owns one B-row chunk of 16 * E elements (all
// of N, or one column chunk of it): lane g holds E elements of each of its
// rows' accumulators.  For row entry i of its rows the group walks the CSR
// run of the row inside the tile (contiguous: the row's columns are sorted
// and the tile is a column range); 16 positions and values are fetched with
// one load per lane and broadcast to the group one at a time (DPP
// row_newbcast), and each nonzero costs one or two conflict-free LDS reads
// (16 lanes read 256 contiguous bytes of one staged row) and E FMAs.  The
// accumulation order of a row is its CSR order inside a unit, and units of a
// split panel are summed in unit order by seg_finalize_kernel: results do
// not depend on the schedule.
//
// Producer.  It issues only global_load_lds_dwordx4 transfers (16 bytes per
// lane land at M0 + 16 * lane) and waits for its own transfers before the
// barrier; it executes no LDS instruction (an LDS instruction of a wavefront
// waits for that wavefront's in-flight transfers).  The byte offsets of the
// tile's B rows come through scalar loads; a transfer's lanes select theirs.
//
// Functionally replaces the reference's multirow_per_tb / multitb_per_row
// (src/our_spmm.cu:24-295) for the rows routed to panels: each output row is
// the sum over the row's nonzeros of value x B row.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "row_kernel.hpp"

namespace tca {

constexpr int kPnWaves = 8;     // consumer wavefronts (planner: kPanelWaves)
constexpr int kPnRpg = 10;      // rows per 16-lane group (planner: kPanelRpg)
constexpr int kPnCntRows = 16;  // count entries per wavefront and tile (planner: kPanelCntRows)
constexpr int kPnThreads = (kPnWaves + 1) * 64;

struct PanelArgs {
    const int4* units;       // {panel, first tile, tiles, segment base or -1}
    const int* panel_units;  // units per panel
    const int* rows;         // [panel * R + slot]
    const uint32_t* boff;    // [tile * P + position]: byte offset in B of the staged row
    const uint8_t* width;    // [tile]: columns of the tile (1..P)
    const uint32_t* cnt;     // [tile][wave][16 entries] dwords: byte g = group g's count
    const void* pos;         // [nnz] bytes, padded to whole dwords (pos_bytes)
    const int* ustart;       // [unit * R + slot]
    const void* val;
    const void* B;
    float* C;
    float* partials;
    int N;
    int chunks;             // column chunks (grid = units * chunks)
    uint32_t pos_bytes, val_bytes;
};

template <typename T, int E>
struct PanelGeom {
    static constexpr int kLaneBytes = E * static_cast<int>(sizeof(T));  // bytes per lane per staged row
    static constexpr int kRowBytes = 16 * kLaneBytes;                   // bytes per staged row chunk
    static constexpr int kP = (65536 / kRowBytes) < 255 ? (65536 / kRowBytes) : 255;  // tile columns
    static constexpr int kInstrs = (kP * kRowBytes + 1023) / 1024;  // 1 KiB transfers per tile
    static constexpr int kBufBytes = kInstrs * 1024;                 // one tile buffer (whole transfers)
    static_assert(kLaneBytes == 8 || kLaneBytes == 16 || kLaneBytes == 32, "lane geometry");
};

constexpr int panel_lds_bytes(int row_bytes) {
    return 2 * ((((65536 / row_bytes) < 255 ? (65536 / row_bytes) : 255) * row_bytes + 1023) / 1024) * 1024;
}

template <int U>
__device__ __forceinline__ int pn_bcast(int x) {
    // lane U of each row of 16 lanes to the whole row
    return __builtin_amdgcn_mov_dpp(x, 0x150 + U, 0xf, 0xf, true);
}

// 16 bytes per lane from base + off (scalar base, 32-bit lane offset) to
// LDS byte address m0 + 16 * lane; the s_nop covers the M0 -> transfer hazard.
__device__ __forceinline__ void pn_dma(const void* base, uint32_t off, uint32_t m0) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(m0) : "memory");
}
__device__ __forceinline__ void pn_wait_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <typename P>
__device__ __forceinline__ uint32_t pn_lds_addr(P* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)p));
}

// E elements of staged row `p` for lane g, widened to fp32 (layout: see the
// column mapping in panel_store).
// lbuf: the tile buffer plus this lane's offset in a staged row (one
// shift-add per step then forms the address).
template <typename T, int E>
__device__ __forceinline__ void pn_read(const char* lbuf, int p, float (&b)[E]) {
    using G = PanelGeom<T, E>;
    const char* row = lbuf + p * G::kRowBytes;
    if constexpr (G::kLaneBytes == 32) {  // fp32, E = 8: two 256-byte halves
        const f32x4 lo = *reinterpret_cast<const f32x4*>(row);
        const f32x4 hi = *reinterpret_cast<const f32x4*>(row + 256);
        b[0] = lo.x; b[1] = lo.y; b[2] = lo.z; b[3] = lo.w;
        b[4] = hi.x; b[5] = hi.y; b[6] = hi.z; b[7] = hi.w;
    } else {
        const Pack<T, E> v = *reinterpret_cast<const Pack<T, E>*>(row);
#pragma unroll
        for (int e = 0; e < E; e++) b[e] = to_f32(v.v[e]);
    }
}

// Column of C (within the chunk) of lane g's element e.
template <typename T, int E>
__device__ __forceinline__ int pn_col(int g, int e) {
    if constexpr (PanelGeom<T, E>::kLaneBytes == 32) return e < 4 ? 4 * g + e : 64 + 4 * g + (e - 4);
    else return E * g + e;
}

template <typename T, int E>
__device__ __forceinline__ void panel_store(float* dst, int g, const float (&acc)[E]) {
    if constexpr (PanelGeom<T, E>::kLaneBytes == 32) {
        __builtin_nontemporal_store(f32x4{acc[0], acc[1], acc[2], acc[3]}, reinterpret_cast<f32x4*>(dst + 4 * g));
        __builtin_nontemporal_store(f32x4{acc[4], acc[5], acc[6], acc[7]},
                                    reinterpret_cast<f32x4*>(dst + 64 + 4 * g));
    } else {
        float v[E];
#pragma unroll
        for (int e = 0; e < E; e++) v[e] = acc[e];
        store_row<E>(dst + E * g, v);
    }
}

// Step U of a batch: nonzero j + U of the group's run.  Lanes past the run
// hold value 0 and the zero row's position (the batch loads are masked), so
// the step needs no branch and its LDS reads can be issued ahead of earlier
// steps' FMAs.
template <typename T, int E, int U>
__device__ __forceinline__ void pn_step(float (&acc)[E], int pv, float vv, const char* lbuf) {
    const int p = pn_bcast<U>(pv);
    const float v = __builtin_bit_cast(float, pn_bcast<U>(__builtin_bit_cast(int, vv)));
    float b[E];
    pn_read<T, E>(lbuf, p, b);
#pragma unroll
    for (int e = 0; e < E; e++) acc[e] = __builtin_fmaf(v, b[e], acc[e]);
}

// Steps 2C and 2C + 1 when the wavefront's longest run reaches them (two
// steps per uniform branch: fewer wasted steps than four, and the second
// step's LDS reads can still be issued ahead of the first step's FMAs).
template <typename T, int E, int C>
__device__ __forceinline__ void pn_chunk(float (&acc)[E], int pv, float vv, int m, const char* lbuf) {
    if (2 * C < m) {
        pn_step<T, E, 2 * C + 0>(acc, pv, vv, lbuf);
        pn_step<T, E, 2 * C + 1>(acc, pv, vv, lbuf);
    }
}

// The run of a group in one tile holds at most 16 nonzeros (the planner cuts
// tiles so), fetched with one load per lane: lane g takes nonzero cur + g
// when g < n (masked buffer loads return 0 for the others).  The position
// byte arrives inside the aligned dword that holds it, as a plain 32-bit
// value, and is extracted only when the run is multiplied: no instruction
// between the load and the next tile waits for it.
template <typename T>
__device__ __forceinline__ void pn_fetch(int cur, int n, int g, __amdgpu_buffer_rsrc_t rpos,
                                         __amdgpu_buffer_rsrc_t rval, int& pl, float& vv) {
    const bool ok = g < n;
    const uint32_t k = static_cast<uint32_t>(cur + g);
    pl = __builtin_amdgcn_raw_buffer_load_b32(rpos, ok ? (k & ~3u) : kOob, 0, 0);
    vv = load_val<T>(rval, k, ok);
}

// One group's run of n nonzeros from CSR index `cur` in the current tile;
// nmax is the longest run of the wavefront's four groups (the wavefront
// steps through nmax nonzeros in chunks of 2).  Lanes past the run use the
// zero row (position zrow, relative to `buf`) and value 0.
template <typename T, int E>
__device__ __forceinline__ void pn_run(float (&acc)[E], int cur, int n, int nmax, int pl, float vv, const char* lbuf,
                                       int zrow, int g) {
    const uint32_t k = static_cast<uint32_t>(cur + g);
    const int pv = g < n ? static_cast<int>((static_cast<uint32_t>(pl) >> (8 * (k & 3))) & 255u) : zrow;
    pn_chunk<T, E, 0>(acc, pv, vv, nmax, lbuf);
    pn_chunk<T, E, 1>(acc, pv, vv, nmax, lbuf);
    pn_chunk<T, E, 2>(acc, pv, vv, nmax, lbuf);
    pn_chunk<T, E, 3>(acc, pv, vv, nmax, lbuf);
    pn_chunk<T, E, 4>(acc, pv, vv, nmax, lbuf);
    pn_chunk<T, E, 5>(acc, pv, vv, nmax, lbuf);
    pn_chunk<T, E, 6>(acc, pv, vv, nmax, lbuf);
    pn_chunk<T, E, 7>(acc, pv, vv, nmax, lbuf);
}

template <typename T, int E>
__global__ __launch_bounds__(kPnThreads, 1) void panel_kernel(PanelArgs a) {
    using G = PanelGeom<T, E>;
    constexpr int R = kPnWaves * 4 * kPnRpg;
    // two tile buffers, then one zero row (the target of masked steps)
    __shared__ __attribute__((aligned(16))) char smem[2 * G::kBufBytes + G::kRowBytes];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int chunk = blockIdx.x % a.chunks;
    const int unit = blockIdx.x / a.chunks;
    const int4 u = a.units[unit];

    if (wave == kPnWaves) {
        // ---- producer: tile t + 1 into buffer (t + 1) & 1 while tile t is used
        const int piece = lane % (G::kRowBytes / 16);
        const int sub = lane / (G::kRowBytes / 16);  // row within one 1 KiB transfer
        constexpr int kRowsPerInstr = 1024 / G::kRowBytes;
        // B rows of this column chunk, addressed by 32-bit offsets from one
        // scalar base held in SGPRs.  readfirstlane returns a signed
        // int: each half goes through uint32_t before widening, so a low half
        // with bit 31 set is not sign-extended into the high half.
        const uint64_t bb = reinterpret_cast<uint64_t>(a.B) + static_cast<uint64_t>(chunk) * G::kRowBytes;
        const uint32_t bb_hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(bb >> 32)));
        const uint32_t bb_lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(bb)));
        const char* bbase = reinterpret_cast<const char*>((static_cast<uint64_t>(bb_hi) << 32) | bb_lo);
        const uint32_t lds0 = pn_lds_addr(smem);
        // A tile's P offsets come through coalesced vector loads, lane l
        // holding position j * 64 + l in o[j]; each transfer takes its rows'
        // offsets by readlane.  The offsets (and width) of tile t + 2 load
        // while tile t + 1's transfers are in flight, so one wait per tile
        // covers both.  Positions past P clamp to P - 1 (never staged).
        constexpr int kOffRegs = (G::kP + 63) / 64;
        auto load_offs = [&](int tile, uint32_t (&o)[kOffRegs]) {
            const uint32_t* bo = a.boff + static_cast<size_t>(tile) * G::kP;
#pragma unroll
            for (int j = 0; j < kOffRegs; j++) {
                const int r = j * 64 + lane;
                o[j] = bo[r < G::kP ? r : G::kP - 1];
            }
        };
        auto n_instr = [&](int tile) { return (a.width[tile] * G::kRowBytes + 1023) / 1024; };
        auto stage = [&](const uint32_t (&o)[kOffRegs], int ninstr, int buf) {
#pragma unroll
            for (int k = 0; k < G::kInstrs; k++) {
                if (k < ninstr) {
                    const int r0 = k * kRowsPerInstr;
                    uint32_t off = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(o[r0 / 64]), r0 % 64));
#pragma unroll
                    for (int j = 1; j < kRowsPerInstr; j++) {
                        const uint32_t oj = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(o[r0 / 64]), r0 % 64 + j));
                        off = sub == j ? oj : off;
                    }
                    pn_dma(bbase, off + 16 * piece, lds0 + buf * G::kBufBytes + k * 1024);
                }
            }
        };
        // The compiler cannot see the transfers (inline asm), so it would
        // wait on the offset loads with vmcnt counts that then also wait for
        // the transfers issued before each readlane.  Passing the offsets
        // through an empty asm after the explicit wait ends their load
        // dependence there, where nothing else is in flight.
        uint32_t o[kOffRegs];
        auto settle = [&](int& nin) {
            pn_wait_all();
#pragma unroll
            for (int j = 0; j < kOffRegs; j++) asm volatile("" : "+v"(o[j]));
            nin = __builtin_amdgcn_readfirstlane(nin);
            asm volatile("" : "+s"(nin));
        };
        int nin = n_instr(u.y);
        load_offs(u.y, o);
        settle(nin);
        stage(o, nin, 0);
        if (u.z > 1) {
            nin = n_instr(u.y + 1);
            load_offs(u.y + 1, o);
        }
        settle(nin);
        for (int t = 0; t < u.z; t++) {
            __syncthreads();
            if (t + 1 < u.z) {
                stage(o, nin, (t + 1) & 1);
                if (t + 2 < u.z) {
                    nin = n_instr(u.y + t + 2);
                    load_offs(u.y + t + 2, o);
                }
                settle(nin);
            }
        }
        return;
    }

    // ---- consumers
    const int group = lane >> 4;
    const int g = lane & 15;
    const __amdgpu_buffer_rsrc_t rpos = make_rsrc(a.pos, a.pos_bytes);
    const __amdgpu_buffer_rsrc_t rval = make_rsrc(a.val, a.val_bytes);
    float acc[kPnRpg][E];
    int cur[kPnRpg];
#pragma unroll
    for (int i = 0; i < kPnRpg; i++) {
        cur[i] = a.ustart[static_cast<size_t>(unit) * R + (wave * kPnRpg + i) * 4 + group];
#pragma unroll
        for (int e = 0; e < E; e++) acc[i][e] = 0.f;
    }
    if (wave == 0)
        for (int o = 16 * lane; o < G::kRowBytes; o += 1024)
            *reinterpret_cast<f32x4*>(smem + 2 * G::kBufBytes + o) = f32x4{0.f, 0.f, 0.f, 0.f};
    const int shift = 8 * group;
    // counts through the constant address space: scalar loads, counted by
    // lgkmcnt, so using them never waits for the vector loads in flight
    using CU32 = const __attribute__((address_space(4))) uint32_t;
    CU32* const cbase = (CU32*)(reinterpret_cast<uintptr_t>(a.cnt)) + (static_cast<size_t>(u.y) * kPnWaves + wave) * kPnCntRows;
    auto counts = [&](int t) { return cbase + static_cast<size_t>(t) * (kPnWaves * kPnCntRows); };
    auto zero_row = [&](int t) { return (2 - (t & 1)) * G::kBufBytes / G::kRowBytes; };  // (t = -1: unused)
    // Entry i's run of tile t + 1 is fetched right after entry i is done with
    // tile t, so its latency hides behind the rest of the tile.  Iteration -1
    // only fetches tile 0, with the same instructions in the same order as
    // every later iteration: the compiler's vmcnt waits then count exactly the
    // loads issued after the one they wait for.  The fetch after the last
    // tile has n = 0 (every lane masked).
    uint32_t cn[kPnRpg];
    int plq[kPnRpg];
    float vvq[kPnRpg];
#pragma unroll
    for (int i = 0; i < kPnRpg; i++) {
        cn[i] = 0;
        plq[i] = 0;
        vvq[i] = 0.f;
    }
    for (int t = -1; t < u.z; t++) {
        if (t >= 0) __syncthreads();
        const char* lbuf = smem + (t & 1) * G::kBufBytes + (G::kLaneBytes == 32 ? 16 : G::kLaneBytes) * g;
        const int zrow = zero_row(t);
        const bool more = t + 1 < u.z;
        uint32_t cnx[kPnRpg];
        {
            CU32* cw = counts(more ? t + 1 : t);
#pragma unroll
            for (int i = 0; i < kPnRpg; i++) cnx[i] = cw[i];
        }
#pragma unroll
        for (int i = 0; i < kPnRpg; i++) {
            const uint32_t c4 = cn[i];
            const int n = (c4 >> shift) & 255;
            const int nmax = max(max(c4 & 255, (c4 >> 8) & 255), max((c4 >> 16) & 255, c4 >> 24));
            if (nmax > 0) pn_run<T, E>(acc[i], cur[i], n, nmax, plq[i], vvq[i], lbuf, zrow, g);
            cur[i] += n;
            pn_fetch<T>(cur[i], more ? (cnx[i] >> shift) & 255 : 0, g, rpos, rval, plq[i], vvq[i]);
            cn[i] = cnx[i];
        }
    }
    // ---- results: C rows, or this unit's partial rows of a split panel
    const int nu = u.w >= 0 ? a.panel_units[u.x] : 0;
    const int col0 = chunk * 16 * E;
#pragma unroll
    for (int i = 0; i < kPnRpg; i++) {
        const int s = (wave * kPnRpg + i) * 4 + group;
        const int row = a.rows[static_cast<size_t>(u.x) * R + s];
        if (row < 0) continue;
        float* dst = u.w < 0 ? a.C + static_cast<size_t>(row) * a.N + col0
                             : a.partials + static_cast<size_t>(u.w + s * nu) * a.N + col0;
        panel_store<T, E>(dst, g, acc[i]);
    }
}

}  // namespace tca
