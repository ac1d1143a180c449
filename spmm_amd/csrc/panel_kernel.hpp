// panel_kernel.hpp -- SpMM over row panels with B rows staged in LDS (VALU).
//
// A workgroup runs one unit of a row panel (planner.hpp, PanelPlan): the
// panel's rows are spread over the 16-lane groups of kPanelWaves consumer
// wavefronts (four groups per wavefront, rpg rows per group), and the unit's
// tiles -- ranges of the panel's sorted column union, P columns each -- are
// staged one after another into two LDS buffers by kPnProducers producer
// wavefronts, each issuing every kPnProducers-th transfer of a tile.  While
// the consumers multiply tile t, the producers' global -> LDS transfers bring
// tile t + 1; one barrier per tile separates the two.  1024 threads, one
// workgroup per CU (LDS), four wavefronts per SIMD.
//
// Consumers.  A 16-lane group owns one B-row chunk of 16 * E elements (all
// of N, or one column chunk of it): lane g holds E elements of each of its
// rows' accumulators.  For row entry i of its rows the group walks the CSR
// run of the row inside the tile (contiguous: the row's columns are sorted
// and the tile is a column range); 16 positions and values are fetched with
// one load per lane, and step U of the run takes lane U's through DPP
// row_newbcast: one VALU instruction for the address, one or two
// conflict-free LDS reads (16 lanes read 256 contiguous bytes of one staged
// row), one broadcast of the value and E FMAs per step, the next step's
// reads issued before the current step's FMAs.  The wavefront steps through
// the longest run of its four groups; lanes past their run read a zero row
// (position 0) and multiply by 0.  The accumulation order of a row is its
// CSR order inside a unit, and units of a split panel are summed in a fixed
// order by seg_finalize_kernel: results do not depend on the schedule.
//
// Producers.  They issue only global_load_lds_dwordx4 transfers (16 bytes
// per lane land at M0 + 16 * lane) and wait for their own transfers before
// the barrier; they execute no LDS instruction (an LDS instruction of a
// wavefront waits for that wavefront's in-flight transfers).  Several
// producers because the staging is latency-bound: with one, the consumers
// waited 57 % of their time at the barriers and the producer 4 %.  The byte
// offsets of a tile's B rows come through vector loads; a transfer's lanes
// select theirs by readlane.  With each tile producer 0 also stages the next
// tile's per-wavefront run counts.
//
// Functionally replaces the reference's multirow_per_tb / multitb_per_row
// (src/our_spmm.cu:24-295) for the rows routed to panels: each output row is
// the sum over the row's nonzeros of value x B row.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "row_kernel.hpp"

namespace tca {

constexpr int kPnProducers = 4;  // producer wavefronts: each issues every kPnProducers-th transfer of a tile
constexpr int kPnWaves = 16 - kPnProducers;  // consumer wavefronts (planner: kPanelWaves)
constexpr int kPnRpg = 4;       // rows per 16-lane group (planner: kPanelRpg)
constexpr int kPnMaxDword = kPnRpg;  // first dword of the entries' longest counts (planner: kPanelMaxDword)
constexpr int kPnCntUsed = kPnMaxDword + (kPnRpg + 3) / 4;  // count dwords a wavefront reads per tile
constexpr int kPnCntRows = (kPnCntUsed + 3) / 4 * 4;  // count dwords per wavefront and tile (planner: kPanelCntRows)
constexpr int kPnThreads = (kPnWaves + kPnProducers) * 64;
constexpr int kPnBufLimit = 77824;  // bytes of one tile buffer at most (two, with zero rows and count slots, fit 160 KiB)

struct PanelArgs {
    const int4* units;       // {panel, first tile, tiles, segment base or -1}
    const int* order;        // [workgroup]: unit, or -1 for an idle workgroup
    const int* panel_units;  // units per panel
    const int* rows;         // [panel * R + slot]
    const uint32_t* boff;    // [tile * P + position]: byte offset in B of the staged row
    const uint32_t* cnt;     // [tile][wave][16 entries] dwords: byte g = group g's count
    const void* pos;         // [nnz] bytes, padded to whole dwords (pos_bytes)
    const int* ustart;       // [unit * R + slot]
    const uint8_t* win;      // [panel]: 1 = run data through per-row windows
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
    static constexpr int kP = (kPnBufLimit / kRowBytes) < 255 ? (kPnBufLimit / kRowBytes) : 255;  // tile columns
    static constexpr int kInstrs = (kP * kRowBytes + 1023) / 1024;  // 1 KiB transfers per tile
    static constexpr int kBufBytes = kInstrs * 1024;                 // one tile buffer (whole transfers)
    static_assert(kLaneBytes == 8 || kLaneBytes == 16 || kLaneBytes == 32, "lane geometry");
    static_assert(kP <= 255, "1-based positions fit a byte");
};

// Counts of one tile (all consumer wavefronts) and their LDS slot: one
// 1 KiB transfer per tile.
constexpr int kPnCntTileBytes = kPnWaves * kPnCntRows * 4;
constexpr int kPnCntSlot = 1024;
static_assert(kPnCntTileBytes <= kPnCntSlot && kPnCntTileBytes % 16 == 0, "counts of a tile in one transfer");

// LDS of the panel kernel: two tile buffers and their zero rows, two count slots.
constexpr int panel_lds_bytes(int row_bytes) {
    return 2 * (((((kPnBufLimit / row_bytes) < 255 ? (kPnBufLimit / row_bytes) : 255) * row_bytes + 1023) / 1024) * 1024 + row_bytes) +
           2 * kPnCntSlot;
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

// The tile hand-off: every LDS access of the wavefront done, then the
// workgroup barrier, with compiler barriers on both sides.  Unlike
// __syncthreads() it does not wait for the wavefront's vector loads (the
// consumers' run fetches for the next tile stay in flight across it; the
// producer waits for its transfers itself before arriving).
__device__ __forceinline__ void pn_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <typename P>
__device__ __forceinline__ uint32_t pn_lds_addr(P* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) char*)p));
}

// LDS layout of a workgroup: two tile buffers, each preceded by one zero row
// (the target of positions 0: lanes past a run), then two count slots:
//   [zero row | buffer 0 (kBufBytes) | zero row | buffer 1 (kBufBytes) | counts 0 | counts 1]
// Staged row q (1-based) of tile t starts at zrow_off(t & 1) + q * kRowBytes;
// count slot t & 1 holds the counts of tile t + 1, staged with tile t.
template <typename T, int E>
constexpr int pn_zrow_off(int buf) {
    return buf * (PanelGeom<T, E>::kBufBytes + PanelGeom<T, E>::kRowBytes);
}
template <typename T, int E>
constexpr int pn_cnt_off(int buf) {
    return pn_zrow_off<T, E>(2) + buf * kPnCntSlot;
}

// E elements of the staged row at LDS byte address `addr` (the row's address
// plus this lane's offset in it), widened to fp32; layout: see the column
// mapping in panel_store.
template <typename T, int E>
__device__ __forceinline__ void pn_read_at(uint32_t addr, float (&b)[E]) {
    using G = PanelGeom<T, E>;
    using LC = const __attribute__((address_space(3))) char;
    LC* row = reinterpret_cast<LC*>(static_cast<uintptr_t>(addr));
    if constexpr (G::kLaneBytes == 32) {  // fp32, E = 8: two 256-byte halves
        const f32x4 lo = *reinterpret_cast<const __attribute__((address_space(3))) f32x4*>(row);
        const f32x4 hi = *reinterpret_cast<const __attribute__((address_space(3))) f32x4*>(row + 256);
        b[0] = lo.x; b[1] = lo.y; b[2] = lo.z; b[3] = lo.w;
        b[4] = hi.x; b[5] = hi.y; b[6] = hi.z; b[7] = hi.w;
    } else {
        typedef int w_t __attribute__((ext_vector_type(G::kLaneBytes / 4)));
        const w_t w = *reinterpret_cast<const __attribute__((address_space(3))) w_t*>(row);
        const Pack<T, E> v = __builtin_bit_cast(Pack<T, E>, w);
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

// Step U of a run (nonzero U of each group's run, held by lane U of the
// group) in two DPP instructions and E plain FMAs: the address of the
// staged row is lane U's row address broadcast to the group plus the lane's
// own offset in the row (v_add_u32 with row_newbcast:U), and lane U's value
// is broadcast once (v_mov_b32 with row_newbcast:U) for the E FMAs.  (A DPP
// VALU instruction issues at about 5.4 cycles per SIMD against 3.1 for a
// plain one, measured on MI355X with four wavefronts per SIMD, so the FMAs
// do not take the broadcast themselves.)  The compiler does not see the DPP
// inside the address statement: a DPP source written by a VALU instruction
// needs two wait states before it is read, so the first statement of a run
// (whose source is computed just before) starts with s_nop 1; later steps
// read the same registers, which nothing writes in between.  The statements
// are volatile so that they keep their program order (otherwise the
// compiler may move a later step's statement above the first one's s_nop).
template <int U, bool kNop>
__device__ __forceinline__ uint32_t pn_addr(uint32_t pa, uint32_t lanepart) {
    uint32_t r;
    if constexpr (kNop)
        asm volatile("s_nop 1\n\tv_add_u32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf bound_ctrl:1"
            : "=v"(r) : "v"(pa), "v"(lanepart), "n"(U));
    else
        asm volatile("v_add_u32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf bound_ctrl:1"
            : "=v"(r) : "v"(pa), "v"(lanepart), "n"(U));
    return r;
}
template <int E, int U>
__device__ __forceinline__ void pn_fmas(float (&acc)[E], float vv, const float (&b)[E]) {
    const float v = __builtin_bit_cast(float, pn_bcast<U>(__builtin_bit_cast(int, vv)));
#pragma unroll
    for (int e = 0; e < E; e++) acc[e] = __builtin_fmaf(v, b[e], acc[e]);
}

// Steps U.. of a run: x holds step U's B row (read one step earlier).  Step
// U + 1's row is read before step U's FMAs (also when the run ends at U: one
// read that is not used), so its LDS latency hides behind them, and the run
// leaves after the FMAs of its last step: every exit comes after the same
// in-place accumulation (no join of differently-allocated results), and the
// compiler's LDS waits count exactly the reads issued after the one they wait
// for.  A uniform branch per step: m is the longest run of the wavefront's
// four groups.
template <typename T, int E, int U>
__device__ __forceinline__ void pn_steps(float (&acc)[E], uint32_t pa, float vv, uint32_t lanepart, int m,
                                         float (&x)[E], float (&y)[E]) {
    if constexpr (U < 15) {
        pn_read_at<T, E>(pn_addr<U + 1, false>(pa, lanepart), y);
        // keeps the read here (otherwise it sinks into the branch that uses it)
        asm volatile("" ::: "memory");
    }
    pn_fmas<E, U>(acc, vv, x);
    if constexpr (U < 15) {
        if (U + 1 < m) pn_steps<T, E, U + 1>(acc, pa, vv, lanepart, m, y, x);
    }
}

// One group's run in the current tile: lane g holds nonzero g of the run
// (value vv, 1-based tile position q; lanes past the run hold 0 and 0, so
// they multiply the zero row by 0).  zb: LDS address of the tile buffer's
// zero row; nmax: the longest run of the wavefront's four groups (>= 1).
template <typename T, int E>
__device__ __forceinline__ void pn_run(float (&acc)[E], uint32_t q, float vv, int nmax, uint32_t zb,
                                       uint32_t lanepart) {
    const uint32_t pa = q * static_cast<uint32_t>(PanelGeom<T, E>::kRowBytes) + zb;
    float b0[E], b1[E];
    pn_read_at<T, E>(pn_addr<0, true>(pa, lanepart), b0);
    pn_steps<T, E, 0>(acc, pa, vv, lanepart, nmax, b0, b1);
}

// Calls f(PnIndex<I>{}) for I = B .. N - 1 (compile-time indices for register arrays).
template <int V>
struct PnIndex {
    static constexpr int value = V;
};
template <int B, int N, typename F>
__device__ __forceinline__ void pn_static_for(F&& f) {
    if constexpr (B < N) {
        f(PnIndex<B>{});
        pn_static_for<B + 1, N>(f);
    }
}

template <typename T, int E>
__global__ __launch_bounds__(kPnThreads, 1) void panel_kernel(PanelArgs a) {
    using G = PanelGeom<T, E>;
    constexpr int R = kPnWaves * 4 * kPnRpg;
    // two tile buffers, each after its zero row (pn_zrow_off), two count slots
    __shared__ __attribute__((aligned(16))) char smem[2 * (G::kBufBytes + G::kRowBytes) + 2 * kPnCntSlot];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int chunk = blockIdx.x % a.chunks;
    const int unit = a.order[blockIdx.x / a.chunks];
    if (unit < 0) return;  // idle: every wavefront leaves before the first barrier
    const int4 u = a.units[unit];

    if (wave >= kPnWaves) {
        // ---- producers: tile t + 1 into buffer (t + 1) & 1 while tile t is used;
        // producer pid issues transfers pid, pid + kPnProducers, ... of a tile (and
        // producer 0 the counts), so each has at most kInstrs / kPnProducers + 1
        // transfers in flight (a wavefront's vmcnt counts 63 at most)
        const int pid = wave - kPnWaves;
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
        // offsets by readlane.  Positions past P clamp to P - 1 (never staged).
        constexpr int kOffRegs = (G::kP + 63) / 64;
        auto load_offs = [&](int tile, uint32_t (&o)[kOffRegs]) {
            const uint32_t* bo = a.boff + static_cast<size_t>(tile) * G::kP;
#pragma unroll
            for (int j = 0; j < kOffRegs; j++) {
                const int r = j * 64 + lane;
                o[j] = bo[r < G::kP ? r : G::kP - 1];
            }
        };
        // counts of tile rel + 1 (clamped to the unit's last tile) into count
        // slot buf; lanes past the counts re-read the first 16 bytes
        const uint32_t cnt_lane = 16u * static_cast<uint32_t>(lane < kPnCntTileBytes / 16 ? lane : 0);
        // Every transfer of the tile, whatever its width: columns past the
        // width repeat the tile's last B row (plan padding) into rows that no
        // consumer reads, so each producer issues the same number of memory
        // operations every tile and its waits below are compile-time counts.
        auto stage = [&](const uint32_t (&o)[kOffRegs], int buf, int rel) {
            const int tn = u.y + (rel + 1 < u.z ? rel + 1 : rel);
            if (pid == 0) pn_dma(a.cnt, static_cast<uint32_t>(tn) * kPnCntTileBytes + cnt_lane, lds0 + pn_cnt_off<T, E>(buf));
#pragma unroll
            for (int k = 0; k < G::kInstrs; k++) {
                if (k % kPnProducers == pid) {
                    const int r0 = k * kRowsPerInstr;
                    uint32_t off = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(o[r0 / 64]), r0 % 64));
#pragma unroll
                    for (int j = 1; j < kRowsPerInstr; j++) {
                        const uint32_t oj = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(o[r0 / 64]), r0 % 64 + j));
                        off = sub == j ? oj : off;
                    }
                    pn_dma(bbase, off + 16 * piece, lds0 + pn_zrow_off<T, E>(buf) + G::kRowBytes + k * 1024);
                }
            }
        };
        // Per tile: the transfers of tile t + 1, then the offsets of tile t + 2
        // (loaded unconditionally, clamped), then a wait that leaves only
        // those kOffRegs loads in flight (land): the tile has landed, while
        // the offsets' latency runs on into the next tile period.  After the
        // barrier only those loads can be in flight: a full wait there, and
        // the offsets pass through an empty asm (ready), which ends their load
        // dependence for the compiler -- it cannot see the transfers (inline
        // asm), and its own wait before each readlane would otherwise also
        // wait for the transfers issued before it.
        auto land = [&]() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kOffRegs) : "memory"); };
        static_assert(kOffRegs <= 15, "vmcnt immediate");
        uint32_t o[kOffRegs];
        auto ready = [&]() {
            pn_wait_all();
#pragma unroll
            for (int j = 0; j < kOffRegs; j++) asm volatile("" : "+v"(o[j]));
        };
        load_offs(u.y, o);
        ready();
        stage(o, 0, 0);
        load_offs(u.y + (u.z > 1 ? 1 : 0), o);
        land();
        for (int t = 0; t < u.z; t++) {
            pn_barrier();
            if (t + 1 < u.z) {
                ready();
                stage(o, (t + 1) & 1, t + 1);
                load_offs(u.y + (t + 2 < u.z ? t + 2 : t + 1), o);
                land();
            }
        }
        return;
    }

    // ---- consumers
    // The panel's choice (PanelPlan::win): run data loaded where it lies, or
    // through per-row windows; one branch per workgroup.
    auto consume = [&](auto win_tag) {
        constexpr bool kWin = decltype(win_tag)::value != 0;
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
            for (int o = 16 * lane; o < G::kRowBytes; o += 1024) {
                *reinterpret_cast<f32x4*>(smem + pn_zrow_off<T, E>(0) + o) = f32x4{0.f, 0.f, 0.f, 0.f};
                *reinterpret_cast<f32x4*>(smem + pn_zrow_off<T, E>(1) + o) = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        const int shift = 8 * group;
        const uint32_t lds0 = pn_lds_addr(smem);
        const uint32_t lanepart = static_cast<uint32_t>((G::kLaneBytes == 32 ? 16 : G::kLaneBytes) * g);
        // Counts: per tile and wavefront kPnCntRows dwords; dword i (i < rpg)
        // holds entry i's four group counts, byte i % 4 of dword kPnMaxDword + i / 4
        // entry i's longest.  Tile 0's come through one vector load before the loop;
        // tile t + 1's are read from the count slot the producer staged with tile
        // t (LDS reads, ordered with the B-row reads: no scalar loads, which
        // share lgkmcnt with the LDS reads and return out of order, and no
        // loop-carried vector loads, whose copies between iterations would wait
        // for every load in flight).
        // Only the kPnCntUsed dwords in use are read (16-byte reads, then one of
        // 4, 8 or 12 bytes): a register loaded and never used would be reused by
        // the compiler while its read is in flight, which costs a wait.
        auto read_counts = [&](const char* p, uint32_t (&c)[kPnCntUsed]) {
            pn_static_for<0, kPnCntUsed / 4>([&](auto jc) {
                constexpr int j = decltype(jc)::value;
                const i32x4v v = *reinterpret_cast<const i32x4v*>(p + 16 * j);
                c[4 * j] = v.x; c[4 * j + 1] = v.y; c[4 * j + 2] = v.z; c[4 * j + 3] = v.w;
            });
            constexpr int b = kPnCntUsed / 4 * 4, rem = kPnCntUsed % 4;
            if constexpr (rem == 1) {
                c[b] = *reinterpret_cast<const uint32_t*>(p + 4 * b);
            } else if constexpr (rem == 2) {
                typedef int i32x2t __attribute__((ext_vector_type(2)));
                const i32x2t v = *reinterpret_cast<const i32x2t*>(p + 4 * b);
                c[b] = v.x; c[b + 1] = v.y;
            } else if constexpr (rem == 3) {
                typedef int i32x3t __attribute__((ext_vector_type(3)));
                const i32x3t v = *reinterpret_cast<const i32x3t*>(p + 4 * b);
                c[b] = v.x; c[b + 1] = v.y; c[b + 2] = v.z;
            }
        };
        // Run data: right after entry i is done with tile t, the run of tile
        // t + 1 ([cur, cur + nn) of its group's row: 1-based position bytes and
        // values, lane g holding nonzero cur + g) is fetched, so its latency hides
        // behind the rest of the tile; lanes past the run take position 0 and
        // value 0 (the zero row, times 0).  Tile 0's runs are fetched before the
        // loop with the same instructions as every later fetch (the compiler's
        // vmcnt waits then count exactly the loads issued after the one they wait
        // for); the fetch after the last tile has nn = 0.
        //   kWin = false: each run is loaded where it lies (masked loads).
        //   kWin = true: through a window per entry, lane g holding nonzero
        //     w0 + g, 16 nonzeros ahead: a run inside the window is taken from it
        //     (ds_bpermute by cur - w0), else a new window is loaded at cur (its
        //     lanes 0 .. nn - 1 are then the run).  A row's runs in consecutive
        //     tiles are consecutive nonzeros, so one window serves several tiles
        //     and each line of the position and value arrays is fetched about
        //     once instead of once per tile (between tiles the B-row staging
        //     pushes those lines out of the L2).  Lanes that keep their window
        //     load out of range (no memory access), so every fetch issues the
        //     same instructions.  Worth its ~10 VALU per entry when runs are short
        //     and the kernel waits on memory (panel_window in planner.cpp).
        // cn: counts of tile t (cursor advance, longest runs); cnx: of tile t + 1.
        uint32_t cn[kPnCntUsed], cnx[kPnCntUsed];
        uint32_t wq[kPnRpg], lq[kPnRpg], rq[kPnRpg];
        float wv[kPnRpg], lv[kPnRpg], rv[kPnRpg];
        int w0[kPnRpg], nnx[kPnRpg];
        bool nd[kPnRpg];
        auto fetch = [&](int i, int nn) {
            const uint32_t k = static_cast<uint32_t>(cur[i] + g);
            if constexpr (kWin) {
                const bool need = nn > 0 && cur[i] + nn > w0[i] + 16;
                const int src = (lane + cur[i] - w0[i]) << 2;
                rq[i] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>(wq[i])));
                rv[i] = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, wv[i])));
                lq[i] = __builtin_amdgcn_raw_buffer_load_b8(rpos, need ? k : kOob, 0, 0);
                lv[i] = load_val<T>(rval, k, need);
                w0[i] = need ? cur[i] : w0[i];
                nd[i] = need;
                nnx[i] = nn;
            } else {
                const bool ok = g < nn;
                lq[i] = __builtin_amdgcn_raw_buffer_load_b8(rpos, ok ? k : kOob, 0, 0);
                lv[i] = load_val<T>(rval, k, ok);
            }
            // loads in the loop's order (no reordering across entries)
            asm volatile("" ::: "memory");
        };
        read_counts(reinterpret_cast<const char*>(a.cnt) + (static_cast<size_t>(u.y) * kPnWaves + wave) * (kPnCntRows * 4),
                    cn);
#pragma unroll
        for (int i = 0; i < kPnRpg; i++) {
            wq[i] = 0u;
            wv[i] = 0.f;
            w0[i] = -64;  // empty: the first run with nonzeros loads a window
            fetch(i, static_cast<int>((cn[i] >> shift) & 255));
        }
        for (int t = 0; t < u.z; t++) {
            pn_barrier();
            const bool more = t + 1 < u.z;
            const uint32_t zb = lds0 + pn_zrow_off<T, E>(t & 1);
            {
                read_counts(smem + pn_cnt_off<T, E>(t & 1) + wave * (kPnCntRows * 4), cnx);
            }
            // entries' longest runs (uniform)
            uint32_t mxw[(kPnRpg + 3) / 4];
#pragma unroll
            for (int w = 0; w < (kPnRpg + 3) / 4; w++)
                mxw[w] = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(cn[kPnMaxDword + w])));
            pn_static_for<0, kPnRpg>([&](auto ic) {
                constexpr int i = decltype(ic)::value;
                const int nmax = static_cast<int>((mxw[i / 4] >> (8 * (i % 4))) & 255);
                uint32_t qq;
                float vv;
                if constexpr (kWin) {
                    // this tile's run: the new window, or the one taken from the old
                    wq[i] = nd[i] ? lq[i] : wq[i];
                    wv[i] = nd[i] ? lv[i] : wv[i];
                    const bool in = g < nnx[i];
                    qq = in ? (nd[i] ? lq[i] : rq[i]) : 0u;
                    vv = in ? (nd[i] ? lv[i] : rv[i]) : 0.f;
                } else {
                    qq = lq[i];
                    vv = lv[i];
                }
                if (nmax > 0) pn_run<T, E>(acc[i], qq, vv, nmax, zb, lanepart);
                cur[i] += static_cast<int>((cn[i] >> shift) & 255);
                fetch(i, more ? static_cast<int>((cnx[i] >> shift) & 255) : 0);
            });
#pragma unroll
            for (int j = 0; j < kPnCntUsed; j++) cn[j] = cnx[j];
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
    };
    if (a.win[u.x]) consume(PnIndex<1>{});
    else consume(PnIndex<0>{});
}

}  // namespace tca
