// tca_spmm.hip -- plan / run / time entry points of libtcaspmm.so and the
// host-pointer driver with the reference our_spmm_balanced contract.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <vector>

#include "common.hpp"
#include "planner.hpp"
#include "row_kernel.hpp"
#include "mfma_common.hpp"
#include "mfma_pair_kernel.hpp"
#include "mfma_dense_kernel.hpp"
#include "mfma_compact_kernel.hpp"
#include "mfma_short_kernel.hpp"
#include "bell_kernel.hpp"
#include "sparse24_kernel.hpp"
#include "device_planner.hpp"
#include "device_panel_planner.hpp"
#include "panel_kernel.hpp"
#include "sddmm_kernel.hpp"

#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

using namespace tca;

#define TCA_HIP_TRY(expr)                                                                               \
    do {                                                                                                \
        hipError_t e_ = (expr);                                                                         \
        if (e_ != hipSuccess)                                                                           \
            return fail(TCA_ERR_HIP, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, __LINE__); \
    } while (0)

struct tca_spmm_plan {
    int32_t M = 0, K = 0, N = 0, nnz = 0, dtype = 0;
    uint32_t flags = 0;
    int device = 0;
    RowPlan rows;
    MfmaPlan mfma;
    int32_t mfma_col_blocks = 0;
    bool mfma_pair = false;  // paired (MFMA + staging wavefront) tile kernel
    bool mfma_short = false; // short-K kernel: every row, windows built in LDS (no pack, no windows table)
    int32_t short_nwin = 0, short_col_blocks = 0, short_steps = 0;
    uint32_t* d_zeros = nullptr;  // 16 zero bytes (short-K kernel: B rows past K, columns past N)
    uint16_t* d_soff = nullptr;   // short-K kernel: per nonzero its half index in its window's A tiles
    int32_t* d_wstart = nullptr;  // short-K kernel: [windows + 1] first nonzero of each window
    std::vector<int32_t> short_wstart;  // the same on the host (kernel arguments when few windows)
    bool mfma_dense = false; // dense-tile kernel (plan keeps dense condensed windows)
    bool mfma_natural = false; // dense kernel: windows span all of K in column order (B rows contiguous)
    bool mfma_compact = false; // dense kernel on compacted steps (non-empty fragment cells only)
    bool mfma_compact_want = false; // compact the dense tiles if every step fits
    int mfma_compact_lb = 3;   // compact kernel: transfer lookahead in iterations (3, or 4 by TCA_COMPACT_LB)
    uint64_t* d_amask = nullptr;  // compact kernel: [global step][8] non-empty cells per row block
    uint16_t* d_adense = nullptr;  // dense kernel: [global step] 8 KiB A tile, then 1 KiB of zeros
    size_t adense_halves = 0;
    int32_t n_dn = 0;              // dense kernel: nonzeros the pack writes
    int* d_dn_src = nullptr;       // per nonzero (sorted by position): its CSR index
    uint32_t* d_dn_pos = nullptr;  // and its half index in d_adense
    int32_t mfma_groups = 0; // paired kernel: groups of 64 entries a step may hold (4 or 8)
    size_t mfma_zeros_at = 0;  // word offset of 16 zero bytes in d_packed (LDS-DMA kernel)
    size_t n_packed = 0;       // words of d_packed
    size_t n_ucols = 0;        // words of d_ucols
    int4* d_windows = nullptr;
    uint32_t* d_ucols = nullptr;
    int* d_eoff = nullptr;
    i32x2v* d_emeta = nullptr;      // paired kernel: {first word of each step's packed block, groups of 64}
    int32_t n_pk_words = 0;         // words of d_packed that the pack kernel writes
    int* d_pk_src = nullptr;        // per packed word: CSR index of its nonzero, -1 for none
    uint16_t* d_pk_cell = nullptr;  // per packed word: its cell (low 16 bits)
    uint32_t* d_packed = nullptr;   // cell | value << 16 per entry word (rewritten each run), then 16 zero bytes
    int32_t ntasks = 0;
    int* d_rowptr = nullptr;
    int* d_colidx = nullptr;
    int4* d_tasks = nullptr;
    int32_t* d_torder = nullptr;  // row-kernel launch order (null: task order)
    int32_t n_torder = 0;
    int* d_perm = nullptr;
    int4* d_longrows = nullptr;
    int32_t n_longrows = 0;   // rows split into segments (entries of d_longrows)
    size_t n_seg_total = 0;   // their segments (rows of d_partials)
    int32_t n_perm = 0;       // rows in multi tasks (entries of d_perm)
    bool device_planned = false;
    float* d_partials = nullptr;
    // row panels (panel kernel)
    PanelPlan panels;
    int32_t n_units = 0, n_pblocks = 0;  // panel units; panel workgroups (units and idle ones)
    int4* d_units = nullptr;
    int32_t* d_porder = nullptr;
    int* d_panel_units = nullptr;
    uint8_t* d_pwin = nullptr;  // [panel]: run data through per-row windows (PanelPlan::win)
    int* d_prows = nullptr;
    int* d_pcols = nullptr;  // panel tiles' staged B rows, as byte offsets into B
    uint32_t* d_pcnt = nullptr;
    uint8_t* d_ppos = nullptr;
    int* d_ustart = nullptr;
    size_t n_pos_bytes = 0;  // d_ppos, whole dwords
    int64_t n_ptiles = 0;    // panel tiles (d_pcols: n_ptiles * P entries)
    int32_t n_plongrows = 0; // the panels' long rows: the last entries of d_longrows
    // A row phase that only clears empty rows (every nonzero is in panels or
    // tiles) runs on this second stream of the plan, beside the panel kernel:
    // forked after the phases before the panels, joined before the segment
    // sums (null: the phases run in order on the caller's stream).
    hipStream_t side = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    tca_plan_info info{};
};

// The allocation-free run's partial rows (tca_spmm_run_static): one
// file-scope device array per GPU, held until the process ends.  Its
// host-side name is not a device address: host code uses only the address
// hipGetSymbolAddress returns for the current device (kept per device).
constexpr size_t kStaticScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's copy of `scratch` (looked up once per device, with that
// device current).
int static_scratch(int dev, float** out) {
    if (dev < 0 || dev >= kMaxDevices) return fail(TCA_ERR_UNSUPPORTED, "device %d: too many devices", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) return fail(TCA_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = static_cast<float*>(g_scratch_ptr[dev]);
    return TCA_OK;
}

__global__ void warm_up_kernel() {}

// Every device allocation of the library goes through here (so
// tca_debug_fail_allocs can make one fail).
static hipError_t dev_malloc(void** p, size_t bytes) {
    if (device_alloc_fails()) {
        *p = nullptr;
        return hipErrorOutOfMemory;
    }
    return hipMalloc(p, bytes);
}

template <typename T>
int dev_upload(T** dst, const void* src, size_t count) {
    *dst = nullptr;
    if (count == 0) return TCA_OK;
    hipError_t e = dev_malloc(reinterpret_cast<void**>(dst), sizeof(T) * count);
    if (e != hipSuccess) {
        *dst = nullptr;
        return fail(TCA_ERR_ALLOC, "hipMalloc(%zu bytes): %s", sizeof(T) * count, hipGetErrorString(e));
    }
    if (src) {
        e = hipMemcpy(*dst, src, sizeof(T) * count, hipMemcpyHostToDevice);
        if (e != hipSuccess) return fail(TCA_ERR_HIP, "hipMemcpy H2D: %s", hipGetErrorString(e));
    }
    return TCA_OK;
}

void free_plan_device(tca_spmm_plan* p) {
    (void)hipFree(p->d_zeros);
    (void)hipFree(p->d_soff);
    (void)hipFree(p->d_wstart);
    (void)hipFree(p->d_rowptr);
    (void)hipFree(p->d_colidx);
    (void)hipFree(p->d_tasks);
    (void)hipFree(p->d_torder);
    (void)hipFree(p->d_perm);
    (void)hipFree(p->d_longrows);
    (void)hipFree(p->d_partials);
    (void)hipFree(p->d_windows);
    (void)hipFree(p->d_ucols);
    (void)hipFree(p->d_eoff);
    (void)hipFree(p->d_emeta);
    (void)hipFree(p->d_pk_src);
    (void)hipFree(p->d_pk_cell);
    (void)hipFree(p->d_packed);
    (void)hipFree(p->d_adense);
    (void)hipFree(p->d_amask);
    (void)hipFree(p->d_dn_src);
    (void)hipFree(p->d_dn_pos);
    (void)hipFree(p->d_units);
    (void)hipFree(p->d_porder);
    (void)hipFree(p->d_panel_units);
    (void)hipFree(p->d_pwin);
    (void)hipFree(p->d_prows);
    (void)hipFree(p->d_pcols);
    (void)hipFree(p->d_pcnt);
    (void)hipFree(p->d_ppos);
    (void)hipFree(p->d_ustart);
    if (p->fork) (void)hipEventDestroy(p->fork);
    if (p->join) (void)hipEventDestroy(p->join);
    if (p->side) (void)hipStreamDestroy(p->side);
}

// Owns a plan under construction: frees it (device buffers included) unless
// released, so every early return and every exception of plan creation
// leaves nothing behind.
struct PlanHolder {
    tca_spmm_plan* p;
    ~PlanHolder() {
        if (p) {
            free_plan_device(p);
            delete p;
        }
    }
    tca_spmm_plan* release() {
        tca_spmm_plan* q = p;
        p = nullptr;
        return q;
    }
};

// Row-kernel workgroups: kRowWaves task slots each (the launch order's
// slots, or the tasks), times the column chunks.
int row_blocks(const tca_spmm_plan* p) {
    const int slots = p->n_torder > 0 ? p->n_torder : p->ntasks;
    return ((slots + kRowWaves - 1) / kRowWaves) * p->rows.col_chunks;
}

// Kernel launch of one phase of a run.  While tca_spmm_time_phases has a
// phase armed (g_phase_ev[0] set on this thread), the dispatch itself
// carries that phase's start and stop timestamps (hipExtLaunchKernelGGL:
// the same span a kernel trace reports, with no event packets between the
// kernels); otherwise it is a plain launch.  Every phase launches one kernel.
thread_local hipEvent_t g_phase_ev[2] = {nullptr, nullptr};
#define TCA_PHASE_LAUNCH(kernel, grid, block, shm, stream, ...)                                                 \
    do {                                                                                                        \
        if (g_phase_ev[0])                                                                                      \
            hipExtLaunchKernelGGL(kernel, grid, block, shm, stream, g_phase_ev[0], g_phase_ev[1], 0, __VA_ARGS__); \
        else                                                                                                    \
            hipLaunchKernelGGL(kernel, grid, block, shm, stream, __VA_ARGS__);                                  \
    } while (0)

template <typename T, int E>
void launch_rows_t(const tca_spmm_plan* p, const void* val, const void* B, float* C, float* W, hipStream_t s) {
    RowArgs a;
    a.tasks = p->d_tasks;
    a.order = p->d_torder;
    a.ntasks = p->ntasks;
    a.rowptr = p->d_rowptr;
    a.perm = p->d_perm;
    a.partials = W;
    a.C = C;
    a.N = p->N;
    a.logG = p->rows.log_lanes;
    a.chunk_lanes = p->rows.chunk_lanes;
    a.col_chunks = p->rows.col_chunks;
    a.colidx = p->d_colidx;
    a.val = val;
    a.B = B;
    // Byte sizes of the buffer ranges (checked < 2^32 - 16 at plan time).
    a.colidx_bytes = static_cast<uint32_t>(static_cast<uint64_t>(p->nnz) * 4);
    a.val_bytes = static_cast<uint32_t>(static_cast<uint64_t>(p->nnz) * sizeof(T));
    a.B_bytes = static_cast<uint32_t>(static_cast<uint64_t>(p->K) * p->N * sizeof(T));
    TCA_PHASE_LAUNCH((row_kernel<T, E>), dim3(row_blocks(p)), dim3(64 * kRowWaves), 0, s, a);
}

// Adds the segments of long rows (after the row kernel, same stream).
void launch_finalize(const tca_spmm_plan* p, float* C, const float* W, hipStream_t s) {
    if (p->n_longrows == 0) return;
    const dim3 fgrid(static_cast<unsigned>(p->n_longrows), (p->N + 4 * fin_lanes(p->N) - 1) / (4 * fin_lanes(p->N)));
    TCA_PHASE_LAUNCH(seg_finalize_kernel, fgrid, dim3(256), 0, s, p->d_longrows, W, C, p->N);
}

template <typename T>
int launch_rows_e(const tca_spmm_plan* p, const void* val, const void* B, float* C, float* W, hipStream_t s) {
    switch (p->rows.elems_per_lane) {
        case 1: launch_rows_t<T, 1>(p, val, B, C, W, s); return TCA_OK;
        case 2: launch_rows_t<T, 2>(p, val, B, C, W, s); return TCA_OK;
        case 4: launch_rows_t<T, 4>(p, val, B, C, W, s); return TCA_OK;
        case 8:
            if constexpr (sizeof(T) == 2) {
                launch_rows_t<T, 8>(p, val, B, C, W, s);
                return TCA_OK;
            }
            [[fallthrough]];
        default: return fail(TCA_ERR_INVALID, "bad lane geometry");
    }
}

// Pairs the MFMA entries with this run's values (before the tile kernel).
void launch_pack(const tca_spmm_plan* p, const void* val, hipStream_t s) {
    if (p->mfma_dense) {
        if (p->n_dn > 0)
            TCA_PHASE_LAUNCH(dense_pack_kernel, dim3((p->n_dn + 255) / 256), dim3(256), 0, s, p->d_dn_src,
                               p->d_dn_pos, p->n_dn, static_cast<const uint16_t*>(val), p->d_adense);
        return;
    }
    const int n = p->n_pk_words;
    if (p->mfma.windows.empty() || n == 0) return;
    TCA_PHASE_LAUNCH(mfma_pack_kernel, dim3((n + 1023) / 1024), dim3(256), 0, s, p->d_pk_src, p->d_pk_cell, n,
                       static_cast<const uint16_t*>(val), p->d_packed);
}

static_assert(kPnWaves == kPanelWaves && kPnRpg == kPanelRpg && kPnCntRows == kPanelCntRows &&
                  kPnMaxDword == kPanelMaxDword, "panel plan layout");
static_assert(PanelGeom<float, 8>::kP == 152 && PanelGeom<float, 4>::kP == 255 && PanelGeom<float, 2>::kP == 255,
              "panel tile widths (panel_tile_cols)");
static_assert(panel_lds_bytes(512) <= 160 * 1024, "panel LDS budget");
static_assert(kMfmaPairShape.max_step_entries == kDmaMaxStepEntries, "planner and paired kernel agree on step size");
static_assert(kMfmaPairShape.win_rows == kDmaWinRows && kMfmaPairShape.tile_cols == kDmaTileCols, "paired tile shape");
static_assert(kMfmaDenseShape.win_rows == kDmaWinRows && kMfmaDenseShape.tile_cols == kDmaTileCols, "dense tile shape");
static_assert(kMfmaPairShape.max_step_entries <= 8 * kPairGroup, "paired kernel: at most 8 entry groups per step");
static_assert(kPairThreads == kDnThreads, "tile kernels share one workgroup size");

int launch_short(const tca_spmm_plan* p, const void* val, const void* B, float* C, hipStream_t s) {
    ShortArgs a;
    a.wstart = p->d_wstart;
    a.soff = p->d_soff;
    a.val = static_cast<const uint16_t*>(val);
    a.B = B;
    a.C = C;
    a.zeros = p->d_zeros;
    a.M = p->M;
    a.K = p->K;
    a.N = p->N;
    a.nwin = p->short_nwin;
    a.col_blocks = p->short_col_blocks;
    a.steps = p->short_steps;
    if (a.nwin <= kShArgWindows)
        for (int w = 0; w <= a.nwin; w++) a.wstart_arg[w] = p->short_wstart[w];
    const dim3 grid(mfma_short_grid(a.nwin, a.col_blocks));
    if (p->dtype == TCA_BF16) TCA_PHASE_LAUNCH(mfma_short_kernel<true>, grid, dim3(kShThreads), 0, s, a);
    else TCA_PHASE_LAUNCH(mfma_short_kernel<false>, grid, dim3(kShThreads), 0, s, a);
    return TCA_OK;
}

int launch_mfma(const tca_spmm_plan* p, const void* val, const void* B, float* C, hipStream_t s) {
    if (p->mfma_short) return launch_short(p, val, B, C, s);
    if (p->mfma.windows.empty()) return TCA_OK;
    MfmaArgs a;
    a.windows = p->d_windows;
    a.ucols = p->d_ucols;
    a.eoff = p->d_eoff;
    a.emeta = p->d_emeta;
    a.packed = p->d_packed;
    a.B = B;
    a.C = C;
    a.M = p->M;
    a.N = p->N;
    a.col_blocks = p->mfma_col_blocks;
    a.B_bytes = static_cast<uint32_t>(static_cast<uint64_t>(p->K) * p->N * 2);
    a.zeros = p->d_packed + p->mfma_zeros_at;
    a.packed_bytes = static_cast<uint32_t>(p->n_packed * 4);
    a.ucols_bytes = static_cast<uint32_t>(p->mfma.ucols.size() * 4);
    a.eoff_bytes = static_cast<uint32_t>(p->mfma.eoff.size() * 4);
    const dim3 grid(static_cast<unsigned>(p->mfma.windows.size()) * p->mfma_col_blocks);
    const bool bf = p->dtype == TCA_BF16;
    if (p->mfma_dense) {
        a.adense = p->d_adense;
        a.zeros = p->d_adense + (p->adense_halves - 512);
        a.n_windows = static_cast<int>(p->mfma.windows.size());
        a.K = p->K;
        a.amask = p->d_amask;
        const dim3 dgrid(mfma_dense_grid(a.n_windows, p->mfma_col_blocks));
        if (p->mfma_compact) {
            const int v = (bf ? 1 : 0) | (p->mfma_natural ? 2 : 0) | (p->mfma_compact_lb == 3 ? 4 : 0);
            switch (v) {
                case 0: TCA_PHASE_LAUNCH((mfma_compact_kernel<false, false, 4>), dgrid, dim3(kDnThreads), 0, s, a); break;
                case 1: TCA_PHASE_LAUNCH((mfma_compact_kernel<true, false, 4>), dgrid, dim3(kDnThreads), 0, s, a); break;
                case 2: TCA_PHASE_LAUNCH((mfma_compact_kernel<false, true, 4>), dgrid, dim3(kDnThreads), 0, s, a); break;
                case 3: TCA_PHASE_LAUNCH((mfma_compact_kernel<true, true, 4>), dgrid, dim3(kDnThreads), 0, s, a); break;
                case 4: TCA_PHASE_LAUNCH((mfma_compact_kernel<false, false, 3>), dgrid, dim3(kDnThreads), 0, s, a); break;
                case 5: TCA_PHASE_LAUNCH((mfma_compact_kernel<true, false, 3>), dgrid, dim3(kDnThreads), 0, s, a); break;
                case 6: TCA_PHASE_LAUNCH((mfma_compact_kernel<false, true, 3>), dgrid, dim3(kDnThreads), 0, s, a); break;
                default: TCA_PHASE_LAUNCH((mfma_compact_kernel<true, true, 3>), dgrid, dim3(kDnThreads), 0, s, a); break;
            }
            return TCA_OK;
        }
        if (p->mfma_natural) {
            if (bf) TCA_PHASE_LAUNCH((mfma_dense_kernel<true, true>), dgrid, dim3(kDnThreads), 0, s, a);
            else TCA_PHASE_LAUNCH((mfma_dense_kernel<false, true>), dgrid, dim3(kDnThreads), 0, s, a);
        } else {
            if (bf) TCA_PHASE_LAUNCH((mfma_dense_kernel<true, false>), dgrid, dim3(kDnThreads), 0, s, a);
            else TCA_PHASE_LAUNCH((mfma_dense_kernel<false, false>), dgrid, dim3(kDnThreads), 0, s, a);
        }
        return TCA_OK;
    }
    if (p->mfma_pair) {
        switch (p->mfma_groups) {
            case 4:
                if (bf) TCA_PHASE_LAUNCH((mfma_pair_kernel<true, 4>), grid, dim3(kPairThreads), 0, s, a);
                else TCA_PHASE_LAUNCH((mfma_pair_kernel<false, 4>), grid, dim3(kPairThreads), 0, s, a);
                return TCA_OK;
            case 8:
                if (bf) TCA_PHASE_LAUNCH((mfma_pair_kernel<true, 8>), grid, dim3(kPairThreads), 0, s, a);
                else TCA_PHASE_LAUNCH((mfma_pair_kernel<false, 8>), grid, dim3(kPairThreads), 0, s, a);
                return TCA_OK;
            default: return fail(TCA_ERR_INVALID, "bad MFMA entry group count %d", p->mfma_groups);
        }
    }
    return fail(TCA_ERR_INVALID, "plan has MFMA windows but no tile kernel");
}

int launch_rows(const tca_spmm_plan* p, const void* val, const void* B, float* C, float* W, hipStream_t s) {
    if (p->ntasks == 0) return TCA_OK;
    switch (p->dtype) {
        case TCA_F16: return launch_rows_e<_Float16>(p, val, B, C, W, s);
        case TCA_BF16: return launch_rows_e<bf16_t>(p, val, B, C, W, s);
        default: return launch_rows_e<float>(p, val, B, C, W, s);
    }
}

template <typename T, int E>
void launch_panels_t(const tca_spmm_plan* p, const void* val, const void* B, float* C, float* W, hipStream_t s) {
    PanelArgs a;
    a.units = p->d_units;
    a.order = p->d_porder;
    a.panel_units = p->d_panel_units;
    a.win = p->d_pwin;
    a.rows = p->d_prows;
    a.boff = reinterpret_cast<const uint32_t*>(p->d_pcols);
    a.cnt = p->d_pcnt;
    a.pos = p->d_ppos;
    a.ustart = p->d_ustart;
    a.val = val;
    a.B = B;
    a.C = C;
    a.partials = W;
    a.N = p->N;
    a.chunks = p->panels.chunks;
    a.pos_bytes = static_cast<uint32_t>(p->n_pos_bytes);
    a.val_bytes = static_cast<uint32_t>(static_cast<uint64_t>(p->nnz) * sizeof(T));
    TCA_PHASE_LAUNCH((panel_kernel<T, E>), dim3(p->n_pblocks * p->panels.chunks), dim3(kPnThreads), 0, s, a);
}

int launch_panels(const tca_spmm_plan* p, const void* val, const void* B, float* C, float* W, hipStream_t s) {
    if (p->n_units == 0) return TCA_OK;
    const int e = p->panels.elems;
    switch (p->dtype) {
        case TCA_F32:
            if (e == 8) launch_panels_t<float, 8>(p, val, B, C, W, s);
            else if (e == 4) launch_panels_t<float, 4>(p, val, B, C, W, s);
            else if (e == 2) launch_panels_t<float, 2>(p, val, B, C, W, s);
            else return fail(TCA_ERR_INVALID, "bad panel geometry");
            return TCA_OK;
        case TCA_F16:
            if (e == 8) launch_panels_t<_Float16, 8>(p, val, B, C, W, s);
            else if (e == 4) launch_panels_t<_Float16, 4>(p, val, B, C, W, s);
            else return fail(TCA_ERR_INVALID, "bad panel geometry");
            return TCA_OK;
        default:
            if (e == 8) launch_panels_t<bf16_t, 8>(p, val, B, C, W, s);
            else if (e == 4) launch_panels_t<bf16_t, 4>(p, val, B, C, W, s);
            else return fail(TCA_ERR_INVALID, "bad panel geometry");
            return TCA_OK;
    }
}

// Bit 1 << TCA_PHASE_* for each phase in which the plan launches a kernel.
uint32_t phases_used(const tca_spmm_plan* p) {
    uint32_t m = 0;
    if (!p->mfma.windows.empty() && (!p->mfma.entries.empty() || p->n_dn > 0)) m |= 1u << TCA_PHASE_PACK;
    if (!p->mfma.windows.empty() || p->mfma_short) m |= 1u << TCA_PHASE_TILES;
    if (p->ntasks > 0) m |= 1u << TCA_PHASE_ROWS;
    if (p->n_longrows > 0) m |= 1u << TCA_PHASE_SEGMENTS;
    if (p->n_units > 0) m |= 1u << TCA_PHASE_PANELS;
    return m;
}

// One SpMM in stream order: pack, tile kernel, panel kernel, row kernel, segment sums.
// W: the partial rows of split rows (plan-owned, or the static scratch).
// mask: the phases to launch (bit 1 << TCA_PHASE_*); all of them for a product.
int run_phases(const tca_spmm_plan* p, const void* val, const void* B, float* C, float* W, hipStream_t s,
               uint32_t mask = ~0u) {
    if (mask & (1u << TCA_PHASE_PACK)) launch_pack(p, val, s);
    int st = TCA_OK;
    if (mask & (1u << TCA_PHASE_TILES)) st = launch_mfma(p, val, B, C, s);
    if (st) return st;
    const uint32_t both = (1u << TCA_PHASE_PANELS) | (1u << TCA_PHASE_ROWS);
    const bool beside = p->side && (mask & both) == both;
    if (beside && (hipEventRecord(p->fork, s) != hipSuccess || hipStreamWaitEvent(p->side, p->fork, 0) != hipSuccess))
        return fail(TCA_ERR_HIP, "fork to the plan's second stream failed");
    if (mask & (1u << TCA_PHASE_PANELS)) st = launch_panels(p, val, B, C, W, s);
    if (st) return st;
    if (mask & (1u << TCA_PHASE_ROWS)) st = launch_rows(p, val, B, C, W, beside ? p->side : s);
    if (st) return st;
    if (beside && (hipEventRecord(p->join, p->side) != hipSuccess || hipStreamWaitEvent(s, p->join, 0) != hipSuccess))
        return fail(TCA_ERR_HIP, "join of the plan's second stream failed");
    if (mask & (1u << TCA_PHASE_SEGMENTS)) launch_finalize(p, C, W, s);
    return TCA_OK;
}

// The second stream of a plan whose row phase only clears empty rows: those
// stores then run beside the panel kernel instead of after it (an R-MAT graph
// with every row in panels: 2.606-2.611 -> 2.552-2.556 ms per step; with
// gathering row tasks beside the panels the step was slower).
// TCA_ROWS_BESIDE=0 keeps every phase on the caller's stream (tuning override).
// The stream and its events are an optimisation: when the runtime cannot
// create them the plan keeps one stream (rows_beside_panels = 0), no error.
void setup_side_stream(tca_spmm_plan* p) {
    if (p->n_units == 0 || p->ntasks == 0) return;
    if (static_cast<int64_t>(p->nnz) - p->panels.nnz - p->mfma.nnz != 0) return;
    if (const char* e = std::getenv("TCA_ROWS_BESIDE"))
        if (std::atoi(e) == 0) return;
    if (hipStreamCreateWithFlags(&p->side, hipStreamNonBlocking) != hipSuccess) p->side = nullptr;
    if (p->side && hipEventCreateWithFlags(&p->fork, hipEventDisableTiming) != hipSuccess) p->fork = nullptr;
    if (p->fork && hipEventCreateWithFlags(&p->join, hipEventDisableTiming) != hipSuccess) p->join = nullptr;
    if (!p->join) {
        if (p->fork) (void)hipEventDestroy(p->fork);
        if (p->side) (void)hipStreamDestroy(p->side);
        p->side = nullptr;
        p->fork = nullptr;
        (void)hipGetLastError();  // the failed creation is not the next call's error
        return;
    }
    p->info.rows_beside_panels = 1;
}

// Plan statistics (tca_plan_info) from a built plan.
void fill_info(tca_spmm_plan* p) {
    tca_plan_info& in = p->info;
    in.M = p->M;
    in.K = p->K;
    in.N = p->N;
    in.nnz = p->nnz;
    in.dtype = p->dtype;
    in.elems_per_lane = p->rows.elems_per_lane;
    in.lanes_per_row = 1 << p->rows.log_lanes;
    in.col_chunks = p->rows.col_chunks;
    in.n_row_tasks = p->ntasks;
    in.n_multi_tasks = p->rows.n_multi;
    in.n_seg_tasks = p->rows.n_seg;
    in.n_long_rows = p->n_longrows;
    in.n_wide_tasks = p->rows.n_wide;
    in.chunk_lanes = p->rows.chunk_lanes;
    in.row_len = p->rows.row_len;
    in.wide_len = p->rows.wide_len;
    in.row_blocks = row_blocks(p);
    in.row_blockdim = 64 * kRowWaves;
    in.seg_len = p->rows.seg_len;
    in.n_windows_mfma = static_cast<int32_t>(p->mfma.windows.size());
    in.rows_mfma = p->mfma.rows;
    in.nnz_mfma = p->mfma.nnz;
    in.cond_cols_mfma = p->mfma.cond_cols;
    in.mfma_blocks = p->mfma_dense ? mfma_dense_grid(in.n_windows_mfma, p->mfma_col_blocks)
                                   : in.n_windows_mfma * p->mfma_col_blocks;
    in.mfma_blockdim = kPairThreads;
    if (p->mfma_dense && p->mfma_compact)
        in.mfma_lds_bytes = p->mfma_compact_lb == 3 ? mfma_compact_lds_bytes<3>() : mfma_compact_lds_bytes<4>();
    else if (p->mfma_dense)
        in.mfma_lds_bytes = mfma_dense_lds_bytes();
    else if (p->mfma_pair)
        in.mfma_lds_bytes = mfma_pair_lds_bytes();
    in.scratch_bytes = static_cast<int64_t>(p->n_seg_total * p->N * sizeof(float));
    in.n_panels = p->panels.n_panels;
    in.n_panel_units = p->n_units;
    in.rows_panels = p->panels.n_rows;
    in.panel_blocks = p->n_pblocks * p->panels.chunks;
    in.nnz_panels = p->panels.nnz;
    in.staged_panels = p->panels.staged;
    in.panel_blockdim = kPnThreads;
    in.panel_lds_bytes =
        p->n_units ? panel_lds_bytes(16 * p->panels.elems * static_cast<int>(dtype_size(p->dtype))) : 0;
    in.panel_window = 0;
    if (p->n_units)
        for (uint8_t w : p->panels.win) in.panel_window += w;
    if (p->mfma_short) {
        in.n_windows_mfma = p->short_nwin;
        in.rows_mfma = p->M;
        in.nnz_mfma = p->nnz;
        in.cond_cols_mfma = static_cast<int64_t>(p->short_nwin) * p->short_steps * kStepK;
        in.mfma_blocks = mfma_short_grid(p->short_nwin, p->short_col_blocks);
        in.mfma_blockdim = kShThreads;
        in.mfma_lds_bytes = kShLdsBytes;
    }
    in.tile_kernel = p->mfma_short          ? TCA_TILES_SHORT
                     : p->mfma.windows.empty() ? TCA_TILES_NONE
                     : p->mfma_compact      ? TCA_TILES_COMPACT
                     : p->mfma_dense        ? (p->mfma_natural ? TCA_TILES_DENSE_K : TCA_TILES_DENSE)
                                            : TCA_TILES_PAIR;
}

// The reference prints its one kernel's grid, block and dynamic LDS
// (src/our_spmm.cu:552).  A plan here launches up to four kernels
// (run_phases); one line per kernel it launches, in launch order, same
// format, the kernel named after it.
void print_launches(const tca_spmm_plan* p) {
    const tca_plan_info& in = p->info;
    auto line = [](long long blocks, int dim, double lds_bytes, const char* name) {
        std::printf("num_block: %lld blockdim: %d shm: %fKB (%s)\n", blocks, dim, lds_bytes / 1024.0, name);
    };
    if (p->mfma_short) line(in.mfma_blocks, in.mfma_blockdim, in.mfma_lds_bytes, "mfma_short_kernel");
    if (!p->mfma.windows.empty()) {
        if (p->mfma_dense) {
            if (p->n_dn > 0) line((p->n_dn + 255) / 256, 256, 0.0, "dense_pack_kernel");
        } else if (p->n_pk_words > 0) {
            line((p->n_pk_words + 1023) / 1024, 256, 0.0, "mfma_pack_kernel");
        }
        static const char* names[] = {"", "", "", "mfma_pair_kernel", "mfma_dense_kernel", "mfma_dense_kernel", "",
                                      "mfma_compact_kernel", "mfma_short_kernel"};
        line(in.mfma_blocks, in.mfma_blockdim, in.mfma_lds_bytes, names[in.tile_kernel]);
    }
    if (p->n_units > 0) line(in.panel_blocks, in.panel_blockdim, in.panel_lds_bytes, "panel_kernel");
    if (p->ntasks > 0)  // static LDS of row_kernel: kRowWaves partial row chunks of 64 lanes x E floats
        line(in.row_blocks, in.row_blockdim, 4.0 * kRowWaves * 64 * p->rows.elems_per_lane, "row_kernel");
    if (p->n_longrows > 0)
        line(static_cast<long long>(p->n_longrows) * ((p->N + 4 * fin_lanes(p->N) - 1) / (4 * fin_lanes(p->N))), 256, 0.0,
             "seg_finalize_kernel");
}

}  // namespace

extern "C" {

int tca_version(void) { return 100; }

int tca_warm_up(void) {
    hipLaunchKernelGGL(warm_up_kernel, dim3(1), dim3(64), 0, nullptr);
    TCA_HIP_TRY(hipGetLastError());
    TCA_HIP_TRY(hipDeviceSynchronize());
    return TCA_OK;
}

int tca_launch_floor(void* stream, int32_t iters, float* avg_ms) {
    if (iters < 1 || !avg_ms) return fail(TCA_ERR_INVALID, "tca_launch_floor: bad argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(warm_up_kernel, dim3(1), dim3(64), 0, s);
    hipEvent_t e0, e1;
    TCA_HIP_TRY(hipEventCreate(&e0));
    TCA_HIP_TRY(hipEventCreate(&e1));
    (void)hipEventRecord(e0, s);
    for (int i = 0; i < iters; i++) hipLaunchKernelGGL(warm_up_kernel, dim3(1), dim3(64), 0, s);
    (void)hipEventRecord(e1, s);
    float ms = 0.f;
    const bool ok = hipEventSynchronize(e1) == hipSuccess && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (!ok) return fail(TCA_ERR_HIP, "event timing failed");
    *avg_ms = ms / static_cast<float>(iters);
    return TCA_OK;
}

int tca_device_count(int32_t* count) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        *count = 0;
        return fail(TCA_ERR_HIP, "hipGetDeviceCount: %s", hipGetErrorString(e));
    }
    *count = n;
    return TCA_OK;
}

// Routing of the short-K kernel: fp16 / bf16, N % 8 == 0, K <= 640, and by
// default rows at least kShMinDensity full on average (and 8 nonzeros).  Its
// cost per window grows with K (B staged, A zeroed, K / 32 MFMA steps), the
// row kernel's with the nonzeros (one B-row gather each).  Measured on the
// MI355X, fp16, N = 256 (short vs row kernel, per SpMM): 65536 x 512 at
// 10 %: 71 vs 166 us; 16384 x 512 at 10 %: 19.2 vs 21.5; 2048 x 512 at
// 10 %: 5.53 vs 5.51; 65536 x 256 at 5 % (N = 128): 27.3 vs 27.1;
// 65536 x 640 at 2 %: 74 vs 38.  TCA_PLAN_MFMA_SHORT asks for it whatever
// the density; the other tile-kernel flags and TCA_PLAN_NO_MFMA keep it off.
constexpr double kShMinDensity = 0.08;
static bool short_route(int32_t M, int32_t K, int32_t nnz, int32_t N, int32_t dtype, uint32_t flags) {
    if (dtype == TCA_F32 || N % 8 != 0 || K > kShMaxSteps * kStepK || M == 0 || (flags & TCA_PLAN_NO_MFMA))
        return false;
    if (flags & TCA_PLAN_MFMA_SHORT) return true;
    if (flags & (TCA_PLAN_MFMA_DENSE | TCA_PLAN_MFMA_PAIR | TCA_PLAN_MFMA_COMPACT)) return false;
    const double per_row = static_cast<double>(nnz) / M;
    return per_row >= 8.0 && per_row >= kShMinDensity * K;
}

// Half index of nonzero (row, col) in its window's A tiles (mfma_short_kernel.hpp).
__host__ __device__ inline uint16_t short_soff(int32_t row, int32_t col) {
    return static_cast<uint16_t>((col >> 5) * (kShATileBytes / 2) + a_cell(row % kShRows, col & 31));
}

// The short-K kernel's plan: sizes, zero bytes, per-nonzero tile offsets and
// window starts (from the host structure).
static int setup_short(tca_spmm_plan* p, const int32_t* rowptr, const int32_t* colidx) {
    p->short_nwin = (p->M + kShRows - 1) / kShRows;
    p->short_col_blocks = (p->N + kDmaTileCols - 1) / kDmaTileCols;
    p->short_steps = (p->K + kStepK - 1) / kStepK;
    const uint32_t z[4] = {0, 0, 0, 0};
    int st = dev_upload(&p->d_zeros, z, 4);
    if (st) return st;
    std::vector<uint16_t> so(static_cast<size_t>(p->nnz));
    for (int32_t r = 0; r < p->M; r++)
        for (int32_t j = rowptr[r]; j < rowptr[r + 1]; j++) so[j] = short_soff(r, colidx[j]);
    p->short_wstart.resize(static_cast<size_t>(p->short_nwin) + 1);
    for (int32_t w = 0; w <= p->short_nwin; w++) p->short_wstart[w] = rowptr[std::min(w * kShRows, p->M)];
    if ((st = dev_upload(&p->d_soff, so.data(), so.size()))) return st;
    return dev_upload(&p->d_wstart, p->short_wstart.data(), p->short_wstart.size());
}

// Device planning of the same: one thread per row.
__global__ void dp_short_kernel(const int32_t* __restrict__ rowptr, const int32_t* __restrict__ colidx, int32_t M,
                                uint16_t* __restrict__ soff, int32_t* __restrict__ wstart) {
    const int32_t r = blockIdx.x * 256 + threadIdx.x;
    if (r > M) return;
    if (r % kShRows == 0 || r == M) wstart[(r + kShRows - 1) / kShRows] = rowptr[r];
    if (r == M) return;
    for (int32_t j = rowptr[r]; j < rowptr[r + 1]; j++) soff[j] = short_soff(r, colidx[j]);
}

int tca_spmm_plan_create(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t K, int32_t nnz,
                         int32_t N, int32_t dtype, uint32_t flags, tca_spmm_plan** plan) {
    return api_guard("tca_spmm_plan_create", [&]() -> int {
        if (!plan) return fail(TCA_ERR_INVALID, "plan is NULL");
        *plan = nullptr;
        if (M < 0 || K < 1 || N < 1 || nnz < 0) return fail(TCA_ERR_INVALID, "bad shape M=%d K=%d N=%d nnz=%d", M, K, N, nnz);
        if (!dtype_ok(dtype)) return fail(TCA_ERR_INVALID, "unknown dtype %d", dtype);
        if (flags & ~TCA_PLAN_KNOWN_FLAGS) return fail(TCA_ERR_INVALID, "unknown plan flags 0x%x", flags & ~TCA_PLAN_KNOWN_FLAGS);
        // The kernels address B, values and column indices through 32-bit buffer
        // offsets, with 0xfffffff0 reserved as the out-of-range marker.
        const uint64_t b_bytes = static_cast<uint64_t>(K) * static_cast<uint64_t>(N) * dtype_size(dtype);
        if (b_bytes >= 0xfffffff0ull || static_cast<uint64_t>(nnz) * 4 >= 0xfffffff0ull)
            return fail(TCA_ERR_UNSUPPORTED, "B (%llu bytes) or the nonzeros exceed the 4 GiB buffer range",
                        (unsigned long long)b_bytes);
        int st = tca_csr_validate(rowptr, colidx, M, K, nnz);
        if (st) return st;
        const auto t0 = std::chrono::steady_clock::now();
        tca_spmm_plan* p = new (std::nothrow) tca_spmm_plan();
        if (!p) return fail(TCA_ERR_ALLOC, "plan allocation failed");
        PlanHolder hold{p};
        p->M = M;
        p->K = K;
        p->N = N;
        p->nnz = nnz;
        p->dtype = dtype;
        p->flags = flags;
        if (hipGetDevice(&p->device) != hipSuccess) return fail(TCA_ERR_HIP, "no HIP device");
        // Dense-enough 128-row windows go to an MFMA tile kernel (fp16 / bf16),
        // 64 columns of C per workgroup: the paired kernel, or the dense-tile
        // kernels (plain or compacted).  TCA_MFMA_MIN_DENSITY (tuning only)
        // overrides the routing threshold.
        const char* md = std::getenv("TCA_MFMA_MIN_DENSITY");
        const MfmaShape* shape = &mfma_shape(flags);
        const double min_density = md ? std::atof(md) : kMfmaMinDensity;
        // Short K (<= 640): every row on the short-K kernel (mfma_short_kernel.hpp).
        p->mfma_short = short_route(M, K, nnz, N, dtype, flags);
        if (!p->mfma_short)
            plan_mfma(rowptr, colidx, M, N, dtype, (flags & TCA_PLAN_FORCE_MFMA) != 0, (flags & TCA_PLAN_NO_MFMA) != 0,
                      min_density, *shape, &p->mfma);
        p->mfma_dense = (flags & (TCA_PLAN_MFMA_DENSE | TCA_PLAN_MFMA_COMPACT)) != 0;
        if ((flags & (TCA_PLAN_MFMA_DENSE | TCA_PLAN_MFMA_PAIR)) == 0 && !p->mfma.windows.empty() &&
            static_cast<double>(p->mfma.cond_cols) >= kNaturalCover * static_cast<double>(p->mfma.windows.size()) * K &&
            p->mfma.windows.size() * static_cast<size_t>((K + 31) / 32) * kDnATileBytes <= kDenseMaxBytes) {
            // Default kernel choice: windows that cover most of K run on the dense
            // tiles in natural column order, compacted when every step fits
            // (measured on MI355X, config 1: 32.4 us per SpMM against 34.5 us for
            // the plain dense tiles and
            // 34.5 us per SpMM against 36.8 us for the paired kernel).
            p->mfma_dense = true;
            p->mfma_compact_want = true;
        }
        if (flags & TCA_PLAN_MFMA_COMPACT) p->mfma_compact_want = true;
        if (p->mfma_dense && (p->mfma.eoff.size() - 1) * static_cast<size_t>(kDnATileBytes) > kDenseMaxBytes) {
            // Dense windows past the budget: the paired kernel, which keeps only the entries.
            p->mfma_dense = false;
            shape = &kMfmaPairShape;
            plan_mfma(rowptr, colidx, M, N, dtype, (flags & TCA_PLAN_FORCE_MFMA) != 0, (flags & TCA_PLAN_NO_MFMA) != 0,
                      min_density, *shape, &p->mfma);
        }
        p->mfma_pair = !p->mfma_dense;
        p->mfma_col_blocks = (N + shape->tile_cols - 1) / shape->tile_cols;
        {
            int32_t most = 0;
            for (size_t i = 0; i + 1 < p->mfma.eoff.size(); i++) most = std::max(most, p->mfma.eoff[i + 1] - p->mfma.eoff[i]);
            p->mfma_groups = most <= 4 * kPairGroup ? 4 : 8;
        }
        // Row panels with B staged in LDS for the rows outside MFMA windows, then
        // the row kernel for the rest.
        if (!p->mfma_short) plan_panels_routed(rowptr, colidx, M, K, N, dtype, flags, p->mfma.row_mfma, &p->panels);
        else p->panels.row_panel.assign(M, 0);
        std::vector<uint8_t> skip_rows(M, p->mfma_short ? 1 : 0);
        for (int32_t r = 0; r < M && !p->mfma_short; r++)
            skip_rows[r] = (!p->mfma.row_mfma.empty() && p->mfma.row_mfma[r]) || p->panels.row_panel[r];
        plan_rows(rowptr, M, N, static_cast<int32_t>(dtype_size(dtype)), skip_rows, default_slices(K, N, dtype),
                  &p->rows);
        order_row_tasks(colidx, &p->rows);
        p->ntasks = static_cast<int32_t>(p->rows.tasks.size());
        const size_t n_seg_rows =
            p->rows.longrows.empty() ? 0 : static_cast<size_t>(p->rows.longrows.back().y + p->rows.longrows.back().z);
        // One partial-row array and one segment-sum table for both kernels: the
        // panels' segments follow the row kernel's.
        {
            const int32_t off = static_cast<int32_t>(n_seg_rows);
            for (Int4& u : p->panels.units)
                if (u.w >= 0) u.w += off;
            for (Int4 lr : p->panels.longrows) {
                lr.y += off;
                p->rows.longrows.push_back(lr);
            }
        }
        const size_t n_seg_total = n_seg_rows + static_cast<size_t>(p->panels.n_segments);
        p->n_units = static_cast<int32_t>(p->panels.units.size());
        p->n_ptiles = p->panels.n_tiles();
        p->n_plongrows = static_cast<int32_t>(p->panels.longrows.size());
        p->n_longrows = static_cast<int32_t>(p->rows.longrows.size());
        p->n_seg_total = n_seg_total;
        p->n_perm = static_cast<int32_t>(p->rows.perm.size());
        const auto t1 = std::chrono::steady_clock::now();

        auto bail = [&](int s) { return s; };  // `hold` frees the plan
        if ((st = dev_upload(&p->d_rowptr, rowptr, static_cast<size_t>(M) + 1))) return bail(st);
        if (p->mfma_short && (st = setup_short(p, rowptr, colidx))) return bail(st);
        if ((st = dev_upload(&p->d_colidx, colidx, static_cast<size_t>(nnz)))) return bail(st);
        if ((st = dev_upload(&p->d_tasks, p->rows.tasks.data(), p->rows.tasks.size()))) return bail(st);
        if ((st = dev_upload(&p->d_torder, p->rows.order.data(), p->rows.order.size()))) return bail(st);
        p->n_torder = static_cast<int32_t>(p->rows.order.size());
        if ((st = dev_upload(&p->d_perm, p->rows.perm.data(), p->rows.perm.size()))) return bail(st);
        if ((st = dev_upload(&p->d_longrows, p->rows.longrows.data(), p->rows.longrows.size()))) return bail(st);
        if (!(flags & TCA_PLAN_NO_SCRATCH) && (st = dev_upload(&p->d_partials, nullptr, n_seg_total * N))) return bail(st);
        if (p->n_units > 0) {
            const PanelPlan& pp = p->panels;
            if ((st = dev_upload(&p->d_units, pp.units.data(), pp.units.size()))) return bail(st);
            if ((st = dev_upload(&p->d_porder, pp.order.data(), pp.order.size()))) return bail(st);
            p->n_pblocks = static_cast<int32_t>(pp.order.size());
            if ((st = dev_upload(&p->d_panel_units, pp.panel_units.data(), pp.panel_units.size()))) return bail(st);
            if ((st = dev_upload(&p->d_pwin, pp.win.data(), pp.win.size()))) return bail(st);
            if ((st = dev_upload(&p->d_prows, pp.rows.data(), pp.rows.size()))) return bail(st);
            {
                // staged rows as byte offsets into B (B < 4 GiB, checked above)
                std::vector<int32_t> boff(pp.cols.size());
                const uint32_t rb = static_cast<uint32_t>(N) * static_cast<uint32_t>(dtype_size(dtype));
                for (size_t j = 0; j < boff.size(); j++) boff[j] = static_cast<int32_t>(static_cast<uint32_t>(pp.cols[j]) * rb);
                if ((st = dev_upload(&p->d_pcols, boff.data(), boff.size()))) return bail(st);
            }
            if ((st = dev_upload(&p->d_pcnt, pp.cnt.data(), pp.cnt.size() / 4))) return bail(st);
            if ((st = dev_upload(&p->d_ppos, pp.pos.data(), pp.pos.size()))) return bail(st);
            p->n_pos_bytes = pp.pos.size();
            if ((st = dev_upload(&p->d_ustart, pp.ustart.data(), pp.ustart.size()))) return bail(st);
            // the kernel needs only the arrays on the device
            p->panels.cols.clear(); p->panels.cols.shrink_to_fit();
            p->panels.width.clear(); p->panels.width.shrink_to_fit();
            p->panels.cnt.clear(); p->panels.cnt.shrink_to_fit();
            p->panels.pos.clear(); p->panels.pos.shrink_to_fit();
            p->panels.ustart.clear(); p->panels.ustart.shrink_to_fit();
        }
        if ((st = dev_upload(&p->d_windows, p->mfma.windows.data(), p->mfma.windows.size()))) return bail(st);
        if (!p->mfma.windows.empty()) {
            // Device forms: B row byte offsets (padding 0xffffffff; paired kernel:
            // each step's 32 offsets permuted, word 4 r + k = column r + 8 k) and
            // the step entry ranges.
            std::vector<uint32_t> uoff(p->mfma.ucols.size());
            for (size_t i = 0; i < uoff.size(); i++) {
                const size_t src = p->mfma_pair ? (i & ~size_t(31)) + ((i & 31) >> 2) + 8 * (i & 3) : i;
                uoff[i] = p->mfma.ucols[src] < 0 ? kNoEntry
                                                  : static_cast<uint32_t>(p->mfma.ucols[src]) * static_cast<uint32_t>(N) * 2u;
            }
            if ((st = dev_upload(&p->d_ucols, uoff.data(), uoff.size()))) return bail(st);
            p->n_ucols = uoff.size();
            if ((st = dev_upload(&p->d_eoff, p->mfma.eoff.data(), p->mfma.eoff.size()))) return bail(st);
        }
        if (!p->mfma.windows.empty() && p->mfma_dense) {
            // Dense condensed windows: 8 KiB per global step (128 rows x 32
            // condensed columns in fragment order), zero except at the entries,
            // whose values the pack kernel writes each run; 1 KiB of zeros after
            // them (the B source for padding rows).  Entries sorted by position.
            // Windows whose column unions cover most of K (on average >= 85 %) keep
            // their columns in natural order instead: every window spans all of K,
            // step j holds columns 32 j .. 32 j + 31, so the kernel's B rows are
            // contiguous and need no row-offset table.
            const int32_t ksteps = (K + 31) / 32;
            const size_t nwin = p->mfma.windows.size();
            p->mfma_natural = static_cast<double>(p->mfma.cond_cols) >= kNaturalCover * static_cast<double>(nwin) * K &&
                              nwin * static_cast<size_t>(ksteps) * kDnATileBytes <= kDenseMaxBytes;
            std::vector<std::pair<uint32_t, int32_t>> ent;
            ent.reserve(p->mfma.entries.size());
            if (p->mfma_natural) {
                std::vector<Int4> wn(nwin);
                for (size_t w = 0; w < nwin; w++) {
                    const Int4 win = p->mfma.windows[w];
                    wn[w] = {win.x, ksteps, static_cast<int32_t>(w) * ksteps, win.w};
                    const int32_t r1 = std::min(M, win.x + kDmaWinRows);
                    for (int32_t r = win.x; r < r1; r++)
                        for (int32_t j = rowptr[r]; j < rowptr[r + 1]; j++) {
                            const int32_t c = colidx[j];
                            ent.emplace_back(static_cast<uint32_t>(wn[w].z + c / 32) * kDmaATile +
                                                 static_cast<uint32_t>(a_cell(r - win.x, c % 32)),
                                             j);
                        }
                }
                (void)hipFree(p->d_windows);
                p->d_windows = nullptr;
                if ((st = dev_upload(&p->d_windows, wn.data(), wn.size()))) return bail(st);
                p->mfma.cond_cols = static_cast<int64_t>(nwin) * ksteps * 32;
            }
            const size_t nsteps_all = p->mfma_natural ? nwin * static_cast<size_t>(ksteps) : p->mfma.eoff.size() - 1;
            p->adense_halves = nsteps_all * static_cast<size_t>(kDmaATile) + 512;
            for (size_t w = 0, e = 0; w < p->mfma.windows.size() && !p->mfma_natural; w++) {
                const Int4 win = p->mfma.windows[w];
                for (int32_t g = win.z; g < win.z + win.y; g++)
                    for (; e < static_cast<size_t>(p->mfma.eoff[g + 1]); e++) {
                        const uint32_t en = p->mfma.entries[e];
                        const uint32_t pos = static_cast<uint32_t>(g) * kDmaATile +
                                             static_cast<uint32_t>(a_cell(static_cast<int>(en & 127u),
                                                                          static_cast<int>((en >> 7) & 31u)));
                        ent.emplace_back(pos, win.w + static_cast<int32_t>(en >> 12));
                    }
            }
            std::sort(ent.begin(), ent.end());
            if (p->mfma_compact_want) {
                // Compacted steps: the non-empty 16-byte cells of each step in
                // cell order (cell = dense half index / 8 within the step, i.e.
                // row block * 64 + lane), at most kCpCells - 1 per step (the last
                // cell stays zero for the empty lanes); else plain dense tiles.
                std::vector<uint64_t> mask(nsteps_all * 8, 0);
                std::vector<std::pair<uint32_t, int32_t>> cent(ent);
                bool fits = true;
                for (size_t x = 0; x < cent.size() && fits;) {
                    const uint32_t g = cent[x].first / kDmaATile;
                    int32_t rank = -1;
                    uint32_t last = ~0u;
                    for (; x < cent.size() && cent[x].first / kDmaATile == g; x++) {
                        const uint32_t h = cent[x].first % kDmaATile, c = h / 8;
                        if (c != last) {
                            rank++;
                            last = c;
                            mask[static_cast<size_t>(g) * 8 + c / 64] |= uint64_t(1) << (c % 64);
                        }
                        if (rank >= kCpCells - 1) fits = false;
                        cent[x].first = g * static_cast<uint32_t>(kCpCells * 8) + static_cast<uint32_t>(rank) * 8u + h % 8;
                    }
                }
                if (fits) {
                    ent.swap(cent);
                    p->mfma_compact = true;
                    p->adense_halves = nsteps_all * static_cast<size_t>(kCpCells * 8) + 512;
                    if (const char* lb = std::getenv("TCA_COMPACT_LB")) p->mfma_compact_lb = std::atoi(lb) == 4 ? 4 : 3;
                    if ((st = dev_upload(&p->d_amask, mask.data(), mask.size()))) return bail(st);
                }
            }
            std::vector<int32_t> dsrc(ent.size());
            std::vector<uint32_t> dpos(ent.size());
            for (size_t x = 0; x < ent.size(); x++) {
                dpos[x] = ent[x].first;
                dsrc[x] = ent[x].second;
            }
            p->n_dn = static_cast<int32_t>(ent.size());
            if ((st = dev_upload(&p->d_dn_src, dsrc.data(), dsrc.size()))) return bail(st);
            if ((st = dev_upload(&p->d_dn_pos, dpos.data(), dpos.size()))) return bail(st);
            if ((st = dev_upload(&p->d_adense, nullptr, p->adense_halves))) return bail(st);
            if (hipMemset(p->d_adense, 0, p->adense_halves * 2) != hipSuccess)
                return bail(fail(TCA_ERR_HIP, "hipMemset of the dense tiles failed"));
        } else if (!p->mfma.windows.empty()) {
            // Packed entries of the paired kernel: step g's block at ebase[g],
            // whole chunks of 256 words (at least one), entries placed by
            // pair_entry_word, unused words the dummy cell of the lane that loads
            // them, with value 0; 16 zero bytes (padding B source) after the blocks.
            const size_t nsteps_all = p->mfma.eoff.size() - 1;
            std::vector<int> ebase(nsteps_all + 1);
            std::vector<i32x2v> emeta(nsteps_all);
            ebase[0] = 0;
            for (size_t g = 0; g < nsteps_all; g++) {
                const int cnt = p->mfma.eoff[g + 1] - p->mfma.eoff[g];
                const int chunks = std::max(1, (cnt + kPairChunk - 1) / kPairChunk);
                ebase[g + 1] = ebase[g] + chunks * kPairChunk;
                emeta[g] = i32x2v{ebase[g], std::max(1, (cnt + kPairGroup - 1) / kPairGroup)};
            }
            const size_t nwords = static_cast<size_t>(ebase.back());
            const size_t npacked = nwords + 4;
            p->mfma_zeros_at = nwords;
            // pack kernel inputs, per word it writes (all words before the
            // zeros): the nonzero's CSR index and the cell
            std::vector<int> src(nwords, -1);
            std::vector<uint16_t> cell(nwords, 0xffffu);
            std::vector<uint32_t> packed(npacked, kNoEntry);
            std::fill(packed.end() - 4, packed.end(), 0u);
            for (size_t w = 0; w < p->mfma.windows.size(); w++) {
                const Int4 win = p->mfma.windows[w];
                for (int32_t j = 0; j < win.y; j++)
                    for (int32_t x = ebase[win.z + j]; x < ebase[win.z + j + 1]; x++) {
                        packed[x] = pair_cell_addr(j % kPairSteps, kDmaATile + ((x - ebase[win.z + j]) % kPairChunk) / 4);
                        cell[x] = static_cast<uint16_t>(packed[x]);
                    }
            }
            const int row_mask = 127, k_shift = 7, idx_shift = 12;
            for (size_t w = 0, e = 0; w < p->mfma.windows.size(); w++) {
                const Int4 win = p->mfma.windows[w];
                for (int32_t g = win.z; g < win.z + win.y; g++)
                    for (; e < static_cast<size_t>(p->mfma.eoff[g + 1]); e++) {
                        const uint32_t en = p->mfma.entries[e];
                        const int acell = a_cell(static_cast<int>(en & row_mask), static_cast<int>((en >> k_shift) & 31u));
                        const size_t x = static_cast<size_t>(ebase[g] + pair_entry_word(static_cast<int>(e - p->mfma.eoff[g])));
                        src[x] = win.w + static_cast<int>(en >> idx_shift);
                        cell[x] = static_cast<uint16_t>(pair_cell_addr((g - win.z) % kPairSteps, acell));
                    }
            }
            p->n_pk_words = static_cast<int32_t>(nwords);
            p->n_packed = npacked;
            if ((st = dev_upload(&p->d_pk_src, src.data(), nwords))) return bail(st);
            if ((st = dev_upload(&p->d_pk_cell, cell.data(), nwords))) return bail(st);
            if ((st = dev_upload(&p->d_packed, packed.data(), npacked))) return bail(st);
            if ((st = dev_upload(&p->d_emeta, emeta.data(), emeta.size()))) return bail(st);
        }
        if (hipDeviceSynchronize() != hipSuccess) return bail(fail(TCA_ERR_HIP, "hipDeviceSynchronize failed"));

        fill_info(p);
        setup_side_stream(p);
        p->info.plan_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
        *plan = hold.release();
        return TCA_OK;
    });
}

// Row panels planned on the GPU (device_panel_planner.hpp), in two phases
// around the row kernel's plan: phase_a picks the panels and their rows (the
// row kernel then plans the other rows), phase_b writes the plan's panel
// arrays once the row kernel's segments are known (the panels' partial rows
// follow them, as in tca_spmm_plan_create).  The decisions that need all
// panels at once -- which candidates are taken, the exclusive sums over
// panels, the XCD launch order -- run on the host over per-panel arrays,
// with the host planner's own rules.
struct DevPanelPlanner {
    hipStream_t s = nullptr;
    int *lenv = nullptr, *lenpre = nullptr, *ucols = nullptr, *upos = nullptr, *ucount = nullptr, *pnnz = nullptr;
    int *take_q = nullptr, *ubase = nullptr, *tbase = nullptr, *tile0 = nullptr, *m = nullptr, *cuts = nullptr;
    int *ntiles = nullptr, *tile_of = nullptr, *tn = nullptr, *ucut = nullptr, *nunits = nullptr;
    int4* poff = nullptr;
    int64_t *ulo = nullptr, *uhi = nullptr;
    uint8_t* in_panel = nullptr;
    void* tmp = nullptr;
    const int* rows_s = nullptr;  // the panels' row order (phase_b: a copy kept past the second sort)
    std::vector<int> h_take, h_nt, h_nu, h_rows_in;
    std::vector<uint8_t> h_win;  // [taken panel]: panel_window
    int n_nz = 0, n_take = 0, n_panel_rows = 0, n_plongrows = 0;
    int64_t n_tiles = 0, n_units = 0, n_segments = 0, nnz = 0, staged = 0, unit_nnz = 0;
    int E = 0, P = 0;

    ~DevPanelPlanner() {
        (void)hipStreamSynchronize(s);
        for (void* q : {(void*)lenv, (void*)lenpre, (void*)ucols, (void*)upos, (void*)ucount, (void*)pnnz, (void*)take_q,
                        (void*)ubase, (void*)tbase, (void*)tile0, (void*)m, (void*)cuts, (void*)ntiles, (void*)tile_of,
                        (void*)tn, (void*)ucut, (void*)nunits, (void*)poff, (void*)ulo, (void*)uhi, (void*)in_panel, tmp})
            (void)hipFree(q);
    }

    DppPanelArgs args(const tca_spmm_plan* p) const {
        DppPanelArgs a{};
        a.rowptr = p->d_rowptr;
        a.rows = rows_s;
        a.lenpre = lenpre;
        a.ucols = ucols;
        a.upos = upos;
        a.ucount = ucount;
        a.take_q = take_q;
        a.ubase = ubase;
        a.tbase = tbase;
        a.tile0 = tile0;
        a.n_nz = n_nz;
        a.P = P;
        a.n_take = n_take;
        a.row_bytes = static_cast<uint32_t>(p->N) * static_cast<uint32_t>(dtype_size(p->dtype));
        a.m = m;
        a.cuts = cuts;
        a.ntiles = ntiles;
        a.tile_of = tile_of;
        a.tn = tn;
        a.cntb = reinterpret_cast<uint8_t*>(p->d_pcnt);
        a.boff = reinterpret_cast<uint32_t*>(p->d_pcols);
        a.pos = p->d_ppos;
        a.ucut = ucut;
        a.nunits = nunits;
        a.poff = poff;
        a.prows = p->d_prows;
        a.units = p->d_units;
        a.ustart = p->d_ustart;
        a.panel_units = p->d_panel_units;
        a.longrows = p->d_longrows;
        a.ulo = ulo;
        a.uhi = uhi;
        return a;
    }

    // keys_s / order: the longest-first order (keys = length + 1, 0 for
    // rows of MFMA windows); n_nz_rows: rows with nonzeros outside windows.
    // On return n_take > 0 when panels are taken, in_panel flags their rows,
    // and the plan's tile arrays (staged rows, counts, positions) are written.
    int phase_a(tca_spmm_plan* p, const uint32_t* keys_s, const int* order, int n_nz_rows) {
        PanelRoute route;
        const int32_t es = static_cast<int32_t>(dtype_size(p->dtype));
        E = panel_elems(p->N, es);
        if (!panel_route(p->K, p->N, p->dtype, p->flags, &route) || E == 0 || p->M == 0 || n_nz_rows == 0) return TCA_OK;
        // (the union kernel's column chunks end below c0 + 2^19: K leaves room for them in an int)
        if (p->K > INT_MAX - 32 * kDppChunkWords) return fail(TCA_ERR_UNSUPPORTED, "K too large for panels planned on the GPU");
        P = panel_tile_cols(16 * E * es);
        n_nz = n_nz_rows;
        rows_s = order;
        const int n_cand = (n_nz + kDppR - 1) / kDppR;
        int st;
        if ((st = dev_upload(&lenv, nullptr, static_cast<size_t>(n_nz) + 1)) ||
            (st = dev_upload(&lenpre, nullptr, static_cast<size_t>(n_nz) + 1)) ||
            (st = dev_upload(&upos, nullptr, static_cast<size_t>(p->nnz))) ||
            (st = dev_upload(&ucount, nullptr, n_cand)) || (st = dev_upload(&pnnz, nullptr, n_cand)))
            return st;
        const dim3 blk(256);
        auto grid_for = [](int64_t n) { return dim3(static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 65536))); };
        hipLaunchKernelGGL(dpp_len_kernel, grid_for(n_nz), blk, 0, s, keys_s, n_nz, lenv);
        if (hipMemsetAsync(lenv + n_nz, 0, sizeof(int), s) != hipSuccess) return fail(TCA_ERR_HIP, "hipMemsetAsync failed");
        size_t tmp_bytes = 0;
        int total = 0;
        if (rocprim::exclusive_scan(nullptr, tmp_bytes, lenv, lenpre, 0, static_cast<size_t>(n_nz) + 1,
                                    rocprim::plus<int>(), s) != hipSuccess ||
            dev_malloc(&tmp, std::max<size_t>(tmp_bytes, 4)) != hipSuccess ||
            rocprim::exclusive_scan(tmp, tmp_bytes, lenv, lenpre, 0, static_cast<size_t>(n_nz) + 1, rocprim::plus<int>(),
                                    s) != hipSuccess ||
            hipMemcpyAsync(&total, lenpre + n_nz, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess)
            return fail(TCA_ERR_HIP, "panel length scan failed");
        if ((st = dev_upload(&ucols, nullptr, std::max(total, 1)))) return st;
        DppUnionArgs ua;
        ua.rowptr = p->d_rowptr;
        ua.colidx = p->d_colidx;
        ua.rows = rows_s;
        ua.lenpre = lenpre;
        ua.n_nz = n_nz;
        ua.ucols = ucols;
        ua.upos = upos;
        ua.ucount = ucount;
        ua.pnnz = pnnz;
        hipLaunchKernelGGL(dpp_union_kernel, dim3(n_cand), dim3(kDppThreads), 0, s, ua);
        std::vector<int> h_ucount(n_cand), h_pnnz(n_cand);
        if (hipMemcpyAsync(h_ucount.data(), ucount, sizeof(int) * n_cand, hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipMemcpyAsync(h_pnnz.data(), pnnz, sizeof(int) * n_cand, hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess)
            return fail(TCA_ERR_HIP, "panel unions failed");
        // which candidates are taken: plan_panels' rule
        int64_t tot = 0;
        for (int q = 0; q < n_cand; q++) {
            const bool take = h_ucount[q] > 0 &&
                              (route.force || static_cast<double>(h_pnnz[q]) >= route.min_reuse * h_ucount[q]);
            if (!take) continue;
            h_take.push_back(q);
            tot += h_pnnz[q];
        }
        if (tot == 0 || (!route.force && tot < route.min_nnz)) {
            h_take.clear();
            return TCA_OK;
        }
        n_take = static_cast<int>(h_take.size());
        unit_nnz = panel_unit_nnz(route.unit_nnz, tot);
        std::vector<int> h_ubase(n_take), h_tbase(n_take);
        int64_t usum = 0, tsum = 0;
        for (int t = 0; t < n_take; t++) {
            const int q = h_take[t];
            h_ubase[t] = static_cast<int>(usum);
            h_tbase[t] = static_cast<int>(tsum);
            usum += h_ucount[q];
            tsum += static_cast<int64_t>(h_ucount[q]) + 1;
            h_rows_in.push_back(std::min(kDppR, n_nz - q * kDppR));
            n_panel_rows += h_rows_in.back();
            nnz += h_pnnz[q];
            staged += h_ucount[q];
            h_win.push_back(panel_window(h_pnnz[q], h_ucount[q]) ? 1 : 0);
        }
        if (tsum >= (int64_t(1) << 31)) return fail(TCA_ERR_UNSUPPORTED, "panel tile scratch past 2^31 entries");
        if ((st = dev_upload(&take_q, h_take.data(), n_take)) || (st = dev_upload(&ubase, h_ubase.data(), n_take)) ||
            (st = dev_upload(&tbase, h_tbase.data(), n_take)) || (st = dev_upload(&ntiles, nullptr, n_take)) ||
            (st = dev_upload(&nunits, nullptr, n_take)) || (st = dev_upload(&m, nullptr, static_cast<size_t>(usum))) ||
            (st = dev_upload(&tile_of, nullptr, static_cast<size_t>(usum))) ||
            (st = dev_upload(&cuts, nullptr, static_cast<size_t>(tsum))) ||
            (st = dev_upload(&tn, nullptr, static_cast<size_t>(tsum))) ||
            (st = dev_upload(&ucut, nullptr, static_cast<size_t>(tsum))) ||
            (st = dev_upload(&in_panel, nullptr, static_cast<size_t>(p->M))))
            return st;
        if (hipMemsetAsync(in_panel, 0, static_cast<size_t>(p->M), s) != hipSuccess ||
            hipMemsetAsync(m, 0x7f, sizeof(int) * static_cast<size_t>(usum), s) != hipSuccess ||
            hipMemsetAsync(tn, 0, sizeof(int) * static_cast<size_t>(tsum), s) != hipSuccess)
            return fail(TCA_ERR_HIP, "hipMemsetAsync failed");
        hipLaunchKernelGGL(dpp_mark_kernel, dim3(n_take), blk, 0, s, rows_s, n_nz, take_q, n_take, in_panel);
        // tile cuts: m, then suffix minimum and walk
        DppPanelArgs a = args(p);
        const dim3 rgrid(static_cast<unsigned>(n_take) * (kDppR / 4));  // one wavefront per panel row
        hipLaunchKernelGGL(dpp_m_kernel, rgrid, blk, 0, s, a);
        hipLaunchKernelGGL(dpp_walk_kernel, dim3(n_take), dim3(1024), 0, s, a);
        h_nt.resize(n_take);
        if (hipMemcpyAsync(h_nt.data(), ntiles, sizeof(int) * n_take, hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess)
            return fail(TCA_ERR_HIP, "panel tile cuts failed");
        std::vector<int> h_tile0(n_take);
        for (int t = 0; t < n_take; t++) {
            h_tile0[t] = static_cast<int>(n_tiles);
            n_tiles += h_nt[t];
        }
        if (n_tiles * P >= (int64_t(1) << 31)) return fail(TCA_ERR_UNSUPPORTED, "panel plan past 2^31 entries");
        p->n_pos_bytes = (static_cast<size_t>(p->nnz) + 3) & ~size_t(3);
        if ((st = dev_upload(&tile0, h_tile0.data(), n_take)) ||
            (st = dev_upload(&p->d_pcols, nullptr, static_cast<size_t>(n_tiles) * P)) ||
            (st = dev_upload(&p->d_pcnt, nullptr, static_cast<size_t>(n_tiles) * kDppCntDwords)) ||
            (st = dev_upload(&p->d_ppos, nullptr, p->n_pos_bytes)))
            return st;
        if (hipMemsetAsync(p->d_ppos, 0, p->n_pos_bytes, s) != hipSuccess ||
            hipMemsetAsync(p->d_pcnt, 0, sizeof(uint32_t) * static_cast<size_t>(n_tiles) * kDppCntDwords, s) != hipSuccess)
            return fail(TCA_ERR_HIP, "hipMemsetAsync failed");
        a = args(p);
        hipLaunchKernelGGL(dpp_tile_fill_kernel, dim3(static_cast<unsigned>(n_tiles)), blk, 0, s, a);
        hipLaunchKernelGGL(dpp_runs_kernel<false>, rgrid, blk, 0, s, a);
        const int64_t nme = n_tiles * kPanelWaves * kPanelRpg;
        hipLaunchKernelGGL(dpp_cnt_max_kernel, dim3(static_cast<unsigned>((nme + 255) / 256)), blk, 0, s,
                           reinterpret_cast<uint8_t*>(p->d_pcnt), n_tiles);
        hipLaunchKernelGGL(dpp_units_kernel, dim3((n_take + 3) / 4), blk, 0, s, take_q, n_take, pnnz, tbase, ntiles, tn,
                           unit_nnz, ucut, nunits);
        h_nu.resize(n_take);
        if (hipMemcpyAsync(h_nu.data(), nunits, sizeof(int) * n_take, hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess)
            return fail(TCA_ERR_HIP, "panel tiles failed");
        for (int t = 0; t < n_take; t++) {
            n_units += h_nu[t];
            if (h_nu[t] > 1) {
                n_plongrows += h_rows_in[t];
                n_segments += static_cast<int64_t>(kDppR) * h_nu[t];
            }
        }
        if (n_units * kDppR >= (int64_t(1) << 31)) return fail(TCA_ERR_UNSUPPORTED, "panel plan past 2^31 entries");
        return TCA_OK;
    }

    // seg_off: the row kernel's segments (the panels' follow them);
    // lr_off: its long rows (the panels' follow them in p->d_longrows).
    // order: the panels' row order (a copy that outlived the second sort).
    int phase_b(tca_spmm_plan* p, const int* order, int64_t seg_off, int lr_off) {
        if (n_take == 0) return TCA_OK;
        rows_s = order;
        std::vector<int4> h_poff(n_take);
        int64_t t0 = 0, unit0 = 0, seg = seg_off, lr = lr_off;
        for (int t = 0; t < n_take; t++) {
            h_poff[t] = make_int4(static_cast<int>(t0), static_cast<int>(unit0), h_nu[t] > 1 ? static_cast<int>(seg) : -1,
                                  static_cast<int>(lr));
            t0 += h_nt[t];
            unit0 += h_nu[t];
            if (h_nu[t] > 1) {
                seg += static_cast<int64_t>(kDppR) * h_nu[t];
                lr += h_rows_in[t];
            }
        }
        int st;
        if ((st = dev_upload(&poff, h_poff.data(), n_take)) ||
            (st = dev_upload(&p->d_prows, nullptr, static_cast<size_t>(n_take) * kDppR)) ||
            (st = dev_upload(&p->d_units, nullptr, static_cast<size_t>(n_units))) ||
            (st = dev_upload(&p->d_ustart, nullptr, static_cast<size_t>(n_units) * kDppR)) ||
            (st = dev_upload(&p->d_panel_units, nullptr, n_take)) ||
            (st = dev_upload(&p->d_pwin, h_win.data(), h_win.size())) ||
            (st = dev_upload(&ulo, nullptr, static_cast<size_t>(n_units))) ||
            (st = dev_upload(&uhi, nullptr, static_cast<size_t>(n_units))))
            return st;
        const DppPanelArgs a = args(p);
        hipLaunchKernelGGL(dpp_emit_units_kernel, dim3(n_take), dim3(256), 0, s, a);
        hipLaunchKernelGGL(dpp_runs_kernel<true>, dim3(static_cast<unsigned>(n_take) * (kDppR / 4)), dim3(256), 0, s, a);
        // XCD launch order of the units (host rule, from each unit's column span)
        std::vector<Int4> units(n_units);
        std::vector<int64_t> lo(n_units), hi(n_units);
        if (hipMemcpyAsync(units.data(), p->d_units, sizeof(int4) * n_units, hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipMemcpyAsync(lo.data(), ulo, sizeof(int64_t) * n_units, hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipMemcpyAsync(hi.data(), uhi, sizeof(int64_t) * n_units, hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess)
            return fail(TCA_ERR_HIP, "panel emission failed");
        std::vector<int32_t> uorder;
        const int32_t chunks = p->N / (16 * E);
        order_unit_spans(p->K, chunks, units, lo, hi, &uorder);
        if ((st = dev_upload(&p->d_porder, uorder.data(), uorder.size()))) return st;
        PanelPlan& pp = p->panels;
        pp.waves = kPanelWaves;
        pp.rpg = kPanelRpg;
        pp.R = kDppR;
        pp.P = P;
        pp.elems = E;
        pp.chunks = chunks;
        pp.n_panels = n_take;
        pp.nnz = nnz;
        pp.staged = staged;
        pp.win = h_win;
        pp.n_rows = n_panel_rows;
        pp.n_segments = n_segments;
        p->n_units = static_cast<int32_t>(n_units);
        p->n_pblocks = static_cast<int32_t>(uorder.size());
        p->n_ptiles = n_tiles;
        p->n_plongrows = n_plongrows;
        return TCA_OK;
    }
};

int tca_spmm_plan_create_device(const int32_t* d_rowptr, const int32_t* d_colidx, int32_t M, int32_t K, int32_t nnz,
                                int32_t N, int32_t dtype, uint32_t flags, void* stream, tca_spmm_plan** plan) {
    return api_guard("tca_spmm_plan_create_device", [&]() -> int {
        if (!plan) return fail(TCA_ERR_INVALID, "plan is NULL");
        *plan = nullptr;
        if (M < 0 || K < 1 || N < 1 || nnz < 0) return fail(TCA_ERR_INVALID, "bad shape M=%d K=%d N=%d nnz=%d", M, K, N, nnz);
        if (!dtype_ok(dtype)) return fail(TCA_ERR_INVALID, "unknown dtype %d", dtype);
        if (!d_rowptr || (nnz > 0 && !d_colidx)) return fail(TCA_ERR_INVALID, "NULL device pointer");
        if (flags & ~TCA_PLAN_KNOWN_FLAGS) return fail(TCA_ERR_INVALID, "unknown plan flags 0x%x", flags & ~TCA_PLAN_KNOWN_FLAGS);
        if (flags & TCA_PLAN_MFMA_PAIR)
            return fail(TCA_ERR_UNSUPPORTED,
                        "device planning builds row-kernel and dense-tile plans (TCA_PLAN_MFMA_PAIR needs the host planner)");
        const uint64_t b_bytes = static_cast<uint64_t>(K) * static_cast<uint64_t>(N) * dtype_size(dtype);
        if (b_bytes >= 0xfffffff0ull || static_cast<uint64_t>(nnz) * 4 >= 0xfffffff0ull)
            return fail(TCA_ERR_UNSUPPORTED, "B (%llu bytes) or the nonzeros exceed the 4 GiB buffer range",
                        (unsigned long long)b_bytes);
        const auto t0 = std::chrono::steady_clock::now();
        tca_spmm_plan* p = new (std::nothrow) tca_spmm_plan();
        if (!p) return fail(TCA_ERR_ALLOC, "plan allocation failed");
        PlanHolder hold{p};
        p->M = M;
        p->K = K;
        p->N = N;
        p->nnz = nnz;
        p->dtype = dtype;
        p->flags = flags;
        p->device_planned = true;
        p->mfma.row_mfma.clear();
        if (hipGetDevice(&p->device) != hipSuccess) return fail(TCA_ERR_HIP, "no HIP device");
        plan_row_params(nnz, N, static_cast<int32_t>(dtype_size(dtype)), default_slices(K, N, dtype), &p->rows);
        const int group = multi_group_rows(64 >> p->rows.log_lanes);  // rows per multi task
        hipStream_t s = static_cast<hipStream_t>(stream);

        // temporaries of the planning, freed on every exit
        uint32_t *keys = nullptr, *keys_s = nullptr, *bm = nullptr, *ekeys = nullptr, *ekeys_s = nullptr;
        int *rows = nullptr, *rows_s = nullptr, *cnt = nullptr, *nseg = nullptr, *segoff = nullptr;
        int *wordpre = nullptr, *scnt = nullptr, *wstat = nullptr, *wmap = nullptr, *wgbase = nullptr, *evals = nullptr,
            *evals_s = nullptr;
        uint8_t* start = nullptr;
        void* tmp = nullptr;
        uint32_t *skey = nullptr, *skey_s = nullptr;  // segment launch order
        int *sidx = nullptr, *sidx_s = nullptr;
        int* dpp_rows = nullptr;  // the panels' row order (phase_b reads it after the second sort)
        auto bail = [&](int st) {
            (void)hipStreamSynchronize(s);
            for (void* q : {(void*)keys, (void*)keys_s, (void*)rows, (void*)rows_s, (void*)cnt, (void*)nseg, (void*)segoff,
                            (void*)start, tmp, (void*)bm, (void*)ekeys, (void*)ekeys_s, (void*)wordpre, (void*)scnt,
                            (void*)wstat, (void*)wmap, (void*)wgbase, (void*)evals, (void*)evals_s, (void*)skey,
                            (void*)skey_s, (void*)sidx, (void*)sidx_s, (void*)dpp_rows})
                (void)hipFree(q);
            return st;  // on failure `hold` frees the plan
        };
        int st;
        // The plan owns its copy of the structure (row kernel and SDDMM read it).
        if ((st = dev_upload(&p->d_rowptr, nullptr, static_cast<size_t>(M) + 1))) return bail(st);
        if ((st = dev_upload(&p->d_colidx, nullptr, static_cast<size_t>(nnz)))) return bail(st);
        if (hipMemcpyAsync(p->d_rowptr, d_rowptr, sizeof(int) * (static_cast<size_t>(M) + 1), hipMemcpyDeviceToDevice, s) !=
                hipSuccess ||
            (nnz > 0 && hipMemcpyAsync(p->d_colidx, d_colidx, sizeof(int) * static_cast<size_t>(nnz),
                                       hipMemcpyDeviceToDevice, s) != hipSuccess))
            return bail(fail(TCA_ERR_HIP, "structure copy failed"));
        // CSR checks
        if ((st = dev_upload(&cnt, nullptr, 4))) return bail(st);  // [0..2] bounds, [3] error bits
        if ((st = dev_upload(&start, nullptr, static_cast<size_t>(nnz) + 1))) return bail(st);
        if (hipMemsetAsync(cnt, 0, 4 * sizeof(int), s) != hipSuccess ||
            hipMemsetAsync(start, 0, static_cast<size_t>(nnz) + 1, s) != hipSuccess)
            return bail(fail(TCA_ERR_HIP, "hipMemsetAsync failed"));
        const dim3 blk(256);
        auto grid_for = [](int64_t n) { return dim3(static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 65536))); };
        if (M > 0) {
            hipLaunchKernelGGL(dp_check_rows_kernel, grid_for(M), blk, 0, s, p->d_rowptr, M, nnz, start, cnt + 3);
            if (nnz > 0) hipLaunchKernelGGL(dp_check_cols_kernel, grid_for(nnz), blk, 0, s, p->d_colidx, nnz, K, start, cnt + 3);
        }
        int h_cnt[4] = {0, 0, 0, 0};
        // the columns index the window bitmaps below: validate first
        if (hipMemcpyAsync(h_cnt, cnt, sizeof h_cnt, hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess)
            return bail(fail(TCA_ERR_HIP, "CSR checks failed"));
        if (h_cnt[3] & 1) return bail(fail(TCA_ERR_INVALID, "CSR row offsets are not 0 .. nnz non-decreasing"));
        if (h_cnt[3] & 2) return bail(fail(TCA_ERR_INVALID, "CSR columns out of range or not strictly ascending in a row"));
        if (short_route(M, K, nnz, N, dtype, flags)) {
            // short K: every row on the short-K kernel, which needs only the structure
            p->mfma_short = true;
            p->short_nwin = (M + kShRows - 1) / kShRows;
            p->short_col_blocks = (N + kDmaTileCols - 1) / kDmaTileCols;
            p->short_steps = (K + kStepK - 1) / kStepK;
            const uint32_t z[4] = {0, 0, 0, 0};
            if ((st = dev_upload(&p->d_zeros, z, 4)) ||
                (st = dev_upload(&p->d_soff, nullptr, static_cast<size_t>(nnz))) ||
                (st = dev_upload(&p->d_wstart, nullptr, static_cast<size_t>(p->short_nwin) + 1)))
                return bail(st);
            hipLaunchKernelGGL(dp_short_kernel, dim3((M + 256) / 256), dim3(256), 0, s, p->d_rowptr, p->d_colidx, M,
                               p->d_soff, p->d_wstart);
            p->short_wstart.resize(static_cast<size_t>(p->short_nwin) + 1);
            if (hipMemcpyAsync(p->short_wstart.data(), p->d_wstart, sizeof(int32_t) * p->short_wstart.size(),
                               hipMemcpyDeviceToHost, s) != hipSuccess ||
                hipStreamSynchronize(s) != hipSuccess)
                return bail(fail(TCA_ERR_HIP, "short-K planning failed"));
            st = bail(TCA_OK);  // frees the temporaries only
            fill_info(p);
            p->info.plan_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
            *plan = hold.release();
            return TCA_OK;
        }

        // MFMA windows: statistics on the GPU, the host planner's routing, then
        // dense tiles (natural column order when the windows cover most of K,
        // else condensed) built on the GPU.  Needs fp16 / bf16, N % 8 == 0 and
        // window bitmaps of at most kDevBitmapWords words.
        int32_t rows_mfma = 0;
        {
            constexpr size_t kDevBitmapWords = size_t(1) << 25;  // 128 MiB per table
            const int nw = (M + kDmaWinRows - 1) / kDmaWinRows, kw = (K + 31) / 32;
            if ((flags & TCA_PLAN_NO_MFMA) == 0 && dtype != TCA_F32 && N % 8 == 0 && M > 0 && nnz > 0 &&
                static_cast<size_t>(nw) * kw <= kDevBitmapWords) {
                const size_t nb = static_cast<size_t>(nw) * kw;
                if ((st = dev_upload(&bm, nullptr, nb)) || (st = dev_upload(&wordpre, nullptr, nb)) ||
                    (st = dev_upload(&scnt, nullptr, nb)) || (st = dev_upload(&wstat, nullptr, 3 * static_cast<size_t>(nw) + 1)))
                    return bail(st);
                if (hipMemsetAsync(bm, 0, nb * 4, s) != hipSuccess || hipMemsetAsync(scnt, 0, nb * 4, s) != hipSuccess)
                    return bail(fail(TCA_ERR_HIP, "hipMemsetAsync failed"));
                int* const ucount = wstat;
                int* const maxper = wstat + nw;
                int* const wrow = wstat + 2 * nw;  // nw + 1
                const dim3 rgrid(static_cast<unsigned>(std::min<int64_t>((static_cast<int64_t>(M) + 3) / 4, 65536)));
                hipLaunchKernelGGL(dm_bitmap_kernel, rgrid, blk, 0, s, p->d_rowptr, p->d_colidx, M, kw, bm);
                hipLaunchKernelGGL(dm_union_kernel, dim3(nw), blk, 0, s, p->d_rowptr, M, nw, kw, bm, wordpre, ucount, wrow);
                hipLaunchKernelGGL(dm_stepcount_kernel, rgrid, blk, 0, s, p->d_rowptr, p->d_colidx, M, kw, bm, wordpre,
                                   scnt);
                hipLaunchKernelGGL(dm_stepmax_kernel, dim3(nw), blk, 0, s, scnt, kw, ucount, maxper);
                std::vector<int> h(3 * static_cast<size_t>(nw) + 1);
                if (hipMemcpyAsync(h.data(), wstat, sizeof(int) * h.size(), hipMemcpyDeviceToHost, s) != hipSuccess ||
                    hipStreamSynchronize(s) != hipSuccess)
                    return bail(fail(TCA_ERR_HIP, "window statistics failed"));
                std::vector<WinStat> ws(nw);
                for (int w = 0; w < nw; w++)
                    ws[w] = {static_cast<int64_t>(h[2 * nw + w + 1]) - h[2 * nw + w], h[w], h[nw + w]};
                const char* md = std::getenv("TCA_MFMA_MIN_DENSITY");
                std::vector<uint8_t> take;
                route_windows(ws, M, nnz, N, (flags & TCA_PLAN_FORCE_MFMA) != 0, md ? std::atof(md) : kMfmaMinDensity,
                              mfma_shape(flags), &take);
                // the host planner's choice between natural and condensed dense tiles
                std::vector<int> h_wmap(nw, -1), h_base;
                int64_t cond_cols = 0, steps_all = 0, nz_take = 0;
                int n_take = 0;
                for (int w = 0; w < nw; w++) {
                    if (!take[w]) continue;
                    h_wmap[w] = n_take++;
                    const int steps = (h[w] + 31) / 32;
                    h_base.push_back(static_cast<int>(steps_all));
                    steps_all += steps;
                    cond_cols += static_cast<int64_t>(steps) * 32;
                    nz_take += ws[w].nz;
                    rows_mfma += std::min(M, (w + 1) * kDmaWinRows) - w * kDmaWinRows;
                }
                const int32_t ksteps = (K + 31) / 32;
                const bool natural = n_take > 0 &&
                                     static_cast<double>(cond_cols) >= kNaturalCover * static_cast<double>(n_take) * K &&
                                     static_cast<size_t>(n_take) * ksteps * kDnATileBytes <= kDenseMaxBytes;
                if (natural) {
                    for (int t = 0; t < n_take; t++) h_base[t] = t * ksteps;
                    steps_all = static_cast<int64_t>(n_take) * ksteps;
                    cond_cols = steps_all * 32;
                }
                if (n_take > 0 && static_cast<size_t>(steps_all) * kDnATileBytes > kDenseMaxBytes) {
                    n_take = 0;  // past the dense-tile budget: every row on the row kernel
                    rows_mfma = 0;
                }
                if (n_take > 0) {
                    std::vector<Int4> win;
                    for (int w = 0; w < nw; w++)
                        if (h_wmap[w] >= 0) {
                            const int t = h_wmap[w];
                            win.push_back({w * kDmaWinRows, natural ? ksteps : (h[w] + 31) / 32, h_base[t], h[2 * nw + w]});
                        }
                    if ((st = dev_upload(&wmap, h_wmap.data(), h_wmap.size())) ||
                        (st = dev_upload(&wgbase, h_base.data(), h_base.size())) ||
                        (st = dev_upload(&p->d_windows, win.data(), win.size())) ||
                        (st = dev_upload(&ekeys, nullptr, nnz)) || (st = dev_upload(&ekeys_s, nullptr, nnz)) ||
                        (st = dev_upload(&evals, nullptr, nnz)) || (st = dev_upload(&evals_s, nullptr, nnz)))
                        return bail(st);
                    DmEntryArgs ea;
                    ea.rowptr = p->d_rowptr;
                    ea.colidx = p->d_colidx;
                    ea.bm = bm;
                    ea.wordpre = wordpre;
                    ea.wmap = wmap;
                    ea.wgbase = wgbase;
                    ea.keys = ekeys;
                    ea.vals = evals;
                    ea.M = M;
                    ea.kw = kw;
                    ea.natural = natural ? 1 : 0;
                    hipLaunchKernelGGL(dm_entries_kernel, rgrid, blk, 0, s, ea);
                    // ascending positions: the routed nonzeros first, in the host planner's order
                    size_t tmp_bytes = 0;
                    if (rocprim::radix_sort_pairs(nullptr, tmp_bytes, ekeys, ekeys_s, evals, evals_s,
                                                  static_cast<size_t>(nnz), 0, 32, s) != hipSuccess ||
                        dev_malloc(reinterpret_cast<void**>(&tmp), tmp_bytes) != hipSuccess ||
                        rocprim::radix_sort_pairs(tmp, tmp_bytes, ekeys, ekeys_s, evals, evals_s, static_cast<size_t>(nnz),
                                                  0, 32, s) != hipSuccess)
                        return bail(fail(TCA_ERR_HIP, "entry sort failed"));
                    (void)hipFree(tmp);
                    tmp = nullptr;
                    p->n_dn = static_cast<int32_t>(nz_take);
                    if ((st = dev_upload(&p->d_dn_pos, nullptr, static_cast<size_t>(nz_take))) ||
                        (st = dev_upload(&p->d_dn_src, nullptr, static_cast<size_t>(nz_take))))
                        return bail(st);
                    if (hipMemcpyAsync(p->d_dn_pos, ekeys_s, 4 * static_cast<size_t>(nz_take), hipMemcpyDeviceToDevice, s) !=
                            hipSuccess ||
                        hipMemcpyAsync(p->d_dn_src, evals_s, 4 * static_cast<size_t>(nz_take), hipMemcpyDeviceToDevice, s) !=
                            hipSuccess)
                        return bail(fail(TCA_ERR_HIP, "entry copy failed"));
                    if (!natural) {
                        if ((st = dev_upload(&p->d_ucols, nullptr, static_cast<size_t>(steps_all) * 32))) return bail(st);
                        p->n_ucols = static_cast<size_t>(steps_all) * 32;
                        if (hipMemsetAsync(p->d_ucols, 0xff, 4 * static_cast<size_t>(steps_all) * 32, s) != hipSuccess)
                            return bail(fail(TCA_ERR_HIP, "hipMemsetAsync failed"));
                        hipLaunchKernelGGL(dm_ucols_kernel, grid_for(static_cast<int64_t>(nw) * kw), blk, 0, s, nw, kw, bm,
                                           wordpre, wmap, wgbase, N, p->d_ucols);
                    }
                    p->adense_halves = static_cast<size_t>(steps_all) * kDmaATile + 512;
                    // Compacted steps under the host planner's rule: by default for
                    // natural-order tiles (unless TCA_PLAN_MFMA_DENSE), always with
                    // TCA_PLAN_MFMA_COMPACT, when every step fits.
                    const bool compact_want = (flags & TCA_PLAN_MFMA_COMPACT) != 0 ||
                                              (natural && (flags & TCA_PLAN_MFMA_DENSE) == 0);
                    if (compact_want && nz_take > 0) {
                        const size_t nmask = static_cast<size_t>(steps_all) * 8;
                        if ((st = dev_upload(&p->d_amask, nullptr, nmask))) return bail(st);
                        if (hipMemsetAsync(p->d_amask, 0, nmask * 8, s) != hipSuccess ||
                            hipMemsetAsync(cnt + 3, 0, sizeof(int), s) != hipSuccess)
                            return bail(fail(TCA_ERR_HIP, "hipMemsetAsync failed"));
                        auto* mk = reinterpret_cast<unsigned long long*>(p->d_amask);
                        hipLaunchKernelGGL(dm_cmask_kernel, grid_for(nz_take), blk, 0, s, p->d_dn_pos,
                                           static_cast<int>(nz_take), mk);
                        hipLaunchKernelGGL(dm_cfit_kernel, grid_for(steps_all), blk, 0, s, mk, steps_all, kCpCells,
                                           cnt + 3);
                        int over = 0;
                        if (hipMemcpyAsync(&over, cnt + 3, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess ||
                            hipStreamSynchronize(s) != hipSuccess)
                            return bail(fail(TCA_ERR_HIP, "compaction check failed"));
                        if (over == 0) {
                            hipLaunchKernelGGL(dm_cpos_kernel, grid_for(nz_take), blk, 0, s, p->d_dn_pos,
                                               static_cast<int>(nz_take), mk, kCpCells);
                            p->mfma_compact = true;
                            p->adense_halves = static_cast<size_t>(steps_all) * (kCpCells * 8) + 512;
                            if (const char* lb = std::getenv("TCA_COMPACT_LB")) p->mfma_compact_lb = std::atoi(lb) == 4 ? 4 : 3;
                        } else {
                            (void)hipFree(p->d_amask);
                            p->d_amask = nullptr;
                        }
                    }
                    if ((st = dev_upload(&p->d_adense, nullptr, p->adense_halves))) return bail(st);
                    if (hipMemsetAsync(p->d_adense, 0, p->adense_halves * 2, s) != hipSuccess)
                        return bail(fail(TCA_ERR_HIP, "hipMemsetAsync of the dense tiles failed"));
                    p->mfma.win_rows = kDmaWinRows;
                    p->mfma.windows = std::move(win);
                    p->mfma.rows = rows_mfma;
                    p->mfma.nnz = nz_take;
                    p->mfma.cond_cols = cond_cols;
                    p->mfma_dense = true;
                    p->mfma_natural = natural;
                    p->mfma_col_blocks = (N + kDmaTileCols - 1) / kDmaTileCols;
                }
            }
        }
        if (p->mfma.windows.empty()) p->flags |= TCA_PLAN_NO_MFMA;
        int Mp = M - rows_mfma;  // rows outside MFMA windows: panels and the row kernel

        // rows longest first (stable descending radix sort of length + 1; rows of
        // the routed windows have key 0 and sort last); with panels, those rows
        // leave too (key 0) and the order is sorted again for the row kernel
        DevPanelPlanner dpp;
        dpp.s = s;
        size_t sort_bytes = 0;
        auto sort_rows = [&](const uint8_t* in_panel) -> int {
            hipLaunchKernelGGL(dp_lengths_kernel, grid_for(M), blk, 0, s, p->d_rowptr, M,
                               p->mfma.windows.empty() ? nullptr : wmap, in_panel, keys, rows);
            size_t tmp_bytes = 0;
            if (rocprim::radix_sort_pairs_desc(nullptr, tmp_bytes, keys, keys_s, rows, rows_s, static_cast<size_t>(M), 0, 32,
                                               s) != hipSuccess)
                return fail(TCA_ERR_HIP, "radix sort sizing failed");
            if (tmp_bytes > sort_bytes) {
                (void)hipStreamSynchronize(s);
                (void)hipFree(tmp);
                tmp = nullptr;
                if (dev_malloc(reinterpret_cast<void**>(&tmp), tmp_bytes) != hipSuccess)
                    return fail(TCA_ERR_ALLOC, "radix sort workspace");
                sort_bytes = tmp_bytes;
            }
            if (rocprim::radix_sort_pairs_desc(tmp, tmp_bytes, keys, keys_s, rows, rows_s, static_cast<size_t>(M), 0, 32, s) !=
                hipSuccess)
                return fail(TCA_ERR_HIP, "radix sort failed");
            if (Mp > 0)
                hipLaunchKernelGGL(dp_bounds_kernel, dim3(1), dim3(64), 0, s, keys_s, Mp, p->rows.wide_len, p->rows.row_len,
                                   p->rows.multi_max, cnt);
            if (hipMemcpyAsync(h_cnt, cnt, sizeof h_cnt, hipMemcpyDeviceToHost, s) != hipSuccess ||
                hipStreamSynchronize(s) != hipSuccess)
                return fail(TCA_ERR_HIP, "planning kernels failed");
            // (cnt[3] held flags before the bounds kernel wrote it; with Mp == 0 it did not run)
            if (Mp == 0) h_cnt[0] = h_cnt[1] = h_cnt[2] = h_cnt[3] = 0;
            return TCA_OK;
        };
        if (M > 0) {
            if ((st = dev_upload(&keys, nullptr, M)) || (st = dev_upload(&keys_s, nullptr, M)) ||
                (st = dev_upload(&rows, nullptr, M)) || (st = dev_upload(&rows_s, nullptr, M)))
                return bail(st);
            if ((st = sort_rows(nullptr))) return bail(st);
            // Row panels from the first h_cnt[3] rows of the order (rows with
            // nonzeros outside MFMA windows), as plan_panels takes them.
            if (!p->mfma_short && (st = dpp.phase_a(p, keys_s, rows_s, h_cnt[3]))) return bail(st);
            if (dpp.n_take > 0) {
                Mp -= dpp.n_panel_rows;
                // the panels keep their order (rows_s) until phase_b: sort a copy
                int* prow_order = nullptr;
                if ((st = dev_upload(&prow_order, nullptr, static_cast<size_t>(dpp.n_nz)))) return bail(st);
                if (hipMemcpyAsync(prow_order, rows_s, sizeof(int) * static_cast<size_t>(dpp.n_nz), hipMemcpyDeviceToDevice,
                                   s) != hipSuccess) {
                    (void)hipFree(prow_order);
                    return bail(fail(TCA_ERR_HIP, "panel order copy failed"));
                }
                dpp_rows = prow_order;
                if ((st = sort_rows(dpp.in_panel))) return bail(st);
            }
        } else if (hipStreamSynchronize(s) != hipSuccess) {
            return bail(fail(TCA_ERR_HIP, "planning kernels failed"));
        }
        const int n_long = h_cnt[0], end_wide = h_cnt[1], end_row = h_cnt[2], end_nz = h_cnt[3];
        // segment slots of the long rows: exclusive sum of their segment counts
        int seg_total = 0;
        if (n_long > 0) {
            if ((st = dev_upload(&nseg, nullptr, static_cast<size_t>(n_long) + 1)) ||
                (st = dev_upload(&segoff, nullptr, static_cast<size_t>(n_long) + 1)))
                return bail(st);
            if (hipMemsetAsync(nseg, 0, sizeof(int) * (static_cast<size_t>(n_long) + 1), s) != hipSuccess)
                return bail(fail(TCA_ERR_HIP, "hipMemsetAsync failed"));
            hipLaunchKernelGGL(dp_nseg_kernel, grid_for(n_long), blk, 0, s, keys_s, n_long, p->rows.seg_len, nseg);
            (void)hipFree(tmp);
            tmp = nullptr;
            size_t tmp_bytes = 0;
            if (rocprim::exclusive_scan(nullptr, tmp_bytes, nseg, segoff, 0, static_cast<size_t>(n_long) + 1,
                                        rocprim::plus<int>(), s) != hipSuccess ||
                dev_malloc(reinterpret_cast<void**>(&tmp), tmp_bytes) != hipSuccess ||
                rocprim::exclusive_scan(tmp, tmp_bytes, nseg, segoff, 0, static_cast<size_t>(n_long) + 1, rocprim::plus<int>(),
                                        s) != hipSuccess ||
                hipMemcpyAsync(&seg_total, segoff + n_long, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess ||
                hipStreamSynchronize(s) != hipSuccess)
                return bail(fail(TCA_ERR_HIP, "segment scan failed"));
        }
        const int n_wide = end_wide - n_long, n_row = end_row - end_wide, n_short = Mp - end_row;
        const int n_multi = (end_nz - end_row + group - 1) / group + (Mp - end_nz + kZeroRows - 1) / kZeroRows;
        p->ntasks = 4 * n_wide + seg_total + n_row + n_multi;
        p->rows.n_wide = 4 * n_wide;
        p->rows.n_seg = seg_total;
        p->rows.n_rowtasks = n_row;
        p->rows.n_multi = n_multi;
        p->n_longrows = n_long + dpp.n_plongrows;  // the panels' long rows follow the row kernel's
        p->n_seg_total = static_cast<size_t>(seg_total) + static_cast<size_t>(dpp.n_segments);
        p->n_perm = n_short;
        if ((st = dev_upload(&p->d_tasks, nullptr, p->ntasks)) || (st = dev_upload(&p->d_perm, nullptr, n_short)) ||
            (st = dev_upload(&p->d_longrows, nullptr, p->n_longrows)) ||
            (!(flags & TCA_PLAN_NO_SCRATCH) && (st = dev_upload(&p->d_partials, nullptr, p->n_seg_total * N))))
            return bail(st);
        if (Mp > 0) {
            DpEmitArgs ea;
            ea.rowptr = p->d_rowptr;
            ea.len = keys_s;
            ea.rows = rows_s;
            ea.segoff = segoff;
            ea.tasks = p->d_tasks;
            ea.perm = p->d_perm;
            ea.longrows = p->d_longrows;
            ea.M = Mp;
            ea.n_long = n_long;
            ea.end_wide = end_wide;
            ea.end_row = end_row;
            ea.end_nz = end_nz;
            ea.group = group;
            ea.seg_total = seg_total;
            hipLaunchKernelGGL(dp_emit_kernel, grid_for(Mp), blk, 0, s, ea);
        }
        if (row_order_on(p->rows)) {
            // the host planner's segment launch order (order_row_tasks):
            // segments stably sorted by the column of their middle nonzero,
            // cut into kXcds queues of equal count, queue x on XCD x
            const int nw = p->rows.n_wide, ns = seg_total, rest = p->ntasks - nw - ns;
            const int b0 = nw / kRowOrderSlots;
            int b_end = b0;
            for (int x = 0; x < kXcds; x++) {
                const int len = static_cast<int>(static_cast<int64_t>(ns) * (x + 1) / kXcds - static_cast<int64_t>(ns) * x / kXcds);
                if (len > 0)
                    b_end = std::max(b_end, b0 + ((x - b0) % kXcds + kXcds) % kXcds +
                                                kXcds * ((len + kRowOrderSlots - 1) / kRowOrderSlots - 1) + 1);
            }
            const int n_slots = (kRowOrderSlots * b_end + rest + kRowOrderSlots - 1) / kRowOrderSlots * kRowOrderSlots;
            if ((st = dev_upload(&skey, nullptr, ns)) || (st = dev_upload(&skey_s, nullptr, ns)) ||
                (st = dev_upload(&sidx, nullptr, ns)) || (st = dev_upload(&sidx_s, nullptr, ns)) ||
                (st = dev_upload(&p->d_torder, nullptr, n_slots)))
                return bail(st);
            hipLaunchKernelGGL(dp_segkey_kernel, grid_for(ns), blk, 0, s, p->d_tasks, nw, ns, p->d_colidx, skey, sidx);
            (void)hipFree(tmp);
            tmp = nullptr;
            size_t tmp_bytes = 0;
            if (rocprim::radix_sort_pairs(nullptr, tmp_bytes, skey, skey_s, sidx, sidx_s, static_cast<size_t>(ns), 0, 32, s) !=
                    hipSuccess ||
                dev_malloc(reinterpret_cast<void**>(&tmp), std::max<size_t>(tmp_bytes, 4)) != hipSuccess ||
                rocprim::radix_sort_pairs(tmp, tmp_bytes, skey, skey_s, sidx, sidx_s, static_cast<size_t>(ns), 0, 32, s) !=
                    hipSuccess)
                return bail(fail(TCA_ERR_HIP, "segment order sort failed"));
            hipLaunchKernelGGL(dp_order_fill_kernel, grid_for(n_slots), blk, 0, s, p->d_torder, n_slots, nw, ns, rest, b_end);
            hipLaunchKernelGGL(dp_order_seg_kernel, grid_for(ns), blk, 0, s, sidx_s, ns, b0, p->d_torder);
            p->n_torder = n_slots;
        }
        if ((st = dpp.phase_b(p, dpp_rows, seg_total, n_long))) return bail(st);
        if (hipGetLastError() != hipSuccess || hipStreamSynchronize(s) != hipSuccess)
            return bail(fail(TCA_ERR_HIP, "task emission failed"));
        st = bail(TCA_OK);  // frees the temporaries only
        fill_info(p);
        setup_side_stream(p);
        p->info.plan_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        *plan = hold.release();
        return TCA_OK;
    });
}

int tca_spmm_plan_export_rows(const tca_spmm_plan* p, int32_t* n_tasks, int32_t* n_perm, int32_t* n_long,
                              int32_t* tasks, int32_t* perm, int32_t* longrows) {
    if (!p || !n_tasks || !n_perm || !n_long) return fail(TCA_ERR_INVALID, "tca_spmm_plan_export_rows: bad argument");
    if (tasks) {
        if (*n_tasks < p->ntasks || *n_perm < p->n_perm || *n_long < p->n_longrows || !perm || !longrows)
            return fail(TCA_ERR_INVALID, "tca_spmm_plan_export_rows: output buffers too small");
        if ((p->ntasks && hipMemcpy(tasks, p->d_tasks, sizeof(int4) * p->ntasks, hipMemcpyDeviceToHost) != hipSuccess) ||
            (p->n_perm && hipMemcpy(perm, p->d_perm, sizeof(int) * p->n_perm, hipMemcpyDeviceToHost) != hipSuccess) ||
            (p->n_longrows &&
             hipMemcpy(longrows, p->d_longrows, sizeof(int4) * p->n_longrows, hipMemcpyDeviceToHost) != hipSuccess))
            return fail(TCA_ERR_HIP, "tca_spmm_plan_export_rows: copy failed");
    }
    *n_tasks = p->ntasks;
    *n_perm = p->n_perm;
    *n_long = p->n_longrows;
    return TCA_OK;
}

int tca_spmm_plan_export_order(const tca_spmm_plan* p, int32_t* n_slots, int32_t* order) {
    if (!p || !n_slots) return fail(TCA_ERR_INVALID, "tca_spmm_plan_export_order: bad argument");
    if (order) {
        if (*n_slots < p->n_torder) return fail(TCA_ERR_INVALID, "tca_spmm_plan_export_order: output buffer too small");
        if (p->n_torder && hipMemcpy(order, p->d_torder, sizeof(int) * p->n_torder, hipMemcpyDeviceToHost) != hipSuccess)
            return fail(TCA_ERR_HIP, "tca_spmm_plan_export_order: copy failed");
    }
    *n_slots = p->n_torder;
    return TCA_OK;
}

int tca_spmm_plan_export_tiles(const tca_spmm_plan* p, int32_t* n_windows, int32_t* n_entries, int32_t* n_ucols,
                               int32_t* windows, uint32_t* pos, int32_t* src, uint32_t* ucols) {
    if (!p || !n_windows || !n_entries || !n_ucols) return fail(TCA_ERR_INVALID, "tca_spmm_plan_export_tiles: bad argument");
    const bool dense = p->mfma_dense && !p->mfma.windows.empty();
    const int32_t nw = dense ? static_cast<int32_t>(p->mfma.windows.size()) : 0;
    const int32_t ne = dense ? p->n_dn : 0;
    const int32_t nu = dense && !p->mfma_natural ? static_cast<int32_t>(p->n_ucols) : 0;
    if (windows) {
        if (*n_windows < nw || *n_entries < ne || *n_ucols < nu || !pos || !src || !ucols)
            return fail(TCA_ERR_INVALID, "tca_spmm_plan_export_tiles: output buffers too small");
        if ((nw && hipMemcpy(windows, p->d_windows, sizeof(int4) * nw, hipMemcpyDeviceToHost) != hipSuccess) ||
            (ne && hipMemcpy(pos, p->d_dn_pos, sizeof(uint32_t) * ne, hipMemcpyDeviceToHost) != hipSuccess) ||
            (ne && hipMemcpy(src, p->d_dn_src, sizeof(int32_t) * ne, hipMemcpyDeviceToHost) != hipSuccess) ||
            (nu && hipMemcpy(ucols, p->d_ucols, sizeof(uint32_t) * nu, hipMemcpyDeviceToHost) != hipSuccess))
            return fail(TCA_ERR_HIP, "tca_spmm_plan_export_tiles: copy failed");
    }
    *n_windows = nw;
    *n_entries = ne;
    *n_ucols = nu;
    return TCA_OK;
}

int tca_spmm_plan_export_panels(const tca_spmm_plan* p, int64_t* sizes, int32_t* rows, uint32_t* boff, uint32_t* cnt,
                                uint8_t* pos, int32_t* units, int32_t* order, int32_t* panel_units, int32_t* ustart,
                                int32_t* longrows, uint8_t* window) {
    if (!p || !sizes) return fail(TCA_ERR_INVALID, "tca_spmm_plan_export_panels: bad argument");
    const bool on = p->n_units > 0;
    const int64_t R = on ? p->panels.R : 0, P = on ? p->panels.P : 0;
    const int64_t want[8] = {on ? p->panels.n_panels : 0, on ? p->n_ptiles : 0, on ? p->n_units : 0,
                             on ? p->n_pblocks : 0, on ? p->n_plongrows : 0, R, P,
                             on ? static_cast<int64_t>(p->n_pos_bytes) : 0};
    if (rows) {
        for (int k = 0; k < 5; k++)
            if (sizes[k] < want[k]) return fail(TCA_ERR_INVALID, "tca_spmm_plan_export_panels: output buffers too small");
        if (sizes[7] < want[7] || !boff || !cnt || !pos || !units || !order || !panel_units || !ustart || !longrows ||
            !window)
            return fail(TCA_ERR_INVALID, "tca_spmm_plan_export_panels: output buffers too small");
        auto get = [](void* dst, const void* src, size_t bytes) {
            return bytes == 0 || hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost) == hipSuccess;
        };
        const size_t lr0 = static_cast<size_t>(p->n_longrows - p->n_plongrows);
        if (!get(rows, p->d_prows, sizeof(int32_t) * want[0] * R) || !get(boff, p->d_pcols, sizeof(uint32_t) * want[1] * P) ||
            !get(cnt, p->d_pcnt, sizeof(uint32_t) * want[1] * kPanelWaves * kPanelCntRows) ||
            !get(pos, p->d_ppos, want[7]) || !get(units, p->d_units, sizeof(int4) * want[2]) ||
            !get(order, p->d_porder, sizeof(int32_t) * want[3]) ||
            !get(panel_units, p->d_panel_units, sizeof(int32_t) * want[0]) ||
            !get(ustart, p->d_ustart, sizeof(int32_t) * want[2] * R) ||
            !get(longrows, p->d_longrows + lr0, sizeof(int4) * want[4]) || !get(window, p->d_pwin, want[0]))
            return fail(TCA_ERR_HIP, "tca_spmm_plan_export_panels: copy failed");
    }
    for (int k = 0; k < 8; k++) sizes[k] = want[k];
    return TCA_OK;
}

int tca_spmm_plan_info(const tca_spmm_plan* plan, tca_plan_info* info) {
    if (!plan || !info) return fail(TCA_ERR_INVALID, "NULL argument");
    *info = plan->info;
    return TCA_OK;
}

int tca_spmm_plan_destroy(tca_spmm_plan* plan) {
    if (!plan) return TCA_OK;
    free_plan_device(plan);
    delete plan;
    return TCA_OK;
}

// Operand checks of tca_spmm_run (p non-NULL, M > 0).
static int check_run_operands(const tca_spmm_plan* p, const void* d_val, const void* d_B, const float* d_C) {
    if ((p->nnz > 0 && (!d_val || !d_B)) || !d_C) return fail(TCA_ERR_INVALID, "NULL device pointer");
    const size_t vb = static_cast<size_t>(p->rows.elems_per_lane) * dtype_size(p->dtype);
    if (reinterpret_cast<uintptr_t>(d_B) % vb != 0)
        return fail(TCA_ERR_INVALID, "B must be aligned to %zu bytes", vb);
    if (reinterpret_cast<uintptr_t>(d_C) % 16 != 0) return fail(TCA_ERR_INVALID, "C must be aligned to 16 bytes");
    if (reinterpret_cast<uintptr_t>(d_val) % dtype_size(p->dtype) != 0)
        return fail(TCA_ERR_INVALID, "values misaligned");
    if (p->n_seg_total > 0 && !p->d_partials)
        return fail(TCA_ERR_INVALID, "plan was created with TCA_PLAN_NO_SCRATCH: run it with tca_spmm_run_static");
    return TCA_OK;
}

int tca_spmm_run(const tca_spmm_plan* p, const void* d_val, const void* d_B, float* d_C, void* stream) {
    if (!p) return fail(TCA_ERR_INVALID, "plan is NULL");
    if (p->M == 0) return TCA_OK;
    int st = check_run_operands(p, d_val, d_B, d_C);
    if (st) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    st = run_phases(p, d_val, d_B, d_C, p->d_partials, s);
    if (st) return st;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TCA_ERR_HIP, "kernel launch: %s", hipGetErrorString(e));
    return TCA_OK;
}

int tca_spmm_run_static(const tca_spmm_plan* p, const void* d_val, const void* d_B, float* d_C, void* stream) {
    if (!p) return fail(TCA_ERR_INVALID, "plan is NULL");
    if (p->M == 0) return TCA_OK;
    if ((p->nnz > 0 && (!d_val || !d_B)) || !d_C) return fail(TCA_ERR_INVALID, "NULL device pointer");
    const size_t vb = static_cast<size_t>(p->rows.elems_per_lane) * dtype_size(p->dtype);
    if (reinterpret_cast<uintptr_t>(d_B) % vb != 0)
        return fail(TCA_ERR_INVALID, "B must be aligned to %zu bytes", vb);
    if (reinterpret_cast<uintptr_t>(d_C) % 16 != 0) return fail(TCA_ERR_INVALID, "C must be aligned to 16 bytes");
    if (reinterpret_cast<uintptr_t>(d_val) % dtype_size(p->dtype) != 0)
        return fail(TCA_ERR_INVALID, "values misaligned");
    const size_t need = p->n_seg_total * static_cast<size_t>(p->N) * sizeof(float);
    if (need > kStaticScratchBytes)
        return fail(TCA_ERR_UNSUPPORTED,
                    "tca_spmm_run_static: the plan's partial rows need %zu bytes, the static scratch holds %zu",
                    need, static_cast<size_t>(kStaticScratchBytes));
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return fail(TCA_ERR_HIP, "hipGetDevice failed");
    if (dev != p->device)
        return fail(TCA_ERR_INVALID, "tca_spmm_run_static: current device %d, plan built on device %d", dev, p->device);
    float* w = nullptr;
    if (need > 0) {
        const int st = static_scratch(dev, &w);
        if (st) return st;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int st = run_phases(p, d_val, d_B, d_C, w, s);
    if (st) return st;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TCA_ERR_HIP, "kernel launch: %s", hipGetErrorString(e));
    return TCA_OK;
}

int tca_spmm_time(const tca_spmm_plan* p, const void* d_val, const void* d_B, float* d_C, void* stream,
                  int32_t warmup, int32_t iters, float* avg_ms) {
    if (!p || !avg_ms || iters < 1 || warmup < 0) return fail(TCA_ERR_INVALID, "tca_spmm_time: bad argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (int i = 0; i < warmup; i++) {
        int st = tca_spmm_run(p, d_val, d_B, d_C, stream);
        if (st) return st;
    }
    hipEvent_t e0, e1;
    TCA_HIP_TRY(hipEventCreate(&e0));
    TCA_HIP_TRY(hipEventCreate(&e1));
    TCA_HIP_TRY(hipEventRecord(e0, s));
    for (int i = 0; i < iters; i++) {
        int st = tca_spmm_run(p, d_val, d_B, d_C, stream);
        if (st) {
            (void)hipEventDestroy(e0);
            (void)hipEventDestroy(e1);
            return st;
        }
    }
    TCA_HIP_TRY(hipEventRecord(e1, s));
    TCA_HIP_TRY(hipEventSynchronize(e1));
    float ms = 0.f;
    TCA_HIP_TRY(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *avg_ms = ms / static_cast<float>(iters);
    return TCA_OK;
}

int tca_sddmm(const tca_spmm_plan* p, const float* d_G, const void* d_B, float* d_out, void* stream) {
    if (!p) return fail(TCA_ERR_INVALID, "plan is NULL");
    if (p->M == 0 || p->nnz == 0) return TCA_OK;
    if (!d_G || !d_B || !d_out) return fail(TCA_ERR_INVALID, "NULL device pointer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid((p->M + kSddmmRowsPerBlock - 1) / kSddmmRowsPerBlock), block(64 * kSddmmRowsPerBlock);
    switch (p->dtype) {
        case TCA_F16:
            hipLaunchKernelGGL(sddmm_kernel<_Float16>, grid, block, 0, s, p->d_rowptr, p->d_colidx, p->M, p->N, d_G,
                               static_cast<const _Float16*>(d_B), d_out);
            break;
        case TCA_BF16:
            hipLaunchKernelGGL(sddmm_kernel<bf16_t>, grid, block, 0, s, p->d_rowptr, p->d_colidx, p->M, p->N, d_G,
                               static_cast<const bf16_t*>(d_B), d_out);
            break;
        default:
            hipLaunchKernelGGL(sddmm_kernel<float>, grid, block, 0, s, p->d_rowptr, p->d_colidx, p->M, p->N, d_G,
                               static_cast<const float*>(d_B), d_out);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TCA_ERR_HIP, "kernel launch: %s", hipGetErrorString(e));
    return TCA_OK;
}

int tca_bell_spmm(const int32_t* d_colind, const void* d_values, int32_t M, int32_t K, int32_t N, int32_t bsize,
                  int32_t ell_blocks, int32_t dtype, const void* d_B, float* d_C, void* stream) {
    if (M < 0 || K < 1 || N < 1 || ell_blocks < 0)
        return fail(TCA_ERR_INVALID, "tca_bell_spmm: bad shape M=%d K=%d N=%d ell_blocks=%d", M, K, N, ell_blocks);
    if (bsize != 32 && bsize != 64) return fail(TCA_ERR_UNSUPPORTED, "tca_bell_spmm: block size %d (32 or 64)", bsize);
    if (dtype != TCA_F16 && dtype != TCA_BF16) return fail(TCA_ERR_UNSUPPORTED, "tca_bell_spmm: fp16 / bf16 values only");
    if (N % 8 != 0) return fail(TCA_ERR_UNSUPPORTED, "tca_bell_spmm: N %% 8 != 0");
    // B is addressed through 32-bit buffer offsets, rows up to the block-padded K.
    if ((static_cast<uint64_t>(K) + bsize) * static_cast<uint64_t>(N) * 2 >= 0xfffffff0ull)
        return fail(TCA_ERR_UNSUPPORTED, "tca_bell_spmm: B exceeds the 4 GiB buffer range");
    if (M == 0) return TCA_OK;
    if (!d_B || !d_C || (ell_blocks > 0 && (!d_colind || !d_values)))
        return fail(TCA_ERR_INVALID, "tca_bell_spmm: NULL device pointer");
    if (reinterpret_cast<uintptr_t>(d_B) % 16 || reinterpret_cast<uintptr_t>(d_values) % 16 ||
        reinterpret_cast<uintptr_t>(d_C) % 4)
        return fail(TCA_ERR_INVALID, "tca_bell_spmm: B and values must be 16-byte aligned, C 4-byte");
    BellArgs a;
    a.colind = d_colind;
    a.values = d_values;
    a.B = d_B;
    a.C = d_C;
    a.M = M;
    a.N = N;
    a.ell_blocks = ell_blocks;
    a.col_groups = (N + kBellCols - 1) / kBellCols;
    a.B_bytes = static_cast<uint32_t>(static_cast<uint64_t>(K) * N * 2);
    const int64_t brows = (static_cast<int64_t>(M) + bsize - 1) / bsize;
    if (brows * a.col_groups > 0x7fffffff) return fail(TCA_ERR_UNSUPPORTED, "tca_bell_spmm: grid too large");
    const dim3 grid(static_cast<unsigned>(brows * a.col_groups));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool bf = dtype == TCA_BF16;
    if (bsize == 32) {
        if (bf) hipLaunchKernelGGL((bell_mfma_kernel<true, 32>), grid, dim3(kBellThreads), 0, s, a);
        else hipLaunchKernelGGL((bell_mfma_kernel<false, 32>), grid, dim3(kBellThreads), 0, s, a);
    } else {
        if (bf) hipLaunchKernelGGL((bell_mfma_kernel<true, 64>), grid, dim3(kBellThreads), 0, s, a);
        else hipLaunchKernelGGL((bell_mfma_kernel<false, 64>), grid, dim3(kBellThreads), 0, s, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TCA_ERR_HIP, "kernel launch: %s", hipGetErrorString(e));
    return TCA_OK;
}

int tca_spmm_24(const void* d_vals, const uint16_t* d_meta, int32_t M, int32_t K, int32_t N, int32_t dtype,
                const void* d_B, float* d_C, void* stream) {
    if (M < 0 || K < 1 || N < 1) return fail(TCA_ERR_INVALID, "tca_spmm_24: bad shape M=%d K=%d N=%d", M, K, N);
    if (dtype != TCA_F16 && dtype != TCA_BF16) return fail(TCA_ERR_UNSUPPORTED, "tca_spmm_24: fp16 / bf16 values only");
    if (N % 8 != 0) return fail(TCA_ERR_UNSUPPORTED, "tca_spmm_24: N %% 8 != 0");
    if ((static_cast<uint64_t>(K) + 64) * static_cast<uint64_t>(N) * 2 >= 0xfffffff0ull)
        return fail(TCA_ERR_UNSUPPORTED, "tca_spmm_24: B exceeds the 4 GiB buffer range");
    if (M == 0) return TCA_OK;
    if (!d_vals || !d_meta || !d_B || !d_C) return fail(TCA_ERR_INVALID, "tca_spmm_24: NULL device pointer");
    if (reinterpret_cast<uintptr_t>(d_B) % 16 || reinterpret_cast<uintptr_t>(d_vals) % 16 ||
        reinterpret_cast<uintptr_t>(d_meta) % 2 || reinterpret_cast<uintptr_t>(d_C) % 4)
        return fail(TCA_ERR_INVALID, "tca_spmm_24: B and vals must be 16-byte aligned, meta 2-byte, C 4-byte");
    S24Args a;
    a.vals = d_vals;
    a.meta = d_meta;
    a.B = d_B;
    a.C = d_C;
    a.M = M;
    a.N = N;
    a.Kp = (K + 63) / 64 * 64;
    a.col_groups = (N + kS24Cols - 1) / kS24Cols;
    a.B_bytes = static_cast<uint32_t>(static_cast<uint64_t>(K) * N * 2);
    const int64_t groups = (static_cast<int64_t>(M) + kS24Rows - 1) / kS24Rows * a.col_groups;
    if (groups > 0x7fffffff) return fail(TCA_ERR_UNSUPPORTED, "tca_spmm_24: grid too large");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == TCA_BF16)
        hipLaunchKernelGGL(sparse24_kernel<true>, dim3(static_cast<unsigned>(groups)), dim3(kS24Threads), 0, s, a);
    else
        hipLaunchKernelGGL(sparse24_kernel<false>, dim3(static_cast<unsigned>(groups)), dim3(kS24Threads), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TCA_ERR_HIP, "kernel launch: %s", hipGetErrorString(e));
    return TCA_OK;
}

int tca_gather_values(const int32_t* d_perm, int32_t n, const void* d_val, int32_t dtype, float* d_out, void* stream) {
    if (n < 0 || !dtype_ok(dtype)) return fail(TCA_ERR_INVALID, "tca_gather_values: bad argument");
    if (n == 0) return TCA_OK;
    if (!d_perm || !d_val || !d_out) return fail(TCA_ERR_INVALID, "NULL device pointer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid((n + 255) / 256);
    switch (dtype) {
        case TCA_F16:
            hipLaunchKernelGGL(gather_values_kernel<_Float16>, grid, dim3(256), 0, s, d_perm, n,
                               static_cast<const _Float16*>(d_val), d_out);
            break;
        case TCA_BF16:
            hipLaunchKernelGGL(gather_values_kernel<bf16_t>, grid, dim3(256), 0, s, d_perm, n,
                               static_cast<const bf16_t*>(d_val), d_out);
            break;
        default:
            hipLaunchKernelGGL(gather_values_kernel<float>, grid, dim3(256), 0, s, d_perm, n,
                               static_cast<const float*>(d_val), d_out);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TCA_ERR_HIP, "kernel launch: %s", hipGetErrorString(e));
    return TCA_OK;
}

int tca_spmm_time_subset(const tca_spmm_plan* p, const void* d_val, const void* d_B, float* d_C, void* stream,
                         uint32_t phase_mask, int32_t warmup, int32_t iters, float* avg_ms) {
    if (!p || !avg_ms || iters < 1 || warmup < 0 || (phase_mask & ~((1u << TCA_PHASES) - 1u)))
        return fail(TCA_ERR_INVALID, "tca_spmm_time_subset: bad argument");
    *avg_ms = 0.f;
    if (p->M == 0) return TCA_OK;
    int st = check_run_operands(p, d_val, d_B, d_C);
    if (st) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (int i = 0; i < warmup && st == TCA_OK; i++) st = run_phases(p, d_val, d_B, d_C, p->d_partials, s, phase_mask);
    if (st) return st;
    hipEvent_t e0, e1;
    TCA_HIP_TRY(hipEventCreate(&e0));
    if (hipEventCreate(&e1) != hipSuccess) {
        (void)hipEventDestroy(e0);
        return fail(TCA_ERR_HIP, "hipEventCreate failed");
    }
    if (hipEventRecord(e0, s) != hipSuccess) st = fail(TCA_ERR_HIP, "hipEventRecord failed");
    for (int i = 0; i < iters && st == TCA_OK; i++) st = run_phases(p, d_val, d_B, d_C, p->d_partials, s, phase_mask);
    float ms = 0.f;
    if (st == TCA_OK && (hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                         hipEventElapsedTime(&ms, e0, e1) != hipSuccess))
        st = fail(TCA_ERR_HIP, "event timing failed");
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (st) return st;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TCA_ERR_HIP, "kernel launch: %s", hipGetErrorString(e));
    *avg_ms = ms / static_cast<float>(iters);
    return TCA_OK;
}

int tca_spmm_plan_phases(const tca_spmm_plan* p, uint32_t* phase_mask) {
    if (!p || !phase_mask) return fail(TCA_ERR_INVALID, "tca_spmm_plan_phases: bad argument");
    *phase_mask = phases_used(p);
    return TCA_OK;
}

int tca_spmm_time_phases(const tca_spmm_plan* p, const void* d_val, const void* d_B, float* d_C, void* stream,
                         int32_t warmup, int32_t iters, float* phase_ms, int32_t n_phase_ms) {
    if (!p || !phase_ms || n_phase_ms < 1 || iters < 1 || iters > 100000 || warmup < 0)
        return fail(TCA_ERR_INVALID, "tca_spmm_time_phases: bad argument");
    const int n_out = n_phase_ms < TCA_PHASES ? n_phase_ms : TCA_PHASES;
    for (int k = 0; k < n_out; k++) phase_ms[k] = 0.f;
    if (n_phase_ms > TCA_PHASE_RUN) phase_ms[TCA_PHASE_RUN] = 0.f;
    for (int i = 0; i < warmup; i++) {
        int st = tca_spmm_run(p, d_val, d_B, d_C, stream);
        if (st) return st;
    }
    if (p->M == 0) return TCA_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint32_t used = phases_used(p);
    // `iters` whole runs back to back, in run_phases' launch order; each
    // phase's one kernel is dispatched with a start and a stop event of its
    // own (TCA_PHASE_LAUNCH), so nothing is inserted between the kernels and
    // a phase's time is the mean over the runs of its kernel's span.  All
    // runs are queued before the first event is read.
    std::vector<hipEvent_t> ev(static_cast<size_t>(iters) * TCA_PHASES * 2, nullptr);
    int st = TCA_OK;
    for (auto& e : ev)
        if (hipEventCreate(&e) != hipSuccess) {
            e = nullptr;
            st = fail(TCA_ERR_HIP, "hipEventCreate failed");
            break;
        }
    hipEvent_t r0 = nullptr, r1 = nullptr;  // around all the runs
    if (st == TCA_OK && (hipEventCreate(&r0) != hipSuccess || hipEventCreate(&r1) != hipSuccess))
        st = fail(TCA_ERR_HIP, "hipEventCreate failed");
    if (st == TCA_OK && hipEventRecord(r0, s) != hipSuccess) st = fail(TCA_ERR_HIP, "hipEventRecord failed");
    auto arm = [&](int i, int k) {
        g_phase_ev[0] = ev[(static_cast<size_t>(i) * TCA_PHASES + k) * 2];
        g_phase_ev[1] = ev[(static_cast<size_t>(i) * TCA_PHASES + k) * 2 + 1];
    };
    for (int i = 0; i < iters && st == TCA_OK; i++) {
        arm(i, TCA_PHASE_PACK);
        launch_pack(p, d_val, s);
        arm(i, TCA_PHASE_TILES);
        st = launch_mfma(p, d_val, d_B, d_C, s);
        arm(i, TCA_PHASE_PANELS);
        if (st == TCA_OK) st = launch_panels(p, d_val, d_B, d_C, p->d_partials, s);
        arm(i, TCA_PHASE_ROWS);
        if (st == TCA_OK) st = launch_rows(p, d_val, d_B, d_C, p->d_partials, s);
        arm(i, TCA_PHASE_SEGMENTS);
        if (st == TCA_OK) launch_finalize(p, d_C, p->d_partials, s);
        g_phase_ev[0] = g_phase_ev[1] = nullptr;
    }
    g_phase_ev[0] = g_phase_ev[1] = nullptr;
    if (st == TCA_OK && hipEventRecord(r1, s) != hipSuccess) st = fail(TCA_ERR_HIP, "hipEventRecord failed");
    if (st == TCA_OK) {
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) st = fail(TCA_ERR_HIP, "kernel launch: %s", hipGetErrorString(e));
    }
    if (st == TCA_OK && hipStreamSynchronize(s) != hipSuccess) st = fail(TCA_ERR_HIP, "stream synchronisation failed");
    double sum[TCA_PHASES] = {0, 0, 0, 0, 0};
    for (int i = 0; i < iters && st == TCA_OK; i++)
        for (int k = 0; k < TCA_PHASES && st == TCA_OK; k++) {
            if (!(used & (1u << k))) continue;
            float ms = 0.f;
            const size_t at = (static_cast<size_t>(i) * TCA_PHASES + k) * 2;
            if (hipEventElapsedTime(&ms, ev[at], ev[at + 1]) != hipSuccess) st = fail(TCA_ERR_HIP, "event timing failed");
            sum[k] += ms;
        }
    float run_ms = 0.f;
    if (st == TCA_OK && hipEventElapsedTime(&run_ms, r0, r1) != hipSuccess) st = fail(TCA_ERR_HIP, "event timing failed");
    for (auto e : ev)
        if (e) (void)hipEventDestroy(e);
    if (r0) (void)hipEventDestroy(r0);
    if (r1) (void)hipEventDestroy(r1);
    if (st != TCA_OK) return st;
    for (int k = 0; k < n_out; k++) phase_ms[k] = (used & (1u << k)) ? static_cast<float>(sum[k] / iters) : 0.f;
    if (n_phase_ms > TCA_PHASE_RUN) phase_ms[TCA_PHASE_RUN] = run_ms / static_cast<float>(iters);
    return TCA_OK;
}

int tca_spmm_host(const int32_t* rowptr, const int32_t* colidx, const void* val, int32_t M, int32_t K, int32_t nnz,
                  const void* B, float* C, int32_t N, int32_t dtype, int32_t n_iter, int32_t verbose,
                  double* elapsed_ms) {
    return api_guard("tca_spmm_host", [&]() -> int {
        if (!rowptr || (nnz > 0 && (!colidx || !val)) || !B || !C || n_iter < 1)
            return fail(TCA_ERR_INVALID, "tca_spmm_host: bad argument");
        if (!dtype_ok(dtype)) return fail(TCA_ERR_INVALID, "unknown dtype %d", dtype);
        const size_t es = dtype_size(dtype);
        void *dval = nullptr, *dB = nullptr;
        float* dC = nullptr;
        tca_spmm_plan* plan = nullptr;
        int st = TCA_OK;
        auto cleanup = [&](int s) {
            (void)hipFree(dval);
            (void)hipFree(dB);
            (void)hipFree(dC);
            tca_spmm_plan_destroy(plan);
            return s;
        };
        // Device copies of the operands (reference src/our_spmm.cu:503-525; C is
        // not copied in: every row of C is written).
        if (dev_malloc(reinterpret_cast<void**>(&dval), es * std::max(nnz, 1)) != hipSuccess ||
            dev_malloc(reinterpret_cast<void**>(&dB), es * static_cast<size_t>(K) * N) != hipSuccess ||
            dev_malloc(reinterpret_cast<void**>(&dC), sizeof(float) * std::max<size_t>(static_cast<size_t>(M) * N, 1)) !=
                hipSuccess)
            return cleanup(fail(TCA_ERR_ALLOC, "tca_spmm_host: device allocation failed"));
        if ((nnz > 0 && hipMemcpy(dval, val, es * nnz, hipMemcpyHostToDevice) != hipSuccess) ||
            hipMemcpy(dB, B, es * static_cast<size_t>(K) * N, hipMemcpyHostToDevice) != hipSuccess)
            return cleanup(fail(TCA_ERR_HIP, "tca_spmm_host: H2D copy failed"));
        const auto t0 = std::chrono::steady_clock::now();
        st = tca_spmm_plan_create(rowptr, colidx, M, K, nnz, N, dtype, TCA_PLAN_DEFAULT, &plan);
        const auto t1 = std::chrono::steady_clock::now();
        if (st) return cleanup(st);
        if (verbose) {
            // Same two lines as reference our_spmm_balanced (src/our_spmm.cu:549,552),
            // describing this build's plan: the row kernel's grid, block and LDS.
            std::printf("preprocess %fms taken\n", std::chrono::duration<float, std::milli>(t1 - t0).count());
            print_launches(plan);
        }
        float ms = 0.f;
        st = tca_spmm_time(plan, dval, dB, dC, nullptr, 5, n_iter, &ms);
        if (st) return cleanup(st);
        if (hipMemcpy(C, dC, sizeof(float) * static_cast<size_t>(M) * N, hipMemcpyDeviceToHost) != hipSuccess)
            return cleanup(fail(TCA_ERR_HIP, "tca_spmm_host: D2H copy failed"));
        if (elapsed_ms) *elapsed_ms = ms;
        return cleanup(TCA_OK);
    });
}

}  // extern "C"
