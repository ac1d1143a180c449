// planner.hpp -- host-side planning of one SpMM: the wavefront task list of
// the row kernel and the 16-row windows routed to the MFMA tile kernel.
//
// Replaces reference workload_manager (src/our_spmm.cu:353-477), which packs
// warps of 32 lanes into 8-warp thread blocks by row length and gives a long
// row at most N/64 blocks.  Here every task is one 64-lane wavefront, tasks
// are ordered longest first across the whole grid, and rows longer than the
// segment length are split across wavefronts with an ordered two-step sum.
#pragma once

#include <cstdint>
#include <vector>

namespace tca {

// Task kinds of the row kernel (int4 {x, y, z, w}).
enum TaskKind : int32_t {
    kTaskRow = 0,    // x = row, y = nnz begin, z = nnz end: all slots split one row
    kTaskMulti = 1,  // x = offset into perm, y = rows in group (<= slots), z = longest row
    kTaskSeg = 2,    // x = long-row id, y = nnz begin, z = nnz end, w = 2 | (segment << 2)
};

struct Int4 {
    int32_t x, y, z, w;
};

struct RowPlan {
    // lane geometry
    int32_t elems_per_lane = 1;  // B columns per lane per load
    int32_t log_lanes = 6;       // log2(lanes covering one B-row chunk)
    int32_t col_chunks = 1;      // chunks of 64 * elems_per_lane columns
    int32_t seg_len = 0;
    int32_t multi_max = 0;       // rows with length <= multi_max go to multi tasks
    std::vector<Int4> tasks;
    std::vector<int32_t> perm;      // row ids of multi tasks
    std::vector<Int4> longrows;     // {row, first segment, segments, 0}
    int32_t n_multi = 0, n_seg = 0, n_rowtasks = 0;
};

struct WindowPlan {
    int32_t win = 16;
    std::vector<int32_t> windows;   // window ids routed to MFMA
    std::vector<int64_t> uoff;      // per routed window: offset into ucols (n+1 entries)
    std::vector<int32_t> ucols;     // condensed column unions (padded per window)
    std::vector<int16_t> cpos;      // per nnz of routed windows: position inside its union
    std::vector<uint8_t> row_mfma;  // per row: 1 when covered by an MFMA window
    int64_t nnz = 0;
    int64_t cond_cols = 0;
};

// Lane geometry for width N and value size `es` bytes: the widest vector
// (<= 16 bytes) whose element count divides N.
void plan_geometry(int32_t N, int32_t es, RowPlan* p);

// Builds the row-kernel task list for rows with skip[r] == 0 (skip may be
// empty).  Rows are assigned longest first; rows longer than seg_len are split.
void plan_rows(const int32_t* rowptr, int32_t M, int32_t N, int32_t es, const std::vector<uint8_t>& skip,
               RowPlan* p);

// Sorted column union of every window of `win` rows and each nonzero's
// position in it (the indexing exported by tca_condense_windows).
void condense(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t win, std::vector<int64_t>* uoff,
              std::vector<int32_t>* ucols, std::vector<int32_t>* cpos);

}  // namespace tca
