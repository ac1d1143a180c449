// planner.hpp -- host-side planning of one SpMM: the wavefront task list of
// the row kernel and the row windows routed to the MFMA tile kernel.
//
// Replaces reference workload_manager (src/our_spmm.cu:353-477), which packs
// warps of 32 lanes into 8-warp thread blocks by row length and gives a long
// row at most N/64 blocks.  Here every task is one 64-lane wavefront over one
// column chunk of C; chunks are mapped to XCDs so each XCD's L2 holds only
// its slice of B; tasks run longest first; long rows are shared by the four
// wavefronts of a workgroup (LDS sum) or, longer still, split across
// workgroups with an ordered two-kernel sum.
#pragma once

#include <cstdint>
#include <utility>
#include <vector>

#include "../../include/tca_spmm.h"

namespace tca {

constexpr int kXcds = 8;  // XCDs of the MI355X: the hardware deals workgroup b to XCD b % 8
constexpr int64_t kMallBytes = int64_t(256) << 20;  // MI355X Infinity Cache (MALL), shared by the XCDs

// Task kinds of the row kernel (int4 {x, y, z, w}).  Multi tasks hold at most
// multi_group_rows(slots) rows, walked `slots` at a time, except zero tasks
// (z == 0), which hold up to kZeroRows empty rows whose C rows the wavefront
// only clears.
enum TaskKind : int32_t {
    kTaskRow = 0,    // x = row, y = nnz begin, z = nnz end: all slots split one row
    kTaskMulti = 1,  // x = offset into perm, y = rows in group, z = longest row; z == 0: empty rows
    kTaskSeg = 2,    // x = long-row id, y = nnz begin, z = nnz end, w = 2 | (segment slot << 2)
    kTaskWide = 3,   // x = row, y = nnz begin, z = nnz end of this quarter; all 4 waves of a workgroup
};

constexpr int32_t kZeroRows = 64;
// Short rows per multi task: kMultiPasses passes of `slots` rows (one row per
// slot and pass), at most 64.  Measured on MI355X against one pass per task
// (config 3's row phase): 2 passes 0.282 ms, 4 passes 0.279, 1 pass 0.297;
// config 4 191.1 against 192.2 us at 4 passes, 203 us at 8.
constexpr int32_t kMultiPasses = 4;
inline int32_t multi_group_rows(int32_t slots) { return slots * kMultiPasses < 64 ? slots * kMultiPasses : 64; }

struct Int4 {
    int32_t x, y, z, w;
};

struct RowPlan {
    // lane geometry
    int32_t elems_per_lane = 1;  // B columns per lane per load (16-byte vectors when possible)
    int32_t log_lanes = 6;       // log2(G): lanes per slot, G >= chunk_lanes
    int32_t chunk_lanes = 64;    // lanes holding data in one column chunk
    int32_t col_chunks = 1;      // column chunks (grid.x = task groups * col_chunks)
    int32_t row_len = 0;         // rows up to this length: one wavefront
    int32_t wide_len = 0;        // rows up to this length: one workgroup (4 wavefronts)
    int32_t seg_len = 0;         // longer rows: segments of at most this length
    int32_t multi_max = 0;       // rows with length <= multi_max go to multi tasks
    std::vector<Int4> tasks;     // wide groups first (4-aligned), then seg, row, multi
    std::vector<int32_t> perm;   // row ids of multi tasks
    std::vector<Int4> longrows;  // {row, first segment slot, segments, 0}
    std::vector<int32_t> order;  // [wavefront slot]: task it runs, -1 idle; empty = task order
    int32_t n_multi = 0, n_seg = 0, n_rowtasks = 0, n_wide = 0;
};

// Row windows of 128 rows routed to an MFMA tile kernel.  For window i:
// windows[i] = {first row, steps, first global step, first nonzero}; step s
// of the window has B rows ucols[(first global step + s) * 32 + 0..31]
// (-1 = padding past the column union) and nonzeros
// entries[eoff[g] .. eoff[g + 1]) with g its global step; an entry packs the
// row within the window (7 bits), the column within the step (5 bits, bit 7)
// and the nonzero index minus the window's first nonzero (bit 12 up).
// Routing.  A window is eligible for the MFMA tile kernel when its condensed
// tile density nnz / (rows * padded |U|) is at least kMfmaMinDensity and no
// step holds more nonzeros than the kernel's entry slots.  The eligible
// windows then go to the tile kernel as a set when a cost model predicts it
// beats the row kernel on them:
//   tile kernel  ~ fixed_us + rounds * (max steps / 4 + fill_iters) * iter_us
//                  (rounds = ceil(workgroups / 256): one workgroup per CU;
//                   4 steps per iteration plus the pipeline fill),
//   row kernel   ~ eligible nnz * N * value size / kRowGatherBytesPerUs
//                  (B-row gathers through L2).
// Constants measured on MI355X (fp16, 4096-row lognormal and Bernoulli
// matrices, N = 256 / 512); the row kernel sustains ~20 TB/s of gathered B
// rows; density below ~0.04 never paid.
constexpr double kMfmaMinDensity = 0.04;
constexpr double kRowGatherBytesPerUs = 20.0e6;

struct MfmaShape {
    int32_t win_rows;          // rows per window
    int32_t tile_cols;         // C columns per workgroup
    int32_t max_step_entries;  // nonzeros a step may hold (entry slots of the kernel)
    double fixed_us, iter_us;  // cost model: launch + prologue, one 4-step iteration
    int32_t fill_iters;        // pipeline fill, in iterations
};
// Paired kernel: 128 x 64 tiles, up to 512 nonzeros per step, a 4-step
// iteration ~0.95 us.  Dense-tile kernels: 128 x 64 tiles, no per-step entry
// limit (a step is a dense 128 x 32 tile), a 4-step iteration ~0.5 us.
constexpr MfmaShape kMfmaPairShape = {128, 64, 512, 3.0, 0.95, 3};
constexpr MfmaShape kMfmaDenseShape = {128, 64, 128 * 32, 3.0, 0.5, 3};
inline const MfmaShape& mfma_shape(uint32_t flags) {
    if (flags & (TCA_PLAN_MFMA_DENSE | TCA_PLAN_MFMA_COMPACT)) return kMfmaDenseShape;
    return kMfmaPairShape;
}

struct MfmaPlan {
    int32_t win_rows = 128;
    std::vector<Int4> windows;
    std::vector<int32_t> ucols;
    std::vector<int32_t> eoff;
    std::vector<uint32_t> entries;
    std::vector<uint8_t> row_mfma;  // per row: covered by an MFMA window
    int64_t nnz = 0;                // nonzeros in MFMA windows
    int64_t cond_cols = 0;          // padded condensed columns, summed over windows
    int32_t rows = 0;
};

// Windows routed by the rule above (min_density replaces kMfmaMinDensity; with
// force every qualifying window, with disable none).  Only for fp16 / bf16 and
// N % 8 == 0; a window qualifies only while its nonzeros fit the entry
// encoding (< 2^20) and no step holds more than shape.max_step_entries.
void plan_mfma(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t N, int32_t dtype, bool force,
               bool disable, double min_density, const MfmaShape& shape, MfmaPlan* p);

// Column chunks per XCD pay only when B overflows the L2s: 0 (automatic
// chunking) when B is larger than 8 MiB, else 1.  TCA_SLICES (tuning only)
// forces the number of chunks.
int32_t default_slices(int32_t K, int32_t N, int32_t dtype);

// Lane geometry for width N and value size `es` bytes: the widest vector
// (<= 16 bytes) whose element count divides N, and the column chunks: up to
// 8 chunks of at least 128 bytes (one L2 line of B per chunk row), at most
// 64 lanes each.  `slices` > 0 forces the number of chunks (tuning).
void plan_geometry(int32_t N, int32_t es, int32_t slices, RowPlan* p);

// Lane geometry and task-length thresholds (row_len, wide_len, seg_len,
// multi_max) of the row kernel for a matrix of nnz nonzeros.
void plan_row_params(int64_t nnz, int32_t N, int32_t es, int32_t slices, RowPlan* p);

// Row panels with B rows staged in LDS (the panel kernel).  Rows are taken
// longest first (ties by row id) in panels of R = waves * 4 * rpg rows; the
// sorted union of a panel's columns is cut into tiles of at most P columns
// in which no row holds more than kPanelMaxRun nonzeros, and a
// workgroup stages one tile's B rows (all N columns of a column chunk) into
// LDS while its consumer wavefronts multiply the previous tile: every row of
// the panel reads the staged rows of its nonzeros instead of gathering them
// from L2.  Since the CSR columns of a row are sorted and a tile is a range
// of the sorted union, a row's nonzeros in one tile are a contiguous CSR run.
//   slot s of panel p (s = (wave * rpg + i) * 4 + group): rows[p * R + s]
//     (-1 = empty slot); lane group `group` of consumer wave `wave` owns it as
//     its i-th row;
//   tile t (global index): cols[t * P + j] = the B row staged at position j
//     for j < width[t] (padding repeats a valid column; never read);
//   cnt[t * waves * 16 * 4 + (wave * 16 + i) * 4 + group] (bytes): nonzeros
//     of slot s's row in tile t (16 dwords per wave and tile: entries
//     i < rpg), and byte i % 4 of dword kPanelMaxDword + i / 4 the longest
//     of entry i's four counts (the steps the wave takes for entry i);
//   pos[k] for a CSR nonzero k of a panel row: 1 + its position in its tile
//     (the kernel's position 0 is a zero row);
//   units[u] = {panel, first tile, tiles, segment base or -1}: one
//     workgroup; a panel whose nonzeros exceed the unit size is split into
//     panel_units[panel] units by tiles, each writing partial rows that are
//     summed in a fixed order: unit k of a panel whose first segment is f has
//     segment base f + k, and slot s writes segment base + s * panel_units;
//   ustart[u * R + s] = CSR index of slot s's first nonzero in unit u;
//   longrows: {row, first segment, segments, 0} for split panels' rows.
// A panel is taken when its reuse nnz / |union| is at least min_reuse (or
// always with force).  Eligible: N % (16 * E) == 0 for the lane geometry of
// panel_geometry.
struct PanelPlan {
    int32_t waves = 0, rpg = 0, R = 0, P = 0;  // consumer waves, rows per lane group, rows per panel, tile columns
    int32_t elems = 0, chunks = 0;             // B elements per lane, column chunks of C
    int32_t n_panels = 0;
    std::vector<int32_t> rows;
    std::vector<int32_t> cols;
    std::vector<uint8_t> width;  // [tile]: columns of the tile (1..P)
    std::vector<uint8_t> cnt;
    std::vector<uint8_t> pos;  // indexed by CSR nonzero (0 outside panels)
    std::vector<Int4> units;
    std::vector<int32_t> order;  // [workgroup]: unit it runs, -1 = idle (see order_units)
    std::vector<int32_t> panel_units;
    std::vector<int32_t> ustart;
    std::vector<Int4> longrows;
    int64_t n_segments = 0;    // partial rows of split panels
    std::vector<uint8_t> row_panel;  // per row: in a panel
    int64_t nnz = 0;           // nonzeros in panels
    int64_t staged = 0;        // union columns summed over panels
    int32_t n_rows = 0;        // rows in panels
    std::vector<uint8_t> win;  // [panel]: 1 = the kernel takes its run data through per-row windows (panel_window)
    int32_t n_tiles() const { return P ? static_cast<int32_t>(cols.size() / P) : 0; }
};
constexpr int kPanelWaves = 12;   // consumer wavefronts per workgroup (plus four producers: 1024 threads)
constexpr int kPanelRpg = 4;      // rows per 16-lane group
constexpr int kPanelMaxDword = kPanelRpg;  // first dword of the entries' longest counts
constexpr int kPanelCntRows = (kPanelMaxDword + (kPanelRpg + 3) / 4 + 3) / 4 * 4;  // count dwords per wave and tile
static_assert(kPanelRpg <= kPanelMaxDword && kPanelMaxDword + (kPanelRpg + 3) / 4 <= kPanelCntRows, "cnt layout");
constexpr int kPanelMaxRun = 16;  // nonzeros of one row in one tile (one 16-lane batch)
// nnz / |union| a panel needs to be kept.  Measured on MI355X (per SpMM,
// config 2 / config 3): 1.2 1.77 / 3.50 ms, 1.05 - / 3.50, 1.02 1.73 / 3.39,
// 1.0 1.75 / 3.39: staged once per panel, even rows that share few columns
// cost less than the row kernel's gathers; rows that share none stay there.
constexpr double kPanelMinReuse = 1.02;
constexpr int64_t kPanelMinNnz = int64_t(1) << 21;  // fewer nonzeros in panels: none (unless forced)
// Whether the panel kernel takes a panel's run data through windows (a
// window of 16 nonzeros per row serves several tiles): when the panel's
// reuse nnz / |union| is below kPanelWindowReuse its rows hold few nonzeros
// per tile, and the kernel waits on memory more than on issue.  Measured on
// MI355X (panel phase; one box, alternating runs): every panel direct /
// every panel windowed: config 3 (reuse 1.67) 2.82 / 2.34 ms, config 2
// (5.74) 1.53 / 1.57 ms; per panel, config 2 / config 3 whole SpMM:
// threshold 3 1.527-1.534 / 2.672-2.679 ms (config 3's nine hub panels
// direct), 6 1.520-1.544 / 2.620-2.632, every panel windowed 1.575-1.591 /
// 2.626-2.631, none 1.546-1.555 / -.  TCA_PANEL_WINDOW=0 / 1 forces it for
// every panel (tests); TCA_PANEL_WINDOW_REUSE overrides the threshold
// (tuning).
constexpr double kPanelWindowReuse = 6.0;
bool panel_window(int64_t nnz, int64_t staged);
// Launch order of the units (PanelPlan::order).
void order_units(int32_t K, PanelPlan* p);
// The same from each unit's first and last staged column (the GPU planner
// builds those and runs this order on the host).
void order_unit_spans(int32_t K, int32_t chunks, const std::vector<Int4>& units, const std::vector<int64_t>& lo,
                      const std::vector<int64_t>& hi, std::vector<int32_t>* order);
// Routing parameters of the panels (shared by the host and the GPU planner):
// false when the plan takes no panels (TCA_PLAN_NO_PANELS, or by default B
// rows under 256 bytes); else force / min_reuse / min_nnz / unit_nnz for
// plan_panels (TCA_PANEL_MIN_REUSE, TCA_PANEL_MIN_NNZ, TCA_PANEL_UNIT: tuning
// overrides).
struct PanelRoute {
    bool force = false;
    double min_reuse = 0.0;
    int64_t min_nnz = 0, unit_nnz = 0;
};
bool panel_route(int32_t K, int32_t N, int32_t dtype, uint32_t flags, PanelRoute* r);
// Nonzeros per unit for panels holding `tot` nonzeros (unit_nnz > 0: forced).
int64_t panel_unit_nnz(int64_t unit_nnz, int64_t tot);
// Launch order of the row kernel's tasks (RowPlan::order): segments of long
// rows by column range, one range per XCD.  row_order_on: whether a plan
// gets one (one column chunk, at least 32 segments; TCA_ROW_ORDER=0 turns it
// off); the GPU planner builds the same order.
constexpr int32_t kRowOrderSlots = 4;  // wavefronts per row-kernel workgroup (kRowWaves)
bool row_order_on(const RowPlan& p);
void order_row_tasks(const int32_t* colidx, RowPlan* p);
// Lane geometry: 16 lanes cover one column chunk of a B row, E elements each
// (E = 8, 4 or 2 with E * elem_size in 8..32 bytes); 0 when N does not fit.
int32_t panel_elems(int32_t N, int32_t es);
// Default routing also needs B rows of at least 256 bytes (N * elem_size).
bool panel_default_ok(int32_t N, int32_t es);
// Tile width P for a chunk of `chunk_bytes` bytes: two LDS buffers of at most
// 76 KiB, positions fit one byte (P <= 255).
int32_t panel_tile_cols(int32_t chunk_bytes);
// plan_panels with the routing of a plan: none with TCA_PLAN_NO_PANELS, every
// eligible row with TCA_PLAN_FORCE_PANELS, else (B rows of >= 256 bytes)
// panels of reuse >= kPanelMinReuse (every panel when B is larger than the
// MALL) when they hold at least kPanelMinNnz nonzeros in all.
void plan_panels_routed(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t K, int32_t N,
                        int32_t dtype, uint32_t flags, const std::vector<uint8_t>& skip, PanelPlan* p);
// Builds the panel plan over the rows with skip[r] == 0 (skip may be empty).
// unit_nnz: nonzeros per workgroup unit (0 = automatic).
// Unless forced, panels are kept only when they hold at least min_nnz nonzeros in all.
void plan_panels(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t K, int32_t N, int32_t es,
                 const std::vector<uint8_t>& skip, bool force, double min_reuse, int64_t min_nnz, int64_t unit_nnz,
                 PanelPlan* p);

// Builds the row-kernel task list for rows with skip[r] == 0 (skip may be
// empty).  Rows are assigned longest first.  The categories, in task order:
// wide rows (row_len < length <= wide_len, 4 tasks each), long rows
// (length > wide_len, segments of at most seg_len, summed in a fixed order),
// row tasks (max(multi_max, 0) < length <= row_len), groups of `slots` short
// rows (0 < length <= multi_max), then groups of up to kZeroRows empty rows.
// Per-window statistics the MFMA routing decides on: nonzeros, size of the
// column union, most nonzeros in one 32-column condensed step.
struct WinStat {
    int64_t nz;
    int32_t ucount;
    int32_t maxper;
};
// Which windows (of shape.win_rows rows) go to the tile kernel: eligibility
// (nonzeros per step fit the kernel, density >= min_density unless forced)
// and the cost model against the row kernel.  Shared by the host planner
// (plan_mfma) and the planner on the GPU (statistics computed there).
void route_windows(const std::vector<WinStat>& st, int32_t M, int64_t nnz_total, int32_t N, bool force,
                   double min_density, const MfmaShape& shape, std::vector<uint8_t>* take);

void plan_rows(const int32_t* rowptr, int32_t M, int32_t N, int32_t es, const std::vector<uint8_t>& skip,
               int32_t slices, RowPlan* p);

// Sorted column union of every window of `win` rows and each nonzero's
// position in it (the indexing exported by tca_condense_windows).
void condense(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t win, std::vector<int64_t>* uoff,
              std::vector<int32_t>* ucols, std::vector<int32_t>* cpos);

}  // namespace tca
