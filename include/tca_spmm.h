/*
 * tca_spmm.h -- C ABI of the MI355X (gfx950) TCA-SpMM library, libtcaspmm.so.
 *
 * Computes C = A * B where A is an M x K CSR matrix (int32 row offsets and
 * column indices, zero based, columns ascending within a row), B is a dense
 * K x N row-major matrix (leading dimension N) and C is a dense M x N
 * row-major fp32 matrix (leading dimension N).  A and B share one value type
 * (fp16, bf16 or fp32); products are accumulated in fp32.
 *
 * Semantics differ from the reference in one documented way: every row of C
 * is written (beta = 0), so empty rows of A produce zero rows of C.  The
 * reference kernel skips empty rows and leaves the caller's C there
 * (reference src/our_spmm.cu:296-352); its harness zeroes C first
 * (reference src/test.cu:72), so harness-visible results are identical.
 *
 * Every function returns an int status (TCA_OK == 0) and never exits the
 * process; the reference's CHECK_CUDA printed and called exit()
 * (reference src/general.cuh:8-16).  tca_last_error() returns a message for
 * the last failure on the calling thread.
 */
#ifndef TCA_SPMM_H
#define TCA_SPMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Value types.  TCA_F16 matches the reference's `half` A/B with fp32 C
 * (reference src/arg_parse.h:39-41, "-d 0"). */
typedef enum tca_dtype {
    TCA_F16 = 0,
    TCA_F32 = 1,
    TCA_BF16 = 2
} tca_dtype;

typedef enum tca_status {
    TCA_OK = 0,
    TCA_ERR_INVALID = 1,     /* bad argument, shape or CSR structure */
    TCA_ERR_ALLOC = 2,       /* host or device allocation failed */
    TCA_ERR_HIP = 3,         /* a HIP runtime call failed */
    TCA_ERR_UNSUPPORTED = 4, /* valid request this build does not handle */
    TCA_ERR_IO = 5,          /* file could not be opened or read */
    TCA_ERR_FORMAT = 6       /* malformed input file */
} tca_status;

/* Plan flags. */
#define TCA_PLAN_DEFAULT 0u
#define TCA_PLAN_NO_MFMA 1u    /* route every row to the wavefront-per-row kernel */
#define TCA_PLAN_FORCE_MFMA 2u /* route every eligible 128-row window to the MFMA tile kernel (fp16/bf16, N % 8 == 0) */
#define TCA_PLAN_MFMA_DENSE 16u /* dense-tile 128 x 64 kernel (plan keeps dense condensed windows) */
/* Default tile kernel: dense tiles spanning all of K when the routed windows'
 * column unions cover on average >= 85 % of K (B rows then need no gather
 * table), compacted (TCA_TILES_COMPACT) when no step has more than 255
 * non-empty fragment cells, else the paired kernel. */
#define TCA_PLAN_MFMA_PAIR 64u  /* paired (MFMA + staging wavefront) 128 x 64 kernel, whatever the windows */
#define TCA_PLAN_MFMA_COMPACT 128u /* dense-tile kernel on compacted steps (only the non-empty 16-byte
                                      fragment cells, at most 255 per step; else plain dense tiles) */
/* Row panels with B staged in LDS (the panel kernel): by default rows not in
 * MFMA windows are grouped longest first into panels of 192 rows, and those
 * whose nonzeros reuse their column union at least 1.02 times on average
 * (every panel when B is larger than the 256 MB MALL) run on the panel
 * kernel, other rows on the row kernel.  Needs N % (16 E) == 0 for an
 * E in {8, 4, 2} with E * element size in 8..32 bytes; by default also B
 * rows of at least 256 bytes and at least 2^21 nonzeros in panels. */
#define TCA_PLAN_NO_PANELS 256u    /* no panels: rows outside MFMA windows go to the row kernel */
#define TCA_PLAN_FORCE_PANELS 512u /* every eligible row in panels, whatever their reuse */
#define TCA_PLAN_NO_SCRATCH 1024u  /* the plan keeps no partial-row scratch: run it with tca_spmm_run_static */
/* Short-K matrix-core kernel (TCA_TILES_SHORT): fp16 / bf16, N % 8 == 0 and
 * K <= 640: every row, in windows of 64 rows x 64 columns built in LDS from
 * the CSR each run (no plan-time tiles, no pack kernel, one launch).  The
 * default for such matrices whose rows hold at least max(8, 0.08 K)
 * nonzeros on average; this flag asks for it whatever the row lengths.  TCA_PLAN_NO_MFMA and the
 * other tile-kernel flags keep it off; on ineligible inputs it is ignored. */
#define TCA_PLAN_MFMA_SHORT 2048u
/* Every flag a plan accepts; other bits (4, 8 and 32 among them, once tile
 * kernel selectors) give TCA_ERR_INVALID. */
#define TCA_PLAN_KNOWN_FLAGS                                                                            \
    (TCA_PLAN_NO_MFMA | TCA_PLAN_FORCE_MFMA | TCA_PLAN_MFMA_DENSE | TCA_PLAN_MFMA_PAIR |                \
     TCA_PLAN_MFMA_COMPACT | TCA_PLAN_NO_PANELS | TCA_PLAN_FORCE_PANELS | TCA_PLAN_NO_SCRATCH |            \
     TCA_PLAN_MFMA_SHORT)

typedef struct tca_spmm_plan tca_spmm_plan;

/* Plan statistics, for the harness's "num_block / blockdim / shm" line
 * (reference src/our_spmm.cu:552) and for the measurement scripts.  New
 * fields are only ever appended, so the struct grows: compile callers against
 * the header of the library they load (tca_spmm_plan_info writes the whole
 * struct). */
typedef struct tca_plan_info {
    int32_t M, K, N, nnz, dtype;
    int32_t elems_per_lane;   /* B columns per lane per load (16-byte vectors when possible) */
    int32_t lanes_per_row;    /* lanes covering one B-row column chunk (power of 2, <= 64) */
    int32_t col_chunks;       /* column chunks of C (one per XCD slice of B when possible) */
    int32_t n_row_tasks;      /* wavefront tasks of the row kernel */
    int32_t n_multi_tasks;    /* of which: several short rows per wavefront */
    int32_t n_seg_tasks;      /* of which: segments of split long rows */
    int32_t n_long_rows;      /* rows split across wavefronts */
    int32_t n_windows_mfma;   /* 128-row windows routed to the MFMA tile kernel */
    int32_t rows_mfma;        /* rows covered by those windows */
    int64_t nnz_mfma;         /* nonzeros covered by those windows */
    int64_t cond_cols_mfma;   /* sum over MFMA windows of the padded condensed width */
    int32_t row_blocks;       /* workgroups of the row kernel */
    int32_t row_blockdim;     /* threads per workgroup of the row kernel */
    int32_t mfma_blocks;      /* workgroups of the MFMA kernel */
    int32_t mfma_blockdim;
    int32_t mfma_lds_bytes;   /* LDS per MFMA workgroup */
    int32_t seg_len;          /* nonzeros per long-row segment */
    int64_t scratch_bytes;    /* device scratch owned by the plan */
    double plan_ms;           /* host planning time */
    int32_t n_wide_tasks;     /* row-kernel tasks that are quarters of workgroup-shared rows */
    int32_t chunk_lanes;      /* lanes holding data in one column chunk */
    int32_t row_len;          /* rows up to this length take one wavefront */
    int32_t wide_len;         /* rows up to this length take one workgroup; longer rows are segmented */
    int32_t tile_kernel;      /* MFMA tile kernel of the plan: TCA_TILES_* */
    int32_t n_panels;         /* row panels on the panel kernel (B rows staged in LDS) */
    int32_t n_panel_units;    /* workgroup units of those panels */
    int32_t rows_panels;      /* rows in panels */
    int32_t panel_blocks;     /* workgroups of the panel kernel */
    int64_t nnz_panels;       /* nonzeros in panels */
    int64_t staged_panels;    /* B rows staged per run (column unions summed over panels) */
    int32_t panel_blockdim;   /* threads per workgroup of the panel kernel */
    int32_t panel_lds_bytes;  /* LDS per panel workgroup */
    int32_t panel_window;     /* panels whose run data go through per-row windows (low reuse) */
    int32_t rows_beside_panels; /* 1: the row phase only clears empty rows and runs on a second
                                   stream of the plan beside the panel kernel (forked and joined
                                   by events on the run's stream; TCA_ROWS_BESIDE=0 turns it off;
                                   0 also when the runtime could not create that stream) */
} tca_plan_info;

/* tca_plan_info.tile_kernel */
#define TCA_TILES_NONE 0       /* no window routed to the matrix cores (1, 2 and 6 are unused) */
#define TCA_TILES_PAIR 3       /* paired MFMA + staging wavefronts (default when windows are narrow) */
#define TCA_TILES_DENSE 4      /* dense condensed tiles (TCA_PLAN_MFMA_DENSE) */
#define TCA_TILES_DENSE_K 5    /* dense tiles spanning all of K (default when the windows cover most of K) */
#define TCA_TILES_COMPACT 7    /* dense tiles with compacted steps (TCA_PLAN_MFMA_COMPACT) */
#define TCA_TILES_SHORT 8      /* short-K kernel over every row (TCA_PLAN_MFMA_SHORT; default when K <= 640) */

/* Replaces reference workload_manager (src/our_spmm.cu:353-477) plus the
 * device uploads of our_spmm_balanced (src/our_spmm.cu:503-525).
 * rowptr[M+1] and colidx[nnz] are HOST arrays; they are validated (rowptr
 * monotone from 0 to nnz, 0 <= col < K, columns strictly ascending per row)
 * and copied to the device.  The plan keeps the structure; values, B and C
 * are supplied per run.  Requires 1 <= N, M >= 0, K >= 1. */
int tca_spmm_plan_create(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t K,
                         int32_t nnz, int32_t N, int32_t dtype, uint32_t flags,
                         tca_spmm_plan** plan);

/* Replaces the kernel launch of our_spmm_balanced (src/our_spmm.cu:555,561)
 * and kernel_our_spmm_balanced (src/our_spmm.cu:296-352).  d_val[nnz],
 * d_B[K*N] (plan dtype) and d_C[M*N] (fp32) are DEVICE pointers; d_B and d_C
 * must be aligned to 16 bytes.  Stream-ordered on `stream` (a hipStream_t,
 * NULL = default stream); does not synchronise.  One plan must not run on two
 * streams at once: long-row partial sums live in plan-owned scratch.  A plan
 * whose row phase only clears empty rows (tca_plan_info.rows_beside_panels)
 * runs it on a second stream it owns, beside the panel kernel: that stream
 * waits for the work queued on `stream` before the call, and `stream` waits
 * for it before the call's last kernel, so the run stays ordered on `stream`
 * (under graph capture the two become a fork and a join of the graph). */
int tca_spmm_run(const tca_spmm_plan* plan, const void* d_val, const void* d_B, float* d_C,
                 void* stream);

/* Allocation-free variant of tca_spmm_run, for callers that cannot allocate
 * device memory while they run (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc); no counterpart in the reference.
 * The kernels are tca_spmm_run's; the partial rows of split rows (row-kernel
 * segments, units of split panels) go to a file-scope device array of
 * 64 MiB per GPU instead of plan-owned memory, so the plan may be created
 * with TCA_PLAN_NO_SCRATCH.  Calls no hipMalloc or hipFree.  Plans whose
 * partial rows exceed 64 MiB are rejected (TCA_ERR_UNSUPPORTED); the
 * current device must be the plan's.  Every call on one GPU shares that
 * GPU's array (each partial row is written before it is read, nothing needs
 * clearing): calls that overlap on one GPU, on any streams, race. */
int tca_spmm_run_static(const tca_spmm_plan* plan, const void* d_val, const void* d_B, float* d_C,
                        void* stream);

/* Times tca_spmm_run the way our_spmm_balanced does (src/our_spmm.cu:553-576):
 * `warmup` untimed launches, then `iters` launches between two hipEvents
 * recorded on `stream`; *avg_ms = elapsed / iters.  Synchronises `stream`. */
int tca_spmm_time(const tca_spmm_plan* plan, const void* d_val, const void* d_B, float* d_C,
                  void* stream, int32_t warmup, int32_t iters, float* avg_ms);

/* Phases of one run, in stream order: value pack for the MFMA tiles, MFMA
 * tile kernel, panel kernel, row kernel, segment sums of split rows (the
 * panel phase has index 4 so the older indices stay as they were). */
#define TCA_PHASES 5
enum { TCA_PHASE_PACK = 0, TCA_PHASE_TILES = 1, TCA_PHASE_ROWS = 2, TCA_PHASE_SEGMENTS = 3, TCA_PHASE_PANELS = 4 };
/* Slot after the phases in tca_spmm_time_phases' output: the whole run. */
#define TCA_PHASE_RUN TCA_PHASES

/* Per-phase timing inside whole runs: `warmup` runs, then `iters` runs back
 * to back on `stream`; each phase's kernel is dispatched with a start and a
 * stop hipEvent of its own (hipExtLaunchKernelGGL: the kernel's span, as a
 * kernel trace reports it, with nothing inserted between the kernels).
 * phase_ms[k] = mean milliseconds of phase k's kernel over the runs, 0 for a
 * phase the plan does not use.  phase_ms holds n_phase_ms floats: the first
 * min(n_phase_ms, TCA_PHASES) entries are written (TCA_PHASES grew from 4 to
 * 5 when the panel phase was added; the length argument keeps an older,
 * shorter buffer in bounds), and when n_phase_ms > TCA_PHASE_RUN also
 * phase_ms[TCA_PHASE_RUN] = mean milliseconds of one whole run of the same
 * runs (hipEvents before the first and after the last, as tca_spmm_time), so
 * every phase of the output lies within its run time.  Dispatches that carry
 * timestamps leave gaps of several microseconds between kernels (measured on
 * MI355X: a 5.6 us single-kernel run takes 17.5 us), so that run time is not
 * the SpMM's: tca_spmm_time gives it.  iters <= 100000.  No counterpart in the
 * reference, which times whole runs only (src/our_spmm.cu:553-576); this is
 * the per-kernel figure a roofline needs. */
int tca_spmm_time_phases(const tca_spmm_plan* plan, const void* d_val, const void* d_B, float* d_C, void* stream,
                         int32_t warmup, int32_t iters, float* phase_ms, int32_t n_phase_ms);

/* Timing of a subset of a run's phases: `warmup`, then `iters` runs of only
 * the phases whose bit (1 << TCA_PHASE_*) is set in phase_mask, in run
 * order, back to back between two hipEvents on `stream`; *avg_ms = mean
 * milliseconds per run.  C holds a full product only when every phase the
 * plan uses is in the mask.  With the full mask it is tca_spmm_time; without
 * one phase, the difference to the full time is that phase's share of the
 * timed step (how bench.py times the roofline's kernel).  No counterpart in
 * the reference (src/our_spmm.cu:553-576 times whole runs). */
int tca_spmm_time_subset(const tca_spmm_plan* plan, const void* d_val, const void* d_B, float* d_C, void* stream,
                         uint32_t phase_mask, int32_t warmup, int32_t iters, float* avg_ms);
/* The phases the plan runs: bit 1 << TCA_PHASE_* set for each. */
int tca_spmm_plan_phases(const tca_spmm_plan* plan, uint32_t* phase_mask);

/* Backward-pass kernels of the PyTorch op (no counterpart in the reference,
 * which has no backward pass).
 *
 * tca_sddmm: d_out[j] = sum_n d_G[row(j) * N + n] * d_B[col(j) * N + n] for
 * every nonzero j of the plan's A (fp32 G of shape M x N, B K x N in the
 * plan's dtype, fp32 out[nnz]): the gradient of C = A * B with respect to
 * A's values.  Deterministic (fixed reduction order).
 *
 * tca_gather_values: d_out[i] = (float)d_val[d_perm[i]] for i < n (A's
 * values in the order of its transpose, see tca_csr_transpose). */
int tca_sddmm(const tca_spmm_plan* plan, const float* d_G, const void* d_B, float* d_out, void* stream);
int tca_gather_values(const int32_t* d_perm, int32_t n, const void* d_val, int32_t dtype, float* d_out,
                      void* stream);

/* C = A * B with A in Blocked-ELL (layout of tca_csr_to_bell, the format
 * reference perform_cuSPARSE_BlockSpMM hands to cusparseSpMM,
 * src/spmm_cusparse.cu:181-445), on the matrix cores.  d_colind is
 * [ceil(M/bsize)][ell_blocks], d_values [ceil(M/bsize)*bsize][ell_blocks*bsize]
 * (fp16 or bf16, 16-byte aligned), B K x N row-major (same dtype, 16-byte
 * aligned), C M x N fp32, every row written (beta = 0).  bsize 32 or 64,
 * N % 8 == 0.  Stream-ordered, deterministic.  The reference times
 * cusparseSpMM on this format; this is its replacement. */
int tca_bell_spmm(const int32_t* d_colind, const void* d_values, int32_t M, int32_t K, int32_t N, int32_t bsize,
                  int32_t ell_blocks, int32_t dtype, const void* d_B, float* d_C, void* stream);

/* C = A * B with A in compressed 2:4 form (layout of tca_csr_to_24; the
 * format reference perform_cuSPARSELT_24sparsity multiplies with
 * cusparseLtMatmul, src/spmm_cusparse.cu:2-179) on gfx950's sparse matrix
 * cores (v_smfmac_f32_16x16x64).  d_vals [M][Kp/2] and B (K x N row-major)
 * fp16 or bf16, 16-byte aligned; d_meta [M][Kp/16] uint16; C M x N fp32,
 * every row written (beta = 0; the reference writes fp16 C).  Kp = K rounded
 * up to 64; N % 8 == 0.  Stream-ordered, deterministic. */
int tca_spmm_24(const void* d_vals, const uint16_t* d_meta, int32_t M, int32_t K, int32_t N, int32_t dtype,
                const void* d_B, float* d_C, void* stream);

/* Planning on the GPU from a device-resident CSR (d_rowptr [M+1], d_colidx
 * [nnz], sorted columns), with no host copy of the structure.  The matrix-core
 * windows are routed by the host planner's rule from statistics computed on
 * the device (column-union bitmaps of the 128-row windows, union sizes,
 * nonzeros per condensed step; a few integers per window come back) and,
 * for the routed windows, the dense tiles are laid out on the device: in
 * natural column order when the windows cover most of K (the host default,
 * TCA_TILES_DENSE_K), else condensed (TCA_TILES_DENSE; the host default
 * there is the paired kernel, whose layout only the host builds).  The row
 * panels of the other rows (the panel kernel) are planned on the device
 * too: column unions of 192-row candidates in LDS bitmaps, the host's reuse
 * rule on a few integers per candidate, tile cuts by a suffix minimum over
 * union positions, counts, positions, units and their cursors per nonzero,
 * the XCD launch order on the host from each unit's column span
 * (tca_spmm_plan_export_panels reads them back).  The row-kernel task list
 * of the remaining rows is built by device kernels (row lengths, a stable
 * descending radix sort, category bounds, a segment scan, task emission).
 * With TCA_PLAN_NO_MFMA, TCA_PLAN_MFMA_DENSE (optionally with
 * TCA_PLAN_FORCE_MFMA), or by default when the windows cover most of K, the
 * plan equals the host planner's for the same flags, entry for entry.
 * TCA_PLAN_MFMA_PAIR gives TCA_ERR_UNSUPPORTED; window tables above 2^25
 * words (windows x ceil(K / 32)) leave every row outside MFMA windows; K
 * above 2^31 - 2^19 with panels gives TCA_ERR_UNSUPPORTED.  The structure is validated on the device
 * (TCA_ERR_INVALID as the host planner).  The plan copies the structure;
 * the caller's buffers may be freed after the call, which synchronises
 * `stream`.  Replaces reference workload_manager (src/our_spmm.cu:353-477),
 * which plans on the host from host arrays on every call. */
int tca_spmm_plan_create_device(const int32_t* d_rowptr, const int32_t* d_colidx, int32_t M, int32_t K, int32_t nnz,
                                int32_t N, int32_t dtype, uint32_t flags, void* stream, tca_spmm_plan** plan);

/* The row-kernel task list of a plan, copied to the host (int4 tasks as 4
 * int32 each, the multi-task row permutation, the long-row table); with
 * tasks == NULL only the counts are returned.  No counterpart in the
 * reference: for tests and tools comparing plans. */
int tca_spmm_plan_export_rows(const tca_spmm_plan* plan, int32_t* n_tasks, int32_t* n_perm, int32_t* n_long,
                              int32_t* tasks, int32_t* perm, int32_t* longrows);

/* The row kernel's launch order (wavefront slot -> task, -1 an idle slot;
 * long rows' segments grouped by column range per XCD), copied to the host;
 * with order == NULL only the count, 0 when the tasks run in task order.  No
 * counterpart in the reference: for tests comparing host and GPU plans. */
int tca_spmm_plan_export_order(const tca_spmm_plan* plan, int32_t* n_slots, int32_t* order);

/* The dense-tile data of a plan whose tile kernel is TCA_TILES_DENSE or
 * TCA_TILES_DENSE_K, copied to the host: the windows ({first row, steps,
 * first global step, first nonzero} as 4 int32 each), per routed nonzero its
 * half index in the dense tiles and its CSR index (sorted by position), and
 * for condensed tiles the B row byte offsets of every step's 32 columns
 * (0xffffffff padding; none for natural order).  With windows == NULL only
 * the counts are returned; other plans report zero counts.  No counterpart
 * in the reference: for tests and tools comparing plans. */
int tca_spmm_plan_export_tiles(const tca_spmm_plan* plan, int32_t* n_windows, int32_t* n_entries, int32_t* n_ucols,
                               int32_t* windows, uint32_t* pos, int32_t* src, uint32_t* ucols);

/* The plan's row panels as the panel kernel reads them (so tests can check a
 * GPU-built plan against the host planner's, entry for entry).  sizes[8] in:
 * capacities, out: {panels, tiles, units, launch-order entries, the panels'
 * long rows, R (rows per panel), P (tile columns), pos bytes}.  With rows ==
 * NULL only the sizes are written.  Arrays: rows [panels * R] (-1: empty
 * slot), boff [tiles * P] (staged B rows as byte offsets), cnt [tiles *
 * waves * 8] (count dwords), pos [pos bytes] (1-based tile position per
 * nonzero, 0 outside panels), units [units * 4], order [launch-order entries]
 * (-1: idle workgroup), panel_units [panels], ustart [units * R], longrows
 * [panel long rows * 4] (segment slots after the row kernel's), window
 * [panels] (1: the panel's run data go through per-row windows).  No
 * counterpart in the reference (its task split, src/our_spmm.cu:353-477, has
 * no panels). */
int tca_spmm_plan_export_panels(const tca_spmm_plan* plan, int64_t* sizes, int32_t* rows, uint32_t* boff, uint32_t* cnt,
                                uint8_t* pos, int32_t* units, int32_t* order, int32_t* panel_units, int32_t* ustart,
                                int32_t* longrows, uint8_t* window);

int tca_spmm_plan_info(const tca_spmm_plan* plan, tca_plan_info* info);

int tca_spmm_plan_destroy(tca_spmm_plan* plan);

/* Host-pointer driver with the contract of reference our_spmm_balanced
 * (src/our_spmm.cu:478-594, declared src/our_spmm.cuh:4): allocates device
 * buffers, copies A, B in, plans, runs 5 warm-ups and n_iter timed launches,
 * copies C back, frees everything.  *elapsed_ms (if not NULL) receives the
 * mean ms per launch.  Prints "preprocess %fms taken" and
 * "num_block: %d blockdim: %d shm: %fKB" like the reference when verbose != 0. */
int tca_spmm_host(const int32_t* rowptr, const int32_t* colidx, const void* val, int32_t M,
                  int32_t K, int32_t nnz, const void* B, float* C, int32_t N, int32_t dtype,
                  int32_t n_iter, int32_t verbose, double* elapsed_ms);

/* ---- condensed row windows (host, exported so tests can pin the indexing) ----
 * For row window w (rows [w*win, min(M,(w+1)*win))), ucols holds the sorted
 * union of the window's column indices at [uoff[w], uoff[w+1]), and for each
 * nonzero j of the window cpos[j] is the position of colidx[j] inside that
 * union (so ucols[uoff[w] + cpos[j]] == colidx[j]).  Pass ucols == NULL to
 * get only uoff (sizes).  uoff has n_windows+1 entries. */
int tca_condense_windows(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t nnz,
                         int32_t win, int64_t* uoff, int32_t* ucols, int32_t* cpos);

/* ---- host-only view of the row kernel's task list (no device needed) ----
 * The wavefront tasks tca_spmm_plan_create builds for this structure, shape
 * (M x K, width N) and dtype, with no rows routed to the MFMA kernel.  Call with tasks == NULL
 * to get the counts, then again with tasks[4*n_tasks], perm[n_perm] and
 * longrows[4*n_long].  Task int4 {x,y,z,w}: w == 0 row task (x row, [y,z)
 * nonzeros); w == 1 multi task (x offset into perm, y rows, z longest row;
 * z == 0: up to 64 empty rows whose C rows are cleared);
 * w & 3 == 2 segment task (x long-row id, [y,z) nonzeros, w >> 2 segment
 * slot); w & 3 == 3 quarter of a wide row (x row, [y,z) nonzeros, w >> 2
 * quarter), four consecutive 4-aligned tasks per wide row.  longrows entry
 * {row, first segment slot, segments, 0}.  Every task runs once per column
 * chunk.  geometry[8] receives elems_per_lane, lanes per slot, column chunks,
 * segment length, lanes per chunk, row-task length limit, wide-row length
 * limit and the multi-task length limit. */
int tca_plan_row_tasks(const int32_t* rowptr, int32_t M, int32_t K, int32_t N, int32_t dtype, int32_t* n_tasks,
                       int32_t* n_perm, int32_t* n_long, int32_t* tasks, int32_t* perm, int32_t* longrows,
                       int32_t* geometry);

/* ---- host-only view of the MFMA window plan (no device needed) ----
 * The 128-row windows tca_spmm_plan_create routes to the MFMA tile kernel for
 * this structure, width N, dtype and flags.  Call with windows == NULL to get
 * the counts, then with windows[4*n_windows], ucols[32*n_steps],
 * eoff[n_steps+1] and entries[n_entries].  windows[i] = {first row, steps,
 * first global step, first nonzero}; global step g gathers B rows
 * ucols[32g .. 32g+31] (-1 = padding) and holds entries eoff[g] ..
 * eoff[g+1]-1, each packing the row within the window (bits 0-6), the
 * column within the step (bits 7-11) and the nonzero index minus the
 * window's first nonzero (bits 12-31). */
int tca_plan_mfma_windows(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t N, int32_t dtype,
                          uint32_t flags, int32_t* n_windows, int32_t* n_steps, int64_t* n_entries,
                          int32_t* windows, int32_t* ucols, int32_t* eoff, uint32_t* entries);

/* ---- host-only view of the panel plan (no device needed) ----
 * The row panels tca_spmm_plan_create gives the panel kernel for this
 * structure, width N, dtype and flags (after MFMA routing).  Call with
 * rows == NULL to get sizes[16] = {panels, tiles, units, long rows, R, P,
 * consumer waves, rows per lane group, elements per lane, column chunks,
 * nonzeros in panels, staged columns, partial segments, rows in panels,
 * count bytes per tile, first dword of the longest runs in a wave's counts}; then with rows[panels*R], cols[tiles*P],
 * width[tiles], cnt[tiles * sizes[14]], pos[nnz], units[4*units], panel_units[panels],
 * ustart[units*R], longrows[4*long rows].  Layouts: see PanelPlan in
 * spmm_amd/csrc/planner.hpp.  No counterpart in the reference. */
int tca_plan_panels(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t K, int32_t N,
                    int32_t dtype, uint32_t flags, int64_t* sizes, int32_t* rows, int32_t* cols,
                    uint8_t* width, uint8_t* cnt, uint8_t* pos, int32_t* units, int32_t* panel_units,
                    int32_t* ustart, int32_t* longrows);

/* ---- host-only view of the launch orders (no device needed) ----
 * Workgroup b of a launch runs on XCD b % 8.  For this structure, width N,
 * dtype and flags (MFMA routing as tca_plan_panels; the short-K kernel is
 * not considered): the panel kernel's workgroup -> unit order (-1 an idle
 * workgroup; units as tca_plan_panels returns them), and the row kernel's
 * task list (int4 tasks as 4 int32, for the rows outside MFMA windows and
 * panels) with its wavefront slot -> task order (-1 an idle slot; empty
 * when the tasks run in task order).  Call with panel_order == NULL for
 * the counts.  No counterpart in the reference: for tests of the planner. */
int tca_plan_launch_orders(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t K, int32_t N,
                           int32_t dtype, uint32_t flags, int32_t* n_blocks, int32_t* panel_order, int32_t* n_tasks,
                           int32_t* tasks, int32_t* n_slots, int32_t* row_order);

/* Launches a trivial kernel on the current device and synchronises
 * (reference warm_up_gpu_kernel, src/miscalleneous.cu:158-164, launched
 * <<<1,32>>> ten times by src/test.cu:50-52). */
int tca_warm_up(void);

/* Launch floor: mean milliseconds per launch of an empty one-wavefront kernel,
 * `iters` launches back to back on `stream` between two hipEvents (the time
 * below which no SpMM launch can go).  No counterpart in the reference. */
int tca_launch_floor(void* stream, int32_t iters, float* avg_ms);

/* ---- library information ---- */
const char* tca_status_string(int status);
const char* tca_last_error(void);
int tca_device_count(int32_t* count);
int tca_version(void);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* TCA_SPMM_H */
