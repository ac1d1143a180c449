/*
 * tca_host.h -- host-side C ABI of libtcaspmm.so: sparse containers, the
 * .smtx / .mtx readers, format conversion, the validation verdict and the
 * seeded input generators.  Everything here runs on the CPU; the SpMM itself
 * is in tca_spmm.h.
 *
 * Values are typed by a tca_dtype (tca_spmm.h): fp16 and bf16 values are
 * stored as their 16-bit IEEE / bfloat16 bit patterns (uint16_t), fp32 as
 * float.  Arrays returned in structs are malloc'ed by the library and released
 * with tca_csr_free / tca_coo_free / tca_free.
 */
#ifndef TCA_HOST_H
#define TCA_HOST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Layout-compatible with the reference struct CSR (src/general.cuh:125-134):
 * {int nRow, nCol, nnz; int* row_offset; int* col_idx; half* value;}, plus the
 * value type at the end. */
typedef struct tca_csr {
    int32_t nRow;
    int32_t nCol;
    int32_t nnz;
    int32_t* row_offset; /* nRow + 1 */
    int32_t* col_idx;    /* nnz, ascending within a row */
    void* value;         /* nnz values of type `dtype` */
    int32_t dtype;
} tca_csr;

/* Coordinate format.  The reference names COO only as a mat_format value
 * (src/mat_format.cuh:10-15) and never defines the container. */
typedef struct tca_coo {
    int32_t nRow;
    int32_t nCol;
    int32_t nnz;
    int32_t* row_idx;
    int32_t* col_idx;
    void* value;
    int32_t dtype;
} tca_coo;

/* Mirrors reference mat_format (src/mat_format.cuh:10-15). */
typedef enum tca_mat_format { TCA_FMT_DENSE = 0, TCA_FMT_CSR = 1, TCA_FMT_COO = 2 } tca_mat_format;

void tca_csr_free(tca_csr* a);
void tca_coo_free(tca_coo* a);
void tca_free(void* p);

/* Test hook: allocation-failure injection.  After host_after further host
 * allocations of arrays the library hands out (CSR / COO / dense results),
 * the next one fails; after device_after further device allocations (plan
 * creation, the host driver), the next one fails; each counter then disarms.
 * -1 disarms a counter.  The failing call returns TCA_ERR_ALLOC and releases
 * what it had allocated.  No counterpart in the reference. */
int tca_debug_fail_allocs(int64_t host_after, int64_t device_after);

/* Checks rowptr[0] == 0, monotone, rowptr[nRow] == nnz, 0 <= col < nCol and
 * strictly ascending columns within each row.  TCA_OK or TCA_ERR_INVALID. */
int tca_csr_validate(const int32_t* rowptr, const int32_t* colidx, int32_t nRow, int32_t nCol,
                     int32_t nnz);

/* ---- .smtx (reference src/file_input.cu:135-193) ----
 * Line 1: "rows, cols, nnz"; line 2: rows+1 row offsets separated by blanks;
 * every further line: column indices separated by blanks.  The format has no
 * values: every listed entry is 1.0 in `dtype`.  Unlike the reference this
 * reader streams the file (no dense intermediate, which would need M*K
 * halves) and rejects malformed input with TCA_ERR_FORMAT: wrong token
 * counts, rowptr not monotone from 0 to nnz, col out of [0, cols),
 * columns not strictly ascending in a row. */
int tca_smtx_read_csr(const char* path, int32_t dtype, tca_csr* out);

/* Reference semantics of smtx_input_to_Dense: dense nRow x nCol matrix of
 * `dtype` with 1.0 at each entry (malloc'ed, release with tca_free). */
int tca_smtx_read_dense(const char* path, int32_t dtype, void** dense, int32_t* nRow,
                        int32_t* nCol, int32_t* nnz);

/* Writes the pattern of `a` as .smtx (header "rows, cols, nnz", the row
 * offsets line, one column-index line), each number followed by a blank like
 * the reference fixture. */
int tca_smtx_write(const char* path, const tca_csr* a);

/* ---- binary CSR cache and values sidecar (no counterpart in the reference) ----
 * Binary CSR: magic "TCACSR01", int32 nRow, nCol, int64 nnz, int32 dtype,
 * int32 0, then rowptr int32[nRow+1], colidx int32[nnz], values (dtype)[nnz],
 * all little endian.  The reader checks the magic, that the header matches
 * the file size exactly and the CSR invariants (tca_csr_validate): a cache
 * that loads a large graph without re-parsing text.
 * Values file: magic "TCAVAL01", int64 nnz, int32 dtype, int32 0, then the
 * values.  tca_smtx_read_csr_values reads a .smtx pattern and attaches the
 * values (converted to `dtype`; the counts must agree), since the .smtx
 * format itself has none (reference src/file_input.cu:189 sets 1.0). */
int tca_csr_write_binary(const char* path, const tca_csr* a);
int tca_csr_read_binary(const char* path, tca_csr* out);
int tca_values_write(const char* path, const void* values, int64_t nnz, int32_t dtype);
int tca_smtx_read_csr_values(const char* smtx_path, const char* values_path, int32_t dtype, tca_csr* out);

/* ---- MatrixMarket coordinate files (reference src/file_input.cu:8-134) ----
 * '%' lines are skipped, then "rows cols nnz", then one "r c [v]" per line.
 * pattern_only: values are 1.0 (only "r c" is read); otherwise a missing
 * value reads as 0, as in the reference.  zero_based == 0: indices are one
 * based.  Values are parsed like the reference's `stream >> float` (the
 * decimal rounded once to fp32), then converted to dtype (RNE).  Blank lines
 * are skipped; entries out of range and an entry count other than the
 * header's give TCA_ERR_FORMAT (the reference asserts the count).
 *
 * tca_mtx_read_csr: entries sorted by (row, col), duplicate (row, col) pairs
 * rejected -- the CSR contract of tca_spmm_plan_create. */
int tca_mtx_read_csr(const char* path, int32_t pattern_only, int32_t zero_based, int32_t dtype,
                     tca_csr* out);
/* The reference's CSR exactly (mtx_input_to_CSR, src/file_input.cu:63-134):
 * rows ascending, each row's entries in file order, duplicates kept.  For
 * files sorted column-major or row-major (MatrixMarket's usual orders) the
 * columns of each row ascend and the result is a valid tca_spmm input;
 * otherwise tca_spmm_plan_create rejects it (columns not ascending). */
int tca_mtx_read_csr_file_order(const char* path, int32_t pattern_only, int32_t zero_based, int32_t dtype,
                                tca_csr* out);
/* The reference's dense reader (mtx_input_to_Dense, src/file_input.cu:8-62):
 * a value is read on every line (1.0 when missing, whatever pattern_only),
 * nRow x nCol row-major elements of dtype (release with tca_free),
 * zero except at the entries, a later duplicate overwriting an earlier one;
 * *nnz = entries read. */
int tca_mtx_read_dense(const char* path, int32_t zero_based, int32_t dtype, void** dense, int32_t* nRow,
                       int32_t* nCol, int32_t* nnz);

/* ---- format conversion (reference src/miscalleneous.cu:29-81) ---- */
/* Keeps entries whose fp32 value != 0 (so +-0 are dropped), row-major. */
int tca_dense_to_csr(const void* dense, int32_t nRow, int32_t nCol, int32_t dtype, tca_csr* out);
/* dense must hold nRow*nCol elements of a->dtype; it is fully overwritten. */
int tca_csr_to_dense(const tca_csr* a, void* dense);
int tca_csr_to_coo(const tca_csr* a, tca_coo* out);
/* Sorts by (row, col); rejects duplicates and out-of-range indices. */
int tca_coo_to_csr(const tca_coo* a, tca_csr* out);

/* Structure of the transpose: A (M x K, CSR) -> A^T (K x M, CSR), columns of
 * each row of A^T ascending; perm[t] = the nonzero of A stored at position t
 * of A^T (values of A^T = values of A gathered through perm).  rowptr_t has
 * K + 1 entries, colidx_t and perm nnz.  No counterpart in the reference
 * (it never transposes); the backward pass of the PyTorch op multiplies by
 * A^T. */
int tca_csr_transpose(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t K, int32_t nnz,
                      int32_t* rowptr_t, int32_t* colidx_t, int32_t* perm);
/* Value conversion of a CSR (same structure, new dtype, RNE rounding). */
int tca_csr_convert(const tca_csr* a, int32_t dtype, tca_csr* out);

/* Blocked-ELL, the format reference perform_cuSPARSE_BlockSpMM builds for
 * cusparseCreateBlockedEll (src/spmm_cusparse.cu:201-342): blocks of
 * bsize x bsize; block row i (rows i*bsize .. i*bsize + bsize - 1, rows past
 * M zero) lists the block columns j that hold a nonzero value (|v| != 0, as
 * the reference counts them at :261-269), ascending, padded with -1 to
 * ell_blocks = the longest such list.  colind is [ceil(M/bsize)][ell_blocks];
 * ell_values is row-major [ceil(M/bsize)*bsize][ell_blocks*bsize] of dtype:
 * element (r, e*bsize + c) = A[r][colind[r/bsize][e]*bsize + c], zero for
 * padding blocks and for columns past K.
 * With colind == NULL and ell_values == NULL only *ell_blocks is computed
 * (the size query); otherwise both arrays must be sized from it. */
int tca_csr_to_bell(const int32_t* rowptr, const int32_t* colidx, const void* values, int32_t M, int32_t K,
                    int32_t nnz, int32_t dtype, int32_t bsize, int32_t* ell_blocks, int32_t* colind,
                    void* ell_values);

/* 2:4 structured sparsity, the format of reference
 * perform_cuSPARSELT_24sparsity (src/spmm_cusparse.cu:2-179), which prunes A
 * with cusparseLtSpMMAPrune(CUSPARSELT_PRUNE_SPMMA_STRIP) and multiplies the
 * compressed A.  Groups are 4 consecutive columns of a row (columns
 * 4g .. 4g + 3).
 *
 * tca_prune_24: the pruned copy of A keeping, in every group, the two
 * entries of largest |value| (STRIP: the kept pair maximises the group's L1
 * norm); equal magnitudes keep the lower column.  Entries whose value is
 * zero are dropped first.  out's arrays are allocated by the library (free
 * with tca_csr_free).
 *
 * tca_csr_to_24: compression of a 2:4 matrix (at most two nonzeros per
 * group, else TCA_ERR_INVALID).  Kp = K rounded up to a multiple of 64.
 * vals24 is [M][Kp / 2] of dtype, meta24 [M][Kp / 16] uint16: word q of row
 * r describes columns 16 q .. 16 q + 15 as 4 groups G; bits 4G .. 4G + 1
 * give the position (0..3) inside group G of the value at
 * vals24[r][8 q + 2 G], bits 4G + 2 .. 4G + 3 that of vals24[r][8 q + 2 G + 1];
 * the positions of a group are ascending and distinct, unused values zero.
 * This is the operand layout of gfx950's v_smfmac_f32_16x16x64 (a lane reads
 * one 16-byte run of vals24 and one meta word). */
int tca_prune_24(const int32_t* rowptr, const int32_t* colidx, const void* values, int32_t M, int32_t K,
                 int32_t nnz, int32_t dtype, tca_csr* out);
int tca_csr_to_24(const int32_t* rowptr, const int32_t* colidx, const void* values, int32_t M, int32_t K,
                  int32_t nnz, int32_t dtype, void* vals24, uint16_t* meta24);

/* ---- scalar conversion (IEEE binary16 / bfloat16, round to nearest even) ---- */
uint16_t tca_f32_to_f16(float x);
float tca_f16_to_f32(uint16_t h);
uint16_t tca_f32_to_bf16(float x);
float tca_bf16_to_f32(uint16_t h);
/* Bulk conversions of n values. */
void tca_convert_array(const void* src, int32_t src_dtype, void* dst, int32_t dst_dtype, int64_t n);

/* ---- validation (reference src/general.cuh:71-123) ---- */
typedef struct tca_compare_result {
    int32_t success;      /* 1 when no element failed */
    int64_t fail_count;   /* failures counted before the scan stopped (stops at 10) */
    int64_t first_fail;   /* index of the first failing element, -1 if none */
    float max_rel;        /* max relative discrepancy over the scanned prefix */
    float max_rel_floor;  /* max over ALL elements of |g-c| / max(|g|, floor) */
} tca_compare_result;

/* Element i fails iff |g-c|/|g| >= tol and |g-c| >= tol (fp32), the
 * reference verdict; the scan stops at the 10th failure.  When verbose != 0
 * each failure is printed in the reference's words.  max_rel_floor is an
 * extra report over every element with an absolute floor `floor` on |g|. */
int tca_compare_mat(const float* gold, const float* cmp, int64_t n, float tol, float floor,
                    int32_t verbose, tca_compare_result* res);

/* ---- CPU products used as the harness's validation gold ----
 * Arithmetic of reference naive_gemm (src/miscalleneous.cu:114-134): fp32
 * multiply, then fp32 add, k ascending.  Never used by tca_spmm_run. */
int tca_naive_gemm(const void* A, const void* B, float* C, int32_t M, int32_t N, int32_t K,
                   int32_t dtype);
int tca_naive_csr_spmm(const tca_csr* a, const void* B, float* C, int32_t N, int32_t threads);

/* ---- seeded generators ----
 * All randomness comes from SplitMix64 streams keyed by (seed, stream id,
 * index), so output is identical for any thread count and platform.
 * fp16/bf16 values are rounded from the fp32 draw with RNE; an entry whose
 * rounded value is +-0 is dropped, as reference convert_dense_to_csr
 * (src/miscalleneous.cu:56) would drop it. */
typedef struct tca_gen_stats {
    int64_t nnz;
    int32_t max_row;
    int32_t empty_rows;
    int32_t rows_over_10k;
    double mean_row;
    int64_t samples;     /* R-MAT: edge samples drawn */
} tca_gen_stats;

/* dist: 0 = U(-1,1), 1 = N(0,1), 2 = U(0,1), 3 = reference prepare_cpu_matrix
 * (src/general.cuh:140-174): U(0,1) with probability 1 - sparsity else 0,
 * but seeded.  Writes rows*cols values of dtype into out. */
int tca_gen_dense(int64_t rows, int64_t cols, int32_t dist, float sparsity, uint64_t seed,
                  int32_t dtype, void* out);

/* Each of the M*K entries kept independently with probability p; values
 * N(0, sigma). (Benchmark configuration 0: 2048 x 512, p = 0.1, sigma = 0.02.) */
int tca_gen_bernoulli(int32_t M, int32_t K, double p, double sigma, uint64_t seed,
                      int32_t dtype, tca_csr* out, tca_gen_stats* st);

/* Row lengths round(LogNormal(ln(mean) - s^2/2, s)) clipped to [0, K];
 * columns uniform without replacement; values N(0, sigma).
 * (Config 1: 4096 x 4096, mean 205, s = 1, sigma = 0.02.) */
int tca_gen_lognormal_rows(int32_t M, int32_t K, double mean, double s, double sigma,
                           uint64_t seed, int32_t dtype, tca_csr* out, tca_gen_stats* st);

/* R-MAT graph on 2^scale ids with ids >= n rejected (a, b, c; d = 1-a-b-c),
 * `samples` accepted non-self-loop samples, symmetrised when symmetric != 0,
 * duplicates removed.  norm: 0 = GCN D^-1/2 (A+I) D^-1/2 (self-loops added,
 * degrees include them), 1 = mean aggregation 1/deg(row) (no self-loops),
 * 2 = all ones. (Configs 2 and 3.) */
int tca_gen_rmat(int32_t scale, int32_t n, int64_t samples, double a, double b, double c,
                 int32_t symmetric, int32_t norm, uint64_t seed, int32_t dtype, tca_csr* out,
                 tca_gen_stats* st);

/* Zipf row lengths: raw length z = floor(u^(-1/(s-1))) (P(z >= k) = k^(1-s)),
 * scaled by one factor f and capped: len = min(cap, floor(f*z)), f chosen by
 * bisection so the total is as close to total_nnz as possible from below,
 * the remainder added one per row to the first uncapped rows of largest
 * fractional part; columns uniform without replacement; values U(-1,1).
 * (Config 4: 2^20 x 2^20, 20M nnz, s = 1.5, cap 200000.) */
int tca_gen_zipf_rows(int32_t M, int32_t K, int64_t total_nnz, double s, int32_t cap,
                      uint64_t seed, int32_t dtype, tca_csr* out, tca_gen_stats* st);

/* The five benchmark configurations (index 0..4) at full size with their GPU
 * value types (config 0: fp16 by default like the reference harness types).
 * dtype < 0 selects the config's own type.  *N receives the dense width. */
int tca_gen_config(int32_t cfg, uint64_t seed, int32_t dtype, tca_csr* out, int32_t* N,
                   tca_gen_stats* st);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* TCA_HOST_H */
