/*
 * oracle.c -- CPU restatement of the reference TCA-SpMM path (YaoLingF/SPMM).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (spmm_amd/, include/, the
 * ./test harness) links or calls this file.  Only tests/, the smoke check of
 * __graft_entry__.py and the cpu_baseline leg of bench.py may load it, and
 * only as the checker (or the timed CPU baseline), never as the thing measured.
 *
 * Parity pins (each function is checked against something other than itself):
 *   oracle_csr_spmm_f32   -- exact-arithmetic vectors (bit equality with an
 *                            fp64 closed form), identity / permutation /
 *                            all-ones closed forms, scipy csr @ B fixtures,
 *                            dense fp64 brute force on tiny inputs.
 *   oracle_dense_spmm_f32 -- the same vectors, and equality with
 *                            oracle_csr_spmm_f32 (skipped terms are +-0).
 *   oracle_compare_mat    -- hand-built cases for every branch of the verdict.
 * The .smtx parser, dense<->CSR conversion and the condensed-window indexing
 * are restated in oracle.py (numpy) and pinned there.
 *
 * Build: see oracle/Makefile (gcc -O3 -fopenmp -ffp-contract=off).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <omp.h>

/* C[r, :] = sum_j val[j] * B[col[j], :] for j in row r, j ascending, fp32
 * multiply then fp32 add (no contraction).  Follows the arithmetic of
 * reference naive_gemm (src/miscalleneous.cu:114-134): `result +=
 * A[m,k] * B[k,n]` with k ascending in fp32; over CSR the skipped k are those
 * with A[m,k] == +-0, whose products are +-0 and leave a finite sum unchanged.
 * Rows with no entries produce 0 (beta = 0).  Rows are split over
 * `threads` OpenMP threads (<= 0: all). */
void oracle_csr_spmm_f32(const int32_t* rowptr, const int32_t* colidx, const float* val,
                         int32_t M, int32_t N, const float* B, float* C, int threads)
{
    if (threads <= 0) threads = omp_get_max_threads();
    int64_t m;
#pragma omp parallel for schedule(dynamic, 64) num_threads(threads)
    for (m = 0; m < M; m++) {
        float* crow = C + (size_t)m * N;
        for (int32_t n = 0; n < N; n++) crow[n] = 0.0f;
        for (int32_t j = rowptr[m]; j < rowptr[m + 1]; j++) {
            const float a = val[j];
            const float* brow = B + (size_t)colidx[j] * N;
            for (int32_t n = 0; n < N; n++) {
                float p = a * brow[n];
                crow[n] = crow[n] + p;
            }
        }
    }
}

/* Same product accumulated in fp64 (for error measurement only). */
void oracle_csr_spmm_f64(const int32_t* rowptr, const int32_t* colidx, const double* val,
                         int32_t M, int32_t N, const double* B, double* C, int threads)
{
    if (threads <= 0) threads = omp_get_max_threads();
    int64_t m;
#pragma omp parallel for schedule(dynamic, 64) num_threads(threads)
    for (m = 0; m < M; m++) {
        double* crow = C + (size_t)m * N;
        for (int32_t n = 0; n < N; n++) crow[n] = 0.0;
        for (int32_t j = rowptr[m]; j < rowptr[m + 1]; j++) {
            const double a = val[j];
            const double* brow = B + (size_t)colidx[j] * N;
            for (int32_t n = 0; n < N; n++) crow[n] += a * brow[n];
        }
    }
}

/* Literal restatement of reference naive_gemm (src/miscalleneous.cu:114-134)
 * over fp32 copies of the half inputs: dense A[M*K], B[K*N], k ascending. */
void oracle_dense_spmm_f32(const float* A, const float* B, float* C, int32_t M, int32_t N,
                           int32_t K, int threads)
{
    if (threads <= 0) threads = omp_get_max_threads();
    int64_t m;
#pragma omp parallel for num_threads(threads)
    for (m = 0; m < M; m++) {
        for (int32_t n = 0; n < N; n++) {
            float result = 0.0f;
            for (int32_t k = 0; k < K; k++) {
                float p = A[(size_t)m * K + k] * B[(size_t)k * N + n];
                result = result + p;
            }
            C[(size_t)m * N + n] = result;
        }
    }
}

/* Restatement of reference compare_mat<float> (src/general.cuh:71-123).
 * Element i fails iff |g - c| / |g| >= tol AND |g - c| >= tol, both in fp32.
 * The scan stops at the 10th failure (src/general.cuh:108-114).
 * Outputs: *fail_count (failures seen before stopping), *first_fail (index of
 * the first failure or -1), *max_rel (running max of the relative
 * discrepancy over the scanned prefix; NaN relative values, from 0/0, are
 * ignored as fmaxf ignores them).  Returns 1 on success, 0 on failure. */
int oracle_compare_mat(const float* gold, const float* cmp, int64_t n, float tol,
                       int64_t* fail_count, int64_t* first_fail, float* max_rel)
{
    int success = 1;
    int64_t count = 0;
    float max_disc = 0.0f;
    *first_fail = -1;
    for (int64_t i = 0; i < n; i++) {
        float v1 = gold[i];
        float v2 = cmp[i];
        float disc = fabsf(v1 - v2);
        float rel_disc = fabsf(disc / v1);
        max_disc = fmaxf(rel_disc, max_disc);
        if (rel_disc >= tol && disc >= tol) {
            success = 0;
            if (*first_fail < 0) *first_fail = i;
            count++;
            if (count >= 10) break;
        }
    }
    *fail_count = count;
    *max_rel = max_disc;
    return success;
}
