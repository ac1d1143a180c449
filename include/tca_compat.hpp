// tca_compat.hpp -- C++ source-compatibility surface for code written against
// the reference YaoLingF/SPMM (TCA-SpMM) headers.  Same names, argument
// meaning and error behaviour as the reference, implemented on libtcaspmm.so
// (link with -ltcaspmm, compile with hipcc for the `half` type).
//
//   reference                                  here
//   struct CSR            src/general.cuh:125   struct CSR (identical layout)
//   entry_dtype           src/general.cuh:54    entry_dtype
//   mat_format            src/mat_format.cuh:10 mat_format (+ struct COO, new)
//   compare_mat<T>        src/general.cuh:71    compare_mat<T>
//   prepare_cpu_matrix<T> src/general.cuh:140   prepare_cpu_matrix<T> (seeded)
//   convert_dense_to_csr  src/miscalleneous.cu:29
//   convert_csr_to_dense  src/miscalleneous.cu:66
//   destroy_csr           src/miscalleneous.cu:82
//   naive_gemm            src/miscalleneous.cu:114
//   Arguments             src/arg_parse.h:15    Arguments (tca_arguments.hpp)
//   smtx_input_to_Dense   src/file_input.cu:135
//   smtx_input_to_CSR     src/file_input.cu:194 (an empty stub there; implemented here)
//   mtx_input_to_CSR      src/file_input.cu:63  (reference signature and CSR order)
//   mtx_input_to_Dense    src/file_input.cu:8
//   our_spmm_balanced     src/our_spmm.cuh:4, src/our_spmm.cu:478
//
// Errors: like the reference's CHECK_CUDA (src/general.cuh:8-16), these
// functions print the failure to stderr and exit(EXIT_FAILURE).  Use the C
// ABI (tca_spmm.h, tca_host.h) for status codes instead.
#pragma once

#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>

#include "tca_arguments.hpp"
#include "tca_host.h"
#include "tca_spmm.h"

typedef struct CSR {
    int nRow;
    int nCol;
    int nnz;
    int* row_offset;
    int* col_idx;
    half* value;
} CSR;

// Coordinate container; the reference names the format only (mat_format::coo).
typedef struct COO {
    int nRow;
    int nCol;
    int nnz;
    int* row_idx;
    int* col_idx;
    half* value;
} COO;

typedef enum entry_dtype { fp16, fp32, fp64 } entry_dtype;
typedef enum _mat_format { dense, csr, coo } mat_format;

#define DEFAULT_TOL 1e-3
#define N_ITER 10

// Dense (row-major) half matrix -> CSR, dropping +-0 (allocates *descr).
void convert_dense_to_csr(half* mat, CSR** descr, int nRow, int nCol);
// CSR -> dense (allocates *mat, nRow * nCol halves).
void convert_csr_to_dense(CSR* descr, half** mat);
void destroy_csr(CSR* descr);
void csr_to_coo(CSR* a, COO** out);
void coo_to_csr(COO* a, CSR** out);
void destroy_coo(COO* a);

// Dense CPU GEMM, fp32 multiply-then-add, k ascending.
void naive_gemm(half* A, half* B, float* C, int M, int N, int K);

// .smtx -> dense nRow x nCol halves with 1.0 at every listed entry; reads
// `fin` (filename only labels errors).
void smtx_input_to_Dense(std::ifstream& fin, half** mat, char* filename, int* nRow, int* nCol, int* nnz);
// .smtx -> CSR directly (no dense intermediate), values 1.0.
void smtx_input_to_CSR(std::ifstream& fin, CSR** csr_mat, const char* filename = nullptr);
// The reference's signature of the same (arg is not consulted: .smtx has no options).
void smtx_input_to_CSR(std::ifstream& fin, CSR** csr_mat, Arguments* arg);
// MatrixMarket coordinate -> CSR with the reference's signature and result
// (src/file_input.cu:63-134): arg->pattern_only (values 1.0, else a missing
// value is 0), arg->input_is_zero_based; rows ascending, each row's entries
// in file order, duplicates kept (tca_mtx_read_csr_file_order).
void mtx_input_to_CSR(std::ifstream& fin, CSR** csr_mat, Arguments* arg);
// MatrixMarket coordinate -> dense nRow x nCol halves, reference signature
// and result (src/file_input.cu:8-62): a value read on every line (1.0 when
// missing), a later duplicate overwriting an earlier one; the dimensions are
// not returned (as in the reference).
void mtx_input_to_Dense(std::ifstream& fin, half** mat, Arguments* arg);
// From a path: CSR sorted by (row, col), duplicates rejected (tca_mtx_read_csr).
void mtx_input_to_CSR(const char* filename, CSR** csr_mat, bool pattern_only, bool zero_based);

// C = A * B on the GPU for host pointers; *elapsed = mean ms of n_iter
// launches after 5 warm-ups.  Prints "preprocess %fms taken" and
// "num_block: %d blockdim: %d shm: %fKB" like the reference.
void our_spmm_balanced(CSR* A_csr, half* B, float* C, int M, int N, int K, int n_iter, double* elapsed = nullptr);

// Seed of prepare_cpu_matrix (the reference used std::random_device).
void set_prepare_seed(uint64_t seed);
uint64_t prepare_seed_next();

// Random dense matrix: U(0,1) with probability 1 - target_sparsity, else 0
// (reference semantics, src/general.cuh:156-166), seeded; zeros when leave_empty.
template <typename T>
void prepare_cpu_matrix(T** mat, size_t nRow, size_t nCol, float target_sparsity, bool leave_empty = false) {
    *mat = static_cast<T*>(std::malloc(sizeof(T) * nRow * nCol));
    if (!*mat) {
        std::fprintf(stderr, "prepare_cpu_matrix: allocation failed\n");
        std::exit(EXIT_FAILURE);
    }
    if (leave_empty) {
        std::memset(*mat, 0, sizeof(T) * nRow * nCol);
        return;
    }
    const int32_t dt = sizeof(T) == 4 ? TCA_F32 : TCA_F16;
    const int st = tca_gen_dense(static_cast<int64_t>(nRow), static_cast<int64_t>(nCol), 3, target_sparsity,
                                 prepare_seed_next(), dt, *mat);
    if (st) {
        std::fprintf(stderr, "prepare_cpu_matrix: %s\n", tca_last_error());
        std::exit(EXIT_FAILURE);
    }
}

// Reference verdict: element i fails iff |g-c|/|g| >= tol and |g-c| >= tol;
// prints each failure, stops at the 10th.  Returns true when none failed.
template <typename T>
bool compare_mat(T* gold, T* comparing, int num_elem, float tolerance) {
    float* g = static_cast<float*>(std::malloc(sizeof(float) * (num_elem > 0 ? num_elem : 1)));
    float* c = static_cast<float*>(std::malloc(sizeof(float) * (num_elem > 0 ? num_elem : 1)));
    for (int i = 0; i < num_elem; i++) {
        g[i] = static_cast<float>(gold[i]);
        c[i] = static_cast<float>(comparing[i]);
    }
    tca_compare_result r;
    const int st = tca_compare_mat(g, c, num_elem, tolerance, 1e-6f, 1, &r);
    std::free(g);
    std::free(c);
    if (st) {
        std::fprintf(stderr, "compare_mat: %s\n", tca_last_error());
        std::exit(EXIT_FAILURE);
    }
    return r.success != 0;
}

// Trivial kernel launch that initialises the device (reference warm_up_gpu_kernel).
void warm_up_gpu();
