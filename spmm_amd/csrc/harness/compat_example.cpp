// compat_example.cpp -- the reference harness flow (src/test.cu:38-78)
// written only against the reference-named API in tca_compat.hpp, as code
// that used the reference's headers would be: .smtx -> dense -> CSR, seeded
// B, dense CPU gold (naive_gemm in place of cuBLAS GemmEx), our_spmm_balanced,
// compare_mat.  Exit status 0 when validation passes.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>

#include "../../../include/tca_compat.hpp"

int main(int argc, char* argv[]) {
    if (argc <= 1) {
        std::puts("Usage : ./compat_example {matrix.smtx} [N]");
        return EXIT_FAILURE;
    }
    std::ifstream fin;
    fin.open(argv[1], std::ifstream::in);
    half *A, *B;
    float *C_gold, *C_our;
    int M, K, nnz;
    smtx_input_to_Dense(fin, &A, argv[1], &M, &K, &nnz);
    const int N = argc > 2 ? std::atoi(argv[2]) : 256;
    warm_up_gpu();
    std::printf("Input file - %s\n", argv[1]);
    set_prepare_seed(1);
    prepare_cpu_matrix(&B, K, N, 0.1);
    prepare_cpu_matrix(&C_gold, M, N, 1, true);
    prepare_cpu_matrix(&C_our, M, N, 1, true);
    naive_gemm(A, B, C_gold, M, N, K);

    CSR* csrA;
    convert_dense_to_csr(A, &csrA, M, K);
    if (csrA->nnz != nnz) std::printf("note: file lists %d entries, CSR has %d\n", nnz, csrA->nnz);
    double e_our = -1.0;
    our_spmm_balanced(csrA, B, C_our, M, N, K, 10, &e_our);
    const bool ok = compare_mat(C_gold, C_our, M * N, DEFAULT_TOL);
    if (!ok) std::printf("\033[35mvalidation failed (Our, balanced)\033[0m\n");

    // the direct .smtx -> CSR reader gives the same matrix
    std::ifstream fin2(argv[1]);
    CSR* csrB;
    smtx_input_to_CSR(fin2, &csrB, argv[1]);
    const bool same = csrB->nnz == csrA->nnz &&
                      std::memcmp(csrB->row_offset, csrA->row_offset, sizeof(int) * (M + 1)) == 0 &&
                      std::memcmp(csrB->col_idx, csrA->col_idx, sizeof(int) * csrA->nnz) == 0;
    if (!same) std::printf("smtx_input_to_CSR differs from the dense path\n");

    destroy_csr(csrA);
    destroy_csr(csrB);
    std::free(A);
    std::free(B);
    std::free(C_gold);
    std::free(C_our);
    std::fprintf(stdout, "our: \033[36m[%lf] ms\033[0m \n", e_our);
    return ok && same ? EXIT_SUCCESS : EXIT_FAILURE;
}
