// compat_formats.cpp -- host-only check of the reference-named format
// helpers in tca_compat.hpp (convert_dense_to_csr, csr_to_coo, coo_to_csr,
// convert_csr_to_dense), used by the CPU test suite; touches no GPU.
//   ./compat_formats        round trips and unsorted COO input; prints
//                           "compat formats ok" and exits 0 on success
//   ./compat_formats dup    a duplicate COO entry: coo_to_csr must exit
//   ./compat_formats range  an out-of-range COO entry: coo_to_csr must exit
//   ./compat_formats mtx FILE PATTERN ZERO_BASED
//                           mtx_input_to_CSR(ifstream&, CSR**, Arguments*):
//                           prints "nRow nCol nnz", then the row offsets, the
//                           column indices and the values (as floats), one
//                           line each
//   ./compat_formats mtxdense FILE ZERO_BASED M K
//                           mtx_input_to_Dense(ifstream&, half**, Arguments*):
//                           prints the M x K values row by row
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <vector>

#include "../../../include/tca_compat.hpp"

namespace {

int fail(const char* what) {
    std::printf("compat formats: %s\n", what);
    return EXIT_FAILURE;
}

COO* make_coo(int nrow, int ncol, const std::vector<int>& r, const std::vector<int>& c) {
    COO* a = static_cast<COO*>(std::malloc(sizeof(COO)));
    a->nRow = nrow;
    a->nCol = ncol;
    a->nnz = static_cast<int>(r.size());
    a->row_idx = static_cast<int*>(std::malloc(sizeof(int) * (r.size() + 1)));
    a->col_idx = static_cast<int*>(std::malloc(sizeof(int) * (r.size() + 1)));
    a->value = static_cast<half*>(std::malloc(sizeof(half) * (r.size() + 1)));
    for (size_t i = 0; i < r.size(); i++) {
        a->row_idx[i] = r[i];
        a->col_idx[i] = c[i];
        a->value[i] = static_cast<half>(static_cast<float>(i + 1));
    }
    return a;
}

}  // namespace

int main(int argc, char* argv[]) {
    if (argc == 5 && std::strcmp(argv[1], "mtx") == 0) {
        Arguments arg;
        arg.pattern_only = std::atoi(argv[3]) != 0;
        arg.input_is_zero_based = std::atoi(argv[4]) != 0;
        std::ifstream fin(argv[2]);
        CSR* a = nullptr;
        mtx_input_to_CSR(fin, &a, &arg);
        std::printf("%d %d %d\n", a->nRow, a->nCol, a->nnz);
        for (int r = 0; r <= a->nRow; r++) std::printf("%d ", a->row_offset[r]);
        std::printf("\n");
        for (int j = 0; j < a->nnz; j++) std::printf("%d ", a->col_idx[j]);
        std::printf("\n");
        for (int j = 0; j < a->nnz; j++) std::printf("%.9g ", static_cast<float>(a->value[j]));
        std::printf("\n");
        destroy_csr(a);
        return EXIT_SUCCESS;
    }
    if (argc == 6 && std::strcmp(argv[1], "mtxdense") == 0) {
        Arguments arg;
        arg.input_is_zero_based = std::atoi(argv[3]) != 0;
        const int M = std::atoi(argv[4]), K = std::atoi(argv[5]);
        std::ifstream fin(argv[2]);
        half* d = nullptr;
        mtx_input_to_Dense(fin, &d, &arg);
        for (int i = 0; i < M * K; i++) std::printf("%.9g ", static_cast<float>(d[i]));
        std::printf("\n");
        std::free(d);
        return EXIT_SUCCESS;
    }
    if (argc > 1) {  // rejection cases: coo_to_csr prints and exits
        const bool dup = std::strcmp(argv[1], "dup") == 0;
        COO* a = dup ? make_coo(3, 4, {0, 2, 0}, {1, 3, 1}) : make_coo(3, 4, {0, 2}, {1, 4});
        CSR* out = nullptr;
        coo_to_csr(a, &out);
        std::printf("coo_to_csr accepted an invalid matrix\n");
        return EXIT_SUCCESS;  // the test expects a failure exit
    }
    // dense -> CSR -> COO -> CSR -> dense
    const int M = 7, K = 9;
    std::vector<half> dense(M * K, static_cast<half>(0.0f));
    int nz = 0;
    for (int r = 0; r < M; r++)
        for (int c = 0; c < K; c++)
            if ((r * 5 + c * 3) % 4 == 0 && r != 3) dense[r * K + c] = static_cast<half>(static_cast<float>(++nz));
    CSR* csrA;
    convert_dense_to_csr(dense.data(), &csrA, M, K);
    if (csrA->nnz != nz) return fail("dense -> CSR nnz");
    COO* coo;
    csr_to_coo(csrA, &coo);
    for (int r = 0; r < M; r++)
        for (int j = csrA->row_offset[r]; j < csrA->row_offset[r + 1]; j++)
            if (coo->row_idx[j] != r || coo->col_idx[j] != csrA->col_idx[j]) return fail("CSR -> COO entries");
    // reverse the entry order: coo_to_csr sorts rows, then columns
    for (int i = 0, j = coo->nnz - 1; i < j; i++, j--) {
        std::swap(coo->row_idx[i], coo->row_idx[j]);
        std::swap(coo->col_idx[i], coo->col_idx[j]);
        std::swap(coo->value[i], coo->value[j]);
    }
    CSR* csrB;
    coo_to_csr(coo, &csrB);
    if (csrB->nnz != csrA->nnz ||
        std::memcmp(csrB->row_offset, csrA->row_offset, sizeof(int) * (M + 1)) != 0 ||
        std::memcmp(csrB->col_idx, csrA->col_idx, sizeof(int) * csrA->nnz) != 0 ||
        std::memcmp(csrB->value, csrA->value, sizeof(half) * csrA->nnz) != 0)
        return fail("COO -> CSR differs from the dense path");
    half* back;
    convert_csr_to_dense(csrB, &back);
    if (std::memcmp(back, dense.data(), sizeof(half) * M * K) != 0) return fail("CSR -> dense round trip");
    std::free(back);
    destroy_coo(coo);
    destroy_csr(csrA);
    destroy_csr(csrB);
    std::printf("compat formats ok (%d entries)\n", nz);
    return EXIT_SUCCESS;
}
