// test.cpp -- the ./test harness: read or synthesise A, make B, run the
// MI355X SpMM, validate against the CPU gold, print timings.
//
// Flow of reference main (src/test.cu:29-88) without the cuBLAS GemmEx gold
// and the cuSPARSE baseline: the gold is the CPU CSR product with
// naive_gemm's arithmetic (fp32 multiply then add, k ascending).  Output
// lines follow the reference ("Input file - ...", "preprocess ...",
// "num_block: ...", "our: [x] ms", the magenta "validation failed (Our,
// balanced)").  Unlike the reference, the exit status is 1 when validation
// fails.
#include <chrono>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../../include/tca_compat.hpp"
#include "../../../include/tca_arguments.hpp"

namespace {

void die(const char* what) {
    std::fprintf(stderr, "%s: %s\n", what, tca_last_error());
    std::exit(EXIT_FAILURE);
}

bool ends_with(const std::string& s, const char* suf) {
    const size_t n = std::strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

}  // namespace

int main(int argc, char* argv[]) {
    if (argc <= 1) {
        std::puts("Usage : ./test {matrix.smtx}");
        return EXIT_FAILURE;
    }
    Arguments arg(argc, argv);
    const int dt = arg.dtype;
    const size_t es = dt == TCA_F32 ? 4 : 2;

    // A as CSR, values in the requested type.
    tca_csr A{};
    if (arg.input_file_exists) {
        int st;
        if (ends_with(arg.input_fname, ".mtx"))
            st = tca_mtx_read_csr(arg.input_fname.c_str(), arg.pattern_only, arg.input_is_zero_based, dt, &A);
        else
            st = tca_smtx_read_csr(arg.input_fname.c_str(), dt, &A);
        if (st) die("reading the input matrix");
        std::printf("Input file - %s\n", arg.input_fname.c_str());
    } else {
        // synthetic A: reference prepare_cpu_matrix semantics, seeded, then CSR
        std::vector<char> dense(es * static_cast<size_t>(arg.M) * arg.K);
        if (tca_gen_dense(arg.M, arg.K, 3, arg.target_sparsity, arg.seed + 1000, dt, dense.data())) die("generating A");
        if (tca_dense_to_csr(dense.data(), arg.M, arg.K, dt, &A)) die("converting A");
        std::printf("Synthetic A - %d x %d, sparsity %.3f, nnz %d\n", arg.M, arg.K, arg.target_sparsity, A.nnz);
    }
    const int M = A.nRow, K = A.nCol, N = arg.N;

    for (int i = 0; i < 10; i++)
        if (tca_warm_up()) die("warm-up");

    // B: U(0,1) with 10% zeros, as the reference harness (src/test.cu:56), seeded.
    std::vector<char> B(es * static_cast<size_t>(K) * N);
    if (tca_gen_dense(K, N, 3, 0.1f, arg.seed, dt, B.data())) die("generating B");
    std::vector<float> C_gold(static_cast<size_t>(M) * N, 0.f), C(static_cast<size_t>(M) * N, 0.f);

    auto t0 = std::chrono::steady_clock::now();
    if (tca_naive_csr_spmm(&A, B.data(), C_gold.data(), N, 0)) die("CPU gold");
    const double gold_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();

    double e_our = -1.0;
    if (tca_spmm_host(A.row_offset, A.col_idx, A.value, M, K, A.nnz, B.data(), C.data(), N, dt, arg.num_iter, 1,
                      &e_our))
        die("our_spmm_balanced");

    tca_compare_result res{};
    if (tca_compare_mat(C_gold.data(), C.data(), static_cast<int64_t>(M) * N, arg.tolerance, 1e-2f, 1, &res))
        die("compare_mat");
    if (!res.success) std::printf("\033[35mvalidation failed (Our, balanced)\033[0m\n");

    std::fprintf(stdout, "CPU gold: \033[36m[%lf] ms\033[0m \n", gold_ms);
    std::fprintf(stdout, "our: \033[36m[%lf] ms\033[0m \n", e_our);
    if (arg.json) {
        const double gflops = 2.0 * A.nnz * N / (e_our * 1e-3) / 1e9;
        const double bytes = 4.0 * (M + 1) + A.nnz * (4.0 + es) + static_cast<double>(K) * N * es + 4.0 * M * N;
        std::printf(
            "{\"M\": %d, \"K\": %d, \"N\": %d, \"nnz\": %d, \"dtype\": %d, \"ms\": %.6f, \"gflops\": %.3f, "
            "\"gbs\": %.3f, \"roofline_frac\": %.5f, \"valid\": %s, \"max_rel_err\": %.3e}\n",
            M, K, N, A.nnz, dt, e_our, gflops, bytes / (e_our * 1e-3) / 1e9, bytes / (e_our * 1e-3) / 8e12,
            res.success ? "true" : "false", res.max_rel_floor);
    }
    tca_csr_free(&A);
    return res.success ? EXIT_SUCCESS : EXIT_FAILURE;
}
