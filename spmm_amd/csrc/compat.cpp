// compat.cpp -- the reference-named C++ surface (include/tca_compat.hpp) on
// top of the C ABI.  Failures print and exit like the reference's CHECK_CUDA.
#include "../../include/tca_compat.hpp"

#include <atomic>
#include <cstring>
#include <iterator>
#include <string>
#include <vector>

#include "common.hpp"

namespace {

[[noreturn]] void die(const char* what) {
    std::fprintf(stderr, "%s: %s\n", what, tca_last_error());
    std::exit(EXIT_FAILURE);
}

void check(int st, const char* what) {
    if (st != TCA_OK) die(what);
}

// Moves a library-allocated tca_csr (fp16 values) into a malloc'ed CSR.
CSR* to_csr(tca_csr* s) {
    CSR* c = static_cast<CSR*>(std::malloc(sizeof(CSR)));
    if (!c) die("CSR allocation");
    c->nRow = s->nRow;
    c->nCol = s->nCol;
    c->nnz = s->nnz;
    c->row_offset = s->row_offset;
    c->col_idx = s->col_idx;
    c->value = static_cast<half*>(s->value);
    return c;
}

tca_csr view(const CSR* c) {
    tca_csr s;
    s.nRow = c->nRow;
    s.nCol = c->nCol;
    s.nnz = c->nnz;
    s.row_offset = c->row_offset;
    s.col_idx = c->col_idx;
    s.value = c->value;
    s.dtype = TCA_F16;
    return s;
}

// Reads an open stream into memory and hands it to the stream parser.
std::string slurp(std::ifstream& fin) {
    return std::string(std::istreambuf_iterator<char>(fin), std::istreambuf_iterator<char>());
}

std::atomic<uint64_t> g_seed{1};

}  // namespace

void set_prepare_seed(uint64_t seed) { g_seed.store(seed); }
uint64_t prepare_seed_next() { return g_seed.fetch_add(1); }

void convert_dense_to_csr(half* mat, CSR** descr, int nRow, int nCol) {
    tca_csr s{};
    check(tca_dense_to_csr(mat, nRow, nCol, TCA_F16, &s), "convert_dense_to_csr");
    *descr = to_csr(&s);
}

void convert_csr_to_dense(CSR* descr, half** mat) {
    *mat = static_cast<half*>(std::malloc(sizeof(half) * static_cast<size_t>(descr->nRow) * descr->nCol + 2));
    if (!*mat) die("convert_csr_to_dense");
    tca_csr s = view(descr);
    check(tca_csr_to_dense(&s, *mat), "convert_csr_to_dense");
}

void destroy_csr(CSR* descr) {
    if (!descr) return;
    std::free(descr->col_idx);
    std::free(descr->row_offset);
    std::free(descr->value);
    std::free(descr);
}

void csr_to_coo(CSR* a, COO** out) {
    tca_csr s = view(a);
    tca_coo o{};
    check(tca_csr_to_coo(&s, &o), "csr_to_coo");
    *out = static_cast<COO*>(std::malloc(sizeof(COO)));
    if (!*out) die("COO allocation");
    (*out)->nRow = o.nRow;
    (*out)->nCol = o.nCol;
    (*out)->nnz = o.nnz;
    (*out)->row_idx = o.row_idx;
    (*out)->col_idx = o.col_idx;
    (*out)->value = static_cast<half*>(o.value);
}

void coo_to_csr(COO* a, CSR** out) {
    tca_coo s{a->nRow, a->nCol, a->nnz, a->row_idx, a->col_idx, a->value, TCA_F16};
    tca_csr o{};
    check(tca_coo_to_csr(&s, &o), "coo_to_csr");
    *out = to_csr(&o);
}

void destroy_coo(COO* a) {
    if (!a) return;
    std::free(a->row_idx);
    std::free(a->col_idx);
    std::free(a->value);
    std::free(a);
}

void naive_gemm(half* A, half* B, float* C, int M, int N, int K) {
    check(tca_naive_gemm(A, B, C, M, N, K, TCA_F16), "naive_gemm");
}

void smtx_input_to_Dense(std::ifstream& fin, half** mat, char* filename, int* nRow, int* nCol, int* nnz) {
    std::string text = slurp(fin);
    FILE* f = fmemopen(text.empty() ? nullptr : &text[0], text.size(), "rb");
    if (!f) {
        std::fprintf(stderr, "smtx_input_to_Dense: cannot read input stream\n");
        std::exit(EXIT_FAILURE);
    }
    void* d = nullptr;
    int32_t m = 0, k = 0, z = 0;
    const int st = tca::smtx_read_dense_file(f, filename ? filename : "<stream>", TCA_F16, &d, &m, &k, &z);
    std::fclose(f);
    check(st, "smtx_input_to_Dense");
    *mat = static_cast<half*>(d);
    *nRow = m;
    *nCol = k;
    *nnz = z;
}

void smtx_input_to_CSR(std::ifstream& fin, CSR** csr_mat, const char* filename) {
    std::string text = slurp(fin);
    FILE* f = fmemopen(text.empty() ? nullptr : &text[0], text.size(), "rb");
    if (!f) {
        std::fprintf(stderr, "smtx_input_to_CSR: cannot read input stream\n");
        std::exit(EXIT_FAILURE);
    }
    tca_csr s{};
    const int st = tca::smtx_read_csr_file(f, filename ? filename : "<stream>", TCA_F16, &s);
    std::fclose(f);
    check(st, "smtx_input_to_CSR");
    *csr_mat = to_csr(&s);
}

void smtx_input_to_CSR(std::ifstream& fin, CSR** csr_mat, Arguments* arg) {
    (void)arg;
    smtx_input_to_CSR(fin, csr_mat, static_cast<const char*>(nullptr));
}

void mtx_input_to_CSR(std::ifstream& fin, CSR** csr_mat, Arguments* arg) {
    if (!arg) {
        std::fprintf(stderr, "mtx_input_to_CSR: Arguments is NULL\n");
        std::exit(EXIT_FAILURE);
    }
    std::string text = slurp(fin);
    FILE* f = fmemopen(text.empty() ? nullptr : &text[0], text.size(), "rb");
    if (!f) {
        std::fprintf(stderr, "mtx_input_to_CSR: cannot read input stream\n");
        std::exit(EXIT_FAILURE);
    }
    tca_csr s{};
    const int st = tca::mtx_read_csr_file(f, "<stream>", arg->pattern_only, arg->input_is_zero_based, TCA_F16, true, &s);
    std::fclose(f);
    check(st, "mtx_input_to_CSR");
    *csr_mat = to_csr(&s);
}

void mtx_input_to_Dense(std::ifstream& fin, half** mat, Arguments* arg) {
    if (!arg) {
        std::fprintf(stderr, "mtx_input_to_Dense: Arguments is NULL\n");
        std::exit(EXIT_FAILURE);
    }
    std::string text = slurp(fin);
    FILE* f = fmemopen(text.empty() ? nullptr : &text[0], text.size(), "rb");
    if (!f) {
        std::fprintf(stderr, "mtx_input_to_Dense: cannot read input stream\n");
        std::exit(EXIT_FAILURE);
    }
    void* d = nullptr;
    int32_t m = 0, k = 0, z = 0;
    const int st = tca::mtx_read_dense_file(f, "<stream>", arg->input_is_zero_based, TCA_F16, &d, &m, &k, &z);
    std::fclose(f);
    check(st, "mtx_input_to_Dense");
    *mat = static_cast<half*>(d);
}

void mtx_input_to_CSR(const char* filename, CSR** csr_mat, bool pattern_only, bool zero_based) {
    tca_csr s{};
    check(tca_mtx_read_csr(filename, pattern_only, zero_based, TCA_F16, &s), "mtx_input_to_CSR");
    *csr_mat = to_csr(&s);
}

void our_spmm_balanced(CSR* A_csr, half* B, float* C, int M, int N, int K, int n_iter, double* elapsed) {
    if (A_csr->nRow != M || A_csr->nCol != K) {
        std::fprintf(stderr, "our_spmm_balanced: CSR is %d x %d, expected M x K = %d x %d\n", A_csr->nRow,
                     A_csr->nCol, M, K);
        std::exit(EXIT_FAILURE);
    }
    double ms = 0.0;
    check(tca_spmm_host(A_csr->row_offset, A_csr->col_idx, A_csr->value, M, K, A_csr->nnz, B, C, N, TCA_F16, n_iter,
                        1, &ms),
          "our_spmm_balanced");
    if (elapsed) *elapsed = ms;
}

void warm_up_gpu() { check(tca_warm_up(), "warm_up_gpu"); }
