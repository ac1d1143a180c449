// host_sanitize.cpp -- the host library under AddressSanitizer and
// UndefinedBehaviorSanitizer (built by `make sanitize` from the host sources
// with g++ -fsanitize=address,undefined; no GPU, no HIP runtime).  Used by
// the CPU test suite:
//   ./host_sanitize CORPUS_DIR
// 1. every file reader on every file of CORPUS_DIR and on deterministic
//    mutations of it (bytes flipped, lines cut, digits inserted, truncation):
//    each call returns a status, results are freed;
// 2. generators, conversions, the CPU products and the host planners on
//    generated matrices (exercises their index arithmetic);
// 3. allocation-failure injection: each operation again with its n-th host
//    allocation failing (tca_debug_fail_allocs), n = 0, 1, ... until it
//    succeeds; every run must return TCA_OK or TCA_ERR_ALLOC and free what it
//    allocated (LeakSanitizer checks at exit);
// 4. a std::bad_alloc inside an entry point becomes TCA_ERR_ALLOC.
// Prints "host sanitize ok: ..." and exits 0; any sanitizer report exits
// non-zero (halt_on_error).
#include <dirent.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <new>
#include <string>
#include <vector>

#include "../../../include/tca_host.h"
#include "../../../include/tca_spmm.h"
#include "../common.hpp"

namespace {

long g_calls = 0;

std::string slurp(const std::string& path) {
    std::string s;
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return s;
    char buf[1 << 14];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) s.append(buf, n);
    std::fclose(f);
    return s;
}

void spit(const std::string& path, const std::string& s) {
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) {
        std::fprintf(stderr, "cannot write %s\n", path.c_str());
        std::exit(2);
    }
    std::fwrite(s.data(), 1, s.size(), f);
    std::fclose(f);
}

void check_status(int st, const char* what) {
    g_calls++;
    if (st < 0 || st > TCA_ERR_FORMAT) {
        std::fprintf(stderr, "%s: status %d outside the tca_status range\n", what, st);
        std::exit(3);
    }
}

// Every reader on one file; results freed.
void read_all(const std::string& path, const std::string& values_path) {
    for (int dt : {TCA_F16, TCA_F32}) {
        tca_csr a{};
        int st = tca_smtx_read_csr(path.c_str(), dt, &a);
        check_status(st, "tca_smtx_read_csr");
        if (!st) tca_csr_free(&a);
        void* d = nullptr;
        int32_t m = 0, k = 0, z = 0;
        st = tca_smtx_read_dense(path.c_str(), dt, &d, &m, &k, &z);
        check_status(st, "tca_smtx_read_dense");
        if (!st) tca_free(d);
        for (int pattern : {0, 1})
            for (int zero : {0, 1}) {
                tca_csr b{};
                st = tca_mtx_read_csr(path.c_str(), pattern, zero, dt, &b);
                check_status(st, "tca_mtx_read_csr");
                if (!st) tca_csr_free(&b);
                tca_csr c{};
                st = tca_mtx_read_csr_file_order(path.c_str(), pattern, zero, dt, &c);
                check_status(st, "tca_mtx_read_csr_file_order");
                if (!st) tca_csr_free(&c);
            }
        d = nullptr;
        st = tca_mtx_read_dense(path.c_str(), 0, dt, &d, &m, &k, &z);
        check_status(st, "tca_mtx_read_dense");
        if (!st) tca_free(d);
        tca_csr e{};
        st = tca_smtx_read_csr_values(path.c_str(), values_path.c_str(), dt, &e);
        check_status(st, "tca_smtx_read_csr_values");
        if (!st) tca_csr_free(&e);
    }
    tca_csr b{};
    const int st = tca_csr_read_binary(path.c_str(), &b);
    check_status(st, "tca_csr_read_binary");
    if (!st) tca_csr_free(&b);
}

// Deterministic mutations of a file's bytes.
std::vector<std::string> mutations(const std::string& s, uint64_t seed) {
    std::vector<std::string> out;
    uint64_t x = seed * 0x9e3779b97f4a7c15ull + 1;
    auto rnd = [&](uint64_t n) {
        x ^= x << 13;
        x ^= x >> 7;
        x ^= x << 17;
        return n ? x % n : 0;
    };
    const size_t n = s.size();
    if (n == 0) return out;
    for (int i = 0; i < 24; i++) {
        std::string t = s;
        switch (i % 6) {
            case 0: t[rnd(n)] = static_cast<char>(rnd(256)); break;                           // one byte
            case 1: t.resize(rnd(n)); break;                                                  // truncated
            case 2: t.insert(rnd(n), std::string(1 + rnd(12), static_cast<char>('0' + rnd(10)))); break;  // digits
            case 3: t.erase(rnd(n), 1 + rnd(40)); break;                                      // a span cut
            case 4: t.insert(rnd(n), "-"); break;                                             // a sign
            default: t.insert(rnd(n), "\n"); break;                                           // a line split
        }
        out.push_back(t);
    }
    return out;
}

// One operation for the injection sweep: returns its status, frees its outputs.
using Op = std::function<int()>;

void sweep(const char* name, const Op& op, long* failures_seen) {
    for (int64_t n = 0;; n++) {
        tca_debug_fail_allocs(n, -1);
        const int st = op();
        tca_debug_fail_allocs(-1, -1);
        check_status(st, name);
        if (st == TCA_OK) return;
        if (st != TCA_ERR_ALLOC) {
            std::fprintf(stderr, "%s: injected failure %lld gave status %d (%s)\n", name, (long long)n, st,
                         tca_last_error());
            std::exit(4);
        }
        (*failures_seen)++;
        if (n > 1000) {
            std::fprintf(stderr, "%s: still failing after %lld injected failures\n", name, (long long)n);
            std::exit(5);
        }
    }
}

}  // namespace

int main(int argc, char* argv[]) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s CORPUS_DIR\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    std::vector<std::string> files;
    if (DIR* d = opendir(dir.c_str())) {
        while (dirent* e = readdir(d))
            if (e->d_name[0] != '.') files.push_back(dir + "/" + e->d_name);
        closedir(d);
    }
    // 1. readers on the corpus and its mutations
    const std::string vals = dir + "/.values.bin";
    const std::string mut = dir + "/.mutant";
    long n_mut = 0;
    for (size_t i = 0; i < files.size(); i++) {
        // a values file sized for a small matrix (wrong for most: exercises the mismatch path)
        const float v[8] = {1, 2, 3, 4, 5, 6, 7, 8};
        tca_values_write(vals.c_str(), v, 8, TCA_F32);
        read_all(files[i], vals);
        const std::string text = slurp(files[i]);
        if (text.size() > (1u << 20)) continue;
        for (const std::string& t : mutations(text, i + 1)) {
            spit(mut, t);
            read_all(mut, vals);
            n_mut++;
        }
    }
    // 2. generators, conversions, products, planners
    tca_csr a{};
    int st = tca_gen_lognormal_rows(300, 200, 20, 1.0, 1.0, 7, TCA_F16, &a, nullptr);
    check_status(st, "tca_gen_lognormal_rows");
    if (st) return 6;
    std::vector<uint16_t> dense(static_cast<size_t>(a.nRow) * a.nCol);
    check_status(tca_csr_to_dense(&a, dense.data()), "tca_csr_to_dense");
    std::vector<uint16_t> b(static_cast<size_t>(a.nCol) * 40);
    check_status(tca_gen_dense(a.nCol, 40, 1, 0.0f, 3, TCA_F16, b.data()), "tca_gen_dense");
    std::vector<float> c1(static_cast<size_t>(a.nRow) * 40), c2(c1.size());
    check_status(tca_naive_gemm(dense.data(), b.data(), c1.data(), a.nRow, 40, a.nCol, TCA_F16), "tca_naive_gemm");
    check_status(tca_naive_csr_spmm(&a, b.data(), c2.data(), 40, 2), "tca_naive_csr_spmm");
    tca_compare_result cr;
    check_status(tca_compare_mat(c1.data(), c2.data(), static_cast<int64_t>(c1.size()), 1e-3f, 1e-6f, 0, &cr),
                 "tca_compare_mat");
    std::vector<int32_t> rpt(a.nCol + 1), cit(a.nnz + 1), perm(a.nnz + 1);
    check_status(tca_csr_transpose(a.row_offset, a.col_idx, a.nRow, a.nCol, a.nnz, rpt.data(), cit.data(), perm.data()),
                 "tca_csr_transpose");
    {
        int32_t eb = 0;
        check_status(tca_csr_to_bell(a.row_offset, a.col_idx, a.value, a.nRow, a.nCol, a.nnz, TCA_F16, 32, &eb,
                                     nullptr, nullptr),
                     "tca_csr_to_bell");
        const int32_t br = (a.nRow + 31) / 32;
        std::vector<int32_t> ci(static_cast<size_t>(br) * eb + 1);
        std::vector<uint16_t> ev(static_cast<size_t>(br) * 32 * eb * 32 + 1);
        check_status(tca_csr_to_bell(a.row_offset, a.col_idx, a.value, a.nRow, a.nCol, a.nnz, TCA_F16, 32, &eb,
                                     ci.data(), ev.data()),
                     "tca_csr_to_bell");
    }
    {
        std::vector<int64_t> uoff(a.nRow / 16 + 2);
        check_status(tca_condense_windows(a.row_offset, a.col_idx, a.nRow, a.nnz, 16, uoff.data(), nullptr, nullptr),
                     "tca_condense_windows");
        const int32_t nw = (a.nRow + 15) / 16;
        std::vector<int32_t> uc(uoff[nw] + 1), cp(a.nnz + 1);
        check_status(tca_condense_windows(a.row_offset, a.col_idx, a.nRow, a.nnz, 16, uoff.data(), uc.data(), cp.data()),
                     "tca_condense_windows");
    }
    for (int32_t n : {8, 64, 256}) {
        int32_t nt = 0, np = 0, nl = 0, geo[8];
        check_status(tca_plan_row_tasks(a.row_offset, a.nRow, a.nCol, n, TCA_F16, &nt, &np, &nl, nullptr, nullptr,
                                        nullptr, geo),
                     "tca_plan_row_tasks");
        std::vector<int32_t> t(4 * static_cast<size_t>(nt) + 4), p(np + 1), l(4 * static_cast<size_t>(nl) + 4);
        check_status(tca_plan_row_tasks(a.row_offset, a.nRow, a.nCol, n, TCA_F16, &nt, &np, &nl, t.data(), p.data(),
                                        l.data(), geo),
                     "tca_plan_row_tasks");
        int32_t nwin = 0, nst = 0;
        int64_t nen = 0;
        check_status(tca_plan_mfma_windows(a.row_offset, a.col_idx, a.nRow, n, TCA_F16, TCA_PLAN_FORCE_MFMA, &nwin,
                                           &nst, &nen, nullptr, nullptr, nullptr, nullptr),
                     "tca_plan_mfma_windows");
        std::vector<int32_t> w(4 * static_cast<size_t>(nwin) + 4), u(32 * static_cast<size_t>(nst) + 32),
            eo(nst + 2);
        std::vector<uint32_t> en(nen + 1);
        check_status(tca_plan_mfma_windows(a.row_offset, a.col_idx, a.nRow, n, TCA_F16, TCA_PLAN_FORCE_MFMA, &nwin,
                                           &nst, &nen, w.data(), u.data(), eo.data(), en.data()),
                     "tca_plan_mfma_windows");
        int64_t sz[16];
        check_status(tca_plan_panels(a.row_offset, a.col_idx, a.nRow, a.nCol, n, TCA_F16,
                                     TCA_PLAN_NO_MFMA | TCA_PLAN_FORCE_PANELS, sz, nullptr, nullptr, nullptr,
                                     nullptr, nullptr, nullptr, nullptr, nullptr, nullptr),
                     "tca_plan_panels");
    }
    // 3. allocation-failure injection
    long injected = 0;
    const std::string smtx = dir + "/.inject.smtx", mtx = dir + "/.inject.mtx";
    tca_smtx_write(smtx.c_str(), &a);
    spit(mtx, "%%MatrixMarket matrix coordinate real general\n4 5 6\n1 1 1.5\n2 3 2\n4 5 -1\n1 2 3\n3 3 4\n2 3 5\n");
    sweep("tca_smtx_read_csr", [&] {
        tca_csr x{};
        const int s = tca_smtx_read_csr(smtx.c_str(), TCA_F16, &x);
        if (!s) tca_csr_free(&x);
        return s;
    }, &injected);
    sweep("tca_smtx_read_dense", [&] {
        void* d = nullptr;
        int32_t m, k, z;
        const int s = tca_smtx_read_dense(smtx.c_str(), TCA_F32, &d, &m, &k, &z);
        if (!s) tca_free(d);
        return s;
    }, &injected);
    sweep("tca_mtx_read_csr_file_order", [&] {
        tca_csr x{};
        const int s = tca_mtx_read_csr_file_order(mtx.c_str(), 0, 0, TCA_F16, &x);
        if (!s) tca_csr_free(&x);
        return s;
    }, &injected);
    sweep("tca_mtx_read_dense", [&] {
        void* d = nullptr;
        int32_t m, k, z;
        const int s = tca_mtx_read_dense(mtx.c_str(), 0, TCA_F16, &d, &m, &k, &z);
        if (!s) tca_free(d);
        return s;
    }, &injected);
    sweep("tca_dense_to_csr", [&] {
        tca_csr x{};
        const int s = tca_dense_to_csr(dense.data(), a.nRow, a.nCol, TCA_F16, &x);
        if (!s) tca_csr_free(&x);
        return s;
    }, &injected);
    sweep("tca_csr_to_coo + tca_coo_to_csr", [&] {
        tca_coo o{};
        int s = tca_csr_to_coo(&a, &o);
        if (s) return s;
        tca_csr x{};
        s = tca_coo_to_csr(&o, &x);
        tca_coo_free(&o);
        if (!s) tca_csr_free(&x);
        return s;
    }, &injected);
    sweep("tca_csr_convert", [&] {
        tca_csr x{};
        const int s = tca_csr_convert(&a, TCA_BF16, &x);
        if (!s) tca_csr_free(&x);
        return s;
    }, &injected);
    sweep("tca_prune_24", [&] {
        tca_csr x{};
        const int s = tca_prune_24(a.row_offset, a.col_idx, a.value, a.nRow, a.nCol, a.nnz, TCA_F16, &x);
        if (!s) tca_csr_free(&x);
        return s;
    }, &injected);
    sweep("tca_gen_rmat", [&] {
        tca_csr x{};
        const int s = tca_gen_rmat(8, 200, 2000, 0.57, 0.19, 0.19, 1, 0, 5, TCA_F32, &x, nullptr);
        if (!s) tca_csr_free(&x);
        return s;
    }, &injected);
    sweep("tca_gen_bernoulli", [&] {
        tca_csr x{};
        const int s = tca_gen_bernoulli(50, 60, 0.1, 1.0, 9, TCA_F16, &x, nullptr);
        if (!s) tca_csr_free(&x);
        return s;
    }, &injected);
    // 4. std::bad_alloc inside an entry point
    const int ba = tca::api_guard("probe", []() -> int { throw std::bad_alloc(); });
    if (ba != TCA_ERR_ALLOC || std::strstr(tca_last_error(), "out of host memory") == nullptr) {
        std::fprintf(stderr, "api_guard gave %d (%s)\n", ba, tca_last_error());
        return 7;
    }
    tca_csr_free(&a);
    std::printf("host sanitize ok: %zu files, %ld mutants, %ld calls, %ld injected failures\n", files.size(), n_mut,
                g_calls, injected);
    return 0;
}
