// host_formats.cpp -- sparse containers, format conversion, the validation
// verdict and the CPU products the ./test harness uses as its gold.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <numeric>
#include <vector>

#include <omp.h>

#include "common.hpp"

namespace tca {

static thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}

void clear_error() { g_last_error.clear(); }

const char* last_error_cstr() { return g_last_error.c_str(); }

// Allocation-failure injection (tca_debug_fail_allocs): allocations left
// before the one that fails, -1 for none.  Reaching 0 fails that allocation
// and disarms the counter.
static std::atomic<int64_t> g_host_budget{-1};
static std::atomic<int64_t> g_device_budget{-1};

static bool spend(std::atomic<int64_t>& budget) {
    int64_t v = budget.load(std::memory_order_relaxed);
    while (v >= 0) {
        if (budget.compare_exchange_weak(v, v - 1, std::memory_order_relaxed)) return v == 0;
    }
    return false;
}

void* host_alloc(size_t bytes, bool zero) {
    if (spend(g_host_budget)) return nullptr;
    const size_t n = bytes > 0 ? bytes : 1;
    return zero ? std::calloc(n, 1) : std::malloc(n);
}

bool device_alloc_fails() { return spend(g_device_budget); }

}  // namespace tca

using namespace tca;

extern "C" {

const char* tca_last_error(void) { return tca::last_error_cstr(); }

int tca_debug_fail_allocs(int64_t host_after, int64_t device_after) {
    tca::g_host_budget.store(host_after < 0 ? -1 : host_after);
    tca::g_device_budget.store(device_after < 0 ? -1 : device_after);
    return TCA_OK;
}

const char* tca_status_string(int status) {
    switch (status) {
        case TCA_OK: return "ok";
        case TCA_ERR_INVALID: return "invalid argument";
        case TCA_ERR_ALLOC: return "allocation failed";
        case TCA_ERR_HIP: return "HIP runtime error";
        case TCA_ERR_UNSUPPORTED: return "unsupported";
        case TCA_ERR_IO: return "I/O error";
        case TCA_ERR_FORMAT: return "malformed input";
        default: return "unknown status";
    }
}

void tca_free(void* p) { std::free(p); }

void tca_csr_free(tca_csr* a) {
    if (!a) return;
    std::free(a->row_offset);
    std::free(a->col_idx);
    std::free(a->value);
    a->row_offset = nullptr;
    a->col_idx = nullptr;
    a->value = nullptr;
    a->nnz = 0;
}

void tca_coo_free(tca_coo* a) {
    if (!a) return;
    std::free(a->row_idx);
    std::free(a->col_idx);
    std::free(a->value);
    a->row_idx = nullptr;
    a->col_idx = nullptr;
    a->value = nullptr;
    a->nnz = 0;
}

int tca_csr_validate(const int32_t* rowptr, const int32_t* colidx, int32_t nRow, int32_t nCol,
                     int32_t nnz) {
    return api_guard("tca_csr_validate", [&]() -> int {
        if (nRow < 0 || nCol < 0 || nnz < 0) return fail(TCA_ERR_INVALID, "negative dimension");
        if (!rowptr) return fail(TCA_ERR_INVALID, "rowptr is NULL");
        if (nnz > 0 && !colidx) return fail(TCA_ERR_INVALID, "colidx is NULL");
        if (rowptr[0] != 0) return fail(TCA_ERR_INVALID, "rowptr[0] = %d, expected 0", rowptr[0]);
        if (rowptr[nRow] != nnz)
            return fail(TCA_ERR_INVALID, "rowptr[%d] = %d, expected nnz = %d", nRow, rowptr[nRow], nnz);
        // Monotone row offsets first: with rowptr[0] == 0 and rowptr[nRow] == nnz
        // this bounds every offset to [0, nnz] before any column index is read.
        int bad_row = -1;
    #pragma omp parallel for schedule(static, 4096) reduction(max : bad_row)
        for (int32_t r = 0; r < nRow; r++)
            if (rowptr[r + 1] < rowptr[r]) bad_row = std::max(bad_row, r);
        if (bad_row >= 0) return fail(TCA_ERR_INVALID, "row %d: rowptr decreases", bad_row);
    #pragma omp parallel for schedule(static, 4096) reduction(max : bad_row)
        for (int32_t r = 0; r < nRow; r++) {
            const int32_t s = rowptr[r], e = rowptr[r + 1];
            bool bad = false;
            for (int32_t j = s; !bad && j < e; j++) {
                const int32_t c = colidx[j];
                if (c < 0 || c >= nCol || (j > s && c <= colidx[j - 1])) bad = true;
            }
            if (bad) bad_row = std::max(bad_row, r);
        }
        if (bad_row >= 0)
            return fail(TCA_ERR_INVALID, "row %d: column index out of range or not strictly ascending", bad_row);
        return TCA_OK;
    });
}

uint16_t tca_f32_to_f16(float x) { return f32_to_f16(x); }
float tca_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t tca_f32_to_bf16(float x) { return f32_to_bf16(x); }
float tca_bf16_to_f32(uint16_t h) { return bf16_to_f32(h); }

void tca_convert_array(const void* src, int32_t src_dtype, void* dst, int32_t dst_dtype, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) store_from_f32(dst, dst_dtype, i, load_as_f32(src, src_dtype, i));
}

static int alloc_csr(tca_csr* out, int32_t nRow, int32_t nCol, int64_t nnz, int32_t dtype) {
    if (nnz > INT32_MAX) return fail(TCA_ERR_UNSUPPORTED, "nnz %lld exceeds int32", (long long)nnz);
    out->nRow = nRow;
    out->nCol = nCol;
    out->nnz = static_cast<int32_t>(nnz);
    out->dtype = dtype;
    out->row_offset = static_cast<int32_t*>(host_alloc(sizeof(int32_t) * (static_cast<size_t>(nRow) + 1)));
    out->col_idx = static_cast<int32_t*>(host_alloc(sizeof(int32_t) * std::max<int64_t>(nnz, 1)));
    out->value = host_alloc(dtype_size(dtype) * std::max<int64_t>(nnz, 1));
    if (!out->row_offset || !out->col_idx || !out->value) {
        tca_csr_free(out);
        return fail(TCA_ERR_ALLOC, "host allocation of CSR (%lld nnz) failed", (long long)nnz);
    }
    return TCA_OK;
}

int tca_dense_to_csr(const void* dense, int32_t nRow, int32_t nCol, int32_t dtype, tca_csr* out) {
    return api_guard("tca_dense_to_csr", [&]() -> int {
        if (!dense || !out || nRow < 0 || nCol < 0 || !dtype_ok(dtype))
            return fail(TCA_ERR_INVALID, "tca_dense_to_csr: bad argument");
        // Pass 1: per-row counts of entries whose fp32 value != 0.0f
        // (reference src/miscalleneous.cu:39-41), so +0 and -0 are both dropped.
        std::vector<int64_t> cnt(static_cast<size_t>(nRow) + 1, 0);
    #pragma omp parallel for schedule(static)
        for (int32_t r = 0; r < nRow; r++) {
            int64_t c = 0;
            for (int32_t k = 0; k < nCol; k++)
                c += load_as_f32(dense, dtype, static_cast<int64_t>(r) * nCol + k) != 0.0f;
            cnt[r + 1] = c;
        }
        for (int32_t r = 0; r < nRow; r++) cnt[r + 1] += cnt[r];
        int st = alloc_csr(out, nRow, nCol, cnt[nRow], dtype);
        if (st) return st;
        const size_t es = dtype_size(dtype);
        // Pass 2: row-major scan, ascending columns (reference src/miscalleneous.cu:51-64).
    #pragma omp parallel for schedule(static)
        for (int32_t r = 0; r < nRow; r++) {
            int64_t idx = cnt[r];
            out->row_offset[r] = static_cast<int32_t>(cnt[r]);
            for (int32_t k = 0; k < nCol; k++) {
                const int64_t i = static_cast<int64_t>(r) * nCol + k;
                if (load_as_f32(dense, dtype, i) != 0.0f) {
                    out->col_idx[idx] = k;
                    std::memcpy(static_cast<char*>(out->value) + idx * es,
                                static_cast<const char*>(dense) + i * es, es);
                    idx++;
                }
            }
        }
        out->row_offset[nRow] = static_cast<int32_t>(cnt[nRow]);
        return TCA_OK;
    });
}

int tca_csr_to_dense(const tca_csr* a, void* dense) {
    return api_guard("tca_csr_to_dense", [&]() -> int {
        if (!a || !dense || !dtype_ok(a->dtype)) return fail(TCA_ERR_INVALID, "tca_csr_to_dense: bad argument");
        const size_t es = dtype_size(a->dtype);
        std::memset(dense, 0, es * static_cast<size_t>(a->nRow) * a->nCol);
    #pragma omp parallel for schedule(static)
        for (int32_t r = 0; r < a->nRow; r++)
            for (int32_t j = a->row_offset[r]; j < a->row_offset[r + 1]; j++)
                std::memcpy(static_cast<char*>(dense) + (static_cast<size_t>(r) * a->nCol + a->col_idx[j]) * es,
                            static_cast<const char*>(a->value) + static_cast<size_t>(j) * es, es);
        return TCA_OK;
    });
}

int tca_csr_to_coo(const tca_csr* a, tca_coo* out) {
    return api_guard("tca_csr_to_coo", [&]() -> int {
        if (!a || !out || !dtype_ok(a->dtype)) return fail(TCA_ERR_INVALID, "tca_csr_to_coo: bad argument");
        const size_t es = dtype_size(a->dtype);
        const size_t n = std::max<size_t>(a->nnz, 1);
        out->nRow = a->nRow;
        out->nCol = a->nCol;
        out->nnz = a->nnz;
        out->dtype = a->dtype;
        out->row_idx = static_cast<int32_t*>(host_alloc(sizeof(int32_t) * n));
        out->col_idx = static_cast<int32_t*>(host_alloc(sizeof(int32_t) * n));
        out->value = host_alloc(es * n);
        if (!out->row_idx || !out->col_idx || !out->value) {
            tca_coo_free(out);
            return fail(TCA_ERR_ALLOC, "tca_csr_to_coo: allocation failed");
        }
    #pragma omp parallel for schedule(static)
        for (int32_t r = 0; r < a->nRow; r++)
            for (int32_t j = a->row_offset[r]; j < a->row_offset[r + 1]; j++) out->row_idx[j] = r;
        std::memcpy(out->col_idx, a->col_idx, sizeof(int32_t) * a->nnz);
        std::memcpy(out->value, a->value, es * a->nnz);
        return TCA_OK;
    });
}

int tca_coo_to_csr(const tca_coo* a, tca_csr* out) {
    return api_guard("tca_coo_to_csr", [&]() -> int {
        if (!a || !out || !dtype_ok(a->dtype) || a->nnz < 0) return fail(TCA_ERR_INVALID, "tca_coo_to_csr: bad argument");
        const int64_t n = a->nnz;
        for (int64_t i = 0; i < n; i++)
            if (a->row_idx[i] < 0 || a->row_idx[i] >= a->nRow || a->col_idx[i] < 0 || a->col_idx[i] >= a->nCol)
                return fail(TCA_ERR_INVALID, "COO entry %lld (%d, %d) out of range", (long long)i, a->row_idx[i],
                            a->col_idx[i]);
        std::vector<int64_t> order(n);
        std::iota(order.begin(), order.end(), 0);
        std::stable_sort(order.begin(), order.end(), [&](int64_t x, int64_t y) {
            return a->row_idx[x] != a->row_idx[y] ? a->row_idx[x] < a->row_idx[y] : a->col_idx[x] < a->col_idx[y];
        });
        for (int64_t i = 1; i < n; i++)
            if (a->row_idx[order[i]] == a->row_idx[order[i - 1]] && a->col_idx[order[i]] == a->col_idx[order[i - 1]])
                return fail(TCA_ERR_INVALID, "duplicate COO entry (%d, %d)", a->row_idx[order[i]], a->col_idx[order[i]]);
        int st = alloc_csr(out, a->nRow, a->nCol, n, a->dtype);
        if (st) return st;
        const size_t es = dtype_size(a->dtype);
        std::fill(out->row_offset, out->row_offset + a->nRow + 1, 0);
        for (int64_t i = 0; i < n; i++) {
            const int64_t o = order[i];
            out->row_offset[a->row_idx[o] + 1]++;
            out->col_idx[i] = a->col_idx[o];
            std::memcpy(static_cast<char*>(out->value) + i * es, static_cast<const char*>(a->value) + o * es, es);
        }
        for (int32_t r = 0; r < a->nRow; r++) out->row_offset[r + 1] += out->row_offset[r];
        return TCA_OK;
    });
}

int tca_csr_transpose(const int32_t* rowptr, const int32_t* colidx, int32_t M, int32_t K, int32_t nnz,
                      int32_t* rowptr_t, int32_t* colidx_t, int32_t* perm) {
    return api_guard("tca_csr_transpose", [&]() -> int {
        if (!rowptr || (nnz > 0 && (!colidx || !colidx_t || !perm)) || !rowptr_t || M < 0 || K < 0 || nnz < 0)
            return fail(TCA_ERR_INVALID, "tca_csr_transpose: bad argument");
        if (rowptr[M] != nnz) return fail(TCA_ERR_INVALID, "tca_csr_transpose: rowptr[M] != nnz");
        // Counting sort by column; rows are visited in order, so each row of the
        // transpose lists its columns (A's rows) ascending.
        std::fill(rowptr_t, rowptr_t + static_cast<size_t>(K) + 1, 0);
        for (int32_t j = 0; j < nnz; j++) {
            const int32_t c = colidx[j];
            if (c < 0 || c >= K) return fail(TCA_ERR_INVALID, "tca_csr_transpose: column %d out of range", c);
            rowptr_t[c + 1]++;
        }
        for (int32_t c = 0; c < K; c++) rowptr_t[c + 1] += rowptr_t[c];
        std::vector<int32_t> fill(rowptr_t, rowptr_t + K);
        for (int32_t r = 0; r < M; r++)
            for (int32_t j = rowptr[r]; j < rowptr[r + 1]; j++) {
                const int32_t t = fill[colidx[j]]++;
                colidx_t[t] = r;
                perm[t] = j;
            }
        return TCA_OK;
    });
}

int tca_csr_convert(const tca_csr* a, int32_t dtype, tca_csr* out) {
    return api_guard("tca_csr_convert", [&]() -> int {
        if (!a || !out || !dtype_ok(dtype) || !dtype_ok(a->dtype)) return fail(TCA_ERR_INVALID, "tca_csr_convert: bad argument");
        int st = alloc_csr(out, a->nRow, a->nCol, a->nnz, dtype);
        if (st) return st;
        std::memcpy(out->row_offset, a->row_offset, sizeof(int32_t) * (static_cast<size_t>(a->nRow) + 1));
        std::memcpy(out->col_idx, a->col_idx, sizeof(int32_t) * a->nnz);
        tca_convert_array(a->value, a->dtype, out->value, dtype, a->nnz);
        return TCA_OK;
    });
}

int tca_csr_to_bell(const int32_t* rowptr, const int32_t* colidx, const void* values, int32_t M, int32_t K,
                    int32_t nnz, int32_t dtype, int32_t bsize, int32_t* ell_blocks, int32_t* colind,
                    void* ell_values) {
    return api_guard("tca_csr_to_bell", [&]() -> int {
        if (!rowptr || (nnz > 0 && (!colidx || !values)) || !ell_blocks || M < 0 || K < 1 || nnz < 0 ||
            !dtype_ok(dtype) || bsize < 1 || ((colind == nullptr) != (ell_values == nullptr)))
            return fail(TCA_ERR_INVALID, "tca_csr_to_bell: bad argument");
        int st = tca_csr_validate(rowptr, colidx, M, K, nnz);
        if (st) return st;
        const int32_t brows = (M + bsize - 1) / bsize;
        const int32_t bcols = (K + bsize - 1) / bsize;
        // Block columns holding a nonzero value, per block row, ascending.
        std::vector<std::vector<int32_t>> blocks(brows);
    #pragma omp parallel for schedule(dynamic, 16)
        for (int32_t i = 0; i < brows; i++) {
            std::vector<uint8_t> seen(bcols, 0);
            const int32_t r1 = std::min<int64_t>(M, static_cast<int64_t>(i + 1) * bsize);
            for (int32_t j = rowptr[static_cast<int64_t>(i) * bsize]; j < rowptr[r1]; j++)
                if (load_as_f32(values, dtype, j) != 0.0f) seen[colidx[j] / bsize] = 1;
            for (int32_t b = 0; b < bcols; b++)
                if (seen[b]) blocks[i].push_back(b);
        }
        int32_t width = 0;
        for (const auto& b : blocks) width = std::max<int32_t>(width, static_cast<int32_t>(b.size()));
        *ell_blocks = width;
        if (!colind) return TCA_OK;
        const size_t es = dtype_size(dtype);
        const int64_t ecols = static_cast<int64_t>(width) * bsize;
        std::memset(ell_values, 0, static_cast<size_t>(brows) * bsize * ecols * es);
    #pragma omp parallel for schedule(dynamic, 16)
        for (int32_t i = 0; i < brows; i++) {
            // slot of each present block column in this block row
            std::vector<int32_t> slot(bcols, -1);
            for (int32_t e = 0; e < width; e++) {
                const int32_t b = e < static_cast<int32_t>(blocks[i].size()) ? blocks[i][e] : -1;
                colind[static_cast<int64_t>(i) * width + e] = b;
                if (b >= 0) slot[b] = e;
            }
            const int32_t r1 = std::min<int64_t>(M, static_cast<int64_t>(i + 1) * bsize);
            for (int32_t r = i * bsize; r < r1; r++)
                for (int32_t j = rowptr[r]; j < rowptr[r + 1]; j++) {
                    const int32_t c = colidx[j];
                    const int32_t e = slot[c / bsize];
                    if (e < 0) continue;  // a block of zeros only
                    std::memcpy(static_cast<char*>(ell_values) +
                                    (static_cast<size_t>(r) * ecols + static_cast<size_t>(e) * bsize + c % bsize) * es,
                                static_cast<const char*>(values) + static_cast<size_t>(j) * es, es);
                }
        }
        return TCA_OK;
    });
}

int tca_prune_24(const int32_t* rowptr, const int32_t* colidx, const void* values, int32_t M, int32_t K,
                 int32_t nnz, int32_t dtype, tca_csr* out) {
    return api_guard("tca_prune_24", [&]() -> int {
        if (!rowptr || (nnz > 0 && (!colidx || !values)) || !out || M < 0 || K < 1 || nnz < 0 || !dtype_ok(dtype))
            return fail(TCA_ERR_INVALID, "tca_prune_24: bad argument");
        int st = tca_csr_validate(rowptr, colidx, M, K, nnz);
        if (st) return st;
        // keep[j]: entry j survives.  Columns ascend within a row, so a group's
        // entries are consecutive.
        std::vector<uint8_t> keep(static_cast<size_t>(nnz), 0);
        std::vector<int32_t> cnt(static_cast<size_t>(M) + 1, 0);
    #pragma omp parallel for schedule(dynamic, 64)
        for (int32_t r = 0; r < M; r++) {
            int32_t j = rowptr[r];
            while (j < rowptr[r + 1]) {
                int32_t e = j;
                while (e < rowptr[r + 1] && colidx[e] / 4 == colidx[j] / 4) e++;
                // the two largest |value| of entries j .. e - 1 (nonzero only), lower column first on ties
                int32_t b0 = -1, b1 = -1;
                for (int32_t x = j; x < e; x++) {
                    const float v = std::fabs(load_as_f32(values, dtype, x));
                    if (!(v > 0.0f)) continue;
                    if (b0 < 0 || v > std::fabs(load_as_f32(values, dtype, b0))) {
                        b1 = b0;
                        b0 = x;
                    } else if (b1 < 0 || v > std::fabs(load_as_f32(values, dtype, b1))) {
                        b1 = x;
                    }
                }
                if (b0 >= 0) keep[b0] = 1;
                if (b1 >= 0) keep[b1] = 1;
                j = e;
            }
            int32_t c = 0;
            for (int32_t x = rowptr[r]; x < rowptr[r + 1]; x++) c += keep[x];
            cnt[r + 1] = c;
        }
        for (int32_t r = 0; r < M; r++) cnt[r + 1] += cnt[r];
        st = alloc_csr(out, M, K, cnt[M], dtype);
        if (st) return st;
        const size_t es = dtype_size(dtype);
        std::copy(cnt.begin(), cnt.end(), out->row_offset);
        for (int32_t r = 0, t = 0; r < M; r++)
            for (int32_t x = rowptr[r]; x < rowptr[r + 1]; x++)
                if (keep[x]) {
                    out->col_idx[t] = colidx[x];
                    std::memcpy(static_cast<char*>(out->value) + static_cast<size_t>(t) * es,
                                static_cast<const char*>(values) + static_cast<size_t>(x) * es, es);
                    t++;
                }
        return TCA_OK;
    });
}

int tca_csr_to_24(const int32_t* rowptr, const int32_t* colidx, const void* values, int32_t M, int32_t K,
                  int32_t nnz, int32_t dtype, void* vals24, uint16_t* meta24) {
    return api_guard("tca_csr_to_24", [&]() -> int {
        if (!rowptr || (nnz > 0 && (!colidx || !values)) || M < 0 || K < 1 || nnz < 0 ||
            (dtype != TCA_F16 && dtype != TCA_BF16) || (M > 0 && (!vals24 || !meta24)))
            return fail(TCA_ERR_INVALID, "tca_csr_to_24: bad argument (fp16 / bf16 values)");
        int st = tca_csr_validate(rowptr, colidx, M, K, nnz);
        if (st) return st;
        const int64_t kp = (static_cast<int64_t>(K) + 63) / 64 * 64;
        const int64_t vcols = kp / 2, mcols = kp / 16;
        uint16_t* const v16 = static_cast<uint16_t*>(vals24);
        const uint16_t* const src = static_cast<const uint16_t*>(values);
        int bad = -1;
    #pragma omp parallel for schedule(dynamic, 64)
        for (int32_t r = 0; r < M; r++) {
            uint16_t* vr = v16 + static_cast<size_t>(r) * vcols;
            uint16_t* mr = meta24 + static_cast<size_t>(r) * mcols;
            std::fill(vr, vr + vcols, uint16_t(0));
            // unused pairs: positions 0 and 1 (ascending, distinct), values zero
            std::fill(mr, mr + mcols, uint16_t(0x4444));
            int32_t j = rowptr[r];
            while (j < rowptr[r + 1]) {
                const int32_t g = colidx[j] / 4;
                int32_t e = j;
                while (e < rowptr[r + 1] && colidx[e] / 4 == g) e++;
                if (e - j > 2) {
    #pragma omp critical
                    bad = r;
                    break;
                }
                int32_t p0, p1, x0 = -1, x1 = -1;
                if (e - j == 2) {
                    p0 = colidx[j] % 4, p1 = colidx[j + 1] % 4, x0 = j, x1 = j + 1;
                } else {
                    // one entry: pair it with a zero at another position, ascending
                    const int32_t p = colidx[j] % 4;
                    if (p == 3) p0 = 2, p1 = 3, x1 = j;
                    else p0 = p, p1 = p + 1, x0 = j;
                }
                const int32_t q = g / 4, G = g % 4;
                if (x0 >= 0) vr[8 * q + 2 * G] = src[x0];
                if (x1 >= 0) vr[8 * q + 2 * G + 1] = src[x1];
                const uint16_t nib = static_cast<uint16_t>(p0 | (p1 << 2));
                mr[q] = static_cast<uint16_t>((mr[q] & ~(0xf << (4 * G))) | (nib << (4 * G)));
                j = e;
            }
        }
        if (bad >= 0) return fail(TCA_ERR_INVALID, "tca_csr_to_24: row %d has more than two nonzeros in a group of 4", bad);
        return TCA_OK;
    });
}

int tca_compare_mat(const float* gold, const float* cmp, int64_t n, float tol, float floor,
                    int32_t verbose, tca_compare_result* res) {
    return api_guard("tca_compare_mat", [&]() -> int {
        if (!gold || !cmp || !res || n < 0) return fail(TCA_ERR_INVALID, "tca_compare_mat: bad argument");
        // Verdict of reference compare_mat (src/general.cuh:96-114), fp32 throughout.
        res->success = 1;
        res->fail_count = 0;
        res->first_fail = -1;
        float max_disc = 0.0f;
        for (int64_t i = 0; i < n; i++) {
            const float v1 = gold[i], v2 = cmp[i];
            const float disc = std::fabs(v1 - v2);
            const float rel = std::fabs(disc / v1);
            max_disc = std::fmax(rel, max_disc);
            if (rel >= tol && disc >= tol) {
                res->success = 0;
                if (res->first_fail < 0) res->first_fail = i;
                if (verbose)
                    std::printf("Discrepancy occured in %lldth element :: %f vs %f ...abs_disc : %f, rel_disc : %f %%\n",
                                (long long)i, v1, v2, disc, rel * 100.0);
                if (++res->fail_count >= 10) break;
            }
        }
        res->max_rel = max_disc;
        // Extra report (not part of the verdict): relative error with an absolute floor.
        double mr = 0.0;
    #pragma omp parallel for reduction(max : mr) schedule(static)
        for (int64_t i = 0; i < n; i++) {
            const double g = gold[i], c = cmp[i];
            const double d = std::fabs(g - c) / std::max(std::fabs(g), static_cast<double>(floor));
            if (d > mr || d != d) mr = (d != d) ? INFINITY : d;
        }
        res->max_rel_floor = static_cast<float>(mr);
        return TCA_OK;
    });
}

int tca_naive_gemm(const void* A, const void* B, float* C, int32_t M, int32_t N, int32_t K, int32_t dtype) {
    return api_guard("tca_naive_gemm", [&]() -> int {
        if (!A || !B || !C || M < 0 || N < 0 || K < 0 || !dtype_ok(dtype)) return fail(TCA_ERR_INVALID, "tca_naive_gemm: bad argument");
        // Reference naive_gemm (src/miscalleneous.cu:114-134): k ascending, fp32 mul then add.
    #pragma omp parallel for schedule(static)
        for (int32_t m = 0; m < M; m++)
            for (int32_t n = 0; n < N; n++) {
                float result = 0.0f;
                for (int32_t k = 0; k < K; k++) {
                    const float p = load_as_f32(A, dtype, static_cast<int64_t>(m) * K + k) *
                                    load_as_f32(B, dtype, static_cast<int64_t>(k) * N + n);
                    result = result + p;
                }
                C[static_cast<int64_t>(m) * N + n] = result;
            }
        return TCA_OK;
    });
}

int tca_naive_csr_spmm(const tca_csr* a, const void* B, float* C, int32_t N, int32_t threads) {
    return api_guard("tca_naive_csr_spmm", [&]() -> int {
        if (!a || !B || !C || N < 1 || !dtype_ok(a->dtype)) return fail(TCA_ERR_INVALID, "tca_naive_csr_spmm: bad argument");
        if (threads <= 0) threads = omp_get_max_threads();
        const int32_t dt = a->dtype;
        // naive_gemm's arithmetic restricted to the stored entries (skipped terms are +-0 products).
    #pragma omp parallel num_threads(threads)
        {
            std::vector<float> brow(N);
    #pragma omp for schedule(dynamic, 64)
            for (int32_t m = 0; m < a->nRow; m++) {
                float* crow = C + static_cast<int64_t>(m) * N;
                for (int32_t n = 0; n < N; n++) crow[n] = 0.0f;
                for (int32_t j = a->row_offset[m]; j < a->row_offset[m + 1]; j++) {
                    const float av = load_as_f32(a->value, dt, j);
                    const int64_t base = static_cast<int64_t>(a->col_idx[j]) * N;
                    for (int32_t n = 0; n < N; n++) brow[n] = load_as_f32(B, dt, base + n);
                    for (int32_t n = 0; n < N; n++) {
                        const float p = av * brow[n];  // built with -ffp-contract=off
                        crow[n] = crow[n] + p;
                    }
                }
            }
        }
        return TCA_OK;
    });
}

}  // extern "C"

int tca::csr_alloc(tca_csr* out, int32_t nRow, int32_t nCol, int64_t nnz, int32_t dtype) {
    return alloc_csr(out, nRow, nCol, nnz, dtype);
}
