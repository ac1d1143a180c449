// file_input.cpp -- .smtx and MatrixMarket readers, .smtx writer.
//
// The reference parses .smtx with getline + stringstream into a dense M x K
// half matrix (src/file_input.cu:135-193), which needs 108 GB for the GCN
// configuration.  This reader streams the file through a fixed buffer and
// builds the CSR directly; its output equals the reference's
// .smtx -> dense -> convert_dense_to_csr pipeline (columns ascending and
// unique per row, value 1.0), and it rejects input the reference would
// mis-read silently (token counts, offsets, column range).
#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "common.hpp"

using namespace tca;

namespace {

class Reader {
  public:
    explicit Reader(FILE* f) : f_(f), buf_(1 << 22) {}
    // Next byte or -1 at end of file.
    int get() {
        if (pos_ == len_) {
            len_ = std::fread(buf_.data(), 1, buf_.size(), f_);
            pos_ = 0;
            if (len_ == 0) return -1;
        }
        return static_cast<unsigned char>(buf_[pos_++]);
    }
    int peek() {
        const int c = get();
        if (c >= 0) pos_--;
        return c;
    }
    // Reads an optionally signed decimal integer, skipping the separators in
    // `seps`.  Stops at '\n' (returned in *stop) or EOF.  Returns true when a
    // number was read.
    bool next_int(const char* seps, int64_t* v, int* stop) {
        int c;
        for (;;) {
            c = get();
            if (c < 0 || c == '\n') { *stop = c; return false; }
            if (c == '\r' || std::strchr(seps, c)) continue;
            break;
        }
        bool neg = false;
        if (c == '-' || c == '+') { neg = c == '-'; c = get(); }
        if (c < '0' || c > '9') { *stop = -2; return false; }  // not a number
        int64_t x = 0;
        while (c >= '0' && c <= '9') {
            x = x * 10 + (c - '0');
            if (x > (int64_t(1) << 40)) { *stop = -2; return false; }
            c = get();
        }
        if (c >= 0) pos_--;  // leave the terminator for the next call
        *v = neg ? -x : x;
        *stop = 0;
        return true;
    }
    // Skips to just after the next '\n'.
    void skip_line() {
        int c;
        while ((c = get()) >= 0 && c != '\n') {}
    }

  private:
    FILE* f_;
    std::vector<char> buf_;
    size_t pos_ = 0, len_ = 0;
};

struct SmtxRaw {
    int32_t nrow = 0, ncol = 0, nnz = 0;
    std::vector<int32_t> rowptr, colidx;
};

// Parses the three parts of a .smtx file (reference src/file_input.cu:141-180)
// and checks counts and ranges; column order inside a row is left as read.
// `path` only names the source in messages; the caller owns `f`.
int parse_smtx_stream(FILE* f, const char* path, SmtxRaw* raw) {
    Reader rd(f);
    int64_t h[3];
    int stop = 0;
    for (int i = 0; i < 3; i++) {
        if (!rd.next_int(" \t,", &h[i], &stop)) {
            return fail(TCA_ERR_FORMAT, "%s: header must be 'rows, cols, nnz'", path);
        }
    }
    int64_t extra;
    if (rd.next_int(" \t,", &extra, &stop)) {
        return fail(TCA_ERR_FORMAT, "%s: header has more than 3 numbers", path);
    }
    if (stop == -2) { return fail(TCA_ERR_FORMAT, "%s: bad header token", path); }
    if (h[0] < 0 || h[1] < 0 || h[2] < 0 || h[0] > INT32_MAX - 1 || h[1] > INT32_MAX || h[2] > INT32_MAX) {
        return fail(TCA_ERR_FORMAT, "%s: header values out of range", path);
    }
    raw->nrow = static_cast<int32_t>(h[0]);
    raw->ncol = static_cast<int32_t>(h[1]);
    raw->nnz = static_cast<int32_t>(h[2]);
    // Line 2: nrow + 1 row offsets.  The arrays grow with what is read (at
    // most 2^24 entries reserved up front), so a header alone cannot make
    // the reader allocate gigabytes.
    constexpr size_t kReserve = size_t(1) << 24;
    raw->rowptr.clear();
    raw->rowptr.reserve(std::min(static_cast<size_t>(raw->nrow) + 1, kReserve));
    int64_t v;
    size_t n = 0;
    while (rd.next_int(" \t", &v, &stop)) {
        if (n > static_cast<size_t>(raw->nrow)) {
            return fail(TCA_ERR_FORMAT, "%s: more than rows+1 = %d row offsets", path, raw->nrow + 1);
        }
        raw->rowptr.push_back(static_cast<int32_t>(v));
        n++;
    }
    if (stop == -2 || n != static_cast<size_t>(raw->nrow) + 1) {
        return fail(TCA_ERR_FORMAT, "%s: expected %d row offsets on line 2, read %zu", path, raw->nrow + 1, n);
    }
    if (raw->rowptr[0] != 0 || raw->rowptr[raw->nrow] != raw->nnz) {
        return fail(TCA_ERR_FORMAT, "%s: row offsets must run from 0 to nnz = %d", path, raw->nnz);
    }
    for (int32_t r = 0; r < raw->nrow; r++)
        if (raw->rowptr[r + 1] < raw->rowptr[r]) {
            return fail(TCA_ERR_FORMAT, "%s: row offsets decrease at row %d", path, r);
        }
    // Remaining lines: nnz column indices.
    raw->colidx.clear();
    raw->colidx.reserve(std::min(static_cast<size_t>(raw->nnz), kReserve));
    n = 0;
    for (;;) {
        if (rd.next_int(" \t", &v, &stop)) {
            if (n >= static_cast<size_t>(raw->nnz)) {
                    return fail(TCA_ERR_FORMAT, "%s: more than nnz = %d column indices", path, raw->nnz);
            }
            if (v < 0 || v >= raw->ncol) {
                    return fail(TCA_ERR_FORMAT, "%s: column index %lld out of [0, %d)", path, (long long)v, raw->ncol);
            }
            raw->colidx.push_back(static_cast<int32_t>(v));
            n++;
            continue;
        }
        if (stop == -2) { return fail(TCA_ERR_FORMAT, "%s: bad column token", path); }
        if (stop < 0) break;  // EOF
    }
    if (n != static_cast<size_t>(raw->nnz))
        return fail(TCA_ERR_FORMAT, "%s: expected %d column indices, read %zu", path, raw->nnz, n);
    return TCA_OK;
}


}  // namespace

extern "C" {

}  // extern "C"

namespace tca {

// MatrixMarket coordinate entries in file order (reference
// src/file_input.cu:8-134): '%' lines are skipped, then "rows cols nnz",
// then one "r c [v]" per line.  A value is read like the reference's
// `stream >> float` (strtof: the decimal rounded once to fp32); a line
// without one keeps `missing`.  Blank lines and later '%' lines are skipped
// (the reference would count them as entries and fail its count assert);
// entries outside the matrix and a count different from the header's are
// errors (the reference asserts the count, and writes out-of-range entries
// nowhere or out of bounds).
static int mtx_parse(FILE* f, const char* path, bool zero_based, bool read_value, float missing, int64_t* rows,
                     int64_t* cols, std::vector<int32_t>& ri, std::vector<int32_t>& ci, std::vector<float>& vv) {
    std::vector<char> line(1 << 16);
    int64_t m = -1, k = -1, meta = -1;
    while (std::fgets(line.data(), static_cast<int>(line.size()), f)) {
        if (line[0] == '%') continue;
        long long a, b, c;
        if (std::sscanf(line.data(), "%lld %lld %lld", &a, &b, &c) != 3)
            return fail(TCA_ERR_FORMAT, "%s: bad size line", path);
        m = a; k = b; meta = c;
        break;
    }
    if (m < 0 || k < 0 || meta < 0 || m > INT32_MAX - 1 || k > INT32_MAX || meta > INT32_MAX)
        return fail(TCA_ERR_FORMAT, "%s: missing or out-of-range size line", path);
    ri.clear(); ci.clear(); vv.clear();
    // reserve at most 2^24 entries up front: a header alone cannot make the
    // reader allocate gigabytes (the vectors grow with the entries read)
    const size_t want = static_cast<size_t>(std::min<int64_t>(meta, int64_t(1) << 24));
    ri.reserve(want);
    ci.reserve(want);
    vv.reserve(want);
    while (std::fgets(line.data(), static_cast<int>(line.size()), f)) {
        const char* p = line.data();
        while (*p == ' ' || *p == '\t') p++;
        if (*p == '%' || *p == '\n' || *p == '\r' || *p == '\0') continue;
        long long r, c;
        float v = missing;
        int used = 0;
        if (std::sscanf(p, "%lld %lld%n", &r, &c, &used) != 2) return fail(TCA_ERR_FORMAT, "%s: bad entry line", path);
        if (read_value) {
            const char* q = p + used;
            while (*q == ' ' || *q == '\t') q++;
            if (*q != '\n' && *q != '\r' && *q != '\0') {
                char* end = nullptr;
                v = std::strtof(q, &end);
                if (end == q) return fail(TCA_ERR_FORMAT, "%s: bad value in entry line", path);
            }
        }
        if (!zero_based) { r--; c--; }
        if (r < 0 || r >= m || c < 0 || c >= k)
            return fail(TCA_ERR_FORMAT, "%s: entry (%lld, %lld) out of range", path, r, c);
        ri.push_back(static_cast<int32_t>(r));
        ci.push_back(static_cast<int32_t>(c));
        vv.push_back(v);
    }
    if (static_cast<int64_t>(ri.size()) != meta)
        return fail(TCA_ERR_FORMAT, "%s: header says %lld entries, read %zu", path, (long long)meta, ri.size());
    *rows = m;
    *cols = k;
    return TCA_OK;
}

int mtx_read_csr_file(FILE* f, const char* path, bool pattern_only, bool zero_based, int32_t dtype, bool file_order,
                      tca_csr* out) {
    if (!f || !out || !dtype_ok(dtype)) return fail(TCA_ERR_INVALID, "mtx_read_csr_file: bad argument");
    std::vector<int32_t> ri, ci;
    std::vector<float> vv;
    int64_t rows = 0, cols = 0;
    // pattern_only: "r c" only, value 1; else a missing value reads as 0
    // (reference src/file_input.cu:84-95)
    int st = mtx_parse(f, path, zero_based, !pattern_only, pattern_only ? 1.0f : 0.0f, &rows, &cols, ri, ci, vv);
    if (st) return st;
    std::vector<uint16_t> v16;
    const void* vals = vv.data();
    if (dtype != TCA_F32) {
        v16.resize(vv.size());
        tca_convert_array(vv.data(), TCA_F32, v16.data(), dtype, static_cast<int64_t>(vv.size()));
        vals = v16.data();
    }
    if (!file_order) {
        tca_coo coo{};
        coo.nRow = static_cast<int32_t>(rows);
        coo.nCol = static_cast<int32_t>(cols);
        coo.nnz = static_cast<int32_t>(ri.size());
        coo.dtype = dtype;
        coo.row_idx = ri.data();
        coo.col_idx = ci.data();
        coo.value = const_cast<void*>(vals);
        return tca_coo_to_csr(&coo, out);
    }
    // The reference's CSR: rows ascending, each row's entries in file order,
    // duplicates kept (a per-row map of vectors, src/file_input.cu:103-134)
    // -- here a stable counting sort by row.
    st = csr_alloc(out, static_cast<int32_t>(rows), static_cast<int32_t>(cols), static_cast<int64_t>(ri.size()), dtype);
    if (st) return st;
    std::vector<int64_t> next(static_cast<size_t>(rows) + 1, 0);
    for (int32_t r : ri) next[static_cast<size_t>(r) + 1]++;
    for (int64_t r = 0; r < rows; r++) next[r + 1] += next[r];
    for (int64_t r = 0; r <= rows; r++) out->row_offset[r] = static_cast<int32_t>(next[r]);
    const size_t es = dtype_size(dtype);
    for (size_t e = 0; e < ri.size(); e++) {
        const int64_t d = next[ri[e]]++;
        out->col_idx[d] = ci[e];
        std::memcpy(static_cast<char*>(out->value) + d * es, static_cast<const char*>(vals) + e * es, es);
    }
    return TCA_OK;
}

int mtx_read_dense_file(FILE* f, const char* path, bool zero_based, int32_t dtype, void** dense, int32_t* nRow,
                        int32_t* nCol, int32_t* nnz) {
    if (!f || !dense || !nRow || !nCol || !nnz || !dtype_ok(dtype))
        return fail(TCA_ERR_INVALID, "mtx_read_dense_file: bad argument");
    std::vector<int32_t> ri, ci;
    std::vector<float> vv;
    int64_t rows = 0, cols = 0;
    // the reference's dense reader always reads a value, 1 when missing
    // (src/file_input.cu:20-30)
    int st = mtx_parse(f, path, zero_based, true, 1.0f, &rows, &cols, ri, ci, vv);
    if (st) return st;
    const size_t total = static_cast<size_t>(rows) * static_cast<size_t>(cols);
    const size_t es = dtype_size(dtype);
    void* d = total <= SIZE_MAX / es ? host_alloc(total * es, true) : nullptr;
    if (!d) return fail(TCA_ERR_ALLOC, "tca_mtx_read_dense: %zu elements", total);
    // entries in file order: a later duplicate overwrites an earlier one
    std::vector<uint16_t> v16(dtype == TCA_F32 ? 0 : vv.size());
    if (dtype != TCA_F32) tca_convert_array(vv.data(), TCA_F32, v16.data(), dtype, static_cast<int64_t>(vv.size()));
    for (size_t e = 0; e < ri.size(); e++) {
        const size_t at = static_cast<size_t>(ri[e]) * static_cast<size_t>(cols) + static_cast<size_t>(ci[e]);
        if (dtype == TCA_F32) static_cast<float*>(d)[at] = vv[e];
        else static_cast<uint16_t*>(d)[at] = v16[e];
    }
    *dense = d;
    *nRow = static_cast<int32_t>(rows);
    *nCol = static_cast<int32_t>(cols);
    *nnz = static_cast<int32_t>(ri.size());
    return TCA_OK;
}

int smtx_read_csr_file(FILE* f, const char* path, int32_t dtype, tca_csr* out) {
    if (!f || !out || !dtype_ok(dtype)) return fail(TCA_ERR_INVALID, "smtx_read_csr_file: bad argument");
    SmtxRaw raw;
    int st = parse_smtx_stream(f, path, &raw);
    if (st) return st;
    // Sort and de-duplicate each row, as .smtx -> dense -> CSR would
    // (reference src/file_input.cu:182-191 then src/miscalleneous.cu:29-65).
    std::vector<int32_t> rp(static_cast<size_t>(raw.nrow) + 1, 0);
    int32_t w = 0;
    for (int32_t r = 0; r < raw.nrow; r++) {
        int32_t* b = raw.colidx.data() + raw.rowptr[r];
        int32_t* e = raw.colidx.data() + raw.rowptr[r + 1];
        if (!std::is_sorted(b, e)) std::sort(b, e);
        for (int32_t* p = b; p < e; p++)
            if (p == b || *p != p[-1]) raw.colidx[w++] = *p;
        rp[r + 1] = w;
    }
    out->nRow = raw.nrow;
    out->nCol = raw.ncol;
    out->nnz = w;
    out->dtype = dtype;
    out->row_offset = static_cast<int32_t*>(host_alloc(sizeof(int32_t) * rp.size()));
    out->col_idx = static_cast<int32_t*>(host_alloc(sizeof(int32_t) * std::max(w, 1)));
    out->value = host_alloc(dtype_size(dtype) * std::max(w, 1));
    if (!out->row_offset || !out->col_idx || !out->value) {
        tca_csr_free(out);
        return fail(TCA_ERR_ALLOC, "tca_smtx_read_csr: allocation failed");
    }
    std::memcpy(out->row_offset, rp.data(), sizeof(int32_t) * rp.size());
    std::memcpy(out->col_idx, raw.colidx.data(), sizeof(int32_t) * w);
    for (int32_t j = 0; j < w; j++) store_from_f32(out->value, dtype, j, 1.0f);
    return TCA_OK;
}

int smtx_read_dense_file(FILE* f, const char* path, int32_t dtype, void** dense, int32_t* nRow, int32_t* nCol,
                         int32_t* nnz) {
    if (!f || !dense || !nRow || !nCol || !nnz || !dtype_ok(dtype))
        return fail(TCA_ERR_INVALID, "smtx_read_dense_file: bad argument");
    SmtxRaw raw;
    int st = parse_smtx_stream(f, path, &raw);
    if (st) return st;
    const size_t es = dtype_size(dtype);
    const size_t total = static_cast<size_t>(raw.nrow) * raw.ncol;
    void* d = total <= SIZE_MAX / es ? host_alloc(total * es, true) : nullptr;
    if (!d) return fail(TCA_ERR_ALLOC, "tca_smtx_read_dense: %zu elements", total);
    // 1.0 at every listed (row, col) (reference src/file_input.cu:182-191).
    for (int32_t r = 0; r < raw.nrow; r++)
        for (int32_t j = raw.rowptr[r]; j < raw.rowptr[r + 1]; j++)
            store_from_f32(d, dtype, static_cast<int64_t>(r) * raw.ncol + raw.colidx[j], 1.0f);
    *dense = d;
    *nRow = raw.nrow;
    *nCol = raw.ncol;
    *nnz = raw.nnz;
    return TCA_OK;
}

}  // namespace tca

extern "C" {

int tca_smtx_read_csr(const char* path, int32_t dtype, tca_csr* out) {
    return api_guard("tca_smtx_read_csr", [&]() -> int {
        if (!path || !out || !dtype_ok(dtype)) return fail(TCA_ERR_INVALID, "tca_smtx_read_csr: bad argument");
        FILE* f = std::fopen(path, "rb");
        if (!f) return fail(TCA_ERR_IO, "cannot open '%s'", path);
        const int st = smtx_read_csr_file(f, path, dtype, out);
        std::fclose(f);
        return st;
    });
}

int tca_smtx_read_dense(const char* path, int32_t dtype, void** dense, int32_t* nRow, int32_t* nCol,
                        int32_t* nnz) {
    return api_guard("tca_smtx_read_dense", [&]() -> int {
        if (!path || !dense || !nRow || !nCol || !nnz || !dtype_ok(dtype))
            return fail(TCA_ERR_INVALID, "tca_smtx_read_dense: bad argument");
        FILE* f = std::fopen(path, "rb");
        if (!f) return fail(TCA_ERR_IO, "cannot open '%s'", path);
        const int st = smtx_read_dense_file(f, path, dtype, dense, nRow, nCol, nnz);
        std::fclose(f);
        return st;
    });
}

int tca_smtx_write(const char* path, const tca_csr* a) {
    return api_guard("tca_smtx_write", [&]() -> int {
        if (!path || !a) return fail(TCA_ERR_INVALID, "tca_smtx_write: bad argument");
        // The stream buffer is allocated before the file is opened: if the
        // allocation throws (api_guard -> TCA_ERR_ALLOC), no FILE is left open.
        std::vector<char> buf(1 << 22);
        FILE* f = std::fopen(path, "wb");
        if (!f) return fail(TCA_ERR_IO, "cannot create '%s'", path);
        std::setvbuf(f, buf.data(), _IOFBF, buf.size());
        std::fprintf(f, "%d, %d, %d\n", a->nRow, a->nCol, a->nnz);
        char tmp[16];
        for (int32_t r = 0; r <= a->nRow; r++) {
            const int k = std::snprintf(tmp, sizeof tmp, "%d ", a->row_offset[r]);
            std::fwrite(tmp, 1, k, f);
        }
        std::fputc('\n', f);
        for (int32_t j = 0; j < a->nnz; j++) {
            const int k = std::snprintf(tmp, sizeof tmp, "%d ", a->col_idx[j]);
            std::fwrite(tmp, 1, k, f);
        }
        std::fputc('\n', f);
        const bool ok = std::ferror(f) == 0;
        if (std::fclose(f) != 0 || !ok) return fail(TCA_ERR_IO, "write to '%s' failed", path);
        return TCA_OK;
    });
}

// ---- binary CSR cache and values sidecar (no reference counterpart) ----
// Little-endian: 8-byte magic, then the fields below, then the arrays.
namespace {
constexpr char kCsrMagic[8] = {'T', 'C', 'A', 'C', 'S', 'R', '0', '1'};
constexpr char kValMagic[8] = {'T', 'C', 'A', 'V', 'A', 'L', '0', '1'};

struct CsrHeader {
    int32_t nRow, nCol;
    int64_t nnz;
    int32_t dtype, reserved;
};
struct ValHeader {
    int64_t nnz;
    int32_t dtype, reserved;
};

bool write_all(FILE* f, const void* p, size_t n) { return n == 0 || std::fwrite(p, 1, n, f) == n; }
bool read_all(FILE* f, void* p, size_t n) { return n == 0 || std::fread(p, 1, n, f) == n; }

// Size of an open file (restores the position to the start).
int64_t file_size(FILE* f) {
    if (std::fseek(f, 0, SEEK_END) != 0) return -1;
    const long n = std::ftell(f);
    std::rewind(f);
    return n;
}
}  // namespace

int tca_csr_write_binary(const char* path, const tca_csr* a) {
    return api_guard("tca_csr_write_binary", [&]() -> int {
        if (!path || !a || !dtype_ok(a->dtype) || a->nRow < 0 || a->nCol < 0 || a->nnz < 0)
            return fail(TCA_ERR_INVALID, "tca_csr_write_binary: bad argument");
        FILE* f = std::fopen(path, "wb");
        if (!f) return fail(TCA_ERR_IO, "cannot create '%s'", path);
        const CsrHeader h{a->nRow, a->nCol, a->nnz, a->dtype, 0};
        bool ok = write_all(f, kCsrMagic, 8) && write_all(f, &h, sizeof h) &&
                  write_all(f, a->row_offset, sizeof(int32_t) * (static_cast<size_t>(a->nRow) + 1)) &&
                  write_all(f, a->col_idx, sizeof(int32_t) * static_cast<size_t>(a->nnz)) &&
                  write_all(f, a->value, dtype_size(a->dtype) * static_cast<size_t>(a->nnz));
        ok = std::fclose(f) == 0 && ok;
        return ok ? TCA_OK : fail(TCA_ERR_IO, "write to '%s' failed", path);
    });
}

int tca_csr_read_binary(const char* path, tca_csr* out) {
    return api_guard("tca_csr_read_binary", [&]() -> int {
        if (!path || !out) return fail(TCA_ERR_INVALID, "tca_csr_read_binary: bad argument");
        FILE* f = std::fopen(path, "rb");
        if (!f) return fail(TCA_ERR_IO, "cannot open '%s'", path);
        const int64_t size = file_size(f);
        char magic[8];
        CsrHeader h{};
        if (!read_all(f, magic, 8) || std::memcmp(magic, kCsrMagic, 8) != 0 || !read_all(f, &h, sizeof h)) {
            std::fclose(f);
            return fail(TCA_ERR_FORMAT, "'%s' is not a binary CSR file", path);
        }
        if (h.nRow < 0 || h.nCol < 0 || h.nnz < 0 || h.nnz > INT32_MAX || !dtype_ok(h.dtype) ||
            size != static_cast<int64_t>(8 + sizeof h + 4 * (static_cast<int64_t>(h.nRow) + 1) + 4 * h.nnz +
                                         static_cast<int64_t>(dtype_size(h.dtype)) * h.nnz)) {
            std::fclose(f);
            return fail(TCA_ERR_FORMAT, "'%s': header (%d x %d, nnz %lld, dtype %d) does not match the file size %lld",
                        path, h.nRow, h.nCol, (long long)h.nnz, h.dtype, (long long)size);
        }
        int st = csr_alloc(out, h.nRow, h.nCol, h.nnz, h.dtype);
        if (st) {
            std::fclose(f);
            return st;
        }
        const bool ok = read_all(f, out->row_offset, sizeof(int32_t) * (static_cast<size_t>(h.nRow) + 1)) &&
                        read_all(f, out->col_idx, sizeof(int32_t) * static_cast<size_t>(h.nnz)) &&
                        read_all(f, out->value, dtype_size(h.dtype) * static_cast<size_t>(h.nnz));
        std::fclose(f);
        if (!ok) {
            tca_csr_free(out);
            return fail(TCA_ERR_IO, "read of '%s' failed", path);
        }
        st = tca_csr_validate(out->row_offset, out->col_idx, out->nRow, out->nCol, out->nnz);
        if (st) tca_csr_free(out);
        return st;
    });
}

int tca_values_write(const char* path, const void* values, int64_t nnz, int32_t dtype) {
    return api_guard("tca_values_write", [&]() -> int {
        if (!path || (nnz > 0 && !values) || nnz < 0 || !dtype_ok(dtype))
            return fail(TCA_ERR_INVALID, "tca_values_write: bad argument");
        FILE* f = std::fopen(path, "wb");
        if (!f) return fail(TCA_ERR_IO, "cannot create '%s'", path);
        const ValHeader h{nnz, dtype, 0};
        bool ok = write_all(f, kValMagic, 8) && write_all(f, &h, sizeof h) &&
                  write_all(f, values, dtype_size(dtype) * static_cast<size_t>(nnz));
        ok = std::fclose(f) == 0 && ok;
        return ok ? TCA_OK : fail(TCA_ERR_IO, "write to '%s' failed", path);
    });
}

int tca_smtx_read_csr_values(const char* smtx_path, const char* values_path, int32_t dtype, tca_csr* out) {
    return api_guard("tca_smtx_read_csr_values", [&]() -> int {
        if (!smtx_path || !values_path || !out || !dtype_ok(dtype))
            return fail(TCA_ERR_INVALID, "tca_smtx_read_csr_values: bad argument");
        FILE* f = std::fopen(values_path, "rb");
        if (!f) return fail(TCA_ERR_IO, "cannot open '%s'", values_path);
        const int64_t size = file_size(f);
        char magic[8];
        ValHeader h{};
        if (!read_all(f, magic, 8) || std::memcmp(magic, kValMagic, 8) != 0 || !read_all(f, &h, sizeof h) ||
            h.nnz < 0 || !dtype_ok(h.dtype) ||
            size != static_cast<int64_t>(8 + sizeof h + static_cast<int64_t>(dtype_size(h.dtype)) * h.nnz)) {
            std::fclose(f);
            return fail(TCA_ERR_FORMAT, "'%s' is not a values file of its stated size", values_path);
        }
        std::vector<char> vals(dtype_size(h.dtype) * static_cast<size_t>(h.nnz) + 1);
        const bool ok = read_all(f, vals.data(), dtype_size(h.dtype) * static_cast<size_t>(h.nnz));
        std::fclose(f);
        if (!ok) return fail(TCA_ERR_IO, "read of '%s' failed", values_path);
        int st = tca_smtx_read_csr(smtx_path, dtype, out);
        if (st) return st;
        if (out->nnz != h.nnz) {
            const int32_t got = out->nnz;
            tca_csr_free(out);
            return fail(TCA_ERR_FORMAT, "'%s' holds %lld values, '%s' has %d nonzeros", values_path, (long long)h.nnz,
                        smtx_path, got);
        }
        tca_convert_array(vals.data(), h.dtype, out->value, dtype, h.nnz);
        return TCA_OK;
    });
}

int tca_mtx_read_csr(const char* path, int32_t pattern_only, int32_t zero_based, int32_t dtype, tca_csr* out) {
    return api_guard("tca_mtx_read_csr", [&]() -> int {
        if (!path || !out || !dtype_ok(dtype)) return fail(TCA_ERR_INVALID, "tca_mtx_read_csr: bad argument");
        FILE* f = std::fopen(path, "rb");
        if (!f) return fail(TCA_ERR_IO, "cannot open '%s'", path);
        const int st = tca::mtx_read_csr_file(f, path, pattern_only != 0, zero_based != 0, dtype, false, out);
        std::fclose(f);
        return st;
    });
}

int tca_mtx_read_csr_file_order(const char* path, int32_t pattern_only, int32_t zero_based, int32_t dtype,
                                tca_csr* out) {
    return api_guard("tca_mtx_read_csr_file_order", [&]() -> int {
        if (!path || !out || !dtype_ok(dtype)) return fail(TCA_ERR_INVALID, "tca_mtx_read_csr_file_order: bad argument");
        FILE* f = std::fopen(path, "rb");
        if (!f) return fail(TCA_ERR_IO, "cannot open '%s'", path);
        const int st = tca::mtx_read_csr_file(f, path, pattern_only != 0, zero_based != 0, dtype, true, out);
        std::fclose(f);
        return st;
    });
}

int tca_mtx_read_dense(const char* path, int32_t zero_based, int32_t dtype, void** dense, int32_t* nRow,
                       int32_t* nCol, int32_t* nnz) {
    return api_guard("tca_mtx_read_dense", [&]() -> int {
        if (!path || !dense || !nRow || !nCol || !nnz || !dtype_ok(dtype))
            return fail(TCA_ERR_INVALID, "tca_mtx_read_dense: bad argument");
        FILE* f = std::fopen(path, "rb");
        if (!f) return fail(TCA_ERR_IO, "cannot open '%s'", path);
        const int st = tca::mtx_read_dense_file(f, path, zero_based != 0, dtype, dense, nRow, nCol, nnz);
        std::fclose(f);
        return st;
    });
}

}  // extern "C"
