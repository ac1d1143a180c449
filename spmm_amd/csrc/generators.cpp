// generators.cpp -- seeded, thread-count-independent input generators for the
// five benchmark configurations (and smaller members of the same families).
//
// The reference draws its inputs from std::random_device (unseeded) with 20
// OpenMP threads all writing every element (src/general.cuh:140-174), so its
// inputs cannot be reproduced; these generators replace it.  Every random
// draw comes from a SplitMix64 stream keyed by (seed, stream id), with one
// stream per row (or per sample chunk), so the output does not depend on the
// number of threads or their schedule.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <numeric>
#include <vector>

#include <omp.h>

#include "common.hpp"

using namespace tca;

namespace {

enum : uint64_t {
    kTagDense = 1,
    kTagBernoulli = 2,
    kTagLognormal = 3,
    kTagRmat = 4,
    kTagZipf = 5,
    kTagZipfCols = 6,
};

inline uint64_t row_stream(uint64_t tag, uint64_t r) { return (tag << 40) | r; }

int alloc_csr(tca_csr* out, int32_t M, int32_t K, int64_t nnz, int32_t dtype) {
    if (nnz > INT32_MAX) return fail(TCA_ERR_UNSUPPORTED, "generated nnz %lld exceeds int32", (long long)nnz);
    out->nRow = M;
    out->nCol = K;
    out->nnz = static_cast<int32_t>(nnz);
    out->dtype = dtype;
    out->row_offset = static_cast<int32_t*>(host_alloc(sizeof(int32_t) * (static_cast<size_t>(M) + 1)));
    out->col_idx = static_cast<int32_t*>(host_alloc(sizeof(int32_t) * std::max<int64_t>(nnz, 1)));
    out->value = host_alloc(dtype_size(dtype) * std::max<int64_t>(nnz, 1));
    if (!out->row_offset || !out->col_idx || !out->value) {
        tca_csr_free(out);
        return fail(TCA_ERR_ALLOC, "generator: host allocation of %lld nnz failed", (long long)nnz);
    }
    return TCA_OK;
}

void fill_stats(const tca_csr* a, tca_gen_stats* st, int64_t samples) {
    if (!st) return;
    int32_t mx = 0, empty = 0, over = 0;
#pragma omp parallel for reduction(max : mx) reduction(+ : empty, over) schedule(static)
    for (int32_t r = 0; r < a->nRow; r++) {
        const int32_t l = a->row_offset[r + 1] - a->row_offset[r];
        mx = std::max(mx, l);
        empty += l == 0;
        over += l > 10000;
    }
    st->nnz = a->nnz;
    st->max_row = mx;
    st->empty_rows = empty;
    st->rows_over_10k = over;
    st->mean_row = a->nRow ? static_cast<double>(a->nnz) / a->nRow : 0.0;
    st->samples = samples;
}

// Selects `len` distinct values of [0, K) uniformly (Floyd's algorithm) and
// writes them ascending to out.  `bits` is caller scratch of >= ceil(K/64)
// zeroed words, left zeroed on return.
void sample_sorted(Rng& rng, int32_t K, int32_t len, std::vector<uint64_t>& bits, int32_t* out) {
    if (len <= 0) return;
    if (len >= K) {
        for (int32_t i = 0; i < K; i++) out[i] = i;
        return;
    }
    int32_t n = 0;
    for (int64_t j = static_cast<int64_t>(K) - len; j < K; j++) {
        const int64_t t = static_cast<int64_t>(rng.below(static_cast<uint64_t>(j) + 1));
        const int64_t pick = (bits[t >> 6] >> (t & 63)) & 1 ? j : t;
        bits[pick >> 6] |= uint64_t(1) << (pick & 63);
        out[n++] = static_cast<int32_t>(pick);
    }
    if (static_cast<int64_t>(len) * 64 >= K) {
        // dense selection: read the bitmap in order (and clear it)
        n = 0;
        for (int32_t w = 0; w < (K + 63) / 64; w++) {
            uint64_t word = bits[w];
            bits[w] = 0;
            while (word) {
                const int b = __builtin_ctzll(word);
                out[n++] = w * 64 + b;
                word &= word - 1;
            }
        }
    } else {
        std::sort(out, out + len);
        for (int32_t i = 0; i < len; i++) bits[out[i] >> 6] = 0;
    }
}

// Removes entries whose value rounded to `dtype` is +-0 (a dense -> CSR
// build would not keep them).  Values are given in fp32 in `vf` and written
// as dtype into out->value.  rowptr/colidx are compacted in place.
void compact_store(tca_csr* out, const std::vector<float>& vf) {
    const int32_t M = out->nRow;
    const int32_t dt = out->dtype;
    std::vector<int64_t> keep(static_cast<size_t>(M) + 1, 0);
#pragma omp parallel for schedule(static)
    for (int32_t r = 0; r < M; r++) {
        int64_t k = 0;
        for (int32_t j = out->row_offset[r]; j < out->row_offset[r + 1]; j++) k += !rounds_to_zero(vf[j], dt);
        keep[r + 1] = k;
    }
    for (int32_t r = 0; r < M; r++) keep[r + 1] += keep[r];
    // Rows move left only (keep[r] <= row_offset[r]), so an in-order serial
    // pass is safe; it only runs when something was dropped.
    if (keep[M] != out->nnz) {
        int64_t w = 0;
        for (int32_t r = 0; r < M; r++) {
            const int32_t s = out->row_offset[r], e = out->row_offset[r + 1];
            out->row_offset[r] = static_cast<int32_t>(w);
            for (int32_t j = s; j < e; j++) {
                if (rounds_to_zero(vf[j], dt)) continue;
                out->col_idx[w] = out->col_idx[j];
                store_from_f32(out->value, dt, w, vf[j]);
                w++;
            }
        }
        out->row_offset[M] = static_cast<int32_t>(w);
        out->nnz = static_cast<int32_t>(w);
    } else {
#pragma omp parallel for schedule(static)
        for (int64_t j = 0; j < out->nnz; j++) store_from_f32(out->value, dt, j, vf[j]);
    }
}

}  // namespace

extern "C" {

int tca_gen_dense(int64_t rows, int64_t cols, int32_t dist, float sparsity, uint64_t seed, int32_t dtype,
                  void* out) {
    return api_guard("tca_gen_dense", [&]() -> int {
        if (rows < 0 || cols < 0 || !out || !dtype_ok(dtype) || dist < 0 || dist > 3)
            return fail(TCA_ERR_INVALID, "tca_gen_dense: bad argument");
        const uint64_t key = stream_key(seed, (kTagDense << 40) | static_cast<uint64_t>(dist));
        const int64_t n = rows * cols;
    #pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n; i++) {
            Rng rng(stream_at(key, static_cast<uint64_t>(i)));
            double v;
            switch (dist) {
                case 0: v = 2.0 * rng.uniform() - 1.0; break;
                case 1: v = rng.normal(); break;
                case 2: v = rng.uniform(); break;
                default: {  // reference prepare_cpu_matrix<half> (src/general.cuh:159-166), seeded
                    const double u = rng.uniform();
                    v = u > sparsity ? rng.uniform() : 0.0;
                }
            }
            store_from_f32(out, dtype, i, static_cast<float>(v));
        }
        return TCA_OK;
    });
}

int tca_gen_bernoulli(int32_t M, int32_t K, double p, double sigma, uint64_t seed, int32_t dtype, tca_csr* out,
                      tca_gen_stats* st) {
    return api_guard("tca_gen_bernoulli", [&]() -> int {
        if (M < 0 || K < 0 || !out || !dtype_ok(dtype) || !(p >= 0.0 && p <= 1.0))
            return fail(TCA_ERR_INVALID, "tca_gen_bernoulli: bad argument");
        // One stream per row; entry k of row r is kept when its first draw is < p,
        // and its value is sigma * N(0,1) from the same entry generator.
        std::vector<int64_t> cnt(static_cast<size_t>(M) + 1, 0);
    #pragma omp parallel for schedule(static)
        for (int32_t r = 0; r < M; r++) {
            const uint64_t key = stream_key(seed, row_stream(kTagBernoulli, r));
            int64_t c = 0;
            for (int32_t k = 0; k < K; k++) {
                Rng rng(stream_at(key, k));
                c += rng.uniform() < p;
            }
            cnt[r + 1] = c;
        }
        for (int32_t r = 0; r < M; r++) cnt[r + 1] += cnt[r];
        int s = alloc_csr(out, M, K, cnt[M], dtype);
        if (s) return s;
        std::vector<float> vf(std::max<int64_t>(cnt[M], 1));
    #pragma omp parallel for schedule(static)
        for (int32_t r = 0; r < M; r++) {
            const uint64_t key = stream_key(seed, row_stream(kTagBernoulli, r));
            int64_t w = cnt[r];
            out->row_offset[r] = static_cast<int32_t>(cnt[r]);
            for (int32_t k = 0; k < K; k++) {
                Rng rng(stream_at(key, k));
                if (rng.uniform() < p) {
                    out->col_idx[w] = k;
                    vf[w] = static_cast<float>(sigma * rng.normal());
                    w++;
                }
            }
        }
        out->row_offset[M] = static_cast<int32_t>(cnt[M]);
        compact_store(out, vf);
        fill_stats(out, st, 0);
        return TCA_OK;
    });
}

int tca_gen_lognormal_rows(int32_t M, int32_t K, double mean, double s, double sigma, uint64_t seed,
                           int32_t dtype, tca_csr* out, tca_gen_stats* st) {
    return api_guard("tca_gen_lognormal_rows", [&]() -> int {
        if (M < 0 || K < 1 || !out || !dtype_ok(dtype) || !(mean > 0.0) || !(s >= 0.0))
            return fail(TCA_ERR_INVALID, "tca_gen_lognormal_rows: bad argument");
        const double mu = std::log(mean) - 0.5 * s * s;  // E[LogNormal(mu, s)] = mean
        std::vector<int64_t> off(static_cast<size_t>(M) + 1, 0);
    #pragma omp parallel for schedule(static)
        for (int32_t r = 0; r < M; r++) {
            Rng rng(stream_key(seed, row_stream(kTagLognormal, r)));
            const double l = std::nearbyint(std::exp(mu + s * rng.normal()));
            off[r + 1] = static_cast<int64_t>(std::min<double>(std::max(l, 0.0), K));
        }
        for (int32_t r = 0; r < M; r++) off[r + 1] += off[r];
        int stt = alloc_csr(out, M, K, off[M], dtype);
        if (stt) return stt;
        std::vector<float> vf(std::max<int64_t>(off[M], 1));
    #pragma omp parallel
        {
            std::vector<uint64_t> bits((K + 63) / 64, 0);
    #pragma omp for schedule(dynamic, 16)
            for (int32_t r = 0; r < M; r++) {
                Rng rng(stream_key(seed, row_stream(kTagLognormal, r)));
                rng.normal();  // the length draw
                const int32_t len = static_cast<int32_t>(off[r + 1] - off[r]);
                out->row_offset[r] = static_cast<int32_t>(off[r]);
                sample_sorted(rng, K, len, bits, out->col_idx + off[r]);
                for (int32_t i = 0; i < len; i++) vf[off[r] + i] = static_cast<float>(sigma * rng.normal());
            }
        }
        out->row_offset[M] = static_cast<int32_t>(off[M]);
        compact_store(out, vf);
        fill_stats(out, st, 0);
        return TCA_OK;
    });
}

int tca_gen_rmat(int32_t scale, int32_t n, int64_t samples, double a, double b, double c, int32_t symmetric,
                 int32_t norm, uint64_t seed, int32_t dtype, tca_csr* out, tca_gen_stats* st) {
    return api_guard("tca_gen_rmat", [&]() -> int {
        if (scale < 1 || scale > 30 || n < 1 || n > (int64_t(1) << scale) || samples < 0 || !out || !dtype_ok(dtype) ||
            norm < 0 || norm > 2 || !(a >= 0 && b >= 0 && c >= 0 && a + b + c <= 1.0))
            return fail(TCA_ERR_INVALID, "tca_gen_rmat: bad argument");
        // 1. Samples.  Chunk q of 2^20 accepted samples draws from its own stream,
        //    so the sample list does not depend on the thread count.  Each level
        //    picks a quadrant from a 32-bit uniform: [0,a) -> (0,0), [a,a+b) ->
        //    (0,1), [a+b,a+b+c) -> (1,0), else (1,1) as (row bit, col bit).
        //    Samples with an id >= n or a self-loop are rejected.
        const int64_t chunk = int64_t(1) << 20;
        const int64_t nchunks = (samples + chunk - 1) / chunk;
        std::vector<int32_t> su(samples), sv(samples);
        const uint64_t ta = static_cast<uint64_t>(a * 4294967296.0);
        const uint64_t tb = static_cast<uint64_t>((a + b) * 4294967296.0);
        const uint64_t tc = static_cast<uint64_t>((a + b + c) * 4294967296.0);
    #pragma omp parallel for schedule(dynamic, 1)
        for (int64_t q = 0; q < nchunks; q++) {
            Rng rng(stream_key(seed, row_stream(kTagRmat, q)));
            const int64_t lo = q * chunk, hi = std::min(samples, lo + chunk);
            for (int64_t i = lo; i < hi;) {
                uint32_t u = 0, v = 0;
                uint64_t bitsrc = 0;
                for (int l = 0; l < scale; l++) {
                    if ((l & 1) == 0) bitsrc = rng.next();
                    const uint64_t x = (l & 1) ? (bitsrc >> 32) : (bitsrc & 0xffffffffu);
                    const uint32_t bu = x >= tb, bv = (x >= ta && x < tb) || x >= tc;
                    u = (u << 1) | bu;
                    v = (v << 1) | bv;
                }
                if (u >= static_cast<uint32_t>(n) || v >= static_cast<uint32_t>(n) || u == v) continue;
                su[i] = static_cast<int32_t>(u);
                sv[i] = static_cast<int32_t>(v);
                i++;
            }
        }
        // 2. Bucket directed entries by row (both directions when symmetric).
        std::vector<std::atomic<int64_t>> cnt(static_cast<size_t>(n) + 1);
        for (auto& x : cnt) x.store(0, std::memory_order_relaxed);
    #pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < samples; i++) {
            cnt[su[i] + 1].fetch_add(1, std::memory_order_relaxed);
            if (symmetric) cnt[sv[i] + 1].fetch_add(1, std::memory_order_relaxed);
        }
        std::vector<int64_t> start(static_cast<size_t>(n) + 1, 0);
        for (int32_t r = 0; r < n; r++) start[r + 1] = start[r] + cnt[r + 1].load(std::memory_order_relaxed);
        std::vector<std::atomic<int64_t>>().swap(cnt);
        const int64_t total = start[n];
        std::vector<int32_t> cols(std::max<int64_t>(total, 1));
        {
            std::vector<std::atomic<int64_t>> fillp(static_cast<size_t>(n));
            for (int32_t r = 0; r < n; r++) fillp[r].store(start[r], std::memory_order_relaxed);
    #pragma omp parallel for schedule(static)
            for (int64_t i = 0; i < samples; i++) {
                cols[fillp[su[i]].fetch_add(1, std::memory_order_relaxed)] = sv[i];
                if (symmetric) cols[fillp[sv[i]].fetch_add(1, std::memory_order_relaxed)] = su[i];
            }
        }
        std::vector<int32_t>().swap(su);
        std::vector<int32_t>().swap(sv);
        // 3. Sort and de-duplicate each row (the scatter order above is not
        //    deterministic, the sorted rows are); GCN adds the self-loop.
        const bool self = norm == 0;
        std::vector<int64_t> len(static_cast<size_t>(n) + 1, 0);
    #pragma omp parallel for schedule(dynamic, 256)
        for (int32_t r = 0; r < n; r++) {
            int32_t* b0 = cols.data() + start[r];
            int32_t* e0 = cols.data() + start[r + 1];
            std::sort(b0, e0);
            len[r + 1] = (std::unique(b0, e0) - b0) + (self ? 1 : 0);
        }
        for (int32_t r = 0; r < n; r++) len[r + 1] += len[r];
        int s2 = alloc_csr(out, n, n, len[n], dtype);
        if (s2) return s2;
    #pragma omp parallel for schedule(dynamic, 256)
        for (int32_t r = 0; r < n; r++) {
            const int32_t* b0 = cols.data() + start[r];
            const int64_t k = len[r + 1] - len[r] - (self ? 1 : 0);
            int32_t* o = out->col_idx + len[r];
            out->row_offset[r] = static_cast<int32_t>(len[r]);
            if (!self) {
                std::copy(b0, b0 + k, o);
            } else {
                int64_t w = 0;
                bool put = false;
                for (int64_t i = 0; i < k; i++) {
                    if (!put && b0[i] > r) { o[w++] = r; put = true; }
                    o[w++] = b0[i];
                }
                if (!put) o[w++] = r;
            }
        }
        out->row_offset[n] = static_cast<int32_t>(len[n]);
        std::vector<int32_t>().swap(cols);
        // 4. Values: GCN 1/sqrt(d_i d_j) (degrees include the self-loop), mean
        //    aggregation 1/d_i, or ones; computed in fp64, rounded once.
        std::vector<float> vf(std::max<int64_t>(len[n], 1));
    #pragma omp parallel for schedule(dynamic, 256)
        for (int32_t r = 0; r < n; r++) {
            const int32_t s0 = out->row_offset[r], e0 = out->row_offset[r + 1];
            const double di = e0 - s0;
            for (int32_t j = s0; j < e0; j++) {
                double v = 1.0;
                if (norm == 0) {
                    const int32_t cc = out->col_idx[j];
                    const double dj = out->row_offset[cc + 1] - out->row_offset[cc];
                    v = 1.0 / std::sqrt(di * dj);
                } else if (norm == 1) {
                    v = 1.0 / di;
                }
                vf[j] = static_cast<float>(v);
            }
        }
        compact_store(out, vf);
        fill_stats(out, st, samples);
        return TCA_OK;
    });
}

int tca_gen_zipf_rows(int32_t M, int32_t K, int64_t total_nnz, double s, int32_t cap, uint64_t seed, int32_t dtype,
                      tca_csr* out, tca_gen_stats* st) {
    return api_guard("tca_gen_zipf_rows", [&]() -> int {
        if (M < 1 || K < 1 || total_nnz < 0 || !(s > 1.0) || cap < 1 || !out || !dtype_ok(dtype))
            return fail(TCA_ERR_INVALID, "tca_gen_zipf_rows: bad argument");
        const int32_t lcap = std::min(cap, K);
        if (total_nnz > static_cast<int64_t>(M) * lcap)
            return fail(TCA_ERR_INVALID, "tca_gen_zipf_rows: total %lld exceeds rows * cap", (long long)total_nnz);
        // Raw Zipf draws z = floor(u^(-1/(s-1))), u in (0, 1].
        std::vector<double> z(M);
        const double ex = -1.0 / (s - 1.0);
    #pragma omp parallel for schedule(static)
        for (int32_t r = 0; r < M; r++) {
            Rng rng(stream_key(seed, row_stream(kTagZipf, r)));
            z[r] = std::floor(std::pow(rng.uniform_pos(), ex));
        }
        auto total_at = [&](double f) {
            int64_t t = 0;
    #pragma omp parallel for reduction(+ : t) schedule(static)
            for (int32_t r = 0; r < M; r++) t += static_cast<int64_t>(std::min<double>(lcap, std::floor(f * z[r])));
            return t;
        };
        // Largest f with total_at(f) <= total_nnz (bisection; total_at is monotone).
        double lo = 0.0, hi = static_cast<double>(lcap) + 1.0;
        for (int it = 0; it < 200; it++) {
            const double mid = 0.5 * (lo + hi);
            if (total_at(mid) <= total_nnz) lo = mid; else hi = mid;
        }
        std::vector<int64_t> off(static_cast<size_t>(M) + 1, 0);
        std::vector<std::pair<double, int32_t>> frac;
        for (int32_t r = 0; r < M; r++) {
            const double x = lo * z[r];
            const int64_t l = static_cast<int64_t>(std::min<double>(lcap, std::floor(x)));
            off[r + 1] = l;
            if (l < lcap) frac.emplace_back(x - std::floor(x), r);
        }
        int64_t rem = total_nnz - std::accumulate(off.begin() + 1, off.end(), int64_t(0));
        // Remainder: +1 to the uncapped rows of largest fractional part (row id breaks ties).
        std::sort(frac.begin(), frac.end(), [](const std::pair<double, int32_t>& x, const std::pair<double, int32_t>& y) {
            return x.first != y.first ? x.first > y.first : x.second < y.second;
        });
        for (size_t i = 0; rem > 0 && i < frac.size(); i++, rem--) off[frac[i].second + 1]++;
        for (int32_t r = 0; r < M; r++) off[r + 1] += off[r];
        int s2 = alloc_csr(out, M, K, off[M], dtype);
        if (s2) return s2;
        std::vector<float> vf(std::max<int64_t>(off[M], 1));
    #pragma omp parallel
        {
            std::vector<uint64_t> bits((K + 63) / 64, 0);
    #pragma omp for schedule(dynamic, 64)
            for (int32_t r = 0; r < M; r++) {
                Rng rng(stream_key(seed, row_stream(kTagZipfCols, r)));
                const int32_t len = static_cast<int32_t>(off[r + 1] - off[r]);
                out->row_offset[r] = static_cast<int32_t>(off[r]);
                sample_sorted(rng, K, len, bits, out->col_idx + off[r]);
                for (int32_t i = 0; i < len; i++) vf[off[r] + i] = static_cast<float>(2.0 * rng.uniform() - 1.0);
            }
        }
        out->row_offset[M] = static_cast<int32_t>(off[M]);
        compact_store(out, vf);
        fill_stats(out, st, 0);
        return TCA_OK;
    });
}

// R-MAT sample counts that give the configured edge counts after
// symmetrisation and de-duplication with these generators (seed 1:
// 114,589,436 directed non-loop edges for config 2; ~61.9M for config 3;
// other seeds differ by well under 0.1%).
static const int64_t kRmatSamplesCfg2 = 90800000;
static const int64_t kRmatSamplesCfg3 = 32150000;

int tca_gen_config(int32_t cfg, uint64_t seed, int32_t dtype, tca_csr* out, int32_t* N, tca_gen_stats* st) {
    return api_guard("tca_gen_config", [&]() -> int {
        if (!out || !N) return fail(TCA_ERR_INVALID, "tca_gen_config: bad argument");
        switch (cfg) {
            case 0:
                *N = 256;
                return tca_gen_bernoulli(2048, 512, 0.1, 0.02, seed, dtype < 0 ? TCA_F16 : dtype, out, st);
            case 1:
                *N = 512;
                return tca_gen_lognormal_rows(4096, 4096, 205.0, 1.0, 0.02, seed, dtype < 0 ? TCA_F16 : dtype, out, st);
            case 2:
                *N = 128;
                return tca_gen_rmat(18, 232965, kRmatSamplesCfg2, 0.57, 0.19, 0.19, 1, 0, seed,
                                    dtype < 0 ? TCA_F32 : dtype, out, st);
            case 3:
                *N = 128;
                return tca_gen_rmat(22, 2449029, kRmatSamplesCfg3, 0.57, 0.19, 0.19, 1, 1, seed,
                                    dtype < 0 ? TCA_F32 : dtype, out, st);
            case 4:
                *N = 64;
                return tca_gen_zipf_rows(1048576, 1048576, 20000000, 1.5, 200000, seed, dtype < 0 ? TCA_F16 : dtype, out,
                                         st);
            default:
                return fail(TCA_ERR_INVALID, "tca_gen_config: config %d not in 0..4", cfg);
        }
    });
}

}  // extern "C"
