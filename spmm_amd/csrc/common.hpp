// common.hpp -- shared host helpers of libtcaspmm.so: status and last-error
// reporting, IEEE binary16 / bfloat16 conversion and the SplitMix64 streams
// used by the seeded generators.
#pragma once

#include <cstdarg>
#include <cstdint>
#include <new>
#include <cstdio>
#include <cstring>
#include <cmath>
#include <string>

#include "../../include/tca_spmm.h"
#include "../../include/tca_host.h"

namespace tca {

// Records a printf-style message as this thread's last error and returns
// `status`, so call sites read `return fail(TCA_ERR_INVALID, "...")`.
int fail(int status, const char* fmt, ...);
void clear_error();

// .smtx readers over an open stream (`name` only labels error messages).
int smtx_read_csr_file(FILE* f, const char* name, int32_t dtype, tca_csr* out);
int smtx_read_dense_file(FILE* f, const char* name, int32_t dtype, void** dense, int32_t* nRow, int32_t* nCol,
                         int32_t* nnz);
// MatrixMarket readers over an open stream: CSR sorted by (row, col) with
// duplicates rejected, or (file_order) the reference's CSR -- rows ascending,
// each row's entries in file order, duplicates kept; and the reference's
// dense reader (later duplicates overwrite earlier ones).
int mtx_read_csr_file(FILE* f, const char* name, bool pattern_only, bool zero_based, int32_t dtype, bool file_order,
                      tca_csr* out);
int mtx_read_dense_file(FILE* f, const char* name, bool zero_based, int32_t dtype, void** dense, int32_t* nRow,
                        int32_t* nCol, int32_t* nnz);

// Runs the body of a C ABI entry point, turning std::bad_alloc from its
// containers into TCA_ERR_ALLOC (exceptions must not cross the C boundary).
template <typename F>
int api_guard(const char* name, F&& body) {
    try {
        return body();
    } catch (const std::bad_alloc&) {
        return fail(TCA_ERR_ALLOC, "%s: out of host memory", name);
    }
}

// The library's host allocations that outlive a call (arrays handed to the
// caller): malloc, or calloc when `zero`.  tca_debug_fail_allocs can make
// the n-th one fail, to test the failure paths; free() releases them.
void* host_alloc(size_t bytes, bool zero = false);
// Whether the next device allocation is to fail (the device side of
// tca_debug_fail_allocs; counts one allocation per call).
bool device_alloc_fails();

// Allocates the arrays of a host CSR (malloc; tca_csr_free releases them).
int csr_alloc(tca_csr* out, int32_t nRow, int32_t nCol, int64_t nnz, int32_t dtype);

inline size_t dtype_size(int32_t dtype) { return dtype == TCA_F32 ? 4 : 2; }
inline bool dtype_ok(int32_t dtype) { return dtype == TCA_F16 || dtype == TCA_F32 || dtype == TCA_BF16; }

inline uint32_t f32_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float bits_f32(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

// fp32 -> binary16, round to nearest even (IEEE 754-2008, 5-bit exponent,
// 10-bit fraction).  NaN stays NaN (quiet), overflow gives +-inf.
inline uint16_t f32_to_f16(float f) {
    const uint32_t x = f32_bits(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u)  // inf / nan
        return static_cast<uint16_t>(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u | ((ax >> 13) & 0x3ffu) : 0u));
    if (ax >= 0x477ff000u)  // >= 65520 rounds to inf
        return static_cast<uint16_t>(sign | 0x7c00u);
    if (ax < 0x38800000u) {  // below 2^-14: subnormal half; |f| * 2^24 is exact
        const float t = std::nearbyint(bits_f32(ax) * 16777216.0f);
        return static_cast<uint16_t>(sign | static_cast<uint32_t>(t));
    }
    // normal: drop 13 fraction bits with round-to-nearest-even, rebias 127 -> 15
    const uint32_t odd = (ax >> 13) & 1u;
    const uint32_t r = (ax + 0xfffu + odd) >> 13;
    return static_cast<uint16_t>(sign | (r - (112u << 10)));
}

inline float f16_to_f32(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {  // zero or subnormal: m * 2^-24 (exact in fp32)
        const float v = static_cast<float>(m) * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

// fp32 -> bfloat16 (upper 16 bits), round to nearest even; NaN stays quiet NaN.
inline uint16_t f32_to_bf16(float f) {
    const uint32_t x = f32_bits(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((x >> 16) | 0x40u);
    return static_cast<uint16_t>((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}
inline float bf16_to_f32(uint16_t h) { return bits_f32(static_cast<uint32_t>(h) << 16); }

// Value of element i of a typed array as fp32 (exact widening).
inline float load_as_f32(const void* p, int32_t dtype, int64_t i) {
    if (dtype == TCA_F32) return static_cast<const float*>(p)[i];
    const uint16_t h = static_cast<const uint16_t*>(p)[i];
    return dtype == TCA_F16 ? f16_to_f32(h) : bf16_to_f32(h);
}
// Stores fp32 v into element i of a typed array (RNE narrowing).
inline void store_from_f32(void* p, int32_t dtype, int64_t i, float v) {
    if (dtype == TCA_F32) static_cast<float*>(p)[i] = v;
    else static_cast<uint16_t*>(p)[i] = dtype == TCA_F16 ? f32_to_f16(v) : f32_to_bf16(v);
}
// The narrowed value compares equal to zero (so a CSR build would drop it).
inline bool rounds_to_zero(float v, int32_t dtype) {
    if (dtype == TCA_F32) return v == 0.0f;
    const uint16_t h = dtype == TCA_F16 ? f32_to_f16(v) : f32_to_bf16(v);
    return (h & 0x7fffu) == 0;
}

// ---- SplitMix64 (Steele, Lea, Flood 2014) counter streams -----------------
constexpr uint64_t kGolden = 0x9e3779b97f4a7c15ull;
inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
// Key of stream `stream` under `seed`; element i of the stream is
// mix64(key + (i + 1) * kGolden), the i-th output of a SplitMix64 generator
// whose state starts at `key`.
inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return mix64(seed ^ mix64(stream * 0xd1b54a32d192ed03ull + 0x632be59bd9b4e019ull));
}
inline uint64_t stream_at(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * kGolden); }

struct Rng {
    uint64_t s;
    explicit Rng(uint64_t key) : s(key) {}
    uint64_t next() { s += kGolden; return mix64(s); }
    double uniform() { return static_cast<double>(next() >> 11) * 0x1.0p-53; }          // [0, 1)
    double uniform_pos() { return static_cast<double>((next() >> 11) + 1) * 0x1.0p-53; } // (0, 1]
    double normal() {  // Box-Muller, cosine branch
        const double u1 = uniform_pos();
        const double u2 = uniform();
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586476925 * u2);
    }
    // uniform integer in [0, n) without modulo bias (Lemire's multiply-shift with rejection)
    uint64_t below(uint64_t n) {
        if (n <= 1) return 0;
        unsigned __int128 m = static_cast<unsigned __int128>(next()) * n;
        uint64_t l = static_cast<uint64_t>(m);
        if (l < n) {
            const uint64_t t = (0 - n) % n;
            while (l < t) {
                m = static_cast<unsigned __int128>(next()) * n;
                l = static_cast<uint64_t>(m);
            }
        }
        return static_cast<uint64_t>(m >> 64);
    }
};

}  // namespace tca
