/*
 * ridge_oracle.c -- CPU restatement of the reference's GEMM checking path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (ridge_amd/, include/) links,
 * loads or calls this file. It is used by tests/, by __graft_entry__.smoke() as
 * the checker, and by bench.py's cpu_baseline leg as the timed CPU baseline.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference repository root).
 *
 * Pinning (what makes each function trustworthy, checked in tests/test_oracle.py):
 *   oracle_f32_to_f16 / oracle_f16_to_f32  -- against numpy's float16 casts over
 *       every finite half and a dense float sweep (independent implementation).
 *   oracle_lcg_fill_f16     -- first values checked by hand integer arithmetic in
 *       the golden fixture, and against a pure-Python restatement that uses
 *       numpy's float16 rounding.
 *   oracle_uniform_fill_f16 -- splitmix64 first outputs against the published
 *       splitmix64 test vector for seed 1234567; range/mean properties.
 *   oracle_gemm_f64 / _omp  -- identity, one-hot, exact small-integer products,
 *       and numpy float64 matmul on random halves.
 *   oracle_error_stats      -- the reference's checker self-test vectors
 *       (exact copy accepted; 5% scale, last 3% halved, one +1.0 rejected) and the
 *       closed form frob = maxRel = e for a uniform (1+e) scale.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* IEEE binary32 -> binary16, round to nearest even, with subnormals, overflow to
 * infinity and NaN kept quiet. Matches __float2half (check-gemm.cu:143). */
uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t absx = x & 0x7fffffffu;
    if (absx >= 0x7f800000u) { /* inf or nan */
        return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0u));
    }
    if (absx >= 0x477ff000u) { /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    const int exp = (int)(absx >> 23) - 127;
    if (exp >= -14) { /* normal half */
        uint32_t mant = absx & 0x7fffffu;
        uint32_t h = ((uint32_t)(exp + 15) << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* carry may bump exponent: correct */
        return (uint16_t)(sign | h);
    }
    if (exp < -25) return (uint16_t)sign; /* below half of the smallest subnormal */
    /* Subnormal half r * 2^-24. The float is mant * 2^(exp-23) with the 24-bit
     * significand, so r = mant * 2^(exp+1): shift right by -(exp+1), 14..24 bits.
     * A round up to r = 1024 correctly produces the smallest normal, 0x0400. */
    const uint32_t mant = (absx & 0x7fffffu) | 0x800000u;
    const int shift = -exp - 1;
    const uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    uint32_t r = h;
    if (rem > halfway || (rem == halfway && (h & 1u))) r += 1u;
    return (uint16_t)(sign | r);
}

float oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: m * 2^-24, exact in float */
            float v = (float)m * (1.0f / 16777216.0f);
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* check-gemm.cu:139-145 (same fill in measure.cu:96-102): 32-bit LCG
 * s = s*1664525 + 1013904223, value ((s>>16)&0x7fff)/32767 - 0.5 in float,
 * rounded to half. */
void oracle_lcg_fill_f16(uint16_t* out, size_t n, uint32_t seed) {
    uint32_t s = seed;
    for (size_t i = 0; i < n; ++i) {
        s = s * 1664525u + 1013904223u;
        const float v = ((float)((s >> 16) & 0x7fffu) / 32767.0f) - 0.5f;
        out[i] = oracle_f32_to_f16(v);
    }
}

/* splitmix64 (Steele, Lea, Flood 2014; Vigna's public-domain reference). The
 * i-th output of the stream seeded with `seed` is mix(seed + (i+1)*golden). */
static uint64_t splitmix64_at(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1u) * 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

uint64_t oracle_splitmix64_at(uint64_t seed, uint64_t i) { return splitmix64_at(seed, i); }

/* The BASELINE fill: U[-1,1) with 24 random bits, (top24 * 2^-23) - 1 computed
 * exactly in float, then rounded to half (RNE). Element i depends only on
 * (seed, i), so a GPU fill kernel reproduces it bit for bit. */
void oracle_uniform_fill_f16(uint16_t* out, size_t n, uint64_t seed) {
    for (size_t i = 0; i < n; ++i) {
        const uint32_t top24 = (uint32_t)(splitmix64_at(seed, i) >> 40);
        const float v = (float)top24 * (1.0f / 8388608.0f) - 1.0f;
        out[i] = oracle_f32_to_f16(v);
    }
}

/* check-gemm.cu:98-108: naive i-j-k, f64 accumulation of half->float->double
 * products. Row-major A (MxK), B (KxN), C (MxN). */
void oracle_gemm_f64(const uint16_t* A, const uint16_t* B, double* C, int M, int N, int K) {
    for (int i = 0; i < M; ++i) {
        for (int j = 0; j < N; ++j) {
            double acc = 0.0;
            for (int k = 0; k < K; ++k) {
                acc += (double)oracle_f16_to_f32(A[(size_t)i * K + k]) *
                       (double)oracle_f16_to_f32(B[(size_t)k * N + j]);
            }
            C[(size_t)i * N + j] = acc;
        }
    }
}

/* The same arithmetic as oracle_gemm_f64 (each C[i][j] is the k-ordered f64 sum
 * of the same products, so results are bit-identical), parallel over rows and
 * with B converted and transposed once so the inner loop is unit-stride.
 * threads <= 0 uses the OpenMP default. Returns the thread count used. */
int oracle_gemm_f64_omp(const uint16_t* A, const uint16_t* B, double* C, int M, int N, int K, int threads) {
    double* Bt = (double*)malloc(sizeof(double) * (size_t)N * (size_t)K);
    double* Ad = (double*)malloc(sizeof(double) * (size_t)M * (size_t)K);
    if (!Bt || !Ad) { free(Bt); free(Ad); return -1; }
    int used = 1;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel
    {
#pragma omp single
        used = omp_get_num_threads();
    }
#pragma omp parallel for schedule(static)
#endif
    for (int k = 0; k < K; ++k)
        for (int j = 0; j < N; ++j) Bt[(size_t)j * K + k] = (double)oracle_f16_to_f32(B[(size_t)k * N + j]);
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (long long t = 0; t < (long long)M * K; ++t) Ad[t] = (double)oracle_f16_to_f32(A[t]);
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 4)
#endif
    for (int i = 0; i < M; ++i) {
        const double* a = Ad + (size_t)i * K;
        for (int j = 0; j < N; ++j) {
            const double* b = Bt + (size_t)j * K;
            double acc = 0.0;
            for (int k = 0; k < K; ++k) acc += a[k] * b[k];
            C[(size_t)i * N + j] = acc;
        }
    }
    free(Bt);
    free(Ad);
    return used;
}

/* check-gemm.cu:120-135: relative Frobenius norm and max element error scaled by
 * the largest reference magnitude, with the same zero-denominator conventions. */
void oracle_error_stats(const float* got, const double* ref, size_t n, double* frob, double* maxRel) {
    double num = 0.0, den = 0.0, maxDiff = 0.0, maxRef = 0.0;
    for (size_t i = 0; i < n; ++i) {
        const double r = ref[i];
        const double d = (double)got[i] - r;
        num += d * d;
        den += r * r;
        if (fabs(d) > maxDiff) maxDiff = fabs(d);
        if (fabs(r) > maxRef) maxRef = fabs(r);
    }
    *frob = den > 0.0 ? sqrt(num) / sqrt(den) : (num == 0.0 ? 0.0 : 1.0);
    *maxRel = maxRef > 0.0 ? maxDiff / maxRef : (maxDiff == 0.0 ? 0.0 : 1.0);
}

/* The north star's tolerance: max|got-ref| / (max|A| * max|B| * K). Not in the
 * reference; it bounds the error by the largest possible |dot product|. */
double oracle_normalized_max_err(const float* got, const double* ref, size_t n, double maxAbsA, double maxAbsB, int K) {
    double maxDiff = 0.0;
    for (size_t i = 0; i < n; ++i) {
        const double d = fabs((double)got[i] - ref[i]);
        if (d > maxDiff) maxDiff = d;
    }
    const double scale = maxAbsA * maxAbsB * (double)K;
    return scale > 0.0 ? maxDiff / scale : (maxDiff == 0.0 ? 0.0 : 1.0);
}

/* check-gemm.cu:203-209: the checker self-test reference vector, LCG seeded
 * 0xc0ffee, values computed in double. */
void oracle_selftest_ref(double* out, size_t n) {
    uint32_t s = 0xc0ffeeu;
    for (size_t i = 0; i < n; ++i) {
        s = s * 1664525u + 1013904223u;
        out[i] = ((double)((s >> 16) & 0x7fffu) / 32767.0) - 0.5;
    }
}

/* Converts halves to floats (for comparing a half output against the f64 ref). */
void oracle_f16_array_to_f32(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = oracle_f16_to_f32(in[i]);
}
