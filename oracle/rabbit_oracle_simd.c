/*
 * rabbit_oracle_simd.c -- the reference's AVX2 and AVX-512F/BW MXFP4 tiers, restated in C with the
 * same intrinsic sequence (kernels.rs:641-797), for the CPU baseline bench.py reports.
 *
 * TEST INFRASTRUCTURE ONLY. The scalar restatement (rabbit_oracle.c) is the parity oracle; these
 * tiers reassociate the sum exactly as the reference's tiers do and are checked against the
 * scalar tier within the reference's own tolerance (kernels.rs:1916-1983: 1e-4 absolute).
 *
 * Each tier is compiled for its ISA with a target attribute and chosen at run time from CPUID,
 * the way kernels.rs:233-244 picks with is_x86_feature_detected!, so the built object runs on any
 * x86-64 host. Rows run in parallel over OpenMP threads (rayon's par_chunks_mut over rows,
 * kernels.rs:44-60); orc_set_threads() fixes the count (one per physical core in bench.py,
 * main.rs:311-318).
 */
#include "rabbit_oracle.h"

#include <immintrin.h>
#include <stdlib.h>
#include <string.h>

int orc_nthreads_internal(void);

static size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }

int orc_cpu_has_avx512(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw");
}
int orc_cpu_has_avx2(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

/* kernels.rs:645 MXFP4_TABLE8: the eight E2M1 magnitudes, indexed by the nibble's low 3 bits. */
static const float TABLE8[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

/* ---- AVX2 tier: kernels.rs:654-696 ----------------------------------------------------------- */
__attribute__((target("avx2,fma"))) static inline __m256 decode8_avx2(__m256i nib32, __m256 table, __m256 sv) {
    __m256i idx = _mm256_and_si256(nib32, _mm256_set1_epi32(0x7));
    __m256 mag = _mm256_permutevar8x32_ps(table, idx);
    __m256i sign = _mm256_slli_epi32(_mm256_and_si256(nib32, _mm256_set1_epi32(0x8)), 28);
    __m256 sgn = _mm256_castsi256_ps(_mm256_xor_si256(_mm256_castps_si256(mag), sign));
    return _mm256_mul_ps(sgn, sv);
}

__attribute__((target("avx2,fma"))) static inline float hsum_avx2(__m256 v) {
    __m128 lo = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    lo = _mm_add_ps(lo, _mm_movehl_ps(lo, lo));
    lo = _mm_add_ss(lo, _mm_shuffle_ps(lo, lo, 1));
    return _mm_cvtss_f32(lo);
}

__attribute__((target("avx2,fma"))) static float dot_mxfp4_avx2(const uint8_t *w, const uint8_t *bs, const float *xs,
                                                               size_t n) {
    const __m128i m4 = _mm_set1_epi8(0x0F);
    const __m256 table = _mm256_loadu_ps(TABLE8);
    __m256 acc = _mm256_setzero_ps();
    size_t i = 0;
    for (; i + 16 <= n; i += 16) {
        __m256 sv = _mm256_set1_ps(orc_e8m0_decode(bs[i / 32]));
        __m128i by = _mm_loadl_epi64((const __m128i *)(w + (i >> 1)));
        __m128i lo = _mm_and_si128(by, m4);
        __m128i hi = _mm_and_si128(_mm_srli_epi16(by, 4), m4);
        __m128i nib = _mm_unpacklo_epi8(lo, hi);
        __m256 wl = decode8_avx2(_mm256_cvtepu8_epi32(nib), table, sv);
        __m256 wh = decode8_avx2(_mm256_cvtepu8_epi32(_mm_srli_si128(nib, 8)), table, sv);
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(xs + i), wl, acc);
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(xs + i + 8), wh, acc);
    }
    float a = hsum_avx2(acc);
    for (; i < n; i++) {
        uint8_t byte = w[i >> 1];
        uint8_t nibble = (i & 1) == 0 ? (byte & 0xF) : (byte >> 4);
        a += xs[i] * orc_e2m1_decode(nibble) * orc_e8m0_decode(bs[i / 32]);
    }
    return a;
}

/* ---- AVX-512F/BW tier: kernels.rs:698-749 ----------------------------------------------------- */
__attribute__((target("avx512f,avx512bw"))) static inline __m512 decode16_avx512(__m512i nib, __m512 table,
                                                                               __m512 sv) {
    __m512i idx = _mm512_and_si512(nib, _mm512_set1_epi32(0x7));
    __m512 mag = _mm512_permutexvar_ps(idx, table);
    __m512i sign = _mm512_slli_epi32(_mm512_and_si512(nib, _mm512_set1_epi32(0x8)), 28);
    return _mm512_mul_ps(_mm512_castsi512_ps(_mm512_xor_si512(_mm512_castps_si512(mag), sign)), sv);
}

__attribute__((target("avx512f,avx512bw"))) static float dot_mxfp4_avx512(const uint8_t *w, const uint8_t *bs,
                                                                        const float *xs, size_t n) {
    const __m128i m4 = _mm_set1_epi8(0x0F);
    float t16[16];
    for (int j = 0; j < 16; j++) t16[j] = TABLE8[j & 7];
    const __m512 table = _mm512_loadu_ps(t16);
    __m512 acc0 = _mm512_setzero_ps(), acc1 = _mm512_setzero_ps();
    size_t i = 0;
    for (; i + 32 <= n; i += 32) {
        __m512 sv = _mm512_set1_ps(orc_e8m0_decode(bs[i / 32]));
        __m128i by = _mm_loadu_si128((const __m128i *)(w + (i >> 1)));
        __m128i lo = _mm_and_si128(by, m4);
        __m128i hi = _mm_and_si128(_mm_srli_epi16(by, 4), m4);
        __m512i n0 = _mm512_cvtepu8_epi32(_mm_unpacklo_epi8(lo, hi));
        __m512i n1 = _mm512_cvtepu8_epi32(_mm_unpackhi_epi8(lo, hi));
        acc0 = _mm512_fmadd_ps(_mm512_loadu_ps(xs + i), decode16_avx512(n0, table, sv), acc0);
        acc1 = _mm512_fmadd_ps(_mm512_loadu_ps(xs + i + 16), decode16_avx512(n1, table, sv), acc1);
    }
    float a = _mm512_reduce_add_ps(_mm512_add_ps(acc0, acc1));
    for (; i < n; i++) {
        uint8_t byte = w[i >> 1];
        uint8_t nibble = (i & 1) == 0 ? (byte & 0xF) : (byte >> 4);
        a += xs[i] * orc_e2m1_decode(nibble) * orc_e8m0_decode(bs[i / 32]);
    }
    return a;
}

/* kernels.rs:751-773 / :775-797: rows in parallel, each (row, token) dot written straight to
 * y[s, o] (the reference's yt[o, s] scratch + transpose_so only exists to split rows across rayon
 * workers; the values are identical). */
void orc_matmul_mxfp4_avx2(float *y, const float *x, const uint8_t *data, const uint8_t *block_scale,
                           size_t s, size_t i, size_t o) {
    size_t rb = div_ceil(i, 2), bpr = div_ceil(i, 32);
#pragma omp parallel for schedule(static) num_threads(orc_nthreads_internal())
    for (long oi = 0; oi < (long)o; oi++)
        for (size_t si = 0; si < s; si++)
            y[si * o + (size_t)oi] = dot_mxfp4_avx2(data + (size_t)oi * rb, block_scale + (size_t)oi * bpr, x + si * i, i);
}

void orc_matmul_mxfp4_avx512(float *y, const float *x, const uint8_t *data, const uint8_t *block_scale,
                             size_t s, size_t i, size_t o) {
    size_t rb = div_ceil(i, 2), bpr = div_ceil(i, 32);
#pragma omp parallel for schedule(static) num_threads(orc_nthreads_internal())
    for (long oi = 0; oi < (long)o; oi++)
        for (size_t si = 0; si < s; si++)
            y[si * o + (size_t)oi] =
                dot_mxfp4_avx512(data + (size_t)oi * rb, block_scale + (size_t)oi * bpr, x + si * i, i);
}

int orc_matmul_mxfp4(float *y, const float *x, const uint8_t *data, const uint8_t *block_scale, size_t s,
                     size_t i, size_t o) {
    if (orc_cpu_has_avx512()) { orc_matmul_mxfp4_avx512(y, x, data, block_scale, s, i, o); return 512; }
    if (orc_cpu_has_avx2()) { orc_matmul_mxfp4_avx2(y, x, data, block_scale, s, i, o); return 2; }
    orc_matmul_mxfp4_scalar(y, x, data, block_scale, s, i, o);
    return 0;
}
