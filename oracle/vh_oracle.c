/*
 * vh_oracle.c -- CPU oracle for the vector-hip kNN / k-means / IVF-PQ hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, in C, the reference's CPU
 * path (the Rust crates vector-simd, vector-index::flat, vector-index::ivf::kmeans
 * and vector-cuda::knn::search_batch_cpu) so that the HIP library can be checked
 * against it on identical inputs.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  The product library never links it.
 *
 * Parity status per function (how each is pinned is listed in tests/test_oracle.py):
 *   vho_distance (all 10 metrics, scalar/AVX2/AVX-512)   pinned: reference KATs + brute force in double
 *   vho_knn_search_batch / vho_flat_search              pinned: reference KATs + sorted brute force
 *   vho_top_k_reduce                                    pinned: reference KATs (collective.rs tests)
 *   vho_kmeans_step / vho_kmeans_fit                    pinned: reference KATs + closed-form means
 *   vho_hamming_packed_knn                              pinned: identity with float-Hamming on unpacked codes
 *   vho_pq_encode / vho_pq_adc_lut                      pinned: reference KATs (pq.rs tests) + brute force in double
 *   vho_pq_distance_with_lut                            pinned: reference KATs + the closed-form sum on integer tables
 *   vho_find_top_centroids                              pinned: full sort in double on tiny inputs
 *   vho_ivfpq_search                                    pinned: brute-force ADC top-k on tiny indexes + reference KATs
 *   Empty-cluster reseeding and random init: parity unpinned (the reference uses an unseeded
 *   thread_rng); this oracle keeps the old centroid, like kmeans.cu:350-356.
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define VHO_EXPORT __attribute__((visibility("default")))

/* Metric codes: the reference's kernel codes (vector-cuda/src/knn.rs:235-246). */
enum { M_L2 = 0, M_DOT = 1, M_COS = 2, M_L1 = 3, M_MINK = 4, M_LINF = 5,
       M_HAM = 6, M_MAHA = 7, M_JACC = 8, M_HELL = 9 };

/* DistanceMetric::higher_is_better (vector-index/src/lib.rs:89-94). */
static int higher_is_better(int m) { return m == M_DOT || m == M_COS; }

/* ------------------------------------------------------------------------- */
/* Scalar backend: vector-simd/src/scalar.rs:14-263                           */
/* ------------------------------------------------------------------------- */
static float sc_dot(const float *a, const float *b, size_t n) {            /* scalar.rs:14-22 */
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) s += a[i] * b[i];
    return s;
}
static float sc_l2(const float *a, const float *b, size_t n) {             /* scalar.rs:35-44 */
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) { float d = a[i] - b[i]; s += d * d; }
    return s;
}
static float sc_cos(const float *a, const float *b, size_t n) {            /* scalar.rs:56-75 */
    float dot = 0.0f, na = 0.0f, nb = 0.0f;
    for (size_t i = 0; i < n; ++i) { dot += a[i] * b[i]; na += a[i] * a[i]; nb += b[i] * b[i]; }
    float den = sqrtf(na) * sqrtf(nb);
    return den <= 1e-9f ? 0.0f : dot / den;
}
static float sc_l1(const float *a, const float *b, size_t n) {             /* scalar.rs:81-89 */
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) s += fabsf(a[i] - b[i]);
    return s;
}
static float sc_mink3(const float *a, const float *b, size_t n) {          /* scalar.rs:103-109 (p=3 branch) */
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) { float d = fabsf(a[i] - b[i]); s += d * d * d; }
    return cbrtf(s);
}
static float sc_linf(const float *a, const float *b, size_t n) {           /* scalar.rs:123-137 */
    if (n == 0) return 0.0f;
    float m = 0.0f;
    for (size_t i = 0; i < n; ++i) { float d = fabsf(a[i] - b[i]); if (d > m) m = d; }
    return m;
}
static float sc_ham(const float *a, const float *b, size_t n) {            /* scalar.rs:143-153 */
    float c = 0.0f;
    for (size_t i = 0; i < n; ++i) if (fabsf(a[i] - b[i]) > 1e-6f) c += 1.0f;
    return c;
}
static float sc_maha(const float *a, const float *b, size_t n) {           /* scalar.rs:215-224 */
    return sqrtf(sc_l2(a, b, n));
}
static float sc_jacc(const float *a, const float *b, size_t n) {           /* scalar.rs:230-248 */
    float smin = 0.0f, smax = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        float x = fabsf(a[i]), y = fabsf(b[i]);
        smin += fminf(x, y); smax += fmaxf(x, y);
    }
    return smax <= 1e-9f ? 0.0f : 1.0f - smin / smax;
}
static float sc_hell(const float *a, const float *b, size_t n) {           /* scalar.rs:254-263 */
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) { float d = sqrtf(fabsf(a[i])) - sqrtf(fabsf(b[i])); s += d * d; }
    return sqrtf(0.5f * s);
}

/* ------------------------------------------------------------------------- */
/* AVX-512F backend: vector-simd/src/avx512.rs                               */
/* Same accumulator count, chunk width and tail order as the reference.       */
/* ------------------------------------------------------------------------- */
#define T512 __attribute__((target("avx512f")))
#define ABS512(v) _mm512_castsi512_ps(_mm512_and_si512(_mm512_castps_si512(v), _mm512_set1_epi32(0x7fffffff)))

T512 static float x5_dot(const float *a, const float *b, size_t n) {       /* avx512.rs:23-76 */
    __m512 s0 = _mm512_setzero_ps(), s1 = s0, s2 = s0, s3 = s0;
    size_t chunks = n / 64, i;
    for (size_t c = 0; c < chunks; ++c) {
        size_t o = c * 64;
        s0 = _mm512_fmadd_ps(_mm512_loadu_ps(a + o), _mm512_loadu_ps(b + o), s0);
        s1 = _mm512_fmadd_ps(_mm512_loadu_ps(a + o + 16), _mm512_loadu_ps(b + o + 16), s1);
        s2 = _mm512_fmadd_ps(_mm512_loadu_ps(a + o + 32), _mm512_loadu_ps(b + o + 32), s2);
        s3 = _mm512_fmadd_ps(_mm512_loadu_ps(a + o + 48), _mm512_loadu_ps(b + o + 48), s3);
    }
    for (i = chunks * 64; i + 16 <= n; i += 16)
        s0 = _mm512_fmadd_ps(_mm512_loadu_ps(a + i), _mm512_loadu_ps(b + i), s0);
    s0 = _mm512_add_ps(s0, s1); s2 = _mm512_add_ps(s2, s3); s0 = _mm512_add_ps(s0, s2);
    float r = _mm512_reduce_add_ps(s0);
    for (; i < n; ++i) r += a[i] * b[i];
    return r;
}
T512 static float x5_l2(const float *a, const float *b, size_t n) {        /* avx512.rs:87-148 */
    __m512 s0 = _mm512_setzero_ps(), s1 = s0, s2 = s0, s3 = s0, d;
    size_t chunks = n / 64, i;
    for (size_t c = 0; c < chunks; ++c) {
        size_t o = c * 64;
        d = _mm512_sub_ps(_mm512_loadu_ps(a + o), _mm512_loadu_ps(b + o));           s0 = _mm512_fmadd_ps(d, d, s0);
        d = _mm512_sub_ps(_mm512_loadu_ps(a + o + 16), _mm512_loadu_ps(b + o + 16)); s1 = _mm512_fmadd_ps(d, d, s1);
        d = _mm512_sub_ps(_mm512_loadu_ps(a + o + 32), _mm512_loadu_ps(b + o + 32)); s2 = _mm512_fmadd_ps(d, d, s2);
        d = _mm512_sub_ps(_mm512_loadu_ps(a + o + 48), _mm512_loadu_ps(b + o + 48)); s3 = _mm512_fmadd_ps(d, d, s3);
    }
    for (i = chunks * 64; i + 16 <= n; i += 16) {
        d = _mm512_sub_ps(_mm512_loadu_ps(a + i), _mm512_loadu_ps(b + i));
        s0 = _mm512_fmadd_ps(d, d, s0);
    }
    s0 = _mm512_add_ps(s0, s1); s2 = _mm512_add_ps(s2, s3); s0 = _mm512_add_ps(s0, s2);
    float r = _mm512_reduce_add_ps(s0);
    for (; i < n; ++i) { float t = a[i] - b[i]; r += t * t; }
    return r;
}
T512 static float x5_cos(const float *a, const float *b, size_t n) {       /* avx512.rs:161-223 */
    __m512 d0 = _mm512_setzero_ps(), d1 = d0, na0 = d0, na1 = d0, nb0 = d0, nb1 = d0;
    size_t chunks = n / 32, i;
    for (size_t c = 0; c < chunks; ++c) {
        size_t o = c * 32;
        __m512 a0 = _mm512_loadu_ps(a + o), b0 = _mm512_loadu_ps(b + o);
        d0 = _mm512_fmadd_ps(a0, b0, d0); na0 = _mm512_fmadd_ps(a0, a0, na0); nb0 = _mm512_fmadd_ps(b0, b0, nb0);
        __m512 a1 = _mm512_loadu_ps(a + o + 16), b1 = _mm512_loadu_ps(b + o + 16);
        d1 = _mm512_fmadd_ps(a1, b1, d1); na1 = _mm512_fmadd_ps(a1, a1, na1); nb1 = _mm512_fmadd_ps(b1, b1, nb1);
    }
    for (i = chunks * 32; i + 16 <= n; i += 16) {
        __m512 av = _mm512_loadu_ps(a + i), bv = _mm512_loadu_ps(b + i);
        d0 = _mm512_fmadd_ps(av, bv, d0); na0 = _mm512_fmadd_ps(av, av, na0); nb0 = _mm512_fmadd_ps(bv, bv, nb0);
    }
    d0 = _mm512_add_ps(d0, d1); na0 = _mm512_add_ps(na0, na1); nb0 = _mm512_add_ps(nb0, nb1);
    float dr = _mm512_reduce_add_ps(d0), nar = _mm512_reduce_add_ps(na0), nbr = _mm512_reduce_add_ps(nb0);
    for (; i < n; ++i) { dr += a[i] * b[i]; nar += a[i] * a[i]; nbr += b[i] * b[i]; }
    float den = sqrtf(nar) * sqrtf(nbr);
    return den <= 1e-9f ? 0.0f : dr / den;
}
T512 static float x5_l1(const float *a, const float *b, size_t n) {        /* avx512.rs:234-280 */
    __m512 s0 = _mm512_setzero_ps(), s1 = s0;
    size_t chunks = n / 32, i;
    for (size_t c = 0; c < chunks; ++c) {
        size_t o = c * 32;
        s0 = _mm512_add_ps(s0, ABS512(_mm512_sub_ps(_mm512_loadu_ps(a + o), _mm512_loadu_ps(b + o))));
        s1 = _mm512_add_ps(s1, ABS512(_mm512_sub_ps(_mm512_loadu_ps(a + o + 16), _mm512_loadu_ps(b + o + 16))));
    }
    for (i = chunks * 32; i + 16 <= n; i += 16)
        s0 = _mm512_add_ps(s0, ABS512(_mm512_sub_ps(_mm512_loadu_ps(a + i), _mm512_loadu_ps(b + i))));
    s0 = _mm512_add_ps(s0, s1);
    float r = _mm512_reduce_add_ps(s0);
    for (; i < n; ++i) r += fabsf(a[i] - b[i]);
    return r;
}
T512 static float x5_mink3(const float *a, const float *b, size_t n) {     /* avx512.rs:292-343 (p=3) */
    __m512 s0 = _mm512_setzero_ps(), s1 = s0;
    size_t chunks = n / 32, i;
    for (size_t c = 0; c < chunks; ++c) {
        size_t o = c * 32;
        __m512 d0 = ABS512(_mm512_sub_ps(_mm512_loadu_ps(a + o), _mm512_loadu_ps(b + o)));
        s0 = _mm512_fmadd_ps(_mm512_mul_ps(d0, d0), d0, s0);
        __m512 d1 = ABS512(_mm512_sub_ps(_mm512_loadu_ps(a + o + 16), _mm512_loadu_ps(b + o + 16)));
        s1 = _mm512_fmadd_ps(_mm512_mul_ps(d1, d1), d1, s1);
    }
    s0 = _mm512_add_ps(s0, s1);
    float s = _mm512_reduce_add_ps(s0);
    for (i = chunks * 32; i < n; ++i) { float d = fabsf(a[i] - b[i]); s += d * d * d; }
    return cbrtf(s);
}
T512 static float x5_linf(const float *a, const float *b, size_t n) {      /* avx512.rs:354-390 */
    if (n == 0) return 0.0f;
    __m512 m = _mm512_setzero_ps();
    size_t chunks = n / 16, i;
    for (size_t c = 0; c < chunks; ++c)
        m = _mm512_max_ps(m, ABS512(_mm512_sub_ps(_mm512_loadu_ps(a + c * 16), _mm512_loadu_ps(b + c * 16))));
    float r = _mm512_reduce_max_ps(m);
    for (i = chunks * 16; i < n; ++i) { float d = fabsf(a[i] - b[i]); if (d > r) r = d; }
    return r;
}
T512 static float x5_ham(const float *a, const float *b, size_t n) {       /* avx512.rs:403-436 */
    float cnt = 0.0f;
    const __m512 eps = _mm512_set1_ps(1e-6f);
    size_t chunks = n / 16, i;
    for (size_t c = 0; c < chunks; ++c) {
        __m512 d = ABS512(_mm512_sub_ps(_mm512_loadu_ps(a + c * 16), _mm512_loadu_ps(b + c * 16)));
        __mmask16 k = _mm512_cmp_ps_mask(d, eps, _CMP_GT_OQ);
        cnt += (float)__builtin_popcount((unsigned)k);
    }
    for (i = chunks * 16; i < n; ++i) if (fabsf(a[i] - b[i]) > 1e-6f) cnt += 1.0f;
    return cnt;
}
T512 static float x5_maha(const float *a, const float *b, size_t n) {      /* avx512.rs:516-518 */
    return sqrtf(x5_l2(a, b, n));
}
T512 static float x5_jacc(const float *a, const float *b, size_t n) {      /* avx512.rs:531-571 */
    __m512 mn = _mm512_setzero_ps(), mx = mn;
    size_t chunks = n / 16, i;
    for (size_t c = 0; c < chunks; ++c) {
        __m512 x = ABS512(_mm512_loadu_ps(a + c * 16)), y = ABS512(_mm512_loadu_ps(b + c * 16));
        mn = _mm512_add_ps(mn, _mm512_min_ps(x, y));
        mx = _mm512_add_ps(mx, _mm512_max_ps(x, y));
    }
    float smin = _mm512_reduce_add_ps(mn), smax = _mm512_reduce_add_ps(mx), rmin = 0.0f;
    for (i = chunks * 16; i < n; ++i) {
        float x = fabsf(a[i]), y = fabsf(b[i]);
        rmin += fminf(x, y); smax += fmaxf(x, y);
    }
    float tmin = smin + rmin;
    return smax <= 1e-9f ? 0.0f : 1.0f - tmin / smax;
}
T512 static float x5_hell(const float *a, const float *b, size_t n) {      /* avx512.rs:581-611 */
    __m512 s = _mm512_setzero_ps();
    size_t chunks = n / 16, i;
    for (size_t c = 0; c < chunks; ++c) {
        __m512 x = ABS512(_mm512_loadu_ps(a + c * 16)), y = ABS512(_mm512_loadu_ps(b + c * 16));
        __m512 d = _mm512_sub_ps(_mm512_sqrt_ps(x), _mm512_sqrt_ps(y));
        s = _mm512_fmadd_ps(d, d, s);
    }
    float r = _mm512_reduce_add_ps(s);
    for (i = chunks * 16; i < n; ++i) { float d = sqrtf(fabsf(a[i])) - sqrtf(fabsf(b[i])); r += d * d; }
    return sqrtf(0.5f * r);
}

/* ------------------------------------------------------------------------- */
/* AVX2+FMA backend: vector-simd/src/avx2.rs                                  */
/* ------------------------------------------------------------------------- */
#define T256 __attribute__((target("avx2,fma")))
#define ABS256(v) _mm256_and_ps(v, _mm256_castsi256_ps(_mm256_set1_epi32(0x7fffffff)))

T256 static float hsum256(__m256 v) {                                      /* avx2.rs:616-631 */
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    __m128 sh = _mm_movehdup_ps(s);
    __m128 ss = _mm_add_ps(s, sh);
    return _mm_cvtss_f32(_mm_add_ss(ss, _mm_movehl_ps(ss, ss)));
}
T256 static float x2_dot(const float *a, const float *b, size_t n) {       /* avx2.rs:23-76 */
    __m256 s0 = _mm256_setzero_ps(), s1 = s0, s2 = s0, s3 = s0;
    size_t chunks = n / 32, i;
    for (size_t c = 0; c < chunks; ++c) {
        size_t o = c * 32;
        s0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + o), _mm256_loadu_ps(b + o), s0);
        s1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + o + 8), _mm256_loadu_ps(b + o + 8), s1);
        s2 = _mm256_fmadd_ps(_mm256_loadu_ps(a + o + 16), _mm256_loadu_ps(b + o + 16), s2);
        s3 = _mm256_fmadd_ps(_mm256_loadu_ps(a + o + 24), _mm256_loadu_ps(b + o + 24), s3);
    }
    for (i = chunks * 32; i + 8 <= n; i += 8)
        s0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), s0);
    s0 = _mm256_add_ps(s0, s1); s2 = _mm256_add_ps(s2, s3); s0 = _mm256_add_ps(s0, s2);
    float r = hsum256(s0);
    for (; i < n; ++i) r += a[i] * b[i];
    return r;
}
T256 static float x2_l2(const float *a, const float *b, size_t n) {        /* avx2.rs:87-148 */
    __m256 s0 = _mm256_setzero_ps(), s1 = s0, s2 = s0, s3 = s0, d;
    size_t chunks = n / 32, i;
    for (size_t c = 0; c < chunks; ++c) {
        size_t o = c * 32;
        d = _mm256_sub_ps(_mm256_loadu_ps(a + o), _mm256_loadu_ps(b + o));           s0 = _mm256_fmadd_ps(d, d, s0);
        d = _mm256_sub_ps(_mm256_loadu_ps(a + o + 8), _mm256_loadu_ps(b + o + 8));   s1 = _mm256_fmadd_ps(d, d, s1);
        d = _mm256_sub_ps(_mm256_loadu_ps(a + o + 16), _mm256_loadu_ps(b + o + 16)); s2 = _mm256_fmadd_ps(d, d, s2);
        d = _mm256_sub_ps(_mm256_loadu_ps(a + o + 24), _mm256_loadu_ps(b + o + 24)); s3 = _mm256_fmadd_ps(d, d, s3);
    }
    for (i = chunks * 32; i + 8 <= n; i += 8) {
        d = _mm256_sub_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i));
        s0 = _mm256_fmadd_ps(d, d, s0);
    }
    s0 = _mm256_add_ps(s0, s1); s2 = _mm256_add_ps(s2, s3); s0 = _mm256_add_ps(s0, s2);
    float r = hsum256(s0);
    for (; i < n; ++i) { float t = a[i] - b[i]; r += t * t; }
    return r;
}
T256 static float x2_cos(const float *a, const float *b, size_t n) {       /* avx2.rs:161-223 */
    __m256 d0 = _mm256_setzero_ps(), d1 = d0, na0 = d0, na1 = d0, nb0 = d0, nb1 = d0;
    size_t chunks = n / 16, i;
    for (size_t c = 0; c < chunks; ++c) {
        size_t o = c * 16;
        __m256 a0 = _mm256_loadu_ps(a + o), b0 = _mm256_loadu_ps(b + o);
        d0 = _mm256_fmadd_ps(a0, b0, d0); na0 = _mm256_fmadd_ps(a0, a0, na0); nb0 = _mm256_fmadd_ps(b0, b0, nb0);
        __m256 a1 = _mm256_loadu_ps(a + o + 8), b1 = _mm256_loadu_ps(b + o + 8);
        d1 = _mm256_fmadd_ps(a1, b1, d1); na1 = _mm256_fmadd_ps(a1, a1, na1); nb1 = _mm256_fmadd_ps(b1, b1, nb1);
    }
    for (i = chunks * 16; i + 8 <= n; i += 8) {
        __m256 av = _mm256_loadu_ps(a + i), bv = _mm256_loadu_ps(b + i);
        d0 = _mm256_fmadd_ps(av, bv, d0); na0 = _mm256_fmadd_ps(av, av, na0); nb0 = _mm256_fmadd_ps(bv, bv, nb0);
    }
    d0 = _mm256_add_ps(d0, d1); na0 = _mm256_add_ps(na0, na1); nb0 = _mm256_add_ps(nb0, nb1);
    float dr = hsum256(d0), nar = hsum256(na0), nbr = hsum256(nb0);
    for (; i < n; ++i) { dr += a[i] * b[i]; nar += a[i] * a[i]; nbr += b[i] * b[i]; }
    float den = sqrtf(nar) * sqrtf(nbr);
    return den <= 1e-9f ? 0.0f : dr / den;
}
T256 static float x2_l1(const float *a, const float *b, size_t n) {        /* avx2.rs:234-285 */
    __m256 s0 = _mm256_setzero_ps(), s1 = s0;
    size_t chunks = n / 16, i;
    for (size_t c = 0; c < chunks; ++c) {
        size_t o = c * 16;
        s0 = _mm256_add_ps(s0, ABS256(_mm256_sub_ps(_mm256_loadu_ps(a + o), _mm256_loadu_ps(b + o))));
        s1 = _mm256_add_ps(s1, ABS256(_mm256_sub_ps(_mm256_loadu_ps(a + o + 8), _mm256_loadu_ps(b + o + 8))));
    }
    for (i = chunks * 16; i + 8 <= n; i += 8)
        s0 = _mm256_add_ps(s0, ABS256(_mm256_sub_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i))));
    s0 = _mm256_add_ps(s0, s1);
    float r = hsum256(s0);
    for (; i < n; ++i) r += fabsf(a[i] - b[i]);
    return r;
}
T256 static float x2_mink3(const float *a, const float *b, size_t n) {     /* avx2.rs:292-343 (p=3) */
    __m256 s0 = _mm256_setzero_ps(), s1 = s0;
    size_t chunks = n / 16, i;
    for (size_t c = 0; c < chunks; ++c) {
        size_t o = c * 16;
        __m256 d0 = ABS256(_mm256_sub_ps(_mm256_loadu_ps(a + o), _mm256_loadu_ps(b + o)));
        s0 = _mm256_fmadd_ps(_mm256_mul_ps(d0, d0), d0, s0);
        __m256 d1 = ABS256(_mm256_sub_ps(_mm256_loadu_ps(a + o + 8), _mm256_loadu_ps(b + o + 8)));
        s1 = _mm256_fmadd_ps(_mm256_mul_ps(d1, d1), d1, s1);
    }
    s0 = _mm256_add_ps(s0, s1);
    float s = hsum256(s0);
    for (i = chunks * 16; i < n; ++i) { float d = fabsf(a[i] - b[i]); s += d * d * d; }
    return cbrtf(s);
}
T256 static float x2_linf(const float *a, const float *b, size_t n) {      /* avx2.rs:354-395 */
    if (n == 0) return 0.0f;
    __m256 m = _mm256_setzero_ps();
    size_t chunks = n / 8, i;
    for (size_t c = 0; c < chunks; ++c)
        m = _mm256_max_ps(m, ABS256(_mm256_sub_ps(_mm256_loadu_ps(a + c * 8), _mm256_loadu_ps(b + c * 8))));
    float arr[8];
    _mm256_storeu_ps(arr, m);
    float r = 0.0f;
    for (int j = 0; j < 8; ++j) r = fmaxf(r, arr[j]);
    for (i = chunks * 8; i < n; ++i) { float d = fabsf(a[i] - b[i]); if (d > r) r = d; }
    return r;
}
T256 static float x2_ham(const float *a, const float *b, size_t n) {       /* avx2.rs:405-440 */
    const __m256 eps = _mm256_set1_ps(1e-6f), one = _mm256_set1_ps(1.0f);
    __m256 cv = _mm256_setzero_ps();
    size_t chunks = n / 8, i;
    for (size_t c = 0; c < chunks; ++c) {
        __m256 d = ABS256(_mm256_sub_ps(_mm256_loadu_ps(a + c * 8), _mm256_loadu_ps(b + c * 8)));
        cv = _mm256_add_ps(cv, _mm256_and_ps(_mm256_cmp_ps(d, eps, _CMP_GT_OQ), one));
    }
    float cnt = hsum256(cv);
    for (i = chunks * 8; i < n; ++i) if (fabsf(a[i] - b[i]) > 1e-6f) cnt += 1.0f;
    return cnt;
}
T256 static float x2_maha(const float *a, const float *b, size_t n) {      /* avx2.rs:522-524 */
    return sqrtf(x2_l2(a, b, n));
}
T256 static float x2_jacc(const float *a, const float *b, size_t n) {      /* avx2.rs:537-575 */
    __m256 mn = _mm256_setzero_ps(), mx = mn;
    size_t chunks = n / 8, i;
    for (size_t c = 0; c < chunks; ++c) {
        __m256 x = ABS256(_mm256_loadu_ps(a + c * 8)), y = ABS256(_mm256_loadu_ps(b + c * 8));
        mn = _mm256_add_ps(mn, _mm256_min_ps(x, y));
        mx = _mm256_add_ps(mx, _mm256_max_ps(x, y));
    }
    float smin = hsum256(mn), smax = hsum256(mx);
    for (i = chunks * 8; i < n; ++i) {
        float x = fabsf(a[i]), y = fabsf(b[i]);
        smin += fminf(x, y); smax += fmaxf(x, y);
    }
    return smax <= 1e-9f ? 0.0f : 1.0f - smin / smax;
}
T256 static float x2_hell(const float *a, const float *b, size_t n) {      /* avx2.rs:585-612 */
    __m256 s = _mm256_setzero_ps();
    size_t chunks = n / 8, i;
    for (size_t c = 0; c < chunks; ++c) {
        __m256 x = ABS256(_mm256_loadu_ps(a + c * 8)), y = ABS256(_mm256_loadu_ps(b + c * 8));
        __m256 d = _mm256_sub_ps(_mm256_sqrt_ps(x), _mm256_sqrt_ps(y));
        s = _mm256_add_ps(s, _mm256_mul_ps(d, d));
    }
    float r = hsum256(s);
    for (i = chunks * 8; i < n; ++i) { float d = sqrtf(fabsf(a[i])) - sqrtf(fabsf(b[i])); r += d * d; }
    return sqrtf(0.5f * r);
}

/* ------------------------------------------------------------------------- */
/* Dispatch: DistanceEngine::auto + detect_best_backend (lib.rs:54-310)       */
/* backend: 0 scalar, 1 AVX2+FMA, 2 AVX-512F, -1 = auto                       */
/* ------------------------------------------------------------------------- */
typedef float (*dist_fn)(const float *, const float *, size_t);

static const dist_fn TABLE[3][10] = {
    {sc_l2, sc_dot, sc_cos, sc_l1, sc_mink3, sc_linf, sc_ham, sc_maha, sc_jacc, sc_hell},
    {x2_l2, x2_dot, x2_cos, x2_l1, x2_mink3, x2_linf, x2_ham, x2_maha, x2_jacc, x2_hell},
    {x5_l2, x5_dot, x5_cos, x5_l1, x5_mink3, x5_linf, x5_ham, x5_maha, x5_jacc, x5_hell},
};

VHO_EXPORT int vho_detect_backend(void) {                                  /* lib.rs:292-310 */
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512f")) return 2;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) return 1;
    return 0;
}

static dist_fn pick(int metric, int backend) {
    if (backend < 0) backend = vho_detect_backend();
    if (backend > 2) backend = 2;
    return TABLE[backend][metric];
}

VHO_EXPORT float vho_distance(int metric, const float *a, const float *b, size_t dim, int backend) {
    if (metric < 0 || metric > 9) return NAN;
    return pick(metric, backend)(a, b, dim);
}

/* Batch of pairwise distances: out[i] = d(a_i, b_i), rows of `dim` floats. */
VHO_EXPORT void vho_distance_rows(int metric, const float *a, const float *b, size_t rows, size_t dim,
                                  int backend, float *out) {
    dist_fn f = pick(metric, backend);
    for (size_t i = 0; i < rows; ++i) out[i] = f(a + i * dim, b + i * dim, dim);
}

/* ------------------------------------------------------------------------- */
/* std::collections::BinaryHeap restated (Rust std, max-heap by Ord).         */
/* The reference's top-k order among equal scores depends on these exact      */
/* sift rules, so they are reproduced: push = sift_up (moves while strictly    */
/* greater than parent); pop = swap root with last, sift_down_to_bottom, then  */
/* sift_up.  Ord compares f32 scores with partial_cmp, NaN treated as Equal.   */
/* ------------------------------------------------------------------------- */
typedef struct { float score; float dist; uint32_t id; } cand_t;

static int cmp_le(float a, float b) { return !(a > b); }      /* partial_cmp(..) != Greater */

static void heap_sift_up(cand_t *h, size_t start, size_t pos) {
    cand_t e = h[pos];
    while (pos > start) {
        size_t parent = (pos - 1) / 2;
        if (cmp_le(e.score, h[parent].score)) break;
        h[pos] = h[parent];
        pos = parent;
    }
    h[pos] = e;
}
static void heap_push(cand_t *h, size_t *len, cand_t c) {
    h[*len] = c;
    *len += 1;
    heap_sift_up(h, 0, *len - 1);
}
static void heap_sift_down_to_bottom(cand_t *h, size_t len, size_t pos) {
    size_t end = len, start = pos;
    cand_t e = h[pos];
    size_t child = 2 * pos + 1;
    while (end >= 2 && child <= end - 2) {
        child += cmp_le(h[child].score, h[child + 1].score) ? 1 : 0;
        h[pos] = h[child];
        pos = child;
        child = 2 * pos + 1;
    }
    if (end >= 1 && child == end - 1) { h[pos] = h[child]; pos = child; }
    h[pos] = e;
    heap_sift_up(h, start, pos);
}
static cand_t heap_pop(cand_t *h, size_t *len) {
    cand_t item = h[*len - 1];
    *len -= 1;
    if (*len > 0) {
        cand_t root = h[0];
        h[0] = item;
        item = root;
        heap_sift_down_to_bottom(h, *len, 0);
    }
    return item;
}
/* Bounded insert used by flat.rs:156-165, knn.rs:351-366 and collective.rs:134-150. */
static void heap_offer(cand_t *h, size_t *len, size_t k, cand_t c) {
    if (*len < k) {
        heap_push(h, len, c);
    } else if (*len > 0 && c.score < h[0].score) {
        (void)heap_pop(h, len);
        heap_push(h, len, c);
    }
}

/* ------------------------------------------------------------------------- */
/* CudaKnnEngine::search_batch_cpu (vector-cuda/src/knn.rs:312-377):           */
/* per query, scan ids ascending, bounded max-heap, pop all then reverse.      */
/* Returns best-first lists; out_len[q] = min(k, n).                           */
/* ------------------------------------------------------------------------- */
VHO_EXPORT int vho_knn_search_batch(const float *base, size_t n, size_t dim, int metric,
                                    const float *queries, size_t nq, size_t k, int backend, int threads,
                                    uint32_t *out_ids, float *out_dist, size_t *out_len) {
    if (metric < 0 || metric > 9) return -1;
    size_t ek = k < n ? k : n;
    dist_fn f = pick(metric, backend);
    int hib = higher_is_better(metric);
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#endif
    for (size_t q = 0; q < nq; ++q) {
        const float *qv = queries + q * dim;
        cand_t *heap = (cand_t *)malloc((ek + 1) * sizeof(cand_t));
        size_t len = 0;
        if (ek > 0) {
            for (size_t i = 0; i < n; ++i) {
                float d = f(qv, base + i * dim, dim);
                cand_t c = {hib ? -d : d, d, (uint32_t)i};
                heap_offer(heap, &len, ek, c);
            }
        }
        size_t m = len;
        out_len[q] = m;
        /* pop (worst first) then reverse -> best first (knn.rs:369-374) */
        for (size_t j = 0; j < m; ++j) {
            cand_t c = heap_pop(heap, &len);
            out_ids[q * k + (m - 1 - j)] = c.id;
            out_dist[q * k + (m - 1 - j)] = c.dist;
        }
        free(heap);
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* FlatIndex::search (vector-index/src/flat.rs:131-189): heap, then the heap's */
/* internal order stably sorted by distance (ascending, or descending for      */
/* similarity).  Returns number of results; -1 EmptyIndex.                     */
/* ------------------------------------------------------------------------- */
VHO_EXPORT long vho_flat_search(const float *base, size_t n, size_t dim, int metric, const float *query,
                                size_t k, int backend, uint32_t *out_ids, float *out_dist) {
    if (n == 0) return -1;
    size_t ek = k < n ? k : n;
    if (ek == 0) return 0;
    dist_fn f = pick(metric, backend);
    int hib = higher_is_better(metric);
    cand_t *heap = (cand_t *)malloc((ek + 1) * sizeof(cand_t));
    size_t len = 0;
    for (size_t i = 0; i < n; ++i) {
        float d = f(query, base + i * dim, dim);
        cand_t c = {hib ? -d : d, d, (uint32_t)i};
        heap_offer(heap, &len, ek, c);
    }
    /* stable insertion sort of the heap vector by raw distance */
    for (size_t i = 1; i < len; ++i) {
        cand_t e = heap[i];
        size_t j = i;
        while (j > 0 && (hib ? (heap[j - 1].dist < e.dist) : (heap[j - 1].dist > e.dist))) {
            heap[j] = heap[j - 1];
            --j;
        }
        heap[j] = e;
    }
    for (size_t i = 0; i < len; ++i) { out_ids[i] = heap[i].id; out_dist[i] = heap[i].dist; }
    free(heap);
    return (long)len;
}

/* ------------------------------------------------------------------------- */
/* CollectiveOps::top_k_reduce (vector-cuda/src/ddp/collective.rs:115-159).    */
/* lists: concatenated (id, dist) entries of all ranks in rank order.          */
/* ------------------------------------------------------------------------- */
VHO_EXPORT size_t vho_top_k_reduce(const uint32_t *ids, const float *dist, size_t total, size_t k, int metric,
                                   uint32_t *out_ids, float *out_dist) {
    if (k == 0 || total == 0) return 0;
    int hib = higher_is_better(metric);
    cand_t *heap = (cand_t *)malloc((k + 1) * sizeof(cand_t));
    size_t len = 0;
    for (size_t i = 0; i < total; ++i) {
        cand_t c = {hib ? -dist[i] : dist[i], dist[i], ids[i]};
        heap_offer(heap, &len, k, c);
    }
    size_t m = len;
    for (size_t j = 0; j < m; ++j) {
        cand_t c = heap_pop(heap, &len);
        out_ids[m - 1 - j] = c.id;
        out_dist[m - 1 - j] = c.dist;
    }
    free(heap);
    return m;
}

/* ------------------------------------------------------------------------- */
/* One Lloyd iteration: KMeans::fit body (vector-index/src/ivf/kmeans.rs:75-150) */
/* with find_nearest_centroid (:264-309, strict compare, lowest index wins).    */
/* Sums accumulate in f32 in ascending point order (one valid rayon schedule;  */
/* the reference's reduction order is nondeterministic).  Empty clusters keep  */
/* the old centroid (kmeans.cu:350-356) instead of a random reseed.            */
/* threads > 1 uses per-thread partial sums (CPU-baseline timing mode).        */
/* Outputs: assign[n], new centroids (in place), counts[k], shift (max), inertia. */
/* ------------------------------------------------------------------------- */
static void nearest(const float *x, const float *cent, size_t k, size_t dim, dist_fn f, int hib,
                    int32_t *best_idx, float *best_score) {
    size_t bi = 0;
    float bs = hib ? -INFINITY : INFINITY;
    for (size_t c = 0; c < k; ++c) {
        float d = f(x, cent + c * dim, dim);
        int better = hib ? (d > bs) : (d < bs);
        if (better) { bs = d; bi = c; }
    }
    *best_idx = (int32_t)bi;
    *best_score = bs;
}

VHO_EXPORT int vho_kmeans_step(const float *data, size_t n, size_t dim, float *centroids, size_t k, int metric,
                               int backend, int threads, int32_t *assign, int64_t *counts, float *shifts,
                               float *max_shift, float *inertia) {
    if (metric < 0 || metric > 9 || k == 0) return -1;
    dist_fn f = pick(metric, backend);
    int hib = higher_is_better(metric);
    int nt = 1;
#ifdef _OPENMP
    nt = threads > 0 ? threads : omp_get_max_threads();
#endif
    if (nt < 1) nt = 1;
    float *psum = (float *)calloc((size_t)nt * k * dim, sizeof(float));
    int64_t *pcnt = (int64_t *)calloc((size_t)nt * k, sizeof(int64_t));
    float *pin = (float *)calloc((size_t)nt, sizeof(float));
    if (nt == 1) {
        for (size_t i = 0; i < n; ++i) {
            int32_t b; float s;
            nearest(data + i * dim, centroids, k, dim, f, hib, &b, &s);
            if (assign) assign[i] = b;
            pcnt[b] += 1;
            for (size_t d = 0; d < dim; ++d) psum[(size_t)b * dim + d] += data[i * dim + d];
            pin[0] += s;
        }
    } else {
#ifdef _OPENMP
#pragma omp parallel num_threads(nt)
        {
            int t = omp_get_thread_num();
            float *ls = psum + (size_t)t * k * dim;
            int64_t *lc = pcnt + (size_t)t * k;
            float li = 0.0f;
#pragma omp for schedule(static)
            for (size_t i = 0; i < n; ++i) {
                int32_t b; float s;
                nearest(data + i * dim, centroids, k, dim, f, hib, &b, &s);
                if (assign) assign[i] = b;
                lc[b] += 1;
                for (size_t d = 0; d < dim; ++d) ls[(size_t)b * dim + d] += data[i * dim + d];
                li += s;
            }
            pin[t] = li;
        }
#endif
    }
    /* reduce partials in thread order (kmeans.rs:109-117) */
    for (int t = 1; t < nt; ++t) {
        for (size_t j = 0; j < k * dim; ++j) psum[j] += psum[(size_t)t * k * dim + j];
        for (size_t c = 0; c < k; ++c) pcnt[c] += pcnt[(size_t)t * k + c];
        pin[0] += pin[t];
    }
    /* update (ivf/kmeans.rs:126-150) */
    float ms = 0.0f;
    for (size_t c = 0; c < k; ++c) {
        if (counts) counts[c] = pcnt[c];
        float sh = 0.0f;
        if (pcnt[c] > 0) {
            float inv = 1.0f / (float)pcnt[c];
            for (size_t d = 0; d < dim; ++d) {
                float v = psum[c * dim + d] * inv;
                float df = v - centroids[c * dim + d];
                sh += df * df;
                centroids[c * dim + d] = v;
            }
            if (sh > ms) ms = sh;
        }
        if (shifts) shifts[c] = sh;
    }
    if (max_shift) *max_shift = ms;
    if (inertia) *inertia = pin[0];
    free(psum); free(pcnt); free(pin);
    return 0;
}

/* Full Lloyd fit from explicit initial centroids (KMeans::fit loop, :70-155):
 * runs up to max_iters iterations, breaks when max_shift <= tol.  Returns the
 * number of iterations run. */
VHO_EXPORT long vho_kmeans_fit(const float *data, size_t n, size_t dim, float *centroids, size_t k, int metric,
                               size_t max_iters, float tol, int backend, int threads, int32_t *assign,
                               float *inertia) {
    long it = 0;
    for (size_t i = 0; i < max_iters; ++i) {
        float ms = 0.0f;
        it = (long)i + 1;
        if (vho_kmeans_step(data, n, dim, centroids, k, metric, backend, threads, assign, NULL, NULL, &ms,
                            inertia) != 0)
            return -1;
        if (ms <= tol) break;
    }
    return it;
}

/* ------------------------------------------------------------------------- */
/* Packed-bit Hamming (extension, not in the reference): popcount(a XOR b).    */
/* Ties broken by lowest id, results ascending by (distance, id).  This equals  */
/* scalar.rs:143-153 on the codes unpacked to 0.0/1.0 floats.                  */
/* ------------------------------------------------------------------------- */
VHO_EXPORT uint32_t vho_hamming_packed(const uint32_t *a, const uint32_t *b, size_t words) {
    uint32_t d = 0;
    for (size_t w = 0; w < words; ++w) d += (uint32_t)__builtin_popcount(a[w] ^ b[w]);
    return d;
}

VHO_EXPORT int vho_hamming_packed_knn(const uint32_t *codes, size_t n, size_t words, const uint32_t *queries,
                                      size_t nq, size_t k, int threads, uint32_t *out_ids, uint32_t *out_dist,
                                      size_t *out_len) {
    size_t ek = k < n ? k : n;
    size_t maxd = words * 32;
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#endif
    for (size_t q = 0; q < nq; ++q) {
        /* counting select over the exact integer distance (0..maxd) */
        size_t *hist = (size_t *)calloc(maxd + 2, sizeof(size_t));
        uint16_t *dd = (uint16_t *)malloc(n * sizeof(uint16_t));
        const uint32_t *qv = queries + q * words;
        for (size_t i = 0; i < n; ++i) {
            uint32_t d = vho_hamming_packed(qv, codes + i * words, words);
            dd[i] = (uint16_t)d;
            hist[d] += 1;
        }
        /* offsets per distance value among the first ek results */
        size_t *pos = (size_t *)calloc(maxd + 2, sizeof(size_t));
        size_t acc = 0;
        for (size_t d = 0; d <= maxd; ++d) { pos[d] = acc; acc += hist[d]; }
        size_t outn = 0;
        for (size_t i = 0; i < n && outn < ek; ++i) {
            size_t d = dd[i];
            if (pos[d] < ek) {
                out_ids[q * k + pos[d]] = (uint32_t)i;
                out_dist[q * k + pos[d]] = (uint32_t)d;
                pos[d] += 1;
                outn += 1;
            }
        }
        out_len[q] = ek;
        free(hist); free(dd); free(pos);
    }
    return 0;
}

/* Unpack packed codes into 0.0/1.0 floats (bit j of word w -> element 32w+j). */
VHO_EXPORT void vho_unpack_bits(const uint32_t *codes, size_t n, size_t words, float *out) {
    for (size_t i = 0; i < n; ++i)
        for (size_t w = 0; w < words; ++w)
            for (int j = 0; j < 32; ++j)
                out[i * words * 32 + w * 32 + j] = (float)((codes[i * words + w] >> j) & 1u);
}

/* ------------------------------------------------------------------------- */
/* Product quantization (vector-index/src/ivf/pq.rs) and the IVF-PQ search     */
/* (vector-index/src/ivf/mod.rs).  Codebooks are M x Ks x ds floats, flat       */
/* (pq.rs:21-25); codes one byte per sub-space.                                 */
/* ------------------------------------------------------------------------- */
static int pq_shape_ok(size_t dim, size_t m_sub, size_t ks, int metric) {
    return metric >= 0 && metric <= 9 && m_sub > 0 && dim % m_sub == 0 && ks > 0 && ks <= 256;
}

/* ProductQuantizer::encode / encode_batch (pq.rs:178-214): per sub-space the
 * nearest sub-centroid of KMeans::find_nearest_centroid (ivf/kmeans.rs:262-309,
 * strict compare in ascending index, so the lowest index wins ties). */
VHO_EXPORT int vho_pq_encode(const float *data, size_t n, size_t dim, size_t m_sub, size_t ks,
                             const float *codebooks, int metric, int backend, uint8_t *out_codes) {
    if (!pq_shape_ok(dim, m_sub, ks, metric)) return -1;
    const size_t ds = dim / m_sub;
    dist_fn f = pick(metric, backend);
    int hib = higher_is_better(metric);
    for (size_t i = 0; i < n; ++i)
        for (size_t m = 0; m < m_sub; ++m) {
            int32_t b;
            float s;
            nearest(data + i * dim + m * ds, codebooks + m * ks * ds, ks, ds, f, hib, &b, &s);
            out_codes[i * m_sub + m] = (uint8_t)b;
        }
    return 0;
}

/* ProductQuantizer::compute_adc_lut (pq.rs:233-266): lut[m * ks + j] = metric of
 * query sub-vector m and sub-centroid (m, j), Minkowski with p = 3. */
VHO_EXPORT int vho_pq_adc_lut(const float *query, size_t dim, size_t m_sub, size_t ks, const float *codebooks,
                              int metric, int backend, float *lut) {
    if (!pq_shape_ok(dim, m_sub, ks, metric)) return -1;
    const size_t ds = dim / m_sub;
    dist_fn f = pick(metric, backend);
    for (size_t m = 0; m < m_sub; ++m)
        for (size_t j = 0; j < ks; ++j) lut[m * ks + j] = f(query + m * ds, codebooks + (m * ks + j) * ds, ds);
    return 0;
}

/* ProductQuantizer::compute_distance_with_lut (pq.rs:270-293): quads of codes
 * summed as (d0 + d1) + (d2 + d3) into the running total, then the remainder
 * one by one. */
VHO_EXPORT float vho_pq_distance_with_lut(const uint8_t *code, size_t m_sub, size_t ks, const float *lut) {
    float total = 0.0f;
    size_t m = 0;
    for (; m + 4 <= m_sub; m += 4) {
        const float d0 = lut[m * ks + code[m]];
        const float d1 = lut[(m + 1) * ks + code[m + 1]];
        const float d2 = lut[(m + 2) * ks + code[m + 2]];
        const float d3 = lut[(m + 3) * ks + code[m + 3]];
        total += (d0 + d1) + (d2 + d3);
    }
    for (; m < m_sub; ++m) total += lut[m * ks + code[m]];
    return total;
}

/* KMeans::find_top_centroids (ivf/kmeans.rs:311-356): every centroid scored, a
 * stable sort (descending for similarities) truncated to min(nprobe, k).  For
 * finite scores a stable sort equals the order by (score, index). */
typedef struct { float s; uint32_t i; int hib; } tc_t;
static int tc_cmp(const void *pa, const void *pb) {
    const tc_t *a = (const tc_t *)pa, *b = (const tc_t *)pb;
    if (a->s != b->s) {
        int a_first = a->hib ? (a->s > b->s) : (a->s < b->s);
        int b_first = a->hib ? (b->s > a->s) : (b->s < a->s);
        if (a_first) return -1;
        if (b_first) return 1;
    }
    return a->i < b->i ? -1 : (a->i > b->i);
}
VHO_EXPORT size_t vho_find_top_centroids(const float *query, const float *cent, size_t k, size_t dim, size_t nprobe,
                                         int metric, int backend, uint32_t *out_idx, float *out_score) {
    size_t p = nprobe < k ? nprobe : k;
    if (p == 0 || metric < 0 || metric > 9) return 0;
    dist_fn f = pick(metric, backend);
    tc_t *t = (tc_t *)malloc(k * sizeof(tc_t));
    for (size_t c = 0; c < k; ++c) {
        t[c].s = f(query, cent + c * dim, dim);
        t[c].i = (uint32_t)c;
        t[c].hib = higher_is_better(metric);
    }
    qsort(t, k, sizeof(tc_t), tc_cmp);
    for (size_t j = 0; j < p; ++j) {
        out_idx[j] = t[j].i;
        if (out_score) out_score[j] = t[j].s;
    }
    free(t);
    return p;
}

/* IvfPqIndex::search_with_nprobe (ivf/mod.rs:256-345) for one query, with the
 * coarse probe list given (best first, as find_top_centroids returns it).  Per
 * probed non-empty list: residual q - c, ADC table, every code scored with
 * compute_distance_with_lut and offered to the bounded BinaryHeap (strict
 * eviction); the heap is popped and reversed.  Lists in CSR form: list c holds
 * entries [list_off[c], list_off[c+1]) of ids / codes (M bytes each), in the
 * order IvfPqIndex::build appended them.  Returns the number of results. */
VHO_EXPORT size_t vho_ivfpq_search(const float *query, size_t dim, int metric, int backend, const float *coarse,
                                   size_t nlist, size_t m_sub, size_t ks, const float *codebooks,
                                   const uint64_t *list_off, const uint32_t *ids, const uint8_t *codes,
                                   const uint32_t *probes, size_t nprobe, size_t k, uint32_t *out_ids,
                                   float *out_dist) {
    if (k == 0 || !pq_shape_ok(dim, m_sub, ks, metric)) return 0;
    const int hib = higher_is_better(metric);
    float *res = (float *)malloc(dim * sizeof(float));
    float *lut = (float *)malloc(m_sub * ks * sizeof(float));
    cand_t *h = (cand_t *)malloc((k + 1) * sizeof(cand_t));
    size_t len = 0;
    for (size_t p = 0; p < nprobe; ++p) {
        const uint32_t c = probes[p];
        if (c >= nlist) continue;
        const uint64_t b = list_off[c], e = list_off[c + 1];
        if (b == e) continue;
        for (size_t d = 0; d < dim; ++d) res[d] = query[d] - coarse[(size_t)c * dim + d];
        vho_pq_adc_lut(res, dim, m_sub, ks, codebooks, metric, backend, lut);
        for (uint64_t i = b; i < e; ++i) {
            const float dist = vho_pq_distance_with_lut(codes + i * m_sub, m_sub, ks, lut);
            cand_t cd = {hib ? -dist : dist, dist, ids[i]};
            heap_offer(h, &len, k, cd);
        }
    }
    const size_t cnt = len;
    for (size_t j = cnt; j-- > 0;) {
        cand_t c = heap_pop(h, &len);
        out_ids[j] = c.id;
        out_dist[j] = c.dist;
    }
    free(res); free(lut); free(h);
    return cnt;
}
