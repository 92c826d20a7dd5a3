/* ORACLE — test infrastructure only.
 *
 * The reference's softmax and SiLU call the C library's expf
 * (kernels/scalar/k_scalar.c:74, :97). glibc is not vendored in the
 * reference; the build image has glibc 2.35, whose expf is the published
 * algorithm of ARM's optimized-routines (math/expf.c, exp2f_data.c, MIT
 * licence), selected in its FMA-compiled form on x86-64 CPUs with FMA:
 *
 *   z = x * 32/ln2;  k = round(z) via the 1.5*2^52 shift;  r = z - k
 *   2^(k/32) from a 32-entry table T[i] = bits(2^(i/32)) - (i << 47)
 *   exp(x) = 2^(k/32) * (1 + C2 r + (C0 r + C1) r^2), evaluated in double
 *
 * with z + shift and z - k each computed by one fused multiply-add, as the
 * compiler contracts them in the FMA build. The table entries are the
 * correctly rounded doubles of 2^(i/32); the three coefficients are the
 * library's published minimax values. tests/test_oracle.py checks this
 * function against the host libm on all 2^32 inputs; the unfused variant
 * differs on exactly 2 of them, so the check tells the two apart.
 */
#include <math.h>
#include <pthread.h>
#include <string.h>
#include "kro.h"

static const uint64_t EXP2_TAB[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
};

static double bits_d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }
static uint64_t d_bits(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float kro_expf(float x) {
    const uint32_t top = (f_bits(x) >> 20) & 0x7ff;
    if (top >= ((f_bits(88.0f) >> 20) & 0x7ff)) {          /* |x| >= 88 or NaN */
        if (f_bits(x) == f_bits(-INFINITY)) return 0.0f;
        if (top >= ((f_bits(INFINITY) >> 20) & 0x7ff)) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;             /* overflow */
        if (x < -0x1.9fe368p6f) return 0.0f;                 /* underflow */
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = fma(inv_ln2_n, xd, shift);
    const uint64_t ki = d_bits(kd);
    kd -= shift;
    const double r = fma(inv_ln2_n, xd, -kd);
    const double s = bits_d(EXP2_TAB[ki % 32] + (ki << 47));
    const double p = fma(c0, r, c1);
    const double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(p, r2, y);
    return (float)(y * s);
}

typedef struct { uint64_t lo, hi, bad; } span;

static void *scan(void *p) {
    span *sp = p;
    for (uint64_t u = sp->lo; u < sp->hi; u++) {
        const uint32_t b = (uint32_t)u;
        float x;
        memcpy(&x, &b, 4);
        const float ref = expf(x), got = kro_expf(x);
        if (f_bits(ref) != f_bits(got) && !(isnan(ref) && isnan(got))) sp->bad++;
    }
    return NULL;
}

uint64_t kro_expf_mismatches(uint64_t lo, uint64_t hi, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t th[64];
    span sp[64];
    for (int i = 0; i < threads; i++) {
        sp[i].lo = lo + (hi - lo) * (uint64_t)i / (uint64_t)threads;
        sp[i].hi = lo + (hi - lo) * (uint64_t)(i + 1) / (uint64_t)threads;
        sp[i].bad = 0;
        pthread_create(&th[i], NULL, scan, &sp[i]);
    }
    uint64_t bad = 0;
    for (int i = 0; i < threads; i++) { pthread_join(th[i], NULL); bad += sp[i].bad; }
    return bad;
}

uint64_t kro_expf_check(const float *x, const float *got, size_t n) {
    uint64_t bad = 0;
    for (size_t i = 0; i < n; i++) {
        const float ref = expf(x[i]);
        if (f_bits(ref) != f_bits(got[i]) && !(isnan(ref) && isnan(got[i]))) bad++;
    }
    return bad;
}

typedef struct { uint64_t lo; const float *got; size_t i0, i1; uint64_t bad; } got_span;

static void *scan_got(void *p) {
    got_span *g = p;
    for (size_t i = g->i0; i < g->i1; i++) {
        const uint32_t b = (uint32_t)(g->lo + i);
        float x;
        memcpy(&x, &b, 4);
        const float ref = expf(x);
        if (f_bits(ref) != f_bits(g->got[i]) && !(isnan(ref) && isnan(g->got[i]))) g->bad++;
    }
    return NULL;
}

uint64_t kro_expf_check_range(uint64_t lo, const float *got, size_t n, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t th[64];
    got_span g[64];
    for (int i = 0; i < threads; i++) {
        g[i] = (got_span){ lo, got, n * (size_t)i / (size_t)threads, n * (size_t)(i + 1) / (size_t)threads, 0 };
        pthread_create(&th[i], NULL, scan_got, &g[i]);
    }
    uint64_t bad = 0;
    for (int i = 0; i < threads; i++) { pthread_join(th[i], NULL); bad += g[i].bad; }
    return bad;
}
