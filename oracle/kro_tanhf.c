/* ORACLE -- test infrastructure only. The C library's tanhf, bit for bit.
 *
 * The reference's GELU and soft-capping call tanhf (kernels/scalar/k_scalar.c:
 * 100-105, ops/ops.c:98-101), which is glibc's; glibc 2.35 (this image's)
 * builds it from the fdlibm algorithm (sysdeps/ieee754/flt-32/s_tanhf.c over
 * s_expm1f.c): tanh(x) = 1 - 2/(expm1(2|x|) + 2) for |x| >= 1, else
 * -t/(t + 2) with t = expm1(-2|x|); x itself below 2^-55 (times 1 + x);
 * +-1 from 22 on. expm1 reduces x = k ln2 + r (ln2 split hi/lo, the
 * rounding error c carried), fits r with a rational form in r^2/2 (five
 * published coefficients), and rescales by 2^k in the exponent bits. Pinned
 * by kro_tanhf_mismatches: equal to the host libm over all 2^32 inputs. */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>
#include "kro.h"

static uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float kro_expm1f(float x) {
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f;
    const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f, Q4 = 4.0082177293e-06f,
                Q5 = -2.0109921195e-07f;
    uint32_t hx = fbits(x);
    const uint32_t neg = hx >> 31;
    hx &= 0x7fffffffu;
    if (hx >= 0x4195b844u) {            /* |x| >= 27 ln2 */
        if (hx >= 0x42b17218u) {        /* |x| >= 88.72...: NaN, inf, overflow */
            if (hx > 0x7f800000u) return x + x;
            if (hx == 0x7f800000u) return neg ? -1.0f : x;
            if (x > 8.8721679688e+01f) return 1.0e30f * 1.0e30f;
        }
        if (neg) return 1.0e-30f - 1.0f;   /* -1 */
    }
    float hi, lo, c = 0.0f;
    int k;
    if (hx > 0x3eb17218u) {             /* |x| > ln2 / 2: x = k ln2 + r */
        if (hx < 0x3F851592u) {         /* and < 1.5 ln2: k = +-1 */
            k = neg ? -1 : 1;
            hi = neg ? x + ln2_hi : x - ln2_hi;
            lo = neg ? -ln2_lo : ln2_lo;
        } else {
            k = (int)(invln2 * x + (neg ? -0.5f : 0.5f));
            const float t = (float)k;
            hi = x - t * ln2_hi;
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) {      /* |x| < 2^-25: x */
        const float t = 1.0e30f + x;
        return x - (t - (1.0e30f + x));
    } else {
        k = 0;
    }
    const float hfx = 0.5f * x, hxs = x * hfx;
    const float r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    const float t = 3.0f - r1 * hfx;
    float e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = (x * (e - c) - c);
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) return x < -0.25f ? -2.0f * (e - (x + 0.5f)) : 1.0f + 2.0f * (x - e);
    float y;
    if (k <= -2 || k > 56) {            /* 2^k (1 + r + ...) - 1 */
        y = 1.0f - (e - x);
        y = k == 128 ? y * 2.0f * 0x1p127f : bitsf(fbits(y) + ((uint32_t)k << 23));
        return y - 1.0f;
    }
    if (k < 23) {
        y = bitsf(0x3f800000u - (0x1000000u >> k)) - (e - x);   /* (1 - 2^-k) + ... */
    } else {
        y = x - (e + bitsf((uint32_t)(0x7f - k) << 23));
        y += 1.0f;
    }
    return bitsf(fbits(y) + ((uint32_t)k << 23));
}

float kro_tanhf(float x) {
    const uint32_t jx = fbits(x), ix = jx & 0x7fffffffu;
    if (ix >= 0x7f800000u) return (jx >> 31) ? 1.0f / x - 1.0f : 1.0f / x + 1.0f;   /* +-1, NaN */
    float z;
    if (ix < 0x41b00000u) {             /* |x| < 22 */
        if (ix == 0) return x;
        if (ix < 0x24000000u) return x * (1.0f + x);   /* |x| < 2^-55 */
        if (ix >= 0x3f800000u) {        /* |x| >= 1 */
            const float t = kro_expm1f(2.0f * fabsf(x));
            z = 1.0f - 2.0f / (t + 2.0f);
        } else {
            const float t = kro_expm1f(-2.0f * fabsf(x));
            z = -t / (t + 2.0f);
        }
    } else {
        z = 1.0f - 1.0e-30f;
    }
    return (jx >> 31) ? -z : z;
}

typedef struct { uint64_t lo, hi, bad; } span;

static void *scan(void *p) {
    span *s = p;
    for (uint64_t u = s->lo; u < s->hi; u++) {
        const float x = bitsf((uint32_t)u), a = tanhf(x), b = kro_tanhf(x);
        if (fbits(a) != fbits(b) && !(isnan(a) && isnan(b))) s->bad++;
        const float c = expm1f(x), d = kro_expm1f(x);
        if (fbits(c) != fbits(d) && !(isnan(c) && isnan(d))) s->bad++;
    }
    return NULL;
}

uint64_t kro_tanhf_mismatches(uint64_t lo, uint64_t hi, int threads) {
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
    for (int i = 0; i < threads; i++) {
        pthread_join(th[i], NULL);
        bad += sp[i].bad;
    }
    return bad;
}

typedef struct { uint64_t lo; const float *got; size_t i0, i1; uint64_t bad; } got_span;

static void *scan_got(void *p) {
    got_span *g = p;
    for (size_t i = g->i0; i < g->i1; i++) {
        const float a = tanhf(bitsf((uint32_t)(g->lo + i)));
        if (fbits(a) != fbits(g->got[i]) && !(isnan(a) && isnan(g->got[i]))) g->bad++;
    }
    return NULL;
}

uint64_t kro_tanhf_check_range(uint64_t lo, const float *got, size_t n, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t th[64];
    got_span sp[64];
    for (int i = 0; i < threads; i++) {
        sp[i] = (got_span){ lo, got, n * (size_t)i / (size_t)threads, n * (size_t)(i + 1) / (size_t)threads, 0 };
        pthread_create(&th[i], NULL, scan_got, &sp[i]);
    }
    uint64_t bad = 0;
    for (int i = 0; i < threads; i++) {
        pthread_join(th[i], NULL);
        bad += sp[i].bad;
    }
    return bad;
}
