/* Normal deviates for the synthetic models, bit-identical on the host and on
 * the device.
 *
 * Box-Muller from one 64-bit draw: u1, u2 are its two 32-bit halves as
 * (h + 0.5) / 2^32, and the pair is r cos(2 pi u2), r sin(2 pi u2) with
 * r = sqrt(-2 log u1), evaluated in double and rounded to float. The C
 * library's and the device library's log / sqrt / sin / cos differ from each
 * other in last bits, so they are not used: log, sqrt and the sine and cosine
 * are evaluated here from IEEE +, -, *, / (round to nearest even, never
 * contracted: both compilers run with -ffp-contract=off) and the exact
 * scalings ldexp / frexp, in one fixed order, so the host C generator and the
 * HIP generator write the same bytes.
 *
 * The includer defines KR_NORMAL_FN, the qualifiers of these functions
 * (`static inline` in C, `static __device__ inline` in HIP), before including. */
#ifndef KR_NORMAL_FN
#error "define KR_NORMAL_FN before including kr_normal.h"
#endif

/* log(v * 2^-33) for an odd v in [1, 2^33): v * 2^-e = m in [1, 2) with e the
 * bit length of v minus one, moved to [sqrt(1/2), sqrt(2)); then
 * log m = 2 atanh(s), s = (m - 1) / (m + 1), |s| <= 0.1716, as the odd series
 * in s through s^25 (truncation below 1e-19 relative). */
KR_NORMAL_FN double krn_log_u(unsigned long long v) {
    int e = 63 - __builtin_clzll(v);
    double m = ldexp((double)v, -e);
    if (m > 1.4142135623730951) {
        m = m * 0.5;
        e = e + 1;
    }
    const double s = (m - 1.0) / (m + 1.0), z = s * s;
    double p = 1.0 / 25.0;
    p = p * z + 1.0 / 23.0;
    p = p * z + 1.0 / 21.0;
    p = p * z + 1.0 / 19.0;
    p = p * z + 1.0 / 17.0;
    p = p * z + 1.0 / 15.0;
    p = p * z + 1.0 / 13.0;
    p = p * z + 1.0 / 11.0;
    p = p * z + 1.0 / 9.0;
    p = p * z + 1.0 / 7.0;
    p = p * z + 1.0 / 5.0;
    p = p * z + 1.0 / 3.0;
    const double ls = 2.0 * (s + (s * z) * p);
    return ls + (double)(e - 33) * 0.6931471805599453;
}

/* sqrt(y), y > 0: y = f 2^k with f in [0.5, 2) and k even; six Newton steps
 * x = (x + f / x) / 2 from a linear first guess (within 3% on [0.5, 2)),
 * then the exact scaling by 2^(k / 2). */
KR_NORMAL_FN double krn_sqrt(double y) {
    int k;
    double f = frexp(y, &k);
    if (k & 1) {
        f = f * 2.0;
        k = k - 1;
    }
    double x = 0.41731 + 0.59016 * f;
    for (int i = 0; i < 6; i++) x = 0.5 * (x + f / x);
    return ldexp(x, k / 2);
}

/* cos and sin of 2 pi u, u = (2 w + 1) 2^-33: with v = 4 u (exact),
 * k = the nearest integer to v (never a tie: v is an odd multiple of 2^-31)
 * and f = v - k (exact), the angle is (k + f) pi / 2; x = f pi / 2 lies in
 * [-pi/4, pi/4], where the Taylor series through x^21 / x^20 are within
 * 1e-21; the quadrant k picks the signs and the swap. */
KR_NORMAL_FN void krn_cossin_2pi(unsigned long long w2, double *c, double *s) {
    const double v = ldexp((double)w2, -31);
    const int k = (int)(v + 0.5);
    const double x = (v - (double)k) * 1.5707963267948966, z = x * x;
    double ps = -1.0 / 51090942171709440000.0;   /* -1/21! */
    ps = ps * z + 1.0 / 121645100408832000.0;    /* 1/19! */
    ps = ps * z - 1.0 / 355687428096000.0;       /* 1/17! */
    ps = ps * z + 1.0 / 1307674368000.0;         /* 1/15! */
    ps = ps * z - 1.0 / 6227020800.0;            /* 1/13! */
    ps = ps * z + 1.0 / 39916800.0;              /* 1/11! */
    ps = ps * z - 1.0 / 362880.0;                /* 1/9! */
    ps = ps * z + 1.0 / 5040.0;                  /* 1/7! */
    ps = ps * z - 1.0 / 120.0;                   /* 1/5! */
    ps = ps * z + 1.0 / 6.0;                     /* 1/3! (the sign below) */
    const double sn = x - (x * z) * ps;
    double pc = 1.0 / 2432902008176640000.0;     /* 1/20! */
    pc = pc * z - 1.0 / 6402373705728000.0;      /* 1/18! */
    pc = pc * z + 1.0 / 20922789888000.0;        /* 1/16! */
    pc = pc * z - 1.0 / 87178291200.0;           /* 1/14! */
    pc = pc * z + 1.0 / 479001600.0;             /* 1/12! */
    pc = pc * z - 1.0 / 3628800.0;               /* 1/10! */
    pc = pc * z + 1.0 / 40320.0;                 /* 1/8! */
    pc = pc * z - 1.0 / 720.0;                   /* 1/6! */
    pc = pc * z + 1.0 / 24.0;                    /* 1/4! */
    pc = pc * z - 1.0 / 2.0;                     /* 1/2! */
    const double cs = 1.0 + z * pc;
    switch (k & 3) {
    case 0: *c = cs; *s = sn; break;
    case 1: *c = -sn; *s = cs; break;
    case 2: *c = -cs; *s = -sn; break;
    default: *c = sn; *s = -cs; break;
    }
}

/* the normal pair of one 64-bit draw z */
KR_NORMAL_FN void krn_pair(unsigned long long z, float *a, float *b) {
    const unsigned long long hi = z >> 32, lo = z & 0xffffffffULL;
    const double r = krn_sqrt(-2.0 * krn_log_u(2 * hi + 1));
    double c, s;
    krn_cossin_2pi(2 * lo + 1, &c, &s);
    *a = (float)(r * c);
    *b = (float)(r * s);
}
