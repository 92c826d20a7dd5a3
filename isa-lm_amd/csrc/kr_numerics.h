// Device numerics shared by every kernel. Every float operation whose
// rounding the scalar reference fixes goes through the helpers below: one
// IEEE operation each, rounded to nearest even. Contraction into fused
// multiply-adds is switched off for every file that includes this header
// (and on the command line), and division and square root are the correctly
// rounded ones (-fhip-fp32-correctly-rounded-divide-sqrt; checked against the
// host exhaustively for sqrt). HIP's __fsqrt_rn is not used: in this ROCm it
// is the approximate native square root.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#pragma clang fp contract(off)

__device__ __forceinline__ float kr_fadd(float a, float b) { return a + b; }
__device__ __forceinline__ float kr_fsub(float a, float b) { return a - b; }
__device__ __forceinline__ float kr_fmul(float a, float b) { return a * b; }
__device__ __forceinline__ float kr_fdiv(float a, float b) { return a / b; }
__device__ __forceinline__ float kr_fsqrt(float a) { return __builtin_sqrtf(a); }

#define KR_QK 32
#define KR_QUANT_TINY 1e-30f

// 2^(i/32) as doubles, minus (i << 47): the table of the C library's expf
// (ARM optimized-routines exp2f_data.c); each entry is the correctly rounded
// double of 2^(i/32) with the exponent bits of i/32 taken out.
__constant__ uint64_t kr_exp2_tab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
};

// expf with the C library's results, bit for bit: the reference's softmax and
// SiLU call glibc's expf (kernels/scalar/k_scalar.c:74, :97), whose x86-64 FMA
// build evaluates x*32/ln2 = k + r with two fused multiply-adds and
// 2^(k/32) * (1 + c2 r + (c0 r + c1) r^2) in double.
// The same expf with the table read from tab (a copy of kr_exp2_tab, e.g.
// in LDS) and the out-of-range cases selected rather than branched to: every
// lane runs the same instructions.
__device__ __forceinline__ float kr_expf_tab(float x, const uint64_t *tab) {
    const uint32_t ux = __float_as_uint(x);
    const uint32_t top = (ux >> 20) & 0x7ff;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd = kd - shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const double s = __longlong_as_double((long long)(tab[ki & 31] + (ki << 47)));
    const double p = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(p, r2, y);
    float res = (float)(y * s);
    if (top >= 0x42bu) {                       // |x| >= 88, inf or NaN
        res = x < -0x1.9fe368p6f ? 0.0f : res;
        res = x > 0x1.62e42ep6f ? __uint_as_float(0x7f800000u) : res;
        res = top >= 0x7f8u ? x + x : res;
        res = ux == 0xff800000u ? 0.0f : res;
    }
    return res;
}

__device__ __forceinline__ float kr_expf(float x) { return kr_expf_tab(x, kr_exp2_tab); }

// The C library's expm1f and tanhf, bit for bit: the reference's GELU and
// soft-capping call glibc's tanhf (kernels/scalar/k_scalar.c:100-105,
// ops/ops.c:98-101), which glibc 2.35 builds from the fdlibm algorithm:
// tanh(x) = 1 - 2/(expm1(2|x|) + 2) from |x| = 1, -t/(t + 2) with
// t = expm1(-2|x|) below; expm1 reduces x = k ln2 + r with the reduction's
// rounding error carried, fits r by a rational form in r^2/2 and scales by
// 2^k through the exponent bits. Checked on every float32 input against the
// host library.
__device__ __forceinline__ float kr_expm1f(float x) {
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f;
    const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f, Q4 = 4.0082177293e-06f,
                Q5 = -2.0109921195e-07f;
    unsigned hx = __float_as_uint(x);
    const unsigned neg = hx >> 31;
    hx &= 0x7fffffffu;
    if (hx >= 0x4195b844u) {
        if (hx >= 0x42b17218u) {
            if (hx > 0x7f800000u) return kr_fadd(x, x);
            if (hx == 0x7f800000u) return neg ? -1.0f : x;
            if (x > 8.8721679688e+01f) return __uint_as_float(0x7f800000u);
        }
        if (neg) return -1.0f;
    }
    float hi, lo, c = 0.0f;
    int k;
    if (hx > 0x3eb17218u) {
        if (hx < 0x3F851592u) {
            k = neg ? -1 : 1;
            hi = neg ? kr_fadd(x, ln2_hi) : kr_fsub(x, ln2_hi);
            lo = neg ? -ln2_lo : ln2_lo;
        } else {
            k = (int)kr_fadd(kr_fmul(invln2, x), neg ? -0.5f : 0.5f);
            const float t = (float)k;
            hi = kr_fsub(x, kr_fmul(t, ln2_hi));
            lo = kr_fmul(t, ln2_lo);
        }
        x = kr_fsub(hi, lo);
        c = kr_fsub(kr_fsub(hi, x), lo);
    } else if (hx < 0x33000000u) {
        return x;
    } else {
        k = 0;
    }
    const float hfx = kr_fmul(0.5f, x), hxs = kr_fmul(x, hfx);
    float r1 = kr_fmul(hxs, Q5);
    r1 = kr_fmul(hxs, kr_fadd(Q4, r1));
    r1 = kr_fmul(hxs, kr_fadd(Q3, r1));
    r1 = kr_fmul(hxs, kr_fadd(Q2, r1));
    r1 = kr_fadd(1.0f, kr_fmul(hxs, kr_fadd(Q1, r1)));
    const float t = kr_fsub(3.0f, kr_fmul(r1, hfx));
    float e = kr_fmul(hxs, kr_fdiv(kr_fsub(r1, t), kr_fsub(6.0f, kr_fmul(x, t))));
    if (k == 0) return kr_fsub(x, kr_fsub(kr_fmul(x, e), hxs));
    e = kr_fsub(kr_fmul(x, kr_fsub(e, c)), c);
    e = kr_fsub(e, hxs);
    if (k == -1) return kr_fsub(kr_fmul(0.5f, kr_fsub(x, e)), 0.5f);
    if (k == 1)
        return x < -0.25f ? kr_fmul(-2.0f, kr_fsub(e, kr_fadd(x, 0.5f))) : kr_fadd(1.0f, kr_fmul(2.0f, kr_fsub(x, e)));
    float y;
    if (k <= -2 || k > 56) {
        y = kr_fsub(1.0f, kr_fsub(e, x));
        y = k == 128 ? kr_fmul(kr_fmul(y, 2.0f), 0x1p127f) : __uint_as_float(__float_as_uint(y) + ((unsigned)k << 23));
        return kr_fsub(y, 1.0f);
    }
    if (k < 23) {
        y = kr_fsub(__uint_as_float(0x3f800000u - (0x1000000u >> k)), kr_fsub(e, x));
    } else {
        y = kr_fsub(x, kr_fadd(e, __uint_as_float((unsigned)(0x7f - k) << 23)));
        y = kr_fadd(y, 1.0f);
    }
    return __uint_as_float(__float_as_uint(y) + ((unsigned)k << 23));
}
__device__ __forceinline__ float kr_tanhf(float x) {
    const unsigned jx = __float_as_uint(x), ix = jx & 0x7fffffffu;
    if (ix >= 0x7f800000u) return (jx >> 31) ? kr_fsub(kr_fdiv(1.0f, x), 1.0f) : kr_fadd(kr_fdiv(1.0f, x), 1.0f);
    float z;
    if (ix < 0x41b00000u) {
        if (ix == 0) return x;
        if (ix < 0x24000000u) return kr_fmul(x, kr_fadd(1.0f, x));
        const float ax = __uint_as_float(ix);
        if (ix >= 0x3f800000u) {
            const float t = kr_expm1f(kr_fmul(2.0f, ax));
            z = kr_fsub(1.0f, kr_fdiv(2.0f, kr_fadd(t, 2.0f)));
        } else {
            const float t = kr_expm1f(kr_fmul(-2.0f, ax));
            z = kr_fdiv(-t, kr_fadd(t, 2.0f));
        }
    } else {
        z = 1.0f;
    }
    return (jx >> 31) ? -z : z;
}

// IEEE binary16 -> float32; exact for every input (subnormals included).
__device__ __forceinline__ float kr_h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// float32 -> IEEE binary16 bits as core/ml.c:39-53 gives them: round to
// nearest even (the conversion instruction in the default round mode, with
// half-precision subnormals kept), overflow to infinity, and every NaN to the
// quiet NaN 0x7e00 with the input's sign.
__device__ __forceinline__ uint16_t kr_f2h(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(((u >> 16) & 0x8000u) | 0x7e00u);
    return __half_as_ushort(__float2half_rn(f));
}

__device__ __forceinline__ float kr_scale(const void *d, size_t i, int d16) {
    return d16 ? kr_h2f(((const uint16_t *)d)[i]) : ((const float *)d)[i];
}

// One element of the Q8_0 rule (docs/file-format.md:133-144,
// kernels/scalar/k_scalar.c:52-54): trunc(x * id + copysign(0.5, x)),
// multiply then add, clamped to +-127, for id = 127 / m where m is the
// block's max |x| seeded with 0 (so m >= |x| for every non-NaN x, m >= the
// tiny bound). Then |fl(x * id)| <= fl(127 (1 + 2^-24)) = 127 + 2^-17 and the
// sum s lies within 127.5 + 2^-17 of 0: the conversion's truncation toward
// zero gives trunc(s), the upper clamp never acts, and fmaxf(s, -127) is the
// lower clamp before or after truncation alike. A NaN s (x NaN or infinite,
// or m infinite with x infinite) clamps to -127 as fmaxf(NaN, -127) does in
// the reference.
__device__ __forceinline__ int kr_q8_elem(float x, float id) {
    return (int)fmaxf(kr_fadd(kr_fmul(x, id), copysignf(0.5f, x)), -127.0f);
}

// Max over the 32 lanes of a half-wave (lanes 0-31 or 32-63). fmaxf is
// exact, so the order of the reduction does not matter.
__device__ __forceinline__ float kr_max32(float v) {
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 32));
    return v;
}

// Quantizes the 32 values held by the 32 lanes of a half-wave (lane j holds
// element j of the block) into q (this lane's element) and the block scale.
__device__ __forceinline__ void kr_quant_block32(float x, int8_t *q, float *d) {
    const float amax = fmaxf(kr_max32(fabsf(x)), 0.0f);   // seeded with 0: NaNs never raise it
    if (amax < KR_QUANT_TINY) {
        *q = 0;
        *d = 0.0f;
        return;
    }
    const float id = kr_fdiv(127.0f, amax);
    *d = kr_fdiv(amax, 127.0f);
    *q = (int8_t)kr_q8_elem(x, id);
}

__device__ __forceinline__ int kr_dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }
