// Ordered fp32 sums of non-negative terms, computed exactly but not one add
// at a time.
//
// The reference adds such terms in index order (rmsnorm's sum of squares,
// kernels/scalar/k_scalar.c:61; softmax's sum of exponentials,
// k_scalar.c:71-74): s = (((0 + t0) + t1) + ...) with one rounding per add.
// On one lane that is a chain of n dependent adds. Here the terms are split
// into chunks of L; the fp32 running sum at a chunk's start lies within a few
// ulps of the exact prefix, which a double-precision prefix sum estimates.
// Each chunk is therefore run from all SC_W consecutive floats around its
// estimate at once (one per lane of a wave). A walk over the chunks then
// picks, for the true running value, the matching end value: the same adds
// in the same order, so the same bits. A true value outside its chunk's
// window is run through that chunk one add at a time, so the result is exact
// whatever the terms; non-finite terms skip the speculation altogether.
#pragma once
#include "kr_numerics.h"

#include <utility>

namespace {

constexpr int SC_W = 64;             // candidate start values per chunk: one per lane
constexpr int SC_H = 32;             // window [estimate - 32 ulps, estimate + 31 ulps]
constexpr int SC_MAX_CHUNKS = 32;
constexpr int SC_LMIN = 128;         // chunk length, doubled while chunks > SC_MAX_CHUNKS
constexpr int SC_BLK = 128;          // terms per register block of a chain (8 VGPRs x 16 lanes)
constexpr unsigned SC_INVALID = 0xFFFFFFFFu;   // a negative NaN: never a sum of terms >= 0

__host__ __device__ constexpr int sc_chunk_len(int n) {
    int L = SC_LMIN;
    while ((n + L - 1) / L > SC_MAX_CHUNKS) L *= 2;
    return L;
}
__host__ __device__ constexpr int sc_chunks(int n) { return (n + sc_chunk_len(n) - 1) / sc_chunk_len(n); }
// floats of term space the caller provides: n rounded up to whole chunks
__host__ __device__ constexpr int sc_terms_cap(int n) { return sc_chunks(n) * sc_chunk_len(n); }
// bytes of LDS scratch kr_spec_sum<NT> needs beside the terms
__host__ __device__ constexpr int sc_lds_bytes(int n, int nt) {
    return sc_chunks(n) * SC_W * 4 + nt * 8 + sc_chunks(n) * 8 + sc_chunks(n) * 4 + 16;
}

// s + t[i0] + ... + t[i1 - 1], one add at a time (one lane)
__device__ __forceinline__ float sc_seq(const float *t, int i0, int i1, float s) {
#pragma unroll 8
    for (int i = i0; i < i1; i++) s = kr_fadd(s, t[i]);
    return s;
}

// s + (lane k of v's row of 16) for k = 0..15 in order: the term comes with
// the add (DPP row broadcast), so a chain step is one instruction
template <int K> __device__ __forceinline__ float sc_bcast(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x150 + K, 0xF, 0xF, false));
}
template <int... K>
__device__ __forceinline__ void sc_add16x4(float (&s)[4], const float (&v)[4], std::integer_sequence<int, K...>) {
    ((s[0] = kr_fadd(s[0], sc_bcast<K>(v[0])), s[1] = kr_fadd(s[1], sc_bcast<K>(v[1])),
      s[2] = kr_fadd(s[2], sc_bcast<K>(v[2])), s[3] = kr_fadd(s[3], sc_bcast<K>(v[3]))), ...);
}

// The ordered sum of t[0..n) (LDS, 16-byte aligned, room for sc_terms_cap(n)
// floats: the tail is zero-filled, and s + 0 == s for s >= +0) by all NT
// threads of the workgroup; every thread gets the result. lds:
// sc_lds_bytes(n, NT) bytes, 8-byte aligned. Terms are expected to be >= 0
// (others only make the walk fall back more often). Contains barriers: all
// threads must call it.
template <int NT>
__device__ __forceinline__ float kr_spec_sum(float *t, int n, unsigned char *lds) {
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int L = sc_chunk_len(n), C = sc_chunks(n);
    float *tab0 = (float *)lds;               // [C][SC_W] chunk end values per candidate
    double *part = (double *)(tab0 + C * SC_W);
    double *csum = part + NT;
    int *lo = (int *)(csum + C);              // first candidate's bits per chunk
    int *flag = lo + C;
    float *res = (float *)(flag + 1);

    for (int i = n + tid; i < C * L; i += NT) t[i] = 0.0f;
    if (tid == 0) *flag = 0;
    __syncthreads();
    // estimates: per-thread partial sums in double over P pieces per chunk,
    // chunk sums, then their exclusive prefix; non-finite terms flagged
    int P = NT / C;
    while (P & (P - 1)) P &= P - 1;           // a power of two
    if (P > L / 4) P = L / 4;
    const int seg = L / P;
    if (tid < C * P) {
        double acc = 0.0;
        bool bad = false;
        const float4 *q = (const float4 *)(t + tid * seg);
        for (int i = 0; i < seg / 4; i++) {
            const float4 v = q[i];
            const float M = 3.402823466e38f;   // FLT_MAX: NaN fails every comparison
            const bool fin = fabsf(v.x) <= M && fabsf(v.y) <= M && fabsf(v.z) <= M && fabsf(v.w) <= M;
            bad = bad || !fin;
            acc += (double)v.x + (double)v.y + (double)v.z + (double)v.w;
        }
        part[tid] = acc;
        if (bad) *flag = 1;
    }
    __syncthreads();
    if (tid < C) {
        double a = 0.0;
        for (int k = 0; k < P; k++) a += part[tid * P + k];
        csum[tid] = a;
    }
    __syncthreads();
    if (*flag) {
        if (tid == 0) *res = sc_seq(t, 0, n, 0.0f);
        __syncthreads();
        return *res;
    }
    if (tid < C) {
        double cs[SC_MAX_CHUNKS];
#pragma unroll
        for (int c = 0; c < SC_MAX_CHUNKS; c++) cs[c] = c < C ? csum[c] : 0.0;
        double e = 0.0;   // the exact prefix before chunk tid, to within double rounding
#pragma unroll
        for (int c = 0; c < SC_MAX_CHUNKS; c++) e += c < tid ? cs[c] : 0.0;
        lo[tid] = max(__float_as_int((float)e) - SC_H, 0);   // the window starts at +0 at the lowest
    }
    __syncthreads();
    // every chunk from every candidate start, 4 chunks per pass of a wave
    // (chunk ids past the end repeat the last chunk, unused); lane
    // (row r, column k) holds terms 16 j + k of a 128-term block in v[.][j]
    for (int c0 = wave; c0 < C; c0 += 4 * NW) {
        int cb[4];
        float s[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int c = min(c0 + k * NW, C - 1);
            cb[k] = c * L;
            s[k] = __int_as_float(lo[c] + lane);
        }
        for (int b0 = 0; b0 < L; b0 += SC_BLK) {
            float v[8][4];
#pragma unroll
            for (int j = 0; j < 8; j++)
#pragma unroll
                for (int k = 0; k < 4; k++) v[j][k] = t[cb[k] + b0 + 16 * j + (lane & 15)];
#pragma unroll
            for (int j = 0; j < 8; j++) sc_add16x4(s, v[j], std::make_integer_sequence<int, 16>());
        }
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (c0 + k * NW < C) tab0[(c0 + k * NW) * SC_W + lane] = s[k];
    }
    __syncthreads();
    // the walk, in wave 0: chunk c's end values sit in one register (lane w:
    // candidate w), so a step is a scalar subtract and compare on the
    // running value and one read of the lane it selects, with no branch (an
    // index out of the window is clamped and clears ok). Any miss: lane 0
    // walks again, one add at a time in the chunks whose window it left
    if (wave == 0) {
        float e[SC_MAX_CHUNKS];
        int l[SC_MAX_CHUNKS];
#pragma unroll
        for (int c = 0; c < SC_MAX_CHUNKS; c++) {
            e[c] = c < C ? tab0[c * SC_W + lane] : 0.0f;
            l[c] = __builtin_amdgcn_readfirstlane(c < C ? lo[c] : 0);
        }
        int sv = 0;   // bits of the running value: +0, candidate 0 of chunk 0
        bool ok = true;
#pragma unroll
        for (int c = 0; c < SC_MAX_CHUNKS; c++) {
            const unsigned idx = (unsigned)(sv - l[c]);
            const int nv = __builtin_amdgcn_readlane(__float_as_int(e[c]), (int)(idx & (SC_W - 1)));
            if (c < C) {
                ok = ok && idx < (unsigned)SC_W;
                sv = nv;
            }
        }
        if (lane == 0) {
            float f = __int_as_float(sv);
            if (!ok) {
                f = 0.0f;
                for (int c = 0; c < C; c++) {
                    const int idx = __float_as_int(f) - lo[c];
                    if ((unsigned)idx < (unsigned)SC_W) f = tab0[c * SC_W + idx];
                    else f = sc_seq(t, c * L, c * L + L, f);
                }
            }
            *res = f;
        }
    }
    __syncthreads();
    return *res;
}

}  // namespace
