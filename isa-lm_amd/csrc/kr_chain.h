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
    return sc_chunks(n) * SC_W * 4 + sc_chunks(n) * 8 + sc_chunks(n) * 4 + (nt / 64) * 4 + 16;
}

// s + t[i0] + ... + t[i1 - 1], one add at a time (one lane)
__device__ __forceinline__ float sc_seq(const float *t, int i0, int i1, float s) {
#pragma unroll 8
    for (int i = i0; i < i1; i++) s = kr_fadd(s, t[i]);
    return s;
}

// s + (lane k of v's row of 16) for k = 0..15 in order: the term comes with
// the add (DPP row broadcast), so a chain step is one instruction; 8 chains
// interleaved
template <int K> __device__ __forceinline__ float sc_bcast(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x150 + K, 0xF, 0xF, false));
}
template <int... K>
__device__ __forceinline__ void sc_add16x8(float (&s)[8], const float (&v)[8], std::integer_sequence<int, K...>) {
    ((s[0] = kr_fadd(s[0], sc_bcast<K>(v[0])), s[1] = kr_fadd(s[1], sc_bcast<K>(v[1])),
      s[2] = kr_fadd(s[2], sc_bcast<K>(v[2])), s[3] = kr_fadd(s[3], sc_bcast<K>(v[3])),
      s[4] = kr_fadd(s[4], sc_bcast<K>(v[4])), s[5] = kr_fadd(s[5], sc_bcast<K>(v[5])),
      s[6] = kr_fadd(s[6], sc_bcast<K>(v[6])), s[7] = kr_fadd(s[7], sc_bcast<K>(v[7]))), ...);
}

// The ordered sum s0 + t[0] + ... + t[n-1] (t in LDS, 16-byte aligned, room
// for sc_terms_cap(n) floats: the tail is zero-filled, and s + 0 == s for
// s >= +0) by all NT threads of the workgroup; every thread gets the result.
// lds: sc_lds_bytes(n, NT) bytes, 8-byte aligned. s0 and the terms are
// expected to be >= 0 (others only make the walk fall back more often).
// Contains barriers: all threads must call it.
//
// Wave w owns chunks w, w + NW, ... (SC_CPW of them at most): it sums them
// in double (16-term pieces per lane, reduced over 8 lanes), publishes the
// sums, then forms its own chunks' window starts from the published sums
// and runs their candidates, 8 chains interleaved.
constexpr int SC_CPW = 8;   // chunks per wave: C <= NW * SC_CPW
template <int NT>
__device__ __forceinline__ float kr_spec_sum(float *t, int n, unsigned char *lds, float s0 = 0.0f) {
    constexpr int NW = NT / 64;
    static_assert(NW * SC_CPW >= SC_MAX_CHUNKS, "every chunk needs a wave");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int L = sc_chunk_len(n), C = sc_chunks(n);
    float *tab0 = (float *)lds;               // [C][SC_W] chunk end values per candidate
    double *csum = (double *)(tab0 + C * SC_W);
    int *lo = (int *)(csum + C);              // first candidate's bits per chunk
    int *bad = lo + C;                        // [NW] a wave saw a non-finite term
    float *res = (float *)(bad + NW);

    if (n % L) {   // the last chunk's tail
        for (int i = n + tid; i < C * L; i += NT) t[i] = 0.0f;
        __syncthreads();
    }
    // this wave's chunk sums: lane (j, p) sums terms [16 q, 16 q + 16) for
    // q = p, p + 8, ... of chunk j of the wave, in double (two accumulators),
    // then the 8 lanes of a chunk add theirs; non-finite terms flagged
    {
        const int j = lane >> 3, p = lane & 7, c = wave + j * NW;
        double acc0 = 0.0, acc1 = 0.0;
        bool nf = false;
        if (c < C) {
            for (int q = p; q < L / 16; q += 8) {
                const float4 *r = (const float4 *)(t + c * L + 16 * q);
                const float4 v0 = r[0], v1 = r[1], v2 = r[2], v3 = r[3];
                const float M = 3.402823466e38f;   // FLT_MAX: NaN fails every comparison
                const float4 vs[4] = {v0, v1, v2, v3};
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float4 v = vs[k];
                    nf = nf || !(fabsf(v.x) <= M && fabsf(v.y) <= M && fabsf(v.z) <= M && fabsf(v.w) <= M);
                    acc0 += (double)v.x + (double)v.y;
                    acc1 += (double)v.z + (double)v.w;
                }
            }
        }
        double acc = acc0 + acc1;
        acc += __shfl_xor(acc, 1);
        acc += __shfl_xor(acc, 2);
        acc += __shfl_xor(acc, 4);
        const bool anynf = __any(nf);
        if (p == 0 && c < C) csum[c] = acc;
        if (lane == 0) bad[wave] = anynf;
    }
    __syncthreads();
    bool anybad = false;
#pragma unroll
    for (int w = 0; w < NW; w++) anybad = anybad || bad[w];
    if (anybad) {
        if (tid == 0) *res = sc_seq(t, 0, n, s0);
        __syncthreads();
        return *res;
    }
    // the window starts of this wave's chunks: lane j < SC_CPW sums the chunk
    // sums before chunk wave + j * NW (all read at once)
    int lov = 0;
    {
        double cs[SC_MAX_CHUNKS];
#pragma unroll
        for (int k = 0; k < SC_MAX_CHUNKS; k++) cs[k] = csum[min(k, C - 1)];
        const int c = wave + lane * NW;
        double e = (double)s0;   // the exact prefix before chunk c, to within double rounding
#pragma unroll
        for (int k = 0; k < SC_MAX_CHUNKS; k++) e += k < min(c, C) ? cs[k] : 0.0;
        lov = max(__float_as_int((float)e) - SC_H, 0);   // chunk 0: s0 is candidate SC_H (or lower near +0)
        if (lane < SC_CPW && c < C) lo[c] = lov;
    }
    // every candidate start of this wave's chunks at once (chunk ids past the
    // end repeat the wave's first chunk, unused); lane (row r, column k)
    // holds terms 16 i + k of a 128-term block in v[i][.]
    {
        int cb[SC_CPW];
        float s[SC_CPW];
#pragma unroll
        for (int j = 0; j < SC_CPW; j++) {
            const int c = wave + j * NW < C ? wave + j * NW : wave;
            cb[j] = c * L;
            s[j] = __int_as_float(__builtin_amdgcn_readlane(lov, j) + lane);
        }
        if (wave < C) {
            for (int b0 = 0; b0 < L; b0 += SC_BLK) {
                float v[8][SC_CPW];
#pragma unroll
                for (int i = 0; i < 8; i++)
#pragma unroll
                    for (int j = 0; j < SC_CPW; j++) v[i][j] = t[cb[j] + b0 + 16 * i + (lane & 15)];
#pragma unroll
                for (int i = 0; i < 8; i++) sc_add16x8(s, v[i], std::make_integer_sequence<int, 16>());
            }
#pragma unroll
            for (int j = 0; j < SC_CPW; j++)
                if (wave + j * NW < C) tab0[(wave + j * NW) * SC_W + lane] = s[j];
        }
    }
    __syncthreads();
    // the walk, in wave 0: chunk c's end values sit in one register (lane w:
    // candidate w), so a step is a scalar subtract and compare on the
    // running value and one read of the lane it selects, with no branch (an
    // index out of the window is clamped and clears ok). Any miss: lane 0
    // walks again, one add at a time in the chunks whose window it left
    if (wave == 0) {
        float e[SC_MAX_CHUNKS];
#pragma unroll
        for (int c = 0; c < SC_MAX_CHUNKS; c++) e[c] = tab0[min(c, C - 1) * SC_W + lane];   // all at once
        const int lv = lo[min(lane, C - 1)];
        int sv = __float_as_int(s0);   // bits of the running value
        bool ok = true;
#pragma unroll
        for (int c = 0; c < SC_MAX_CHUNKS; c++) {
            const unsigned idx = (unsigned)(sv - __builtin_amdgcn_readlane(lv, c));
            const int nv = __builtin_amdgcn_readlane(__float_as_int(e[c]), (int)(idx & (SC_W - 1)));
            if (c < C) {
                ok = ok && idx < (unsigned)SC_W;
                sv = nv;
            }
        }
        if (lane == 0) {
            float f = __int_as_float(sv);
            if (!ok) {
                f = s0;
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
