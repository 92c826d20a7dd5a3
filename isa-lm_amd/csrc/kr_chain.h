// Ordered fp32 sums of non-negative terms, computed exactly but not one add
// at a time.
//
// The reference adds such terms in index order (rmsnorm's sum of squares,
// kernels/scalar/k_scalar.c:61; softmax's sum of exponentials,
// k_scalar.c:71-74): s = (((s0 + t0) + t1) + ...) with one rounding per add.
// On one lane that is a chain of n dependent adds.
//
// The shortcut rests on one property of round-to-nearest-even. In a binade
// [2^e, 2^(e+1)) the floats are the multiples m u of one spacing u, and a
// rounding picks the nearest multiple, ties to the even m. Moving a real sum
// by an even number of spacings moves its rounding by the same amount, ties
// included. So if a chain a_{j+1} = fl(a_j + t_j) over some terms stays
// inside one binade, then started from a + 2 k u it ends exactly 2 k u higher
// (and, the terms being >= 0, it is monotone, so its two ends tell whether it
// stayed inside). In bits: a run maps a start s to s + d[s & 1], where d[0]
// and d[1] come from running it from one even start and the odd start above.
//
// The terms are split into chunks (128 terms, at most 128 chunks). For
// each chunk a pair of lanes runs the chain from an even and an odd start in
// the binade where the prefix before the chunk lies (estimated by fp32
// partial sums: only its binade matters), checking every SC_BLK terms
// whether the pair left that binade. A block where it did is marked to be
// added one term at a time later, and the pair starts again after it in the
// new binade. Maps of the form s -> s + d[s & 1] compose into maps of the same
// form, so the walk over the chunks is a segmented prefix scan of the chunks'
// first runs across lanes; it cuts at the chunks with marked blocks, whose
// rest (marked blocks term by term, later runs by their maps) runs on the
// true value between segments. Then every run checks, from its true start,
// that start, run start and moved end share one binade, which holds exactly
// when the true chain stayed in it; from the first run that fails, the walk
// goes on chunk by chunk and runs any failing run one add at a time. So the
// result is the sequential loop's bits whatever the terms. A negative or
// non-finite term sends the whole sum through the sequential loop.
//
// With REC the walk also records each chunk's true start value (the partial
// sum before its first term): from those, any prefix sum is one chunk's
// chain away, which is how a sequential "first partial sum above a bound"
// search runs in parallel.
#pragma once
#include "kr_numerics.h"

namespace {

constexpr int SC_LOG_LMIN = 7;                // chunks of 128 terms, doubled while more than SC_MAXC
constexpr int SC_MAXC = 128;
constexpr int SC_PAD = 4;                     // floats after each chunk's terms (spreads LDS banks)
constexpr int SC_BLK = 16;                    // terms between binade checks
constexpr int SC_MAXNB = 8;                   // blocks per chunk, at most
constexpr int SC_NSEG = SC_MAXNB / 2;         // runs of unbroken blocks in a chunk, at most
constexpr int SC_CPW = 32;                    // chunks per wave: one lane pair each
constexpr int SC_REC = 1 + 3 * SC_NSEG;       // ints of walk record per chunk
constexpr int SC_MAX_N = SC_MAXC * SC_MAXNB * SC_BLK;

// log2 of the chunk length for n terms
__host__ __device__ constexpr int sc_log_len(int n) {
    int sh = SC_LOG_LMIN;
    while (((n + (1 << sh) - 1) >> sh) > SC_MAXC) sh++;
    return sh;
}
__host__ __device__ constexpr int sc_chunks(int n) { return (n + (1 << sc_log_len(n)) - 1) >> sc_log_len(n); }
// the LDS float index of term i, sh = sc_log_len(n) (every chunk padded)
__host__ __device__ constexpr int sc_at(int i, int sh) { return i + ((i >> sh) << 2); }
// floats of term space the caller provides
__host__ __device__ constexpr int sc_terms_cap(int n) { return sc_chunks(n) * ((1 << sc_log_len(n)) + SC_PAD); }
// bytes of LDS scratch kr_spec_sum<NT> needs beside the terms
__host__ __device__ constexpr int sc_lds_bytes(int n, int nt) {
    return (nt / 64) * 8 + sc_chunks(n) * SC_REC * 4 + 16;
}

__device__ __forceinline__ void kr_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// s + t[i0] + ... + t[i1 - 1], one add at a time, i0 and i1 - 1 in one chunk
__device__ __forceinline__ float sc_seq(const float *t, int sh, int i0, int i1, float s) {
    const float *p = t + sc_at(i0, sh);
#pragma unroll 8
    for (int i = 0; i < i1 - i0; i++) s = kr_fadd(s, p[i]);
    return s;
}
__device__ __forceinline__ float sc_seq_all(const float *t, int n, int sh, float s) {
    for (int i0 = 0; i0 < n; i0 += 1 << sh) s = sc_seq(t, sh, i0, min(i0 + (1 << sh), n), s);
    return s;
}
__device__ __forceinline__ unsigned sc_uni(unsigned v) { return (unsigned)__builtin_amdgcn_readfirstlane((int)v); }
__device__ __forceinline__ unsigned sc_lane(unsigned v, int l) { return (unsigned)__builtin_amdgcn_readlane((int)v, l); }

template <int CTRL> __device__ __forceinline__ unsigned sc_quad(unsigned v) {
    return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
constexpr int SC_QP_SWAP = 0xB1;   // quad_perm [1, 0, 3, 2]: the other lane of the pair
constexpr int SC_QP_EVEN = 0xA0;   // quad_perm [0, 0, 2, 2]: the pair's even lane
// DPP moves of a wave scan: row_shr:1, 2, 4, 8 (lane l - n of the row of 16),
// row_bcast:15 (lane 15 of the row before, into rows 1 and 3), row_bcast:31
// (lane 31, into rows 2 and 3); a lane uses the moved value only where the
// source lane exists
template <int CTRL> __device__ __forceinline__ unsigned sc_mv(unsigned v) {
    return (unsigned)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}
constexpr int SC_SHR1 = 0x111, SC_SHR2 = 0x112, SC_SHR4 = 0x114, SC_SHR8 = 0x118, SC_BC15 = 0x142, SC_BC31 = 0x143;
// the value of lane - 1 (0 for lane 0)
__device__ __forceinline__ unsigned sc_prev(unsigned v, int lane) {
    const unsigned a = sc_mv<SC_SHR1>(v), b15 = sc_mv<SC_BC15>(v), b31 = sc_mv<SC_BC31>(v);
    return (lane & 15) ? a : (lane == 16 || lane == 48) ? b15 : lane == 32 ? b31 : 0u;
}
// inclusive prefix sum over the wave's lanes (fp32; an estimate)
__device__ __forceinline__ float sc_scan_add(float v, int lane) {
    const int rl = lane & 15;
    float u;
    u = __uint_as_float(sc_mv<SC_SHR1>(__float_as_uint(v)));
    v = rl >= 1 ? v + u : v;
    u = __uint_as_float(sc_mv<SC_SHR2>(__float_as_uint(v)));
    v = rl >= 2 ? v + u : v;
    u = __uint_as_float(sc_mv<SC_SHR4>(__float_as_uint(v)));
    v = rl >= 4 ? v + u : v;
    u = __uint_as_float(sc_mv<SC_SHR8>(__float_as_uint(v)));
    v = rl >= 8 ? v + u : v;
    u = __uint_as_float(sc_mv<SC_BC15>(__float_as_uint(v)));
    v = (lane & 31) >= 16 ? v + u : v;
    u = __uint_as_float(sc_mv<SC_BC31>(__float_as_uint(v)));
    v = lane >= 32 ? v + u : v;
    return v;
}
// one step of the segmented scan of run maps s -> s + d[s & 1]: the lane
// prepends the window of the source lane unless its own window holds a
// segment start (hf)
template <int CTRL>
__device__ __forceinline__ void sc_seg_step(unsigned &d0, unsigned &d1, unsigned &hf, bool valid) {
    const unsigned p0 = sc_mv<CTRL>(d0), p1 = sc_mv<CTRL>(d1), ph = sc_mv<CTRL>(hf);
    if (valid && !hf) {
        const unsigned n0 = p0 + ((p0 & 1u) ? d1 : d0), n1 = p1 + ((p1 & 1u) ? d0 : d1);
        d0 = n0;
        d1 = n1;
        hf = ph;
    }
}
// s + 16 terms from i0 (a block), one add at a time, one batch of LDS reads
__device__ __forceinline__ float sc_blk16(const float *t, int sh, int i0, float s) {
    const float4 *q = (const float4 *)(t + sc_at(i0, sh));
    const float4 v0 = q[0], v1 = q[1], v2 = q[2], v3 = q[3];
    const float4 v[4] = {v0, v1, v2, v3};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        s = kr_fadd(s, v[k].x);
        s = kr_fadd(s, v[k].y);
        s = kr_fadd(s, v[k].z);
        s = kr_fadd(s, v[k].w);
    }
    return s;
}

// whether the run with even start b and ends e0, e1 maps the true start sv
// to sv + (its end's offset) inside one binade; end: that value
__device__ __forceinline__ bool sc_shift(unsigned sv, unsigned b, unsigned e0, unsigned e1, unsigned &end) {
    const unsigned k = sv - b;
    const unsigned par = k & 1u;
    const unsigned e = par ? e1 : e0;
    end = e + (k - par);
    return ((sv ^ b) >> 23) == 0 && ((e ^ b) >> 23) == 0 && ((end ^ b) >> 23) == 0 && (b >> 23) < 0xFFu;
}

// chunk c from block blk (its run number seg) to its end, from the true
// value sv: marked blocks one add at a time, runs by their maps (one add at a
// time when the check fails)
__device__ __forceinline__ unsigned sc_rest(const float *t, int sh, int c, int m, unsigned sv, int blk, int seg,
                                            const int *rb, const int *re0, const int *re1) {
    const int L = 1 << sh, NB = L / SC_BLK;
    while (blk < NB) {
        const int i0 = c * L + blk * SC_BLK;
        if ((m >> blk) & 1) {
            sv = sc_uni(__float_as_uint(sc_blk16(t, sh, i0, __uint_as_float(sv))));
            blk++;
        } else {
            const int e = blk + __builtin_ctz(((unsigned)m >> blk) | (1u << (NB - blk)));
            const int ri = c * SC_NSEG + seg;
            unsigned end;
            if (sc_shift(sv, sc_uni(rb[ri]), sc_uni(re0[ri]), sc_uni(re1[ri]), end))
                sv = end;
            else
                sv = sc_uni(__float_as_uint(sc_seq(t, sh, i0, c * L + e * SC_BLK, __uint_as_float(sv))));
            seg++;
            blk = e;
        }
    }
    return sv;
}

// The ordered sum s0 + t[0] + ... + t[n-1] (n <= SC_MAX_N) by all NT threads
// of the workgroup; every thread gets the result. Term i sits at
// t[sc_at(i, sc_log_len(n))] in LDS (16-byte aligned, sc_terms_cap(n)
// floats: the last chunk's tail is zero-filled here, and s + 0 == s for
// s >= +0). lds: sc_lds_bytes(n, NT) bytes, 4-byte aligned. s0 is expected to
// be >= +0. Contains barriers: all threads must call it, after a barrier that
// follows the terms' stores. REC: cst[c] (c < sc_chunks(n)) receives the bits
// of the partial sum before chunk c, and cst[sc_chunks(n)] is 1 when a
// negative or non-finite term sent the sum through the sequential loop (the
// starts are then not written), else 0. WAVE: the calling wave alone
// (NT = 64) computes the sum, with wave syncs in place of barriers, for n of
// at most SC_CPW chunks (4096 terms); the workgroup's other waves take no part.
// LEAN: fewer reads in flight (4 float4 per estimate batch instead of 16, one
// block of the chains read ahead instead of three): fewer registers, so more
// workgroups share a CU where many sums run side by side
template <int NT, bool REC = false, bool WAVE = false, bool LEAN = false>
__device__ __forceinline__ float kr_spec_sum(float *t, int n, unsigned char *lds, float s0 = 0.0f,
                                             unsigned *cst = nullptr) {
    constexpr int NW = NT / 64;
    static_assert(WAVE ? NT == 64 : NW * SC_CPW >= SC_MAXC, "every chunk needs a lane pair");
    const int tid = WAVE ? (int)(threadIdx.x & 63) : (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sh = sc_log_len(n), L = 1 << sh, NB = L / SC_BLK;
    const int C = (n + L - 1) >> sh, NA = (C + SC_CPW - 1) / SC_CPW;   // waves with chunks
    float *wtot = (float *)lds;                   // [NW] a wave's chunk total
    int *wbad = (int *)(wtot + NW);               // [NW] a wave saw a negative or non-finite term
    int *rm = wbad + NW;                          // [C] marked blocks
    int *rb = rm + C;                             // [C][SC_NSEG] even start of each run
    int *re0 = rb + C * SC_NSEG, *re1 = re0 + C * SC_NSEG;   // its ends from the even and odd starts
    float *res = (float *)(re1 + C * SC_NSEG);

    const int p = lane & 1, c = wave * SC_CPW + (lane >> 1);
    if ((n & (L - 1)) && wave == (C - 1) / SC_CPW) {   // the wave that owns the last chunk
        for (int i = n + lane; i < C * L; i += 64) t[sc_at(i, sh)] = 0.0f;
        kr_wave_sync();
    }
    // the chunk's sum (lane p: its half), the prefix sums over the wave's
    // chunks; a set sign bit (a negative term, or -0) or a sum that is not
    // finite (a term that is not) sends everything to the sequential loop
    const float *tc = t + c * (L + SC_PAD);
    float acc = 0.0f;
    unsigned sg = 0;
    if (c < C) {
        // a lane's half chunk, 16 float4 reads at a time, all issued before
        // their adds
        const float4 *h = (const float4 *)(tc + (L / 2) * p);
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        constexpr int EB = LEAN ? 4 : 16;
        for (int k0 = 0; k0 < L / 8; k0 += EB) {   // L / 8 is a multiple of 16 (L >= 128)
            float4 v[EB];
#pragma unroll
            for (int k = 0; k < EB; k++) v[k] = h[k0 + k];
#pragma unroll
            for (int k = 0; k < EB; k++) {
                sg |= __float_as_uint(v[k].x) | __float_as_uint(v[k].y) | __float_as_uint(v[k].z) |
                      __float_as_uint(v[k].w);
                a0 += v[k].x;
                a1 += v[k].y;
                a2 += v[k].z;
                a3 += v[k].w;
            }
        }
        acc = (a0 + a1) + (a2 + a3);
    }
    acc += __uint_as_float(sc_quad<SC_QP_SWAP>(__float_as_uint(acc)));
    // prefix over chunks: each chunk counted at its even lane; the pair takes
    // the even lane's exclusive value
    const float inc = sc_scan_add(p ? 0.0f : acc, lane);
    const float pre = __uint_as_float(sc_quad<SC_QP_EVEN>(sc_prev(__float_as_uint(inc), lane)));
    const float wsum = __uint_as_float(sc_lane(__float_as_uint(inc), 63));
    bool bad = __any((sg >> 31) != 0 || !(acc <= 3.402823466e38f));   // FLT_MAX: NaN fails
    float before = s0;
    if (!WAVE && NA > 1) {   // the other waves' chunk totals and flags
        if (lane == 0 && wave < NA) {
            wtot[wave] = wsum;
            wbad[wave] = bad;
        }
        __syncthreads();
        for (int w = 0; w < NA; w++) {
            if (w < wave) before += wtot[w];
            bad = bad || wbad[w];
        }
    }
    // the pair's chains: lane p from the even start + p (chunk 0 from the
    // true start: its chain is exact)
    if (c < C && !bad) {
        unsigned b = 0;
        float s = s0;
        if (c > 0) {
            b = __float_as_uint(before + pre) & ~1u;
            s = __uint_as_float(b | (unsigned)p);
        }
        int mask = 0, nseg = 0;
        bool run = false;
        int *re = p ? re1 : re0;
        // the bits at which the odd chain (the pair's upper one: rounding is
        // monotone in the start) leaves b's binade (the terms are >= 0, so
        // the chain only grows); the even lanes and chunk 0 never test
        auto lim = [&](unsigned bb) { return p && c > 0 ? (bb & 0xFF800000u) + 0x00800000u : 0xFFFFFFFFu; };
        unsigned blim = lim(b);
        // four register buffers in turn: block blk + 3's LDS reads are issued
        // before block blk's adds, so three blocks of adds cover their
        // latency (one block ahead, every block waited for its reads; a copy
        // out of one prefetch buffer let the compiler issue the reads after
        // the adds)
        float4 ba[4], bb[4], bc[4], bd[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            ba[q] = ((const float4 *)tc)[q];
            bb[q] = ((const float4 *)(tc + SC_BLK))[q];
            bc[q] = ((const float4 *)(tc + 2 * SC_BLK))[q];
        }
        auto block = [&](int blk, const float4 (&cur)[4], float4 (&nxt)[4]) {
            const float4 *nb4 = (const float4 *)(tc + min(blk + (LEAN ? 1 : 3), NB - 1) * SC_BLK);
#pragma unroll
            for (int q = 0; q < 4; q++) nxt[q] = nb4[q];
            __builtin_amdgcn_sched_barrier(0);
            const float s_start = s;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                s = kr_fadd(s, cur[q].x);
                s = kr_fadd(s, cur[q].y);
                s = kr_fadd(s, cur[q].z);
                s = kr_fadd(s, cur[q].w);
            }
            const unsigned sb = __float_as_uint(s);
            // no odd chain of the wave left its binade: every pair's run goes on
            if (__builtin_expect(__ballot(sb >= blim) == 0ull, 1)) {
                run = true;
                return;
            }
            unsigned cr = (c > 0) && ((sb ^ b) >> 23) != 0;
            cr |= sc_quad<SC_QP_SWAP>(cr);
            const unsigned nbits = sc_quad<SC_QP_EVEN>(sb) & ~1u;
            if (cr) {   // the pair left the binade in this block: mark it, start again after it
                if (run) {
                    if (p == 0) rb[c * SC_NSEG + nseg] = (int)b;
                    re[c * SC_NSEG + nseg] = (int)__float_as_uint(s_start);
                    nseg++;
                }
                mask |= 1 << blk;
                b = nbits;
                blim = lim(b);
                s = __uint_as_float(nbits | (unsigned)p);
                run = false;
            } else {
                run = true;
            }
        };
        if constexpr (LEAN) {   // two buffers: block blk + 1's reads before block blk's adds
            for (int blk = 0; blk < NB; blk += 2) {
                block(blk, ba, bb);
                block(blk + 1, bb, ba);
            }
        } else {
            for (int blk = 0; blk < NB; blk += 4) {   // NB = L / 16 is a multiple of 4 (L >= 128)
                block(blk, ba, bd);
                block(blk + 1, bb, ba);
                block(blk + 2, bc, bb);
                block(blk + 3, bd, bc);
            }
        }
        if (run) {
            if (p == 0) rb[c * SC_NSEG + nseg] = (int)b;
            re[c * SC_NSEG + nseg] = (int)__float_as_uint(s);
        }
        if (p == 0) rm[c] = mask;
    }
    if (!WAVE && NA > 1) __syncthreads();
    else kr_wave_sync();
    // the walk, in wave 0, 64 chunks (one per lane) at a time
    if (wave == 0) {
        float r;
        if constexpr (REC) {
            if (lane == 0) {
                cst[0] = __float_as_uint(s0);
                cst[C] = bad ? 1u : 0u;
            }
        }
        if (bad) {
            r = sc_seq_all(t, n, sh, s0);
        } else {
            unsigned sv = sc_uni(re0[0]);   // chunk 0's end: exact
            int cser = C;                   // chunks from here on go one by one
            for (int g0 = 0; g0 < C; g0 += 64) {
                const int cnt = min(64, C - g0), cc = g0 + lane, cl = min(cc, C - 1);
                const int m = rm[cl];
                const unsigned b = rb[cl * SC_NSEG], e0 = re0[cl * SC_NSEG], e1 = re1[cl * SC_NSEG];
                // the run after a chunk's first marked block (its number: 1
                // if a run comes before the mark, else 0)
                const int r1 = cl * SC_NSEG + ((m & 1) ? 0 : 1);
                const unsigned b1 = rb[r1], e01 = re0[r1], e11 = re1[r1];
                // the chunk's first run (a run before its first marked block)
                const bool pre = lane < cnt && cc > 0 && (m & 1) == 0;
                const bool brk = lane < cnt && m != 0;
                // each lane's chunk's first marked block, read before the
                // serial pass (which then adds it from registers)
                float4 mb[4];
                {
                    const int fbl = m ? __builtin_ctz((unsigned)m) : 0;
                    const float4 *q = (const float4 *)(t + sc_at(cl * L + fbl * SC_BLK, sh));
#pragma unroll
                    for (int k = 0; k < 4; k++) mb[k] = q[k];
                }
                unsigned d0 = pre ? e0 - b : 0u, d1 = pre ? e1 - b - 1u : 0u;
                const unsigned long long bm = __ballot(brk);
                // segments start at lane 0 and after each chunk with marks;
                // inclusive scan of the first-run maps within segments
                const bool head = lane == 0 || (((bm << 1) >> lane) & 1ull);
                unsigned hf = head;
                const int rl = lane & 15;
                sc_seg_step<SC_SHR1>(d0, d1, hf, rl >= 1);
                sc_seg_step<SC_SHR2>(d0, d1, hf, rl >= 2);
                sc_seg_step<SC_SHR4>(d0, d1, hf, rl >= 4);
                sc_seg_step<SC_SHR8>(d0, d1, hf, rl >= 8);
                sc_seg_step<SC_BC15>(d0, d1, hf, (lane & 31) >= 16);
                sc_seg_step<SC_BC31>(d0, d1, hf, lane >= 32);
                unsigned x0 = sc_prev(d0, lane), x1 = sc_prev(d1, lane);
                if (head) x0 = x1 = 0u;
                // the true value entering each segment, serially
                unsigned hv = 0;
                for (int pos = 0; pos < cnt;) {
                    const unsigned long long rest = bm >> pos;
                    const int k = rest ? pos + __builtin_ctzll(rest) : cnt - 1;
                    if (lane >= pos && lane <= k) hv = sv;
                    const unsigned kd0 = sc_lane(d0, k), kd1 = sc_lane(d1, k);
                    sv += (sv & 1u) ? kd1 : kd0;
                    if (rest & 1ull << (k - pos)) {   // chunk g0 + k has marks: the rest of it
                        const int mk = (int)sc_lane((unsigned)m, k);
                        const int fb = __builtin_ctz((unsigned)mk);
                        const int i0 = (g0 + k) * L + fb * SC_BLK;
                        float x = __uint_as_float(sv);   // every lane adds its own block; lane k's is the one
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            x = kr_fadd(x, mb[q].x);
                            x = kr_fadd(x, mb[q].y);
                            x = kr_fadd(x, mb[q].z);
                            x = kr_fadd(x, mb[q].w);
                        }
                        sv = sc_lane(__float_as_uint(x), k);
                        if ((mk & (mk - 1)) == 0) {   // one mark: at most one run after it
                            if (fb + 1 < NB) {
                                unsigned end;
                                if (sc_shift(sv, sc_lane(b1, k), sc_lane(e01, k), sc_lane(e11, k), end))
                                    sv = end;
                                else
                                    sv = sc_uni(__float_as_uint(sc_seq(t, sh, i0 + SC_BLK, (g0 + k + 1) * L,
                                                                       __uint_as_float(sv))));
                            }
                        } else {
                            sv = sc_rest(t, sh, g0 + k, mk, sv, fb + 1, (mk & 1) ? 0 : 1, rb, re0, re1);
                        }
                    }
                    pos = k + 1;
                }
                // every first run's check from its true start
                const unsigned hp = hv & 1u;
                const unsigned st = hv + (hp ? x1 : x0), en = hv + (hp ? d1 : d0);
                bool ok = true;
                if (pre) {
                    const unsigned e = (st & 1u) ? e1 : e0;
                    ok = ((st ^ b) >> 23) == 0 && ((e ^ b) >> 23) == 0 && ((en ^ b) >> 23) == 0 &&
                         (b >> 23) < 0xFFu;
                }
                const unsigned long long fail = __ballot(!ok);
                if constexpr (REC) {   // starts up to the first failed run are true
                    const int lim = fail ? __builtin_ctzll(fail) : cnt - 1;
                    if (lane <= lim && cc > 0) cst[cc] = st;
                }
                if (fail) {
                    const int f = __builtin_ctzll(fail);
                    sv = sc_lane(st, f);
                    cser = g0 + f;
                    break;
                }
            }
            for (int k = cser; k < C; k++) {
                if constexpr (REC) {
                    if (lane == 0) cst[k] = sv;
                }
                sv = sc_rest(t, sh, k, (int)sc_uni(rm[k]), sv, 0, 0, rb, re0, re1);
            }
            r = __uint_as_float(sv);
        }
        if (lane == 0) *res = r;
    }
    if (WAVE) kr_wave_sync();
    else __syncthreads();
    return *res;
}

}  // namespace
