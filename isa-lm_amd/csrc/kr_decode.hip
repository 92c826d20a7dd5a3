// Decode-step kernels for gfx950 (one token at a time, batch 1).
//
// Matvec (k_matvec): HBM-streaming, no MFMA. A workgroup owns R output rows
// (of up to three matrices that share the input, or the w1/w3 row pairs of
// SwiGLU). Its 256 threads walk the rows' 32-element blocks in memory order,
// so each wave reads one contiguous span per step (2 x 16-byte loads per
// lane for Q8, one for Q4), and form the exact int32 block dot with v_dot4
// against the Q8_0 activation staged in LDS. The per-block term
// ((float)s * wd) * xd is computed in parallel into LDS; one lane per row then
// adds the terms in block order, which is the reference's float order
// (kernels/scalar/k_scalar.c:13, :34). Fused epilogues: plain store,
// residual add, QKV bias + RoPE + KV-cache write, SwiGLU + Q8_0 quantize.
#include <type_traits>

#include "kr_internal.h"
#include "kr_numerics.h"
#include "kr_chain.h"

namespace {

struct KMat {
    const uint8_t *q;
    const void *d;
    int rows, cols, type, d16;
};

KMat to_kmat(const krh_mat *m) {
    KMat k = { (const uint8_t *)m->q, m->d, m->rows, m->cols, m->type, m->d16 };
    return k;
}

enum { EPI_STORE = 0, EPI_ADD = 1, EPI_QKV = 2, EPI_SWIGLU = 3 };
// weight type template argument: ML_Q8_0, ML_Q4_0, or QT_MIXED, the type of
// each matrix read from its KMat at run time (q|k|v of a Q4 model with its
// v in Q8: one launch and one prologue; an item lies in one matrix, so the
// branch is uniform across the wave)
constexpr int QT_MIXED = 7;
template <int QT> __device__ __forceinline__ bool qt_is_q8(int type) {
    return QT == QT_MIXED ? type == ML_Q8_0 : QT == ML_Q8_0;
}

struct MvArgs {
    KMat m[3];
    int tile0[4];        // first workgroup of matrix i; tile0[nmat] = grid size
    int nmat;
    int R;               // output rows per tile
    int nbc;             // blocks per chunk (set by launch_mv)
    const int8_t *xq;    // Q8_0 activation; or NULL: quantize xf in the prologue,
    const float *xd;     // after rmsnorm with weight nw when nw is set
    const float *xf;
    const float *nw;
    float eps;
    int K;
    float *y[3];
    const float *bias[3];
    const float *rope_cos, *rope_sin;
    int head_dim, ld_cache;
    const int *pos;
    int kv16;            // EPI_QKV: k and v rows are the F16 cache's (halves)
    float *keep;         // EPI_ADD: receives the product W x as well; EPI_SWIGLU: receives w3 x
    // workgroup 0 stores the prologue's results when set (float inputs):
    // the normalized x (with nw) and its Q8_0 quants and scales, as the
    // reference's separate rmsnorm and quantize_q8 calls leave them in memory
    float *keep_xb;
    int8_t *keep_xq;
    float *keep_xd;
    int touch;           // touches ahead (set by launch_mv: every matrix below 4 GiB)
};

constexpr int MV_THREADS = 256;
constexpr int MV_NPT = 2;   // weight blocks per thread per work item
constexpr int MV_DEPTH = 2;    // work items in flight per wave: a wave that issues more loads than the
                               // memory pipeline holds stalls at issue
#ifndef KR_MV_TOUCH
#define KR_MV_TOUCH 2
#endif
// Items a wave touches ahead (the item MV_TOUCH after the one whose dots run;
// 1: none): a 2-byte read per 128-byte line of an item's quants and per row
// of its scales, so that the lines are in this XCD's L2 (and the Infinity
// Cache) when the item's own loads go out, above all under a prologue, when
// the register-loaded item is the only other memory traffic. 2 or 4; 4
// (three items touched) was slower: a wave's loads return in order, so the
// item loads wait behind touches further out.
constexpr int MV_TOUCH = KR_MV_TOUCH;
// Activations held in registers by the prologue (longer ones are staged
// through LDS from memory): sized so that the kernel fits 128 VGPRs, four
// workgroups per CU
constexpr int MV_XQ_MAX = 8192;   // quantized activations up to this length are staged from registers
constexpr int MV_XF_MAX = 4096;    // float activations up to this length are normalized and quantized from registers
constexpr int MV_XF_PLAIN_MAX = 16384;  // float activations without a norm: quantized from registers up to this length,
constexpr int MV_XF_PASS = 4096;        // in passes of this many

template <typename T> __device__ __forceinline__ T pick3(int i, T a, T b, T c) { return i == 0 ? a : (i == 1 ? b : c); }

// Exact int32 dot of one weight block with the activation block in LDS.
template <int QT>
__device__ __forceinline__ int block_dot(const int4 w0, const int4 w1, const int8_t *xb) {
    const int4 xa = *(const int4 *)xb, xc = *(const int4 *)(xb + 16);
    int s = 0;
    if (QT == ML_Q8_0) {
        s = kr_dot4(w0.x, xa.x, s); s = kr_dot4(w0.y, xa.y, s);
        s = kr_dot4(w0.z, xa.z, s); s = kr_dot4(w0.w, xa.w, s);
        s = kr_dot4(w1.x, xc.x, s); s = kr_dot4(w1.y, xc.y, s);
        s = kr_dot4(w1.z, xc.z, s); s = kr_dot4(w1.w, xc.w, s);
    } else {
        // byte j holds element j (low nibble) and j+16 (high); nibble n is
        // weight n-8, so the dot is sum(n x) - 8 sum(x), all exact in int32
        const unsigned M = 0x0F0F0F0Fu;
        s = kr_dot4((int)((unsigned)w0.x & M), xa.x, s); s = kr_dot4((int)((unsigned)w0.y & M), xa.y, s);
        s = kr_dot4((int)((unsigned)w0.z & M), xa.z, s); s = kr_dot4((int)((unsigned)w0.w & M), xa.w, s);
        s = kr_dot4((int)(((unsigned)w0.x >> 4) & M), xc.x, s); s = kr_dot4((int)(((unsigned)w0.y >> 4) & M), xc.y, s);
        s = kr_dot4((int)(((unsigned)w0.z >> 4) & M), xc.z, s); s = kr_dot4((int)(((unsigned)w0.w >> 4) & M), xc.w, s);
        const int one = 0x01010101;
        int sx = 0;
        sx = kr_dot4(one, xa.x, sx); sx = kr_dot4(one, xa.y, sx); sx = kr_dot4(one, xa.z, sx); sx = kr_dot4(one, xa.w, sx);
        sx = kr_dot4(one, xc.x, sx); sx = kr_dot4(one, xc.y, sx); sx = kr_dot4(one, xc.z, sx); sx = kr_dot4(one, xc.w, sx);
        s -= 8 * sx;
    }
    return s;
}

// Q8_0 of the 4 values v = x[i..i+3] (k_scalar.c:39-57): 8 consecutive
// lanes hold a 32-block (all 8 must call together); the block max is exact in
// any order. q[i..i+3] receive the values, d[(i / 32) * dstep] the scale.
__device__ __forceinline__ void kr_quant4(float4 v, int i, int8_t *q, float *d, size_t dstep) {
    // seeded with 0 as the reference's loop is: NaNs never raise the max
    float m = fmaxf(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))), 0.0f);
    m = fmaxf(m, __shfl_xor(m, 1, 8));
    m = fmaxf(m, __shfl_xor(m, 2, 8));
    m = fmaxf(m, __shfl_xor(m, 4, 8));
    int packed = 0;
    float dd = 0.0f;
    if (!(m < KR_QUANT_TINY)) {
        const float id = kr_fdiv(127.0f, m);
        dd = kr_fdiv(m, 127.0f);
        packed = (kr_q8_elem(v.x, id) & 0xff) | (kr_q8_elem(v.y, id) & 0xff) << 8 |
                 (kr_q8_elem(v.z, id) & 0xff) << 16 | (int)((unsigned)kr_q8_elem(v.w, id) << 24);
    }
    *(int *)(q + i) = packed;
    if ((i & 31) == 0) d[(size_t)(i >> 5) * dstep] = dd;
}

// Q8_0 of the 16 values v = x[i..i+15] held by this lane (k_scalar.c:39-57):
// a 32-block is two lanes' halves, lanes 2j and 2j + 1 (both must call
// together; i % 32 == 16 in the odd one). The block max is exact in any
// order; the two divisions are paid once per 16 values instead of per 4.
// q[i..i+15] receive the values, d[i / 32] the scale.
__device__ __forceinline__ void kr_quant16(const float4 (&v)[4], int i, int8_t *q, float *d) {
    float m = 0.0f;   // seeded with 0 as the reference's loop is: NaNs never raise the max
#pragma unroll
    for (int k = 0; k < 4; k++)
        m = fmaxf(fmaxf(m, fmaxf(fabsf(v[k].x), fabsf(v[k].y))), fmaxf(fabsf(v[k].z), fabsf(v[k].w)));
    m = fmaxf(m, __uint_as_float((unsigned)__builtin_amdgcn_mov_dpp((int)__float_as_uint(m), 0xB1, 0xF, 0xF, false)));
    int4 packed = make_int4(0, 0, 0, 0);
    float dd = 0.0f;
    if (!(m < KR_QUANT_TINY)) {
        const float id = kr_fdiv(127.0f, m);
        dd = kr_fdiv(m, 127.0f);
        auto p4 = [&](float4 x) {
            return (kr_q8_elem(x.x, id) & 0xff) | (kr_q8_elem(x.y, id) & 0xff) << 8 |
                   (kr_q8_elem(x.z, id) & 0xff) << 16 | (int)((unsigned)kr_q8_elem(x.w, id) << 24);
        };
        packed = make_int4(p4(v[0]), p4(v[1]), p4(v[2]), p4(v[3]));
    }
    *(int4 *)(q + i) = packed;
    if ((i & 31) == 0) d[i >> 5] = dd;
}

// the rmsnorm output (x * inv) * w (k_scalar.c:63)
__device__ __forceinline__ float4 kr_norm4(float4 x, float inv, float4 w) {
    return make_float4(kr_fmul(kr_fmul(x.x, inv), w.x), kr_fmul(kr_fmul(x.y, inv), w.y),
                       kr_fmul(kr_fmul(x.z, inv), w.z), kr_fmul(kr_fmul(x.w, inv), w.w));
}

// Q8_0 of K floats into LDS: each thread takes 4 consecutive values, 8
// threads a 32-block. K % 32 == 0, x 16-byte aligned. With w: the rmsnorm
// output (x * inv) * w is quantized, and also stored into xb when it is set.
__device__ __forceinline__ void quantize_to_lds(const float *x, int K, int8_t *xs, float *xds,
                                                const float *w = nullptr, float inv = 1.0f, float *xb = nullptr) {
    constexpr int B = 4;   // float4 loads in flight per thread
    for (int base = 0; base < K; base += 4 * B * MV_THREADS) {
        float4 vs[B], ws[B];
#pragma unroll
        for (int k = 0; k < B; k++) {
            const int i = base + 4 * (k * MV_THREADS + threadIdx.x);
            if (i < K) {
                vs[k] = *(const float4 *)(x + i);
                if (w) ws[k] = *(const float4 *)(w + i);
            }
        }
#pragma unroll
        for (int k = 0; k < B; k++) {
            const int i = base + 4 * (k * MV_THREADS + threadIdx.x);   // K % 32 == 0: 8-lane groups all in or all out
            if (i < K) {
                const float4 o = w ? kr_norm4(vs[k], inv, ws[k]) : vs[k];
                kr_quant4(o, i, xs, xds, 1);
                if (xb) *(float4 *)(xb + i) = o;
            }
        }
    }
}

// rmsnorm + Q8_0 of one row of n floats by the NT threads of a workgroup
// (n <= NT * V4 * 4, n % 32 == 0, rows 16-byte aligned): every thread keeps
// its float4 slices of x and w in registers; the squares x_i * x_i (each one
// rounded product, as in the scalar loop) go to LDS (sq: sc_terms_cap(n)
// floats and then sc_lds_bytes(n, NT) bytes) for the ordered sum
// (k_scalar.c:59-64); then every thread forms (x * inv) * w for its values
// and 8-thread groups quantize their 32-element blocks (k_scalar.c:39-57).
// q[i] and d[(i / 32) * dstep] receive them, xb (nullable) the floats.
constexpr int RN_THREADS = 256, RN_V4 = 16, RN_MAX = RN_THREADS * RN_V4 * 4;

template <int NT, int V4>
__device__ __forceinline__ void rmsnorm_q8_block(int8_t *q, float *d, size_t dstep, float *xb, const float *x,
                                                 const float *w, int n, float eps, bool norm, float *sq) {
    const int tid = threadIdx.x;
    float4 xv[V4], wv[V4];
#pragma unroll
    for (int k = 0; k < V4; k++) {
        const int i = min((k * NT + tid) * 4, n - 4);
        xv[k] = *(const float4 *)(x + i);
        if (norm) wv[k] = *(const float4 *)(w + i);
    }
    float inv = 1.0f;
    if (norm) {
        const int sh = sc_log_len(n);
#pragma unroll
        for (int k = 0; k < V4; k++) {
            const int i = (k * NT + tid) * 4;
            if (i < n)
                *(float4 *)(sq + sc_at(i, sh)) = make_float4(kr_fmul(xv[k].x, xv[k].x), kr_fmul(xv[k].y, xv[k].y),
                                                  kr_fmul(xv[k].z, xv[k].z), kr_fmul(xv[k].w, xv[k].w));
        }
        __syncthreads();
        const float ss = kr_spec_sum<NT>(sq, n, (unsigned char *)(sq + sc_terms_cap(n)));
        inv = kr_fdiv(1.0f, kr_fsqrt(kr_fadd(kr_fdiv(ss, (float)n), eps)));
    }
#pragma unroll
    for (int k = 0; k < V4; k++) {
        const int i = (k * NT + tid) * 4;
        if (i < n) {   // n % 32 == 0: 8-thread groups are all in or all out
            const float4 o = norm ? kr_norm4(xv[k], inv, wv[k]) : xv[k];
            if (xb) *(float4 *)(xb + i) = o;
            kr_quant4(o, i, q, d, dstep);
        }
    }
}

// Loads of one work item (row tile, block chunk) by one wave: slot k of lane
// l is local block l + 64 k of the item, blocks fastest, so each load
// instruction reads contiguous spans (a Q8_0 block as two 16-byte loads, a
// Q4_0 block as one). Every slot loads (slots past the item re-read its first
// block and are not used), so no load waits on a branch.
struct MvSlots {
    int4 w0[MV_NPT], w1[MV_NPT];
    uint32_t wd[MV_NPT];   // raw scale bits: widened at use, after every load is in flight
};

// Where a work item lies: matrix mi, first row, rows, local rows (SwiGLU's w3
// rows follow its w1 rows), first block and block count of the chunk.
struct MvItem {
    int mi, row0, nr, nloc, c0, nbc;
};

template <int EPI>
__device__ __forceinline__ MvItem mv_item(const MvArgs &a, int tile, int chunk, int nb) {
    // constant indices only: a runtime index into the argument block makes
    // the compiler read it with a vector load, whose wait would drain the
    // weight loads in flight
    MvItem it;
    it.mi = 0;
    if (EPI != EPI_SWIGLU)
        it.mi = (a.nmat > 1 && tile >= a.tile0[1]) + (a.nmat > 2 && tile >= a.tile0[2]);
    const int rows = pick3(it.mi, a.m[0].rows, a.m[1].rows, a.m[2].rows);
    it.row0 = (tile - pick3(it.mi, a.tile0[0], a.tile0[1], a.tile0[2])) * a.R;
    it.nr = min(a.R, rows - it.row0);
    it.nloc = EPI == EPI_SWIGLU ? 2 * it.nr : it.nr;
    it.c0 = chunk * a.nbc;
    it.nbc = min(a.nbc, nb - it.c0);
    return it;
}

template <int EPI, int QT, int D16>
__device__ __forceinline__ void mv_load(MvSlots &S, const MvArgs &a, const MvItem &it, int nb, int lane) {
    const KMat W = pick3(it.mi, a.m[0], a.m[1], a.m[2]);
    const KMat W2 = a.m[1];
    const int n = it.nloc * it.nbc;
    int lr = lane / it.nbc, b = lane - lr * it.nbc;
    const int sr = 64 / it.nbc, sb = 64 - sr * it.nbc;
#pragma unroll
    for (int k = 0; k < MV_NPT; k++) {
        const bool in = lane + k * 64 < n;
        const bool second = EPI == EPI_SWIGLU && in && lr >= it.nr;
        const uint8_t *q = second ? W2.q : W.q;
        const void *d = second ? W2.d : W.d;
        const size_t blk = in ? (size_t)(it.row0 + (second ? lr - it.nr : lr)) * nb + it.c0 + b
                              : (size_t)it.row0 * nb + it.c0;
        if (qt_is_q8<QT>(W.type)) {
            const int4 *p = (const int4 *)(q + blk * 32);
            S.w0[k] = p[0];
            S.w1[k] = p[1];
        } else {
            S.w0[k] = *(const int4 *)(q + blk * 16);
            S.w1[k] = make_int4(0, 0, 0, 0);
        }
        S.wd[k] = D16 ? (uint32_t)((const uint16_t *)d)[blk] : ((const uint32_t *)d)[blk];
        b += sb;
        lr += sr;
        if (b >= it.nbc) { b -= it.nbc; lr++; }
    }
}

// One dword per lane from one of the item's lines (a touch: the value is not
// used): lanes l < n / 4 read local block 4 l (a 128-byte line of Q8_0 quants,
// half of one of Q4_0), the next lanes the first and the middle scale of each
// local row. The local blocks map to rows and blocks as in mv_load. Offsets
// are 32-bit: the launcher sets touch only when every matrix's quants and
// scales stay below 4 GiB.
// (a 2-byte read of the block's first quants or of the scale itself)
template <int EPI, int QT, int D16>
__device__ __forceinline__ int mv_touch(const MvArgs &a, const MvItem &it, int nb, int lane) {
    const KMat W = pick3(it.mi, a.m[0], a.m[1], a.m[2]);
    const KMat W2 = a.m[1];
    const int n = max(it.nloc * it.nbc, 1), nql = (n + 3) >> 2;
    const bool scale = lane >= nql;
    const int sl = lane - nql;
    int j = scale ? min(sl >> 1, max(it.nloc, 1) - 1) * it.nbc + (sl & 1) * (it.nbc >> 1) : 4 * lane;
    j = min(j, n - 1);
    const int lr = j / it.nbc, b = j - lr * it.nbc;
    const bool second = EPI == EPI_SWIGLU && lr >= it.nr;
    const unsigned blk = (unsigned)(it.row0 + (second ? lr - it.nr : lr)) * (unsigned)nb + (unsigned)(it.c0 + b);
    const uint8_t *base = scale ? (const uint8_t *)(second ? W2.d : W.d) : (second ? W2.q : W.q);
    const unsigned off = scale ? blk * (D16 ? 2u : 4u) : blk * (qt_is_q8<QT>(W.type) ? 32u : 16u);
    return *(const uint16_t *)(base + off);   // 2 bytes: in bounds for every block and scale
}

// LDS layout of k_matvec (byte offsets, every region 16-byte aligned): the
// Q8_0 activation and its scales, each wave's chunk terms (rows of ts floats:
// a multiple of 4 plus 4, for 16-byte reads with a 4-bank shift between
// rows) and row sums, and for a normalizing launch the squares and the
// ordered sum's scratch.
constexpr int MV_WAVES = MV_THREADS / 64;
struct MvLds {
    int ts, xds, t2, sums, sq, total;
};
__host__ __device__ constexpr int mv_align16(int b) { return (b + 15) & ~15; }
__host__ __device__ inline MvLds mv_lds(int K, int maxloc, int nbc, bool norm) {
    MvLds l = {};
    l.ts = (nbc + 3) / 4 * 4 + 4;
    l.xds = mv_align16(K);
    l.t2 = mv_align16(l.xds + 4 * (K / KR_QK));
    l.sums = mv_align16(l.t2 + 4 * MV_WAVES * maxloc * l.ts);
    l.sq = mv_align16(l.sums + 4 * MV_WAVES * maxloc);
    l.total = norm ? l.sq + 4 * sc_terms_cap(K) + sc_lds_bytes(K, MV_THREADS) : l.sq;
    return l;
}

// Orders one wave's LDS writes before its later reads for the compiler (a
// wave's LDS operations execute in order).

// y rows [row0, row0 + R) of up to three matrices sharing the activation
// (QKV), or the w1 and w3 rows [row0, row0 + R) (SwiGLU). Each wave streams
// its own row tiles (tiles gw, gw + GW, ... of the GW waves of the grid),
// each split into chunks of nbc blocks, and issues the loads of item i + 1
// before it uses item i's; waves never wait for each other, so the weight
// stream never stops for the dots, the ordered sums or the epilogues. Per
// item: the exact int32 block dots and their terms ((float)s * wd) * xd go to
// the wave's LDS rows; one lane per row continues its row's ordered sum over
// the chunk's terms, in block order (kernels/scalar/k_scalar.c:13, :34). On a
// tile's last chunk the sums go through the epilogue. Before the first item's
// dots the workgroup stages the activation into LDS (while the first loads
// are in flight): copied, quantized, or normalized first (rmsnorm's ordered
// sum, k_scalar.c:59-64) and quantized.
// workgroups of a launch resident on one CU: three (up to 168 VGPRs, three
// waves a SIMD). With the prologue's Q8_0 in half-blocks per lane and one
// item touched ahead, the 8B decode ran at 316.0 tok/s with four (128
// VGPRs) and 319.3 with three; with the 4-value quantization and no
// touches, four had been ahead (307.5 against 310.9 with three and
// touches). The q|k|v grid of the 8B shape is 768 workgroups in any case
// (3,072 two-row tiles).
#ifndef KR_MV_WGS
#define KR_MV_WGS 3
#endif
constexpr int mv_wgs_per_cu(int epi) { return epi == EPI_QKV ? 3 : KR_MV_WGS; }

template <int EPI, int QT, int D16>
__global__ void __launch_bounds__(MV_THREADS, mv_wgs_per_cu(EPI)) k_matvec(const MvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int K = a.K, nb = K / KR_QK, tid = threadIdx.x;
    const int ntiles = a.nmat == 1 ? a.tile0[1] : a.nmat == 2 ? a.tile0[2] : a.tile0[3];
    const int lane = tid & 63, wave = tid >> 6;
    const int gw = blockIdx.x * MV_WAVES + wave, GW = gridDim.x * MV_WAVES;   // this wave; waves in the grid
    const int pos = EPI == EPI_QKV ? *a.pos : 0;
    const int maxloc = EPI == EPI_SWIGLU ? 2 * a.R : a.R;
    const MvLds L = mv_lds(K, maxloc, a.nbc, a.nw != nullptr);
    const int ts = L.ts;
    int8_t *xs = (int8_t *)smem;
    float *xds = (float *)(smem + L.xds);
    float *T = (float *)(smem + L.t2) + wave * maxloc * ts;   // this wave's terms [maxloc][ts]
    float *sums = (float *)(smem + L.sums) + wave * maxloc;   // and row sums
    float *sq = (float *)(smem + L.sq);      // rmsnorm prologue only: the squares, then the ordered sum's scratch
    if ((int)blockIdx.x * MV_WAVES >= ntiles) return;
    const int nch = (nb + a.nbc - 1) / a.nbc;

    // items are loaded MV_DEPTH - 1 ahead of the one whose dots run: S[P]
    // holds item P of every MV_DEPTH; (ltile, lchunk) is the next item to load
    int tile = gw, chunk = 0, ltile = gw, lchunk = 0;
    auto next_item = [&](int &t, int &c) {
        if (++c == nch) { c = 0; t += GW; }
    };
    auto load_item = [&](MvSlots &dst, MvItem &it) {
        // past the last item: an item of no rows, whose slots all read one
        // block (not used), so the prefetch beyond the end costs one line
        it = mv_item<EPI>(a, min(ltile, ntiles - 1), ltile < ntiles ? lchunk : 0, nb);
        it.nloc = ltile < ntiles ? it.nloc : 0;
        mv_load<EPI, QT, D16>(dst, a, it, nb, lane);
        next_item(ltile, lchunk);
    };
    MvSlots S[MV_DEPTH];
    MvItem I[MV_DEPTH];
    // touches: item i + MV_TOUCH is touched in item i's step, into slot
    // i % MV_TOUCH, whose value (item i's touch, older than item i's own
    // loads, so already back when item i's dots have run) is folded into sink
    // first; the prologue touches items 1 .. MV_TOUCH - 1
    int tv[MV_TOUCH > 1 ? MV_TOUCH : 1] = {};
    int sink = 0, ttile = gw, tchunk = 0;
    auto touch_item = [&]() -> int {
        MvItem it = mv_item<EPI>(a, min(ttile, ntiles - 1), ttile < ntiles ? tchunk : 0, nb);
        next_item(ttile, tchunk);
        return a.touch ? mv_touch<EPI, QT, D16>(a, it, nb, lane) : 0;
    };
    auto prime_touch = [&]() {
        if (MV_TOUCH > 1) {
            next_item(ttile, tchunk);
#pragma unroll
            for (int t = 1; t < MV_TOUCH; t++) tv[t] = touch_item();
        }
    };
    if (a.xq && K <= MV_XQ_MAX) {
        // a quantized activation (just written by the previous launch, so
        // not yet in this die's L2): it is read and stored to LDS before the
        // weight stream starts, so it never queues behind it
        int4 xv[MV_XQ_MAX / 16 / MV_THREADS];
        float xdv[MV_XQ_MAX / 32 / MV_THREADS];
#pragma unroll
        for (int k = 0; k < MV_XQ_MAX / 16 / MV_THREADS; k++)
            xv[k] = ((const int4 *)a.xq)[min(tid + k * MV_THREADS, K / 16 - 1)];
#pragma unroll
        for (int k = 0; k < MV_XQ_MAX / 32 / MV_THREADS; k++) xdv[k] = a.xd[min(tid + k * MV_THREADS, nb - 1)];
#pragma unroll
        for (int k = 0; k < MV_XQ_MAX / 16 / MV_THREADS; k++)
            if (tid + k * MV_THREADS < K / 16) ((int4 *)xs)[tid + k * MV_THREADS] = xv[k];
#pragma unroll
        for (int k = 0; k < MV_XQ_MAX / 32 / MV_THREADS; k++)
            if (tid + k * MV_THREADS < nb) xds[tid + k * MV_THREADS] = xdv[k];
#pragma unroll
        for (int d = 0; d < MV_DEPTH - 1; d++) load_item(S[d], I[d]);
        prime_touch();
    } else if (!a.xq && !a.nw && K <= MV_XF_PLAIN_MAX) {
        // a float activation without a norm (ao before wo, h before w2), in
        // passes of MV_XF_PASS floats held in registers: the first pass's
        // loads go out first, then the first item's weight loads, and the
        // first quantization waits on the activation alone; later passes
        // (h of more than MV_XF_PASS) follow
        // thread t takes the 16 values base + 16 t .. + 15, half of a
        // 32-block (kr_quant16)
        static_assert(MV_XF_PASS == 16 * MV_THREADS, "a pass is one half-block per thread");
        // Two passes' registers in turn: a pass's loads go out before the
        // pass ahead of it is quantized (h of 14,336 floats: four load round
        // trips in series otherwise).
        float4 xa[4], xb[4];
        auto pass_load = [&](float4 (&xv)[4], int base) {
            const int i = min(base + 16 * tid, K - 16);
#pragma unroll
            for (int k = 0; k < 4; k++) xv[k] = *(const float4 *)(a.xf + i + 4 * k);
        };
        auto pass_quant = [&](const float4 (&xv)[4], int base) {
            const int i = base + 16 * tid;   // K % 32 == 0: both halves of a block are in or out
            if (i < K) kr_quant16(xv, i, xs, xds);
        };
        pass_load(xa, 0);
        if (MV_XF_PASS < K) pass_load(xb, MV_XF_PASS);
#pragma unroll
        for (int d = 0; d < MV_DEPTH - 1; d++) load_item(S[d], I[d]);
        prime_touch();
        pass_quant(xa, 0);
        for (int base = MV_XF_PASS; base < K; base += 2 * MV_XF_PASS) {
            if (base + MV_XF_PASS < K) pass_load(xa, base + MV_XF_PASS);
            pass_quant(xb, base);
            if (base + MV_XF_PASS < K) {
                if (base + 2 * MV_XF_PASS < K) pass_load(xb, base + 2 * MV_XF_PASS);
                pass_quant(xa, base + MV_XF_PASS);
            }
        }
    } else if (!a.xq && K <= MV_XF_MAX) {
        // a float activation (normalized first when nw is set), held in
        // registers: its loads go out before the weight loads; the squares
        // and the quantization read the registers
        // thread t holds the 16 values 16 t .. 16 t + 15 (half of a
        // 32-block, kr_quant16) and their norm weights
        static_assert(MV_XF_MAX == 16 * MV_THREADS, "one half-block per thread");
        constexpr int XV = 4;
        float4 xv[XV], wv[XV];
        const int i0 = 16 * tid;
        const bool live = i0 < K;   // K % 32 == 0: both halves of a block are live or not
        {
            const int i = min(i0, K - 16);
#pragma unroll
            for (int k = 0; k < XV; k++) xv[k] = *(const float4 *)(a.xf + i + 4 * k);
        }
        float inv = 1.0f;
        if (a.nw) {
            // the squares wait on x alone; the weight stream then runs under
            // the ordered sum
            const int sh = sc_log_len(K);
            if (live) {
#pragma unroll
                for (int k = 0; k < XV; k++)   // 16 | chunk length: the 16 terms are contiguous in sq
                    *(float4 *)(sq + sc_at(i0, sh) + 4 * k) =
                        make_float4(kr_fmul(xv[k].x, xv[k].x), kr_fmul(xv[k].y, xv[k].y), kr_fmul(xv[k].z, xv[k].z),
                                    kr_fmul(xv[k].w, xv[k].w));
            }
            // the norm weights go out once x is in (every workgroup reads x
            // at once; the weights, needed only by the quantization, return
            // under the ordered sum), ahead of the weight stream, whose
            // loads return after them
            {
                const int i = min(i0, K - 16);
#pragma unroll
                for (int k = 0; k < XV; k++) wv[k] = *(const float4 *)(a.nw + i + 4 * k);
            }
#pragma unroll
            for (int d = 0; d < MV_DEPTH - 1; d++) load_item(S[d], I[d]);
            prime_touch();
            __syncthreads();
            const float ss = kr_spec_sum<MV_THREADS>(sq, K, (unsigned char *)(sq + sc_terms_cap(K)));
            inv = kr_fdiv(1.0f, kr_fsqrt(kr_fadd(kr_fdiv(ss, (float)K), a.eps)));
        }
        if (live) {
            float4 o[XV];
#pragma unroll
            for (int k = 0; k < XV; k++) o[k] = a.nw ? kr_norm4(xv[k], inv, wv[k]) : xv[k];
            kr_quant16(o, i0, xs, xds);
            if (a.keep_xb && blockIdx.x == 0) {
#pragma unroll
                for (int k = 0; k < XV; k++) *(float4 *)(a.keep_xb + i0 + 4 * k) = o[k];
            }
        }
        if (!a.nw) {
#pragma unroll
            for (int d = 0; d < MV_DEPTH - 1; d++) load_item(S[d], I[d]);
            prime_touch();
        }
    } else {
#pragma unroll
        for (int d = 0; d < MV_DEPTH - 1; d++) load_item(S[d], I[d]);
        prime_touch();
        if (a.xq) {
            for (int i = tid; i < K / 16; i += MV_THREADS) ((int4 *)xs)[i] = ((const int4 *)a.xq)[i];
            for (int i = tid; i < nb; i += MV_THREADS) xds[i] = a.xd[i];
        } else if (a.nw) {
            for (int i = 4 * tid; i < K; i += 4 * MV_THREADS) {
                const float4 v = *(const float4 *)(a.xf + i);
                *(float4 *)(sq + sc_at(i, sc_log_len(K))) = make_float4(kr_fmul(v.x, v.x), kr_fmul(v.y, v.y), kr_fmul(v.z, v.z),
                                                  kr_fmul(v.w, v.w));
            }
            __syncthreads();
            const float ss = kr_spec_sum<MV_THREADS>(sq, K, (unsigned char *)(sq + sc_terms_cap(K)));
            const float inv = kr_fdiv(1.0f, kr_fsqrt(kr_fadd(kr_fdiv(ss, (float)K), a.eps)));
            quantize_to_lds(a.xf, K, xs, xds, a.nw, inv, blockIdx.x == 0 ? a.keep_xb : nullptr);
        } else {
            quantize_to_lds(a.xf, K, xs, xds);
        }
    }
    __syncthreads();
    if (a.keep_xq && blockIdx.x == 0) {   // the prologue's Q8_0 of x, from LDS
        for (int i = tid; i < K / 16; i += MV_THREADS) ((int4 *)a.keep_xq)[i] = ((const int4 *)xs)[i];
        for (int i = tid; i < nb; i += MV_THREADS) a.keep_xd[i] = xds[i];
    }

    float acc = 0.0f;   // row sum of lane < nloc
    // one item (step P4 of an unrolled group of 2 or 4): S[P4 % MV_DEPTH] holds it;
    // the slot before receives the loads MV_DEPTH - 1 ahead
    auto step = [&](auto P4_) -> bool {
        constexpr int P4 = decltype(P4_)::value, P = P4 % MV_DEPTH;
        const MvItem cur = I[P];
        load_item(S[(P + MV_DEPTH - 1) % MV_DEPTH], I[(P + MV_DEPTH - 1) % MV_DEPTH]);
        int ntile = tile, nchunk = chunk;
        next_item(ntile, nchunk);
        // the epilogue's inputs for this tile's rows, read before this
        // step's item loads go out, so the epilogue waits on them alone;
        // every lane reads (a clamped row; a missing bias reads the RoPE
        // table and is not used): no load sits in a branch
        float ep0 = 0.0f, ep1 = 0.0f, ep2 = 0.0f;
        {
            const int row = cur.row0 + min(lane, cur.nr - 1);
            if (EPI == EPI_ADD) ep0 = pick3(cur.mi, a.y[0], a.y[1], a.y[2])[row];
            if (EPI == EPI_QKV) {
                const float *bias = pick3(cur.mi, a.bias[0], a.bias[1], a.bias[2]);
                ep0 = *(bias ? bias + row : a.rope_cos);
                const int hd = a.head_dim, h2 = hd >> 1, j = row % hd;
                ep1 = a.rope_cos[(size_t)pos * h2 + (j >> 1)];
                ep2 = a.rope_sin[(size_t)pos * h2 + (j >> 1)];
            }
        }

        {
            int lr = lane / cur.nbc, b = lane - lr * cur.nbc;
            const int sr = 64 / cur.nbc, sb = 64 - sr * cur.nbc;
            const int n = cur.nloc * cur.nbc;
#pragma unroll
            for (int k = 0; k < MV_NPT; k++) {
                if (lane + k * 64 < n) {
                    const int bb = cur.c0 + b;
                    const int sdot = QT != QT_MIXED ? block_dot<QT>(S[P].w0[k], S[P].w1[k], xs + bb * 32)
                                     : qt_is_q8<QT>(pick3(cur.mi, a.m[0].type, a.m[1].type, a.m[2].type))
                                         ? block_dot<ML_Q8_0>(S[P].w0[k], S[P].w1[k], xs + bb * 32)
                                         : block_dot<ML_Q4_0>(S[P].w0[k], S[P].w1[k], xs + bb * 32);
                    const float sc = D16 ? kr_h2f((uint16_t)S[P].wd[k]) : __uint_as_float(S[P].wd[k]);
                    T[lr * ts + b] = kr_fmul(kr_fmul((float)sdot, sc), xds[bb]);
                }
                b += sb;
                lr += sr;
                if (b >= cur.nbc) { b -= cur.nbc; lr++; }
            }
        }
        if (MV_TOUCH > 1) {
            constexpr int TS = P4 % (MV_TOUCH > 1 ? MV_TOUCH : 1);
            sink ^= tv[TS];
            tv[TS] = touch_item();
        }
        kr_wave_sync();
        if (lane < cur.nloc) {
            if (chunk == 0) acc = 0.0f;
            const float *p = T + lane * ts;
            int j = 0;
            for (; j + 32 <= cur.nbc; j += 32) {
                float4 r[8];
#pragma unroll
                for (int k = 0; k < 8; k++) r[k] = *(const float4 *)(p + j + 4 * k);
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    acc = kr_fadd(acc, r[k].x);
                    acc = kr_fadd(acc, r[k].y);
                    acc = kr_fadd(acc, r[k].z);
                    acc = kr_fadd(acc, r[k].w);
                }
            }
            for (; j + 4 <= cur.nbc; j += 4) {   // under 32 left (a 896-wide row's 28): 16-byte reads
                const float4 r = *(const float4 *)(p + j);
                acc = kr_fadd(acc, r.x);
                acc = kr_fadd(acc, r.y);
                acc = kr_fadd(acc, r.z);
                acc = kr_fadd(acc, r.w);
            }
            for (; j < cur.nbc; j++) acc = kr_fadd(acc, p[j]);
        }
        if (nchunk == 0) {   // the tile's last chunk: epilogue
            if (lane < cur.nloc) sums[lane] = acc;
            kr_wave_sync();
            const int mi = cur.mi, row0 = cur.row0, nr = cur.nr;
            if (EPI == EPI_STORE) {
                if (lane < nr) pick3(mi, a.y[0], a.y[1], a.y[2])[row0 + lane] = sums[lane];
            } else if (EPI == EPI_ADD) {
                if (lane < nr) {
                    pick3(mi, a.y[0], a.y[1], a.y[2])[row0 + lane] = kr_fadd(ep0, sums[lane]);
                    if (a.keep) a.keep[row0 + lane] = sums[lane];
                }
            } else if (EPI == EPI_QKV) {
                // bias (model/transformer.c:276-277), then RoPE on q and k
                // (k_scalar.c:79-94: pairs 2i, 2i+1 of each head, unfused)
                const float *bias = pick3(mi, a.bias[0], a.bias[1], a.bias[2]);
                float v = 0.0f;
                if (lane < nr) {
                    v = sums[lane];
                    if (bias) v = kr_fadd(v, ep0);
                }
                kr_wave_sync();
                if (lane < nr) sums[lane] = v;
                kr_wave_sync();
                if (lane < nr) {
                    const int row = row0 + lane;
                    float o = v;
                    if (mi < 2) {
                        const float c = ep1, sn = ep2;
                        const float pa = sums[lane & ~1], pb = sums[lane | 1];
                        o = (lane & 1) == 0 ? kr_fsub(kr_fmul(pa, c), kr_fmul(pb, sn))
                                            : kr_fadd(kr_fmul(pa, sn), kr_fmul(pb, c));
                    }
                    if (mi == 0) a.y[0][row] = o;
                    else if (a.kv16)   // store_kv's rounding (model/transformer.c:195-197)
                        ((uint16_t *)pick3(mi, a.y[0], a.y[1], a.y[2]))[(size_t)pos * a.ld_cache + row] = kr_f2h(o);
                    else pick3(mi, a.y[0], a.y[1], a.y[2])[(size_t)pos * a.ld_cache + row] = o;
                }
            } else if (EPI == EPI_SWIGLU) {
                // g = g / (1 + expf(-g)) * u (k_scalar.c:96-98)
                if (lane < nr) {
                    const float h1 = sums[lane], h3 = sums[nr + lane];
                    a.y[0][row0 + lane] = kr_fmul(kr_fdiv(h1, kr_fadd(1.0f, kr_expf(-h1))), h3);
                    if (a.keep) a.keep[row0 + lane] = h3;
                }
            }
        }
        tile = ntile;
        chunk = nchunk;
        return tile < ntiles;
    };
    static_assert(MV_DEPTH == 2, "the step loop is unrolled by 2 or 4");
    static_assert(MV_TOUCH == 1 || MV_TOUCH == 2 || MV_TOUCH == 4, "touch slots divide the unrolled 4");
    if (gw >= ntiles) return;   // a wave with no tile (after the workgroup's one barrier)
    if (MV_TOUCH == 4) {
        while (step(std::integral_constant<int, 0>()) && step(std::integral_constant<int, 1>()) &&
               step(std::integral_constant<int, 2>()) && step(std::integral_constant<int, 3>())) {
        }
    } else {
        while (step(std::integral_constant<int, 0>()) && step(std::integral_constant<int, 1>())) {
        }
    }
    if (MV_TOUCH > 1) {
        // keeps the touches (their values are never otherwise used)
#pragma unroll
        for (int t = 0; t < MV_TOUCH; t++) sink ^= tv[t];
        if (sink == 0x5bd1e995 && K < 0) a.y[0][0] = 0.0f;
    }
}

// workgroups resident at once: mv_wgs_per_cu per compute unit of this
// device (768 on an MI355X's 256 CUs)
int mv_resident(int epi = EPI_STORE) { return mv_wgs_per_cu(epi) * (krh_device_cus() > 0 ? krh_device_cus() : 256); }

// Rows per tile (one wave's): the largest power of two (at most cap, even for
// the RoPE pairs) that still gives every resident wave a tile; blocks per
// chunk: as many as MV_NPT slots per lane allow (a multiple of 4, for the
// 16-byte term reads).
constexpr int MV_MAX_LOC = 8;   // local rows per tile: a row's chunk then spans >= MV_NPT * 8 blocks

int mv_rows(int K, int total_rows, int local_per_row, int cap, int epi = EPI_STORE) {
    (void)K;
    int R = cap / local_per_row;
    if (R * local_per_row > 64) R = 64 / local_per_row;
    if (R * local_per_row > MV_MAX_LOC) R = MV_MAX_LOC / local_per_row;
    while (R > 2 && (total_rows + R - 1) / R < mv_resident(epi) * MV_WAVES) R /= 2;
    if (R > 1) R &= ~1;
    return R < 1 ? 1 : R;
}

int mv_chunk(int nb, int nloc) {
    int c = (MV_NPT * 64 / nloc) & ~3;
    if (c < 4) c = 4;
    return c < nb ? c : nb;
}

template <int EPI>
void launch_mv(MvArgs &a, const KMat &W) {
    const int nb = a.K / KR_QK;
    const int nloc = EPI == EPI_SWIGLU ? 2 * a.R : a.R;
    a.nbc = mv_chunk(nb, nloc);
    a.touch = 1;
    for (int i = 0; i < a.nmat; i++)
        if ((size_t)a.m[i].rows * (size_t)a.K >= ((size_t)1 << 32) / 32 * 32) a.touch = 0;
    const size_t lds = mv_lds(a.K, nloc, a.nbc, a.nw != nullptr).total;
    const int ntiles = a.tile0[a.nmat];
    const int wgs = (ntiles + MV_WAVES - 1) / MV_WAVES;
    const int grid = wgs > mv_resident(EPI) ? mv_resident(EPI) : wgs;
    if (a.K % KR_QK || lds > 64 * 1024 || grid <= 0 || nloc > 64 || nloc * a.nbc > MV_NPT * 64 ||
        (!a.xq && !a.xf)) {
        kr_fail(ML_E_SHAPE, "matvec shape", hipSuccess);
        return;
    }
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3(grid), dim3(MV_THREADS), lds, kr_stream(), a);
    };
    bool mixed = false;
    for (int i = 1; i < a.nmat; i++) mixed = mixed || a.m[i].type != a.m[0].type;
    if constexpr (EPI == EPI_QKV) {
        if (mixed) {
            if (W.d16) go(k_matvec<EPI, QT_MIXED, 1>); else go(k_matvec<EPI, QT_MIXED, 0>);
            kr_check_launch("matvec");
            return;
        }
    }
    if (mixed) {
        kr_fail(ML_E_SHAPE, "matvec: matrices of one launch differ in type", hipSuccess);
        return;
    }
    if (W.type == ML_Q8_0) {
        if (W.d16) go(k_matvec<EPI, ML_Q8_0, 1>); else go(k_matvec<EPI, ML_Q8_0, 0>);
    } else {
        if (W.d16) go(k_matvec<EPI, ML_Q4_0, 1>); else go(k_matvec<EPI, ML_Q4_0, 0>);
    }
    kr_check_launch("matvec");
}

// ---- rmsnorm + quantize, quantize ----

// One workgroup per token; each thread keeps its float4 slices of x and w in
// registers (n <= RN_MAX); see rmsnorm_q8_block.
// V4: float4 slices of x and w per thread (n <= RN_THREADS * V4 * 4): 4 for
// rows up to 4096 keep the kernel at a quarter of the registers of 16, so
// four times the tokens are in flight (each token's ordered sum is latency)
template <int V4>
__global__ void __launch_bounds__(RN_THREADS) k_rmsnorm_q8(int8_t *q, float *d, int dld, float *xb, const float *x,
                                                           const float *w, int n, float eps, int norm) {
    const size_t t = blockIdx.x;
    // scales [t][n / 32], or transposed [n / 32][dld] when dld > 0
    extern __shared__ __align__(16) float rn_smem[];
    rmsnorm_q8_block<RN_THREADS, V4>(q + t * n, d + (dld > 0 ? t : t * (n / KR_QK)), dld > 0 ? (size_t)dld : 1,
                                     xb ? xb + t * n : nullptr, x + t * n, w, n, eps, norm != 0, rn_smem);
}

// Q8_0 of ntok rows of n floats, QZ_CHUNK values per workgroup: thread t
// takes 4 consecutive values, 8 threads a 32-block (k_scalar.c:39-57).
constexpr int QZ_CHUNK = 1024;
__global__ void __launch_bounds__(256) k_quantize_q8(int8_t *q, size_t ldq, float *d, size_t ldd, int dld,
                                                    const float *x, size_t ldx, int n) {
    const size_t row = blockIdx.y;
    const int i = blockIdx.x * QZ_CHUNK + 4 * threadIdx.x;
    if (i >= n) return;   // n % 32 == 0: 8-thread groups are all in or all out
    const float4 v = *(const float4 *)(x + row * ldx + i);
    float m = fmaxf(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))), 0.0f);   // seeded with 0
    m = fmaxf(m, __shfl_xor(m, 1, 8));
    m = fmaxf(m, __shfl_xor(m, 2, 8));
    m = fmaxf(m, __shfl_xor(m, 4, 8));
    int packed = 0;
    float dd = 0.0f;
    if (!(m < KR_QUANT_TINY)) {
        const float id = kr_fdiv(127.0f, m);
        dd = kr_fdiv(m, 127.0f);
        packed = (kr_q8_elem(v.x, id) & 0xff) | (kr_q8_elem(v.y, id) & 0xff) << 8 |
                 (kr_q8_elem(v.z, id) & 0xff) << 16 | (int)((unsigned)kr_q8_elem(v.w, id) << 24);
    }
    *(int *)(q + row * ldq + i) = packed;
    if ((i & 31) == 0) {
        if (dld > 0) d[(size_t)(i >> 5) * dld + row] = dd;
        else d[row * ldd + (i >> 5)] = dd;
    }
}

// ---- embedding ----

__global__ void k_embed(float *x, const KMat e, const int *tok, float scale) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= e.cols) return;
    const int nb = e.cols / KR_QK, row = *tok, b = i / KR_QK, j = i % KR_QK;
    const float d = kr_scale(e.d, (size_t)row * nb + b, e.d16);
    int v;
    if (e.type == ML_Q8_0) {
        v = ((const int8_t *)e.q)[(size_t)row * e.cols + i];
    } else {
        const uint8_t p = e.q[((size_t)row * nb + b) * 16 + (j & 15)];
        v = (j < 16 ? (p & 0xF) : (p >> 4)) - 8;
    }
    float o = kr_fmul((float)v, d);
    if (scale != 1.0f) o = kr_fmul(o, scale);
    x[i] = o;
}

// ---- greedy pick ----

// First index of the maximum (model/sampler.c:57-61): NaN entries never win,
// and a NaN at index 0 keeps 0, as the sequential loop does.
// Greedy pick (model/sampler.c:57-61): the first index of the largest value,
// NaNs never chosen, index 0 when v[0] is NaN or every value is NaN. Each
// workgroup reduces a span of float4s (all its loads in flight together) to
// (value, smallest index among equal values); the last workgroup to finish
// (a counter it resets, so graph replays need no memset) reduces the
// partials. The partials live in static device memory: calls that overlap on
// one device race.
constexpr int AM_THREADS = 256, AM_V4 = 4;   // float4s per thread
constexpr int AM_MAX_WG = 1024;
__device__ float g_am_v[AM_MAX_WG];
__device__ int g_am_i[AM_MAX_WG];
__device__ unsigned g_am_count;

__device__ __forceinline__ void am_take(float &bv, int &bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

__device__ __forceinline__ void am_reduce_block(float &bv, int &bi, float *sv, int *si) {
    for (int o = 32; o >= 1; o >>= 1) am_take(bv, bi, __shfl_xor(bv, o), __shfl_xor(bi, o));
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[w] = bv; si[w] = bi; }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int k = 1; k < AM_THREADS / 64; k++) am_take(bv, bi, sv[k], si[k]);
}

__global__ void __launch_bounds__(AM_THREADS) k_argmax(int *tok, const float *v, int n, int *pos, int *log) {
    __shared__ float sv[AM_THREADS / 64];
    __shared__ int si[AM_THREADS / 64];
    __shared__ bool last;
    float bv = -INFINITY;
    int bi = INT_MAX;   // -inf with no index: any real value, -inf included, replaces it
    const int n4 = n / 4;
    const int base = blockIdx.x * AM_THREADS * AM_V4 + threadIdx.x;
    float4 x[AM_V4];
    if (n4 > 0) {
#pragma unroll
        for (int k = 0; k < AM_V4; k++) {
            const int i = base + k * AM_THREADS;
            x[k] = ((const float4 *)v)[min(i, n4 - 1)];
        }
    }
#pragma unroll
    for (int k = 0; k < AM_V4; k++) {
        const int i = base + k * AM_THREADS;
        if (i < n4) {
            am_take(bv, bi, x[k].x, 4 * i);
            am_take(bv, bi, x[k].y, 4 * i + 1);
            am_take(bv, bi, x[k].z, 4 * i + 2);
            am_take(bv, bi, x[k].w, 4 * i + 3);
        }
    }
    if (blockIdx.x == gridDim.x - 1 && threadIdx.x < n - 4 * n4) am_take(bv, bi, v[4 * n4 + threadIdx.x], 4 * n4 + threadIdx.x);
    am_reduce_block(bv, bi, sv, si);
    if (threadIdx.x == 0) {
        g_am_v[blockIdx.x] = bv;
        g_am_i[blockIdx.x] = bi;
        __threadfence();
        last = atomicAdd(&g_am_count, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    bv = -INFINITY;
    bi = INT_MAX;
    for (int k = threadIdx.x; k < (int)gridDim.x; k += AM_THREADS) am_take(bv, bi, g_am_v[k], g_am_i[k]);
    am_reduce_block(bv, bi, sv, si);
    if (threadIdx.x == 0) {
        g_am_count = 0;
        if (bi == INT_MAX || v[0] != v[0]) bi = 0;
        *tok = bi;
        if (pos) {
            const int p = *pos + 1;
            if (log) log[p] = bi;
            *pos = p;
        }
    }
}

__global__ void k_take_token(int *tok, const int *prompt, const int *pos) { *tok = prompt[*pos]; }
__global__ void k_advance(int *pos) { *pos += 1; }

__global__ void k_math_batch(int op, float *y, const float *a, const float *b, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    switch (op) {
    case KRH_MATH_EXPF: y[i] = kr_expf(a[i]); break;
    case KRH_MATH_SQRT: y[i] = kr_fsqrt(a[i]); break;
    case KRH_MATH_DIV: y[i] = kr_fdiv(a[i], b[i]); break;
    case KRH_MATH_RMS_INV: y[i] = kr_fdiv(1.0f, kr_fsqrt(kr_fadd(kr_fdiv(a[i], b[i]), 1e-5f))); break;
    case KRH_MATH_F2H: y[i] = __uint_as_float(kr_f2h(a[i])); break;   // the half's bits in the low 16
    default: y[i] = 0.0f;
    }
}
__global__ void __launch_bounds__(256) k_ordered_sum(float *out, const float *t, int n, float s0) {
    extern __shared__ __align__(16) float os_t[];
    for (int i = threadIdx.x; i < n; i += 256) os_t[sc_at(i, sc_log_len(n))] = t[i];
    __syncthreads();
    const float s = kr_spec_sum<256>(os_t, n, (unsigned char *)(os_t + sc_terms_cap(n)), s0);
    if (threadIdx.x == 0) *out = s;
}
// the same with fewer reads in flight (the long-row prefill softmax's form)
__global__ void __launch_bounds__(256) k_ordered_sum_lean(float *out, const float *t, int n, float s0) {
    extern __shared__ __align__(16) float osl_t[];
    for (int i = threadIdx.x; i < n; i += 256) osl_t[sc_at(i, sc_log_len(n))] = t[i];
    __syncthreads();
    const float s = kr_spec_sum<256, false, false, true>(osl_t, n, (unsigned char *)(osl_t + sc_terms_cap(n)), s0);
    if (threadIdx.x == 0) *out = s;
}
// the same by 1024 threads, the decode softmax's workgroup
__global__ void __launch_bounds__(1024) k_ordered_sum_1024(float *out, const float *t, int n, float s0) {
    extern __shared__ __align__(16) float osk_t[];
    for (int i = threadIdx.x; i < n; i += 1024) osk_t[sc_at(i, sc_log_len(n))] = t[i];
    __syncthreads();
    const float s = kr_spec_sum<1024>(osk_t, n, (unsigned char *)(osk_t + sc_terms_cap(n)), s0);
    if (threadIdx.x == 0) *out = s;
}
// the single-wave mode, run by the second wave of the workgroup (its lanes
// and LDS are not the workgroup's first)
__global__ void __launch_bounds__(128) k_ordered_sum_wave(float *out, const float *t, int n, float s0) {
    extern __shared__ __align__(16) float osw_t[];
    if (threadIdx.x < 64) return;
    const int lane = threadIdx.x & 63, sh = sc_log_len(n);
    for (int i = lane; i < n; i += 64) osw_t[sc_at(i, sh)] = t[i];
    kr_wave_sync();
    const float s = kr_spec_sum<64, false, true>(osw_t, n, (unsigned char *)(osw_t + sc_terms_cap(n)), s0);
    if (lane == 0) *out = s;
}
__global__ void k_h2f_batch(float *y, const uint16_t *h, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = kr_h2f(h[i]);
}
__global__ void k_block_dots(int32_t *out, const KMat W, const int8_t *xq) {
    const int nb = W.cols / KR_QK;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)W.rows * nb) return;
    const int b = (int)(i % nb);
    int4 w0, w1 = make_int4(0, 0, 0, 0);
    int s;
    __align__(16) int8_t xb[32];
    for (int j = 0; j < 32; j++) xb[j] = xq[b * 32 + j];
    if (W.type == ML_Q8_0) {
        w0 = ((const int4 *)(W.q + i * 32))[0];
        w1 = ((const int4 *)(W.q + i * 32))[1];
        s = block_dot<ML_Q8_0>(w0, w1, xb);
    } else {
        w0 = *(const int4 *)(W.q + i * 16);
        s = block_dot<ML_Q4_0>(w0, w1, xb);
    }
    out[i] = s;
}

}  // namespace

// ---- C ABI ----

extern "C" void krh_embed(float *x, const krh_mat *emb, const int *tok, float embed_scale) {
    hipLaunchKernelGGL(k_embed, dim3((emb->cols + 255) / 256), dim3(256), 0, kr_stream(), x, to_kmat(emb), tok,
                       embed_scale);
    kr_check_launch("embed");
}

extern "C" void krh_rmsnorm_q8(int8_t *q, float *d, float *xb, const float *x, const float *w, int n, float eps,
                               int ntok) {
    krh_rmsnorm_q8_t(q, d, 0, xb, x, w, n, eps, ntok);
}

extern "C" void krh_rmsnorm_q8_t(int8_t *q, float *d, int dld, float *xb, const float *x, const float *w, int n,
                                 float eps, int ntok) {
    // LDS: the squares and the ordered sum's scratch, within 64 KB
    const size_t lds = sizeof(float) * (size_t)sc_terms_cap(n) + sc_lds_bytes(n, RN_THREADS);
    if (n % KR_QK || n > RN_MAX || lds > 64 * 1024 || ntok <= 0 || (dld > 0 && dld < ntok)) {
        kr_fail(ML_E_SHAPE, "rmsnorm shape", hipSuccess);
        return;
    }
    if (n <= RN_THREADS * 4 * 4)
        hipLaunchKernelGGL(k_rmsnorm_q8<4>, dim3(ntok), dim3(RN_THREADS), lds, kr_stream(), q, d, dld, xb, x, w, n,
                           eps, 1);
    else
        hipLaunchKernelGGL(k_rmsnorm_q8<RN_V4>, dim3(ntok), dim3(RN_THREADS), lds, kr_stream(), q, d, dld, xb, x, w,
                           n, eps, 1);
    kr_check_launch("rmsnorm_q8");
}

extern "C" void krh_quantize_q8(int8_t *q, float *d, const float *x, int n, int ntok) {
    krh_quantize_q8_t(q, d, 0, x, n, ntok);
}

extern "C" void krh_quantize_q8_t(int8_t *q, float *d, int dld, const float *x, int n, int ntok) {
    if (n % KR_QK || n <= 0 || ntok <= 0 || (dld > 0 && dld < ntok)) {
        kr_fail(ML_E_SHAPE, "quantize shape", hipSuccess);
        return;
    }
    hipLaunchKernelGGL(k_quantize_q8, dim3((n + QZ_CHUNK - 1) / QZ_CHUNK, ntok), dim3(256), 0, kr_stream(), q,
                       (size_t)n, d, (size_t)(n / KR_QK), dld, x, (size_t)n, n);
    kr_check_launch("quantize_q8");
}

extern "C" void krh_quantize_q8_rows(int8_t *q, size_t ldq, float *d, size_t ldd, const float *x, size_t ldx, int n,
                                     int rows) {
    if (n % KR_QK || n <= 0 || rows < 0 || rows > KRH_ROWS_MAX || ldq % 4 || ldx % 4 || ((uintptr_t)x & 15) ||
        ((uintptr_t)q & 3)) {
        kr_fail(ML_E_SHAPE, "quantize_q8 rows: shape or alignment", hipSuccess);
        return;
    }
    if (rows == 0) return;
    hipLaunchKernelGGL(k_quantize_q8, dim3((n + QZ_CHUNK - 1) / QZ_CHUNK, rows), dim3(256), 0, kr_stream(), q, ldq, d,
                       ldd, 0, x, ldx, n);
    kr_check_launch("quantize_q8");
}

// the prologue results a launch also stores (MvArgs::keep_*): for a float
// input of any length (the register prologue and the one staged through LDS
// both store them), the normalized x only with a norm
struct MvKeep {
    float *xb;
    int8_t *xq;
    float *xd;
};

static bool keep_ok(const MvKeep &k, const float *xf, const float *nw, int K) {
    if (!k.xb && !k.xq) return true;
    const bool ok = xf && (k.xq != nullptr) == (k.xd != nullptr) && (!k.xb || nw) && !((uintptr_t)k.xq & 15) &&
                    !((uintptr_t)k.xb & 15);
    if (!ok) kr_fail(ML_E_SHAPE, "matvec keep: a float input, 16-byte aligned outputs", hipSuccess);
    return ok;
}

static void set_keep(MvArgs &a, const MvKeep &k) {
    a.keep_xb = k.xb;
    a.keep_xq = k.xq;
    a.keep_xd = k.xd;
}

static void mv_plain(float *y, const krh_mat *W, const int8_t *xq, const float *xd, const float *xf,
                     const float *nw, float eps, int accumulate, float *keep = nullptr, MvKeep kp = {}) {
    if (!keep_ok(kp, xf, nw, W->cols)) return;
    MvArgs a = {};
    a.keep = keep;
    set_keep(a, kp);
    a.m[0] = to_kmat(W);
    a.nmat = 1;
    a.R = mv_rows(W->cols, W->rows, 1, 64);
    // one-row tiles when two-row ones would give at most half of the
    // resident waves a tile (the 0.5B and 1B shapes' wo and w2: twice the
    // waves, a shorter chain of items each): 0.5B decode 888 -> 904 tok/s,
    // 1B 858 -> 866; the 8B's 4096-row matrices keep two rows (one-row
    // tiles measured slower there)
    if (a.R == 2 && (W->rows + 1) / 2 * 2 <= mv_resident() * MV_WAVES) a.R = 1;
    a.tile0[0] = 0;
    a.tile0[1] = (W->rows + a.R - 1) / a.R;
    a.xq = xq;
    a.xd = xd;
    a.xf = xf;
    a.nw = nw;
    a.eps = eps;
    a.K = W->cols;
    a.y[0] = y;
    if (accumulate) launch_mv<EPI_ADD>(a, a.m[0]);
    else launch_mv<EPI_STORE>(a, a.m[0]);
}

extern "C" void krh_matvec(float *y, const krh_mat *W, const int8_t *xq, const float *xd, int accumulate) {
    mv_plain(y, W, xq, xd, nullptr, nullptr, 0.0f, accumulate);
}

extern "C" void krh_matvec_residual(float *r, float *y, const krh_mat *W, const int8_t *xq, const float *xd) {
    mv_plain(r, W, xq, xd, nullptr, nullptr, 0.0f, 1, y);
}

extern "C" void krh_matvec_f_residual_keep(float *r, float *y, const krh_mat *W, const float *x, int8_t *xq,
                                           float *xd) {
    mv_plain(r, W, nullptr, nullptr, x, nullptr, 0.0f, 1, y, MvKeep{ nullptr, xq, xd });
}

extern "C" void krh_matvec_multi(float *const *y, const krh_mat *const *W, int nmat, const int8_t *xq,
                                 const float *xd) {
    if (nmat < 1 || nmat > 3) {
        kr_fail(ML_E_SHAPE, "matvec_multi: 1 to 3 matrices", hipSuccess);
        return;
    }
    for (int i = 1; i < nmat; i++)
        if (W[i]->cols != W[0]->cols || W[i]->type != W[0]->type || W[i]->d16 != W[0]->d16) {
            kr_fail(ML_E_SHAPE, "matvec_multi: one input length, type and scale kind", hipSuccess);
            return;
        }
    MvArgs a = {};
    int rows = 0;
    for (int i = 0; i < nmat; i++) rows += W[i]->rows;
    a.nmat = nmat;
    a.R = mv_rows(W[0]->cols, rows, 1, 64);
    a.tile0[0] = 0;
    for (int i = 0; i < nmat; i++) {
        a.m[i] = to_kmat(W[i]);
        a.y[i] = y[i];
        a.tile0[i + 1] = a.tile0[i] + (W[i]->rows + a.R - 1) / a.R;
    }
    a.xq = xq;
    a.xd = xd;
    a.K = W[0]->cols;
    launch_mv<EPI_STORE>(a, a.m[0]);
}

extern "C" void krh_matvec_f(float *y, const krh_mat *W, const float *x, int accumulate) {
    mv_plain(y, W, nullptr, nullptr, x, nullptr, 0.0f, accumulate);
}

extern "C" void krh_rmsnorm_matvec(float *y, const krh_mat *W, const float *x, const float *nw, float eps,
                                   int accumulate) {
    mv_plain(y, W, nullptr, nullptr, x, nw, eps, accumulate);
}

// k and v go to row *pos of the F32 cache (kv16: of the F16 cache, rounded
// to halves), or with stage set to the staging rows kc, vc of a Q8 cache
// (model/transformer.c:262-263)
static void qkv(float *q, float *kc, float *vc, const krh_mat *wq, const krh_mat *wk, const krh_mat *wv,
                const float *bq, const float *bk, const float *bv, const int8_t *xq, const float *xd, const float *xf,
                const float *nw, float eps, const float *rope_cos, const float *rope_sin, int head_dim,
                const int *pos, bool stage = false, bool kv16 = false, MvKeep kp = {}) {
    if (wq->cols != wk->cols || wq->cols != wv->cols || wk->rows != wv->rows || head_dim % 2 || wq->rows % 2 ||
        wk->rows % 2 || wq->type != wk->type || wq->d16 != wk->d16 || wv->d16 != wq->d16) {
        kr_fail(ML_E_SHAPE, "qkv shapes", hipSuccess);
        return;
    }
    if (!keep_ok(kp, xf, nw, wq->cols)) return;
    MvArgs a = {};
    a.m[0] = to_kmat(wq);
    a.m[1] = to_kmat(wk);
    a.m[2] = to_kmat(wv);
    a.nmat = 3;
    a.R = mv_rows(wq->cols, wq->rows + 2 * wk->rows, 1, 64, EPI_QKV);
    a.tile0[0] = 0;
    a.tile0[1] = (wq->rows + a.R - 1) / a.R;
    a.tile0[2] = a.tile0[1] + (wk->rows + a.R - 1) / a.R;
    a.tile0[3] = a.tile0[2] + (wv->rows + a.R - 1) / a.R;
    a.xq = xq;
    a.xd = xd;
    a.xf = xf;
    a.nw = nw;
    a.eps = eps;
    a.K = wq->cols;
    a.y[0] = q;
    a.y[1] = kc;
    a.y[2] = vc;
    a.bias[0] = bq;
    a.bias[1] = bk;
    a.bias[2] = bv;
    a.rope_cos = rope_cos;
    a.rope_sin = rope_sin;
    a.head_dim = head_dim;
    a.ld_cache = stage ? 0 : wk->rows;
    a.pos = pos;
    a.kv16 = kv16;
    set_keep(a, kp);
    // wv may be Q8 in a Q4 model: the launch then reads each matrix's type
    launch_mv<EPI_QKV>(a, a.m[0]);
}

extern "C" void krh_matvec_qkv(float *q, float *kc, float *vc, const krh_mat *wq, const krh_mat *wk,
                               const krh_mat *wv, const float *bq, const float *bk, const float *bv, const int8_t *xq,
                               const float *xd, const float *rope_cos, const float *rope_sin, int head_dim,
                               const int *pos) {
    qkv(q, kc, vc, wq, wk, wv, bq, bk, bv, xq, xd, nullptr, nullptr, 0.0f, rope_cos, rope_sin, head_dim, pos);
}

extern "C" void krh_rmsnorm_matvec_qkv(float *q, float *kc, float *vc, const krh_mat *wq, const krh_mat *wk,
                                       const krh_mat *wv, const float *bq, const float *bk, const float *bv,
                                       const float *x, const float *nw, float eps, const float *rope_cos,
                                       const float *rope_sin, int head_dim, const int *pos) {
    qkv(q, kc, vc, wq, wk, wv, bq, bk, bv, nullptr, nullptr, x, nw, eps, rope_cos, rope_sin, head_dim, pos);
}

extern "C" void krh_rmsnorm_matvec_qkv_f16(float *q, uint16_t *kc, uint16_t *vc, const krh_mat *wq,
                                           const krh_mat *wk, const krh_mat *wv, const float *bq, const float *bk,
                                           const float *bv, const float *x, const float *nw, float eps,
                                           const float *rope_cos, const float *rope_sin, int head_dim,
                                           const int *pos) {
    qkv(q, (float *)kc, (float *)vc, wq, wk, wv, bq, bk, bv, nullptr, nullptr, x, nw, eps, rope_cos, rope_sin,
        head_dim, pos, false, true);
}

extern "C" void krh_rmsnorm_matvec_qkv_keep(float *q, float *k, float *v, const krh_mat *wq, const krh_mat *wk,
                                            const krh_mat *wv, const float *bq, const float *bk, const float *bv,
                                            const float *x, const float *nw, float eps, const float *rope_cos,
                                            const float *rope_sin, int head_dim, const int *pos, float *xb,
                                            int8_t *xq, float *xd) {
    qkv(q, k, v, wq, wk, wv, bq, bk, bv, nullptr, nullptr, x, nw, eps, rope_cos, rope_sin, head_dim, pos, true, false,
        MvKeep{ xb, xq, xd });
}

extern "C" void krh_rmsnorm_matvec_qkv_stage(float *q, float *k, float *v, const krh_mat *wq, const krh_mat *wk,
                                             const krh_mat *wv, const float *bq, const float *bk, const float *bv,
                                             const float *x, const float *nw, float eps, const float *rope_cos,
                                             const float *rope_sin, int head_dim, const int *pos) {
    qkv(q, k, v, wq, wk, wv, bq, bk, bv, nullptr, nullptr, x, nw, eps, rope_cos, rope_sin, head_dim, pos, true);
}

static void swiglu(float *h, const krh_mat *w1, const krh_mat *w3, const int8_t *xq, const float *xd, const float *xf,
                   const float *nw, float eps, float *keep = nullptr, MvKeep kp = {}) {
    if (!keep_ok(kp, xf, nw, w1->cols)) return;
    if (w1->rows != w3->rows || w1->cols != w3->cols || w1->type != w3->type || w1->d16 != w3->d16) {
        kr_fail(ML_E_SHAPE, "swiglu shapes", hipSuccess);
        return;
    }
    MvArgs a = {};
    a.m[0] = to_kmat(w1);
    a.m[1] = to_kmat(w3);
    a.nmat = 1;
    a.R = mv_rows(w1->cols, w1->rows, 2, 4);   // 2 rows of w1 and w3 a tile: measured fastest
    a.tile0[0] = 0;
    a.tile0[1] = (w1->rows + a.R - 1) / a.R;
    a.xq = xq;
    a.xd = xd;
    a.xf = xf;
    a.nw = nw;
    a.eps = eps;
    a.K = w1->cols;
    a.y[0] = h;
    a.keep = keep;
    set_keep(a, kp);
    launch_mv<EPI_SWIGLU>(a, a.m[0]);
}

extern "C" void krh_rmsnorm_matvec_swiglu_keep(float *h, float *u, const krh_mat *w1, const krh_mat *w3,
                                               const float *x, const float *nw, float eps, float *xb, int8_t *xq,
                                               float *xd) {
    swiglu(h, w1, w3, nullptr, nullptr, x, nw, eps, u, MvKeep{ xb, xq, xd });
}

extern "C" void krh_matvec_swiglu_keep(float *h, float *u, const krh_mat *w1, const krh_mat *w3, const int8_t *xq,
                                       const float *xd) {
    swiglu(h, w1, w3, xq, xd, nullptr, nullptr, 0.0f, u);
}

extern "C" void krh_matvec_swiglu(float *h, const krh_mat *w1, const krh_mat *w3, const int8_t *xq, const float *xd) {
    swiglu(h, w1, w3, xq, xd, nullptr, nullptr, 0.0f);
}

extern "C" void krh_rmsnorm_matvec_swiglu(float *h, const krh_mat *w1, const krh_mat *w3, const float *x,
                                          const float *nw, float eps) {
    swiglu(h, w1, w3, nullptr, nullptr, x, nw, eps);
}

extern "C" void krh_argmax(int *tok, const float *logits, int n, int *pos, int *log) {
    const int per_wg = AM_THREADS * AM_V4 * 4;
    const int grid = (n + per_wg - 1) / per_wg;
    if (n < 1 || grid > AM_MAX_WG) {
        kr_fail(ML_E_SHAPE, "argmax size", hipSuccess);
        return;
    }
    hipLaunchKernelGGL(k_argmax, dim3(grid), dim3(AM_THREADS), 0, kr_stream(), tok, logits, n, pos, log);
    kr_check_launch("argmax");
}

extern "C" void krh_take_token(int *tok, const int *prompt, const int *pos) {
    hipLaunchKernelGGL(k_take_token, dim3(1), dim3(1), 0, kr_stream(), tok, prompt, pos);
    kr_check_launch("take_token");
}

extern "C" void krh_advance(int *pos) {
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(1), 0, kr_stream(), pos);
    kr_check_launch("advance");
}

extern "C" void krh_math_batch(int op, float *y, const float *a, const float *b, size_t n) {
    hipLaunchKernelGGL(k_math_batch, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, kr_stream(), op, y, a, b, n);
    kr_check_launch("math_batch");
}

extern "C" void krh_ordered_sum(float *out, const float *t, int n, float s0) {
    if (n < 1 || n > KRH_ORDERED_SUM_MAX) {
        kr_fail(ML_E_SHAPE, "ordered_sum size", hipSuccess);
        return;
    }
    const size_t lds = sizeof(float) * (size_t)sc_terms_cap(n) + sc_lds_bytes(n, RN_THREADS);
    hipLaunchKernelGGL(k_ordered_sum, dim3(1), dim3(256), lds, kr_stream(), out, t, n, s0);
    kr_check_launch("ordered_sum");
}

extern "C" void krh_ordered_sum_lean(float *out, const float *t, int n, float s0) {
    if (n < 1 || n > KRH_ORDERED_SUM_MAX) {
        kr_fail(ML_E_SHAPE, "ordered_sum_lean size", hipSuccess);
        return;
    }
    const size_t lds = sizeof(float) * (size_t)sc_terms_cap(n) + sc_lds_bytes(n, RN_THREADS);
    hipLaunchKernelGGL(k_ordered_sum_lean, dim3(1), dim3(256), lds, kr_stream(), out, t, n, s0);
    kr_check_launch("ordered_sum_lean");
}

extern "C" void krh_ordered_sum_1024(float *out, const float *t, int n, float s0) {
    if (n < 1 || n > KRH_ORDERED_SUM_MAX) {
        kr_fail(ML_E_SHAPE, "ordered_sum_1024 size", hipSuccess);
        return;
    }
    const size_t lds = sizeof(float) * (size_t)sc_terms_cap(n) + sc_lds_bytes(n, 1024);
    hipLaunchKernelGGL(k_ordered_sum_1024, dim3(1), dim3(1024), lds, kr_stream(), out, t, n, s0);
    kr_check_launch("ordered_sum_1024");
}
extern "C" void krh_ordered_sum_wave(float *out, const float *t, int n, float s0) {
    if (n < 1 || n > KRH_ORDERED_SUM_WAVE_MAX) {
        kr_fail(ML_E_SHAPE, "ordered_sum_wave size", hipSuccess);
        return;
    }
    const size_t lds = sizeof(float) * (size_t)sc_terms_cap(n) + sc_lds_bytes(n, 64);
    hipLaunchKernelGGL(k_ordered_sum_wave, dim3(1), dim3(128), lds, kr_stream(), out, t, n, s0);
    kr_check_launch("ordered_sum_wave");
}

extern "C" void krh_h2f_batch(float *y, const uint16_t *h, size_t n) {
    hipLaunchKernelGGL(k_h2f_batch, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, kr_stream(), y, h, n);
    kr_check_launch("h2f_batch");
}

extern "C" void krh_block_dots(int32_t *s, const krh_mat *W, const int8_t *xq) {
    const size_t n = (size_t)W->rows * (W->cols / KR_QK);
    hipLaunchKernelGGL(k_block_dots, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, kr_stream(), s, to_kmat(W),
                       xq);
    kr_check_launch("block_dots");
}
