// Batched prompt prefill on gfx950: the matrix products as int8 MFMA.
//
// Y[t][r] = sum over blocks b, in block order, of ((float)S * wd[r][b]) * xd[t][b]
// where S = the exact int32 dot of block b of weight row r with block b of
// token t's Q8_0 activation: the scalar kernel's float order for every token
// (kernels/scalar/k_scalar.c:4-37, ops/ops.c:51-73), so each token's result is
// bit-identical to the decode matvec's (model/transformer.c:381-384).
//
// One v_mfma_i32_32x32x32_i8 computes S for a 32-token x 32-row tile and one
// block (K = 32 = one Q8_0 block). Operand lanes (checked on the device):
// lane l supplies A[l % 32][16 (l / 32) .. +15] and B[16 (l / 32) .. +15][l % 32];
// result register r of lane l is C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
// A = the tokens' activations, B = the weight rows, so each lane holds one
// weight row (one scale per block) and 16 tokens, whose scales come from the
// transposed activation scales xdT[b][t] through the workgroup's LDS tile. The per-block rescale and the
// ordered accumulation are 4 unfused VALU operations per output and block,
// which bound the kernel, not the MFMA.
#include "kr_internal.h"
#include "kr_numerics.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

struct MMat {
    const uint8_t *q;
    const void *d;
    int rows, cols, type, d16;
};

enum { MM_STORE = 0, MM_ADD = 1, MM_QKV = 2, MM_SWIGLU = 3 };

struct MmArgs {
    MMat w[3];
    int tile0[4];        // first workgroup of matrix i; tile0[nmat] = grid size
    int nmat;
    const int8_t *xq;    // [T][K] (rows up to the padded token count readable)
    const float *xdT;    // activation scale of block b of token t: xdT[b * xsb + t * xst]
    int ldx;             // T rounded up to MM_TT: xq's readable rows
    int xsb, xst;        // transposed [K / 32][ldx]: ldx and 1; token rows [T][K / 32]: 1 and K / 32
    int T, K;
    float *y[3];         // y[i][t * ldy[i] + r]
    int ldy[3];
    const float *bias[3];
    const float *rope_cos, *rope_sin;
    int head_dim, pos0;
    int ng;              // row groups per wave (the kernel's NG)
    int tw;              // waves per workgroup (the kernel's TW): 32 TW tokens a workgroup
    int8_t *hq;          // MM_SWIGLU: h's Q8_0 quants [T][rows] and scales [rows / 32][ldx]
    float *hdT;
};

constexpr int MM_TT = 128;   // tokens per workgroup

// 16 signed quant bytes of half h (elements 16h .. 16h+15) of a weight block
template <int QT>
__device__ __forceinline__ v4i weight_frag(const uint8_t *blk, int h) {
    if (QT == ML_Q8_0) {
        const int4 v = *(const int4 *)(blk + 16 * h);
        return v4i{ v.x, v.y, v.z, v.w };
    }
    // byte p of a Q4 block holds element p (low nibble) and p + 16 (high);
    // nibble n is weight n - 8: (n | 0x80) - 8 never borrows across bytes,
    // and ^ 0x80 then leaves n - 8 as a signed byte
    const int4 v = *(const int4 *)blk;
    const unsigned sh = 4u * (unsigned)h, M = 0x0F0F0F0Fu;
    v4i r;
    r.x = (int)((((((unsigned)v.x >> sh) & M) | 0x80808080u) - 0x08080808u) ^ 0x80808080u);
    r.y = (int)((((((unsigned)v.y >> sh) & M) | 0x80808080u) - 0x08080808u) ^ 0x80808080u);
    r.z = (int)((((((unsigned)v.z >> sh) & M) | 0x80808080u) - 0x08080808u) ^ 0x80808080u);
    r.w = (int)((((((unsigned)v.w >> sh) & M) | 0x80808080u) - 0x08080808u) ^ 0x80808080u);
    return r;
}

// A wave computes NG row groups x 1 token group of 32 (NG MFMA tiles per
// block); the workgroup's 4 waves take 4 token groups of the same 32 NG rows.
// NG = 4 when the grid of 128-row tiles fills the device (long prompts);
// NG = 1 gives four times the workgroups for short batches (the reference's
// 128-token prefill steps), whose few 128-row tiles would leave most CUs idle
// with each tile's VALU work in series.

// Per wave and block: the wave's 32 tokens.
struct XFrag {
    v4i xa;              // the wave's 32 tokens
};

// Per thread and block, for the workgroup's tile: 16 quant bytes of weight
// row tid / 2 (half tid % 2, Q4 unpacked to n - 8), that row's raw scale, and
// the scale of the workgroup's token tid % 128.
struct WReg {
    v4i w;
    uint32_t d;
    float xs;
};

constexpr int MM_ST = 3;   // LDS ring stages of the weight tile
constexpr int MM_PD = 8;   // NG = 1: blocks of load lookahead (even: the LDS stage of step k is k % 2)

template <int NG, int TT>
struct MmLds {
    v4i w[MM_ST][32 * NG][2];     // [stage][row][half]
    uint32_t d[MM_ST][32 * NG];   // [stage][row] raw scale bits
    float xs[MM_ST][TT];          // [stage][token] the tokens' scales
};

__device__ __forceinline__ void x_load(XFrag &f, const MmArgs &a, int b, int tokl, int lane) {
    const int t = tokl + (lane & 31);   // readable: the caller pads the activations to ldx rows
    const int4 v = *(const int4 *)(a.xq + (size_t)t * a.K + (size_t)b * 32 + 16 * (lane >> 5));
    f.xa = v4i{ v.x, v.y, v.z, v.w };
}

// thread tid loads half tid % 2 of tile row (tid / 2) mod 32 NG (for NG < 4
// the surplus threads repeat a row's load, which keeps every load
// unconditional; only the first 64 NG store it)
// (xcol: the scales of this thread's token, tid % TT of the workgroup's,
// clamped to the last token; threads TT.. repeat thread tid % TT's load,
// unused; xsb: the stride from block to block). PAIR (NG
// 4): tile rows 0-63 are rows rowl.. of W, tile rows 64-127 the same rows of
// W2 (SwiGLU's w1 and w3).
template <int QT, int D16, int NG, int TT, bool PAIR = false>
__device__ __forceinline__ void w_load(WReg &R, const MMat &W, const float *xcol, int xsb, int nb, int b, int rowl,
                                       int tid, const MMat &W2 = MMat{}) {
    const int tr = (tid >> 1) & (32 * NG - 1);
    int r = rowl + (PAIR ? tr & 63 : tr);
    r = r < W.rows ? r : W.rows - 1;   // rows past the end re-read the last row (not stored)
    const size_t blk = (size_t)r * nb + b;
    const uint8_t *wq = PAIR && tr >= 64 ? W2.q : W.q;
    const void *wd = PAIR && tr >= 64 ? W2.d : W.d;
    R.w = weight_frag<QT>(wq + blk * (QT == ML_Q8_0 ? 32 : 16), tid & 1);
    R.d = D16 ? (uint32_t)((const uint16_t *)wd)[blk] : ((const uint32_t *)wd)[blk];
    R.xs = xcol[(size_t)b * xsb];
}

template <int NG, int TT>
__device__ __forceinline__ void w_store(MmLds<NG, TT> &L, int st, const WReg &R, int tid) {
    if (tid < TT) L.xs[st][tid] = R.xs;
    if ((tid >> 1) >= 32 * NG) return;
    L.w[st][tid >> 1][tid & 1] = R.w;
    if ((tid & 1) == 0) L.d[st][tid >> 1] = R.d;
}

// Row group g + 1's MFMA is issued after the whole rescale of group g: an
// empty asm takes every rescaled value of group g as input and the MFMA's
// weight operand as in-out, so only one 16-register result set is live.
// Left to itself the compiler issues all NG MFMAs of a step together and
// holds NG result sets (64 VGPRs at NG 4: 183 VGPRs, 2 waves per SIMD);
// with one set the kernel takes 146 VGPRs and runs 3 waves per SIMD, whose
// interleaving hides the MFMA latency the wave itself now waits out (8B-shape
// prefill 22.0k -> 23.0k tok/s; an MFMA lookahead of half a group, or 4
// waves per SIMD, spills). The 16 token scales a lane needs
// (tokens 8 (r / 4) + 4 (lane / 32) + r % 4 of the wave's 32: the same for
// the 32 lanes of a half-wave) are four 16-byte LDS broadcast reads of the
// tile's token scales (16 cross-lane shuffles of one loaded scale per lane
// cost 3-6% more time). The weight fragments and scales come from the
// workgroup's LDS tile as well.
template <int D16, int NG, int TT>
__device__ __forceinline__ void mm_step(float (&acc)[NG][16], const XFrag &f, const MmLds<NG, TT> &L, int st, int lane,
                                        int tokw) {
    const int ln = lane & 31, hf = lane >> 5;
    v4i wb[NG];
    uint32_t wdr[NG];
#pragma unroll
    for (int g = 0; g < NG; g++) {
        wb[g] = L.w[st][32 * g + ln][hf];
        wdr[g] = L.d[st][32 * g + ln];
    }
    float xd[16];
    const float4 *xv = (const float4 *)&L.xs[st][tokw + 4 * hf];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float4 v = xv[2 * q];   // tokens 8 q + 4 hf .. + 3
        xd[4 * q] = v.x;
        xd[4 * q + 1] = v.y;
        xd[4 * q + 2] = v.z;
        xd[4 * q + 3] = v.w;
    }
    v16i s = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.xa, wb[0], v16i{}, 0, 0, 0);
    // one row group: the loads around the step stay on their side of its
    // MFMA (measured 10% faster on the 32-row tiles than a free schedule)
    if constexpr (NG == 1) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int g = 0; g < NG; g++) {
        const float wd = D16 ? kr_h2f((uint16_t)wdr[g]) : __uint_as_float(wdr[g]);
#pragma unroll
        for (int r = 0; r < 16; r++)
            acc[g][r] = kr_fadd(acc[g][r], kr_fmul(kr_fmul((float)s[r], wd), xd[r]));
        if (g + 1 < NG) {
            v4i w = wb[g + 1];
#pragma unroll
            for (int r = 0; r < 16; r++) asm volatile("" : "+v"(w) : "v"(acc[g][r]));
            s = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.xa, w, v16i{}, 0, 0, 0);
        }
    }
}

// Workgroup = TW waves (4, or 1 for short batches) over a 32 NG-row x
// 32 TW-token tile; wave w takes all the tile's rows (NG row groups) and
// tokens 32 w .. 32 w + 31. The workgroup's
// threads load each block's weight tile and its scales once (16 bytes and
// one scale per thread) into an LDS ring of 3 stages: block b + 1 is stored
// during step b into the stage step b - 2 read, and the barrier closing each
// step orders those stores before step b + 1 reads them.
template <int EPI, int QT, int D16, int NG, int TW = 4>
__global__ void __launch_bounds__(64 * TW, NG == 1 ? 2 : 3) k_matmul(const MmArgs a) {   // waves per SIMD, at least
    constexpr int TT = 32 * TW;   // tokens per workgroup
    __shared__ MmLds<NG, TT> L;
    int mi = 0;
    while (mi + 1 < a.nmat && (int)blockIdx.x >= a.tile0[mi + 1]) mi++;
    const MMat W = mi == 0 ? a.w[0] : (mi == 1 ? a.w[1] : a.w[2]);
    const int ntt = (a.T + TT - 1) / TT;
    const int local = (int)blockIdx.x - a.tile0[mi];
    const int rt = local / ntt, tt = local - rt * ntt;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    constexpr bool PAIR = EPI == MM_SWIGLU;   // 64 rows of w1 and the same 64 of w3
    const int rowl = rt * (PAIR ? 64 : 32 * NG), tokl = tt * TT + 32 * wave;
    const int nb = a.K / KR_QK;
    const float *xcol = a.xdT + (size_t)min(tt * TT + (tid & (TT - 1)), a.T - 1) * a.xst;

    float acc[NG][16];
#pragma unroll
    for (int g = 0; g < NG; g++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[g][r] = 0.0f;

    // Loads are unconditional (block indices past the end re-read the last
    // block, unused): a load issued on only one path makes the wait-count
    // pass drain every in-flight load at the loop head, which would cancel
    // the prefetch. Only the odd tail's step is conditional; every thread
    // reaches every barrier.
    const int bl = nb - 1;
    if constexpr (NG >= 2) {
        WReg R;
        XFrag x0, x1;
        w_load<QT, D16, NG, TT, PAIR>(R, W, xcol, a.xsb, nb, 0, rowl, tid, a.w[1]);
        w_store(L, 0, R, tid);
        w_load<QT, D16, NG, TT, PAIR>(R, W, xcol, a.xsb, nb, 1 < bl ? 1 : bl, rowl, tid, a.w[1]);
        x_load(x0, a, 0, tokl, lane);
        x_load(x1, a, 1 < bl ? 1 : bl, tokl, lane);
        __syncthreads();
        int st = 0;   // stage of block b
        for (int b = 0; b < nb; b += 2) {
            const int s1 = st == MM_ST - 1 ? 0 : st + 1, s2 = s1 == MM_ST - 1 ? 0 : s1 + 1;
            w_store(L, s1, R, tid);
            w_load<QT, D16, NG, TT, PAIR>(R, W, xcol, a.xsb, nb, b + 2 < bl ? b + 2 : bl, rowl, tid, a.w[1]);
            mm_step<D16, NG, TT>(acc, x0, L, st, lane, 32 * wave);
            x_load(x0, a, b + 2 < bl ? b + 2 : bl, tokl, lane);
            __syncthreads();
            w_store(L, s2, R, tid);
            w_load<QT, D16, NG, TT, PAIR>(R, W, xcol, a.xsb, nb, b + 3 < bl ? b + 3 : bl, rowl, tid, a.w[1]);
            if (b + 1 < nb) mm_step<D16, NG, TT>(acc, x1, L, s1, lane, 32 * wave);
            x_load(x1, a, b + 3 < bl ? b + 3 : bl, tokl, lane);
            __syncthreads();
            st = s2;
        }
    } else {
        // One row group: a block's VALU work is a quarter of NG = 4's, too
        // little to cover a load's latency, so the weight and token loads
        // run MM_PD blocks ahead in register rings (R[j], x[j]: the blocks
        // congruent to j mod MM_PD), and the weight tile passes through a
        // 2-stage LDS ring. Step t stores block t + 1 (loaded MM_PD steps
        // earlier) into stage (t + 1) % 2, loads block t + 1 + MM_PD in its
        // place, runs block t from stage t % 2 and reloads x with block
        // t + MM_PD; the barrier closing each step orders the stage writes
        // against the reads of the steps either side.
        WReg R[MM_PD];
        XFrag x[MM_PD];
#pragma unroll
        for (int j = 0; j < MM_PD; j++) {
            w_load<QT, D16, NG, TT, PAIR>(R[j], W, xcol, a.xsb, nb, j < bl ? j : bl, rowl, tid, a.w[1]);
            x_load(x[j], a, j < bl ? j : bl, tokl, lane);
        }
        w_store(L, 0, R[0], tid);
        w_load<QT, D16, NG, TT, PAIR>(R[0], W, xcol, a.xsb, nb, MM_PD < bl ? MM_PD : bl, rowl, tid, a.w[1]);
        __syncthreads();
        for (int b0 = 0; b0 < nb; b0 += MM_PD) {
#pragma unroll
            for (int k = 0; k < MM_PD; k++) {
                const int t = b0 + k, k1 = (k + 1) % MM_PD;
                w_store(L, (k + 1) & 1, R[k1], tid);
                w_load<QT, D16, NG, TT, PAIR>(R[k1], W, xcol, a.xsb, nb, t + 1 + MM_PD < bl ? t + 1 + MM_PD : bl, rowl,
                                          tid, a.w[1]);
                if (t < nb) mm_step<D16, NG, TT>(acc, x[k], L, k & 1, lane, 32 * wave);
                x_load(x[k], a, t + MM_PD < bl ? t + MM_PD : bl, tokl, lane);
                __syncthreads();
            }
        }
    }

    // epilogue: lane = one row (32 g + lane % 32), tokens 8 (r / 4) + 4 (lane / 32) + r % 4
    if constexpr (PAIR) {
        // h = silu(w1 x) * (w3 x) (k_scalar.c:96-98), then its Q8_0 in blocks
        // of 32 rows (k_scalar.c:39-57): a block's 32 values are the 32 lanes
        // of a half-wave (groups 0, 1: w1 rows; 2, 3: the same w3 rows)
#pragma unroll
        for (int g = 0; g < 2; g++) {
            const int row = rowl + 32 * g + (lane & 31);
            const bool bin = rowl + 32 * g < W.rows;   // rows % 32 == 0: whole blocks in or out
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int t = tokl + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const float h1 = acc[g][r], h3 = acc[g + 2][r];
                const float v = kr_fmul(kr_fdiv(h1, kr_fadd(1.0f, kr_expf(-h1))), h3);
                int8_t q;
                float d;
                kr_quant_block32(v, &q, &d);
                if (bin && t < a.T) {
                    a.hq[(size_t)t * W.rows + row] = q;
                    if ((lane & 31) == 0) a.hdT[(size_t)(row >> 5) * a.ldx + t] = d;
                }
            }
        }
        return;
    }
    float *Y = mi == 0 ? a.y[0] : (mi == 1 ? a.y[1] : a.y[2]);
    const int ldy = mi == 0 ? a.ldy[0] : (mi == 1 ? a.ldy[1] : a.ldy[2]);
    const float *bias = mi == 0 ? a.bias[0] : (mi == 1 ? a.bias[1] : a.bias[2]);
#pragma unroll
    for (int g = 0; g < NG; g++) {
        const int row = rowl + 32 * g + (lane & 31);
        const bool rin = row < W.rows;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int t = tokl + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            float v = acc[g][r];
            if (EPI == MM_QKV) {
                // bias (model/transformer.c:276-277), then RoPE on q and k
                // (k_scalar.c:79-94): rows 2i, 2i+1 sit in lanes 2i, 2i+1
                if (bias && rin) v = kr_fadd(v, bias[row]);
                const float o = __shfl_xor(v, 1);
                if (mi < 2) {
                    const int hd = a.head_dim, j = row % hd, h2 = hd >> 1;
                    const int pos = a.pos0 + (t < a.T ? t : 0);
                    const float c = a.rope_cos[(size_t)pos * h2 + (j >> 1)];
                    const float sn = a.rope_sin[(size_t)pos * h2 + (j >> 1)];
                    v = (j & 1) == 0 ? kr_fsub(kr_fmul(v, c), kr_fmul(o, sn)) : kr_fadd(kr_fmul(o, sn), kr_fmul(v, c));
                }
            }
            if (rin && t < a.T) {
                float *p = Y + (size_t)t * ldy + row;
                if (EPI == MM_ADD) *p = kr_fadd(*p, v);
                else *p = v;
            }
        }
    }
}

template <int EPI>
void launch_mm(const MmArgs &a, const MMat &W) {
    const int grid = a.tile0[a.nmat];
    if (a.K % KR_QK || a.T <= 0 || grid <= 0 || a.ldx % MM_TT || a.T > a.ldx || a.xsb <= 0 || a.xst <= 0 || (a.tw != 4 && (a.tw != 1 || a.ng != 1))) {
        kr_fail(ML_E_SHAPE, "matmul shape", hipSuccess);
        return;
    }
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * a.tw), 0, kr_stream(), a); };
    if (EPI == MM_SWIGLU && a.ng != 4) {
        kr_fail(ML_E_SHAPE, "matmul: SwiGLU pairs take 128-row tiles", hipSuccess);
        return;
    }
    if (a.ng == 4) {
        if (W.type == ML_Q8_0) {
            if (W.d16) go(k_matmul<EPI, ML_Q8_0, 1, 4>); else go(k_matmul<EPI, ML_Q8_0, 0, 4>);
        } else {
            if (W.d16) go(k_matmul<EPI, ML_Q4_0, 1, 4>); else go(k_matmul<EPI, ML_Q4_0, 0, 4>);
        }
    } else if constexpr (EPI != MM_SWIGLU) {
        if (a.ng == 2) {
            if (W.type == ML_Q8_0) {
                if (W.d16) go(k_matmul<EPI, ML_Q8_0, 1, 2>); else go(k_matmul<EPI, ML_Q8_0, 0, 2>);
            } else {
                if (W.d16) go(k_matmul<EPI, ML_Q4_0, 1, 2>); else go(k_matmul<EPI, ML_Q4_0, 0, 2>);
            }
            kr_check_launch("matmul");
            return;
        }
        if (a.tw == 1) {
            if (W.type == ML_Q8_0) {
                if (W.d16) go(k_matmul<EPI, ML_Q8_0, 1, 1, 1>); else go(k_matmul<EPI, ML_Q8_0, 0, 1, 1>);
            } else {
                if (W.d16) go(k_matmul<EPI, ML_Q4_0, 1, 1, 1>); else go(k_matmul<EPI, ML_Q4_0, 0, 1, 1>);
            }
        } else if (W.type == ML_Q8_0) {
            if (W.d16) go(k_matmul<EPI, ML_Q8_0, 1, 1>); else go(k_matmul<EPI, ML_Q8_0, 0, 1>);
        } else {
            if (W.d16) go(k_matmul<EPI, ML_Q4_0, 1, 1>); else go(k_matmul<EPI, ML_Q4_0, 0, 1>);
        }
    }
    kr_check_launch("matmul");
}

MMat to_mmat(const krh_mat *m) {
    MMat k = { (const uint8_t *)m->q, m->d, m->rows, m->cols, m->type, m->d16 };
    return k;
}

int row_tiles(int rows, int ng) { return (rows + 32 * ng - 1) / (32 * ng); }

// NG for a launch over these row counts and ntt token tiles: 4 when it has
// at least two 128-row tiles per CU, else 2 when it has half a 64-row tile
// per CU (w1 and w3 at the reference's 128-token steps: its 8B prefill
// through ml_run 5,674 -> 5,844 tok/s), else 1. One 128-row tile per CU
// leaves each SIMD one wave, which issues a VALU instruction only every 6.5
// cycles or more: the 1B shape's wo and w2 (256 tiles at 2048 tokens) on
// 64-row tiles took its 4000-token prefill from 65.4k-65.7k to 67.6k-67.8k
// tok/s (the threshold was 3/4 of a tile per CU); 64-row tiles up to 3 or 4
// tiles per CU took the 8B shape's from 21.6k-21.8k to 20.4k-20.5k. Measured (K = 4096, 256
// CUs): a 128-row tile does 4 times a 32-row tile's work in 1.9 times its
// time, so from about 200 tiles, where the 32-row grid needs two rounds of
// resident workgroups, the 128-row grid's one round is the shorter (14336
// rows at T = 512: 152 against 300 us); below it, 32-row tiles keep more CUs
// busy (T = 128, 112 tiles: 89 us, where one round of 128-row tiles takes
// about what it takes at T = 192, 125 us).
int pick_ng(int rows0, int rows1, int rows2, int ntt) {
    const int tiles = row_tiles(rows0, 4) + row_tiles(rows1, 4) + row_tiles(rows2, 4);
    const int cus = krh_device_cus() > 0 ? krh_device_cus() : 256;
    const int tiles2 = row_tiles(rows0, 2) + row_tiles(rows1, 2) + row_tiles(rows2, 2);
    return tiles * ntt >= 2L * cus ? 4 : 2L * tiles2 * ntt >= cus ? 2 : 1;
}

// Waves per workgroup (TW) for an NG 1 launch whose grid of 128-token tiles
// leaves CUs idle (fewer than two 32-row tiles per CU: the reference's
// 128-token steps over wq, wk, wv, wo and w2): one wave and 32 tokens a
// workgroup gives 4 times the workgroups. Else 4.
int pick_tw(int ng, int grid128) {
    const int cus = krh_device_cus() > 0 ? krh_device_cus() : 256;
    return ng == 1 && grid128 < 2 * cus ? 1 : 4;
}

// ---- per-token work of a batched step ----

// h = silu(g) * u (k_scalar.c:96-98) for ntok rows of n, then Q8_0 of h
// into q [t][n] and the transposed scales dT[b * ldd + t].
__global__ void __launch_bounds__(256) k_silu_quant(int8_t *q, float *dT, int ldd, const float *g, const float *u,
                                                    int n) {
    const size_t t = blockIdx.y;
    const int i = blockIdx.x * 1024 + 4 * threadIdx.x;
    if (i >= n) return;   // n % 32 == 0
    const float4 gv = *(const float4 *)(g + t * n + i), uv = *(const float4 *)(u + t * n + i);
    float4 v;
    v.x = kr_fmul(kr_fdiv(gv.x, kr_fadd(1.0f, kr_expf(-gv.x))), uv.x);
    v.y = kr_fmul(kr_fdiv(gv.y, kr_fadd(1.0f, kr_expf(-gv.y))), uv.y);
    v.z = kr_fmul(kr_fdiv(gv.z, kr_fadd(1.0f, kr_expf(-gv.z))), uv.z);
    v.w = kr_fmul(kr_fdiv(gv.w, kr_fadd(1.0f, kr_expf(-gv.w))), uv.w);
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
    *(int *)(q + t * n + i) = packed;
    if ((i & 31) == 0) dT[(size_t)(i >> 5) * ldd + t] = dd;
}

__global__ void k_embed_batch(float *x, const MMat e, const int *tok, float scale) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x, t = blockIdx.y;
    if (i >= e.cols) return;
    const int nb = e.cols / KR_QK, row = tok[t], b = i / KR_QK, j = i % KR_QK;
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
    x[(size_t)t * e.cols + i] = o;
}

}  // namespace

// ---- C ABI ----

extern "C" void krh_matmul_swiglu(int8_t *hq, float *hdT, const krh_mat *w1, const krh_mat *w3, const int8_t *xq,
                                  const float *xdT, int ldx, int T) {
    if (!hq || !hdT || w1->rows != w3->rows || w1->cols != w3->cols || w1->type != w3->type || w1->d16 != w3->d16 ||
        w1->rows % KR_QK) {
        kr_fail(ML_E_SHAPE, "matmul_swiglu: w1 and w3 of one shape, type and scale width, rows % 32 == 0",
                hipSuccess);
        return;
    }
    MmArgs a = {};
    a.w[0] = to_mmat(w1);
    a.w[1] = to_mmat(w3);
    a.nmat = 1;
    a.tile0[0] = 0;
    const int ntt = (T + MM_TT - 1) / MM_TT;
    a.ng = 4;
    a.tw = 4;
    a.tile0[1] = (w1->rows + 63) / 64 * ntt;
    a.xq = xq;
    a.xdT = xdT;
    a.ldx = ldx;
    a.xsb = ldx;
    a.xst = 1;
    a.T = T;
    a.K = w1->cols;
    a.hq = hq;
    a.hdT = hdT;
    launch_mm<MM_SWIGLU>(a, a.w[0]);
}

// one matrix over T tokens; the scales' strides say their layout
static void matmul_one(float *Y, int ldy, const krh_mat *W, const int8_t *xq, const float *xd, int ldx, int T,
                       int accumulate, int xsb, int xst) {
    MmArgs a = {};
    a.w[0] = to_mmat(W);
    a.nmat = 1;
    a.tile0[0] = 0;
    const int ntt128 = (T + MM_TT - 1) / MM_TT;
    a.ng = pick_ng(W->rows, 0, 0, ntt128);
    a.tw = pick_tw(a.ng, row_tiles(W->rows, a.ng) * ntt128);
    const int ntt = (T + 32 * a.tw - 1) / (32 * a.tw);
    a.tile0[1] = row_tiles(W->rows, a.ng) * ntt;
    a.xq = xq;
    a.xdT = xd;
    a.ldx = ldx;
    a.xsb = xsb;
    a.xst = xst;
    a.T = T;
    a.K = W->cols;
    a.y[0] = Y;
    a.ldy[0] = ldy;
    if (accumulate) launch_mm<MM_ADD>(a, a.w[0]);
    else launch_mm<MM_STORE>(a, a.w[0]);
}

extern "C" void krh_matmul(float *Y, int ldy, const krh_mat *W, const int8_t *xq, const float *xdT, int ldx, int T,
                           int accumulate) {
    matmul_one(Y, ldy, W, xq, xdT, ldx, T, accumulate, ldx, 1);
}

extern "C" void krh_matmul_rows(float *Y, int ldy, const krh_mat *W, const int8_t *xq, const float *xd, int ldx,
                                int T, int accumulate) {
    matmul_one(Y, ldy, W, xq, xd, ldx, T, accumulate, 1, W->cols / KR_QK);
}

// k and v go to the F32 cache rows pos0 + t, or with stage set to the
// staging rows kc, vc [T][kv_dim] of an F16 / Q8 cache
static void matmul_qkv(float *q, float *kc, float *vc, const krh_mat *wq, const krh_mat *wk, const krh_mat *wv,
                       const float *bq, const float *bk, const float *bv, const int8_t *xq, const float *xdT, int ldx,
                       int T, const float *rope_cos, const float *rope_sin, int head_dim, int pos0, bool stage) {
    if (wq->cols != wk->cols || wq->cols != wv->cols || wk->rows != wv->rows || head_dim % 2 || wq->type != wk->type ||
        wq->d16 != wk->d16 || wv->d16 != wq->d16) {
        kr_fail(ML_E_SHAPE, "matmul qkv shapes", hipSuccess);
        return;
    }
    const int ntt128 = (T + MM_TT - 1) / MM_TT;
    MmArgs a = {};
    a.w[0] = to_mmat(wq);
    a.w[1] = to_mmat(wk);
    a.w[2] = to_mmat(wv);
    a.xq = xq;
    a.xdT = xdT;
    a.ldx = ldx;
    a.xsb = ldx;
    a.xst = 1;
    a.T = T;
    a.K = wq->cols;
    // q rows [t][q_dim]; k and v straight into the cache rows pos0 + t
    a.y[0] = q;
    a.ldy[0] = wq->rows;
    a.y[1] = kc + (stage ? 0 : (size_t)pos0 * wk->rows);
    a.ldy[1] = wk->rows;
    a.y[2] = vc + (stage ? 0 : (size_t)pos0 * wv->rows);
    a.ldy[2] = wv->rows;
    a.bias[0] = bq;
    a.bias[1] = bk;
    a.bias[2] = bv;
    a.rope_cos = rope_cos;
    a.rope_sin = rope_sin;
    a.head_dim = head_dim;
    a.pos0 = pos0;
    a.ng = pick_ng(wq->rows, wk->rows, wv->rows, ntt128);
    a.tw = pick_tw(a.ng, (row_tiles(wq->rows, a.ng) + 2 * row_tiles(wk->rows, a.ng)) * ntt128);
    const int ntt = (T + 32 * a.tw - 1) / (32 * a.tw);
    a.tile0[0] = 0;
    a.tile0[1] = row_tiles(wq->rows, a.ng) * ntt;
    a.tile0[2] = a.tile0[1] + row_tiles(wk->rows, a.ng) * ntt;
    a.tile0[3] = a.tile0[2] + row_tiles(wv->rows, a.ng) * ntt;
    if (wv->type == wq->type) {
        a.nmat = 3;
        launch_mm<MM_QKV>(a, a.w[0]);
        return;
    }
    MmArgs b = a;   // q and k
    b.nmat = 2;
    launch_mm<MM_QKV>(b, b.w[0]);
    MmArgs c = a;   // v alone, as matrix 2 of the same epilogue
    c.tile0[0] = c.tile0[1] = c.tile0[2] = 0;
    c.tile0[3] = row_tiles(wv->rows, a.ng) * ntt;
    c.w[0] = c.w[1] = c.w[2];
    c.nmat = 3;
    launch_mm<MM_QKV>(c, c.w[2]);
}

extern "C" void krh_matmul_qkv(float *q, float *kc, float *vc, const krh_mat *wq, const krh_mat *wk,
                               const krh_mat *wv, const float *bq, const float *bk, const float *bv, const int8_t *xq,
                               const float *xdT, int ldx, int T, const float *rope_cos, const float *rope_sin,
                               int head_dim, int pos0) {
    matmul_qkv(q, kc, vc, wq, wk, wv, bq, bk, bv, xq, xdT, ldx, T, rope_cos, rope_sin, head_dim, pos0, false);
}

extern "C" void krh_matmul_qkv_stage(float *q, float *k, float *v, const krh_mat *wq, const krh_mat *wk,
                                     const krh_mat *wv, const float *bq, const float *bk, const float *bv,
                                     const int8_t *xq, const float *xdT, int ldx, int T, const float *rope_cos,
                                     const float *rope_sin, int head_dim, int pos0) {
    matmul_qkv(q, k, v, wq, wk, wv, bq, bk, bv, xq, xdT, ldx, T, rope_cos, rope_sin, head_dim, pos0, true);
}

extern "C" void krh_silu_quant(int8_t *q, float *dT, int ldd, const float *g, const float *u, int n, int ntok) {
    if (n % KR_QK || ntok <= 0) { kr_fail(ML_E_SHAPE, "silu_quant shape", hipSuccess); return; }
    hipLaunchKernelGGL(k_silu_quant, dim3((n + 1023) / 1024, ntok), dim3(256), 0, kr_stream(), q, dT, ldd, g, u, n);
    kr_check_launch("silu_quant");
}

extern "C" void krh_embed_batch(float *x, const krh_mat *emb, const int *tok, int ntok, float embed_scale) {
    hipLaunchKernelGGL(k_embed_batch, dim3((emb->cols + 255) / 256, ntok), dim3(256), 0, kr_stream(), x, to_mmat(emb),
                       tok, embed_scale);
    kr_check_launch("embed_batch");
}
