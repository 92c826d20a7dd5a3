// Attention over one layer's KV cache for gfx950: scores, softmax and the
// position-ordered mix, for the F32, F16 and Q8 caches (ops/ops.c:124-238,
// kernels/scalar/k_scalar.c:66-77, :111-155), and the F16 / Q8 cache stores
// (model/transformer.c:191-205). Every float operation is the reference's,
// in its order.
#include "kr_internal.h"
#include "kr_numerics.h"
#include "kr_chain.h"

namespace {

// ---- attention (F32 cache) ----
//
// Per layer and position (ops/ops.c:124-155): for query head h (KV head
// h / group), s_t = (sum_i q_i k_t,i in index order) * scale
// (k_scalar.c:111-117), softmax over t (k_scalar.c:66-77: max, expf(x - max),
// the sum in position order, then x * (1 / sum)), and out_i = 0,
// out_i += a_t v_t,i in position order (k_scalar.c:119-122). The ordered
// chains run from LDS; the loads feeding them are wide and parallel.

constexpr int AT_T = 64;          // positions per score tile of a batched (prefill) launch
constexpr int AT_TD = 16;         // of a decode launch: more, smaller tiles hide the K loads better
constexpr int AT_THREADS = 256;

// positions attended by token blockIdx.z of the launch, at position *pos_p + blockIdx.z
__device__ __forceinline__ void attn_range(const int *pos_p, int window, int *first, int *n) {
    const int pos = *pos_p + (int)blockIdx.z;
    *first = window && pos >= window ? pos + 1 - window : 0;
    *n = pos + 1 - *first;
}

// The cache a launch reads (ml_kv_layer, ops/ops.h:16-22, of one layer): K
// and V rows [max_seq][kv_dim] of floats, halves or int8, and for the Q8
// cache the row scales kd, vd [max_seq][n_kv_heads] (model/transformer.c:169-180).
enum { KV_F32 = 0, KV_F16 = 1, KV_Q8 = 2 };
struct KvView {
    const void *k, *v;
    const float *kd, *vd;
    int n_kv;
    const float *ks, *vs;   // Q8 decode: row *pos's K and V, still to be stored (else null)
};

// 4 consecutive cache elements: the registers as loaded, and widened to
// floats (halves exactly, k_scalar.c:124-135; int8 to its value, :148-155)
template <int KT> struct Kv4;
template <> struct Kv4<KV_F32> {
    using T = float4;
    static constexpr int REGS = 4;
    __device__ static T load(const void *p, size_t i) { return *(const float4 *)((const float *)p + i); }
    __device__ static float4 wide(T v) { return v; }
};
template <> struct Kv4<KV_F16> {
    using T = uint2;
    static constexpr int REGS = 2;
    __device__ static T load(const void *p, size_t i) { return *(const uint2 *)((const uint16_t *)p + i); }
    __device__ static float4 wide(T v) {
        return make_float4(kr_h2f((uint16_t)v.x), kr_h2f((uint16_t)(v.x >> 16)), kr_h2f((uint16_t)v.y),
                           kr_h2f((uint16_t)(v.y >> 16)));
    }
};
template <> struct Kv4<KV_Q8> {
    using T = int;
    static constexpr int REGS = 1;
    __device__ static T load(const void *p, size_t i) { return *(const int *)((const int8_t *)p + i); }
    __device__ static float4 wide(T v) {
        return make_float4((float)(int8_t)v, (float)(int8_t)(v >> 8), (float)(int8_t)(v >> 16), (float)(v >> 24));
    }
};

// Scores of one KV head's query heads for TT positions. The K tile is staged
// in LDS as floats (F16 rows widened exactly, k_scalar.c:124-129), rows hd + 4
// floats apart so that the 16-byte reads of 8 consecutive lanes cover all
// banks once; thread (t, j) computes heads j, j + 4, ... of the group for
// position t, adding the products in index order.
template <int KT, int TT>
__device__ __forceinline__ void attn_scores(float *att, const float *q, const KvView kv, int group, int hd, int kv_dim,
                                            int max_seq, int window, float scale, const int *pos_p) {
    extern __shared__ __align__(16) float at_smem[];
    int first, n;
    attn_range(pos_p, window, &first, &n);
    att += (size_t)blockIdx.z * gridDim.x * group * max_seq;   // token z: [n_heads][max_seq]
    q += (size_t)blockIdx.z * gridDim.x * group * hd;
    const int g = blockIdx.x, t0 = blockIdx.y * TT, tid = threadIdx.x;
    if (t0 >= n) return;
    const int nt = min(TT, n - t0), ks = hd + 4, h4 = hd / 4;
    float *qs = at_smem, *kt = at_smem + group * hd;
    const float4 *qg = (const float4 *)(q + (size_t)g * group * hd);
    for (int i = tid; i < group * h4; i += AT_THREADS) ((float4 *)qs)[i] = qg[i];
    for (int e = tid; e < nt * h4; e += AT_THREADS) {
        const int r = e / h4, c = e - r * h4;
        *(float4 *)(kt + r * ks + 4 * c) =
            Kv4<KT>::wide(Kv4<KT>::load(kv.k, (size_t)(first + t0 + r) * kv_dim + (size_t)g * hd + 4 * c));
    }
    __syncthreads();
    const int t = tid % TT;
    if (t >= nt) return;
    const float *kr = kt + t * ks;
    for (int j = tid / TT; j < group; j += AT_THREADS / TT) {
        const float *qh = qs + j * hd;
        float acc = 0.0f;
#pragma unroll 4
        for (int i = 0; i < hd; i += 4) {
            const float4 a = *(const float4 *)(qh + i), b = *(const float4 *)(kr + i);
            acc = kr_fadd(acc, kr_fmul(a.x, b.x));
            acc = kr_fadd(acc, kr_fmul(a.y, b.y));
            acc = kr_fadd(acc, kr_fmul(a.z, b.z));
            acc = kr_fadd(acc, kr_fmul(a.w, b.w));
        }
        att[(size_t)(g * group + j) * max_seq + t0 + t] = kr_fmul(acc, scale);
    }
}

// the F32 cache (its own argument list: the view is built on the device)
template <int TT>
__global__ void __launch_bounds__(AT_THREADS) k_attn_scores(float *att, const float *q, const float *kc, int group,
                                                            int hd, int kv_dim, int max_seq, int window, float scale,
                                                            const int *pos_p) {
    const KvView kv = { kc, nullptr, nullptr, nullptr, 0 };
    attn_scores<KV_F32, TT>(att, q, kv, group, hd, kv_dim, max_seq, window, scale, pos_p);
}

// Batched (prefill) scores over the F32 or F16 cache without a window, a
// block of AT_TB tokens at a time (F16 rows widened exactly as the K tile is
// staged). Every token of the block attends from position 0,
// so one K tile of AT_T positions, staged once in LDS, serves the whole block
// (the per-token kernel stages it again for every token). The queries of QB
// tokens at a time follow in LDS; thread (position t, head j) runs the QB
// chains of those tokens in one pass over the head's dims, one K read feeding
// them all (QB independent chains: the LDS latency hides under them). Each
// chain is the per-token kernel's: s = sum_i q_i k_i in index order, then
// * scale; a token stores only the positions it attends. HD: the head size
// when it is 64 or 128, else 0 (any). TP: positions per K tile, AT_T, or
// AT_T / 2 for heads whose AT_T-position tile and queries exceed 64 KB of
// LDS (Gemma's 256-wide heads).
constexpr int AT_TB = 16;
template <int HD, int QB, int KT, int TP = AT_T>
__global__ void __launch_bounds__(AT_THREADS) k_attn_scores_blk(float *att, const float *q, const KvView kv, int group,
                                                                int hd_arg, int kv_dim, int max_seq, float scale,
                                                                const int *pos_p, int ntok) {
    extern __shared__ __align__(16) float at_smem[];
    const int hd = HD ? HD : hd_arg;
    const int g = blockIdx.x, t0 = blockIdx.y * TP, z0 = blockIdx.z * AT_TB, tid = threadIdx.x;
    const int pos0 = *pos_p, zn = min(AT_TB, ntok - z0);
    const int nlast = pos0 + z0 + zn;   // positions the block's last token attends
    if (t0 >= nlast) return;
    const int nt = min(TP, nlast - t0), ks = hd + 4, h4 = hd / 4, n_heads = gridDim.x * group;
    float *kt = at_smem, *qs = at_smem + TP * ks;   // K tile [TP][ks]; queries [QB][group][hd]
    for (int e = tid; e < nt * h4; e += AT_THREADS) {
        const int r = e / h4, c = e - r * h4;
        *(float4 *)(kt + r * ks + 4 * c) =
            Kv4<KT>::wide(Kv4<KT>::load(kv.k, (size_t)(t0 + r) * kv_dim + (size_t)g * hd + 4 * c));
    }
    const int t = tid % TP, p = t0 + t;   // this thread's position (absolute: no window)
    const size_t qstride = (size_t)group * hd;   // floats between two tokens' queries in LDS
    for (int zb = 0; zb < zn; zb += QB) {
        const int qn = min(QB, zn - zb), gh4 = group * h4;
        __syncthreads();   // the last queries are read
        for (int e = tid; e < qn * gh4; e += AT_THREADS) {
            const int zz = e / gh4, r = e - zz * gh4;
            ((float4 *)qs)[e] = ((const float4 *)(q + (size_t)(z0 + zb + zz) * n_heads * hd + (size_t)g * group * hd))[r];
        }
        __syncthreads();
        if (t >= nt) continue;
        const float *kr = kt + t * ks;
        for (int j = tid / TP; j < group; j += AT_THREADS / TP) {
            // tokens zb + u, u < QB (slots past qn read an earlier block's
            // queries and are not stored)
            const float *qh = qs + (size_t)j * hd;
            float acc[QB];
#pragma unroll
            for (int u = 0; u < QB; u++) acc[u] = 0.0f;
#pragma unroll 2
            for (int i = 0; i < hd; i += 4) {
                const float4 b = *(const float4 *)(kr + i);
#pragma unroll
                for (int u = 0; u < QB; u++) {
                    const float4 a = *(const float4 *)(qh + u * qstride + i);
                    acc[u] = kr_fadd(acc[u], kr_fmul(a.x, b.x));
                    acc[u] = kr_fadd(acc[u], kr_fmul(a.y, b.y));
                    acc[u] = kr_fadd(acc[u], kr_fmul(a.z, b.z));
                    acc[u] = kr_fadd(acc[u], kr_fmul(a.w, b.w));
                }
            }
#pragma unroll
            for (int u = 0; u < QB; u++) {
                const int z = z0 + zb + u;
                if (u < qn && p <= pos0 + z)
                    att[((size_t)z * n_heads + (size_t)g * group + j) * max_seq + p] = kr_fmul(acc[u], scale);
            }
        }
    }
}

// Batched (prefill) scores without a window for heads of HD = 64 or 128
// dims, blocked in registers: the rows (token z, query head j) of KV head g,
// numbered z * group + j, go to workgroups RB_R at a time, each over a chunk
// of RB_PC tiles of RB_T positions. The workgroup stages its rows' queries
// in LDS once and each K tile in turn (F16 rows widened exactly), rows HD + 4
// floats apart; lane (row group rg, position group pg) owns the scores of rows
// 4 rg .. 4 rg + 3 at positions pg + 16 k (k < 4): per 4 dims it reads 4 query
// and 4 K 16-byte values, which feed 64 multiplies and 64 adds, each of its
// 16 sums s = sum_i q_i k_i in index order, then * scale, as in the per-token
// kernel. A row stores only the positions its token attends. The next tile's
// loads are in flight while a tile is summed.
constexpr int RB_R = 64, RB_T = 64;   // rows of a register-blocked workgroup; positions of its tiles
constexpr int RB_PC = 8;             // K tiles per scores workgroup
// the register-blocked kernels take 64- and 128-dim heads whose rows fill at
// least 512 workgroups (two a CU): a 511-token prompt over 2 KV heads of 7
// query heads gives 112, and there the per-token-block kernels measured twice
// as fast (scores 45.6 against 21.6 us a layer, mix 51.2 against 28.5)
static int g_rb_min_wg = 512;
static bool rb_shape(int hd, int ntok, int group, int n_kv) {
    return (hd == 64 || hd == 128) && (long)n_kv * ((ntok * group + RB_R - 1) / RB_R) >= g_rb_min_wg;
}
constexpr int RB_NT128 = 512;        // threads of the 128-dim heads' workgroups (4 outputs' rows a lane, LDS for 2
                                     // workgroups a CU: 4 waves a SIMD; 256 threads gave 2 and measured the same)
template <int HD, int KT, int NT>
__global__ void __launch_bounds__(NT) k_attn_scores_rb(float *att, const float *q, const KvView kv, int group,
                                                       int kv_dim, int max_seq, float scale, const int *pos_p,
                                                       int ntok) {
    constexpr int S = HD + 4;                     // LDS row stride (floats)
    constexpr int NPG = NT / 16, PPL = RB_T / NPG;   // position groups; positions a lane (pg + NPG k)
    constexpr int NL = RB_T * HD / 4 / NT;        // 4-element K loads a thread stages per tile
    constexpr int NQL = RB_R * HD / 4 / NT;       // query float4 a thread stages
    __shared__ __align__(16) float qs[RB_R * S];
    __shared__ __align__(16) float ks[RB_T * S];
    const int g = blockIdx.x, tid = threadIdx.x, pg = tid % NPG, rg = tid / NPG;
    const int nrow = ntok * group, R0 = blockIdx.y * RB_R;
    const int pos0 = *pos_p, n_heads = gridDim.x * group;
    const int nlast = pos0 + (min(R0 + RB_R, nrow) - 1) / group + 1;   // positions the block's last row attends
    const int p0 = blockIdx.z * RB_PC * RB_T;
    if (p0 >= nlast) return;
    const int ntl = min(RB_PC, (nlast - p0 + RB_T - 1) / RB_T);
#pragma unroll
    for (int u = 0; u < NQL; u++) {
        const int e = tid + NT * u, rr = e / (HD / 4), c4 = e % (HD / 4);
        const int R = min(R0 + rr, nrow - 1), z = R / group, j = R - z * group;
        *(float4 *)(qs + rr * S + 4 * c4) = *(const float4 *)(q + ((size_t)z * n_heads + (size_t)g * group + j) * HD + 4 * c4);
    }
    typename Kv4<KT>::T kr[NL];
    auto load = [&](int t0) {
#pragma unroll
        for (int u = 0; u < NL; u++) {
            const int e = tid + NT * u, p = e / (HD / 4), c4 = e % (HD / 4);
            kr[u] = Kv4<KT>::load(kv.k, (size_t)min(t0 + p, nlast - 1) * kv_dim + (size_t)g * HD + 4 * c4);
        }
    };
    int zr[4];   // the tokens of the lane's rows (past the last row: -1)
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int R = R0 + 4 * rg + r;
        zr[r] = R < nrow ? R / group : -1;
    }
    load(p0);
    for (int ti = 0; ti < ntl; ti++) {
        const int t0 = p0 + ti * RB_T;
        __syncthreads();   // the last tile is read
#pragma unroll
        for (int u = 0; u < NL; u++) {
            const int e = tid + NT * u, p = e / (HD / 4), c4 = e % (HD / 4);
            *(float4 *)(ks + p * S + 4 * c4) = Kv4<KT>::wide(kr[u]);
        }
        __syncthreads();
        if (ti + 1 < ntl) load(t0 + RB_T);
        float acc[4][PPL];
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int k = 0; k < PPL; k++) acc[r][k] = 0.0f;
        const float *qp = qs + 4 * rg * S, *kp = ks + pg * S;
#pragma unroll 4
        for (int i = 0; i < HD; i += 4) {
            float4 a[4], b[PPL];
#pragma unroll
            for (int r = 0; r < 4; r++) a[r] = *(const float4 *)(qp + r * S + i);
#pragma unroll
            for (int k = 0; k < PPL; k++) b[k] = *(const float4 *)(kp + NPG * k * S + i);
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int k = 0; k < PPL; k++) acc[r][k] = kr_fadd(acc[r][k], kr_fmul(a[r].x, b[k].x));
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int k = 0; k < PPL; k++) acc[r][k] = kr_fadd(acc[r][k], kr_fmul(a[r].y, b[k].y));
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int k = 0; k < PPL; k++) acc[r][k] = kr_fadd(acc[r][k], kr_fmul(a[r].z, b[k].z));
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int k = 0; k < PPL; k++) acc[r][k] = kr_fadd(acc[r][k], kr_fmul(a[r].w, b[k].w));
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            if (zr[r] < 0) continue;
            const int R = R0 + 4 * rg + r, j = R - zr[r] * group;
            float *dst = att + ((size_t)zr[r] * n_heads + (size_t)g * group + j) * max_seq;
#pragma unroll
            for (int k = 0; k < PPL; k++) {
                const int p = t0 + pg + NPG * k;
                if (p <= pos0 + zr[r]) dst[p] = kr_fmul(acc[r][k], scale);
            }
        }
    }
}

template <int KT, int TT>
__global__ void __launch_bounds__(AT_THREADS) k_attn_scores_kv(float *att, const float *q, const KvView kv, int group,
                                                               int hd, int kv_dim, int max_seq, int window, float scale,
                                                               const int *pos_p) {
    attn_scores<KT, TT>(att, q, kv, group, hd, kv_dim, max_seq, window, scale, pos_p);
}

// One query head of hd floats as the Q8 rule does it for the score
// (ops/ops.c:81-96): the max |x| from 0, one scale for the head, each value
// trunc(x * 127 / max + copysign(0.5, x)); a head of zeros (max below the
// rule's tiny) has scale 0 and zero quants. One wave; lane 0 writes the scale.
__device__ __forceinline__ void q8_head(const float *x, int hd, int8_t *dst, float *dd, int lane) {
    float m = 0.0f;
    for (int i = lane; i < hd; i += 64) m = fmaxf(m, fabsf(x[i]));
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    const bool zero = m < KR_QUANT_TINY;
    const float id = zero ? 0.0f : kr_fdiv(127.0f, m);
    for (int i = lane; i < hd; i += 64) dst[i] = zero ? (int8_t)0 : (int8_t)kr_q8_elem(x[i], id);
    if (lane == 0) *dd = zero ? 0.0f : kr_fdiv(m, 127.0f);
}

// Scores over the Q8 cache (ops/ops.c:171-173, k_scalar.c:137-146): each query
// head of the group quantized with one scale (ops/ops.c:81-96; every
// workgroup quantizes its group's heads itself, the same bits), then per
// position the exact int32 dot of the int8 rows (v_dot4) and
// ((float)sum * (dq * scale)) * dk_t. K rows are staged in LDS with a stride
// of hd + 4 bytes (33 words for hd 128: the lanes of a wave spread over the
// banks).
__global__ void __launch_bounds__(AT_THREADS) k_attn_scores_q8(float *att, const float *q, const KvView kv, int group,
                                                               int hd, int kv_dim, int max_seq, int window, float scale,
                                                               const int *pos_p) {
    extern __shared__ __align__(16) float at_smem[];
    int first, n;
    attn_range(pos_p, window, &first, &n);
    att += (size_t)blockIdx.z * gridDim.x * group * max_seq;
    q += (size_t)blockIdx.z * gridDim.x * group * hd;
    const int g = blockIdx.x, t0 = blockIdx.y * AT_T, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (t0 >= n) return;
    const int nt = min(AT_T, n - t0), ks = hd + 4;
    float *qd = at_smem;                            // [16] query scales
    int8_t *qs = (int8_t *)(at_smem + 16);          // [group][hd]
    int8_t *kt = qs + (group * hd + 15) / 16 * 16;  // [AT_T][ks]
    for (int j = wave; j < group; j += AT_THREADS / 64) q8_head(q + (size_t)(g * group + j) * hd, hd, qs + j * hd, qd + j, lane);
    // store_kv folded into decode (model/transformer.c:198-203): the tile
    // holding the current position quantizes its KV head's K row (wave 0,
    // straight into the tile as well) and V row (wave 1) into the cache
    __shared__ float fresh_dk;
    const bool fresh = kv.ks && t0 + nt == n;
    if (fresh && wave < 2) {
        const float *x = (wave ? kv.vs : kv.ks) + (size_t)g * hd;
        float m = 0.0f;
        for (int i = lane; i < hd; i += 64) m = fmaxf(m, fabsf(x[i]));
        for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        const bool zero = m < KR_QUANT_TINY;
        const float id = zero ? 0.0f : kr_fdiv(127.0f, m), d = zero ? 0.0f : kr_fdiv(m, 127.0f);
        const size_t row = (size_t)(first + n - 1);
        int8_t *dst = (int8_t *)(wave ? kv.v : kv.k) + row * kv_dim + (size_t)g * hd;
        for (int i = lane; i < hd; i += 64) {
            const int8_t qv = zero ? (int8_t)0 : (int8_t)kr_q8_elem(x[i], id);
            dst[i] = qv;
            if (wave == 0) kt[(nt - 1) * ks + i] = qv;
        }
        if (lane == 0) {
            ((float *)(wave ? kv.vd : kv.kd))[row * kv.n_kv + g] = d;
            if (wave == 0) fresh_dk = d;
        }
    }
    const int h4 = hd / 4;
    for (int e = tid; e < nt * h4; e += AT_THREADS) {
        const int r = e / h4, c = e - r * h4;
        if (fresh && r == nt - 1) continue;   // written above
        *(int *)(kt + r * ks + 4 * c) =
            *(const int *)((const int8_t *)kv.k + (size_t)(first + t0 + r) * kv_dim + (size_t)g * hd + 4 * c);
    }
    __syncthreads();
    const int t = tid % AT_T;
    if (t >= nt) return;
    const int8_t *kr = kt + t * ks;
    const float dk = fresh && t == nt - 1 ? fresh_dk : kv.kd[(size_t)(first + t0 + t) * kv.n_kv + g];
    for (int j = tid / AT_T; j < group; j += AT_THREADS / AT_T) {
        const int8_t *qh = qs + j * hd;
        int sum = 0;
        for (int i = 0; i < hd; i += 4) sum = kr_dot4(*(const int *)(qh + i), *(const int *)(kr + i), sum);
        const float c = kr_fmul(qd[j], scale);
        att[(size_t)(g * group + j) * max_seq + t0 + t] = kr_fmul(kr_fmul((float)sum, c), dk);
    }
}

// Batched (prefill) scores over the Q8 cache without a window, a block of
// AT_TB tokens at a time: the int8 K tile of AT_T positions and its row
// scales are staged once for the block; then, QB tokens at a time, the
// workgroup quantizes those tokens' query heads of its group into LDS
// (q8_head: the per-token kernel's bits) and thread (position t, head j)
// runs the QB exact int32 dots against its K row in one pass, each finished
// as in the per-token kernel: ((float)sum * (dq * scale)) * dk_t.
template <int QB>
__global__ void __launch_bounds__(AT_THREADS) k_attn_scores_blk_q8(float *att, const float *q, const KvView kv,
                                                                   int group, int hd, int kv_dim, int max_seq,
                                                                   float scale, const int *pos_p, int ntok) {
    extern __shared__ __align__(16) float at_smem[];
    const int g = blockIdx.x, t0 = blockIdx.y * AT_T, z0 = blockIdx.z * AT_TB, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int pos0 = *pos_p, zn = min(AT_TB, ntok - z0);
    const int nlast = pos0 + z0 + zn;   // positions the block's last token attends
    if (t0 >= nlast) return;
    const int nt = min(AT_T, nlast - t0), ks = hd + 4, n_heads = gridDim.x * group, h4 = hd / 4;
    float *dks = at_smem;                                   // [AT_T] K row scales
    float *qd = dks + AT_T;                                 // [QB][group] query head scales
    int8_t *kt = (int8_t *)(qd + (QB * group + 3) / 4 * 4);   // [AT_T][ks]
    int8_t *qs = kt + (AT_T * ks + 15) / 16 * 16;          // [QB][group][hd]
    for (int e = tid; e < nt * h4; e += AT_THREADS) {
        const int r = e / h4, c = e - r * h4;
        *(int *)(kt + r * ks + 4 * c) =
            *(const int *)((const int8_t *)kv.k + (size_t)(t0 + r) * kv_dim + (size_t)g * hd + 4 * c);
    }
    for (int r = tid; r < nt; r += AT_THREADS) dks[r] = kv.kd[(size_t)(t0 + r) * kv.n_kv + g];
    const int t = tid % AT_T, p = t0 + t;   // this thread's position (absolute: no window)
    for (int zb = 0; zb < zn; zb += QB) {
        const int qn = min(QB, zn - zb);
        __syncthreads();   // the last queries are read
        for (int h = wave; h < qn * group; h += AT_THREADS / 64) {
            const int zz = h / group, jj = h - zz * group;
            q8_head(q + ((size_t)(z0 + zb + zz) * n_heads + (size_t)g * group + jj) * hd, hd, qs + (size_t)h * hd,
                    qd + h, lane);
        }
        __syncthreads();
        if (t >= nt) continue;
        const int8_t *kr = kt + t * ks;
        const float dk = dks[t];
        for (int j = tid / AT_T; j < group; j += AT_THREADS / AT_T) {
            // tokens zb + u, u < QB (slots past qn hold an earlier block's
            // queries and are not stored)
            int acc[QB];
#pragma unroll
            for (int u = 0; u < QB; u++) acc[u] = 0;
            for (int i = 0; i < hd; i += 4) {
                const int k4 = *(const int *)(kr + i);
#pragma unroll
                for (int u = 0; u < QB; u++) acc[u] = kr_dot4(*(const int *)(qs + ((size_t)u * group + j) * hd + i), k4, acc[u]);
            }
#pragma unroll
            for (int u = 0; u < QB; u++) {
                const int z = z0 + zb + u;
                if (u < qn && p <= pos0 + z) {
                    const float c = kr_fmul(qd[u * group + j], scale);
                    att[((size_t)z * n_heads + (size_t)g * group + j) * max_seq + p] = kr_fmul(kr_fmul((float)acc[u], c), dk);
                }
            }
        }
    }
}

// Softmax of one head's n scores in place (k_scalar.c:66-77): the max, the
// exponentials x - max, their ordered sum (kr_spec_sum: the sequential
// loop's bits), x * (1 / sum). Up to AT_CHUNK scores stay in registers
// between one batched read and one write (every load issued at once, from an
// index clamped into the row); longer rows go AT_CHUNK at a time through LDS,
// the sum continuing from chunk to chunk.
// NT threads a row, CH scores of it in registers at once: the decode launch
// spreads its loads, exponentials and stores over 1024 threads; prefill rows
// of up to 4096 scores take 256 (the ordered sum needs 4 waves, and a small
// workgroup lets 8 rows share a CU's LDS and SIMDs).
constexpr int SMX_THREADS = 1024, AT_CHUNK = 8192;   // the decode launch
template <int NT, int CH, bool LEAN = false>
__global__ void __launch_bounds__(NT) k_attn_softmax(float *att, int max_seq, int window, const int *pos_p) {
    constexpr int SMX_THREADS = NT, AT_CHUNK = CH, AT_V = CH / NT;
    __shared__ __align__(16) float es[sc_terms_cap(AT_CHUNK)];
    __shared__ __align__(16) unsigned char scr[sc_lds_bytes(AT_CHUNK, SMX_THREADS)];
    __shared__ float red[SMX_THREADS / 64];
    __shared__ uint64_t xtab[32];   // expf's table
    int first, n;
    attn_range(pos_p, window, &first, &n);
    float *a = att + ((size_t)blockIdx.z * gridDim.x + blockIdx.x) * max_seq;
    const int tid = threadIdx.x;
    if (tid < 32) xtab[tid] = kr_exp2_tab[tid];
    const bool fits = n <= AT_CHUNK;
    float v[AT_V];
    float m = -INFINITY;
    if (fits) {
        // slots past the row's end are skipped (a uniform test); the last
        // live slot's index is clamped: repeats change no max
#pragma unroll
        for (int k = 0; k < AT_V; k++)
            if (k * SMX_THREADS < n) v[k] = a[min(k * SMX_THREADS + tid, n - 1)];
#pragma unroll
        for (int k = 0; k < AT_V; k++)
            if (k * SMX_THREADS < n) m = fmaxf(m, v[k]);
    } else {
        for (int t = tid; t < n; t += SMX_THREADS) m = fmaxf(m, a[t]);
    }
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    float mx = red[0];
    for (int k = 1; k < SMX_THREADS / 64; k++) mx = fmaxf(mx, red[k]);
    if (mx == -INFINITY) {   // every score -inf: the scalar loop's 1/n
        for (int t = tid; t < n; t += SMX_THREADS) a[t] = kr_fdiv(1.0f, (float)n);
        return;
    }
    if (fits) {
        const int sh = sc_log_len(n);
#pragma unroll
        for (int k = 0; k < AT_V; k++) {
            if (k * SMX_THREADS >= n) break;   // the rest of the slots are clamped repeats
            const int t = k * SMX_THREADS + tid;
            v[k] = kr_expf_tab(kr_fsub(v[k], mx), xtab);
            if (t < n) es[sc_at(t, sh)] = v[k];
        }
        __syncthreads();
        const float inv = kr_fdiv(1.0f, kr_spec_sum<SMX_THREADS, false, false, LEAN>(es, n, scr));
#pragma unroll
        for (int k = 0; k < AT_V; k++) {
            if (k * SMX_THREADS >= n) break;
            const int t = k * SMX_THREADS + tid;
            if (t < n) a[t] = kr_fmul(v[k], inv);
        }
        return;
    }
    float sum = 0.0f;
    for (int c0 = 0; c0 < n; c0 += AT_CHUNK) {
        const int cn = min(AT_CHUNK, n - c0), sh = sc_log_len(cn);
        for (int t = tid; t < cn; t += SMX_THREADS) {
            const float e = kr_expf_tab(kr_fsub(a[c0 + t], mx), xtab);
            es[sc_at(t, sh)] = e;
            a[c0 + t] = e;
        }
        __syncthreads();
        sum = kr_spec_sum<SMX_THREADS, false, false, LEAN>(es, cn, scr, sum);   // ends with a barrier: es is free again
    }
    const float inv = kr_fdiv(1.0f, sum);
    for (int t = tid; t < n; t += SMX_THREADS) a[t] = kr_fmul(a[t], inv);
}

// Batched (prefill) softmax, one row per wave and RW rows per workgroup:
// rows r = token * n_heads + head of up to SM_WN = 4096 entries (the
// single-wave ordered sum's limit). Per row, as k_attn_softmax: the max,
// the exponentials x - max, their ordered sum (kr_spec_sum in single-wave
// mode), x * (1 / sum); an all -inf row becomes 1/n. The per-row kernel keeps
// three of its four waves idle in the ordered sum of rows this short; here
// every wave sums its own row. SV: register slots per lane (rows of at most
// 64 SV entries). The launch takes rows up to 2048 (32 slots: fewer
// registers, more rows in flight); longer rows measured faster on the
// per-row kernel with 256 threads (64 slots a lane here leave each CU two
// waves a SIMD, its LDS then holding 8 rows' terms).
constexpr int SM_WN = SC_CPW << SC_LOG_LMIN, SM_V = SM_WN / 64;
template <int RW, int SV = SM_V>
__global__ void __launch_bounds__(64 * RW) k_attn_softmax_rows(float *att, int n_heads, int max_seq, int window,
                                                               const int *pos_p, int nrows, int terms_cap,
                                                               int scr_bytes) {
    extern __shared__ __align__(16) unsigned char sm_lds[];
    __shared__ uint64_t xtab[32];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (threadIdx.x < 32) xtab[threadIdx.x] = kr_exp2_tab[threadIdx.x];
    __syncthreads();
    const int r = blockIdx.x * RW + wave;
    if (r >= nrows) return;
    const int z = r / n_heads, pos = *pos_p + z;
    const int first = window && pos >= window ? pos + 1 - window : 0, n = pos + 1 - first;
    float *a = att + (size_t)r * max_seq;
    float *es = (float *)(sm_lds + (size_t)wave * (4 * terms_cap + scr_bytes));
    unsigned char *scr = (unsigned char *)(es + terms_cap);
    float v[SV];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < SV; k++)
        if (k * 64 < n) v[k] = a[min(k * 64 + lane, n - 1)];   // the last live slot clamped: repeats change no max
#pragma unroll
    for (int k = 0; k < SV; k++)
        if (k * 64 < n) m = fmaxf(m, v[k]);
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if (m == -INFINITY) {   // every score -inf: the scalar loop's 1/n
        for (int t = lane; t < n; t += 64) a[t] = kr_fdiv(1.0f, (float)n);
        return;
    }
    const int sh = sc_log_len(n);
#pragma unroll
    for (int k = 0; k < SV; k++) {
        if (k * 64 >= n) break;
        const int t = k * 64 + lane;
        v[k] = kr_expf_tab(kr_fsub(v[k], m), xtab);
        if (t < n) es[sc_at(t, sh)] = v[k];
    }
    kr_wave_sync();
    const float inv = kr_fdiv(1.0f, kr_spec_sum<64, false, true>(es, n, scr));
#pragma unroll
    for (int k = 0; k < SV; k++) {
        if (k * 64 >= n) break;
        const int t = k * 64 + lane;
        if (t < n) a[t] = kr_fmul(v[k], inv);
    }
}

// out for one KV head's query heads and DW of their dims: lane = (head j of
// the group, dim d), DW = 64 / (group rounded up to a power of two). Each
// lane runs its ordered chain o += a_t * v_t,d (k_scalar.c:119-122). ao is
// written as floats (its quantization happens where it is consumed).
//
// The chain (one dependent add per position) is the bound, so the workgroup
// splits the work by role and keeps the adding wave free of everything else.
// Wave 0 only adds. MX_P producer waves load V and the weights, form the
// products a_t * v_t,d (each the rounded product, as in the scalar loop) and
// hand them over through a ring of three LDS tiles of MX_T positions, laid out
// [lane][position] so that one 16-byte read feeds 4 adds. Producer p owns
// positions [p MX_TH, (p + 1) MX_TH) of every tile and loads them MX_D tiles
// ahead into registers: a lane holds 4 dims of V at one position and the
// weights of every head at that position, and writes its products straight
// into the adder's layout (4-byte writes: the transpose costs no LDS reads).
// LDS bandwidth is what the roles share, so each product crosses LDS once each
// way. One barrier per step hands tiles over: producers write tile s in step
// s; the adder reads tile s into registers in step s + 1 and adds it in step
// s + 2, so no add waits on an LDS read.
// Three producers and the adder: one wave per SIMD of the CU (a fourth
// producer would share the adder's SIMD and slow its chain). The adder, not
// the producers, is the slower side: a tile's 96 dependent adds and its 24
// reads take about 800 cycles, the producers' products and loads 550-700.
// Rows of MX_TS = 100 floats put a 16-lane group's 16-byte reads on 64
// distinct banks.
constexpr int MX_P = 3, MX_TH = 32;                  // producers; their positions per tile
constexpr int MX_T = MX_P * MX_TH, MX_TS = MX_T + 4;   // positions per tile; padded product row

__device__ __forceinline__ void kr_lds_order() { asm volatile("" ::: "memory"); }

// Slot k of a producer lane: position r of the producer's MX_TH positions and
// first dim c of its 4 dims. Lanes 0-31 and 32-63 take neighbouring dim
// quads of the same 32 positions, so the 32 stores of a half-wave into the
// adder's rows (MX_TS floats apart: 4 quads = 16 banks) hit 32 distinct banks.
static_assert(MX_TH == 32, "the slot map covers 32 positions a slot");
template <int DW>
__device__ __forceinline__ void mx_slot(int k, int lane, int &r, int &c) {
    if (DW >= 8) {
        r = lane & 31;
        c = 4 * (2 * k + (lane >> 5));
    } else {   // one dim quad: lanes 32-63 hold no slot (r >= MX_TH)
        r = lane;
        c = 0;
    }
}

template <int DW, int KT>
__device__ __forceinline__ void attn_mix(float *ao, const float *att, const KvView kv, int group, int hd, int kv_dim,
                                         int max_seq, int window, const int *pos_p) {
    constexpr int GP = 64 / DW;                        // head slots
    constexpr int NV = (MX_TH * DW / 4 + 63) / 64;     // 4-element groups of V per producer lane per tile
    constexpr int ND = KT == KV_Q8 ? NV : 0;           // V row scales per producer lane per tile
    constexpr int PT = Kv4<KT>::REGS * NV + NV * GP + ND;   // registers per tile: V, the weights, the scales
    constexpr int LT = NV + NV * GP + ND;              // loads per tile
    // tiles in flight: within 128 registers and within the 63 loads the wait
    // counter can track (past that every wait would drain it)
    constexpr int DR = 128 / PT < 60 / LT ? 128 / PT : 60 / LT;
    constexpr int MX_D = DR > 8 ? 8 : DR < 2 ? 2 : DR;
    __shared__ __align__(16) float prod[4][64 * MX_TS];   // the ring, and a sink for steps past the end
    int first, n;
    attn_range(pos_p, window, &first, &n);
    const int g = blockIdx.x, c0 = blockIdx.y * DW, lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane / DW, d = lane % DW;
    const int ntiles = (n + MX_T - 1) / MX_T;
    if (c0 >= hd) {
        // a helper workgroup (grid rows past the head's dim chunks, decode
        // only): it reads one 2-byte word of every 128-byte line of KV head
        // g's V rows and of its query heads' weight rows, earliest positions
        // first, so that they wait in the L2 of this XCD (workgroups are
        // dealt to the 8 XCDs by linear id, so with 8 KV heads per launch
        // row all of head g's workgroups share one) before the producers ask
        constexpr int eb = KT == KV_F32 ? 4 : KT == KV_F16 ? 2 : 1;
        const int lpr = (hd * eb + 127) / 128, nhelp = gridDim.y - (hd + DW - 1) / DW;
        const int hi = (blockIdx.y - (hd + DW - 1) / DW) * (64 * (1 + MX_P)) + threadIdx.x, hn = nhelp * 64 * (1 + MX_P);
        const unsigned char *vb = (const unsigned char *)kv.v + ((size_t)first * kv_dim + (size_t)g * hd) * eb;
        const float *ab = att + (size_t)g * group * max_seq;
        const int vl = n * lpr, al = (n * 4 + 127) / 128;   // V lines; weight-row lines per head
        int sink = 0;
        for (int i = hi; i < vl + group * al; i += hn) {
            if (i < vl) {
                const int t = i / lpr;
                sink ^= *(const unsigned short *)(vb + (size_t)t * kv_dim * eb + (size_t)(i - t * lpr) * 128);
            } else {
                const int h = (i - vl) / al;
                sink ^= *(const unsigned short *)((const unsigned char *)(ab + (size_t)h * max_seq) + (size_t)(i - vl - h * al) * 128);
            }
        }
        if (sink == 0x5bd1 && max_seq < 0) ao[0] = 0.0f;   // keeps the reads (never true)
        return;
    }
    // Steps with a barrier: one per tile the producers write, rounded up to
    // MX_S (every wave runs as many barriers); the adder's last two steps
    // (the last tile's read, the last adds) follow without one. The
    // producers' loop runs in groups of MX_D steps (one per register slot)
    // and may stop after a third (or half) of a group: whole groups ran up
    // to 4 empty steps past the end (the 0.5B shape at 550 positions: 12
    // steps for 8); a test after every step measured no better than one per
    // third.
    constexpr int MX_S = MX_D % 3 == 0 ? MX_D / 3 : MX_D % 2 == 0 ? MX_D / 2 : MX_D;
    const int steps = (ntiles + MX_S - 1) / MX_S * MX_S;
    const size_t q_dim = (size_t)gridDim.x * group * hd;

    if (wave == 0) {
        // the adder: in step s it reads all of tile s - 1 into registers
        // (finished a step earlier) while it adds tile s - 2 from the
        // registers read in step s - 1, so every LDS read has a whole tile
        // of adds to arrive in
        float o = 0.0f;
        auto step = [&](int s, float4 *cur, float4 *nxt, bool bar = true) {
            if (s - 1 >= 0 && s - 1 < ntiles) {
                const float *P = prod[(s - 1) % 3] + lane * MX_TS;
#pragma unroll
                for (int i = 0; i < MX_T / 4; i++) nxt[i] = *(const float4 *)(P + 4 * i);
            }
            const int tile = s - 2;
            if (tile >= 0 && tile < ntiles) {
                const int nt = min(MX_T, n - tile * MX_T);
                if (nt == MX_T) {
#pragma unroll
                    for (int i = 0; i < MX_T / 4; i++) {
                        o = kr_fadd(o, cur[i].x);
                        o = kr_fadd(o, cur[i].y);
                        o = kr_fadd(o, cur[i].z);
                        o = kr_fadd(o, cur[i].w);
                    }
                } else {   // the last, partial tile: only its live steps (a zero would turn -0 to +0)
                    const float *P = prod[tile % 3] + lane * MX_TS;
                    for (int r = 0; r < nt; r++) o = kr_fadd(o, P[r]);
                }
            }
            if (bar) {
                kr_lds_order();
                __syncthreads();
            }
        };
        float4 ta[MX_T / 4], tb[MX_T / 4];
        for (int s = 0; s < steps; s += 2) {
            step(s, ta, tb);
            if (s + 1 < steps) step(s + 1, tb, ta);
        }
        for (int s = steps; s < steps + 2; s++) {   // the producers are done: no barrier
            if (s & 1) step(s, tb, ta, false);
            else step(s, ta, tb, false);
        }
        if (j < group && d < min(DW, hd - c0)) ao[blockIdx.z * q_dim + (size_t)(g * group + j) * hd + c0 + d] = o;
        return;
    }

    // producer p: lane slot k holds V dims c..c+3 at position r of its half
    // tile, and the weights of heads 0..GP-1 at that position
    const int p = wave - 1;
    const int cw = min(DW, hd - c0);   // valid dims of the chunk (a multiple of 4)
    const size_t vb = (size_t)first * kv_dim + (size_t)g * hd + c0;   // element offset of V row `first`
    const float *abase = att + ((size_t)blockIdx.z * gridDim.x * group + (size_t)g * group) * max_seq;
    // Every load is unconditional from an address clamped into the live
    // range (position n - 1, the chunk's last 4 elements, the group's last
    // head, the row's last element): values loaded for positions >= n, dims
    // >= cw or heads >= group only feed products that are never added or
    // stored, and a branch-free loop keeps the loads of MX_D tiles in flight.
    using VT = typename Kv4<KT>::T;
    VT rv[MX_D][NV];
    float ra[MX_D][NV][GP];
    float rd[MX_D][ND > 0 ? ND : 1];   // Q8: the V rows' scales
    auto load = [&](int tile, VT *v, float (*a)[GP], float *dv) {
        const int t0 = min(tile, ntiles - 1) * MX_T + p * MX_TH;
#pragma unroll
        for (int k = 0; k < NV; k++) {
            int r, c;
            mx_slot<DW>(k, lane, r, c);
            r = min(r, MX_TH - 1);
            c = min(c, cw - 4);
            const int t = min(t0 + r, n - 1);
            v[k] = Kv4<KT>::load(kv.v, vb + (size_t)t * kv_dim + c);
            if (KT == KV_Q8) dv[k] = kv.vd[(size_t)(first + t) * kv.n_kv + g];
            const int q = min(t0 + r, max_seq - 1);
#pragma unroll
            for (int jj = 0; jj < GP; jj++) a[k][jj] = abase[(size_t)min(jj, group - 1) * max_seq + q];
        }
    };
    auto products = [&](int tile, const VT *v, const float (*a)[GP], const float *dv) {
        float *P = prod[tile < ntiles ? tile % 3 : 3] + p * MX_TH;
#pragma unroll
        for (int k = 0; k < NV; k++) {
            int r, c;
            mx_slot<DW>(k, lane, r, c);
            if (r < MX_TH) {
                const float4 x = Kv4<KT>::wide(v[k]);
#pragma unroll
                for (int jj = 0; jj < GP; jj++) {
                    // Q8: the weight a_t * dv_t, then its products (k_scalar.c:151-153)
                    const float w = KT == KV_Q8 ? kr_fmul(a[k][jj], dv[k]) : a[k][jj];
                    float *o = P + (jj * DW + c) * MX_TS + r;
                    o[0] = kr_fmul(w, x.x);
                    o[MX_TS] = kr_fmul(w, x.y);
                    o[2 * MX_TS] = kr_fmul(w, x.z);
                    o[3 * MX_TS] = kr_fmul(w, x.w);
                }
            }
        }
        kr_lds_order();
    };
    // in slot order (the loop's waits count on slot 0 being the oldest)
#pragma unroll
    for (int u = 0; u < MX_D; u++) {
        load(u, rv[u], ra[u], rd[u]);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int s0 = 0; s0 < steps; s0 += MX_D) {
#pragma unroll
        for (int u = 0; u < MX_D; u++) {
            if (u > 0 && u % MX_S == 0 && s0 + u >= steps) break;   // a part group ends the loop
            const int s = s0 + u;   // tile s sits in slot u
            // fenced for the scheduler: a step's products wait on its own
            // slot's loads only
            __builtin_amdgcn_sched_barrier(0);
            products(s, rv[u], ra[u], rd[u]);   // past the end: into the sink, unread
            load(s + MX_D, rv[u], ra[u], rd[u]);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
        }
    }
}

template <int DW>
__global__ void __launch_bounds__(64 * (1 + MX_P)) k_attn_mix(float *ao, const float *att, const float *vc,
                                                              int group, int hd, int kv_dim, int max_seq, int window,
                                                              const int *pos_p) {
    const KvView kv = { nullptr, vc, nullptr, nullptr, 0 };
    attn_mix<DW, KV_F32>(ao, att, kv, group, hd, kv_dim, max_seq, window, pos_p);
}

template <int DW, int KT>
__global__ void __launch_bounds__(64 * (1 + MX_P)) k_attn_mix_kv(float *ao, const float *att, const KvView kv,
                                                                 int group, int hd, int kv_dim, int max_seq,
                                                                 int window, const int *pos_p) {
    attn_mix<DW, KT>(ao, att, kv, group, hd, kv_dim, max_seq, window, pos_p);
}

// The same for a batch of positions (prefill: one workgroup per position and
// head chunk, so throughput, not one chain's latency, is what counts), one wave
// per workgroup: lane = (head j of the group, dim d), DW = 64 / (group rounded up
// to a power of two). Each lane runs its ordered chain o += a_t * v_t,d
// (k_scalar.c:119-122). ao is written as floats (its quantization happens
// where it is consumed).
//
// The chain is the bound (one dependent add per position), so everything else
// is pipelined under it: tiles of MB_T positions of V and of the heads' weights
// are loaded MB_DEPTH tiles ahead into registers; tile t + 1 is staged into
// the other half of a double LDS buffer while tile t is read, V transposed
// ([dim][position]) so one 16-byte LDS read feeds 4 steps; the reads of each
// 16-step chunk are issued before the adds of the chunk before it. The
// workgroup is one wave, whose LDS operations execute in order, so LDS needs
// only compiler ordering (kr_lds_order), not barriers.
constexpr int MB_T = 64, MB_TS = MB_T + 4;   // positions per tile; padded LDS row

template <int DW, int KT>
__device__ __forceinline__ void attn_mix_batch(float *ao, const float *att, const KvView kv, int group, int hd,
                                               int kv_dim, int max_seq, int window, const int *pos_p) {
    constexpr int GP = 64 / DW;                    // head slots per wave
    constexpr int NV = MB_T * DW / 4 / 64;         // float4 of V per lane per tile
    constexpr int NA = (GP * MB_T / 4 + 63) / 64;  // float4 of weights per lane per tile
    constexpr int MB_DEPTH = NV + NA > 8 ? 2 : 4;  // tiles in flight (even: LDS halves alternate)
    __shared__ __align__(16) float vt[2][DW * MB_TS];
    constexpr int AW = GP * MB_T > NA * 256 ? GP * MB_T : NA * 256;   // padded: every lane stores
    __shared__ __align__(16) float aw[2][AW];
    int first, n;
    attn_range(pos_p, window, &first, &n);
    const int g = blockIdx.x, c0 = blockIdx.y * DW, lane = threadIdx.x;
    const int j = lane / DW, d = lane % DW;
    const size_t vb = (size_t)first * kv_dim + (size_t)g * hd + c0;   // element offset of V row `first`
    const size_t q_dim = (size_t)gridDim.x * group * hd;
    const float *abase = att + ((size_t)blockIdx.z * gridDim.x * group + (size_t)g * group) * max_seq;
    ao += blockIdx.z * q_dim;
    const int ntiles = (n + MB_T - 1) / MB_T;
    const int cw = min(DW, hd - c0);   // valid dims of the chunk (a multiple of 4)

    // Every load is unconditional from an address clamped into the live
    // range (position n - 1, the chunk's last float4, the group's last head,
    // the row's last float4): values loaded for positions >= n, dims >= cw or
    // heads >= group only feed lanes and steps that are never stored or run,
    // and a branch-free load stream lets the compiler's wait counts keep the
    // loads of MB_DEPTH tiles in flight together.
    using VT = typename Kv4<KT>::T;
    constexpr int ND = KT == KV_Q8 ? NA : 1;   // Q8: V row scales at the weights' positions
    VT rv[MB_DEPTH][NV];
    float4 ra[MB_DEPTH][NA], rd[MB_DEPTH][ND];
    auto load = [&](int tile, VT *v, float4 *a, float4 *dv) {
        const int t0 = min(tile, ntiles - 1) * MB_T;
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int e = (k * 64 + lane) * 4, r = e / DW, c = min(e % DW, cw - 4);   // position r, dims c..c+3
            v[k] = Kv4<KT>::load(kv.v, vb + (size_t)min(t0 + r, n - 1) * kv_dim + c);
        }
#pragma unroll
        for (int k = 0; k < NA; k++) {
            const int e = (k * 64 + lane) * 4, jj = min(e / MB_T, group - 1), r = e % MB_T;
            const float *src = abase + (size_t)jj * max_seq + min(t0 + r, max_seq - 4);
            a[k] = make_float4(src[0], src[1], src[2], src[3]);
            if (KT == KV_Q8) {
                const float *d = kv.vd + (size_t)first * kv.n_kv + g;
                dv[k] = make_float4(d[(size_t)min(t0 + r, n - 1) * kv.n_kv], d[(size_t)min(t0 + r + 1, n - 1) * kv.n_kv],
                                    d[(size_t)min(t0 + r + 2, n - 1) * kv.n_kv], d[(size_t)min(t0 + r + 3, n - 1) * kv.n_kv]);
            }
        }
    };
    auto stage = [&](int buf, int tile, const VT *v, const float4 *a, const float4 *dv) {
        float *V = vt[buf], *A = aw[buf];
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int e = (k * 64 + lane) * 4, r = e / DW, c = e % DW;
            const float4 x = Kv4<KT>::wide(v[k]);
            V[(c + 0) * MB_TS + r] = x.x;
            V[(c + 1) * MB_TS + r] = x.y;
            V[(c + 2) * MB_TS + r] = x.z;
            V[(c + 3) * MB_TS + r] = x.w;
        }
#pragma unroll
        for (int k = 0; k < NA; k++) {
            const int e = (k * 64 + lane) * 4, r = e % MB_T;
            // a float4 clamped back from the row's end holds position p at
            // element p - (max_seq - 4): shift it down to element p - p0
            const int sh = tile * MB_T + r - min(tile * MB_T + r, max_seq - 4);
            const float4 x = a[k];
            float4 y;
            y.x = sh == 0 ? x.x : sh == 1 ? x.y : sh == 2 ? x.z : x.w;
            y.y = sh == 0 ? x.y : sh == 1 ? x.z : x.w;
            y.z = sh == 0 ? x.z : x.w;
            y.w = x.w;
            if (KT == KV_Q8) {   // the weights a_t * dv_t (k_scalar.c:151)
                y.x = kr_fmul(y.x, dv[k].x);
                y.y = kr_fmul(y.y, dv[k].y);
                y.z = kr_fmul(y.z, dv[k].z);
                y.w = kr_fmul(y.w, dv[k].w);
            }
            *(float4 *)(A + e) = y;
        }
        kr_lds_order();
    };
    struct Chunk { float4 v[4], a[4]; };   // 16 steps of one lane
    auto read = [&](Chunk &c, int buf, int k) {
        const float *V = vt[buf] + d * MB_TS + 16 * k, *A = aw[buf] + j * MB_T + 16 * k;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            c.v[i] = *(const float4 *)(V + 4 * i);
            c.a[i] = *(const float4 *)(A + 4 * i);
        }
    };
    float o = 0.0f;
    auto chain = [&](const Chunk &c) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o = kr_fadd(o, kr_fmul(c.a[i].x, c.v[i].x));
            o = kr_fadd(o, kr_fmul(c.a[i].y, c.v[i].y));
            o = kr_fadd(o, kr_fmul(c.a[i].z, c.v[i].z));
            o = kr_fadd(o, kr_fmul(c.a[i].w, c.v[i].w));
        }
    };

#pragma unroll
    for (int s = 0; s < MB_DEPTH; s++) load(s, rv[s], ra[s], rd[s]);
    stage(0, 0, rv[0], ra[0], rd[0]);
    load(MB_DEPTH, rv[0], ra[0], rd[0]);
    Chunk c0r, c1r;
    read(c0r, 0, 0);
    // main loop: groups of MB_DEPTH full tiles; tile k0 + s sits in LDS half
    // s & 1 and its first chunk is in c0r when its step begins
    const int ngroups = n / (MB_T * MB_DEPTH);
    int k0 = 0;
    for (; k0 < ngroups * MB_DEPTH; k0 += MB_DEPTH) {
#pragma unroll
        for (int s = 0; s < MB_DEPTH; s++) {
            const int b = s & 1, nx = (s + 1) % MB_DEPTH;
            // phases fenced for the scheduler: a chunk's reads are issued
            // one phase before its products and adds, and the staging of
            // the next tile shares a phase with the first chunk's adds
            read(c1r, b, 1);
            __builtin_amdgcn_sched_barrier(0);
            chain(c0r);
            stage(b ^ 1, k0 + s + 1, rv[nx], ra[nx], rd[nx]);
            load(k0 + s + 1 + MB_DEPTH, rv[nx], ra[nx], rd[nx]);
            __builtin_amdgcn_sched_barrier(0);
            read(c0r, b, 2);
            __builtin_amdgcn_sched_barrier(0);
            chain(c1r);
            __builtin_amdgcn_sched_barrier(0);
            read(c1r, b, 3);
            __builtin_amdgcn_sched_barrier(0);
            chain(c0r);
            __builtin_amdgcn_sched_barrier(0);
            read(c0r, b ^ 1, 0);
            __builtin_amdgcn_sched_barrier(0);
            chain(c1r);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // the last tiles (at most MB_DEPTH; tile k0 is staged in half 0, tile
    // k0 + s is in rv[s]); the last may be partial, and only its live steps
    // run: a zero weight would turn -0 to +0
#pragma unroll
    for (int s = 0; s < MB_DEPTH; s++) {
        const int tile = k0 + s;
        if (tile < ntiles) {
            if (s > 0) stage(s & 1, tile, rv[s], ra[s], rd[s]);
            const int nt = min(MB_T, n - tile * MB_T);
            const float *V = vt[s & 1] + d * MB_TS, *A = aw[s & 1] + j * MB_T;
            for (int r = 0; r < nt; r++) o = kr_fadd(o, kr_fmul(A[r], V[r]));
            kr_lds_order();
        }
    }
    if (j < group && d < cw) ao[(size_t)(g * group + j) * hd + c0 + d] = o;
}

// Batched (prefill) mix without a window, by blocks of MK_W x MK_U tokens: a
// workgroup per (KV head g, DW dims from c0, MK_W MK_U consecutive tokens),
// MK_U consecutive tokens per wave, lane = (head j of the group, dim d); each
// lane runs its tokens' chains o += a_t * v_t,d over positions t in order
// (k_scalar.c:119-122), each product rounded before its add. The block's waves
// share each V tile, staged once in LDS as [dim][position] so one 16-byte read
// gives a lane 4 positions, and each V value read serves the lane's MK_U
// chains, whose adds interleave (a chain's next add need not wait for its
// last). The weights take no LDS: a lane holds its head's weights of 16
// positions in one register a token (lane d of a 16-lane row holds position
// t0 + d), and a DPP row broadcast (row_newbcast) hands position t0 + k's
// weight to every lane of the row as the multiply's operand. So a row of 16
// lanes must hold one head: DW >= 16. Tiles are double-buffered: tile k + 1
// is stored while tile k is read, the loads of tile k + 2 already in flight.
// F16 and Q8 cache rows are widened exactly as they are staged; over the Q8
// cache a lane's weight is a_t * dv_t (the row's scale, k_scalar.c:151)
// before the broadcast, as in the per-token mix.
constexpr int MK_W = 4, MK_U = 2, MK_T = 64, MK_TS = MK_T + 4;

template <int K> __device__ __forceinline__ float row_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + K, 0xF, 0xF, false));
}

// o[u] += a_{t0+4q+i} * v4.i for i < 4 and every token u, positions
// t0 + 4q + i of a 16-position block whose weights sit in a[u] (lane k of
// each row: position t0 + k); the tokens' adds of one position go out together
template <int Q, int U>
__device__ __forceinline__ void mk_quad(float (&o)[U], const float (&a)[U], float4 v) {
#pragma unroll
    for (int u = 0; u < U; u++) o[u] = kr_fadd(o[u], kr_fmul(row_bcast<4 * Q + 0>(a[u]), v.x));
#pragma unroll
    for (int u = 0; u < U; u++) o[u] = kr_fadd(o[u], kr_fmul(row_bcast<4 * Q + 1>(a[u]), v.y));
#pragma unroll
    for (int u = 0; u < U; u++) o[u] = kr_fadd(o[u], kr_fmul(row_bcast<4 * Q + 2>(a[u]), v.z));
#pragma unroll
    for (int u = 0; u < U; u++) o[u] = kr_fadd(o[u], kr_fmul(row_bcast<4 * Q + 3>(a[u]), v.w));
}

template <int DW, int KT>
__global__ void __launch_bounds__(64 * MK_W) k_attn_mix_blk(float *ao, const float *att, const KvView kv, int group,
                                                            int hd, int kv_dim, int max_seq, const int *pos_p,
                                                            int ntok) {
    static_assert(DW >= 16, "a 16-lane row must hold one head");
    constexpr int U = MK_U;
    constexpr int QPR = DW / 4;                 // float4 per staged row of DW dims
    constexpr int RPP = 64 * MK_W / QPR;        // rows the workgroup stages per pass
    constexpr int NP = MK_T / RPP;              // passes per tile
    __shared__ __align__(16) float vt[2][DW * MK_TS];
    __shared__ float dvs[2][KT == KV_Q8 ? MK_T : 1];   // Q8: the tile's V row scales
    const int g = blockIdx.x, c0 = blockIdx.y * DW, z0 = blockIdx.z * MK_W * U, tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, j = lane / DW, d = lane % DW;
    const int zw = z0 + wave * U, pos0 = *pos_p;      // the wave's first token
    const int nmax = pos0 + min(z0 + MK_W * U, ntok);   // positions the block's last token attends
    const int n_heads = gridDim.x * group, cw = min(DW, hd - c0), ntiles = (nmax + MK_T - 1) / MK_T;
    int n[U];   // positions token zw + u attends (0 past the last token)
    const float *arow[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        n[u] = zw + u < ntok ? pos0 + zw + u + 1 : 0;
        arow[u] = att + ((size_t)min(zw + u, ntok - 1) * n_heads + (size_t)g * group + min(j, group - 1)) * max_seq;
    }
    const size_t vbase = (size_t)g * hd + c0;   // element offset of the chunk in a V row
    // staging slot of this thread in pass p: row p * RPP + srow, dims scol .. scol + 3
    const int srow = tid / QPR, scol = min(4 * (tid % QPR), cw - 4);
    using VT = typename Kv4<KT>::T;
    VT sv[NP];
    float sd = 0.0f;
    auto stage_load = [&](int tile) {
#pragma unroll
        for (int p = 0; p < NP; p++)
            sv[p] = Kv4<KT>::load(kv.v, vbase + (size_t)min(tile * MK_T + p * RPP + srow, nmax - 1) * kv_dim + scol);
        if (KT == KV_Q8 && tid < MK_T) sd = kv.vd[(size_t)min(tile * MK_T + tid, nmax - 1) * kv.n_kv + g];
    };
    auto stage_store = [&](int buf) {
        float *V = vt[buf];
#pragma unroll
        for (int p = 0; p < NP; p++) {
            const int r = p * RPP + srow, c = 4 * (tid % QPR);
            const float4 x = Kv4<KT>::wide(sv[p]);
            V[(c + 0) * MK_TS + r] = x.x;
            V[(c + 1) * MK_TS + r] = x.y;
            V[(c + 2) * MK_TS + r] = x.z;
            V[(c + 3) * MK_TS + r] = x.w;
        }
        if (KT == KV_Q8 && tid < MK_T) dvs[buf][tid] = sd;
    };
    // the weights of a tile, loaded two tiles ahead like V: one tile's adds
    // are shorter than a load's round trip
    auto a_load = [&](int tile, float (&a)[U][MK_T / 16]) {
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int b = 0; b < MK_T / 16; b++) a[u][b] = arow[u][min(tile * MK_T + 16 * b + (lane & 15), max_seq - 1)];
    };
    float o[U];
#pragma unroll
    for (int u = 0; u < U; u++) o[u] = 0.0f;
    float acur[U][MK_T / 16], anext[U][MK_T / 16], anext2[U][MK_T / 16];
    stage_load(0);
    stage_store(0);
    a_load(0, acur);
    a_load(min(1, ntiles - 1), anext);
    if (ntiles > 1) stage_load(1);
    __syncthreads();
    for (int k = 0; k < ntiles; k++) {
        const int buf = k & 1, t0 = k * MK_T;
        if (k + 1 < ntiles) stage_store(buf ^ 1);   // its last reader finished before the last barrier
        a_load(min(k + 2, ntiles - 1), anext2);
        // unconditional (a clamped tile past the end is loaded and never
        // stored): with a fixed count of loads behind them, the waits for
        // the weights at the end of the step leave this load in flight
        stage_load(min(k + 2, ntiles - 1));
        const float *V = vt[buf] + d * MK_TS;
        float aw[MK_T / 16][U];   // the weights (Q8: a_t * dv_t)
#pragma unroll
        for (int b = 0; b < MK_T / 16; b++)
#pragma unroll
            for (int u = 0; u < U; u++)
                aw[b][u] = KT == KV_Q8 ? kr_fmul(acur[u][b], dvs[buf][KT == KV_Q8 ? 16 * b + (lane & 15) : 0]) : acur[u][b];
        if (t0 + MK_T <= n[0]) {   // a full tile for every token of the wave (tokens past the last are not stored)
#pragma unroll
            for (int b = 0; b < MK_T / 16; b++) {
                const float4 v0 = *(const float4 *)(V + 16 * b), v1 = *(const float4 *)(V + 16 * b + 4);
                const float4 v2 = *(const float4 *)(V + 16 * b + 8), v3 = *(const float4 *)(V + 16 * b + 12);
                mk_quad<0>(o, aw[b], v0);
                mk_quad<1>(o, aw[b], v1);
                mk_quad<2>(o, aw[b], v2);
                mk_quad<3>(o, aw[b], v3);
            }
        } else {   // the last tiles: each token its live positions
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (t0 >= n[u]) continue;
#pragma unroll
                for (int b = 0; b < MK_T / 16; b++) {
                    const float ab = aw[b][u];
                    float w[16];
                    w[0] = row_bcast<0>(ab); w[1] = row_bcast<1>(ab); w[2] = row_bcast<2>(ab); w[3] = row_bcast<3>(ab);
                    w[4] = row_bcast<4>(ab); w[5] = row_bcast<5>(ab); w[6] = row_bcast<6>(ab); w[7] = row_bcast<7>(ab);
                    w[8] = row_bcast<8>(ab); w[9] = row_bcast<9>(ab); w[10] = row_bcast<10>(ab); w[11] = row_bcast<11>(ab);
                    w[12] = row_bcast<12>(ab); w[13] = row_bcast<13>(ab); w[14] = row_bcast<14>(ab); w[15] = row_bcast<15>(ab);
                    for (int i = 0; i < 16 && t0 + 16 * b + i < n[u]; i++) o[u] = kr_fadd(o[u], kr_fmul(w[i], V[16 * b + i]));
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int b = 0; b < MK_T / 16; b++) {
                acur[u][b] = anext[u][b];
                anext[u][b] = anext2[u][b];
            }
        kr_lds_order();
        __syncthreads();
    }
    if (j < group && d < cw) {
#pragma unroll
        for (int u = 0; u < U; u++)
            if (zw + u < ntok) ao[(size_t)(zw + u) * n_heads * hd + (size_t)(g * group + j) * hd + c0 + d] = o[u];
    }
}

// Batched (prefill) mix without a window for heads of HD = 64 or 128 dims,
// blocked in registers: the rows (token z, query head j) of KV head g,
// numbered z * group + j, go to workgroups RB_R at a time (the longest
// first), and lane (row group rg, dim group dg) of a workgroup owns the
// 4 x HD / 16 outputs of rows 4 rg .. 4 rg + 3 and dims 64 k + 4 dg + i: one
// chain o += a_t * v_t,d per output over positions t in order
// (k_scalar.c:119-122), each product rounded before its add. Per tile of
// RB_T positions the weights [row][position] (Q8: a_t * dv_t, the per-token
// kernel's product) and the V rows [position][dim] (F16 widened, Q8 as its
// int8 values) are staged in LDS; per 4 positions a lane reads its rows' 4
// weights and, per position, its dims' V values, 16-byte reads that feed
// every product they take part in (4 x HD / 16 chains a lane, 2 to 4 reads
// for 64 to 128 multiplies and as many adds: no broadcasts of a weight
// across lanes). In the tiles past some row's own positions a select leaves
// those terms out of that row's sums, so no weight or V value there (rows of
// later tokens, stale rows) reaches them. The next tile's loads are in flight
// while a tile is summed.
template <int HD, int KT, int NT>
__global__ void __launch_bounds__(NT) k_attn_mix_rb(float *ao, const float *att, const KvView kv, int group,
                                                    int kv_dim, int max_seq, const int *pos_p, int ntok) {
    constexpr int NDG = NT / 16, DPL = HD / NDG, NQ = DPL / 4;   // dim groups; dims a lane, NQ quads 4 NDG apart
    constexpr int AS = RB_T + 4;                      // weight row stride (floats)
    constexpr int NA = RB_R * RB_T / 4 / NT;          // 4-weight loads a thread stages per tile
    constexpr int NV = RB_T * HD / 4 / NT;            // 4-element V loads a thread stages per tile
    __shared__ __align__(16) float as[RB_R * AS];
    __shared__ __align__(16) float vs[RB_T * HD];
    const int g = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, dg = tid % NDG, rg = tid / NDG;
    const int nrow = ntok * group, R0 = (gridDim.y - 1 - blockIdx.y) * RB_R;
    const int pos0 = *pos_p, n_heads = gridDim.x * group;
    const int nlast = pos0 + (min(R0 + RB_R, nrow) - 1) / group + 1;   // positions the block's last row attends
    const int ntl = (nlast + RB_T - 1) / RB_T;
    const int zw = (R0 + 4 * (64 / NDG) * wave) / group;   // the token of the wave's first row
    const int zlw = (min(R0 + 4 * (64 / NDG) * (wave + 1), nrow) - 1) / group;   // of its last (within the rows)
    typename Kv4<KT>::T vr[NV];
    float4 ar[NA];
    float dv[NA][4];   // Q8: the V row scales of the staged weights' positions
    auto load = [&](int t0) {
#pragma unroll
        for (int u = 0; u < NV; u++) {
            const int e = tid + NT * u, p = e / (HD / 4), c4 = e % (HD / 4);
            vr[u] = Kv4<KT>::load(kv.v, (size_t)min(t0 + p, nlast - 1) * kv_dim + (size_t)g * HD + 4 * c4);
        }
#pragma unroll
        for (int u = 0; u < NA; u++) {
            const int e = tid + NT * u, rr = e / (RB_T / 4), q4 = e % (RB_T / 4);
            const int R = min(R0 + rr, nrow - 1), z = R / group, j = R - z * group;
            ar[u] = *(const float4 *)(att + ((size_t)z * n_heads + (size_t)g * group + j) * max_seq +
                                      min(t0 + 4 * q4, max_seq - 4));
            if (KT == KV_Q8) {
#pragma unroll
                for (int i = 0; i < 4; i++) dv[u][i] = kv.vd[(size_t)min(t0 + 4 * q4 + i, nlast - 1) * kv.n_kv + g];
            }
        }
    };
    float acc[4][DPL];
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int c = 0; c < DPL; c++) acc[r][c] = 0.0f;
    load(0);
    for (int ti = 0; ti < ntl; ti++) {
        const int t0 = ti * RB_T;
        __syncthreads();   // the last tile is read
#pragma unroll
        for (int u = 0; u < NV; u++) {
            const int e = tid + NT * u;
            *(float4 *)(vs + 4 * e) = Kv4<KT>::wide(vr[u]);   // [position][dim]: e = p HD / 4 + c4
        }
#pragma unroll
        for (int u = 0; u < NA; u++) {
            const int e = tid + NT * u, rr = e / (RB_T / 4), q4 = e % (RB_T / 4);
            float4 a = ar[u];
            if (KT == KV_Q8)
                a = make_float4(kr_fmul(a.x, dv[u][0]), kr_fmul(a.y, dv[u][1]), kr_fmul(a.z, dv[u][2]),
                                kr_fmul(a.w, dv[u][3]));
            *(float4 *)(as + rr * AS + 4 * q4) = a;
        }
        __syncthreads();
        if (ti + 1 < ntl) load(t0 + RB_T);
        const float *ap = as + 4 * rg * AS, *vp = vs + 4 * dg;
        int lim[4];   // in a masked step: position t0 + k counts for row r iff k <= lim[r]
#pragma unroll
        for (int r = 0; r < 4; r++) lim[r] = pos0 + (R0 + 4 * rg + r) / group - t0;
        // positions t .. t + 3 of the tile, every row's terms (UPTO: each
        // row's up to its own position)
        auto step = [&](int t, auto upto) {
            constexpr bool UPTO = decltype(upto)::value;
            float4 a[4];
#pragma unroll
            for (int r = 0; r < 4; r++) a[r] = *(const float4 *)(ap + r * AS + t);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float4 v[NQ];
#pragma unroll
                for (int q = 0; q < NQ; q++) v[q] = *(const float4 *)(vp + (t + k) * HD + 4 * NDG * q);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float w = k == 0 ? a[r].x : k == 1 ? a[r].y : k == 2 ? a[r].z : a[r].w;
                    const bool in = !UPTO || t + k <= lim[r];
#pragma unroll
                    for (int q = 0; q < NQ; q++) {
                        const float4 x = v[q];
                        float *o = acc[r] + 4 * q;
                        o[0] = in ? kr_fadd(o[0], kr_fmul(w, x.x)) : o[0];
                        o[1] = in ? kr_fadd(o[1], kr_fmul(w, x.y)) : o[1];
                        o[2] = in ? kr_fadd(o[2], kr_fmul(w, x.z)) : o[2];
                        o[3] = in ? kr_fadd(o[3], kr_fmul(w, x.w)) : o[3];
                    }
                }
            }
        };
        if (t0 + RB_T - 1 <= pos0 + zw) {   // every position counts for every row of the wave
#pragma unroll 2
            for (int t = 0; t < RB_T; t += 4) step(t, std::false_type{});
        } else {
            // the tile that holds the wave's own positions: whole steps below
            // its first row's position, masked steps up to its last row's
            const int full = pos0 + zw - t0, any = pos0 + zlw - t0;
            for (int t = 0; t < RB_T && t <= any; t += 4) {
                if (t + 3 <= full) step(t, std::false_type{});
                else step(t, std::true_type{});
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int R = R0 + 4 * rg + r;
        if (R >= nrow) continue;
        const int z = R / group, j = R - z * group;
        float *dst = ao + (size_t)z * n_heads * HD + (size_t)(g * group + j) * HD + 4 * dg;
#pragma unroll
        for (int q = 0; q < NQ; q++)
            *(float4 *)(dst + 4 * NDG * q) = make_float4(acc[r][4 * q], acc[r][4 * q + 1], acc[r][4 * q + 2], acc[r][4 * q + 3]);
    }
}

template <int DW>
__global__ void __launch_bounds__(64) k_attn_mix_batch(float *ao, const float *att, const float *vc, int group, int hd,
                                                       int kv_dim, int max_seq, int window, const int *pos_p) {
    const KvView kv = { nullptr, vc, nullptr, nullptr, 0 };
    attn_mix_batch<DW, KV_F32>(ao, att, kv, group, hd, kv_dim, max_seq, window, pos_p);
}

template <int DW, int KT>
__global__ void __launch_bounds__(64) k_attn_mix_batch_kv(float *ao, const float *att, const KvView kv, int group,
                                                          int hd, int kv_dim, int max_seq, int window,
                                                          const int *pos_p) {
    attn_mix_batch<DW, KT>(ao, att, kv, group, hd, kv_dim, max_seq, window, pos_p);
}

// ---- F16 / Q8 cache rows ----

// store_kv (model/transformer.c:191-205) for the positions *pos0 + t: the
// staging rows k, v [ntok][kv_dim] (the projections' output) into one
// layer's F16 cache (every value rounded to half precision, core/ml.c:39-53)
// or Q8 cache (each KV head's head_dim values with one scale,
// ops/ops.c:81-96). One wave per (KV head, K or V, token).
struct KvOut {
    void *k, *v;
    float *kd, *vd;
    int n_kv;
};

template <int KT>
__global__ void __launch_bounds__(64) k_store_kv(const KvOut o, const float *k, const float *v, int kv_dim, int hd,
                                                 const int *pos0) {
    const int h = blockIdx.x, which = blockIdx.y, t = blockIdx.z, lane = threadIdx.x;
    const float *x = (which ? v : k) + (size_t)t * kv_dim + (size_t)h * hd;
    const size_t at = (size_t)(*pos0 + t) * kv_dim + (size_t)h * hd;
    if (KT == KV_F16) {
        uint16_t *dst = (uint16_t *)(which ? o.v : o.k) + at;
        for (int i = lane; i < hd; i += 64) dst[i] = kr_f2h(x[i]);
        return;
    }
    int8_t *dst = (int8_t *)(which ? o.v : o.k) + at;
    float m = 0.0f;
    for (int i = lane; i < hd; i += 64) m = fmaxf(m, fabsf(x[i]));
    for (int sh = 32; sh >= 1; sh >>= 1) m = fmaxf(m, __shfl_xor(m, sh));
    const bool zero = m < KR_QUANT_TINY;
    const float id = zero ? 0.0f : kr_fdiv(127.0f, m);
    for (int i = lane; i < hd; i += 64) dst[i] = zero ? (int8_t)0 : (int8_t)kr_q8_elem(x[i], id);
    if (lane == 0) (which ? o.vd : o.kd)[(size_t)(*pos0 + t) * o.n_kv + h] = zero ? 0.0f : kr_fdiv(m, 127.0f);
}

}   // namespace

// ---- C ABI ----

template <int KT, int DW>
static void launch_mix(const dim3 &grid, int ntok, float *ao, const float *att, const KvView &kv, int group, int hd,
                       int kv_dim, int max_seq, int window, const int *pos) {
    const float *vc = (const float *)kv.v;
    if (ntok > 1 && window == 0 && rb_shape(hd, ntok, group, grid.x) && max_seq % 4 == 0) {
        // prefill without a window, 64- or 128-dim heads: register-blocked rows
        const dim3 rgrid(grid.x, (ntok * group + RB_R - 1) / RB_R, 1);
        if (hd == 64)
            hipLaunchKernelGGL((k_attn_mix_rb<64, KT, 256>), rgrid, dim3(256), 0, kr_stream(), ao, att, kv, group,
                               kv_dim, max_seq, pos, ntok);
        else
            hipLaunchKernelGGL((k_attn_mix_rb<128, KT, RB_NT128>), rgrid, dim3(RB_NT128), 0, kr_stream(), ao, att, kv,
                               group, kv_dim, max_seq, pos, ntok);
        return;
    }
    if constexpr (DW >= 16) {
        if (ntok > 1 && window == 0) {   // prefill without a window: blocks of MK_W tokens share the V tiles
            const dim3 bgrid(grid.x, grid.y, (ntok + MK_W * MK_U - 1) / (MK_W * MK_U));
            hipLaunchKernelGGL((k_attn_mix_blk<DW, KT>), bgrid, dim3(64 * MK_W), 0, kr_stream(), ao, att, kv, group,
                               hd, kv_dim, max_seq, pos, ntok);
            return;
        }
    }
    if (ntok > 1) {
        if constexpr (KT == KV_F32)
            hipLaunchKernelGGL(k_attn_mix_batch<DW>, grid, dim3(64), 0, kr_stream(), ao, att, vc, group, hd, kv_dim,
                               max_seq, window, pos);
        else
            hipLaunchKernelGGL((k_attn_mix_batch_kv<DW, KT>), grid, dim3(64), 0, kr_stream(), ao, att, kv, group, hd,
                               kv_dim, max_seq, window, pos);
    } else {
        // decode: helper rows fill the chip (about 256 workgroups in all)
        const int rows = grid.x ? 256 / (int)grid.x : 0;
        const dim3 hgrid(grid.x, rows > (int)grid.y ? rows : grid.y, 1);
        if constexpr (KT == KV_F32)
            hipLaunchKernelGGL(k_attn_mix<DW>, hgrid, dim3(64 * (1 + MX_P)), 0, kr_stream(), ao, att, vc, group, hd,
                               kv_dim, max_seq, window, pos);
        else
            hipLaunchKernelGGL((k_attn_mix_kv<DW, KT>), hgrid, dim3(64 * (1 + MX_P)), 0, kr_stream(), ao, att, kv, group,
                               hd, kv_dim, max_seq, window, pos);
    }
}

// scores, softmax and mix of ntok positions *pos + t over one layer's cache
// of type KT; max_pos (the last position) sizes the launch
template <int KT>
static void attention(float *ao, float *att, const float *q, const KvView &kv, int n_heads, int n_kv_heads,
                      int head_dim, int max_seq, int window, float scale, const int *pos, int ntok, int max_pos,
                      float cap = 0.0f) {
    if (n_kv_heads <= 0 || n_heads % n_kv_heads || head_dim % 4 || (n_heads * head_dim) % KR_QK ||
        n_heads / n_kv_heads > 16 || head_dim > 1024 || max_seq < 4) {
        kr_fail(ML_E_SHAPE, "attention shape", hipSuccess);
        return;
    }
    const int group = n_heads / n_kv_heads, kv_dim = n_kv_heads * head_dim;
    // the per-token score kernels' LDS: the group's queries and a K tile of
    // tt positions. F32/F16 tiles of wide heads (Gemma's 256) take AT_TD
    // positions; the int8 Q8 tile fits at AT_T up to heads of 512 and more.
    auto tile_lds = [&](int tt) {
        return KT == KV_Q8 ? 64 + (size_t)(group * head_dim + 15) / 16 * 16 + (size_t)tt * (head_dim + 4)
                           : sizeof(float) * ((size_t)group * head_dim + (size_t)tt * (head_dim + 4));
    };
    const int tt = tile_lds(AT_T) <= 64 * 1024 ? AT_T : KT != KV_Q8 && tile_lds(AT_TD) <= 64 * 1024 ? AT_TD : 0;
    if (!tt) {
        kr_fail(ML_E_SHAPE, "attention: head_dim too large for the score tile", hipSuccess);
        return;
    }
    const size_t lds = tile_lds(tt);
    const dim3 sgrid(n_kv_heads, (max_pos + tt) / tt, ntok);
    if constexpr (KT == KV_Q8) {
        // prefill: the K tile and the quantized queries of QB tokens in LDS
        auto qlds = [&](int qb) {
            return sizeof(float) * (AT_T + (size_t)(qb * group + 3) / 4 * 4) + (size_t)(AT_T * (head_dim + 4) + 15) / 16 * 16 +
                   (size_t)qb * group * head_dim;
        };
        const int qb = qlds(16) <= 64 * 1024 ? 16 : qlds(8) <= 64 * 1024 ? 8 : qlds(4) <= 64 * 1024 ? 4 : 0;
        if (ntok > 1 && window == 0 && qb) {
            const dim3 bgrid(n_kv_heads, (max_pos + AT_T) / AT_T, (ntok + AT_TB - 1) / AT_TB);
            auto go = [&](auto kern) {
                hipLaunchKernelGGL(kern, bgrid, dim3(AT_THREADS), qlds(qb), kr_stream(), att, q, kv, group, head_dim,
                                   kv_dim, max_seq, scale, pos, ntok);
            };
            if (qb == 16) go(k_attn_scores_blk_q8<16>);
            else if (qb == 8) go(k_attn_scores_blk_q8<8>);
            else go(k_attn_scores_blk_q8<4>);
        } else {
            hipLaunchKernelGGL(k_attn_scores_q8, sgrid, dim3(AT_THREADS), lds, kr_stream(), att, q, kv, group,
                               head_dim, kv_dim, max_seq, window, scale, pos);
        }
    }
    else {
        // the queries of QB tokens beside a K tile of tp positions, within
        // 64 KB of LDS (tp = AT_T, or AT_T / 2 for wide heads)
        const size_t qtok = sizeof(float) * (size_t)group * head_dim;
        auto ktile = [&](int tp) { return sizeof(float) * (size_t)tp * (head_dim + 4); };
        auto pick_qb = [&](int tp) { return ktile(tp) + 8 * qtok <= 64 * 1024 ? 8 : ktile(tp) + 4 * qtok <= 64 * 1024 ? 4 : 0; };
        const int tp = pick_qb(AT_T) ? AT_T : AT_T / 2, qb = pick_qb(tp);
        if (ntok > 1 && window == 0 && rb_shape(head_dim, ntok, group, n_kv_heads)) {   // prefill: register-blocked rows
            const dim3 rgrid(n_kv_heads, (ntok * group + RB_R - 1) / RB_R, (max_pos + RB_PC * RB_T) / (RB_PC * RB_T));
            if (head_dim == 64)
                hipLaunchKernelGGL((k_attn_scores_rb<64, KT, 256>), rgrid, dim3(256), 0, kr_stream(), att, q, kv,
                                   group, kv_dim, max_seq, scale, pos, ntok);
            else
                hipLaunchKernelGGL((k_attn_scores_rb<128, KT, RB_NT128>), rgrid, dim3(RB_NT128), 0, kr_stream(), att,
                                   q, kv, group, kv_dim, max_seq, scale, pos, ntok);
        } else if (ntok > 1 && window == 0 && qb) {   // prefill: blocks of AT_TB tokens share a K tile
            const dim3 bgrid(n_kv_heads, (max_pos + tp) / tp, (ntok + AT_TB - 1) / AT_TB);
            const size_t blds = ktile(tp) + qb * qtok;
            auto go = [&](auto kern) {
                hipLaunchKernelGGL(kern, bgrid, dim3(AT_THREADS), blds, kr_stream(), att, q, kv, group, head_dim,
                                   kv_dim, max_seq, scale, pos, ntok);
            };
            if (tp != AT_T) {
                if (qb == 8) go(k_attn_scores_blk<0, 8, KT, AT_T / 2>);
                else go(k_attn_scores_blk<0, 4, KT, AT_T / 2>);
            } else if (qb == 8) {
                if (head_dim == 128) go(k_attn_scores_blk<128, 8, KT>);
                else if (head_dim == 64) go(k_attn_scores_blk<64, 8, KT>);
                else go(k_attn_scores_blk<0, 8, KT>);
            } else {
                if (head_dim == 128) go(k_attn_scores_blk<128, 4, KT>);
                else if (head_dim == 64) go(k_attn_scores_blk<64, 4, KT>);
                else go(k_attn_scores_blk<0, 4, KT>);
            }
        } else if (KT != KV_F32) {
            if (tt == AT_T)
                hipLaunchKernelGGL((k_attn_scores_kv<KT, AT_T>), sgrid, dim3(AT_THREADS), lds, kr_stream(), att, q, kv,
                                   group, head_dim, kv_dim, max_seq, window, scale, pos);
            else
                hipLaunchKernelGGL((k_attn_scores_kv<KT, AT_TD>), sgrid, dim3(AT_THREADS), lds, kr_stream(), att, q,
                                   kv, group, head_dim, kv_dim, max_seq, window, scale, pos);
        } else if (ntok == 1 || tt == AT_TD) {   // decode (or a wide head): tiles of AT_TD positions
            const dim3 dgrid(n_kv_heads, (max_pos + AT_TD) / AT_TD, ntok);
            hipLaunchKernelGGL(k_attn_scores<AT_TD>, dgrid, dim3(AT_THREADS), tile_lds(AT_TD), kr_stream(), att, q,
                               (const float *)kv.k, group, head_dim, kv_dim, max_seq, window, scale, pos);
        } else {
            hipLaunchKernelGGL(k_attn_scores<AT_T>, sgrid, dim3(AT_THREADS), lds, kr_stream(), att, q,
                               (const float *)kv.k, group, head_dim, kv_dim, max_seq, window, scale, pos);
        }
    }
    if (cap > 0.0f) krh_softcap_att(att, n_heads, max_seq, window, pos, ntok, cap);   // ops/ops.c:141
    if (ntok > 1 && max_pos + 1 > SM_WN / 2 && max_pos + 1 <= 4096) {
        // prefill rows of 2049 to 4096 scores: a 256-thread workgroup each
        // (measured: 1B-shape 4000-token prompt 59.9k -> 61.7k tok/s; rows
        // up to 2048 run faster one wave each), the ordered sum's lean form
        // (90 VGPRs against 111: 5 waves a SIMD; 64.5k -> 65.5k)
        hipLaunchKernelGGL((k_attn_softmax<256, 4096, true>), dim3(n_heads, 1, ntok), dim3(256), 0, kr_stream(), att,
                           max_seq, window, pos);
    } else if (ntok > 1 && max_pos + 1 <= SM_WN / 2) {   // prefill rows of up to 2048 scores: one wave each
        const int tcap = sc_terms_cap(max_pos + 1), scr = (sc_lds_bytes(max_pos + 1, 64) + 15) / 16 * 16;
        const size_t per_wave = 4 * (size_t)tcap + scr;
        const int nrows = n_heads * ntok;
        hipLaunchKernelGGL((k_attn_softmax_rows<4, SM_V / 2>), dim3((nrows + 3) / 4), dim3(256), 4 * per_wave,
                           kr_stream(), att, n_heads, max_seq, window, pos, nrows, tcap, scr);
    } else {
        hipLaunchKernelGGL((k_attn_softmax<SMX_THREADS, AT_CHUNK>), dim3(n_heads, 1, ntok), dim3(SMX_THREADS), 0, kr_stream(), att, max_seq,
                           window, pos);
    }
    const int gp = group <= 1 ? 1 : group <= 2 ? 2 : group <= 4 ? 4 : group <= 8 ? 8 : 16;
    const int dw = 64 / gp;
    const dim3 grid(n_kv_heads, (head_dim + dw - 1) / dw, ntok);
    switch (dw) {
    case 64: launch_mix<KT, 64>(grid, ntok, ao, att, kv, group, head_dim, kv_dim, max_seq, window, pos); break;
    case 32: launch_mix<KT, 32>(grid, ntok, ao, att, kv, group, head_dim, kv_dim, max_seq, window, pos); break;
    case 16: launch_mix<KT, 16>(grid, ntok, ao, att, kv, group, head_dim, kv_dim, max_seq, window, pos); break;
    case 8: launch_mix<KT, 8>(grid, ntok, ao, att, kv, group, head_dim, kv_dim, max_seq, window, pos); break;
    default: launch_mix<KT, 4>(grid, ntok, ao, att, kv, group, head_dim, kv_dim, max_seq, window, pos); break;
    }
    kr_check_launch("attention");
}

static KvView f32_view(const float *kc, const float *vc) {
    KvView v = { kc, vc, nullptr, nullptr, 0 };
    return v;
}

extern "C" void krh_attention(float *ao, int8_t *aq, float *ad, float *att, const float *q, const float *kc,
                              const float *vc, int n_heads, int n_kv_heads, int head_dim, int max_seq, int window,
                              float scale, const int *pos) {
    attention<KV_F32>(ao, att, q, f32_view(kc, vc), n_heads, n_kv_heads, head_dim, max_seq, window, scale, pos, 1,
                      max_seq - 1);
    if (aq) krh_quantize_q8(aq, ad, ao, n_heads * head_dim, 1);
}

// ---- decode attention without a workspace argument ----
//
// The score rows live in one file-scope device array, `scratch`, of
// KRH_ATTN_SCRATCH_FLOATS floats (8 MiB), which each device holds for the
// life of the process. Host code never passes the array's name to a kernel
// (on the host it only names a stand-in): its device address, one per device,
// comes from hipGetSymbolAddress at set-up (kr_attn_setup, from krh_init).
// Every call on a device shares that device's array, so calls that overlap on
// one device race. No entry of it needs clearing: each call writes every
// score row entry it reads back.
static __device__ __align__(256) float scratch[KRH_ATTN_SCRATCH_FLOATS];
static float *g_scratch_ptr[KR_MAX_DEVICES];

ml_status kr_attn_setup(int dev) {
    if (dev < 0 || dev >= KR_MAX_DEVICES) return ML_E_ISA;
    if (g_scratch_ptr[dev]) return ML_OK;
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
        kr_fail(ML_E_ISA, "hipGetSymbolAddress(scratch)", e);
        return ML_E_ISA;
    }
    g_scratch_ptr[dev] = (float *)ptr;
    return ML_OK;
}

extern "C" void krh_attention_noalloc(float *ao, const float *q, const float *kc, const float *vc, int n_heads,
                                      int n_kv_heads, int head_dim, int max_seq, int window, float scale,
                                      const int *pos) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= KR_MAX_DEVICES || !g_scratch_ptr[dev]) {
        kr_fail(ML_E_ISA, "attention_noalloc: the device's scratch address is not set up (krh_init)", hipSuccess);
        return;
    }
    if (n_heads <= 0 || max_seq <= 0 || (size_t)n_heads * (size_t)max_seq > (size_t)KRH_ATTN_SCRATCH_FLOATS) {
        kr_fail(ML_E_SHAPE, "attention_noalloc: n_heads * max_seq exceeds the static scratch of "
                            "KRH_ATTN_SCRATCH_FLOATS floats", hipSuccess);
        return;
    }
    attention<KV_F32>(ao, g_scratch_ptr[dev], q, f32_view(kc, vc), n_heads, n_kv_heads, head_dim, max_seq, window,
                      scale, pos, 1, max_seq - 1);
}

extern "C" void krh_set_attn_rb_min(int min_wg) { g_rb_min_wg = min_wg < 0 ? 0 : min_wg; }

extern "C" void krh_attention_batch(float *ao, float *att, const float *q, const float *kc, const float *vc,
                                    int n_heads, int n_kv_heads, int head_dim, int max_seq, int window, float scale,
                                    const int *pos0, int ntok, int last_pos) {
    if (ntok <= 0 || last_pos >= max_seq) {
        kr_fail(ML_E_SHAPE, "attention batch shape", hipSuccess);
        return;
    }
    attention<KV_F32>(ao, att, q, f32_view(kc, vc), n_heads, n_kv_heads, head_dim, max_seq, window, scale, pos0, ntok,
                      last_pos);
}

extern "C" void krh_attention_kv(float *ao, float *att, const float *q, const ml_kv_layer *kv, int n_heads,
                                 int n_kv_heads, int head_dim, int max_seq, float scale, const int *pos0, int ntok,
                                 int last_pos) {
    krh_attention_kv_softcap(ao, att, q, kv, n_heads, n_kv_heads, head_dim, max_seq, scale, pos0, ntok, last_pos, 0.0f);
}

extern "C" void krh_attention_kv_softcap(float *ao, float *att, const float *q, const ml_kv_layer *kv, int n_heads,
                                         int n_kv_heads, int head_dim, int max_seq, float scale, const int *pos0,
                                         int ntok, int last_pos, float cap) {
    if (ntok <= 0 || last_pos >= max_seq || !kv) {
        kr_fail(ML_E_SHAPE, "attention shape", hipSuccess);
        return;
    }
    if (kv->k && kv->v) {
        attention<KV_F32>(ao, att, q, f32_view(kv->k, kv->v), n_heads, n_kv_heads, head_dim, max_seq, kv->window,
                          scale, pos0, ntok, last_pos, cap);
    } else if (kv->kh && kv->vh) {
        KvView v = { kv->kh, kv->vh, nullptr, nullptr, n_kv_heads };
        attention<KV_F16>(ao, att, q, v, n_heads, n_kv_heads, head_dim, max_seq, kv->window, scale, pos0, ntok,
                          last_pos, cap);
    } else if (kv->kq && kv->vq && kv->kd && kv->vd) {
        KvView v = { kv->kq, kv->vq, kv->kd, kv->vd, n_kv_heads };
        attention<KV_Q8>(ao, att, q, v, n_heads, n_kv_heads, head_dim, max_seq, kv->window, scale, pos0, ntok,
                         last_pos, cap);
    } else {
        kr_fail(ML_E_SHAPE, "attention: the cache view has no F32, F16 or Q8 rows", hipSuccess);
    }
}

extern "C" void krh_attention_q8_store(float *ao, float *att, const float *q, const ml_kv_layer *kv,
                                       const float *k_row, const float *v_row, int n_heads, int n_kv_heads,
                                       int head_dim, int max_seq, float scale, const int *pos) {
    if (!kv || !kv->kq || !kv->vq || !kv->kd || !kv->vd || !k_row || !v_row) {
        kr_fail(ML_E_SHAPE, "attention_q8_store: a Q8 cache view and the staging rows", hipSuccess);
        return;
    }
    KvView v = { kv->kq, kv->vq, kv->kd, kv->vd, n_kv_heads, k_row, v_row };
    attention<KV_Q8>(ao, att, q, v, n_heads, n_kv_heads, head_dim, max_seq, kv->window, scale, pos, 1, max_seq - 1);
}

extern "C" void krh_store_kv(int kv_type, void *kc, void *vc, float *kd, float *vd, const float *k, const float *v,
                             int n_kv_heads, int head_dim, const int *pos0, int ntok) {
    if (ntok <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim % 4 || !kc || !vc ||
        (kv_type == ML_Q8_0 && (!kd || !vd)) || (kv_type != ML_Q8_0 && kv_type != ML_F16)) {
        kr_fail(ML_E_SHAPE, "store_kv: an F16 or Q8 cache and its shape", hipSuccess);
        return;
    }
    const dim3 grid(n_kv_heads, 2, ntok);
    const int kv_dim = n_kv_heads * head_dim;
    KvOut o = { kc, vc, kd, vd, n_kv_heads };
    if (kv_type == ML_F16)
        hipLaunchKernelGGL(k_store_kv<KV_F16>, grid, dim3(64), 0, kr_stream(), o, k, v, kv_dim, head_dim, pos0);
    else
        hipLaunchKernelGGL(k_store_kv<KV_Q8>, grid, dim3(64), 0, kr_stream(), o, k, v, kv_dim, head_dim, pos0);
    kr_check_launch("store_kv");
}

