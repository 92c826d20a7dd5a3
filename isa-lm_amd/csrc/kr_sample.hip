// The reference's sampler (model/sampler.c) on the device, with its results:
// the same id, the same penalized logits and the same generator state after
// every draw, so the token loop needs no logits on the host.
//
// One workgroup runs the penalty, the greedy pick, the temperature softmax
// and the multinomial walk. The top-k and top-p draws order their candidates
// by a stable radix sort over many workgroups, then one workgroup runs the
// nucleus cut and the draw. Every sum the reference forms one add at a time
// (the softmax's normalizer, the cumulative sums of the draws) is formed in
// that order, exactly, by the shifted-run ordered sum; a draw's "first
// partial sum above a bound" is one chunk's chain away from the chunk starts
// that sum records.
#include <climits>
#include "kr_internal.h"
#include "kr_chain.h"

struct krh_sampler_dev {
    float temperature, topp, rp;
    int topk, R, vocab;
    unsigned long long *rng;   // xorshift64* state
    int *ring;                 // [2 + R]: n_recent, recent_at, then the ids
    int *first;                // [vocab]: the penalty's first ring slot per id
    float *probs;              // [vocab]
    unsigned *keys;            // [2][vocab]: sort keys, two buffers
    int *ids;                  // [2][vocab]
    int *hist;                 // [blocks][256]: digit counts per sort workgroup
    float *part;               // [blocks]: the elementwise workgroups' maxima
    int *pnan;                 // [blocks]: and whether they saw a NaN
    int *meta;                 // [8]: see MT_*
};

struct krh_sampler {
    krh_sampler_dev d;
    void *mem;
};

namespace {

constexpr int SM_NT = 1024;                                       // threads of the one-workgroup kernels
constexpr int SM_G = 12288;                                       // terms per ordered-sum group (in LDS)
constexpr int SM_RT = 256, SM_ROWS = 4, SM_E = SM_RT * SM_ROWS;   // radix sort: threads, rows, ids per workgroup
constexpr int SM_HB = 16;                                         // digit counts read at a time
constexpr int SM_EB = 2048;                                       // ids per elementwise workgroup (256 x 8)
constexpr int SM_TERMS = sc_terms_cap(SM_G) * 4;
constexpr int SM_SCR = (sc_lds_bytes(SM_G, SM_NT) + 15) & ~15;
constexpr int SM_CST = (sc_chunks(SM_G) + 1) * 4;
constexpr int SM_LDS = SM_TERMS + SM_SCR + SM_CST + 16;
static_assert(SM_G % SM_NT == 0, "a thread keeps its ids across the softmax's passes");
static_assert(SM_LDS <= 64 * 1024, "LDS");

enum { SM_GREEDY = 0, SM_MULT = 1, SM_TOPK = 2, SM_TOPP = 3 };
// meta: candidates after the sort's first pass, the coin's bits, whether the
// id is already decided (NaN probabilities), and that id
enum { MT_M = 0, MT_COIN = 1, MT_DONE = 2, MT_ID = 3, MT_KIND = 4 };
// the softmax's case, from the maxima: numerators expf(p - max), all -inf
// (uniform 1/n), or a NaN term (every probability NaN)
enum { SK_EXP = 0, SK_UNIFORM = 1, SK_NAN = 2 };

using Dev = krh_sampler_dev;

__device__ __forceinline__ int sm_tid() { return (int)threadIdx.x; }

// a workgroup barrier after which every thread sees the others' global
// stores and atomics: the device-scope fences wait for them and drop stale
// L1 lines
__device__ __forceinline__ void sm_sync_global() {
    __threadfence();
    __syncthreads();
    __threadfence();
}

// model/sampler.c:57-61: the first index of the largest value; NaN never
// wins, except at index 0 (nothing compares greater than it)
__device__ __forceinline__ void sm_take(float &bv, int &bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}
__device__ int sm_argmax(const float *v, int n, float *rv, int *ri) {
    float bv = -INFINITY;
    int bi = INT_MAX;
    for (int i = sm_tid(); i < n; i += SM_NT) sm_take(bv, bi, v[i], i);
    for (int o = 32; o >= 1; o >>= 1) sm_take(bv, bi, __shfl_xor(bv, o), __shfl_xor(bi, o));
    if ((sm_tid() & 63) == 0) {
        rv[sm_tid() >> 6] = bv;
        ri[sm_tid() >> 6] = bi;
    }
    __syncthreads();
    bv = rv[0];
    bi = ri[0];
    for (int w = 1; w < SM_NT / 64; w++) sm_take(bv, bi, rv[w], ri[w]);
    __syncthreads();
    return (bi == INT_MAX || v[0] != v[0]) ? 0 : bi;
}

// model/sampler.c:39-48: every distinct id of the ring that is below n, once
// (at its first slot): a positive logit divided by the penalty, any other
// multiplied. The first slot of each id is found with an atomic minimum.
__device__ void sm_penalize(float *logits, int n, const Dev &d) {
    if (d.rp == 1.0f) return;
    const int nr = d.ring[0];
    if (nr == 0) return;
    const int *rid = d.ring + 2;
    for (int i = sm_tid(); i < nr; i += SM_NT)
        __hip_atomic_store(&d.first[rid[i]], INT_MAX, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sm_sync_global();
    for (int i = sm_tid(); i < nr; i += SM_NT) atomicMin(&d.first[rid[i]], i);
    sm_sync_global();
    for (int i = sm_tid(); i < nr; i += SM_NT) {
        const int t = rid[i];
        if (t >= n || __hip_atomic_load(&d.first[t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != i) continue;
        const float x = logits[t];
        logits[t] = x > 0.0f ? kr_fdiv(x, d.rp) : kr_fmul(x, d.rp);
    }
    sm_sync_global();
}

// model/sampler.c:30-35 (one thread)
__device__ void sm_accept(const Dev &d, int t) {
    if (d.R <= 0 || t < 0 || t >= d.vocab) return;
    const int at = d.ring[1];
    d.ring[2 + at] = t;
    d.ring[1] = (at + 1) % d.R;
    if (d.ring[0] < d.R) d.ring[0] += 1;
}

// the id out, as krh_argmax writes it, then accepted (one thread)
__device__ void sm_finish(int t, int *tok, int *pos, int *log, const Dev &d) {
    *tok = t;
    if (pos) {
        const int p = *pos + 1;
        if (log) log[p] = t;
        *pos = p;
    }
    sm_accept(d, t);
}

// model/sampler.c:50-55: xorshift64*, the top 24 bits of the product's high
// word over 2^24 (both exact in float)
__device__ float sm_coin(unsigned long long *st) {
    unsigned long long x = *st;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *st = x;
    const unsigned hi = (unsigned)((x * 0x2545F4914F6CDD1Dull) >> 32);
    return kr_fdiv((float)(hi >> 8), 16777216.0f);
}

// The first i < m with thr < term(0) + ... + term(i), the sum formed one add
// at a time from +0 (model/sampler.c:63-70, :113-128, :140-151); -1 when none.
// val: that partial sum, or the whole sum. SM_G terms at a time go to LDS;
// the group whose end passes thr is searched from the chunk starts its
// ordered sum recorded: the first chunk whose end passes thr holds the
// answer, and one lane runs that chunk's chain from its true start. All
// SM_NT threads call it.
template <class Term>
__device__ int sm_first_above(Term term, int m, float thr, unsigned char *lds, float &val) {
    float *t = (float *)lds;
    unsigned char *scr = lds + SM_TERMS;
    unsigned *cst = (unsigned *)(scr + SM_SCR);
    int *res = (int *)(lds + SM_TERMS + SM_SCR + SM_CST);
    const int tid = sm_tid(), lane = tid & 63;
    float S = 0.0f;
    for (int g0 = 0; g0 < m; g0 += SM_G) {
        const int ng = min(SM_G, m - g0), sh = sc_log_len(ng), C = sc_chunks(ng), L = 1 << sh;
        for (int i = tid; i < ng; i += SM_NT) t[sc_at(i, sh)] = term(g0 + i);
        __syncthreads();
        const float E = kr_spec_sum<SM_NT, true>(t, ng, scr, S, cst);
        if (thr < E) {
            if (tid < 64) {
                int c = -1;
                if (cst[C] == 0) {
                    for (int c0 = 0; c0 < C && c < 0; c0 += 64) {
                        const int cc = c0 + lane;
                        const float end = cc + 1 < C ? __uint_as_float(cst[min(cc + 1, C - 1)]) : E;
                        const unsigned long long b = __ballot(cc < C && thr < end);
                        if (b) c = c0 + __builtin_ctzll(b);
                    }
                }
                if (lane == 0) {
                    // c < 0: the sum went through the sequential loop; so does the search
                    float s = c >= 0 ? __uint_as_float(cst[c]) : S;
                    const int i0 = c >= 0 ? c * L : 0, i1 = c >= 0 ? min(i0 + L, ng) : ng;
                    int f = ng - 1;
                    for (int i = i0; i < i1; i++) {
                        s = kr_fadd(s, t[sc_at(i, sh)]);
                        if (thr < s) {
                            f = i;
                            break;
                        }
                    }
                    res[0] = g0 + f;
                    res[1] = __float_as_int(s);
                }
            }
            __syncthreads();
            val = __int_as_float(res[1]);
            const int r = res[0];
            __syncthreads();
            return r;
        }
        S = E;
    }
    val = S;
    return -1;
}

// The penalty alone (one workgroup), ahead of the kernels that read the logits.
__global__ void __launch_bounds__(SM_NT) k_smp_penalize(float *logits, int n, Dev d) { sm_penalize(logits, n, d); }

// Temperature (model/sampler.c:158): p = logits / T, and each workgroup's
// maximum (NaN-ignoring, as fmaxf) and whether it saw a NaN.
__global__ void __launch_bounds__(256) k_smp_scale(const float *logits, int n, Dev d) {
    __shared__ float red[4];
    __shared__ int rn[4];
    float mx = __int_as_float(0x7fc00000);
    int nan = 0;
    const int base = (int)blockIdx.x * SM_EB + sm_tid();
#pragma unroll
    for (int k = 0; k < SM_EB / 256; k++) {
        const int i = base + k * 256;
        if (i < n) {
            const float v = kr_fdiv(logits[i], d.temperature);
            d.probs[i] = v;
            mx = fmaxf(mx, v);
            nan |= v != v;
        }
    }
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    nan = __any(nan);
    if ((sm_tid() & 63) == 0) {
        red[sm_tid() >> 6] = mx;
        rn[sm_tid() >> 6] = nan;
    }
    __syncthreads();
    if (sm_tid() == 0) {
        d.part[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        d.pnan[blockIdx.x] = rn[0] | rn[1] | rn[2] | rn[3];
    }
}

// The softmax's numerators (kernels/scalar/k_scalar.c:66-77): the maximum
// of all workgroups' maxima, then expf(p - max); every value -inf: 1/n; a NaN
// term (a NaN value, or inf - inf): NaN everywhere, as the sum and every
// probability become.
__global__ void __launch_bounds__(256) k_smp_exp(int n, int nblk, Dev d) {
    __shared__ float sp[256];
    __shared__ int sn[256];
    if (sm_tid() < nblk) {
        sp[sm_tid()] = d.part[sm_tid()];
        sn[sm_tid()] = d.pnan[sm_tid()];
    }
    __syncthreads();
    float mx = __int_as_float(0x7fc00000);
    int nan = 0;
    for (int k = 0; k < nblk; k++) {
        mx = fmaxf(mx, sp[k]);
        nan |= sn[k];
    }
    const int kind = mx == -INFINITY ? SK_UNIFORM : (nan || mx != mx || mx == INFINITY) ? SK_NAN : SK_EXP;
    if (blockIdx.x == 0 && sm_tid() == 0) d.meta[MT_KIND] = kind;
    const float u = kr_fdiv(1.0f, (float)n);
    const int base = (int)blockIdx.x * SM_EB + sm_tid();
#pragma unroll
    for (int k = 0; k < SM_EB / 256; k++) {
        const int i = base + k * 256;
        if (i < n) {
            const float p = d.probs[i];
            d.probs[i] = kind == SK_EXP ? kr_expf(kr_fsub(p, mx)) : kind == SK_UNIFORM ? u : __int_as_float(0x7fc00000);
        }
    }
}

// The softmax's ordered sum and x * (1/sum) (kernels/scalar/k_scalar.c:
// 73-76), the coin, and for the multinomial walk the draw. For the sorted
// draws it leaves the probabilities and the coin for the kernels after it.
template <int MODE>
__global__ void __launch_bounds__(SM_NT) k_smp_main(int *tok, int n, Dev d, int *pos, int *log) {
    extern __shared__ __align__(16) unsigned char sm_lds[];
    __shared__ float scoin;
    const int tid = sm_tid();
    {
        float *p = d.probs;
        const int kind = d.meta[MT_KIND];
        // NaN probabilities: the walk passes no coin (the last id), top-p
        // keeps no candidate (the argmax of all-NaN: 0), and top-k keeps the
        // first k ids in id order (the last of them)
        const int decided = kind != SK_NAN ? -1 : MODE == SM_MULT ? n - 1 : MODE == SM_TOPK ? d.topk - 1 : 0;
        if (kind == SK_EXP) {
            float *t = (float *)sm_lds;
            float S = 0.0f;
            for (int g0 = 0; g0 < n; g0 += SM_G) {
                const int ng = min(SM_G, n - g0), sh = sc_log_len(ng);
                for (int i = tid; i < ng; i += SM_NT) t[sc_at(i, sh)] = p[g0 + i];
                __syncthreads();
                S = kr_spec_sum<SM_NT>(t, ng, sm_lds + SM_TERMS, S);
            }
            const float inv = kr_fdiv(1.0f, S);
            for (int i = tid; i < n; i += SM_NT) p[i] = kr_fmul(p[i], inv);
        }
        if (tid == 0) scoin = sm_coin(d.rng);
        __syncthreads();
        const float coin = scoin;
        if constexpr (MODE == SM_MULT) {
            int t = decided;
            if (t < 0) {
                float v;
                const int j = sm_first_above([&](int i) { return p[i]; }, n, coin, sm_lds, v);
                t = j >= 0 ? j : n - 1;
            }
            if (tid == 0) sm_finish(t, tok, pos, log, d);
        } else {
            if (tid == 0) {
                d.meta[MT_COIN] = __float_as_int(coin);
                d.meta[MT_DONE] = decided >= 0;
                d.meta[MT_ID] = decided;
            }
        }
    }
}

// The stable radix sort of the candidates, 8 bits a pass from the lowest.
// The key is the complement of the probability's bits: non-negative floats
// order as their bits, so ascending keys are descending probabilities, and
// the sort's stability keeps ids ascending among equal ones -- the order of
// model/sampler.c:72-80. Pass 0 reads the probabilities and keeps the
// candidates (all for top-k; top-p: those >= cutoff, model/sampler.c:134-137)
// in id order; the passes alternate between the two key buffers and end in
// the second. Each workgroup takes SM_E ids as SM_ROWS rows of SM_RT.
template <int P>
__device__ __forceinline__ void sm_in(const Dev &d, int i, int m, float cutoff, int filt, unsigned &key, int &id,
                                      bool &keep) {
    keep = i < m;
    key = 0;
    id = 0;
    if (!keep) return;
    if constexpr (P == 0) {
        const float p = d.probs[i];
        keep = !filt || p >= cutoff;
        key = ~__float_as_uint(p);
        id = i;
    } else {
        const int src = (P & 1) ? 0 : d.vocab;
        key = d.keys[src + i];
        id = d.ids[src + i];
    }
}

template <int P>
__global__ void __launch_bounds__(SM_RT) k_smp_hist(Dev d, int n, float cutoff, int filt) {
    __shared__ int cnt[256];
    if (d.meta[MT_DONE]) return;
    const int tid = sm_tid();
    cnt[tid] = 0;
    __syncthreads();
    const int m = P == 0 ? n : d.meta[MT_M];
    for (int r = 0; r < SM_ROWS; r++) {
        unsigned key;
        int id;
        bool keep;
        sm_in<P>(d, (int)blockIdx.x * SM_E + r * SM_RT + tid, m, cutoff, filt, key, id, keep);
        if (keep) atomicAdd(&cnt[(key >> (8 * P)) & 255], 1);
    }
    __syncthreads();
    d.hist[blockIdx.x * 256 + tid] = cnt[tid];
}

template <int P>
__global__ void __launch_bounds__(SM_RT) k_smp_scatter(Dev d, int n, float cutoff, int filt) {
    constexpr int NW = SM_RT / 64;
    __shared__ int wc[SM_ROWS][NW][256];   // per row and wave: digit counts, then first slots
    __shared__ int goff[256];
    __shared__ int wsum[NW];
    if (d.meta[MT_DONE]) return;
    const int tid = sm_tid(), lane = tid & 63, w = tid >> 6, NB = (int)gridDim.x, b = (int)blockIdx.x;
    const int m = P == 0 ? n : d.meta[MT_M];
    // digit tid: ids of this digit in earlier workgroups, and in all; the
    // counts are read SM_HB at a time, so their L2 latencies overlap
    int tot = 0, pre = 0;
    for (int k0 = 0; k0 < NB; k0 += SM_HB) {
        int c[SM_HB];
#pragma unroll
        for (int j = 0; j < SM_HB; j++) c[j] = d.hist[min(k0 + j, NB - 1) * 256 + tid];
#pragma unroll
        for (int j = 0; j < SM_HB; j++) {
            const int v = k0 + j < NB ? c[j] : 0;
            tot += v;
            pre += k0 + j < b ? v : 0;
        }
    }
    int inc = tot;
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(inc, o);
        if (lane >= o) inc += u;
    }
    if (lane == 63) wsum[w] = inc;
    for (int k = tid; k < SM_ROWS * NW * 256; k += SM_RT) (&wc[0][0][0])[k] = 0;
    // each row's ids: the rank among equal digits of the wave (lanes match
    // on all 8 digit bits)
    unsigned key[SM_ROWS];
    int id[SM_ROWS], dg[SM_ROWS], rk[SM_ROWS], cw[SM_ROWS];
    bool keep[SM_ROWS];
    const unsigned long long lt = (1ull << lane) - 1ull;
#pragma unroll
    for (int r = 0; r < SM_ROWS; r++) {
        sm_in<P>(d, b * SM_E + r * SM_RT + tid, m, cutoff, filt, key[r], id[r], keep[r]);
        dg[r] = (int)((key[r] >> (8 * P)) & 255u);
        unsigned long long pm = __ballot(keep[r]);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const unsigned long long bk = __ballot((dg[r] >> k) & 1);
            pm &= ((dg[r] >> k) & 1) ? bk : ~bk;
        }
        rk[r] = __popcll(pm & lt);
        cw[r] = __popcll(pm);
    }
    __syncthreads();
    int base = inc - tot;
    for (int k = 0; k < w; k++) base += wsum[k];
    goff[tid] = base + pre;
    if (P == 0 && b == 0 && tid == 255) d.meta[MT_M] = base + tot;
#pragma unroll
    for (int r = 0; r < SM_ROWS; r++)
        if (keep[r] && rk[r] == 0) wc[r][w][dg[r]] = cw[r];
    __syncthreads();
    int run = 0;
    for (int r = 0; r < SM_ROWS; r++)
        for (int ww = 0; ww < NW; ww++) {
            const int c = wc[r][ww][tid];
            wc[r][ww][tid] = run;
            run += c;
        }
    __syncthreads();
    const int dst0 = (P & 1) ? d.vocab : 0;
#pragma unroll
    for (int r = 0; r < SM_ROWS; r++)
        if (keep[r]) {
            const int at = goff[dg[r]] + wc[r][w][dg[r]] + rk[r];
            d.keys[dst0 + at] = key[r];
            d.ids[dst0 + at] = id[r];
        }
}

// The sorted draws: model/sampler.c:111-130 over the k first candidates
// (top-k), or :138-152 over the kept ones (top-p; none kept: the argmax of
// the probabilities).
template <int MODE>
__global__ void __launch_bounds__(SM_NT) k_smp_final(int *tok, int n, Dev d, int *pos, int *log) {
    extern __shared__ __align__(16) unsigned char sm_lds[];
    __shared__ float rv[SM_NT / 64];
    __shared__ int ri[SM_NT / 64];
    int t;
    if (d.meta[MT_DONE]) {
        t = d.meta[MT_ID];
    } else {
        const float coin = __int_as_float(d.meta[MT_COIN]);
        const unsigned *keys = d.keys + d.vocab;
        const int *ids = d.ids + d.vocab;
        auto term = [&](int i) { return __uint_as_float(~keys[i]); };
        if constexpr (MODE == SM_TOPK) {
            const int k = d.topk;
            float total, cum, c;
            sm_first_above(term, k, INFINITY, sm_lds, total);
            int last = k - 1;
            if (d.topp > 0.0f && d.topp < 1.0f) {
                const int i = sm_first_above(term, k, kr_fmul(d.topp, total), sm_lds, cum);
                if (i >= 0) last = i;
                total = cum;
            }
            const int j = sm_first_above(term, last + 1, kr_fmul(coin, total), sm_lds, c);
            t = ids[j >= 0 ? j : last];
        } else {
            const int m = d.meta[MT_M];
            if (m == 0) {
                t = sm_argmax(d.probs, n, rv, ri);
            } else {
                float cum, c;
                const int i = sm_first_above(term, m, d.topp, sm_lds, cum);
                const int last = i >= 0 ? i : m - 1;
                const int j = sm_first_above(term, last + 1, kr_fmul(coin, cum), sm_lds, c);
                t = ids[j >= 0 ? j : last];
            }
        }
    }
    if (sm_tid() == 0) sm_finish(t, tok, pos, log, d);
}

__global__ void k_smp_accept(Dev d, const int *tokens, int n) {
    for (int i = 0; i < n; i++) sm_accept(d, tokens[i]);
}

template <int P>
void sort_pass(const Dev &d, int n, float cutoff, int filt) {
    const int nb = (n + SM_E - 1) / SM_E;
    hipLaunchKernelGGL(k_smp_hist<P>, dim3(nb), dim3(SM_RT), 0, kr_stream(), d, n, cutoff, filt);
    hipLaunchKernelGGL(k_smp_scatter<P>, dim3(nb), dim3(SM_RT), 0, kr_stream(), d, n, cutoff, filt);
}

}  // namespace

extern "C" ml_status krh_sampler_new(krh_sampler **out, int vocab, const krh_sampler_opts *o) {
    *out = nullptr;
    if (vocab < 1 || !o) {
        kr_fail(ML_E_SHAPE, "sampler vocab", hipSuccess);
        return ML_E_SHAPE;
    }
    krh_sampler *s = (krh_sampler *)calloc(1, sizeof *s);
    if (!s) return ML_E_NOMEM;
    Dev &d = s->d;
    d.temperature = o->temperature;
    d.topp = o->topp;
    d.topk = o->topk;
    d.rp = o->repeat_penalty;
    d.R = o->repeat_last_n > 0 ? o->repeat_last_n : 0;
    d.vocab = vocab;
    const size_t V = (size_t)vocab, nb = (V + SM_E - 1) / SM_E;
    if (V > (size_t)256 * SM_EB) {   // the exp kernel gathers at most 256 workgroup maxima
        free(s);
        kr_fail(ML_E_SHAPE, "sampler vocab", hipSuccess);
        return ML_E_SHAPE;
    }
    // rng, probs, keys and ids (two buffers each), hist, part, pnan, meta, first, ring
    const size_t bytes = 8 + 4 * (V + 4 * V + nb * 256 + 2 * nb + 8 + V + 2 + (size_t)d.R);
    hipError_t e = hipMalloc(&s->mem, bytes);
    if (e != hipSuccess) {
        free(s);
        kr_fail(ML_E_NOMEM, "sampler memory", e);
        return ML_E_NOMEM;
    }
    char *p = (char *)s->mem;
    d.rng = (unsigned long long *)p;
    p += 8;
    d.probs = (float *)p;
    p += 4 * V;
    d.keys = (unsigned *)p;
    p += 8 * V;
    d.ids = (int *)p;
    p += 8 * V;
    d.hist = (int *)p;
    p += 4 * nb * 256;
    d.part = (float *)p;
    p += 4 * nb;
    d.pnan = (int *)p;
    p += 4 * nb;
    d.meta = (int *)p;
    p += 32;
    d.first = (int *)p;
    p += 4 * V;
    d.ring = (int *)p;
    // model/sampler.c:10: a zero seed takes the golden-ratio constant
    const unsigned long long seed = o->seed ? (unsigned long long)o->seed : 0x9E3779B97F4A7C15ull;
    const int zero[2] = {0, 0};
    e = hipMemcpyAsync(d.rng, &seed, 8, hipMemcpyHostToDevice, kr_stream());
    if (e == hipSuccess) e = hipMemcpyAsync(d.ring, zero, 8, hipMemcpyHostToDevice, kr_stream());
    if (e == hipSuccess) e = hipStreamSynchronize(kr_stream());
    if (e != hipSuccess) {
        (void)hipFree(s->mem);
        free(s);
        kr_fail(ML_E_IO, "sampler set-up", e);
        return ML_E_IO;
    }
    *out = s;
    return ML_OK;
}

extern "C" void krh_sampler_free(krh_sampler *s) {
    if (!s) return;
    (void)hipFree(s->mem);
    free(s);
}

extern "C" void krh_sampler_accept(krh_sampler *s, const int *tokens, int n) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_smp_accept, dim3(1), dim3(1), 0, kr_stream(), s->d, tokens, n);
    kr_check_launch("sampler_accept");
}

extern "C" uint64_t krh_sampler_rng(const krh_sampler *s) {
    unsigned long long v = 0;
    if (hipMemcpyAsync(&v, s->d.rng, 8, hipMemcpyDeviceToHost, kr_stream()) != hipSuccess ||
        hipStreamSynchronize(kr_stream()) != hipSuccess)
        kr_fail(ML_E_IO, "sampler rng read", hipGetLastError());
    return v;
}

extern "C" void krh_sample(krh_sampler *s, int *tok, float *logits, int n, int *pos, int *log) {
    const Dev &d = s->d;
    if (n < 1 || n > d.vocab) {
        kr_fail(ML_E_SHAPE, "sample size", hipSuccess);
        return;
    }
    // model/sampler.c:157-164
    const int mode = d.temperature == 0.0f                ? SM_GREEDY
                     : (d.topk > 0 && d.topk < n)         ? SM_TOPK
                     : (d.topp <= 0.0f || d.topp >= 1.0f) ? SM_MULT
                                                          : SM_TOPP;
    hipStream_t st = kr_stream();
    if (d.rp != 1.0f) hipLaunchKernelGGL(k_smp_penalize, dim3(1), dim3(SM_NT), 0, st, logits, n, d);
    if (mode == SM_GREEDY) {   // the many-workgroup argmax; the ring only matters with a penalty
        krh_argmax(tok, logits, n, pos, log);
        if (d.rp != 1.0f) hipLaunchKernelGGL(k_smp_accept, dim3(1), dim3(1), 0, st, d, (const int *)tok, 1);
        kr_check_launch("sample");
        return;
    }
    const int nblk = (n + SM_EB - 1) / SM_EB;
    hipLaunchKernelGGL(k_smp_scale, dim3(nblk), dim3(256), 0, st, logits, n, d);
    hipLaunchKernelGGL(k_smp_exp, dim3(nblk), dim3(256), 0, st, n, nblk, d);
    switch (mode) {
    case SM_MULT:
        hipLaunchKernelGGL(k_smp_main<SM_MULT>, dim3(1), dim3(SM_NT), SM_LDS, st, tok, n, d, pos, log);
        break;
    default: {
        const int topp = mode == SM_TOPP;
        // model/sampler.c:134, in float as there
        const float cutoff = topp && n > 1 ? (1.0f - d.topp) / (float)(n - 1) : 0.0f;
        if (topp)
            hipLaunchKernelGGL(k_smp_main<SM_TOPP>, dim3(1), dim3(SM_NT), SM_LDS, st, tok, n, d, pos, log);
        else
            hipLaunchKernelGGL(k_smp_main<SM_TOPK>, dim3(1), dim3(SM_NT), SM_LDS, st, tok, n, d, pos, log);
        sort_pass<0>(d, n, cutoff, topp);
        sort_pass<1>(d, n, cutoff, topp);
        sort_pass<2>(d, n, cutoff, topp);
        sort_pass<3>(d, n, cutoff, topp);
        if (topp)
            hipLaunchKernelGGL(k_smp_final<SM_TOPP>, dim3(1), dim3(SM_NT), SM_LDS, st, tok, n, d, pos, log);
        else
            hipLaunchKernelGGL(k_smp_final<SM_TOPK>, dim3(1), dim3(SM_NT), SM_LDS, st, tok, n, d, pos, log);
    }
    }
    kr_check_launch("sample");
}
