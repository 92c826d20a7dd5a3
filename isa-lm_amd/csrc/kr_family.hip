// The model families' own steps on the token path (model/transformer.c):
// the per-head q/k RMSNorm of Qwen3 (:246-248) ahead of RoPE, RoPE at the
// position held in device memory (so the step can be captured once and
// replayed), and F32 cache rows written from the projections' staging rows.
// The post-norms of Gemma 3 (:240-243) use the unfused rmsnorm and add.
#include "kr_internal.h"
#include "kr_numerics.h"

namespace {

constexpr int HN_MAX_HD = 512;

// One wave per head: q's heads [0, nh), then k's. With a weight the head is
// RMS-normalized first (kernels/scalar/k_scalar.c:59-64: the squares summed
// in index order by one lane, inv = 1/sqrtf(ss/n + eps), then (x*inv)*w);
// then its pairs (2i, 2i+1) rotate by the tables' row *pos (k_scalar.c:79-94).
__global__ void __launch_bounds__(64) k_heads_norm_rope(float *q, float *k, const float *qw, const float *kw,
                                                        const float *cs, const float *sn, int hd, int nh, float eps,
                                                        const int *pos) {
    __shared__ float v[HN_MAX_HD];
    __shared__ float s_inv;
    const int h = (int)blockIdx.x, lane = (int)threadIdx.x;
    float *x = h < nh ? q + (size_t)h * hd : k + (size_t)(h - nh) * hd;
    const float *w = h < nh ? qw : kw;
    for (int i = lane; i < hd; i += 64) v[i] = x[i];
    __syncthreads();
    if (w) {
        if (lane == 0) {
            float ss = 0.0f;
            for (int i = 0; i < hd; i++) ss = kr_fadd(ss, kr_fmul(v[i], v[i]));
            s_inv = kr_fdiv(1.0f, kr_fsqrt(kr_fadd(kr_fdiv(ss, (float)hd), eps)));
        }
        __syncthreads();
        const float inv = s_inv;
        for (int i = lane; i < hd; i += 64) v[i] = kr_fmul(kr_fmul(v[i], inv), w[i]);
        __syncthreads();
    }
    const int h2 = hd >> 1;
    const size_t row = (size_t)*pos * h2;
    for (int i = lane; i < h2; i += 64) {
        const float c = cs[row + i], s = sn[row + i];
        const float a = v[2 * i], b = v[2 * i + 1];
        x[2 * i] = kr_fsub(kr_fmul(a, c), kr_fmul(b, s));
        x[2 * i + 1] = kr_fadd(kr_fmul(a, s), kr_fmul(b, c));
    }
}

// ops/ops.c:141: the scores of the positions attended become
// cap * tanhf(score / cap) before the softmax. Row (token z, head x) holds
// max_seq floats; its length follows from the position and the window as
// the score kernels count it.
__global__ void k_softcap_att(float *att, int max_seq, int window, const int *pos_p, float cap) {
    const int pos = *pos_p + (int)blockIdx.z;
    const int first = window && pos >= window ? pos + 1 - window : 0, n = pos + 1 - first;
    float *a = att + ((size_t)blockIdx.z * gridDim.x + blockIdx.x) * max_seq;
    for (int t = (int)threadIdx.x; t < n; t += (int)blockDim.x) a[t] = kr_fmul(cap, kr_tanhf(kr_fdiv(a[t], cap)));
}

__global__ void k_tanhf_range(float *y, unsigned lo, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = kr_tanhf(__uint_as_float(lo + (unsigned)i));
}

__global__ void k_store_rows_f32(float *kc, float *vc, const float *k, const float *v, int n, const int *pos) {
    const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) {
        const size_t r = (size_t)*pos * n;
        kc[r + i] = k[i];
        vc[r + i] = v[i];
    }
}

}  // namespace

extern "C" void krh_heads_norm_rope(float *q, float *k, const float *q_norm, const float *k_norm, const float *cos_t,
                                    const float *sin_t, int head_dim, int n_heads, int n_kv_heads, float eps,
                                    const int *pos) {
    if (head_dim <= 0 || head_dim > HN_MAX_HD || (head_dim & 1) || n_heads < 0 || n_kv_heads < 0 ||
        (!q_norm) != (!k_norm)) {
        kr_fail(ML_E_SHAPE, "heads_norm_rope shape", hipSuccess);
        return;
    }
    if (n_heads + n_kv_heads == 0) return;
    hipLaunchKernelGGL(k_heads_norm_rope, dim3(n_heads + n_kv_heads), dim3(64), 0, kr_stream(), q, k, q_norm, k_norm,
                       cos_t, sin_t, head_dim, n_heads, eps, pos);
    kr_check_launch("heads_norm_rope");
}

extern "C" void krh_store_rows_f32(float *kc, float *vc, const float *k, const float *v, int kv_dim, const int *pos) {
    if (kv_dim <= 0) {
        kr_fail(ML_E_SHAPE, "store_rows size", hipSuccess);
        return;
    }
    hipLaunchKernelGGL(k_store_rows_f32, dim3((kv_dim + 255) / 256), dim3(256), 0, kr_stream(), kc, vc, k, v, kv_dim,
                       pos);
    kr_check_launch("store_rows_f32");
}

extern "C" void krh_softcap_att(float *att, int n_heads, int max_seq, int window, const int *pos, int ntok,
                                float cap) {
    if (n_heads <= 0 || ntok <= 0 || !(cap > 0.0f)) {
        kr_fail(ML_E_SHAPE, "softcap_att shape", hipSuccess);
        return;
    }
    hipLaunchKernelGGL(k_softcap_att, dim3(n_heads, 1, ntok), dim3(256), 0, kr_stream(), att, max_seq, window, pos,
                       cap);
    kr_check_launch("softcap_att");
}

extern "C" void krh_tanhf_range(float *y, uint32_t lo, size_t n) {
    if (n == 0) return;
    hipLaunchKernelGGL(k_tanhf_range, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, kr_stream(), y, lo, n);
    kr_check_launch("tanhf_range");
}
