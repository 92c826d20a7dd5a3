// The reference's unfused kernels as device ops, one launch each, for the
// op-table binding (ml_k_<op>_hip under config/ml_config.h): every kernel in
// the scalar kernel's float order (kernels/scalar/k_scalar.c), so an
// unchanged model/transformer.c gets the scalar build's bits.
#include "kr_internal.h"
#include "kr_chain.h"
#include "kr_numerics.h"

namespace {

constexpr int OP_T = 256;

// o = (x * inv) * w, inv = 1 / sqrtf(ss / n + eps), ss = sum x_i * x_i in
// index order (k_scalar.c:59-64). One workgroup per row (row r at o + r*ldo,
// x + r*ldx, w + r*ldw). SPEC: the squares go to LDS in kr_spec_sum's chunk
// layout and the workgroup computes the ordered sum together (the same bits
// as the one-lane loop); else lane 0 adds them one by one (rows whose LDS
// need passes 64 KB). o may alias x: each element is read and written by the
// same thread.
template <bool SPEC>
__global__ void __launch_bounds__(OP_T) k_rmsnorm(float *o, size_t ldo, const float *x, size_t ldx, const float *w,
                                                  size_t ldw, int n, float eps) {
    extern __shared__ __align__(16) float sq[];
    __shared__ float s_inv;
    const size_t r = blockIdx.x;
    o += r * ldo;
    x += r * ldx;
    w += r * ldw;
    const int tid = threadIdx.x;
    float inv;
    if (SPEC) {
        const int sh = sc_log_len(n);
        for (int i = tid; i < n; i += OP_T) sq[sc_at(i, sh)] = kr_fmul(x[i], x[i]);
        __syncthreads();
        const float ss = kr_spec_sum<OP_T>(sq, n, (unsigned char *)(sq + sc_terms_cap(n)));
        inv = kr_fdiv(1.0f, kr_fsqrt(kr_fadd(kr_fdiv(ss, (float)n), eps)));
    } else {
        for (int i = tid; i < n; i += OP_T) sq[i] = kr_fmul(x[i], x[i]);
        __syncthreads();
        if (tid == 0) {
            float ss = 0.0f;
            for (int i = 0; i < n; i++) ss = kr_fadd(ss, sq[i]);
            s_inv = kr_fdiv(1.0f, kr_fsqrt(kr_fadd(kr_fdiv(ss, (float)n), eps)));
        }
        __syncthreads();
        inv = s_inv;
    }
    for (int i = tid; i < n; i += OP_T) o[i] = kr_fmul(kr_fmul(x[i], inv), w[i]);
}

// The elementwise ops below take row r = blockIdx.y of a batch of rows,
// each pointer with its own row stride (0: the same vector for every row).

__global__ void k_add(float *y, size_t ldy, const float *x, size_t ldx, int n) {   // k_scalar.c:107-109
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const size_t r = blockIdx.y;
    if (i < n) y[r * ldy + i] = kr_fadd(y[r * ldy + i], x[r * ldx + i]);
}

// pairs (2i, 2i+1) of every head of q (nh heads) and k (nkv heads):
// (a c - b s, a s + b c) (k_scalar.c:79-94)
__global__ void k_rope(float *q, size_t ldq, float *k, size_t ldk, const float *c, size_t ldc, const float *s,
                       size_t lds, int hd, int nh, int nkv) {
    const int p = blockIdx.x * blockDim.x + threadIdx.x, h2 = hd / 2;
    if (p >= (nh + nkv) * h2) return;
    const size_t r = blockIdx.y;
    c += r * ldc;
    s += r * lds;
    float *v = p < nh * h2 ? q + r * ldq + (size_t)(p / h2) * hd : k + r * ldk + (size_t)(p / h2 - nh) * hd;
    const int i = p % h2;
    const float a = v[2 * i], b = v[2 * i + 1];
    v[2 * i] = kr_fsub(kr_fmul(a, c[i]), kr_fmul(b, s[i]));
    v[2 * i + 1] = kr_fadd(kr_fmul(a, s[i]), kr_fmul(b, c[i]));
}

__global__ void k_silu_mul(float *g, size_t ldg, const float *u, size_t ldu, int n) {   // k_scalar.c:96-98
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const size_t r = blockIdx.y;
    if (i >= n) return;
    g += r * ldg;
    g[i] = kr_fmul(kr_fdiv(g[i], kr_fadd(1.0f, kr_expf(-g[i]))), u[r * ldu + i]);
}

// k_scalar.c:100-105, with the C library's tanhf (kr_tanhf)
__global__ void k_gelu_mul(float *g, size_t ldg, const float *u, size_t ldu, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const size_t r = blockIdx.y;
    if (i >= n) return;
    g += r * ldg;
    const float x = g[i];
    const float c = kr_fmul(kr_fmul(kr_fmul(0.044715f, x), x), x);
    const float t = kr_tanhf(kr_fmul(0.7978845608f, kr_fadd(x, c)));
    g[i] = kr_fmul(kr_fmul(kr_fmul(0.5f, x), kr_fadd(1.0f, t)), u[r * ldu + i]);
}

// k_scalar.c:66-77: max, expf(x - max), the sum in index order, x * (1/sum);
// all -inf: 1/n
__global__ void __launch_bounds__(OP_T) k_softmax(float *x, int n) {
    __shared__ float red[OP_T / 64];
    __shared__ float s_inv;
    const int tid = threadIdx.x;
    float m = -INFINITY;
    for (int i = tid; i < n; i += OP_T) m = fmaxf(m, x[i]);
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    float mx = red[0];
    for (int k = 1; k < OP_T / 64; k++) mx = fmaxf(mx, red[k]);
    if (mx == -INFINITY) {
        for (int i = tid; i < n; i += OP_T) x[i] = kr_fdiv(1.0f, (float)n);
        return;
    }
    for (int i = tid; i < n; i += OP_T) x[i] = kr_expf(kr_fsub(x[i], mx));
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        for (int i = 0; i < n; i++) sum = kr_fadd(sum, x[i]);
        s_inv = kr_fdiv(1.0f, sum);
    }
    __syncthreads();
    for (int i = tid; i < n; i += OP_T) x[i] = kr_fmul(x[i], s_inv);
}

// s[t] = (sum_i q_i k_t,i in index order) * scale (k_scalar.c:111-117)
__global__ void k_dot_rows(float *s, const float *q, const float *k, size_t ldk, int rows, int n, float scale) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows) return;
    const float *kt = k + (size_t)t * ldk;
    float acc = 0.0f;
    for (int i = 0; i < n; i++) acc = kr_fadd(acc, kr_fmul(q[i], kt[i]));
    s[t] = kr_fmul(acc, scale);
}

// y[i] += a[t] * x_t,i for t in order (k_scalar.c:119-122)
__global__ void k_axpy_rows(float *y, const float *a, const float *x, size_t ldx, int rows, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float o = y[i];
    for (int t = 0; t < rows; t++) o = kr_fadd(o, kr_fmul(a[t], x[(size_t)t * ldx + i]));
    y[i] = o;
}

// one scale over n values (ops/ops.c:81-96): the quantize_q8 rule; one
// workgroup per row
__global__ void __launch_bounds__(OP_T) k_quantize_row(int8_t *q, size_t ldq, float *d, size_t ldd,
                                                       const float *x, size_t ldx, int n) {
    __shared__ float red[OP_T / 64];
    const size_t r = blockIdx.x;
    q += r * ldq;
    d += r * ldd;
    x += r * ldx;
    const int tid = threadIdx.x;
    float m = 0.0f;
    for (int i = tid; i < n; i += OP_T) m = fmaxf(m, fabsf(x[i]));
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    float amax = red[0];
    for (int k = 1; k < OP_T / 64; k++) amax = fmaxf(amax, red[k]);
    if (amax < KR_QUANT_TINY) {
        if (tid == 0) *d = 0.0f;
        for (int i = tid; i < n; i += OP_T) q[i] = 0;
        return;
    }
    const float id = kr_fdiv(127.0f, amax);
    if (tid == 0) *d = kr_fdiv(amax, 127.0f);
    for (int i = tid; i < n; i += OP_T) q[i] = (int8_t)kr_q8_elem(x[i], id);
}

// x = cap * tanhf(x / cap) (ops/ops.c:98-101; the C library's tanhf)
__global__ void k_softcap(float *x, size_t ld, int rows, int n, float cap) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= (size_t)rows * n) return;
    float *p = x + (e / n) * ld + e % n;
    *p = kr_fmul(cap, kr_tanhf(kr_fdiv(*p, cap)));
}

__global__ void k_set_int(int *dst, int v) { *dst = v; }

unsigned blocks(size_t n) { return (unsigned)((n + OP_T - 1) / OP_T); }

}  // namespace

static bool rows_ok(int rows, const char *what) {
    if (rows >= 0 && rows <= KRH_ROWS_MAX) return true;
    kr_fail(ML_E_SHAPE, what, hipSuccess);
    return false;
}

extern "C" void krh_rmsnorm(float *o, const float *x, const float *w, int n, float eps) {
    krh_rmsnorm_rows(o, 0, x, 0, w, 0, n, eps, 1);
}
extern "C" void krh_rmsnorm_rows(float *o, size_t ldo, const float *x, size_t ldx, const float *w, size_t ldw, int n,
                                 float eps, int rows) {
    if (n <= 0 || n > 16384) { kr_fail(ML_E_SHAPE, "rmsnorm size", hipSuccess); return; }
    if (!rows_ok(rows, "rmsnorm rows") || rows == 0) return;
    const size_t spec = sizeof(float) * (size_t)sc_terms_cap(n) + sc_lds_bytes(n, OP_T);
    if (spec <= 64 * 1024)
        hipLaunchKernelGGL(k_rmsnorm<true>, dim3(rows), dim3(OP_T), spec, kr_stream(), o, ldo, x, ldx, w, ldw, n, eps);
    else
        hipLaunchKernelGGL(k_rmsnorm<false>, dim3(rows), dim3(OP_T), sizeof(float) * (size_t)n, kr_stream(), o, ldo, x,
                           ldx, w, ldw, n, eps);
    kr_check_launch("rmsnorm");
}
// Plain HBM read rate (a measurement op): every 16-byte word of p read once,
// UNROLL loads in flight per thread, XOR-folded into one word per workgroup
// (out[blockIdx.x]) so that no load is dropped.
constexpr int SR_T = 256, SR_UNROLL = 8;
__global__ void __launch_bounds__(SR_T) k_stream_read(unsigned *out, const int4 *p, size_t n16) {
    __shared__ unsigned red[SR_T / 64];
    const size_t stride = (size_t)gridDim.x * SR_T;
    size_t i = (size_t)blockIdx.x * SR_T + threadIdx.x;
    unsigned acc = 0;
    for (; i + (SR_UNROLL - 1) * stride < n16; i += SR_UNROLL * stride) {
        int4 v[SR_UNROLL];
#pragma unroll
        for (int k = 0; k < SR_UNROLL; k++) v[k] = p[i + k * stride];
#pragma unroll
        for (int k = 0; k < SR_UNROLL; k++) acc ^= (unsigned)(v[k].x ^ v[k].y ^ v[k].z ^ v[k].w);
    }
    for (; i < n16; i += stride) {
        const int4 v = p[i];
        acc ^= (unsigned)(v.x ^ v.y ^ v.z ^ v.w);
    }
    for (int o = 32; o >= 1; o >>= 1) acc ^= __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

extern "C" void krh_stream_read(unsigned *out, const void *p, size_t bytes, int grid) {
    if (bytes % 16 || grid <= 0 || ((uintptr_t)p & 15)) {
        kr_fail(ML_E_SHAPE, "stream_read: 16-byte aligned bytes and a positive grid", hipSuccess);
        return;
    }
    hipLaunchKernelGGL(k_stream_read, dim3(grid), dim3(SR_T), 0, kr_stream(), out, (const int4 *)p, bytes / 16);
    kr_check_launch("stream_read");
}

// Int8 MFMA issue rate (a measurement op): every wave runs iters rounds of
// four independent v_mfma_i32_32x32x32_i8 accumulations (65,536 int8
// operations each) on register operands, then stores one word per wave
// (out[wave]) so that no MFMA is dropped.
__global__ void __launch_bounds__(256) k_mfma_rate(int *out, int iters) {
    typedef int v4i __attribute__((ext_vector_type(4)));
    typedef int v16i __attribute__((ext_vector_type(16)));
    const int tid = threadIdx.x;
    const v4i a = v4i{ tid, tid * 3 + 1, tid ^ 0x55, tid + 7 }, b = v4i{ tid * 5, tid + 11, ~tid, tid * 7 + 2 };
    v16i c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int i = 0; i < iters; i++) {
        c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, a, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, a, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, b, c3, 0, 0, 0);
    }
    int v = 0;
#pragma unroll
    for (int r = 0; r < 16; r++) v ^= c0[r] + c1[r] + c2[r] + c3[r];
    for (int o = 32; o >= 1; o >>= 1) v ^= __shfl_xor(v, o);
    if ((tid & 63) == 0) out[blockIdx.x * 4 + (tid >> 6)] = v;
}

extern "C" void krh_mfma_rate(int *out, int grid, int iters) {
    if (grid <= 0 || iters <= 0) {
        kr_fail(ML_E_SHAPE, "mfma_rate: a positive grid and iteration count", hipSuccess);
        return;
    }
    hipLaunchKernelGGL(k_mfma_rate, dim3(grid), dim3(256), 0, kr_stream(), out, iters);
    kr_check_launch("mfma_rate");
}

extern "C" void krh_add(float *y, const float *x, int n) { krh_add_rows(y, 0, x, 0, n, 1); }
extern "C" void krh_add_rows(float *y, size_t ldy, const float *x, size_t ldx, int n, int rows) {
    if (n <= 0 || !rows_ok(rows, "add rows") || rows == 0) return;
    hipLaunchKernelGGL(k_add, dim3(blocks(n), rows), dim3(OP_T), 0, kr_stream(), y, ldy, x, ldx, n);
    kr_check_launch("add");
}
extern "C" void krh_rope(float *q, float *k, const float *cos_t, const float *sin_t, int head_dim, int n_heads,
                         int n_kv_heads) {
    krh_rope_rows(q, 0, k, 0, cos_t, 0, sin_t, 0, head_dim, n_heads, n_kv_heads, 1);
}
extern "C" void krh_rope_rows(float *q, size_t ldq, float *k, size_t ldk, const float *cos_t, size_t ldc,
                              const float *sin_t, size_t lds, int head_dim, int n_heads, int n_kv_heads, int rows) {
    const size_t n = (size_t)(n_heads + n_kv_heads) * (head_dim / 2);
    if (n == 0 || !rows_ok(rows, "rope rows") || rows == 0) return;
    hipLaunchKernelGGL(k_rope, dim3(blocks(n), rows), dim3(OP_T), 0, kr_stream(), q, ldq, k, ldk, cos_t, ldc, sin_t,
                       lds, head_dim, n_heads, n_kv_heads);
    kr_check_launch("rope");
}
extern "C" void krh_silu_mul(float *g, const float *u, int n) { krh_silu_mul_rows(g, 0, u, 0, n, 1); }
extern "C" void krh_silu_mul_rows(float *g, size_t ldg, const float *u, size_t ldu, int n, int rows) {
    if (n <= 0 || !rows_ok(rows, "silu_mul rows") || rows == 0) return;
    hipLaunchKernelGGL(k_silu_mul, dim3(blocks(n), rows), dim3(OP_T), 0, kr_stream(), g, ldg, u, ldu, n);
    kr_check_launch("silu_mul");
}
extern "C" void krh_gelu_mul(float *g, const float *u, int n) { krh_gelu_mul_rows(g, 0, u, 0, n, 1); }
extern "C" void krh_gelu_mul_rows(float *g, size_t ldg, const float *u, size_t ldu, int n, int rows) {
    if (n <= 0 || !rows_ok(rows, "gelu_mul rows") || rows == 0) return;
    hipLaunchKernelGGL(k_gelu_mul, dim3(blocks(n), rows), dim3(OP_T), 0, kr_stream(), g, ldg, u, ldu, n);
    kr_check_launch("gelu_mul");
}
extern "C" void krh_softmax(float *x, int n) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_softmax, dim3(1), dim3(OP_T), 0, kr_stream(), x, n);
    kr_check_launch("softmax");
}
extern "C" void krh_dot_rows(float *s, const float *q, const float *k, size_t ldk, int rows, int n, float scale) {
    if (rows <= 0) return;
    hipLaunchKernelGGL(k_dot_rows, dim3(blocks(rows)), dim3(OP_T), 0, kr_stream(), s, q, k, ldk, rows, n, scale);
    kr_check_launch("dot_rows");
}
extern "C" void krh_axpy_rows(float *y, const float *a, const float *x, size_t ldx, int rows, int n) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_axpy_rows, dim3(blocks(n)), dim3(OP_T), 0, kr_stream(), y, a, x, ldx, rows, n);
    kr_check_launch("axpy_rows");
}
extern "C" void krh_quantize_row(int8_t *q, float *d, const float *x, int n) {
    krh_quantize_row_rows(q, 0, d, 0, x, 0, n, 1);
}
extern "C" void krh_quantize_row_rows(int8_t *q, size_t ldq, float *d, size_t ldd, const float *x, size_t ldx, int n,
                                      int rows) {
    if (n <= 0 || !rows_ok(rows, "quantize_row rows") || rows == 0) return;
    hipLaunchKernelGGL(k_quantize_row, dim3(rows), dim3(OP_T), 0, kr_stream(), q, ldq, d, ldd, x, ldx, n);
    kr_check_launch("quantize_row");
}
extern "C" void krh_softcap_rows(float *x, size_t ld, int rows, int n, float cap) {
    const size_t e = (size_t)rows * n;
    if (e == 0) return;
    hipLaunchKernelGGL(k_softcap, dim3(blocks(e)), dim3(OP_T), 0, kr_stream(), x, ld, rows, n, cap);
    kr_check_launch("softcap");
}
extern "C" void krh_set_int(int *dst, int value) {
    hipLaunchKernelGGL(k_set_int, dim3(1), dim3(1), 0, kr_stream(), dst, value);
    kr_check_launch("set_int");
}
