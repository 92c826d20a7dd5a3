/* CPU check of the op-table binding's per-token op queue
 * (isa-lm_amd/optable/kh_queue.h): random per-token stages of row ops over
 * one host "arena", made one call at a time on one copy and through
 * q_push / q_flush on the other, must leave both copies byte-identical.
 * The rows kernels are emulated on the host (any deterministic per-row
 * function will do: the check is the replay order, not the arithmetic).
 * Stages include planted cross-row hazards: an op that keeps reading one
 * row while a later op writes it, an op that reads the previous token's
 * row, shared scalars written by every token. Prints the failures and the
 * launch counts; exit status 1 on any difference.
 *
 *   queue_sim [trials] [mutate]
 * mutate = 1 replaces the overlap test by "never overlaps", which must make
 * some trial differ (the harness can see a wrong replay).
 *
 *   queue_sim meet [cases]
 * checks rows_meet against brute force over every pair of rows: never a
 * miss, and exact when the two strides are equal and non-zero.
 *
 *   queue_sim fuse [trials] [mutate]
 * one token's decode sequences (rmsnorm + quantize, q/k/v products + bias
 * adds + RoPE, w1/w3 products + silu_mul, a product + residual add, products
 * of one input; rmsnorm + quantize + q/k/v or w1/w3, quantize + product +
 * residual add) with random buffer choices, some of them aliased: the fused
 * launches (emulated as the calls they stand for) must leave the same bytes
 * as the calls one by one, and every pattern must fire in some trial.
 * mutate = 1 drops the aliasing checks of the patterns. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "krafla_hip.h"

static uint8_t *g_base;
static size_t g_size;
static int g_mutate;

/* the one registered range maps to itself */
static uint8_t *dev_addr(const void *p, size_t n) {
    const uint8_t *b = p;
    return b >= g_base && n <= g_size && (size_t)(b - g_base) <= g_size - n ? (uint8_t *)b : NULL;
}

static int meet_or_not(const uint8_t *A, ptrdiff_t sa, size_t la, const uint8_t *B, ptrdiff_t sb, size_t lb, int T);
static int fusable_or_not(int i, int k, const unsigned char (*link)[2], int nlink);
#define KH_ROWS_MEET meet_or_not
#define KH_FUSABLE fusable_or_not
#include "kh_queue.h"

static long g_fired[9];   /* rmsnorm_q8, qkv, swiglu, residual, multi, rmsnorm_q8 rows, norm+qkv, norm+swiglu,
                             quantize+residual */

static int fusable_or_not(int i, int k, const unsigned char (*link)[2], int nlink) {
    return g_mutate ? 1 : fusable(i, k, link, nlink);
}

static long g_launches;

/* the emulated arithmetic of one row (the rows stubs and the fused stubs
 * share it, so a fused launch's bytes equal the calls it stands for) */
static void sim_norm(float *out, const float *x, const float *w, int n, float eps) {
    float ss = 0;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    const float inv = 1.0f / sqrtf(ss / n + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}
static void sim_q8(int8_t *q, float *d, const float *x, int n) {
    for (int b = 0; b < n / 32; b++) {
        float m = 0;
        for (int i = 0; i < 32; i++) m = fmaxf(m, fabsf(x[b * 32 + i]));
        d[b] = m / 127;
        for (int i = 0; i < 32; i++) q[b * 32 + i] = (int8_t)(m > 0 ? roundf(x[b * 32 + i] * 127 / m) : 0);
    }
}

void krh_rmsnorm_rows(float *o, size_t ldo, const float *x, size_t ldx, const float *w, size_t ldw, int n, float eps,
                      int rows) {
    g_launches++;
    float tmp[1024];
    for (int r = 0; r < rows; r++) {
        sim_norm(tmp, x + r * ldx, w + r * ldw, n, eps);
        memcpy(o + r * ldo, tmp, sizeof(float) * n);
    }
}
void krh_add_rows(float *y, size_t ldy, const float *x, size_t ldx, int n, int rows) {
    g_launches++;
    for (int r = 0; r < rows; r++)
        for (int i = 0; i < n; i++) y[r * ldy + i] += x[r * ldx + i];
}
void krh_silu_mul_rows(float *g, size_t ldg, const float *u, size_t ldu, int n, int rows) {
    g_launches++;
    for (int r = 0; r < rows; r++)
        for (int i = 0; i < n; i++) g[r * ldg + i] = g[r * ldg + i] * 0.5f * u[r * ldu + i] + 1.0f;
}
void krh_gelu_mul_rows(float *g, size_t ldg, const float *u, size_t ldu, int n, int rows) {
    g_launches++;
    for (int r = 0; r < rows; r++)
        for (int i = 0; i < n; i++) g[r * ldg + i] = g[r * ldg + i] * 0.25f - u[r * ldu + i];
}
void krh_rope_rows(float *q, size_t ldq, float *k, size_t ldk, const float *c, size_t ldc, const float *s, size_t lds,
                   int hd, int nh, int nkv, int rows) {
    g_launches++;
    const int h2 = hd / 2;
    for (int r = 0; r < rows; r++)
        for (int p = 0; p < (nh + nkv) * h2; p++) {
            float *v = p < nh * h2 ? q + r * ldq + (p / h2) * hd : k + r * ldk + (p / h2 - nh) * hd;
            const int i = p % h2;
            const float a = v[2 * i], b = v[2 * i + 1];
            v[2 * i] = a * c[r * ldc + i] - b * s[r * lds + i];
            v[2 * i + 1] = a * s[r * lds + i] + b * c[r * ldc + i];
        }
}
void krh_quantize_row_rows(int8_t *q, size_t ldq, float *d, size_t ldd, const float *x, size_t ldx, int n, int rows) {
    g_launches++;
    for (int r = 0; r < rows; r++) {
        float m = 0;
        for (int i = 0; i < n; i++) m = fmaxf(m, fabsf(x[r * ldx + i]));
        d[r * ldd] = m / 127;
        for (int i = 0; i < n; i++) q[r * ldq + i] = (int8_t)(m > 0 ? roundf(x[r * ldx + i] * 127 / m) : 0);
    }
}
void krh_quantize_q8_rows(int8_t *q, size_t ldq, float *d, size_t ldd, const float *x, size_t ldx, int n, int rows) {
    g_launches++;
    if (ldq % 4 || ldx % 4 || ((uintptr_t)x & 15) || ((uintptr_t)q & 3)) {
        printf("quantize_q8 rows: misaligned\n");
        exit(2);
    }
    for (int r = 0; r < rows; r++) {
        int8_t qq[1024];
        float dd[32];
        sim_q8(qq, dd, x + r * ldx, n);
        memcpy(q + r * ldq, qq, (size_t)n);
        memcpy(d + r * ldd, dd, sizeof(float) * (n / 32));
    }
}

/* products: y[r] (+)= sum_c W[r][c] * x[c] * the two block scales (int8
 * weights, float scales; the arithmetic only has to be deterministic) */
static void mv(float *out, const krh_mat *W, const int8_t *xq, const float *xd) {
    const int8_t *q = W->q;
    const float *d = W->d;
    const int nb = W->cols / 32;
    for (int r = 0; r < W->rows; r++) {
        float acc = 0;
        for (int c = 0; c < W->cols; c++)
            acc += q[(size_t)r * W->cols + c] * xq[c] * d[(size_t)r * nb + c / 32] * xd[c / 32];
        out[r] = acc;
    }
}
void krh_matvec(float *y, const krh_mat *W, const int8_t *xq, const float *xd, int accumulate) {
    g_launches++;
    float out[1024];
    mv(out, W, xq, xd);
    for (int r = 0; r < W->rows; r++) y[r] = accumulate ? y[r] + out[r] : out[r];
}

/* The fused launches as a fused kernel behaves: every input read before any
 * output is written (so an aliasing the patterns should have refused gives
 * other bytes than the calls one by one). */
void krh_matvec_multi(float *const *y, const krh_mat *const *W, int nmat, const int8_t *xq, const float *xd) {
    g_fired[4]++;
    float out[3][1024];
    for (int i = 0; i < nmat; i++) mv(out[i], W[i], xq, xd);
    for (int i = 0; i < nmat; i++) memcpy(y[i], out[i], sizeof(float) * W[i]->rows);
}
void krh_matvec_residual(float *r, float *y, const krh_mat *W, const int8_t *xq, const float *xd) {
    g_fired[3]++;
    float out[1024], res[1024];
    mv(out, W, xq, xd);
    for (int i = 0; i < W->rows; i++) res[i] = r[i] + out[i];
    memcpy(y, out, sizeof(float) * W->rows);
    memcpy(r, res, sizeof(float) * W->rows);
}
void krh_matvec_swiglu_keep(float *h, float *u, const krh_mat *w1, const krh_mat *w3, const int8_t *xq,
                            const float *xd) {
    g_fired[2]++;
    float a[1024], b[1024];
    mv(a, w1, xq, xd);
    mv(b, w3, xq, xd);
    for (int i = 0; i < w1->rows; i++) a[i] = a[i] * 0.5f * b[i] + 1.0f;   /* krh_silu_mul_rows's stand-in */
    memcpy(h, a, sizeof(float) * w1->rows);
    memcpy(u, b, sizeof(float) * w3->rows);
}
void krh_matvec_qkv(float *q, float *kc, float *vc, const krh_mat *wq, const krh_mat *wk, const krh_mat *wv,
                    const float *bq, const float *bk, const float *bv, const int8_t *xq, const float *xd,
                    const float *rope_cos, const float *rope_sin, int head_dim, const int *pos) {
    g_fired[1]++;
    float o[3][1024], c[512], sn[512];
    mv(o[0], wq, xq, xd);
    mv(o[1], wk, xq, xd);
    mv(o[2], wv, xq, xd);
    const size_t off = (size_t)*pos * (head_dim / 2);
    memcpy(c, rope_cos + off, sizeof(float) * (head_dim / 2));
    memcpy(sn, rope_sin + off, sizeof(float) * (head_dim / 2));
    if (bq) {
        for (int i = 0; i < wq->rows; i++) o[0][i] += bq[i];
        for (int i = 0; i < wk->rows; i++) o[1][i] += bk[i];
        for (int i = 0; i < wv->rows; i++) o[2][i] += bv[i];
    }
    for (int m = 0; m < 2; m++)
        for (int p = 0; p < (m ? wk->rows : wq->rows) / 2; p++) {
            const int i = p % (head_dim / 2);
            const float a = o[m][2 * p], b = o[m][2 * p + 1];
            o[m][2 * p] = a * c[i] - b * sn[i];
            o[m][2 * p + 1] = a * sn[i] + b * c[i];
        }
    memcpy(q, o[0], sizeof(float) * wq->rows);
    memcpy(kc, o[1], sizeof(float) * wk->rows);
    memcpy(vc, o[2], sizeof(float) * wv->rows);
}
/* the keep forms: the norm and Q8_0 of x computed first, every output
 * written after every input is read */
void krh_rmsnorm_matvec_qkv_keep(float *q, float *k, float *v, const krh_mat *wq, const krh_mat *wk,
                                 const krh_mat *wv, const float *bq, const float *bk, const float *bv, const float *x,
                                 const float *nw, float eps, const float *rope_cos, const float *rope_sin,
                                 int head_dim, const int *pos, float *xb, int8_t *xq, float *xd) {
    g_fired[6]++;
    const int n = wq->cols;
    float o[1024], dd[32];
    int8_t qq[1024];
    sim_norm(o, x, nw, n, eps);
    sim_q8(qq, dd, o, n);
    float out[3][1024], c[512], sn[512];
    mv(out[0], wq, qq, dd);
    mv(out[1], wk, qq, dd);
    mv(out[2], wv, qq, dd);
    const size_t off = (size_t)*pos * (head_dim / 2);
    memcpy(c, rope_cos + off, sizeof(float) * (head_dim / 2));
    memcpy(sn, rope_sin + off, sizeof(float) * (head_dim / 2));
    if (bq) {
        for (int i = 0; i < wq->rows; i++) out[0][i] += bq[i];
        for (int i = 0; i < wk->rows; i++) out[1][i] += bk[i];
        for (int i = 0; i < wv->rows; i++) out[2][i] += bv[i];
    }
    for (int m = 0; m < 2; m++)
        for (int p = 0; p < (m ? wk->rows : wq->rows) / 2; p++) {
            const int i = p % (head_dim / 2);
            const float a = out[m][2 * p], b = out[m][2 * p + 1];
            out[m][2 * p] = a * c[i] - b * sn[i];
            out[m][2 * p + 1] = a * sn[i] + b * c[i];
        }
    memcpy(xb, o, sizeof(float) * n);
    memcpy(xq, qq, (size_t)n);
    memcpy(xd, dd, sizeof(float) * (n / 32));
    memcpy(q, out[0], sizeof(float) * wq->rows);
    memcpy(k, out[1], sizeof(float) * wk->rows);
    memcpy(v, out[2], sizeof(float) * wv->rows);
}
void krh_rmsnorm_matvec_swiglu_keep(float *h, float *u, const krh_mat *w1, const krh_mat *w3, const float *x,
                                    const float *nw, float eps, float *xb, int8_t *xq, float *xd) {
    g_fired[7]++;
    const int n = w1->cols;
    float o[1024], dd[32], a[1024], b[1024];
    int8_t qq[1024];
    sim_norm(o, x, nw, n, eps);
    sim_q8(qq, dd, o, n);
    mv(a, w1, qq, dd);
    mv(b, w3, qq, dd);
    for (int i = 0; i < w1->rows; i++) a[i] = a[i] * 0.5f * b[i] + 1.0f;
    memcpy(xb, o, sizeof(float) * n);
    memcpy(xq, qq, (size_t)n);
    memcpy(xd, dd, sizeof(float) * (n / 32));
    memcpy(h, a, sizeof(float) * w1->rows);
    memcpy(u, b, sizeof(float) * w3->rows);
}
void krh_matvec_f_residual_keep(float *r, float *y, const krh_mat *W, const float *x, int8_t *xq, float *xd) {
    g_fired[8]++;
    const int n = W->cols;
    float dd[32], out[1024], res[1024];
    int8_t qq[1024];
    sim_q8(qq, dd, x, n);
    mv(out, W, qq, dd);
    for (int i = 0; i < W->rows; i++) res[i] = r[i] + out[i];
    memcpy(xq, qq, (size_t)n);
    memcpy(xd, dd, sizeof(float) * (n / 32));
    memcpy(y, out, sizeof(float) * W->rows);
    memcpy(r, res, sizeof(float) * W->rows);
}

void krh_rmsnorm_q8(int8_t *q, float *d, float *xb, const float *x, const float *w, int n, float eps, int ntok) {
    g_fired[ntok > 1 ? 5 : 0]++;
    for (int t = 0; t < ntok; t++) {
        float o[1024], ss = 0, dd[32];
        int8_t qq[1024];
        for (int i = 0; i < n; i++) ss += x[(size_t)t * n + i] * x[(size_t)t * n + i];
        const float inv = 1.0f / sqrtf(ss / n + eps);
        for (int i = 0; i < n; i++) o[i] = x[(size_t)t * n + i] * inv * w[i];
        for (int b = 0; b < n / 32; b++) {
            float m = 0;
            for (int i = 0; i < 32; i++) m = fmaxf(m, fabsf(o[b * 32 + i]));
            dd[b] = m / 127;
            for (int i = 0; i < 32; i++) qq[b * 32 + i] = (int8_t)(m > 0 ? roundf(o[b * 32 + i] * 127 / m) : 0);
        }
        memcpy(xb + (size_t)t * n, o, sizeof(float) * n);
        memcpy(q + (size_t)t * n, qq, (size_t)n);
        memcpy(d + (size_t)t * (n / 32), dd, sizeof(float) * (n / 32));
    }
}

static int meet_or_not(const uint8_t *A, ptrdiff_t sa, size_t la, const uint8_t *B, ptrdiff_t sb, size_t lb, int T) {
    return g_mutate ? 0 : rows_meet(A, sa, la, B, sb, lb, T);
}

/* ---- the random stages ---- */

typedef struct {
    int op, n, a, b;
    size_t off[4];
} call;

static uint64_t g_rs;
static unsigned rnd(unsigned n) {
    g_rs ^= g_rs << 13;
    g_rs ^= g_rs >> 7;
    g_rs ^= g_rs << 17;
    return (unsigned)(g_rs % n);
}

static void run(int queued, uint8_t *base, const call *c) {
    float *f[4];
    for (int p = 0; p < 4; p++) f[p] = (float *)(base + c->off[p]);
    if (!queued) {
        kh_op o;
        memset(&o, 0, sizeof o);
        o.op = c->op;
        o.np = 4;
        o.n = c->n;
        o.a = c->a;
        o.b = c->b;
        o.f = 1e-5f;
        for (int p = 0; p < 4; p++) o.d[p] = (uint8_t *)f[p];
        launch(&o, NULL, 1);
        return;
    }
    const void *h[4] = { f[0], f[1], f[2], f[3] };
    size_t len[4] = { 0 };
    int wr[4] = { 0 }, np = 3;
    const int n = c->n;
    switch (c->op) {
    case QOP_RMSNORM: len[0] = len[1] = len[2] = 4 * (size_t)n; wr[0] = 1; break;
    case QOP_QUANT_Q8: len[0] = n; len[1] = 4 * (size_t)(n / 32); len[2] = 4 * (size_t)n; wr[0] = wr[1] = 1; break;
    case QOP_QUANT_ROW: len[0] = n; len[1] = 4; len[2] = 4 * (size_t)n; wr[0] = wr[1] = 1; break;
    case QOP_ROPE:
        np = 4;
        len[0] = 4 * (size_t)c->a * n;
        len[1] = 4 * (size_t)c->b * n;
        len[2] = len[3] = 4 * (size_t)(n / 2);
        wr[0] = wr[1] = 1;
        break;
    default: np = 2; len[0] = len[1] = 4 * (size_t)n; wr[0] = 1; break;
    }
    if (!q_push(c->op, c->n, c->a, c->b, 1e-5f, np, h, len, wr)) {
        printf("q_push refused op %d\n", c->op);
        exit(2);
    }
}

static int brute_meet(uintptr_t A, ptrdiff_t sa, size_t la, uintptr_t B, ptrdiff_t sb, size_t lb, int T) {
    for (int t = 0; t < T; t++)
        for (int u = 0; u < T; u++) {
            const uintptr_t a0 = A + (uintptr_t)(t * sa), b0 = B + (uintptr_t)(u * sb);
            if (t != u && a0 < b0 + lb && b0 < a0 + la) return 1;
        }
    return 0;
}

static int check_meet(long cases) {
    long miss = 0, inexact = 0;
    g_rs = 0x2545F4914F6CDD1Dull;
    for (long it = 0; it < cases; it++) {
        const int T = 2 + (int)rnd(9);
        const ptrdiff_t sa = rnd(5) == 0 ? 0 : (ptrdiff_t)rnd(40);
        const ptrdiff_t sb = rnd(3) == 0 ? sa : (ptrdiff_t)rnd(40);
        const size_t la = 1 + rnd(40), lb = 1 + rnd(40);
        const uintptr_t A = 100000 + rnd(300), B = 100000 + rnd(300);
        const int got = rows_meet((const uint8_t *)A, sa, la, (const uint8_t *)B, sb, lb, T);
        const int want = brute_meet(A, sa, la, B, sb, lb, T);
        miss += want && !got;
        inexact += !want && got && sa == sb && sa != 0;
    }
    printf("meet cases %ld misses %ld inexact %ld\n", cases, miss, inexact);
    return miss || inexact;
}

/* ---- one token's decode sequences ---- */

enum { FB = 24, FBUF = 4096 };   /* float buffers of FBUF bytes */

typedef struct {
    uint8_t *base;
    size_t fb, i8, d8, wq, wd, end;
} fuse_mem;

static float *fbuf(const fuse_mem *m, int b, int shift) { return (float *)(m->base + m->fb + (size_t)b * FBUF) + shift; }

/* buffer b; or, one time in den, buffer a itself or a shifted by 4 floats */
static int pick(int b, int a, int den, int *shift) {
    *shift = 0;
    if (den && rnd(den) == 0) {
        *shift = rnd(2) ? 4 : 0;
        return a;
    }
    return b;
}

static void push(int op, int n, int a, int b, float f, int np, const void *const *h, const size_t *l, const int *w) {
    if (!q_push(op, n, a, b, f, np, h, l, w)) {
        printf("q_push refused op %d\n", op);
        exit(2);
    }
}

static void seq_matvec(int queued, float *y, const krh_mat *W, const int8_t *xq, const float *xd) {
    if (!queued) {
        krh_matvec(y, W, xq, xd, 0);
        return;
    }
    const void *h[] = { y, xq, xd, W->q, W->d };
    const size_t l[] = { 4 * (size_t)W->rows, (size_t)W->cols, 4 * (size_t)(W->cols / 32),
                         (size_t)W->rows * W->cols, 4 * (size_t)W->rows * (W->cols / 32) };
    const int w[] = { 1, 0, 0, 0, 0 };
    push(QOP_MATVEC, W->rows, W->cols, ML_Q8_0, 0.0f, 5, h, l, w);
}

static void seq_add(int queued, float *y, const float *x, int n) {
    if (!queued) {
        krh_add_rows(y, 0, x, 0, n, 1);
        return;
    }
    const void *h[] = { y, x };
    const size_t l[] = { 4 * (size_t)n, 4 * (size_t)n };
    const int w[] = { 1, 0 };
    push(QOP_ADD, n, 0, 0, 0.0f, 2, h, l, w);
}

/* pattern: 0 rmsnorm + quantize, 1 q/k/v [+ biases] + rope, 2 w1/w3 +
 * silu_mul, 3 product + residual add, 4 products of one input */
static void one_seq(int queued, const fuse_mem *m, int pat, uint64_t seed) {   /* pat: 0..7 */
    g_rs = seed;
    const int K = 32 * (2 + (int)rnd(3)), hd = 16, nh = 2 + (int)rnd(3), nkv = 1 + (int)rnd(2), den = 4;
    int8_t *xq = (int8_t *)(m->base + m->i8);
    float *xd = (float *)(m->base + m->d8);
    krh_mat W[3];
    for (int i = 0; i < 3; i++)
        W[i] = (krh_mat){ m->base + m->wq + (size_t)i * 65536, m->base + m->wd + (size_t)i * 16384, 32, K, ML_Q8_0, 0 };
    int b[8], sh[8];
    for (int i = 0; i < 8; i++) {
        b[i] = (int)rnd(FB);
        sh[i] = 0;
    }
    if (pat == 0 || pat == 5 || pat == 6 || pat == 7) {
        /* rmsnorm into o and quantize_q8 of o into the products' input (5, 6),
         * or quantize_q8 of a float row alone (7) */
        const int n = K;
        int nb_[3], ns = 0;
        for (int i = 0; i < 3; i++) nb_[i] = (int)rnd(FB);
        nb_[0] = pick(nb_[0], nb_[1], den, &ns);
        float *o = fbuf(m, nb_[0], ns), *x = fbuf(m, nb_[1], 0), *w = fbuf(m, nb_[2], 0);
        int8_t *q = xq;
        float *d = rnd(den) ? xd : fbuf(m, nb_[1], 0);   /* sometimes the scales land on x */
        if (!queued) {
            if (pat != 7) krh_rmsnorm_rows(o, 0, x, 0, w, 0, n, 1e-5f, 1);
            krh_quantize_q8_rows(q, 0, d, 0, pat == 7 ? x : o, 0, n, 1);
        } else {
            if (pat != 7) {
                const void *h1[] = { o, x, w };
                const size_t l1[] = { 4 * (size_t)n, 4 * (size_t)n, 4 * (size_t)n };
                const int w1[] = { 1, 0, 0 };
                push(QOP_RMSNORM, n, 0, 0, 1e-5f, 3, h1, l1, w1);
            }
            const void *h2[] = { q, d, pat == 7 ? x : o };
            const size_t l2[] = { (size_t)n, 4 * (size_t)(n / 32), 4 * (size_t)n };
            const int w2[] = { 1, 1, 0 };
            push(QOP_QUANT_Q8, n, 0, 0, 0.0f, 3, h2, l2, w2);
        }
        if (pat == 0) return;
        if (d != xd) return;   /* the products read xq, xd: no chain to fuse */
        pat = pat == 5 ? 1 : pat == 6 ? 2 : 3;
    }
    const int nm = pat == 1 ? 3 : pat == 2 ? 2 : pat == 3 ? 1 : 2 + (int)rnd(2);
    if (pat == 1) {
        W[0].rows = nh * hd;
        W[1].rows = W[2].rows = nkv * hd;
    }
    b[1] = pick(b[1], b[0], den, &sh[1]);
    b[2] = pick(b[2], b[1], den, &sh[2]);
    float *y[3];
    for (int i = 0; i < nm; i++) {
        y[i] = fbuf(m, b[i], sh[i]);
        seq_matvec(queued, y[i], &W[i], xq, xd);
    }
    if (pat == 1) {
        if (rnd(2))
            for (int i = 0; i < 3; i++) {
                int s;
                const int bb = pick(b[3 + i], b[i], den, &s);
                seq_add(queued, y[i], fbuf(m, bb, bb == b[i] ? sh[i] + s : s), W[i].rows);
            }
        float *cs = fbuf(m, b[6], 0), *sn = fbuf(m, b[7], 0);
        if (!queued) {
            krh_rope_rows(y[0], 0, y[1], 0, cs, 0, sn, 0, hd, nh, nkv, 1);
        } else {
            const void *h[] = { y[0], y[1], cs, sn };
            const size_t l[] = { 4 * (size_t)nh * hd, 4 * (size_t)nkv * hd, 4 * (size_t)(hd / 2), 4 * (size_t)(hd / 2) };
            const int w[] = { 1, 1, 0, 0 };
            push(QOP_ROPE, hd, nh, nkv, 0.0f, 4, h, l, w);
        }
    } else if (pat == 2) {
        if (!queued) {
            krh_silu_mul_rows(y[0], 0, y[1], 0, W[0].rows, 1);
        } else {
            const void *h[] = { y[0], y[1] };
            const size_t l[] = { 4 * (size_t)W[0].rows, 4 * (size_t)W[0].rows };
            const int w[] = { 1, 0 };
            push(QOP_SILU_MUL, W[0].rows, 0, 0, 0.0f, 2, h, l, w);
        }
    } else if (pat == 3) {
        int s;
        const int r = pick(b[3], b[0], den, &s);
        seq_add(queued, fbuf(m, r, r == b[0] ? s : 0), y[0], W[0].rows);
    }
}

static int check_fuse(int trials) {
    static int zero = 0;
    fuse_mem mem[2];
    for (int side = 0; side < 2; side++) {
        fuse_mem *m = &mem[side];
        size_t o = 0;
        m->fb = o;
        o += (size_t)FB * FBUF;
        m->i8 = o;
        o += 1024;
        m->d8 = o;
        o += 1024;
        m->wq = o;
        o += 3 * 65536;
        m->wd = o;
        o += 3 * 16384;
        m->end = o;
        m->base = aligned_alloc(64, o);
    }
    g_base = mem[1].base;
    g_size = mem[1].end;
    g_qzero = &zero;
    int fails = 0;
    for (int trial = 0; trial < trials; trial++) {
        for (int side = 0; side < 2; side++) {
            const fuse_mem *m = &mem[side];
            uint64_t fill = 777 + (uint64_t)trial;
            for (size_t i = 0; i < m->end; i += 4) {
                fill = fill * 6364136223846793005ull + 1442695040888963407ull;
                float v = (float)((int)((fill >> 33) % 2001) - 1000) / 500.0f;
                if (i >= m->wd || (i >= m->d8 && i < m->wq)) v = 0.01f + fabsf(v) * 0.01f;   /* scales */
                memcpy(m->base + i, &v, 4);
            }
            for (size_t i = m->i8; i < m->d8; i++) m->base[i] = (uint8_t)(i * 37 + (size_t)trial);
            for (size_t i = m->wq; i < m->wd; i++) m->base[i] = (uint8_t)(i * 13 + (size_t)trial * 7);
        }
        const int pat = trial % 8;
        for (int side = 0; side < 2; side++) {
            one_seq(side, &mem[side], pat, 0xABCDEFull ^ (uint64_t)trial * 31);
            if (side) q_flush();
        }
        if (memcmp(mem[0].base, mem[1].base, mem[0].end)) {
            if (++fails <= 5) printf("fuse trial %d (pattern %d) differs\n", trial, pat);
        }
    }
    printf("fuse trials %d failures %d fired rmsnorm_q8 %ld qkv %ld swiglu %ld residual %ld multi %ld norm+qkv %ld "
           "norm+swiglu %ld quantize+residual %ld\n", trials, fails, g_fired[0], g_fired[1], g_fired[2], g_fired[3],
           g_fired[4], g_fired[6], g_fired[7], g_fired[8]);
    for (int i = 0; i < 9; i++)
        if (i != 5 && !g_fired[i]) {
            printf("pattern %d never fired\n", i);
            return 1;
        }
    return fails != 0;
}

int main(int argc, char **argv) {
    if (argc > 1 && !strcmp(argv[1], "meet")) return check_meet(argc > 2 ? atol(argv[2]) : 1000000);
    if (argc > 1 && !strcmp(argv[1], "fuse")) {
        g_mutate = argc > 3 && atoi(argv[3]);
        return check_fuse(argc > 2 ? atoi(argv[2]) : 5000);
    }

    const int trials = argc > 1 ? atoi(argv[1]) : 3000;
    g_mutate = argc > 2 && atoi(argv[2]);
    enum { ARENA = 1 << 22 };
    uint8_t *one = aligned_alloc(64, ARENA), *queued = aligned_alloc(64, ARENA);
    g_base = queued;
    g_size = ARENA;
    long calls = 0, launches = 0;
    int fails = 0;
    for (int trial = 0; trial < trials; trial++) {
        g_rs = 0x9E3779B97F4A7C15ull ^ (uint64_t)trial * 7919;
        const int T = 1 + rnd(40), W = 32 * (1 + rnd(4)), m = 1 + rnd(6), hazard = rnd(4) == 0;
        /* six row buffers [T][W] floats (ragged gaps between them), two shared
         * vectors, an int8 row buffer and a scale buffer */
        size_t rowbuf[6], shared[2], o = 0;
        for (int b = 0; b < 6; b++) {
            rowbuf[b] = o;
            o = (o + (size_t)4 * T * W + 64 * rnd(3) + 63) & ~(size_t)63;
        }
        for (int b = 0; b < 2; b++) {
            shared[b] = o;
            o = (o + (size_t)4 * W * 48 + 63) & ~(size_t)63;
        }
        const size_t i8 = o;
        o = (o + (size_t)T * W + 63) & ~(size_t)63;
        const size_t dbuf = o;
        o = (o + (size_t)4 * T * W + 63) & ~(size_t)63;
        call pat[8];
        for (int k = 0; k < m; k++) {
            call *c = &pat[k];
            memset(c, 0, sizeof *c);
            c->op = (int)rnd(7);
            c->n = W;
            const int b0 = (int)rnd(6), b1 = (int)rnd(6);
            switch (c->op) {
            case QOP_RMSNORM: c->off[0] = rowbuf[b0]; c->off[1] = rowbuf[b1]; c->off[2] = shared[rnd(2)]; break;
            case QOP_QUANT_Q8: case QOP_QUANT_ROW: c->off[0] = i8; c->off[1] = dbuf; c->off[2] = rowbuf[b1]; break;
            case QOP_ROPE:
                c->n = 16;
                c->a = W / 32;
                c->b = 1;
                c->off[0] = rowbuf[b0];
                c->off[1] = rowbuf[b0 == b1 ? (b1 + 1) % 6 : b1];
                c->off[2] = shared[0];
                c->off[3] = shared[1];
                break;
            default: c->off[0] = rowbuf[b0]; c->off[1] = rnd(3) ? rowbuf[b1] : shared[rnd(2)]; break;
            }
        }
        for (int side = 0; side < 2; side++) {
            uint8_t *base = side ? queued : one;
            uint64_t fill = 12345 + (uint64_t)trial;
            for (size_t i = 0; i < o / 4; i++) {
                fill = fill * 6364136223846793005ull + 1442695040888963407ull;
                ((float *)base)[i] = (float)((int)((fill >> 33) % 2001) - 1000) / 250.0f;
            }
            for (int t = 0; t < T; t++)
                for (int k = 0; k < m; k++) {
                    call c = pat[k];
                    for (int p = 0; p < 4; p++) {
                        int row = 0;
                        for (int b = 0; b < 6; b++) row |= c.off[p] == rowbuf[b];
                        size_t step = row ? (size_t)4 * W : 0;
                        if (c.off[p] == i8) step = c.op == QOP_QUANT_ROW ? (size_t)W : (size_t)W;
                        if (c.off[p] == dbuf) step = c.op == QOP_QUANT_ROW ? 4 : (size_t)4 * (W / 32);
                        if (hazard && k == 0 && p == 1 && row && t > 0) step = 0;   /* keeps reading row 0 */
                        c.off[p] += step * t;
                    }
                    int row1 = 0;
                    for (int b = 0; b < 6; b++) row1 |= pat[k].off[1] == rowbuf[b];
                    if (hazard && k == m - 1 && c.op == QOP_ADD && row1 && c.off[1] >= pat[k].off[1] + 4 * W)
                        c.off[1] -= 4 * (size_t)W;   /* reads the previous token's row */
                    if (c.op == QOP_ROPE) {   /* position tables; hazard: one shared cos row */
                        c.off[2] += hazard ? 0 : 32 * (size_t)t;
                        c.off[3] += 32 * (size_t)t;
                    }
                    run(side, base, &c);
                    calls += side == 0;
                }
            if (side) {
                const long before = g_launches;
                q_flush();
                launches += g_launches - before;
            }
        }
        if (memcmp(one, queued, o)) {
            if (++fails <= 5) printf("trial %d differs (rows %d, period %d, hazard %d)\n", trial, T, m, hazard);
        }
    }
    printf("trials %d failures %d calls %ld queued launches %ld\n", trials, fails, calls, launches);
    if (!g_mutate && !g_fired[5]) {
        printf("no run fused rmsnorm and quantize_q8\n");
        return 1;
    }
    return fails != 0;
}
