/* The per-token op queue of the ISA=hip op-table binding (ml_hip.c, which
 * includes this file once, after defining dev_addr: the HBM address of a
 * host address range, or NULL). Static functions only.
 *
 * model/transformer.c's batched step runs each per-token stage as a loop
 * over the step's tokens (token_task, :366-369): one op call per token, about
 * a dozen launches per token and layer. Here the row ops whose buffers all
 * have an HBM copy are held in a queue, which is replayed before any other
 * call (a matrix product, attention, a copy, a status read). Replay cuts the
 * queue into runs: T >= 2 repetitions of one sequence of m calls, with equal
 * signatures (op, sizes, scalars) and addresses that advance by a fixed
 * stride per repetition, where no repetition writes memory that another one
 * reads or writes. Each of a run's m calls is launched once over T rows
 * (krh_<op>_rows); any other call is launched on its own, in queue order. A
 * row's calls keep their order and rows share no written memory, so the bits
 * are those of the calls made one by one.
 *
 * Matrix-vector products on arena buffers are queued too (not the
 * classifier's, whose logits the host reads at once), and short sequences of
 * single calls that model/transformer.c makes for one token are launched as
 * one fused kernel with the same effects on memory, every intermediate
 * buffer included (fuse_at):
 *   rmsnorm + quantize_q8 + q, k, v [+ biases]
 *     + RoPE                                     krh_rmsnorm_matvec_qkv_keep
 *   rmsnorm + quantize_q8 + w1, w3 + silu_mul    krh_rmsnorm_matvec_swiglu_keep
 *   quantize_q8 of x + its product + the add
 *     of the product into a residual             krh_matvec_f_residual_keep
 *   rmsnorm into o, quantize_q8 of o             krh_rmsnorm_q8 (also for runs)
 *   ml_matvec q, k, v [+ bias adds] + rope       krh_matvec_qkv (:273-281)
 *   ml_matvec w1, w3 + silu_mul                  krh_matvec_swiglu_keep (:290-293)
 *   ml_matvec into y + add of y into r           krh_matvec_residual (:284-287)
 *   2 or 3 ml_matvec of one input                krh_matvec_multi
 * A pattern applies only when the buffers it writes are apart from every
 * other buffer it touches (the same address for the same role excepted). */
#ifndef KH_QUEUE_H
#define KH_QUEUE_H

#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { QOP_RMSNORM, QOP_QUANT_Q8, QOP_ADD, QOP_SILU_MUL, QOP_GELU_MUL, QOP_ROPE, QOP_QUANT_ROW, QOP_MATVEC };

#define KH_NP 5
typedef struct {
    int op, np, n, a, b;   /* n: row length (rope: head_dim; matvec: rows); rope: a, b = n_heads, n_kv_heads */
    float f;               /* rmsnorm: eps */
    uint8_t *d[KH_NP];     /* device addresses of the pointer arguments (matvec: y, xq, xd, W's q, W's d) */
    size_t len[KH_NP];     /* bytes each one spans */
    int wr[KH_NP];         /* written (or read and written) */
    krh_mat m;             /* matvec: the matrix, device addresses */
} kh_op;

#define KH_QUEUE 65536
#define KH_PERIOD_MAX 256
static kh_op *g_q;
static int g_nq;
static ptrdiff_t g_st[KH_PERIOD_MAX][KH_NP], g_best[KH_PERIOD_MAX][KH_NP];   /* byte strides of a run's calls */
static const int *g_qzero;   /* a device int holding 0: the row of the RoPE tables krh_matvec_qkv reads */

static int same_sig(const kh_op *x, const kh_op *y) {
    if (x->op == QOP_MATVEC || y->op == QOP_MATVEC) return 0;   /* matrix products never form runs */
    if (x->op != y->op || x->np != y->np || x->n != y->n || x->a != y->a || x->b != y->b ||
        memcmp(&x->f, &y->f, sizeof x->f))
        return 0;
    for (int p = 0; p < x->np; p++)
        if (x->len[p] != y->len[p] || x->wr[p] != y->wr[p]) return 0;
    return 1;
}

/* bytes per element of argument p: the int8 outputs of the quantizers, else float */
static ptrdiff_t elem(const kh_op *o, int p) { return (o->op == QOP_QUANT_Q8 || o->op == QOP_QUANT_ROW) && p == 0 ? 1 : 4; }

/* strides a rows kernel takes: non-negative whole elements; quantize_q8
 * also keeps its int stores and float4 loads aligned */
static int strides_ok(const kh_op *o, const ptrdiff_t *st) {
    for (int p = 0; p < o->np; p++)
        if (st[p] < 0 || st[p] % elem(o, p)) return 0;
    return o->op != QOP_QUANT_Q8 || (st[0] % 4 == 0 && st[2] % 16 == 0);
}

static ptrdiff_t floor_div(ptrdiff_t a, ptrdiff_t b) { return a / b - (a % b != 0 && (a < 0) != (b < 0)); }

/* Whether [A + t*sa, A + t*sa + la) and [B + u*sb, B + u*sb + lb) meet for
 * some rows t != u in [0, T), strides >= 0; unequal strides count as
 * meeting unless the rows' hulls are apart. */
static int rows_meet(const uint8_t *A, ptrdiff_t sa, size_t la, const uint8_t *B, ptrdiff_t sb, size_t lb, int T) {
    const uintptr_t a0 = (uintptr_t)A, a1 = a0 + (uintptr_t)(sa * (T - 1)) + la;
    const uintptr_t b0 = (uintptr_t)B, b1 = b0 + (uintptr_t)(sb * (T - 1)) + lb;
    if (a1 <= b0 || b1 <= a0) return 0;
    if (sa != sb || sa == 0) return 1;
    /* rows t and u = t - d meet iff -la < (A - B) + d*s < lb, for d != 0, |d| < T */
    const ptrdiff_t D = (ptrdiff_t)(a0 - b0);
    ptrdiff_t lo = floor_div(-(ptrdiff_t)la - D, sa) + 1, hi = -floor_div(D - (ptrdiff_t)lb, sa) - 1;
    if (lo < 1 - T) lo = 1 - T;
    if (hi > T - 1) hi = T - 1;
    return lo <= hi && !(lo == 0 && hi == 0);
}

/* the overlap test a run must pass (a CPU check of the replay substitutes
 * its own to show that a wrong one is caught) */
#ifndef KH_ROWS_MEET
#define KH_ROWS_MEET rows_meet
#endif

/* one queued call (st NULL) or call k of a run over T rows */
static void launch(const kh_op *o, const ptrdiff_t *st, int T) {
    float *f[KH_NP];
    size_t ld[KH_NP] = { 0 };
    for (int p = 0; p < o->np; p++) {
        f[p] = (float *)o->d[p];
        if (st) ld[p] = (size_t)(st[p] / elem(o, p));
    }
    switch (o->op) {
    case QOP_RMSNORM: krh_rmsnorm_rows(f[0], ld[0], f[1], ld[1], f[2], ld[2], o->n, o->f, T); break;
    case QOP_QUANT_Q8: krh_quantize_q8_rows((int8_t *)o->d[0], ld[0], f[1], ld[1], f[2], ld[2], o->n, T); break;
    case QOP_ADD: krh_add_rows(f[0], ld[0], f[1], ld[1], o->n, T); break;
    case QOP_SILU_MUL: krh_silu_mul_rows(f[0], ld[0], f[1], ld[1], o->n, T); break;
    case QOP_GELU_MUL: krh_gelu_mul_rows(f[0], ld[0], f[1], ld[1], o->n, T); break;
    case QOP_ROPE: krh_rope_rows(f[0], ld[0], f[1], ld[1], f[2], ld[2], f[3], ld[3], o->n, o->a, o->b, T); break;
    case QOP_QUANT_ROW: krh_quantize_row_rows((int8_t *)o->d[0], ld[0], f[1], ld[1], f[2], ld[2], o->n, T); break;
    case QOP_MATVEC: krh_matvec(f[0], &o->m, (const int8_t *)o->d[1], f[2], 0); break;
    }
}

/* ---- fusion ---- */

/* Whether ops [i, i + k) may run as one fused kernel: argument pairs named
 * in link (op offset and argument index of each end: 16 * j + p) are one
 * buffer passed along (same address and length required); every other pair
 * of arguments, one of them written, must be apart. */
#define KH_FUSE_OPS 12   /* calls in one fused pattern, at most */
static int fusable(int i, int k, const unsigned char (*link)[2], int nlink) {
    int cls[KH_FUSE_OPS * 16];
    if (k > KH_FUSE_OPS) return 0;
    for (int e = 0; e < KH_FUSE_OPS * 16; e++) cls[e] = e;
    for (int l = 0; l < nlink; l++) {
        const int a = link[l][0], b = link[l][1];
        const kh_op *x = &g_q[i + (a >> 4)], *y = &g_q[i + (b >> 4)];
        if (x->d[a & 15] != y->d[b & 15] || x->len[a & 15] != y->len[b & 15]) return 0;
        const int ca = cls[a], cb = cls[b];
        for (int e = 0; e < KH_FUSE_OPS * 16; e++)
            if (cls[e] == cb) cls[e] = ca;
    }
    for (int ja = 0; ja < k; ja++)
        for (int pa = 0; pa < g_q[i + ja].np; pa++) {
            const kh_op *x = &g_q[i + ja];
            if (!x->wr[pa]) continue;
            for (int jb = 0; jb < k; jb++)
                for (int pb = 0; pb < g_q[i + jb].np; pb++) {
                    const kh_op *y = &g_q[i + jb];
                    if (cls[16 * ja + pa] == cls[16 * jb + pb]) continue;
                    if (x->d[pa] < y->d[pb] + y->len[pb] && y->d[pb] < x->d[pa] + x->len[pa]) return 0;
                }
        }
    return 1;
}

#define KH_L(j, p) (unsigned char)(16 * (j) + (p))

/* the aliasing test a fusion must pass (a CPU check of the replay
 * substitutes its own to show that a wrong one is caught) */
#ifndef KH_FUSABLE
#define KH_FUSABLE fusable
#endif

static int is_op(int i, int op) { return i < g_nq && g_q[i].op == op; }

/* matvec j reads the input of matvec i */
static int same_input(int i, int j) {
    return g_q[i].d[1] == g_q[j].d[1] && g_q[i].d[2] == g_q[j].d[2] && g_q[i].m.cols == g_q[j].m.cols;
}

static int same_kind(const krh_mat *a, const krh_mat *b) {
    return a->cols == b->cols && a->type == b->type && a->d16 == b->d16;
}

/* rmsnorm rows feeding quantize_q8 rows through o, as krh_rmsnorm_q8 lays
 * them out (rows of n, scales rows of n / 32, one weight row); st: the two
 * calls' row strides (NULL: one row) */
static int norm_q8_ok(const kh_op *nm, const kh_op *qz, const ptrdiff_t *sn, const ptrdiff_t *sq) {
    const int n = nm->n;
    if (qz->d[2] != nm->d[0] || qz->n != n || n % 32 || n > 8192) return 0;
    if (((uintptr_t)nm->d[0] | (uintptr_t)nm->d[1] | (uintptr_t)nm->d[2]) & 15 || (uintptr_t)qz->d[0] & 3) return 0;
    if (nm->d[0] != nm->d[1] && !(nm->d[0] + 4 * (size_t)n <= nm->d[1] || nm->d[1] + 4 * (size_t)n <= nm->d[0]))
        return 0;
    if (!sn) return 1;
    return sn[0] == 4 * n && sn[1] == 4 * n && sn[2] == 0 && sq[0] == n && sq[1] == 4 * (n / 32) && sq[2] == 4 * n;
}

/* quantize_q8 at queue index z feeds the product at m (its q and scales are
 * the product's input) */
static int feeds(int z, int m) {
    return g_q[m].d[1] == g_q[z].d[0] && g_q[m].d[2] == g_q[z].d[1] && g_q[m].len[1] == g_q[z].len[0] &&
           g_q[m].len[2] == g_q[z].len[1];
}

/* rmsnorm at i into o, quantize_q8 of o at i + 1, for a launch whose
 * prologue normalizes x in registers (n <= 8192) and stores o and its Q8_0
 * (16-byte aligned x, weight, o and quants; o apart from x: the other
 * workgroups read x after the first one wrote o) */
static int norm_keep_ok(int i) {
    const kh_op *nm = &g_q[i], *qz = &g_q[i + 1];
    const int n = nm->n;
    return qz->d[2] == nm->d[0] && qz->n == n && n % 32 == 0 && n <= 8192 &&
           !(((uintptr_t)nm->d[0] | (uintptr_t)nm->d[1] | (uintptr_t)nm->d[2] | (uintptr_t)qz->d[0]) & 15) &&
           (nm->d[0] + 4 * (size_t)n <= nm->d[1] || nm->d[1] + 4 * (size_t)n <= nm->d[0]);
}

/* A fused launch for the single calls at queue index i: how many calls it
 * covers (0: none applies). */
static int fuse_at(int i) {
    const kh_op *o = &g_q[i];
    /* rmsnorm + quantize_q8 + q, k, v [+ biases] + RoPE, or + w1, w3 + silu_mul */
    if (o->op == QOP_RMSNORM && is_op(i + 1, QOP_QUANT_Q8) && is_op(i + 2, QOP_MATVEC) && is_op(i + 3, QOP_MATVEC) &&
        norm_keep_ok(i) && feeds(i + 1, i + 2) && feeds(i + 1, i + 3) && g_q[i + 2].m.cols == o->n) {
        const kh_op *z = &g_q[i + 1];
        if (is_op(i + 4, QOP_MATVEC) && feeds(i + 1, i + 4) && g_qzero) {
            const kh_op *q = &g_q[i + 2], *k = &g_q[i + 3], *v = &g_q[i + 4];
            int j = i + 5;
            const uint8_t *bias[3] = { NULL, NULL, NULL };
            if (is_op(j, QOP_ADD) && is_op(j + 1, QOP_ADD) && is_op(j + 2, QOP_ADD) && g_q[j].d[0] == q->d[0] &&
                g_q[j + 1].d[0] == k->d[0] && g_q[j + 2].d[0] == v->d[0] && g_q[j].n == q->n &&
                g_q[j + 1].n == k->n && g_q[j + 2].n == v->n) {
                for (int b = 0; b < 3; b++) bias[b] = g_q[j + b].d[1];
                j += 3;
            }
            const kh_op *r = is_op(j, QOP_ROPE) ? &g_q[j] : NULL;
            const int hd = r ? r->n : 0, jr = j - i;
            const unsigned char l_nqkv[15][2] = {
                { KH_L(0, 0), KH_L(1, 2) }, { KH_L(1, 0), KH_L(2, 1) }, { KH_L(1, 1), KH_L(2, 2) },
                { KH_L(1, 0), KH_L(3, 1) }, { KH_L(1, 1), KH_L(3, 2) }, { KH_L(1, 0), KH_L(4, 1) },
                { KH_L(1, 1), KH_L(4, 2) }, { KH_L(2, 0), KH_L(jr, 0) }, { KH_L(3, 0), KH_L(jr, 1) },
                { KH_L(2, 0), KH_L(5, 0) }, { KH_L(3, 0), KH_L(6, 0) }, { KH_L(4, 0), KH_L(7, 0) } };
            if (r && r->d[0] == q->d[0] && r->d[1] == k->d[0] && r->a * hd == q->n && r->b * hd == k->n &&
                k->n == v->n && hd % 2 == 0 && q->n % 2 == 0 && k->n % 2 == 0 && same_kind(&q->m, &k->m) &&
                q->m.cols == v->m.cols && q->m.d16 == v->m.d16 &&
                KH_FUSABLE(i, jr + 1, l_nqkv, bias[0] ? 12 : 9)) {
                krh_rmsnorm_matvec_qkv_keep((float *)q->d[0], (float *)k->d[0], (float *)v->d[0], &q->m, &k->m, &v->m,
                                            (const float *)bias[0], (const float *)bias[1], (const float *)bias[2],
                                            (const float *)o->d[1], (const float *)o->d[2], o->f,
                                            (const float *)r->d[2], (const float *)r->d[3], hd, g_qzero,
                                            (float *)o->d[0], (int8_t *)z->d[0], (float *)z->d[1]);
                return jr + 1;
            }
        }
        static const unsigned char l_nsw[7][2] = {
            { KH_L(0, 0), KH_L(1, 2) }, { KH_L(1, 0), KH_L(2, 1) }, { KH_L(1, 1), KH_L(2, 2) },
            { KH_L(1, 0), KH_L(3, 1) }, { KH_L(1, 1), KH_L(3, 2) }, { KH_L(2, 0), KH_L(4, 0) },
            { KH_L(3, 0), KH_L(4, 1) } };
        const kh_op *w1 = &g_q[i + 2], *w3 = &g_q[i + 3], *sm = is_op(i + 4, QOP_SILU_MUL) ? &g_q[i + 4] : NULL;
        if (sm && sm->d[0] == w1->d[0] && sm->d[1] == w3->d[0] && sm->n == w1->n && w1->n == w3->n &&
            same_kind(&w1->m, &w3->m) && KH_FUSABLE(i, 5, l_nsw, 7)) {
            krh_rmsnorm_matvec_swiglu_keep((float *)w1->d[0], (float *)w3->d[0], &w1->m, &w3->m,
                                           (const float *)o->d[1], (const float *)o->d[2], o->f, (float *)o->d[0],
                                           (int8_t *)z->d[0], (float *)z->d[1]);
            return 5;
        }
    }
    /* quantize_q8 of x + its product into y + the add of y into r */
    static const unsigned char l_qres[3][2] = { { KH_L(0, 0), KH_L(1, 1) }, { KH_L(0, 1), KH_L(1, 2) },
                                                { KH_L(1, 0), KH_L(2, 1) } };
    if (o->op == QOP_QUANT_Q8 && is_op(i + 1, QOP_MATVEC) && is_op(i + 2, QOP_ADD) && feeds(i, i + 1) &&
        g_q[i + 1].m.cols == o->n && o->n % 32 == 0 && o->n <= 16384 &&
        !(((uintptr_t)o->d[0] | (uintptr_t)o->d[2]) & 15) && g_q[i + 2].d[1] == g_q[i + 1].d[0] &&
        g_q[i + 2].n == g_q[i + 1].n && KH_FUSABLE(i, 3, l_qres, 3)) {
        const kh_op *mv = &g_q[i + 1];
        krh_matvec_f_residual_keep((float *)g_q[i + 2].d[0], (float *)mv->d[0], &mv->m, (const float *)o->d[2],
                                   (int8_t *)o->d[0], (float *)o->d[1]);
        return 3;
    }
    static const unsigned char l_nq[2][2] = { { KH_L(0, 0), KH_L(1, 2) }, { KH_L(0, 0), KH_L(0, 1) } };
    if (o->op == QOP_RMSNORM && is_op(i + 1, QOP_QUANT_Q8) && norm_q8_ok(o, &g_q[i + 1], NULL, NULL) &&
        KH_FUSABLE(i, 2, l_nq, o->d[0] == o->d[1] ? 2 : 1)) {
        const kh_op *z = &g_q[i + 1];
        krh_rmsnorm_q8((int8_t *)z->d[0], (float *)z->d[1], (float *)o->d[0], (const float *)o->d[1],
                       (const float *)o->d[2], o->n, o->f, 1);
        return 2;
    }
    if (o->op != QOP_MATVEC) return 0;
    /* q, k, v products of one input [+ the three bias adds] + RoPE */
    if (is_op(i + 1, QOP_MATVEC) && is_op(i + 2, QOP_MATVEC) && same_input(i, i + 1) && same_input(i, i + 2) &&
        g_qzero) {
        const kh_op *q = &g_q[i], *k = &g_q[i + 1], *v = &g_q[i + 2];
        int j = i + 3;
        const uint8_t *bias[3] = { NULL, NULL, NULL };
        if (is_op(j, QOP_ADD) && is_op(j + 1, QOP_ADD) && is_op(j + 2, QOP_ADD) && g_q[j].d[0] == q->d[0] &&
            g_q[j + 1].d[0] == k->d[0] && g_q[j + 2].d[0] == v->d[0] && g_q[j].n == q->n && g_q[j + 1].n == k->n &&
            g_q[j + 2].n == v->n) {
            for (int b = 0; b < 3; b++) bias[b] = g_q[j + b].d[1];
            j += 3;
        }
        const kh_op *r = is_op(j, QOP_ROPE) ? &g_q[j] : NULL;
        const int hd = r ? r->n : 0, jr = j - i;
        /* q, k, v through their bias adds; q and k into RoPE */
        const unsigned char l_qkv[7][2] = { { KH_L(0, 0), KH_L(jr, 0) }, { KH_L(1, 0), KH_L(jr, 1) },
                                            { KH_L(0, 0), KH_L(3, 0) }, { KH_L(1, 0), KH_L(4, 0) },
                                            { KH_L(2, 0), KH_L(5, 0) } };
        if (r && r->d[0] == q->d[0] && r->d[1] == k->d[0] && r->a * hd == q->n && r->b * hd == k->n &&
            k->n == v->n && hd % 2 == 0 && q->n % 2 == 0 && k->n % 2 == 0 && same_kind(&q->m, &k->m) &&
            q->m.cols == v->m.cols && q->m.d16 == v->m.d16 && KH_FUSABLE(i, jr + 1, l_qkv, bias[0] ? 5 : 2)) {
            krh_matvec_qkv((float *)q->d[0], (float *)k->d[0], (float *)v->d[0], &q->m, &k->m, &v->m,
                           (const float *)bias[0], (const float *)bias[1], (const float *)bias[2],
                           (const int8_t *)q->d[1], (const float *)q->d[2], (const float *)r->d[2],
                           (const float *)r->d[3], hd, g_qzero);
            return j + 1 - i;
        }
    }
    /* w1 and w3 products of one input + silu_mul */
    if (is_op(i + 1, QOP_MATVEC) && is_op(i + 2, QOP_SILU_MUL) && same_input(i, i + 1)) {
        const kh_op *w1 = &g_q[i], *w3 = &g_q[i + 1], *sm = &g_q[i + 2];
        static const unsigned char l_sw[2][2] = { { KH_L(0, 0), KH_L(2, 0) }, { KH_L(1, 0), KH_L(2, 1) } };
        if (sm->d[0] == w1->d[0] && sm->d[1] == w3->d[0] && sm->n == w1->n && w1->n == w3->n &&
            same_kind(&w1->m, &w3->m) && KH_FUSABLE(i, 3, l_sw, 2)) {
            krh_matvec_swiglu_keep((float *)w1->d[0], (float *)w3->d[0], &w1->m, &w3->m, (const int8_t *)w1->d[1],
                                   (const float *)w1->d[2]);
            return 3;
        }
    }
    /* a product into y, then y added into the residual r */
    static const unsigned char l_res[1][2] = { { KH_L(0, 0), KH_L(1, 1) } };
    if (is_op(i + 1, QOP_ADD) && g_q[i + 1].d[1] == o->d[0] && g_q[i + 1].n == o->n && KH_FUSABLE(i, 2, l_res, 1)) {
        krh_matvec_residual((float *)g_q[i + 1].d[0], (float *)o->d[0], &o->m, (const int8_t *)o->d[1],
                            (const float *)o->d[2]);
        return 2;
    }
    /* 2 or 3 products of one input, one type */
    int k = 1;
    while (k < 3 && is_op(i + k, QOP_MATVEC) && same_input(i, i + k) && same_kind(&o->m, &g_q[i + k].m)) k++;
    if (k > 1 && KH_FUSABLE(i, k, NULL, 0)) {
        float *y[3];
        const krh_mat *W[3];
        for (int j = 0; j < k; j++) {
            y[j] = (float *)g_q[i + j].d[0];
            W[j] = &g_q[i + j].m;
        }
        krh_matvec_multi(y, W, k, (const int8_t *)o->d[1], (const float *)o->d[2]);
        return k;
    }
    return 0;
}

/* The run starting at queue index i that covers the most calls (the
 * shortest period among equals): its period m (0: none) and rows *T, its
 * strides in g_best. */
static int run_at(int i, int *T_out) {
    int best_m = 0, best_T = 0;
    for (int m = 1; m <= KH_PERIOD_MAX && i + 2 * m <= g_nq; m++) {
        /* no run of period m can cover more calls than are left in whole
         * periods: once the best covers that many, longer periods cannot
         * beat it (a stage of T tokens would otherwise extend every multiple
         * of its period over all T rows) */
        if (best_m && m * ((g_nq - i) / m) <= best_m * best_T) break;
        if (!same_sig(&g_q[i], &g_q[i + m])) continue;
        int ok = 1;
        for (int k = 0; k < m && ok; k++) {
            const kh_op *x = &g_q[i + k], *y = &g_q[i + m + k];
            ok = same_sig(x, y);
            for (int p = 0; ok && p < x->np; p++) g_st[k][p] = (ptrdiff_t)((uintptr_t)y->d[p] - (uintptr_t)x->d[p]);
            ok = ok && strides_ok(x, g_st[k]);
        }
        if (!ok) continue;
        int T = 2;
        for (int more = 1; more && T < KRH_ROWS_MAX && i + (T + 1) * m <= g_nq;) {
            for (int k = 0; k < m && more; k++) {
                const kh_op *x = &g_q[i + k], *y = &g_q[i + T * m + k];
                more = same_sig(x, y);
                for (int p = 0; more && p < x->np; p++)
                    more = (uintptr_t)y->d[p] == (uintptr_t)x->d[p] + (uintptr_t)(T * g_st[k][p]);
            }
            if (more) T++;
        }
        if (m * T <= best_m * best_T) continue;
        int meet = 0;
        for (int a = 0; a < m && !meet; a++)
            for (int pa = 0; pa < g_q[i + a].np && !meet; pa++) {
                const kh_op *x = &g_q[i + a];
                if (!x->wr[pa]) continue;
                for (int b = 0; b < m && !meet; b++)
                    for (int pb = 0; pb < g_q[i + b].np && !meet; pb++)
                        meet = KH_ROWS_MEET(x->d[pa], g_st[a][pa], x->len[pa], g_q[i + b].d[pb], g_st[b][pb],
                                         g_q[i + b].len[pb], T);
            }
        if (meet) continue;
        best_m = m;
        best_T = T;
        memcpy(g_best, g_st, sizeof g_st[0] * (size_t)m);
    }
    *T_out = best_T;
    return best_m;
}

static void q_flush(void) {
    for (int i = 0; i < g_nq;) {
        int T, m = run_at(i, &T), f;
        if (m) {
            for (int k = 0; k < m; k++) {
                const kh_op *o = &g_q[i + k], *z = &g_q[i + k + 1];
                if (k + 1 < m && o->op == QOP_RMSNORM && z->op == QOP_QUANT_Q8 &&
                    norm_q8_ok(o, z, g_best[k], g_best[k + 1])) {   /* rows of one rmsnorm_q8 launch */
                    krh_rmsnorm_q8((int8_t *)z->d[0], (float *)z->d[1], (float *)o->d[0], (const float *)o->d[1],
                                   (const float *)o->d[2], o->n, o->f, T);
                    k++;
                } else {
                    launch(o, g_best[k], T);
                }
            }
            i += m * T;
        } else if ((f = fuse_at(i)) > 0) {
            i += f;
        } else {
            launch(&g_q[i++], NULL, 1);
        }
    }
    g_nq = 0;
}

/* Queues a row op when every pointer argument has an HBM copy; 0 when one
 * does not (the caller runs it at once, after q_flush). */
static int q_push(int op, int n, int a, int b, float f, int np, const void *const *h, const size_t *len,
                  const int *wr) {
    kh_op o;
    memset(&o, 0, sizeof o);
    o.op = op;
    o.np = np;
    o.n = n;
    o.a = a;
    o.b = b;
    o.f = f;
    for (int p = 0; p < np; p++) {
        if (!h[p] || !(o.d[p] = dev_addr(h[p], len[p]))) return 0;
        o.len[p] = len[p];
        o.wr[p] = wr[p];
    }
    if (!g_q && !(g_q = malloc(sizeof *g_q * KH_QUEUE))) return 0;
    if (g_nq == KH_QUEUE) q_flush();
    if (op == QOP_MATVEC) {   /* the matrix: rows n, cols a; its type and scale kind in b */
        o.m = (krh_mat){ o.d[3], o.d[4], n, a, b & 0xff, b >> 8 };
    }
    g_q[g_nq++] = o;
    return 1;
}

#endif
