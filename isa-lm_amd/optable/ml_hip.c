/* ISA=hip: the modules an ISA=hip build of Krafla owns, over the MI355X
 * backend (libkrafla_hip.so), so that the reference's model/transformer.c,
 * model/mlb.c, model/sampler.c and app/ml_run.c run unchanged:
 *
 *   core/arena.c       ml_arena_*: pinned host memory plus an HBM twin
 *   core/threads.c     ml_pool_*: one worker (the stream orders the work);
 *                      creating the pool (the last step of ml_state_init,
 *                      model/transformer.c:163) uploads the arenas, after the
 *                      host has written the RoPE tables into them
 *   model/pack_model.c ml_model_pack*: uploads the mapped model file
 *   core/quant_ref.c   ml_dequant_row: a device gather when the output row
 *                      has an HBM copy; host buffers go to the reference's
 *                      own core/quant_ref.c, compiled beside this file with
 *                      that one function renamed ml_dequant_row_host (its
 *                      ml_quantize_row_q4 is used unchanged)
 *   core/isa_check.c   ml_isa_check: a gfx950 device or ML_E_ISA (exit 3)
 *   ops/ops.c          ml_matvec, ml_matmul (int8 MFMA), ml_attention(_batch),
 *                      ml_quantize_row, ml_softcap_rows
 *   kernels/hip        ml_k_<op>_hip, bound by config/ml_config.h
 *
 * Pointer contract (the reference code passes host addresses): an address
 * inside a registered range (an arena, a model file) stands for its HBM copy;
 * any other buffer is staged to the device for the call and copied back.
 * The host reads activations only as logits: the classifier's matvec copies
 * them back and synchronizes, which is also where device errors surface.
 * Row ops on arena buffers are queued and launched row-batched (below, "the
 * per-token op queue"); every other call first launches what is queued.
 * The embedding's scale (model/transformer.c:228-229, a host loop over the
 * row) is applied on the device by ml_dequant_row instead, so the host loop
 * only touches the arena's host copy, which nothing reads.
 * KV caches: F32 and Q8 (store_kv quantizes through ml_quantize_row), and
 * F16: store_kv converts K and V to halves in a host loop
 * (model/transformer.c:195-197) from staging rows that live on the device
 * here, so the attention call first converts this step's staging rows on
 * the device (the halves ml_f32_to_f16 gives, core/ml.c:39-53) into the
 * cache rows it reads; the host loop's copy is never read.
 * --imatrix: the importance statistics are host reads of each matrix input
 * right after its Q8_0 quantization (model/transformer.c:250-255, :272-301,
 * :399-421). With --imatrix on the command line, every ml_k_quantize_q8 call
 * runs at once (not queued) and copies its float input back to the host
 * copy, so the host loop reads the device's values. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "config/ml_config.h"
#include "core/arena.h"
#include "core/isa_check.h"
#include "core/quant_ref.h"
#include "core/threads.h"
#include "model/pack_model.h"
#include "model/transformer.h"   /* ML_BATCH_MAX: the staging rows of an F16 cache */
#include "ops/ops.h"
#define KRAFLA_TYPES_H   /* the types come from the reference's core/ml.h */
#include "krafla_hip.h"

/* core/quant_ref.c's ml_dequant_row, compiled under this name */
void ml_dequant_row_host(float *out, const ml_qtensor *W, int row);

/* ---- address ranges with an HBM copy ---- */

typedef struct {
    const uint8_t *h;
    size_t n;
    uint8_t *d;
    int uploaded;
} kh_range;

#define KH_RANGES 64
static kh_range g_rg[KH_RANGES];
static int g_nrg;
static int *g_ints;                 /* device ints: [0] position, [1] token row, [2] zero */
static int g_pos_set = -1;          /* the position g_ints[0] holds (-1: none yet) */
static int g_row_set;               /* g_ints[1] holds 0 */
static float *g_batt;               /* batched attention scratch */
static size_t g_batt_n;
/* each packed model's embedding table, its row scale and its classifier's
 * quants (ml_model_pack): the scale applies to that model's rows only, and
 * its classifier's products are not queued (the host reads the logits) */
typedef struct {
    const ml_qtensor *emb;
    float emb_scale;
    const void *cls_q;
} kh_packed;
#define KH_MODELS 16
static kh_packed g_pk[KH_MODELS];
static int g_npk;
static int g_reported;

/* whether this process's command line holds --imatrix (app/ml_run.c:276):
 * then the inputs of the Q8_0 quantizations are copied back to the host */
static int g_imat = -1;
static int imatrix_on(void) {
    if (g_imat < 0) {
        g_imat = 0;
        FILE *f = fopen("/proc/self/cmdline", "rb");
        if (f) {
            static char buf[1 << 16];
            const size_t n = fread(buf, 1, sizeof buf - 1, f);
            fclose(f);
            buf[n] = 0;
            for (size_t i = 0; i < n; i += strlen(buf + i) + 1)
                if (!strcmp(buf + i, "--imatrix")) g_imat = 1;
        }
    }
    return g_imat;
}

static int ready(void) {
    if (krh_init() != ML_OK) return 0;
    if (!g_ints && (g_ints = krh_alloc(3 * sizeof(int)))) krh_set_int(g_ints + 2, 0);
    return g_ints != NULL;
}

/* g_ints[0] = pos, written only when it changes: every layer of a token
 * attends at one position, and the launches run in order on one stream */
static void set_pos(int pos) {
    if (pos == g_pos_set) return;
    krh_set_int(g_ints, pos);
    g_pos_set = pos;
}

static uint8_t *dev_addr(const void *p, size_t n) {
    const uint8_t *b = p;
    for (int i = 0; i < g_nrg; i++) {
        const kh_range *r = &g_rg[i];
        if (b >= r->h && n <= r->n && (size_t)(b - r->h) <= r->n - n) return r->d + (b - r->h);
    }
    return NULL;
}

static void drop_range(const void *h) {
    for (int i = 0; i < g_nrg; i++)
        if (g_rg[i].h == h) {
            g_rg[i] = g_rg[--g_nrg];
            return;
        }
}

static int add_range(const void *h, size_t n, uint8_t *d, int uploaded) {
    drop_range(h);
    if (g_nrg == KH_RANGES) return 0;
    g_rg[g_nrg++] = (kh_range){ h, n, d, uploaded };
    return 1;
}

static void *grow(void *p, size_t *have, size_t need) {
    if (need <= *have) return p;
    krh_sync();
    krh_free(p);
    p = krh_alloc(need);
    *have = p ? need : 0;
    return p;
}

/* ---- one call's arguments ---- */

typedef struct {
    void *h;
    uint8_t *d;
    size_t n;
    int out;
} kh_buf;

typedef struct {
    kh_buf st[16], mir[8];   /* staged buffers; arena outputs */
    int nst, nmir, staged, fail;
} kh_call;

/* The device address of caller buffer h of n bytes for one call: its HBM
 * copy, or a staged copy (filled when `in`, copied back when `out`). */
static void *arg(kh_call *c, const void *h, size_t n, int in, int out) {
    if (!h || !n || c->fail) return (void *)h;
    uint8_t *d = dev_addr(h, n);
    if (d) {
        if (out && c->nmir < 8) c->mir[c->nmir++] = (kh_buf){ (void *)h, d, n, 1 };
        return d;
    }
    if (c->nst == 16 || !(d = krh_alloc(n)) || (in && krh_copy_h2d(d, h, n) != ML_OK)) {
        krh_free(d);
        c->fail = 1;
        return NULL;
    }
    c->st[c->nst++] = (kh_buf){ (void *)h, d, n, out };
    c->staged = 1;
    return d;
}

/* Copies staged outputs back (and, when weights were staged, outputs that
 * live in the arena too: their host copy is what a host reader sees) */
static void done(kh_call *c) {
    for (int i = 0; i < c->nst; i++)
        if (c->st[i].out) krh_copy_d2h(c->st[i].h, c->st[i].d, c->st[i].n);
    if (c->staged)
        for (int i = 0; i < c->nmir; i++) krh_copy_d2h(c->mir[i].h, c->mir[i].d, c->mir[i].n);
    if (c->nst) krh_sync();
    for (int i = 0; i < c->nst; i++) krh_free(c->st[i].d);
}

/* rows [r0, r1) of W as a device matrix (the file's f16 scales when it has them) */
static void mat_of(kh_call *c, const ml_qtensor *W, int r0, int r1, krh_mat *m) {
    const size_t nb = (size_t)W->cols / QK, rowq = W->type == ML_Q8_0 ? (size_t)W->cols : (size_t)W->cols / 2;
    const size_t nr = (size_t)(r1 - r0);
    m->rows = r1 - r0;
    m->cols = W->cols;
    m->type = W->type;
    m->q = arg(c, (const uint8_t *)W->q + (size_t)r0 * rowq, nr * rowq, 1, 0);
    if (W->dh) {
        m->d16 = 1;
        m->d = arg(c, W->dh + (size_t)r0 * nb, nr * nb * 2, 1, 0);
    } else {
        m->d16 = 0;
        m->d = arg(c, W->d + (size_t)r0 * nb, nr * nb * 4, 1, 0);
    }
}

static void fail_call(const char *what) {
    if (!g_reported) fprintf(stderr, "error: hip backend: %s\n", what);
    g_reported = 1;
}


#include "kh_queue.h"

ml_status ml_hip_status(void) {
    q_flush();
    return krh_status();
}
const char *ml_hip_last_error(void) {
    q_flush();
    return krh_last_error();
}

/* ---- core/isa_check.c ---- */

const char *ml_isa_build_name(void) { return ML_ISA_NAME; }

ml_status ml_isa_check(const char **missing) {
    if (ready()) return ML_OK;
    *missing = "an AMD Instinct MI355X (gfx950) GPU";
    return ML_E_ISA;
}

/* ---- core/arena.c: the same bump allocator (core/arena.c:3-26) over
 * pinned host memory, with an HBM twin registered for translation ---- */

/* the arenas' allocations in order (ml_state_init's F16 cache is kh, vh,
 * then the staging rows kbuf, vbuf: model/transformer.c:114-117) */
typedef struct {
    const uint8_t *p;
    size_t n;
} kh_alloc;
#define KH_ALLOCS 512
static kh_alloc g_al[KH_ALLOCS];
static int g_nal;

ml_status ml_arena_init(ml_arena *a, size_t cap) {
    a->base = NULL;
    a->cap = a->off = 0;
    if (cap > (size_t)-1 - ML_ALIGN || !ready()) return cap > (size_t)-1 - ML_ALIGN ? ML_E_NOMEM : ML_E_ISA;
    cap = (cap + ML_ALIGN - 1) & ~(size_t)(ML_ALIGN - 1);
    uint8_t *h = krh_host_alloc(cap), *d = krh_alloc(cap);
    if (!h || !d || !add_range(h, cap, d, 0)) {
        krh_host_free(h);
        krh_free(d);
        return ML_E_NOMEM;
    }
    a->base = h;
    a->cap = cap;
    return ML_OK;
}

void *ml_arena_alloc(ml_arena *a, size_t n) {
    const size_t need = (n + ML_ALIGN - 1) & ~(size_t)(ML_ALIGN - 1);
    if (need > a->cap - a->off) return NULL;
    void *p = a->base + a->off;
    a->off += need;
    if (g_nal < KH_ALLOCS) g_al[g_nal++] = (kh_alloc){ p, n };
    return p;
}

void ml_arena_free(ml_arena *a) {
    if (a->base) {
        int k = 0;
        for (int i = 0; i < g_nal; i++)
            if (!(g_al[i].p >= a->base && g_al[i].p < a->base + a->cap)) g_al[k++] = g_al[i];
        g_nal = k;
        q_flush();
        krh_sync();
        uint8_t *d = dev_addr(a->base, 1);
        drop_range(a->base);
        krh_free(d);
        krh_host_free(a->base);
    }
    a->base = NULL;
    a->cap = a->off = 0;
}

/* ---- core/threads.c: one worker ---- */

struct ml_pool { int n; };

ml_status ml_pool_create(ml_pool **p, int n) {
    (void)n;
    *p = NULL;
    if (!ready()) return ML_E_ISA;
    q_flush();
    for (int i = 0; i < g_nrg; i++)   /* the arenas, as the host has filled them */
        if (!g_rg[i].uploaded) {
            if (krh_copy_h2d(g_rg[i].d, g_rg[i].h, g_rg[i].n) != ML_OK) return ML_E_IO;
            g_rg[i].uploaded = 1;
        }
    *p = malloc(sizeof **p);
    if (!*p) return ML_E_NOMEM;
    (*p)->n = 1;
    return ML_OK;
}

void ml_pool_run(ml_pool *p, ml_task_fn fn, void *ctx) { (void)p; fn(ctx, 0, 1); }
int ml_pool_size(const ml_pool *p) { (void)p; return 1; }
int ml_pool_threads(int n) { (void)n; return 1; }
void ml_pool_destroy(ml_pool *p) {
    q_flush();
    free(p);
}

/* ---- model/pack_model.c: the model file to HBM, once ---- */

ml_status ml_model_pack(ml_model *m, ml_pool *pool) {
    (void)pool;
    if (!ready()) return ML_E_ISA;
    q_flush();
    const uint8_t *h = m->file.data;
    const size_t n = m->file.size;
    uint8_t *d = dev_addr(h, n);
    if (!d) {
        d = krh_alloc(n);
        if (!d) return ML_E_NOMEM;
        if (krh_copy_h2d(d, h, n) != ML_OK || !add_range(h, n, d, 1)) {
            krh_free(d);
            return ML_E_IO;
        }
    } else if (krh_copy_h2d(d, h, n) != ML_OK) {   /* the same address may be a new file */
        return ML_E_IO;
    }
    int k = 0;
    while (k < g_npk && g_pk[k].emb != &m->tok_emb) k++;
    if (k == KH_MODELS) return ML_E_NOMEM;
    if (k == g_npk) g_npk++;
    g_pk[k] = (kh_packed){ &m->tok_emb, m->cfg.embed_scale, m->wcls.q };
    return ML_OK;
}

/* the embedding scale of the packed model whose table W is (1 otherwise) */
static float emb_scale_of(const ml_qtensor *W) {
    for (int k = 0; k < g_npk; k++)
        if (g_pk[k].emb == W) return g_pk[k].emb_scale;
    return 1.0f;
}

static int is_classifier(const void *q) {
    for (int k = 0; k < g_npk; k++)
        if (g_pk[k].cls_q == q) return 1;
    return 0;
}

ml_status ml_model_pack_cached(ml_model *m, ml_pool *pool, const char *path, const char **how) {
    (void)path;
    *how = "none";
    return ml_model_pack(m, pool);
}

int ml_pack_group(void) { return 0; }

/* ---- core/quant_ref.c ---- */

void ml_dequant_row(float *out, const ml_qtensor *W, int row) {
    q_flush();
    if (dev_addr(out, sizeof(float) * (size_t)W->cols) && ready()) {   /* the embedding of ml_forward */
        kh_call c = { 0 };
        krh_mat m;
        mat_of(&c, W, row, row + 1, &m);
        float *o = arg(&c, out, sizeof(float) * (size_t)W->cols, 0, 1);
        if (!c.fail) {
            if (!g_row_set) {
                krh_set_int(g_ints + 1, 0);
                g_row_set = 1;
            }
            krh_embed(o, &m, g_ints + 1, emb_scale_of(W));
        }
        done(&c);
        return;
    }
    ml_dequant_row_host(out, W, row);   /* a host buffer: the reference's own rule */
}

/* ---- kernels/hip ---- */

#define F(n) (sizeof(float) * (size_t)(n))

/* a product on arena buffers into the queue (not the classifier's: the host
 * reads the logits next) */
static int queue_matvec(float *y, const ml_qtensor *W, const ml_qact *x, int r0, int r1) {
    if (is_classifier(W->q)) return 0;
    const size_t nb = (size_t)W->cols / QK, rowq = W->type == ML_Q8_0 ? (size_t)W->cols : (size_t)W->cols / 2;
    const size_t nr = (size_t)(r1 - r0);
    const void *h[] = { y + r0, x->q, x->d, (const uint8_t *)W->q + (size_t)r0 * rowq,
                        W->dh ? (const void *)(W->dh + (size_t)r0 * nb) : (const void *)(W->d + (size_t)r0 * nb) };
    const size_t len[] = { F(nr), (size_t)W->cols, F(nb), nr * rowq, nr * nb * (W->dh ? 2 : 4) };
    const int wr[] = { 1, 0, 0, 0, 0 };
    g_qzero = g_ints + 2;
    return q_push(QOP_MATVEC, (int)nr, W->cols, W->type | (W->dh ? 1 << 8 : 0), 0.0f, 5, h, len, wr);
}

static void matvec_rows(float *y, const ml_qtensor *W, const ml_qact *x, int r0, int r1) {
    if (r0 >= r1 || !ready()) return;
    if (queue_matvec(y, W, x, r0, r1)) return;
    q_flush();
    kh_call c = { 0 };
    krh_mat m;
    mat_of(&c, W, r0, r1, &m);
    const int8_t *xq = arg(&c, x->q, (size_t)W->cols, 1, 0);
    const float *xd = arg(&c, x->d, F(W->cols / QK), 1, 0);
    float *yd = arg(&c, y + r0, F(r1 - r0), 0, 1);
    if (!c.fail) krh_matvec(yd, &m, xq, xd, 0);
    if (is_classifier(W->q) && !c.staged && yd && yd != (void *)(y + r0)) {
        /* the logits: the host reads them next (app/ml_run.c:388-392) */
        if (krh_copy_d2h(y + r0, yd, F(r1 - r0)) != ML_OK || krh_status() != ML_OK) {
            fail_call(krh_last_error());
            for (int r = r0; r < r1; r++) y[r] = NAN;
        }
    }
    done(&c);
    if (c.fail) fail_call("cannot stage a buffer");
}

void ml_k_matvec_q8_hip(float *y, const ml_qtensor *W, const ml_qact *x, int r0, int r1) { matvec_rows(y, W, x, r0, r1); }
void ml_k_matvec_q4_hip(float *y, const ml_qtensor *W, const ml_qact *x, int r0, int r1) { matvec_rows(y, W, x, r0, r1); }

void ml_k_quantize_q8_hip(ml_qact *out, const float *x, int k) {
    if (!ready()) return;
    const void *h[] = { out->q, out->d, x };
    const size_t len[] = { (size_t)k, F(k / QK), F(k) };
    const int wr[] = { 1, 1, 0 };
    const int imat = imatrix_on();
    if (!imat && q_push(QOP_QUANT_Q8, k, 0, 0, 0.0f, 3, h, len, wr)) return;
    q_flush();
    kh_call c = { 0 };
    const float *xd = arg(&c, x, F(k), 1, 0);
    int8_t *q = arg(&c, out->q, (size_t)k, 0, 1);
    float *d = arg(&c, out->d, F(k / QK), 0, 1);
    if (!c.fail) krh_quantize_q8(q, d, xd, k, 1);
    if (imat && !c.fail && xd != x && krh_copy_d2h((float *)x, xd, F(k)) != ML_OK) fail_call(krh_last_error());
    done(&c);
}

void ml_k_rmsnorm_hip(float *o, const float *x, const float *w, int n, float eps) {
    if (!ready()) return;
    const void *h[] = { o, x, w };
    const size_t len[] = { F(n), F(n), F(n) };
    const int wr[] = { 1, 0, 0 };
    if (q_push(QOP_RMSNORM, n, 0, 0, eps, 3, h, len, wr)) return;
    q_flush();
    kh_call c = { 0 };
    const float *xd = arg(&c, x, F(n), 1, 0), *wd = arg(&c, w, F(n), 1, 0);
    float *od = arg(&c, o, F(n), 0, 1);
    if (!c.fail) krh_rmsnorm(od, xd, wd, n, eps);
    done(&c);
}

void ml_k_softmax_hip(float *x, int n) {
    if (!ready()) return;
    q_flush();
    kh_call c = { 0 };
    float *xd = arg(&c, x, F(n), 1, 1);
    if (!c.fail) krh_softmax(xd, n);
    done(&c);
}

void ml_k_rope_hip(float *q, float *k, const float *cos_t, const float *sin_t, int head_dim, int n_heads,
                   int n_kv_heads) {
    if (!ready()) return;
    const void *h[] = { q, k, cos_t, sin_t };
    const size_t len[] = { F(n_heads * head_dim), F(n_kv_heads * head_dim), F(head_dim / 2), F(head_dim / 2) };
    const int wr[] = { 1, 1, 0, 0 };
    if (q_push(QOP_ROPE, head_dim, n_heads, n_kv_heads, 0.0f, 4, h, len, wr)) return;
    q_flush();
    kh_call c = { 0 };
    float *qd = arg(&c, q, F(n_heads * head_dim), 1, 1), *kd = arg(&c, k, F(n_kv_heads * head_dim), 1, 1);
    const float *cd = arg(&c, cos_t, F(head_dim / 2), 1, 0), *sd = arg(&c, sin_t, F(head_dim / 2), 1, 0);
    if (!c.fail) krh_rope(qd, kd, cd, sd, head_dim, n_heads, n_kv_heads);
    done(&c);
}

static void pair_op(int qop, void (*op)(float *, const float *, int), float *g, const float *u, int n) {
    if (!ready()) return;
    const void *h[] = { g, u };
    const size_t len[] = { F(n), F(n) };
    const int wr[] = { 1, 0 };
    if (q_push(qop, n, 0, 0, 0.0f, 2, h, len, wr)) return;
    q_flush();
    kh_call c = { 0 };
    float *gd = arg(&c, g, F(n), 1, 1);
    const float *ud = arg(&c, u, F(n), 1, 0);
    if (!c.fail) op(gd, ud, n);
    done(&c);
}

void ml_k_silu_mul_hip(float *g, const float *u, int n) { pair_op(QOP_SILU_MUL, krh_silu_mul, g, u, n); }
void ml_k_gelu_mul_hip(float *g, const float *u, int n) { pair_op(QOP_GELU_MUL, krh_gelu_mul, g, u, n); }
void ml_k_add_hip(float *y, const float *x, int n) { pair_op(QOP_ADD, krh_add, y, x, n); }

void ml_k_dot_f32_hip(float *s, const float *q, const float *k, size_t ldk, int rows, int n, float scale) {
    if (rows <= 0 || !ready()) return;
    q_flush();
    kh_call c = { 0 };
    float *sd = arg(&c, s, F(rows), 0, 1);
    const float *qd = arg(&c, q, F(n), 1, 0), *kd = arg(&c, k, F((size_t)(rows - 1) * ldk + n), 1, 0);
    if (!c.fail) krh_dot_rows(sd, qd, kd, ldk, rows, n, scale);
    done(&c);
}

void ml_k_axpy_f32_hip(float *y, const float *a, const float *x, size_t ldx, int rows, int n) {
    if (rows <= 0 || !ready()) return;
    q_flush();
    kh_call c = { 0 };
    float *yd = arg(&c, y, F(n), 1, 1);
    const float *ad = arg(&c, a, F(rows), 1, 0), *xd = arg(&c, x, F((size_t)(rows - 1) * ldx + n), 1, 0);
    if (!c.fail) krh_axpy_rows(yd, ad, xd, ldx, rows, n);
    done(&c);
}

/* ---- ops/ops.c ---- */

void ml_matvec(ml_pool *pool, float *y, const ml_qtensor *W, const ml_qact *x) {
    (void)pool;
    matvec_rows(y, W, x, 0, W->rows);
}

/* Y[t * ldy + r] = W x_t (ops/ops.c:51-79): the MFMA matmul over the batch,
 * each token's row the matvec's bit for bit, reading the batch's scales in
 * their token rows */
void ml_matmul(ml_pool *pool, float *Y, int ldy, const ml_qtensor *W, const ml_qbatch *X) {
    (void)pool;
    const int n = X->n, k = X->k, nb = k / QK, ldx = (n + 127) / 128 * 128;
    if (n <= 0 || !ready()) return;
    q_flush();
    kh_call c = { 0 };
    krh_mat m;
    mat_of(&c, W, 0, W->rows, &m);
    /* the activations must be readable for ldx rows: arena batches hold
     * ML_BATCH_MAX rows; anything shorter is staged padded */
    const int8_t *xq = (const int8_t *)dev_addr(X->q, (size_t)ldx * k);
    if (!xq) {
        int8_t *pad = krh_alloc((size_t)ldx * k);
        const int8_t *src = arg(&c, X->q, (size_t)n * k, 1, 0);
        if (pad && src) krh_copy_d2d_async(pad, src, (size_t)n * k);
        if (pad && c.nst < 16) c.st[c.nst++] = (kh_buf){ NULL, (uint8_t *)pad, 0, 0 };
        else c.fail = 1;
        xq = pad;
    }
    const float *xd = arg(&c, X->d, F((size_t)n * nb), 1, 0);
    /* in and out: rows of Y are ldy apart and the gaps are the caller's */
    float *yd = arg(&c, Y, F((size_t)(n - 1) * ldy + W->rows), 1, 1);
    if (!c.fail) krh_matmul_rows(yd, ldy, &m, xq, xd, ldx, n, 0);
    done(&c);
    if (c.fail) fail_call("cannot stage a buffer");
}

void ml_quantize_row(int8_t *q, float *d, const float *x, int n) {
    if (!ready()) return;
    const void *h[] = { q, d, x };
    const size_t len[] = { (size_t)n, F(1), F(n) };
    const int wr[] = { 1, 1, 0 };
    if (q_push(QOP_QUANT_ROW, n, 0, 0, 0.0f, 3, h, len, wr)) return;
    q_flush();
    kh_call c = { 0 };
    const float *xd = arg(&c, x, F(n), 1, 0);
    int8_t *qd = arg(&c, q, (size_t)n, 0, 1);
    float *dd = arg(&c, d, F(1), 0, 1);
    if (!c.fail) krh_quantize_row(qd, dd, xd, n);
    done(&c);
}

void ml_softcap_rows(float *x, size_t ld, int rows, int n, float cap) {
    if (rows <= 0 || !ready()) return;
    q_flush();
    kh_call c = { 0 };
    const size_t bytes = F((size_t)(rows - 1) * ld + n);
    float *xd = arg(&c, x, bytes, 1, 1);
    if (!c.fail) krh_softcap_rows(xd, ld, rows, n, cap);
    /* soft-capped logits in the arena are read on the host next */
    if (!c.staged && xd && xd != x) krh_copy_d2h(x, xd, bytes);
    done(&c);
}

int ml_attention_batch_heads(const ml_config *cfg, int nthreads) {
    (void)nthreads;
    return cfg->n_heads / cfg->n_kv_heads;
}

/* The F16 cache's staging rows: the two allocations after the ones holding
 * the layer views kh and vh (model/transformer.c:114-117), each
 * ML_BATCH_MAX rows of kv_dim floats. */
static int f16_staging(const ml_kv_layer *kv, const ml_config *cfg, const float **kb, const float **vb) {
    const size_t rows = F((size_t)ML_BATCH_MAX * cfg->kv_dim);
    for (int i = 0; i + 3 < g_nal; i++) {
        const uint8_t *h = (const uint8_t *)kv->kh;
        if (!(h >= g_al[i].p && h < g_al[i].p + g_al[i].n)) continue;
        const uint8_t *v = (const uint8_t *)kv->vh;
        if (!(v >= g_al[i + 1].p && v < g_al[i + 1].p + g_al[i + 1].n) || g_al[i + 2].n != rows || g_al[i + 3].n != rows)
            return 0;
        *kb = (const float *)g_al[i + 2].p;
        *vb = (const float *)g_al[i + 3].p;
        return 1;
    }
    return 0;
}

static int attn_supported(const ml_kv_layer *kv, const ml_config *cfg) {
    const float *kb, *vb;
    if ((kv->kh || kv->vh) && !(kv->kh && kv->vh && f16_staging(kv, cfg, &kb, &vb))) {
        fail_call("an F16 KV cache whose staging rows are not the state's (model/transformer.c:114-117)");
        return 0;
    }
    if (!(kv->k && kv->v) && !(kv->kh && kv->vh) && !(kv->kq && kv->vq && kv->kd && kv->vd)) {
        fail_call("attention without KV cache rows");
        return 0;
    }
    if (!ready()) return 0;
    q_flush();
    return 1;
}

/* F16 cache: store_kv's halves of this step's ntok staging rows into the
 * cache rows at positions g_ints[0] + t, on the device; 0 when the call
 * must not go on */
static int f16_store(kh_call *c, const ml_kv_layer *kv, const ml_kv_layer *d, const ml_config *cfg, int ntok) {
    const float *kb, *vb;
    if (!kv->kh) return !c->fail;
    if (c->fail || !f16_staging(kv, cfg, &kb, &vb)) return 0;
    const float *kd = arg(c, kb, F((size_t)ntok * cfg->kv_dim), 1, 0);
    const float *vd = arg(c, vb, F((size_t)ntok * cfg->kv_dim), 1, 0);
    if (c->fail) return 0;
    krh_store_kv(ML_F16, d->kh, d->vh, NULL, NULL, kd, vd, cfg->n_kv_heads, cfg->head_dim, g_ints, ntok);
    return 1;
}

/* the layer's cache as device pointers: F32 rows, F16 rows, or Q8 rows and
 * their row scales (written on the device by ml_quantize_row in store_kv) */
static ml_kv_layer dev_kv(kh_call *c, const ml_kv_layer *kv, const ml_config *cfg) {
    const size_t n = (size_t)cfg->max_seq * cfg->kv_dim, ns = (size_t)cfg->max_seq * cfg->n_kv_heads;
    ml_kv_layer d;
    memset(&d, 0, sizeof d);
    d.window = kv->window;
    if (kv->k) {
        d.k = arg(c, kv->k, F(n), 1, 0);
        d.v = arg(c, kv->v, F(n), 1, 0);
    } else if (kv->kh) {
        d.kh = arg(c, kv->kh, 2 * n, 1, 0);
        d.vh = arg(c, kv->vh, 2 * n, 1, 0);
    } else {
        d.kq = arg(c, kv->kq, n, 1, 0);
        d.vq = arg(c, kv->vq, n, 1, 0);
        d.kd = arg(c, kv->kd, F(ns), 1, 0);
        d.vd = arg(c, kv->vd, F(ns), 1, 0);
    }
    return d;
}

/* ops/ops.c:169-180; the Q8 cache's quantized query heads (qq, qd) are
 * formed inside the score kernel, so the caller's scratch is not used */
void ml_attention(ml_pool *pool, float *out, const float *q, const ml_kv_layer *kv, float *att_scratch, int8_t *qq,
                  float *qd, const ml_config *cfg, int pos) {
    (void)pool; (void)qq; (void)qd;
    if (!attn_supported(kv, cfg)) return;
    kh_call c = { 0 };
    float *o = arg(&c, out, F(cfg->q_dim), 0, 1);
    const float *qv = arg(&c, q, F(cfg->q_dim), 1, 0);
    float *att = arg(&c, att_scratch, F((size_t)cfg->n_heads * cfg->max_seq), 0, 0);
    const ml_kv_layer d = dev_kv(&c, kv, cfg);
    if (!c.fail) {
        set_pos(pos);
        if (f16_store(&c, kv, &d, cfg, 1))
            krh_attention_kv_softcap(o, att, qv, &d, cfg->n_heads, cfg->n_kv_heads, cfg->head_dim, cfg->max_seq,
                                     cfg->attn_scale, g_ints, 1, cfg->max_seq - 1, cfg->attn_softcap);
    }
    done(&c);
}

/* ops/ops.c:216-238 */
void ml_attention_batch(ml_pool *pool, float *out, const float *q, const ml_kv_layer *kv, float *att_scratch,
                        int8_t *qq, float *qd, const ml_config *cfg, int pos0, int n) {
    (void)pool; (void)qq; (void)qd; (void)att_scratch;
    if (n <= 0 || !attn_supported(kv, cfg)) return;
    g_batt = grow(g_batt, &g_batt_n, F((size_t)n * cfg->n_heads * cfg->max_seq));
    kh_call c = { 0 };
    float *o = arg(&c, out, F((size_t)n * cfg->q_dim), 0, 1);
    const float *qv = arg(&c, q, F((size_t)n * cfg->q_dim), 1, 0);
    const ml_kv_layer d = dev_kv(&c, kv, cfg);
    if (!c.fail && g_batt) {
        set_pos(pos0);
        if (f16_store(&c, kv, &d, cfg, n))
            krh_attention_kv_softcap(o, g_batt, qv, &d, cfg->n_heads, cfg->n_kv_heads, cfg->head_dim, cfg->max_seq,
                                     cfg->attn_scale, g_ints, n, pos0 + n - 1, cfg->attn_softcap);
    }
    done(&c);
}
