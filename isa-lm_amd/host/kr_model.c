/* The token loop on the device: model upload, decoding state, and
 * ml_forward / ml_prefill / ml_run's greedy loop as sequences of fused HIP
 * ops, each sequence captured once into a graph and replayed per token.
 *
 * One decode step (model/transformer.c:257-306), per layer:
 *   rmsnorm+quantize(attn_norm) -> q,k,v matvec + bias + RoPE + cache write
 *   -> attention -> x += wo.q8(ao) -> rmsnorm+quantize(ffn_norm)
 *   -> silu(w1.x) * (w3.x) -> x += w2.q8(h)
 * then rmsnorm+quantize(final_norm) -> logits = wcls.x. Every op reads the
 * token and position from device memory, so the captured step replays for
 * any position without new arguments. */
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <time.h>
#include "kr_host.h"

static char g_err[512];

ml_status kr_seterr(ml_status s, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return s;
}

const char *kr_error(void) { return g_err; }

/* core/ml.c:21-33 */
const char *kr_status_str(ml_status s) {
    switch (s) {
    case ML_OK: return "ok";
    case ML_E_IO: return "i/o error";
    case ML_E_FORMAT: return "bad file format";
    case ML_E_SHAPE: return "bad tensor shape";
    case ML_E_NOMEM: return "out of memory";
    case ML_E_ISA: return "no gfx950 device";
    }
    return "unknown";
}

double kr_now(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}

/* ---- upload ---- */

#define RUP(n) (((size_t)(n) + 255) & ~(size_t)255)

static size_t mat_bytes(const ml_qtensor *W, int f16) {
    const size_t n = (size_t)W->rows * W->cols;
    return RUP(W->type == ML_Q4_0 ? n / 2 : n) + RUP(n / QK * (f16 ? 2 : 4));
}

typedef struct { uint8_t *base; size_t off; ml_status st; } placer;

static void *place(placer *p, const void *src, size_t n) {
    void *dst = p->base + p->off;
    p->off += RUP(n);
    if (p->st == ML_OK && n && krh_copy_h2d(dst, src, n) != ML_OK) p->st = kr_seterr(ML_E_IO, "%s", krh_last_error());
    return dst;
}

static krh_mat place_mat(placer *p, const ml_qtensor *W, int f16) {
    const size_t n = (size_t)W->rows * W->cols;
    krh_mat d;
    d.rows = W->rows;
    d.cols = W->cols;
    d.type = W->type;
    d.d16 = f16;
    d.q = place(p, W->q, W->type == ML_Q4_0 ? n / 2 : n);
    d.d = place(p, f16 ? (const void *)W->dh : (const void *)W->d, n / QK * (f16 ? 2 : 4));
    return d;
}

ml_status kr_model_upload(kr_model *m) {
    if (m->dev) return ML_OK;
    ml_status st = krh_init();
    if (st != ML_OK) return kr_seterr(st, "%s", krh_last_error());
    const ml_config *c = &m->cfg;
    const int f16 = c->scale_f16;
    const size_t fd = sizeof(float) * (size_t)c->dim;
    size_t total = mat_bytes(&m->tok_emb, f16) + RUP(fd);
    if (!m->shared) total += mat_bytes(&m->wcls, f16);
    for (int l = 0; l < c->n_layers; l++) {
        const ml_layer *L = &m->layers[l];
        const ml_qtensor *ws[7] = { &L->wq, &L->wk, &L->wv, &L->wo, &L->w1, &L->w2, &L->w3 };
        for (int k = 0; k < 7; k++) total += mat_bytes(ws[k], f16);
        total += 2 * RUP(fd);
        if (L->bq) total += RUP(sizeof(float) * c->q_dim) + 2 * RUP(sizeof(float) * c->kv_dim);
        if (L->q_norm) total += 2 * RUP(sizeof(float) * c->head_dim);
        if (L->post_attn_norm) total += 2 * RUP(fd);
    }
    m->dev = krh_alloc(total);
    if (!m->dev) return kr_seterr(ML_E_NOMEM, "cannot allocate %zu bytes of HBM for the weights", total);
    m->dev_bytes = total;
    m->d_layers = calloc((size_t)c->n_layers, sizeof *m->d_layers);
    if (!m->d_layers) return ML_E_NOMEM;
    placer p = { m->dev, 0, ML_OK };
    m->d_tok_emb = place_mat(&p, &m->tok_emb, f16);
    for (int l = 0; l < c->n_layers; l++) {
        const ml_layer *L = &m->layers[l];
        struct kr_dev_layer *D = &m->d_layers[l];
        D->attn_norm = place(&p, L->attn_norm, fd);
        D->ffn_norm = place(&p, L->ffn_norm, fd);
        D->wq = place_mat(&p, &L->wq, f16);
        D->wk = place_mat(&p, &L->wk, f16);
        D->wv = place_mat(&p, &L->wv, f16);
        D->wo = place_mat(&p, &L->wo, f16);
        D->w1 = place_mat(&p, &L->w1, f16);
        D->w2 = place_mat(&p, &L->w2, f16);
        D->w3 = place_mat(&p, &L->w3, f16);
        if (L->bq) {
            D->bq = place(&p, L->bq, sizeof(float) * c->q_dim);
            D->bk = place(&p, L->bk, sizeof(float) * c->kv_dim);
            D->bv = place(&p, L->bv, sizeof(float) * c->kv_dim);
        }
        if (L->q_norm) {
            D->q_norm = place(&p, L->q_norm, sizeof(float) * c->head_dim);
            D->k_norm = place(&p, L->k_norm, sizeof(float) * c->head_dim);
        }
        if (L->post_attn_norm) {
            D->post_attn_norm = place(&p, L->post_attn_norm, fd);
            D->post_ffn_norm = place(&p, L->post_ffn_norm, fd);
        }
    }
    m->d_final_norm = place(&p, m->final_norm, fd);
    m->d_wcls = m->shared ? m->d_tok_emb : place_mat(&p, &m->wcls, f16);
    return p.st;
}

size_t kr_model_device_bytes(const kr_model *m) { return m->dev_bytes; }

const krh_mat *kr_model_device_mat(const kr_model *m, int layer, const char *name) {
    if (!m->dev) return NULL;
    if (!strcmp(name, "tok_emb")) return &m->d_tok_emb;
    if (!strcmp(name, "wcls")) return &m->d_wcls;
    if (layer < 0 || layer >= m->cfg.n_layers) return NULL;
    const struct kr_dev_layer *D = &m->d_layers[layer];
    static const char *const names[] = { "wq", "wk", "wv", "wo", "w1", "w2", "w3" };
    const krh_mat *mats[] = { &D->wq, &D->wk, &D->wv, &D->wo, &D->w1, &D->w2, &D->w3 };
    for (int i = 0; i < 7; i++)
        if (!strcmp(names[i], name)) return mats[i];
    return NULL;
}

const float *kr_model_device_vec(const kr_model *m, int layer, const char *name) {
    if (!m->dev) return NULL;
    if (!strcmp(name, "final_norm")) return m->d_final_norm;
    if (layer < 0 || layer >= m->cfg.n_layers) return NULL;
    const struct kr_dev_layer *D = &m->d_layers[layer];
    if (!strcmp(name, "attn_norm")) return D->attn_norm;
    if (!strcmp(name, "ffn_norm")) return D->ffn_norm;
    if (!strcmp(name, "bq")) return D->bq;
    if (!strcmp(name, "bk")) return D->bk;
    if (!strcmp(name, "bv")) return D->bv;
    return NULL;
}

void kr_model_free(kr_model *m) {
    if (!m) return;
    krh_free(m->dev);
    free(m->d_layers);
    free(m->layers);
    if (m->map) munmap(m->map, m->size);
    free(m);
}

/* ---- state ---- */

struct kr_state {
    kr_model *m;
    /* device buffers */
    float *x, *q, *ao, *hb, *att, *logits, *rope_cos, *rope_sin, *rope_cos_l, *rope_sin_l;
    int kv_type;              /* ML_F32, ML_F16 or ML_Q8_0 (ml_state.kv_type, model/transformer.h:19-26) */
    void *kcache, *vcache;    /* [n_layers][max_seq][kv_dim] floats, halves or int8 */
    float *kd, *vd;           /* Q8: row scales [n_layers][max_seq][n_kv_heads] */
    float *kst, *vst;         /* Q8 and the families' path: the projections' K and V rows (kbuf, vbuf) */
    float *yb;                /* post-norms: a block's output before its norm (xb2) */
    float *hb2;               /* GELU: the up projection (hb2) */
    int family;               /* q/k-norm, post-norms, GELU or soft-capping: the unfused layer path */
    int8_t *qa_dim, *qa_q, *qa_hid;
    float *qd_dim, *qd_q, *qd_hid;
    int *tok, *pos, *prompt, *log;
    void *mem;
    float *h_logits;          /* pinned */
    int *h_ints;              /* pinned: tok, pos */
    krh_graph *g_logits, *g_greedy, *g_prefill, *g_sample;
    krh_sampler *smp;         /* the device sampler of kr_generate, or NULL: greedy */
    int batch;                /* tokens per batched prefill step; 1: token by token */
    int eager;                /* issue ops directly instead of replaying graphs */
    /* batched prefill buffers (allocated on first use): [ldx] token rows */
    void *bmem;
    int ldx;                  /* capacity, a multiple of 128 */
    float *bx, *bq, *bao, *bh1, *bh3, *batt, *blog, *bxd, *bkst, *bvst;
    int8_t *bxq;
};

static size_t kv_elem(int kv_type) { return kv_type == ML_F32 ? 4 : kv_type == ML_F16 ? 2 : 1; }

/* layer l's cache view (model/transformer.c:169-180) over device memory */
static ml_kv_layer kv_layer(const kr_state *s, int l) {
    const ml_config *c = &s->m->cfg;
    const size_t rows = (size_t)l * c->max_seq, e = (size_t)c->kv_dim * kv_elem(s->kv_type);
    const char *kc = (const char *)s->kcache + rows * e, *vc = (const char *)s->vcache + rows * e;
    ml_kv_layer kv = { 0 };
    kv.window = s->m->layers[l].window;
    if (s->kv_type == ML_F32) {
        kv.k = (const float *)kc;
        kv.v = (const float *)vc;
    } else if (s->kv_type == ML_F16) {
        kv.kh = (const uint16_t *)kc;
        kv.vh = (const uint16_t *)vc;
    } else {
        kv.kq = (const int8_t *)kc;
        kv.vq = (const int8_t *)vc;
        kv.kd = s->kd + rows * c->n_kv_heads;
        kv.vd = s->vd + rows * c->n_kv_heads;
    }
    return kv;
}

/* store_kv of ntok positions from *s->pos into layer l (F16 / Q8) */
static void store_kv(kr_state *s, int l, const float *k, const float *v, int ntok) {
    const ml_config *c = &s->m->cfg;
    const size_t rows = (size_t)l * c->max_seq, e = (size_t)c->kv_dim * kv_elem(s->kv_type);
    const int q8 = s->kv_type == ML_Q8_0;
    krh_store_kv(s->kv_type, (char *)s->kcache + rows * e, (char *)s->vcache + rows * e,
                 q8 ? s->kd + rows * c->n_kv_heads : NULL, q8 ? s->vd + rows * c->n_kv_heads : NULL, k, v,
                 c->n_kv_heads, c->head_dim, s->pos, ntok);
}

/* tokens per batched prefill step by default (the attention scratch is
 * [step][n_heads][max_seq] floats) */
#define KR_PREFILL_STEP 2048

/* model/transformer.c:16-38: inverse frequency of rotary pair i */
static double rope_inv_freq(const ml_config *c, int i) {
    const double inv = pow((double)c->rope_theta, -2.0 * i / c->head_dim);
    if (c->rope_type == ML_ROPE_LINEAR) return inv / c->rope_factor;
    if (c->rope_type == ML_ROPE_YARN) {
        const double hd = c->head_dim, orig = c->rope_orig_max_seq, lb = 2.0 * log((double)c->rope_theta);
        const double pi2 = 2.0 * 3.14159265358979323846;
        double lo = floor(hd * log(orig / ((double)c->rope_low_freq_factor * pi2)) / lb);
        double hi = ceil(hd * log(orig / ((double)c->rope_high_freq_factor * pi2)) / lb);
        lo = lo < 0.0 ? 0.0 : lo;
        hi = hi > hd - 1.0 ? hd - 1.0 : hi;
        if (lo == hi) hi += 0.001;
        double ramp = (i - lo) / (hi - lo);
        ramp = ramp < 0.0 ? 0.0 : (ramp > 1.0 ? 1.0 : ramp);
        return inv / c->rope_factor * ramp + inv * (1.0 - ramp);
    }
    if (c->rope_type != ML_ROPE_LLAMA3) return inv;
    const double f = c->rope_factor, lo = c->rope_low_freq_factor, hi = c->rope_high_freq_factor;
    const double orig = c->rope_orig_max_seq, wavelen = 2.0 * 3.14159265358979323846 / inv;
    if (wavelen < orig / hi) return inv;
    if (wavelen > orig / lo) return inv / f;
    const double smooth = (orig / wavelen - lo) / (hi - lo);
    return (1.0 - smooth) * inv / f + smooth * inv;
}

/* The tables in double on the host, then rounded to float, exactly as
 * model/transformer.c:147-162 builds them. */
static void rope_tables(const ml_config *c, float *cs, float *sn, float *cs_l, float *sn_l) {
    const int h2 = c->head_dim / 2;
    const double af = c->rope_type == ML_ROPE_YARN ? c->rope_attn_factor : 1.0;
    for (int i = 0; i < h2; i++) {
        const double freq = rope_inv_freq(c, i);
        const double lfreq = cs_l ? pow((double)c->rope_local_theta, -2.0 * i / c->head_dim) : 0.0;
        for (int p = 0; p < c->max_seq; p++) {
            const double ang = p * freq;
            cs[(size_t)p * h2 + i] = (float)(cos(ang) * af);
            sn[(size_t)p * h2 + i] = (float)(sin(ang) * af);
            if (cs_l) {
                cs_l[(size_t)p * h2 + i] = (float)cos(p * lfreq);
                sn_l[(size_t)p * h2 + i] = (float)sin(p * lfreq);
            }
        }
    }
}

/* ml_forward's ops for the token in s->tok at position s->pos; cls: run the
 * final norm and the classifier too */
static void issue_family_layer(kr_state *s, int l, const float *cs, const float *sn);
static void issue_step(kr_state *s, int cls) {
    const kr_model *m = s->m;
    const ml_config *c = &m->cfg;
    const size_t lkv = (size_t)c->max_seq * c->kv_dim;
    krh_embed(s->x, &m->d_tok_emb, s->tok, c->embed_scale);
    for (int l = 0; l < c->n_layers; l++) {
        const struct kr_dev_layer *D = &m->d_layers[l];
        const ml_layer *L = &m->layers[l];
        const float *cs = L->local_rope ? s->rope_cos_l : s->rope_cos, *sn = L->local_rope ? s->rope_sin_l : s->rope_sin;
        if (s->family) {
            issue_family_layer(s, l, cs, sn);
            continue;
        }
        /* each norm runs inside the launch that consumes it, under that
         * launch's first weight loads */
        if (s->kv_type == ML_F32) {
            float *kc = (float *)s->kcache + (size_t)l * lkv, *vc = (float *)s->vcache + (size_t)l * lkv;
            krh_rmsnorm_matvec_qkv(s->q, kc, vc, &D->wq, &D->wk, &D->wv, D->bq, D->bk, D->bv, s->x, D->attn_norm,
                                   c->norm_eps, cs, sn, c->head_dim, s->pos);
            krh_attention(s->ao, NULL, NULL, s->att, s->q, kc, vc, c->n_heads, c->n_kv_heads, c->head_dim,
                          c->max_seq, L->window, c->attn_scale, s->pos);
        } else {
            const ml_kv_layer kv = kv_layer(s, l);
            if (s->kv_type == ML_F16) {   /* the rows rounded to halves in the projection's epilogue */
                uint16_t *kh = (uint16_t *)s->kcache + (size_t)l * lkv, *vh = (uint16_t *)s->vcache + (size_t)l * lkv;
                krh_rmsnorm_matvec_qkv_f16(s->q, kh, vh, &D->wq, &D->wk, &D->wv, D->bq, D->bk, D->bv, s->x,
                                           D->attn_norm, c->norm_eps, cs, sn, c->head_dim, s->pos);
                krh_attention_kv(s->ao, s->att, s->q, &kv, c->n_heads, c->n_kv_heads, c->head_dim, c->max_seq,
                                 c->attn_scale, s->pos, 1, c->max_seq - 1);
            } else {   /* Q8: the score launch stores row *pos (store_kv) before reading it */
                krh_rmsnorm_matvec_qkv_stage(s->q, s->kst, s->vst, &D->wq, &D->wk, &D->wv, D->bq, D->bk, D->bv, s->x,
                                             D->attn_norm, c->norm_eps, cs, sn, c->head_dim, s->pos);
                krh_attention_q8_store(s->ao, s->att, s->q, &kv, s->kst, s->vst, c->n_heads, c->n_kv_heads,
                                       c->head_dim, c->max_seq, c->attn_scale, s->pos);
            }
        }
        krh_matvec_f(s->x, &D->wo, s->ao, 1);
        krh_rmsnorm_matvec_swiglu(s->hb, &D->w1, &D->w3, s->x, D->ffn_norm, c->norm_eps);
        krh_matvec_f(s->x, &D->w2, s->hb, 1);   /* h quantized in the w2 launch's prologue */
    }
    if (!cls) return;
    krh_rmsnorm_matvec(s->logits, &m->d_wcls, s->x, m->d_final_norm, c->norm_eps, 0);
    if (c->final_softcap > 0.0f)   /* model/transformer.c:304 */
        krh_softcap_rows(s->logits, (size_t)c->vocab, 1, c->vocab, c->final_softcap);
}

/* A layer of a model with q/k-norm (Qwen3), post-norms (Gemma 3), GELU or
 * soft-capped scores (Gemma 2), in
 * ml_forward's order with unfused launches (model/transformer.c:266-297): the
 * projections store q and the staging rows k, v unrotated; the biases; each
 * head normalized, then rotated at *pos; the cache row stored; attention;
 * each block's output normalized before its residual add. */
static void issue_family_layer(kr_state *s, int l, const float *cs, const float *sn) {
    const kr_model *m = s->m;
    const ml_config *c = &m->cfg;
    const struct kr_dev_layer *D = &m->d_layers[l];
    krh_rmsnorm_q8(s->qa_dim, s->qd_dim, NULL, s->x, D->attn_norm, c->dim, c->norm_eps, 1);
    krh_matvec(s->q, &D->wq, s->qa_dim, s->qd_dim, 0);
    krh_matvec(s->kst, &D->wk, s->qa_dim, s->qd_dim, 0);
    krh_matvec(s->vst, &D->wv, s->qa_dim, s->qd_dim, 0);
    if (D->bq) {
        krh_add(s->q, D->bq, c->q_dim);
        krh_add(s->kst, D->bk, c->kv_dim);
        krh_add(s->vst, D->bv, c->kv_dim);
    }
    krh_heads_norm_rope(s->q, s->kst, D->q_norm, D->k_norm, cs, sn, c->head_dim, c->n_heads, c->n_kv_heads,
                        c->norm_eps, s->pos);
    const ml_kv_layer kv = kv_layer(s, l);
    if (s->kv_type == ML_F32)
        krh_store_rows_f32((float *)kv.k, (float *)kv.v, s->kst, s->vst, c->kv_dim, s->pos);
    else
        store_kv(s, l, s->kst, s->vst, 1);
    krh_attention_kv_softcap(s->ao, s->att, s->q, &kv, c->n_heads, c->n_kv_heads, c->head_dim, c->max_seq,
                             c->attn_scale, s->pos, 1, c->max_seq - 1, c->attn_softcap);
    if (D->post_attn_norm) {
        krh_matvec_f(s->yb, &D->wo, s->ao, 0);
        krh_rmsnorm(s->yb, s->yb, D->post_attn_norm, c->dim, c->norm_eps);
        krh_add(s->x, s->yb, c->dim);
    } else {
        krh_matvec_f(s->x, &D->wo, s->ao, 1);
    }
    if (c->act == ML_ACT_GELU_TANH) {   /* act_mul (model/transformer.c:233-236) */
        krh_rmsnorm_q8(s->qa_dim, s->qd_dim, NULL, s->x, D->ffn_norm, c->dim, c->norm_eps, 1);
        krh_matvec(s->hb, &D->w1, s->qa_dim, s->qd_dim, 0);
        krh_matvec(s->hb2, &D->w3, s->qa_dim, s->qd_dim, 0);
        krh_gelu_mul(s->hb, s->hb2, c->hidden_dim);
    } else {
        krh_rmsnorm_matvec_swiglu(s->hb, &D->w1, &D->w3, s->x, D->ffn_norm, c->norm_eps);
    }
    if (D->post_ffn_norm) {
        krh_matvec_f(s->yb, &D->w2, s->hb, 0);
        krh_rmsnorm(s->yb, s->yb, D->post_ffn_norm, c->dim, c->norm_eps);
        krh_add(s->x, s->yb, c->dim);
    } else {
        krh_matvec_f(s->x, &D->w2, s->hb, 1);
    }
}

enum { STEP_LOGITS = 0, STEP_GREEDY = 1, STEP_PREFILL = 2, STEP_SAMPLE = 3 };

/* The ops of one replayed step: STEP_LOGITS (ml_forward), STEP_GREEDY
 * (ml_forward + the greedy pick, appended to the id log), STEP_PREFILL (the
 * next prompt token into the cache, no classifier), STEP_SAMPLE (ml_forward
 * + the sampler's draw and accept, appended to the id log). */
static void issue(kr_state *s, int kind) {
    if (kind == STEP_PREFILL) krh_take_token(s->tok, s->prompt, s->pos);
    issue_step(s, kind != STEP_PREFILL);
    if (kind == STEP_GREEDY) krh_argmax(s->tok, s->logits, s->m->cfg.vocab, s->pos, s->log);
    if (kind == STEP_SAMPLE) krh_sample(s->smp, s->tok, s->logits, s->m->cfg.vocab, s->pos, s->log);
    if (kind == STEP_PREFILL) krh_advance(s->pos);
}

static ml_status capture(kr_state *s, krh_graph **g, int kind) {
    ml_status st = krh_graph_begin();
    if (st != ML_OK) return kr_seterr(st, "%s", krh_last_error());
    issue(s, kind);
    st = krh_graph_end(g);
    return st == ML_OK ? ML_OK : kr_seterr(st, "%s", krh_last_error());
}

/* Runs a step: replays its graph, or issues its ops one by one when the
 * state is eager (KRAFLA_EAGER=1 in the environment: for profilers that
 * trace kernel dispatches, and for debugging) */
static ml_status run_step(kr_state *s, int kind) {
    if (s->eager) {
        issue(s, kind);
        return krh_status();
    }
    const krh_graph *g = kind == STEP_LOGITS   ? s->g_logits
                         : kind == STEP_GREEDY ? s->g_greedy
                         : kind == STEP_SAMPLE ? s->g_sample
                                               : s->g_prefill;
    return krh_graph_launch(g);
}

ml_status kr_state_new(kr_state **out, kr_model *m, int kv_type) {
    *out = NULL;
    const ml_config *c = &m->cfg;
    if (kv_type != ML_F32 && kv_type != ML_F16 && kv_type != ML_Q8_0)
        return kr_seterr(ML_E_SHAPE, "KV cache type %d: F32, F16 or Q8_0", kv_type);
    ml_status st = kr_model_upload(m);
    if (st != ML_OK) return st;
    kr_state *s = calloc(1, sizeof *s);
    if (!s) return ML_E_NOMEM;
    s->m = m;
    s->kv_type = kv_type;
    const size_t f = sizeof(float), kv = (size_t)c->n_layers * c->max_seq * c->kv_dim;
    const size_t ks = (size_t)c->n_layers * c->max_seq * c->n_kv_heads;
    const int gelu = c->act == ML_ACT_GELU_TANH;
    const int q8 = kv_type == ML_Q8_0,
              fam = c->qk_norm || c->post_norms || gelu || c->attn_softcap > 0.0f || c->final_softcap > 0.0f;
    s->family = fam;
    const size_t half = (size_t)c->max_seq * (c->head_dim / 2);
    const int local = c->rope_local_theta > 0.0f;
    struct { void **p; size_t n; } parts[] = {
        { (void **)&s->x, f * c->dim }, { (void **)&s->q, f * c->q_dim }, { (void **)&s->ao, f * c->q_dim },
        { (void **)&s->hb, f * c->hidden_dim },
        { (void **)&s->att, f * (size_t)c->n_heads * c->max_seq }, { (void **)&s->logits, f * c->vocab },
        { (void **)&s->kcache, kv_elem(kv_type) * kv }, { (void **)&s->vcache, kv_elem(kv_type) * kv },
        { (void **)&s->kd, q8 ? f * ks : 0 }, { (void **)&s->vd, q8 ? f * ks : 0 },
        { (void **)&s->kst, q8 || fam ? f * c->kv_dim : 0 }, { (void **)&s->vst, q8 || fam ? f * c->kv_dim : 0 },
        { (void **)&s->yb, c->post_norms ? f * c->dim : 0 }, { (void **)&s->hb2, gelu ? f * c->hidden_dim : 0 },
        { (void **)&s->rope_cos, f * half }, { (void **)&s->rope_sin, f * half },
        { (void **)&s->rope_cos_l, local ? f * half : 0 }, { (void **)&s->rope_sin_l, local ? f * half : 0 },
        { (void **)&s->qa_dim, (size_t)c->dim }, { (void **)&s->qd_dim, f * c->dim / QK },
        { (void **)&s->qa_q, (size_t)c->q_dim }, { (void **)&s->qd_q, f * c->q_dim / QK },
        { (void **)&s->qa_hid, (size_t)c->hidden_dim }, { (void **)&s->qd_hid, f * c->hidden_dim / QK },
        { (void **)&s->tok, sizeof(int) }, { (void **)&s->pos, sizeof(int) },
        { (void **)&s->prompt, sizeof(int) * ((size_t)c->max_seq + 1) },
        { (void **)&s->log, sizeof(int) * ((size_t)c->max_seq + 2) },
    };
    const int np = (int)(sizeof parts / sizeof parts[0]);
    size_t total = 0;
    for (int i = 0; i < np; i++) total += RUP(parts[i].n);
    s->mem = krh_alloc(total);
    s->h_logits = krh_host_alloc(f * c->vocab);
    s->h_ints = krh_host_alloc(sizeof(int) * 4);
    if (!s->mem || !s->h_logits || !s->h_ints) {
        kr_state_free(s);
        return kr_seterr(ML_E_NOMEM, "cannot allocate the decoding state (%zu bytes of HBM)", total);
    }
    size_t off = 0;
    for (int i = 0; i < np; i++) {
        *parts[i].p = parts[i].n ? (uint8_t *)s->mem + off : NULL;
        off += RUP(parts[i].n);
    }
    float *cs = malloc(f * half), *sn = malloc(f * half);
    float *csl = local ? malloc(f * half) : NULL, *snl = local ? malloc(f * half) : NULL;
    if (!cs || !sn || (local && (!csl || !snl))) {
        free(cs); free(sn); free(csl); free(snl);
        kr_state_free(s);
        return ML_E_NOMEM;
    }
    rope_tables(c, cs, sn, csl, snl);
    st = krh_copy_h2d(s->rope_cos, cs, f * half);
    if (st == ML_OK) st = krh_copy_h2d(s->rope_sin, sn, f * half);
    if (st == ML_OK && local) st = krh_copy_h2d(s->rope_cos_l, csl, f * half);
    if (st == ML_OK && local) st = krh_copy_h2d(s->rope_sin_l, snl, f * half);
    free(cs); free(sn); free(csl); free(snl);
    s->batch = c->max_seq < KR_PREFILL_STEP ? c->max_seq : KR_PREFILL_STEP;
    const char *ev = getenv("KRAFLA_EAGER");
    s->eager = ev && ev[0] == '1';
    if (st == ML_OK && !s->eager) st = capture(s, &s->g_logits, STEP_LOGITS);
    if (st == ML_OK && !s->eager) st = capture(s, &s->g_greedy, STEP_GREEDY);
    if (st == ML_OK && !s->eager) st = capture(s, &s->g_prefill, STEP_PREFILL);
    if (st != ML_OK) {
        kr_state_free(s);
        return kr_seterr(st, "%s", krh_last_error());
    }
    *out = s;
    return ML_OK;
}

void kr_state_free(kr_state *s) {
    if (!s) return;
    krh_free(s->bmem);
    krh_graph_free(s->g_logits);
    krh_graph_free(s->g_greedy);
    krh_graph_free(s->g_prefill);
    krh_graph_free(s->g_sample);
    krh_sampler_free(s->smp);
    krh_free(s->mem);
    krh_host_free(s->h_logits);
    krh_host_free(s->h_ints);
    free(s);
}

ml_status kr_state_set_sampler(kr_state *s, const krh_sampler_opts *o) {
    krh_graph_free(s->g_sample);
    krh_sampler_free(s->smp);
    s->g_sample = NULL;
    s->smp = NULL;
    if (!o) return ML_OK;
    ml_status st = krh_sampler_new(&s->smp, s->m->cfg.vocab, o);
    if (st == ML_OK && !s->eager) st = capture(s, &s->g_sample, STEP_SAMPLE);
    if (st != ML_OK) {
        krh_sampler_free(s->smp);
        s->smp = NULL;
        return kr_seterr(st, "%s", krh_last_error());
    }
    return ML_OK;
}

void kr_state_set_batch(kr_state *s, int batch) {
    if (batch < 1) batch = KR_PREFILL_STEP;
    if (batch > s->m->cfg.max_seq) batch = s->m->cfg.max_seq;
    if (batch != s->batch && s->bmem) {   /* re-sized on next use */
        krh_free(s->bmem);
        s->bmem = NULL;
    }
    s->batch = batch;
}
const float *kr_state_x_device(const kr_state *s) { return s->x; }

const void *kr_state_buffer(const kr_state *s, const char *name) {
    static const char *const names[] = { "x", "q", "ao", "hb", "att", "logits", "kcache", "vcache", "rope_cos",
                                         "rope_sin", "qa_dim", "qd_dim", "qa_q", "qd_q", "qa_hid", "qd_hid", "kd", "vd" };
    const void *ptrs[] = { s->x, s->q, s->ao, s->hb, s->att, s->logits, s->kcache, s->vcache, s->rope_cos,
                           s->rope_sin, s->qa_dim, s->qd_dim, s->qa_q, s->qd_q, s->qa_hid, s->qd_hid, s->kd, s->vd };
    for (size_t i = 0; i < sizeof names / sizeof names[0]; i++)
        if (!strcmp(names[i], name)) return ptrs[i];
    return NULL;
}

static ml_status set_ints(kr_state *s, int tok, int pos) {
    s->h_ints[0] = tok;
    s->h_ints[1] = pos;
    ml_status st = krh_copy_h2d(s->tok, &s->h_ints[0], sizeof(int));
    if (st == ML_OK) st = krh_copy_h2d(s->pos, &s->h_ints[1], sizeof(int));
    return st;
}

static ml_status dev_status(void) {
    const ml_status st = krh_sync();
    return st == ML_OK ? ML_OK : kr_seterr(st, "%s", krh_last_error());
}

ml_status kr_forward(kr_state *s, int token, int pos, float *logits) {
    const ml_config *c = &s->m->cfg;
    if (pos < 0 || pos >= c->max_seq || token < 0 || token >= c->vocab) return ML_E_SHAPE;
    ml_status st = set_ints(s, token, pos);
    if (st == ML_OK) st = run_step(s, STEP_LOGITS);
    if (st == ML_OK && logits) st = krh_copy_d2h(logits, s->logits, sizeof(float) * c->vocab);
    return st == ML_OK ? dev_status() : st;
}

static ml_status batch_buffers(kr_state *s, int with_logits) {
    const ml_config *c = &s->m->cfg;
    const int ldx = (s->batch + 127) / 128 * 128;
    if (s->bmem && (!with_logits || s->blog)) return ML_OK;
    krh_free(s->bmem);
    s->bmem = NULL;
    s->blog = NULL;
    const size_t f = sizeof(float), L = (size_t)ldx;
    const int wide = c->hidden_dim > c->q_dim ? (c->hidden_dim > c->dim ? c->hidden_dim : c->dim)
                                              : (c->q_dim > c->dim ? c->q_dim : c->dim);
    struct { void **p; size_t n; } parts[] = {
        { (void **)&s->bx, f * L * c->dim }, { (void **)&s->bq, f * L * c->q_dim },
        { (void **)&s->bao, f * L * c->q_dim }, { (void **)&s->bh1, f * L * c->hidden_dim },
        { (void **)&s->bh3, f * L * (c->hidden_dim > c->dim ? c->hidden_dim : c->dim) }, { (void **)&s->batt, f * L * c->n_heads * (size_t)c->max_seq },
        { (void **)&s->bxq, L * wide }, { (void **)&s->bxd, f * L * (wide / QK) },
        { (void **)&s->blog, with_logits ? f * L * c->vocab : 0 },
        { (void **)&s->bkst, s->kv_type != ML_F32 || s->family ? f * L * c->kv_dim : 0 },
        { (void **)&s->bvst, s->kv_type != ML_F32 || s->family ? f * L * c->kv_dim : 0 },
    };
    size_t total = 0;
    for (size_t i = 0; i < sizeof parts / sizeof parts[0]; i++) total += RUP(parts[i].n);
    s->bmem = krh_alloc(total);
    if (!s->bmem) return kr_seterr(ML_E_NOMEM, "cannot allocate %zu bytes of HBM for batched prefill", total);
    size_t off = 0;
    for (size_t i = 0; i < sizeof parts / sizeof parts[0]; i++) {
        *parts[i].p = parts[i].n ? (uint8_t *)s->bmem + off : NULL;
        off += RUP(parts[i].n);
    }
    s->ldx = ldx;
    return ML_OK;
}

/* whether a prompt step of T tokens takes the FFN as one launch
 * (krh_matmul_swiglu: 64-row tiles of w1 and w3 together): from 3/4 of a
 * tile per compute unit, where the single launch fills the device; shorter
 * steps keep the separate products, whose 32-row tiles do. */
static int swiglu_fused(const kr_state *s, const struct kr_dev_layer *D, int T) {
    const ml_config *c = &s->m->cfg;
    if (D->w1.type != D->w3.type || D->w1.d16 != D->w3.d16 || c->hidden_dim % 32) return 0;
    const long tiles = (long)(c->hidden_dim + 63) / 64 * ((T + 127) / 128);
    const int cus = krh_device_cus() > 0 ? krh_device_cus() : 256;
    return 4 * tiles >= 3L * cus;
}

/* rmsnorm of rows rows of n floats in place, w shared, in launches of at
 * most KRH_ROWS_MAX rows (the per-head norms of a batch) */
static void norm_rows(float *x, const float *w, int n, float eps, long rows) {
    for (long r = 0; r < rows; r += KRH_ROWS_MAX) {
        const int k = rows - r < KRH_ROWS_MAX ? (int)(rows - r) : KRH_ROWS_MAX;
        krh_rmsnorm_rows(x + (size_t)r * n, (size_t)n, x + (size_t)r * n, (size_t)n, w, 0, n, eps, k);
    }
}

/* A block's output y [T][dim] into the residual x (residual_add,
 * model/transformer.c:240-243): normalized first when the model has
 * post-norms */
static void residual_rows(kr_state *s, float *y, const float *post_norm, int T) {
    const ml_config *c = &s->m->cfg;
    if (post_norm) krh_rmsnorm_rows(y, (size_t)c->dim, y, (size_t)c->dim, post_norm, 0, c->dim, c->norm_eps, T);
    krh_add_rows(s->bx, (size_t)c->dim, y, (size_t)c->dim, c->dim, T);
}

/* One batched layer of a model with q/k-norm, post-norms, GELU or
 * soft-capped scores: the per-token stages of model/transformer.c:324-365
 * (token_stage) as row launches over the T tokens, the products as int8
 * MFMA matmuls without fused RoPE. K and V rows go straight into an F32
 * cache's rows (its rows are the projections' outputs, :390-391), else to
 * the staging rows that store_kv converts. */
static void family_prefill_layer(kr_state *s, int l, int T, int p0) {
    const kr_model *m = s->m;
    const ml_config *c = &m->cfg;
    const struct kr_dev_layer *D = &m->d_layers[l];
    const ml_layer *L = &m->layers[l];
    const int ldx = s->ldx, hd = c->head_dim, h2 = hd / 2;
    const size_t lkv = (size_t)c->max_seq * c->kv_dim;
    const float *cs = L->local_rope ? s->rope_cos_l : s->rope_cos, *sn = L->local_rope ? s->rope_sin_l : s->rope_sin;
    const int f32 = s->kv_type == ML_F32;
    float *k = f32 ? (float *)s->kcache + (size_t)l * lkv + (size_t)p0 * c->kv_dim : s->bkst;
    float *v = f32 ? (float *)s->vcache + (size_t)l * lkv + (size_t)p0 * c->kv_dim : s->bvst;
    krh_rmsnorm_q8_t(s->bxq, s->bxd, ldx, NULL, s->bx, D->attn_norm, c->dim, c->norm_eps, T);   /* TOK_ATTN_IN */
    krh_matmul(s->bq, c->q_dim, &D->wq, s->bxq, s->bxd, ldx, T, 0);
    krh_matmul(k, c->kv_dim, &D->wk, s->bxq, s->bxd, ldx, T, 0);
    krh_matmul(v, c->kv_dim, &D->wv, s->bxq, s->bxd, ldx, T, 0);
    if (D->bq) {   /* TOK_QKV_OUT */
        krh_add_rows(s->bq, (size_t)c->q_dim, D->bq, 0, c->q_dim, T);
        krh_add_rows(k, (size_t)c->kv_dim, D->bk, 0, c->kv_dim, T);
        krh_add_rows(v, (size_t)c->kv_dim, D->bv, 0, c->kv_dim, T);
    }
    if (D->q_norm) {
        norm_rows(s->bq, D->q_norm, hd, c->norm_eps, (long)T * c->n_heads);
        norm_rows(k, D->k_norm, hd, c->norm_eps, (long)T * c->n_kv_heads);
    }
    krh_rope_rows(s->bq, (size_t)c->q_dim, k, (size_t)c->kv_dim, cs + (size_t)p0 * h2, (size_t)h2,
                  sn + (size_t)p0 * h2, (size_t)h2, hd, c->n_heads, c->n_kv_heads, T);
    if (!f32) store_kv(s, l, s->bkst, s->bvst, T);
    const ml_kv_layer kv = kv_layer(s, l);
    krh_attention_kv_softcap(s->bao, s->batt, s->bq, &kv, c->n_heads, c->n_kv_heads, hd, c->max_seq,
                             c->attn_scale, s->pos, T, p0 + T - 1, c->attn_softcap);
    krh_quantize_q8_t(s->bxq, s->bxd, ldx, s->bao, c->q_dim, T);   /* TOK_WO_IN */
    if (D->post_attn_norm) {   /* TOK_FFN_IN: bh3 holds the block's output rows [T][dim] */
        krh_matmul(s->bh3, c->dim, &D->wo, s->bxq, s->bxd, ldx, T, 0);
        residual_rows(s, s->bh3, D->post_attn_norm, T);
    } else {
        krh_matmul(s->bx, c->dim, &D->wo, s->bxq, s->bxd, ldx, T, 1);
    }
    krh_rmsnorm_q8_t(s->bxq, s->bxd, ldx, NULL, s->bx, D->ffn_norm, c->dim, c->norm_eps, T);
    krh_matmul(s->bh1, c->hidden_dim, &D->w1, s->bxq, s->bxd, ldx, T, 0);
    krh_matmul(s->bh3, c->hidden_dim, &D->w3, s->bxq, s->bxd, ldx, T, 0);
    if (c->act == ML_ACT_GELU_TANH) {   /* TOK_DOWN_IN */
        krh_gelu_mul_rows(s->bh1, (size_t)c->hidden_dim, s->bh3, (size_t)c->hidden_dim, c->hidden_dim, T);
        krh_quantize_q8_t(s->bxq, s->bxd, ldx, s->bh1, c->hidden_dim, T);
    } else {
        krh_silu_quant(s->bxq, s->bxd, ldx, s->bh1, s->bh3, c->hidden_dim, T);
    }
    if (D->post_ffn_norm) {   /* TOK_RESID */
        krh_matmul(s->bh3, c->dim, &D->w2, s->bxq, s->bxd, ldx, T, 0);
        residual_rows(s, s->bh3, D->post_ffn_norm, T);
    } else {
        krh_matmul(s->bx, c->dim, &D->w2, s->bxq, s->bxd, ldx, T, 1);
    }
}

/* One batched step (model/transformer.c:385-425): T tokens at positions
 * p0.. through every layer with the matrix products shared by the tokens;
 * every per-token operation is ml_forward's, so the cache and the logits are
 * those of token-by-token decoding, bit for bit. */
static ml_status prefill_step(kr_state *s, const int *tokens, int T, int p0, float *logits) {
    const kr_model *m = s->m;
    const ml_config *c = &m->cfg;
    const size_t lkv = (size_t)c->max_seq * c->kv_dim;
    const int ldx = s->ldx;
    ml_status st = krh_copy_h2d(s->prompt, tokens, sizeof(int) * (size_t)T);
    if (st == ML_OK) st = set_ints(s, 0, p0);
    if (st != ML_OK) return kr_seterr(st, "%s", krh_last_error());
    krh_embed_batch(s->bx, &m->d_tok_emb, s->prompt, T, c->embed_scale);
    for (int l = 0; l < c->n_layers; l++) {
        const struct kr_dev_layer *D = &m->d_layers[l];
        const ml_layer *L = &m->layers[l];
        const float *cs = L->local_rope ? s->rope_cos_l : s->rope_cos, *sn = L->local_rope ? s->rope_sin_l : s->rope_sin;
        if (s->family) {
            family_prefill_layer(s, l, T, p0);
            continue;
        }
        krh_rmsnorm_q8_t(s->bxq, s->bxd, ldx, NULL, s->bx, D->attn_norm, c->dim, c->norm_eps, T);
        if (s->kv_type == ML_F32) {
            float *kc = (float *)s->kcache + (size_t)l * lkv, *vc = (float *)s->vcache + (size_t)l * lkv;
            krh_matmul_qkv(s->bq, kc, vc, &D->wq, &D->wk, &D->wv, D->bq, D->bk, D->bv, s->bxq, s->bxd, ldx, T, cs,
                           sn, c->head_dim, p0);
            krh_attention_batch(s->bao, s->batt, s->bq, kc, vc, c->n_heads, c->n_kv_heads, c->head_dim, c->max_seq,
                                L->window, c->attn_scale, s->pos, T, p0 + T - 1);
        } else {
            const ml_kv_layer kv = kv_layer(s, l);
            krh_matmul_qkv_stage(s->bq, s->bkst, s->bvst, &D->wq, &D->wk, &D->wv, D->bq, D->bk, D->bv, s->bxq, s->bxd,
                                 ldx, T, cs, sn, c->head_dim, p0);
            store_kv(s, l, s->bkst, s->bvst, T);
            krh_attention_kv(s->bao, s->batt, s->bq, &kv, c->n_heads, c->n_kv_heads, c->head_dim, c->max_seq,
                             c->attn_scale, s->pos, T, p0 + T - 1);
        }
        krh_quantize_q8_t(s->bxq, s->bxd, ldx, s->bao, c->q_dim, T);
        krh_matmul(s->bx, c->dim, &D->wo, s->bxq, s->bxd, ldx, T, 1);
        krh_rmsnorm_q8_t(s->bxq, s->bxd, ldx, NULL, s->bx, D->ffn_norm, c->dim, c->norm_eps, T);
        if (swiglu_fused(s, D, T)) {   /* h's Q8_0 in bh1's space (4x what it needs) */
            int8_t *hq = (int8_t *)s->bh1;
            float *hd = (float *)((uint8_t *)s->bh1 + RUP((size_t)ldx * c->hidden_dim));
            krh_matmul_swiglu(hq, hd, &D->w1, &D->w3, s->bxq, s->bxd, ldx, T);
            krh_matmul(s->bx, c->dim, &D->w2, hq, hd, ldx, T, 1);
        } else {
            krh_matmul(s->bh1, c->hidden_dim, &D->w1, s->bxq, s->bxd, ldx, T, 0);
            krh_matmul(s->bh3, c->hidden_dim, &D->w3, s->bxq, s->bxd, ldx, T, 0);
            krh_silu_quant(s->bxq, s->bxd, ldx, s->bh1, s->bh3, c->hidden_dim, T);
            krh_matmul(s->bx, c->dim, &D->w2, s->bxq, s->bxd, ldx, T, 1);
        }
    }
    if (logits) {
        krh_rmsnorm_q8_t(s->bxq, s->bxd, ldx, NULL, s->bx, m->d_final_norm, c->dim, c->norm_eps, T);
        krh_matmul(s->blog, c->vocab, &m->d_wcls, s->bxq, s->bxd, ldx, T, 0);
        if (c->final_softcap > 0.0f)   /* model/transformer.c:304 */
            krh_softcap_rows(s->blog, (size_t)c->vocab, T, c->vocab, c->final_softcap);
        st = krh_copy_d2h(logits, s->blog, sizeof(float) * (size_t)T * c->vocab);
        if (st != ML_OK) return kr_seterr(st, "%s", krh_last_error());
    }
    return krh_status() == ML_OK ? ML_OK : kr_seterr(krh_status(), "%s", krh_last_error());
}

/* ml_prefill (model/transformer.c:427-438): n tokens at positions pos0.. in
 * batched steps of s->batch tokens; with batch 1, each token replays the
 * captured decode step instead. Every per-token op is ml_forward's, so the
 * results are the same either way (model/transformer.c:381-384). */
ml_status kr_prefill(kr_state *s, const int *tokens, int n, int pos0, float *logits) {
    const ml_config *c = &s->m->cfg;
    if (n < 0 || pos0 < 0 || pos0 + n > c->max_seq) return ML_E_SHAPE;
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= c->vocab) return ML_E_SHAPE;
    if (s->batch > 1 && n > 1) {
        ml_status st = batch_buffers(s, logits != NULL);
        for (int i = 0; st == ML_OK && i < n; i += s->batch) {
            const int T = n - i < s->batch ? n - i : s->batch;
            st = prefill_step(s, tokens + i, T, pos0 + i, logits ? logits + (size_t)i * c->vocab : NULL);
        }
        return st == ML_OK ? dev_status() : st;
    }
    if (logits) {
        for (int i = 0; i < n; i++) {
            const ml_status st = kr_forward(s, tokens[i], pos0 + i, logits + (size_t)i * c->vocab);
            if (st != ML_OK) return st;
        }
        return ML_OK;
    }
    if (n == 0) return ML_OK;
    ml_status st = krh_copy_h2d(s->prompt + pos0, tokens, sizeof(int) * (size_t)n);
    if (st == ML_OK) st = set_ints(s, 0, pos0);
    for (int i = 0; st == ML_OK && i < n; i++) st = run_step(s, STEP_PREFILL);
    return st == ML_OK ? dev_status() : st;
}

int kr_generate(kr_state *s, const int *prompt, int np, int steps, int *out, double *prefill_s, double *decode_s) {
    const ml_config *c = &s->m->cfg;
    if (np < 1 || np > c->max_seq || steps < 1) return -1;
    if (steps > c->max_seq) steps = c->max_seq;
    int n = 0, pos = 0, token = prompt[0];
    const int npre = np - 1 < steps - 1 ? np - 1 : steps - 1;
    double t0 = kr_now();
    if (s->smp) {   /* app/ml_run.c:369: the prompt's ids first */
        if (krh_copy_h2d(s->prompt, prompt, sizeof(int) * (size_t)np) != ML_OK) return -1;
        krh_sampler_accept(s->smp, s->prompt, np);
    }
    if (npre > 0) {
        if (kr_prefill(s, prompt, npre, 0, NULL) != ML_OK) return -1;
        for (pos = 0; pos < npre; pos++) out[n++] = prompt[pos + 1];
        token = prompt[npre];
    }
    const double t1 = kr_now();
    if (prefill_s) *prefill_s = t1 - t0;
    /* positions where ml_run takes the next id from the prompt (only when
     * the prompt is longer than steps) run one at a time */
    while (pos < steps && pos + 1 < np) {
        if (kr_forward(s, token, pos, NULL) != ML_OK) return -1;
        token = prompt[pos + 1];
        out[n++] = token;
        pos++;
    }
    if (pos < steps) {
        const int first = pos;
        if (set_ints(s, token, pos) != ML_OK) return -1;
        const int kind = s->smp ? STEP_SAMPLE : STEP_GREEDY;
        for (; pos < steps; pos++)
            if (run_step(s, kind) != ML_OK) return -1;
        if (dev_status() != ML_OK) return -1;
        if (krh_copy_d2h(out + n, s->log + first + 1, sizeof(int) * (size_t)(steps - first)) != ML_OK) return -1;
        n += steps - first;
    }
    if (decode_s) *decode_s = kr_now() - t1;
    return n;
}
