/* ORACLE — test infrastructure only. Minimal .mlb reader for the oracle's
 * forward pass, restating the body walk of model/mlb.c:161-218 (header
 * fields model/mlb.c:80-159, layout docs/file-format.md:16-119). f16 scales
 * are widened to f32 exactly, as expand_scales does (model/mlb.c:44-75).
 * It checks only what the oracle needs; the product's loader validates. */
#include <fcntl.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include "kro.h"

struct kro_model {
    ml_config cfg;
    const uint8_t *map;
    size_t size;
    ml_qtensor tok_emb, wcls;
    const float *final_norm;
    ml_layer *layers;
    float **scales;   /* widened f16 scales, one array per matrix */
    int nscales;
};

void kro_mlb_close(kro_model *m);

typedef struct { const uint8_t *base; size_t off, size; int ok; } cursor;

static const void *take(cursor *c, size_t n) {
    if (!c->ok || n > c->size - c->off) { c->ok = 0; return NULL; }
    const void *p = c->base + c->off;
    c->off = (c->off + n + ML_ALIGN - 1) & ~(size_t)(ML_ALIGN - 1);
    if (c->off > c->size) c->off = c->size;
    return p;
}

static ml_qtensor take_mat(kro_model *m, cursor *c, int rows, int cols, int type) {
    ml_qtensor t = { NULL, NULL, rows, cols, (uint8_t)type, NULL, NULL, NULL, 0 };
    const size_t n = (size_t)rows * cols, nb = n / QK;
    t.q = take(c, type == ML_Q4_0 ? n / 2 : n);
    if (m->cfg.scale_f16) {
        const uint16_t *dh = take(c, nb * 2);
        if (!c->ok) return t;
        float *d = malloc(nb * sizeof(float));
        if (!d) { c->ok = 0; return t; }
        for (size_t i = 0; i < nb; i++) d[i] = kro_f16_to_f32(dh[i]);
        m->scales[m->nscales++] = d;
        t.dh = dh;
        t.d = d;
    } else {
        t.d = take(c, nb * sizeof(float));
    }
    return t;
}

static uint32_t u32(const uint8_t *p) { uint32_t v; memcpy(&v, p, 4); return v; }
static float f32(const uint8_t *p) { float v; memcpy(&v, p, 4); return v; }

int kro_mlb_open(kro_model **out, const char *path) {
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return ML_E_IO;
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 256) { close(fd); return ML_E_FORMAT; }
    const uint8_t *map = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return ML_E_IO;
    kro_model *m = calloc(1, sizeof *m);
    m->map = map;
    m->size = (size_t)st.st_size;
    ml_config *c = &m->cfg;
    const uint8_t *h = map;
    if (memcmp(h, "MLB1", 4) || u32(h + 4) != 1) { kro_mlb_close(m); return ML_E_FORMAT; }
    c->dim = (int)u32(h + 8); c->n_layers = (int)u32(h + 12); c->n_heads = (int)u32(h + 16);
    c->n_kv_heads = (int)u32(h + 20); c->hidden_dim = (int)u32(h + 24); c->vocab = (int)u32(h + 28);
    c->max_seq = (int)u32(h + 32);
    c->rope_theta = f32(h + 36); c->norm_eps = f32(h + 40);
    c->wtype = (int)u32(h + 44);
    const int shared = u32(h + 48) != 0;
    c->rope_type = (int)u32(h + 52); c->rope_factor = f32(h + 56);
    c->rope_low_freq_factor = f32(h + 60); c->rope_high_freq_factor = f32(h + 64);
    c->rope_orig_max_seq = (int)u32(h + 68);
    c->q8_mask = u32(h + 72); c->qkv_bias = (int)u32(h + 76);
    const uint32_t hd = u32(h + 80);
    c->head_dim = hd ? (int)hd : c->dim / c->n_heads;
    c->q_dim = c->head_dim * c->n_heads;
    c->kv_dim = c->head_dim * c->n_kv_heads;
    c->qk_norm = (int)u32(h + 84); c->rope_attn_factor = f32(h + 88);
    c->sliding_window = (int)u32(h + 92); c->layer_flags = (int)u32(h + 96);
    c->rope_local_theta = f32(h + 100); c->act = (int)u32(h + 104); c->post_norms = (int)u32(h + 108);
    c->embed_scale = f32(h + 112); c->attn_scale = f32(h + 116); c->scale_f16 = (int)u32(h + 120);
    c->attn_softcap = f32(h + 124); c->final_softcap = f32(h + 128);
    if (c->embed_scale == 0.0f) c->embed_scale = 1.0f;
    if (c->attn_scale == 0.0f) c->attn_scale = 1.0f / sqrtf((float)c->head_dim);
#define WT(bits) (c->wtype == ML_Q8_0 || (c->q8_mask & (bits)) ? ML_Q8_0 : ML_Q4_0)
    m->layers = calloc((size_t)c->n_layers, sizeof(ml_layer));
    m->scales = calloc((size_t)c->n_layers * 7 + 2, sizeof(float *));
    cursor cur = { map, 256, m->size, 1 };
    const size_t normsz = (size_t)c->dim * sizeof(float);
    const uint8_t *lf = c->layer_flags ? take(&cur, (size_t)c->n_layers) : NULL;
    m->tok_emb = take_mat(m, &cur, c->vocab, c->dim, WT(ML_Q8M_EMB | (shared ? ML_Q8M_CLS : 0)));
    for (int l = 0; l < c->n_layers; l++) {
        ml_layer *L = &m->layers[l];
        L->window = !lf || (lf[l] & ML_LAYER_SLIDING) ? c->sliding_window : 0;
        L->local_rope = lf && (lf[l] & ML_LAYER_LOCAL_ROPE);
        L->attn_norm = take(&cur, normsz);
        L->wq = take_mat(m, &cur, c->q_dim, c->dim, WT(ML_Q8M_QK));
        L->wk = take_mat(m, &cur, c->kv_dim, c->dim, WT(ML_Q8M_QK));
        L->wv = take_mat(m, &cur, c->kv_dim, c->dim, WT(ML_Q8M_V));
        L->wo = take_mat(m, &cur, c->dim, c->q_dim, WT(ML_Q8M_O));
        if (c->qkv_bias) {
            L->bq = take(&cur, (size_t)c->q_dim * sizeof(float));
            L->bk = take(&cur, (size_t)c->kv_dim * sizeof(float));
            L->bv = take(&cur, (size_t)c->kv_dim * sizeof(float));
        }
        if (c->qk_norm) {
            L->q_norm = take(&cur, (size_t)c->head_dim * sizeof(float));
            L->k_norm = take(&cur, (size_t)c->head_dim * sizeof(float));
        }
        L->ffn_norm = take(&cur, normsz);
        L->w1 = take_mat(m, &cur, c->hidden_dim, c->dim, WT(ML_Q8M_UP));
        L->w2 = take_mat(m, &cur, c->dim, c->hidden_dim, WT(ML_Q8M_DOWN));
        L->w3 = take_mat(m, &cur, c->hidden_dim, c->dim, WT(ML_Q8M_UP));
        if (c->post_norms) {
            L->post_attn_norm = take(&cur, normsz);
            L->post_ffn_norm = take(&cur, normsz);
        }
    }
    m->final_norm = take(&cur, normsz);
    m->wcls = shared ? m->tok_emb : take_mat(m, &cur, c->vocab, c->dim, WT(ML_Q8M_CLS));
#undef WT
    if (!cur.ok) { kro_mlb_close(m); return ML_E_FORMAT; }
    *out = m;
    return ML_OK;
}

void kro_mlb_close(kro_model *m) {
    if (!m) return;
    for (int i = 0; i < m->nscales; i++) free(m->scales[i]);
    free(m->scales);
    free(m->layers);
    if (m->map) munmap((void *)m->map, m->size);
    free(m);
}

const ml_config *kro_mlb_config(const kro_model *m) { return &m->cfg; }
const ml_qtensor *kro_mlb_tok_emb(const kro_model *m) { return &m->tok_emb; }
const ml_qtensor *kro_mlb_wcls(const kro_model *m) { return &m->wcls; }
const float *kro_mlb_final_norm(const kro_model *m) { return m->final_norm; }
const ml_layer *kro_mlb_layer(const kro_model *m, int l) { return &m->layers[l]; }
