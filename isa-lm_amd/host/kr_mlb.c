/* .mlb loader: maps the file and points ml_qtensor views into it, with the
 * reference loader's validation rules and status codes (model/mlb.c:80-218,
 * docs/file-format.md:16-119, :214-222). Scales stay in the file's width
 * (f32 or f16): the device widens f16 exactly where it reads them. */
#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include "kr_host.h"

#define MAX_DIM (1 << 16)
#define MAX_TOKENS (1 << 24)

typedef struct { const uint8_t *base; size_t off, size; int ok; } cursor;

static const void *take(cursor *c, size_t n) {
    if (!c->ok || n > c->size - c->off) { c->ok = 0; return NULL; }
    const void *p = c->base + c->off;
    c->off += n;
    c->off = (c->off + ML_ALIGN - 1) & ~(size_t)(ML_ALIGN - 1);
    if (c->off > c->size) c->off = c->size;
    return p;
}

/* model/mlb.c:24-38: quants, then scales; a Q8 quant of -128 is rejected */
static ml_qtensor take_mat(cursor *c, int rows, int cols, int type, int f16) {
    ml_qtensor t = { NULL, NULL, rows, cols, (uint8_t)type, NULL, NULL, NULL, 0 };
    const size_t n = (size_t)rows * cols, nd = n / QK * (f16 ? 2 : 4);
    t.q = take(c, type == ML_Q4_0 ? n / 2 : n);
    if (f16) t.dh = take(c, nd);
    else t.d = take(c, nd);
    if (c->ok && type == ML_Q8_0 && memchr(t.q, 0x80, n)) c->ok = 0;
    return t;
}

static uint32_t rd32(const uint8_t *p) { uint32_t v; memcpy(&v, p, 4); return v; }
static float rdf(const uint8_t *p) { float v; memcpy(&v, p, 4); return v; }

/* model/mlb.c:80-159 */
ml_status kr_parse_header(ml_config *cfg, int *shared, const uint8_t *h) {
    memset(cfg, 0, sizeof *cfg);
    if (memcmp(h, "MLB1", 4) != 0 || rd32(h + 4) != 1) return ML_E_FORMAT;
    uint32_t v[7];
    for (int i = 0; i < 7; i++) v[i] = rd32(h + 8 + 4 * i);
    for (int i = 0; i < 7; i++)
        if (v[i] == 0 || v[i] > (i == 5 || i == 6 ? MAX_TOKENS : MAX_DIM)) return ML_E_SHAPE;
    if (v[5] < 3) return ML_E_SHAPE;
    cfg->dim = (int)v[0]; cfg->n_layers = (int)v[1]; cfg->n_heads = (int)v[2];
    cfg->n_kv_heads = (int)v[3]; cfg->hidden_dim = (int)v[4]; cfg->vocab = (int)v[5];
    cfg->max_seq = (int)v[6];
    cfg->rope_theta = rdf(h + 36);
    cfg->norm_eps = rdf(h + 40);
    cfg->wtype = (int)rd32(h + 44);
    *shared = rd32(h + 48) != 0;
    if (cfg->wtype != ML_Q8_0 && cfg->wtype != ML_Q4_0) return ML_E_FORMAT;
    cfg->q8_mask = rd32(h + 72);
    if ((cfg->q8_mask & ~(unsigned)ML_Q8M_ALL) || (cfg->wtype == ML_Q8_0 && cfg->q8_mask)) return ML_E_FORMAT;
    const uint32_t bias = rd32(h + 76);
    if (bias > 1) return ML_E_FORMAT;
    cfg->qkv_bias = (int)bias;
    if (cfg->dim % QK || cfg->hidden_dim % QK) return ML_E_SHAPE;
    if (cfg->n_heads % cfg->n_kv_heads) return ML_E_SHAPE;
    const uint32_t hd = rd32(h + 80);
    if (hd > MAX_DIM || (!hd && cfg->dim % cfg->n_heads)) return ML_E_SHAPE;
    cfg->head_dim = hd ? (int)hd : cfg->dim / cfg->n_heads;
    if ((uint64_t)cfg->head_dim * (uint64_t)cfg->n_heads > MAX_DIM) return ML_E_SHAPE;
    cfg->q_dim = cfg->head_dim * cfg->n_heads;
    cfg->kv_dim = cfg->head_dim * cfg->n_kv_heads;
    if (cfg->head_dim % 2 || cfg->q_dim % QK) return ML_E_SHAPE;
    const uint32_t qkn = rd32(h + 84), win = rd32(h + 92);
    if (qkn > 1 || win > MAX_TOKENS) return ML_E_FORMAT;
    cfg->qk_norm = (int)qkn;
    cfg->sliding_window = (int)win;
    const uint32_t lflags = rd32(h + 96);
    if (lflags > 1) return ML_E_FORMAT;
    cfg->layer_flags = (int)lflags;
    cfg->rope_local_theta = rdf(h + 100);
    if (!(cfg->rope_local_theta >= 0.0f && cfg->rope_local_theta < 1e30f)) return ML_E_FORMAT;
    const uint32_t act = rd32(h + 104), pn = rd32(h + 108);
    if (act > ML_ACT_GELU_TANH || pn > 1) return ML_E_FORMAT;
    cfg->act = (int)act;
    cfg->post_norms = (int)pn;
    cfg->embed_scale = rdf(h + 112);
    cfg->attn_scale = rdf(h + 116);
    if (!(cfg->embed_scale >= 0.0f && cfg->embed_scale < 1e6f) || !(cfg->attn_scale >= 0.0f && cfg->attn_scale < 1e6f))
        return ML_E_FORMAT;
    if (cfg->embed_scale == 0.0f) cfg->embed_scale = 1.0f;
    if (cfg->attn_scale == 0.0f) cfg->attn_scale = 1.0f / sqrtf((float)cfg->head_dim);
    const uint32_t f16 = rd32(h + 120);
    if (f16 > 1) return ML_E_FORMAT;
    cfg->scale_f16 = (int)f16;
    cfg->attn_softcap = rdf(h + 124);
    cfg->final_softcap = rdf(h + 128);
    if (!(cfg->attn_softcap >= 0.0f && cfg->attn_softcap < 1e6f) || !(cfg->final_softcap >= 0.0f && cfg->final_softcap < 1e6f))
        return ML_E_FORMAT;
    if (!(cfg->rope_theta > 0.0f) || !(cfg->norm_eps >= 0.0f)) return ML_E_FORMAT;
    cfg->rope_type = (int)rd32(h + 52);
    cfg->rope_factor = rdf(h + 56);
    cfg->rope_low_freq_factor = rdf(h + 60);
    cfg->rope_high_freq_factor = rdf(h + 64);
    cfg->rope_orig_max_seq = (int)rd32(h + 68);
    cfg->rope_attn_factor = rdf(h + 88);
    if (cfg->rope_type != ML_ROPE_YARN && cfg->rope_attn_factor != 0.0f) return ML_E_FORMAT;
    if (cfg->rope_type == ML_ROPE_LLAMA3) {
        if (!(cfg->rope_factor > 0.0f && cfg->rope_factor < 1e6f) || !(cfg->rope_low_freq_factor > 0.0f) ||
            !(cfg->rope_high_freq_factor > cfg->rope_low_freq_factor && cfg->rope_high_freq_factor < 1e6f) ||
            cfg->rope_orig_max_seq <= 0)
            return ML_E_FORMAT;
    } else if (cfg->rope_type == ML_ROPE_LINEAR) {
        if (!(cfg->rope_factor > 0.0f && cfg->rope_factor < 1e6f)) return ML_E_FORMAT;
    } else if (cfg->rope_type == ML_ROPE_YARN) {
        if (!(cfg->rope_factor > 0.0f && cfg->rope_factor < 1e6f) || !(cfg->rope_high_freq_factor > 0.0f) ||
            !(cfg->rope_low_freq_factor > cfg->rope_high_freq_factor && cfg->rope_low_freq_factor < 1e6f) ||
            cfg->rope_orig_max_seq <= 0 || !(cfg->rope_attn_factor > 0.0f && cfg->rope_attn_factor < 1e3f))
            return ML_E_FORMAT;
    } else if (cfg->rope_type != ML_ROPE_NONE) {
        return ML_E_FORMAT;
    }
    return ML_OK;
}

ml_status kr_model_load(kr_model **out, const char *path) {
    *out = NULL;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return kr_seterr(ML_E_IO, "cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); return kr_seterr(ML_E_IO, "cannot stat %s", path); }
    if (st.st_size < 256) { close(fd); return kr_seterr(ML_E_FORMAT, "%s: shorter than the header", path); }
    void *map = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return kr_seterr(ML_E_IO, "cannot map %s", path);
    kr_model *m = calloc(1, sizeof *m);
    if (!m) { munmap(map, (size_t)st.st_size); return ML_E_NOMEM; }
    m->map = map;
    m->size = (size_t)st.st_size;
    int shared = 0;
    ml_status s = kr_parse_header(&m->cfg, &shared, map);
    if (s != ML_OK) { kr_model_free(m); return kr_seterr(s, "%s: bad header", path); }
    const ml_config *c = &m->cfg;
#define WT(bits) (c->wtype == ML_Q8_0 || (c->q8_mask & (bits)) ? ML_Q8_0 : ML_Q4_0)
    m->layers = calloc((size_t)c->n_layers, sizeof(ml_layer));
    if (!m->layers) { kr_model_free(m); return ML_E_NOMEM; }
    cursor cur = { map, 256, m->size, 1 };
    const size_t normsz = (size_t)c->dim * sizeof(float);
    const uint8_t *lf = c->layer_flags ? take(&cur, (size_t)c->n_layers) : NULL;
    for (int l = 0; lf && cur.ok && l < c->n_layers; l++)
        if ((lf[l] & ~ML_LAYER_ALL) || ((lf[l] & ML_LAYER_LOCAL_ROPE) && !(c->rope_local_theta > 0.0f))) {
            kr_model_free(m);
            return kr_seterr(ML_E_FORMAT, "%s: bad layer flags", path);
        }
    m->tok_emb = take_mat(&cur, c->vocab, c->dim, WT(ML_Q8M_EMB | (shared ? ML_Q8M_CLS : 0)), c->scale_f16);
    for (int l = 0; l < c->n_layers; l++) {
        ml_layer *L = &m->layers[l];
        L->window = !lf || (lf[l] & ML_LAYER_SLIDING) ? c->sliding_window : 0;
        L->local_rope = lf && (lf[l] & ML_LAYER_LOCAL_ROPE);
        L->attn_norm = take(&cur, normsz);
        L->wq = take_mat(&cur, c->q_dim, c->dim, WT(ML_Q8M_QK), c->scale_f16);
        L->wk = take_mat(&cur, c->kv_dim, c->dim, WT(ML_Q8M_QK), c->scale_f16);
        L->wv = take_mat(&cur, c->kv_dim, c->dim, WT(ML_Q8M_V), c->scale_f16);
        L->wo = take_mat(&cur, c->dim, c->q_dim, WT(ML_Q8M_O), c->scale_f16);
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
        L->w1 = take_mat(&cur, c->hidden_dim, c->dim, WT(ML_Q8M_UP), c->scale_f16);
        L->w2 = take_mat(&cur, c->dim, c->hidden_dim, WT(ML_Q8M_DOWN), c->scale_f16);
        L->w3 = take_mat(&cur, c->hidden_dim, c->dim, WT(ML_Q8M_UP), c->scale_f16);
        if (c->post_norms) {
            L->post_attn_norm = take(&cur, normsz);
            L->post_ffn_norm = take(&cur, normsz);
        }
    }
    m->final_norm = take(&cur, normsz);
    m->shared = shared;
    m->wcls = shared ? m->tok_emb : take_mat(&cur, c->vocab, c->dim, WT(ML_Q8M_CLS), c->scale_f16);
#undef WT
    if (!cur.ok) { kr_model_free(m); return kr_seterr(ML_E_FORMAT, "%s: truncated or bad tensor data", path); }
    *out = m;
    return ML_OK;
}

const ml_config *kr_model_config(const kr_model *m) { return &m->cfg; }
const ml_layer *kr_model_layer(const kr_model *m, int l) {
    return l >= 0 && l < m->cfg.n_layers ? &m->layers[l] : NULL;
}
const ml_qtensor *kr_model_tok_emb(const kr_model *m) { return &m->tok_emb; }
const ml_qtensor *kr_model_wcls(const kr_model *m) { return &m->wcls; }
