/* .mlb model loader, written from the format specification
 * (docs/file-format.md:16-119, validation table :214-222).
 *
 * The file is mapped read-only and the model's tensors are views into it.
 * Loading runs in three stages:
 *   1. the 256-byte header through a table of per-field rules (offset, type,
 *      accepted range, status when outside it) and the rules that relate
 *      fields to each other (derived dimensions, the q8 mask, RoPE scaling),
 *      in four phases that give a header with several faults the reference
 *      loader's status;
 *   2. the per-layer flag bytes, when the header announces them;
 *   3. a plan of the body: every array the configuration implies, in file
 *      order, each with its byte size and the pointer it fills; one pass lays
 *      the plan out at 64-byte boundaries against the file's size and checks
 *      the Q8 quants for the forbidden -128.
 * The status codes are the reference loader's: ML_E_IO when the file cannot
 * be read, ML_E_FORMAT for encodings and truncation, ML_E_SHAPE for
 * impossible dimensions. f16 scales stay f16 here: the device widens them
 * exactly where it reads them. Sizes are size_t products of dimensions
 * bounded by 2^24 x 2^16, which cannot overflow on a 64-bit host. */
#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include "kr_host.h"

#define HEADER_BYTES 256
#define LIM_DIM 65536.0        /* dim, n_layers, heads, hidden_dim, head_dim */
#define LIM_TOKENS 16777216.0  /* vocab, max_seq, sliding_window */

/* ---- stage 1: the header ---- */

enum { FIELD_U32 = 0, FIELD_F32 = 1 };

/* one header field's acceptance rule: lo < v (open) or lo <= v, and v < hi
 * (open) or v <= hi; a NaN passes no rule. phase: when it is checked. A
 * header with several faults gets the status of the first fault in the
 * reference's order, which interleaves field ranges with the rules between
 * fields in four phases, each of one status:
 *   1 the dimensions' ranges (ML_E_SHAPE),
 *   2 the weight encoding: wtype, the q8 mask, qkv_bias (ML_E_FORMAT),
 *   3 the derived dimensions: divisibility, head_dim, q_dim (ML_E_SHAPE),
 *   4 everything else (ML_E_FORMAT). */
typedef struct {
    uint8_t off, kind, status, lo_open, hi_open, phase;
    double lo, hi;
    const char *name;
} field_rule;

#define U32(ph, off, lo, hi, st, name) { off, FIELD_U32, st, 0, 0, ph, lo, hi, name }
#define F32(ph, off, lo_open, lo, hi, hi_open, name) { off, FIELD_F32, ML_E_FORMAT, lo_open, hi_open, ph, lo, hi, name }

static const field_rule FIELD_RULES[] = {
    U32(1, 8, 1, LIM_DIM, ML_E_SHAPE, "dim"),
    U32(1, 12, 1, LIM_DIM, ML_E_SHAPE, "n_layers"),
    U32(1, 16, 1, LIM_DIM, ML_E_SHAPE, "n_heads"),
    U32(1, 20, 1, LIM_DIM, ML_E_SHAPE, "n_kv_heads"),
    U32(1, 24, 1, LIM_DIM, ML_E_SHAPE, "hidden_dim"),
    U32(1, 28, 3, LIM_TOKENS, ML_E_SHAPE, "vocab"),   /* ids 1 and 2 are BOS and EOS */
    U32(1, 32, 1, LIM_TOKENS, ML_E_SHAPE, "max_seq"),
    U32(2, 44, ML_Q8_0, ML_Q4_0, ML_E_FORMAT, "wtype"),
    U32(2, 76, 0, 1, ML_E_FORMAT, "qkv_bias"),
    U32(3, 80, 0, LIM_DIM, ML_E_SHAPE, "head_dim"),
    F32(4, 36, 1, 0.0, INFINITY, 0, "rope_theta"),
    F32(4, 40, 0, 0.0, INFINITY, 0, "norm_eps"),
    U32(4, 52, ML_ROPE_NONE, ML_ROPE_YARN, ML_E_FORMAT, "rope_type"),
    U32(4, 84, 0, 1, ML_E_FORMAT, "qk_norm"),
    U32(4, 92, 0, LIM_TOKENS, ML_E_FORMAT, "sliding_window"),
    U32(4, 96, 0, 1, ML_E_FORMAT, "layer_flags"),
    F32(4, 100, 0, 0.0, 1e30, 1, "rope_local_theta"),
    U32(4, 104, ML_ACT_SILU, ML_ACT_GELU_TANH, ML_E_FORMAT, "act"),
    U32(4, 108, 0, 1, ML_E_FORMAT, "post_norms"),
    F32(4, 112, 0, 0.0, 1e6, 1, "embed_scale"),
    F32(4, 116, 0, 0.0, 1e6, 1, "attn_scale"),
    U32(4, 120, 0, 1, ML_E_FORMAT, "scale_f16"),
    F32(4, 124, 0, 0.0, 1e6, 1, "attn_softcap"),
    F32(4, 128, 0, 0.0, 1e6, 1, "final_softcap"),
};
#undef U32
#undef F32

static uint32_t le32(const uint8_t *h, int off) {
    uint32_t v;
    memcpy(&v, h + off, 4);
    return v;
}

static float lef(const uint8_t *h, int off) {
    float v;
    memcpy(&v, h + off, 4);
    return v;
}

static double field_value(const uint8_t *h, const field_rule *r) {
    return r->kind == FIELD_U32 ? (double)le32(h, r->off) : (double)lef(h, r->off);
}

static int field_ok(double v, const field_rule *r) {
    const int lo = r->lo_open ? v > r->lo : v >= r->lo;
    const int hi = r->hi_open ? v < r->hi : v <= r->hi;
    return lo && hi;
}

/* the RoPE scaling parameters of each rope_type (the specification's header
 * notes at offsets 52-68 and 88) */
static int rope_params_ok(const ml_config *c) {
    const float f = c->rope_factor, lo = c->rope_low_freq_factor, hi = c->rope_high_freq_factor;
    const int factor_ok = f > 0.0f && f < 1e6f;
    switch (c->rope_type) {
    case ML_ROPE_NONE:
        return 1;
    case ML_ROPE_LINEAR:
        return factor_ok;
    case ML_ROPE_LLAMA3:
        return factor_ok && lo > 0.0f && hi > lo && hi < 1e6f && c->rope_orig_max_seq > 0;
    default:   /* yarn: lo is beta_fast, hi beta_slow, with beta_fast > beta_slow > 0 */
        return factor_ok && hi > 0.0f && lo > hi && lo < 1e6f && c->rope_orig_max_seq > 0 &&
               c->rope_attn_factor > 0.0f && c->rope_attn_factor < 1e3f;
    }
}

/* the header's field ranges of one phase */
static ml_status check_fields(const uint8_t *h, int phase) {
    for (size_t i = 0; i < sizeof FIELD_RULES / sizeof FIELD_RULES[0]; i++) {
        const field_rule *r = &FIELD_RULES[i];
        if (r->phase != phase) continue;
        const double v = field_value(h, r);
        if (!field_ok(v, r)) return kr_seterr((ml_status)r->status, "header field %s = %g out of range", r->name, v);
    }
    return ML_OK;
}

ml_status kr_parse_header(ml_config *cfg, int *shared, const uint8_t *h) {
    memset(cfg, 0, sizeof *cfg);
    if (memcmp(h, "MLB1", 4) != 0) return kr_seterr(ML_E_FORMAT, "magic is not MLB1");
    if (le32(h, 4) != 1) return kr_seterr(ML_E_FORMAT, "version %u (1 expected)", le32(h, 4));
    ml_config *c = cfg;
    c->dim = (int)le32(h, 8);
    c->n_layers = (int)le32(h, 12);
    c->n_heads = (int)le32(h, 16);
    c->n_kv_heads = (int)le32(h, 20);
    c->hidden_dim = (int)le32(h, 24);
    c->vocab = (int)le32(h, 28);
    c->max_seq = (int)le32(h, 32);
    c->rope_theta = lef(h, 36);
    c->norm_eps = lef(h, 40);
    c->wtype = (int)le32(h, 44);
    *shared = le32(h, 48) != 0;
    c->rope_type = (int)le32(h, 52);
    c->rope_factor = lef(h, 56);
    c->rope_low_freq_factor = lef(h, 60);
    c->rope_high_freq_factor = lef(h, 64);
    c->rope_orig_max_seq = (int)le32(h, 68);
    c->q8_mask = le32(h, 72);
    c->qkv_bias = (int)le32(h, 76);
    const int head_dim = (int)le32(h, 80);
    c->qk_norm = (int)le32(h, 84);
    c->rope_attn_factor = lef(h, 88);
    c->sliding_window = (int)le32(h, 92);
    c->layer_flags = (int)le32(h, 96);
    c->rope_local_theta = lef(h, 100);
    c->act = (int)le32(h, 104);
    c->post_norms = (int)le32(h, 108);
    c->embed_scale = lef(h, 112);
    c->attn_scale = lef(h, 116);
    c->scale_f16 = (int)le32(h, 120);
    c->attn_softcap = lef(h, 124);
    c->final_softcap = lef(h, 128);
    ml_status st;

    /* 1: the dimensions */
    if ((st = check_fields(h, 1)) != ML_OK) return st;
    /* 2: the weight encoding */
    if ((st = check_fields(h, 2)) != ML_OK) return st;
    if ((c->q8_mask & ~(unsigned)ML_Q8M_ALL) || (c->wtype == ML_Q8_0 && c->q8_mask))
        return kr_seterr(ML_E_FORMAT, "q8_mask 0x%x with wtype %d", c->q8_mask, c->wtype);
    /* 3: the derived dimensions */
    if (c->dim % QK || c->hidden_dim % QK) return kr_seterr(ML_E_SHAPE, "dim and hidden_dim must be multiples of 32");
    if (c->n_heads % c->n_kv_heads) return kr_seterr(ML_E_SHAPE, "n_kv_heads must divide n_heads");
    if ((st = check_fields(h, 3)) != ML_OK) return st;
    if (!head_dim && c->dim % c->n_heads) return kr_seterr(ML_E_SHAPE, "n_heads must divide dim");
    c->head_dim = head_dim ? head_dim : c->dim / c->n_heads;
    if ((double)c->head_dim * c->n_heads > LIM_DIM) return kr_seterr(ML_E_SHAPE, "q_dim above 65536");
    c->q_dim = c->head_dim * c->n_heads;
    c->kv_dim = c->head_dim * c->n_kv_heads;
    if (c->head_dim % 2 || c->q_dim % QK) return kr_seterr(ML_E_SHAPE, "odd head_dim or q_dim not a multiple of 32");
    /* 4: the rest */
    if ((st = check_fields(h, 4)) != ML_OK) return st;
    if (c->rope_type != ML_ROPE_YARN && c->rope_attn_factor != 0.0f)
        return kr_seterr(ML_E_FORMAT, "rope_attn_factor without yarn scaling");
    if (!rope_params_ok(c)) return kr_seterr(ML_E_FORMAT, "RoPE scaling parameters of rope_type %d", c->rope_type);

    /* zeros that stand for defaults */
    if (c->embed_scale == 0.0f) c->embed_scale = 1.0f;
    if (c->attn_scale == 0.0f) c->attn_scale = 1.0f / sqrtf((float)c->head_dim);
    return ML_OK;
}

/* ---- stage 3: the body plan ---- */

typedef struct {
    size_t bytes;
    const void **dst;   /* receives the array's address */
    int q8;             /* Q8 quants: no byte may be -128 */
} plan_item;

typedef struct {
    plan_item *items;
    int n, cap;
} body_plan;

static void plan_array(body_plan *p, const void *dst_field, size_t bytes, int q8) {
    if (p->n < p->cap) p->items[p->n++] = (plan_item){ bytes, (const void **)dst_field, q8 };
}

/* storage type of a matrix class: Q8 when the model is, or when one of its
 * q8_mask bits is set */
static int class_type(const ml_config *c, unsigned bits) {
    return c->wtype == ML_Q8_0 || (c->q8_mask & bits) ? ML_Q8_0 : ML_Q4_0;
}

/* a quantized matrix: its quants, then its scales (f32 or f16) */
static void plan_matrix(body_plan *p, ml_qtensor *t, const ml_config *c, int rows, int cols, unsigned bits) {
    const int type = class_type(c, bits);
    const size_t n = (size_t)rows * (size_t)cols, nblocks = n / QK;
    memset(t, 0, sizeof *t);
    t->rows = rows;
    t->cols = cols;
    t->type = (uint8_t)type;
    plan_array(p, &t->q, type == ML_Q4_0 ? n / 2 : n, type == ML_Q8_0);
    if (c->scale_f16) plan_array(p, &t->dh, nblocks * 2, 0);
    else plan_array(p, &t->d, nblocks * 4, 0);
}

static void plan_floats(body_plan *p, const float **dst, int n) { plan_array(p, dst, (size_t)n * sizeof(float), 0); }

/* every array after the layer flags, in the order the specification lists
 * them (docs/file-format.md:81-101) */
static void plan_body(body_plan *p, kr_model *m) {
    const ml_config *c = &m->cfg;
    plan_matrix(p, &m->tok_emb, c, c->vocab, c->dim, ML_Q8M_EMB | (m->shared ? ML_Q8M_CLS : 0));
    for (int l = 0; l < c->n_layers; l++) {
        ml_layer *L = &m->layers[l];
        plan_floats(p, &L->attn_norm, c->dim);
        plan_matrix(p, &L->wq, c, c->q_dim, c->dim, ML_Q8M_QK);
        plan_matrix(p, &L->wk, c, c->kv_dim, c->dim, ML_Q8M_QK);
        plan_matrix(p, &L->wv, c, c->kv_dim, c->dim, ML_Q8M_V);
        plan_matrix(p, &L->wo, c, c->dim, c->q_dim, ML_Q8M_O);
        if (c->qkv_bias) {
            plan_floats(p, &L->bq, c->q_dim);
            plan_floats(p, &L->bk, c->kv_dim);
            plan_floats(p, &L->bv, c->kv_dim);
        }
        if (c->qk_norm) {
            plan_floats(p, &L->q_norm, c->head_dim);
            plan_floats(p, &L->k_norm, c->head_dim);
        }
        plan_floats(p, &L->ffn_norm, c->dim);
        plan_matrix(p, &L->w1, c, c->hidden_dim, c->dim, ML_Q8M_UP);
        plan_matrix(p, &L->w2, c, c->dim, c->hidden_dim, ML_Q8M_DOWN);
        plan_matrix(p, &L->w3, c, c->hidden_dim, c->dim, ML_Q8M_UP);
        if (c->post_norms) {
            plan_floats(p, &L->post_attn_norm, c->dim);
            plan_floats(p, &L->post_ffn_norm, c->dim);
        }
    }
    plan_floats(p, &m->final_norm, c->dim);
    if (!m->shared) plan_matrix(p, &m->wcls, c, c->vocab, c->dim, ML_Q8M_CLS);
}

static size_t align_up(size_t off) { return (off + ML_ALIGN - 1) & ~(size_t)(ML_ALIGN - 1); }

/* lays the plan out from byte `off` of the map: each array must lie within
 * the file (the padding after the last one may be missing) */
static ml_status lay_out(const body_plan *p, const uint8_t *map, size_t size, size_t off) {
    for (int i = 0; i < p->n; i++) {
        const plan_item *it = &p->items[i];
        if (off > size || it->bytes > size - off)
            return kr_seterr(ML_E_FORMAT, "file ends inside array %d of the body (%zu bytes at offset %zu)", i,
                             it->bytes, off);
        *it->dst = map + off;
        if (it->q8 && memchr(map + off, 0x80, it->bytes))
            return kr_seterr(ML_E_FORMAT, "a Q8 quant equal to -128 in array %d", i);
        off = align_up(off + it->bytes);
    }
    return ML_OK;
}

/* ---- loading ---- */

static ml_status map_file(const char *path, void **map, size_t *size) {
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return kr_seterr(ML_E_IO, "cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        close(fd);
        return kr_seterr(ML_E_IO, "%s is not a readable file", path);
    }
    if (st.st_size < HEADER_BYTES) {
        close(fd);
        return kr_seterr(ML_E_FORMAT, "%s: %lld bytes, shorter than the header", path, (long long)st.st_size);
    }
    void *p = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (p == MAP_FAILED) return kr_seterr(ML_E_IO, "cannot map %s", path);
    *map = p;
    *size = (size_t)st.st_size;
    return ML_OK;
}

static ml_status load(kr_model *m) {
    ml_status s = kr_parse_header(&m->cfg, &m->shared, m->map);
    if (s != ML_OK) return s;
    const ml_config *c = &m->cfg;
    const uint8_t *map = m->map;
    m->layers = calloc((size_t)c->n_layers, sizeof(ml_layer));
    if (!m->layers) return kr_seterr(ML_E_NOMEM, "layer table");

    /* stage 2: one flag byte per layer; without them a window applies to
     * every layer */
    size_t off = HEADER_BYTES;
    const uint8_t *flags = NULL;
    if (c->layer_flags) {
        if ((size_t)c->n_layers > m->size - off) return kr_seterr(ML_E_FORMAT, "file ends inside the layer flags");
        flags = map + off;
        off = align_up(off + (size_t)c->n_layers);
        for (int l = 0; l < c->n_layers; l++) {
            if (flags[l] & ~ML_LAYER_ALL) return kr_seterr(ML_E_FORMAT, "layer %d: unknown flag bits 0x%x", l, flags[l]);
            if ((flags[l] & ML_LAYER_LOCAL_ROPE) && !(c->rope_local_theta > 0.0f))
                return kr_seterr(ML_E_FORMAT, "layer %d: local RoPE without rope_local_theta", l);
        }
    }
    for (int l = 0; l < c->n_layers; l++) {
        m->layers[l].window = !flags || (flags[l] & ML_LAYER_SLIDING) ? c->sliding_window : 0;
        m->layers[l].local_rope = flags && (flags[l] & ML_LAYER_LOCAL_ROPE);
    }

    /* stage 3 */
    body_plan plan = { NULL, 0, 5 + 23 * c->n_layers };   /* tok_emb, final_norm, wcls; 23 arrays a layer at most */
    plan.items = malloc(sizeof(plan_item) * (size_t)plan.cap);
    if (!plan.items) return kr_seterr(ML_E_NOMEM, "body plan");
    plan_body(&plan, m);
    s = lay_out(&plan, map, m->size, off);
    free(plan.items);
    if (s != ML_OK) return s;
    if (m->shared) m->wcls = m->tok_emb;
    return ML_OK;
}

ml_status kr_model_load(kr_model **out, const char *path) {
    *out = NULL;
    kr_model *m = calloc(1, sizeof *m);
    if (!m) return kr_seterr(ML_E_NOMEM, "model");
    ml_status s = map_file(path, &m->map, &m->size);
    if (s == ML_OK) s = load(m);
    if (s != ML_OK) {
        kr_model_free(m);
        return s;
    }
    *out = m;
    return ML_OK;
}

const ml_config *kr_model_config(const kr_model *m) { return &m->cfg; }
const ml_layer *kr_model_layer(const kr_model *m, int l) {
    return l >= 0 && l < m->cfg.n_layers ? &m->layers[l] : NULL;
}
const ml_qtensor *kr_model_tok_emb(const kr_model *m) { return &m->tok_emb; }
const ml_qtensor *kr_model_wcls(const kr_model *m) { return &m->wcls; }
