/* Seeded synthetic .mlb models and microbench matrices.
 *
 * Random numbers: element i of stream s is splitmix64 of a Weyl sequence
 * keyed by (seed, s), so any element can be drawn independently and the
 * output does not depend on the thread count. Normals come in Box-Muller
 * pairs from the two 32-bit halves of one draw, with log, sqrt, sin and cos
 * evaluated from IEEE arithmetic alone (csrc/kr_normal.h), so that the device
 * generator writes the same bytes. Streams are numbered in file
 * order. Quantization follows docs/file-format.md:133-159: Q8 with the
 * activation rule (d rounded to f16 first when scales are f16, quants against
 * the rounded d); Q4 with the amax/7 rule of core/quant_ref.c:21-38. */
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "kr_host.h"

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return mix64(seed * 0x9E3779B97F4A7C15ULL + stream * 0xD1B54A32D192ED03ULL + 0x632BE59BD9B4E019ULL);
}

static uint64_t draw(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * 0x9E3779B97F4A7C15ULL); }

#define KR_NORMAL_FN static inline
#include "../csrc/kr_normal.h"

/* normals 2j and 2j+1 of the stream (the device generator draws the same
 * bits: csrc/kr_normal.h) */
static void normal_pair(uint64_t key, uint64_t j, float *a, float *b) { krn_pair(draw(key, j), a, b); }

static float normal_at(uint64_t key, uint64_t i) {
    float a, b;
    normal_pair(key, i >> 1, &a, &b);
    return i & 1 ? b : a;
}

/* f32 -> f16, round to nearest even (same results as core/ml.c:39-53) */
static uint16_t to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    x &= 0x7fffffff;
    if (x > 0x7f800000) return sign | 0x7e00;
    if (x >= 0x477ff000) return sign | 0x7c00;
    if (x < 0x38800000) {
        float a;
        memcpy(&a, &x, 4);
        return sign | (uint16_t)lrintf(a * 16777216.0f);
    }
    x += 0xfff + ((x >> 13) & 1);
    return sign | (uint16_t)((x >> 13) - (112u << 10));
}

static float from_f16(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    if (e == 0) return (sign ? -1.0f : 1.0f) * (float)m * (1.0f / 16777216.0f);
    const uint32_t x = sign | (e == 31 ? 0x7f800000u | (m << 13) : ((e + 112u) << 23) | (m << 13));
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* one 32-block of x into Q8 or Q4 quants and its scale (f32 or f16 bits) */
static void quant_block(const float *x, int type, int f16, uint8_t *q, void *d) {
    float amax = 0.0f;
    for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(x[j]));
    const float lim = type == ML_Q8_0 ? 127.0f : 7.0f, lo = type == ML_Q8_0 ? -127.0f : -8.0f;
    float dv = amax < ML_QUANT_TINY ? 0.0f : amax / lim;
    if (f16) {
        const uint16_t h = to_f16(dv);
        dv = from_f16(h);
        *(uint16_t *)d = h;
    } else {
        *(float *)d = dv;
    }
    const float id = dv != 0.0f ? (f16 ? 1.0f / dv : lim / amax) : 0.0f;
    int v[QK];
    for (int j = 0; j < QK; j++) {
        float t = truncf(x[j] * id + copysignf(0.5f, x[j]));
        t = fminf(fmaxf(t, lo), lim);
        v[j] = (int)t;
    }
    if (type == ML_Q8_0) {
        for (int j = 0; j < QK; j++) q[j] = (uint8_t)(int8_t)v[j];
    } else {
        for (int j = 0; j < QK / 2; j++) q[j] = (uint8_t)((v[j] + 8) | ((v[j + QK / 2] + 8) << 4));
    }
}

typedef struct {
    uint64_t key;
    int rows, cols, type, f16;
    float std;
    uint8_t *q;
    uint8_t *d;
    int r0, r1;
} mat_job;

static void *mat_rows(void *p) {
    mat_job *j = p;
    float x[QK];
    const int nb = j->cols / QK, qb = j->type == ML_Q8_0 ? QK : QK / 2, db = j->f16 ? 2 : 4;
    for (int r = j->r0; r < j->r1; r++)
        for (int b = 0; b < nb; b++) {
            const uint64_t base = (uint64_t)r * j->cols + (uint64_t)b * QK;
            for (int k = 0; k < QK; k += 2) normal_pair(j->key, (base + k) >> 1, &x[k], &x[k + 1]);
            for (int k = 0; k < QK; k++) x[k] *= j->std;
            const size_t blk = (size_t)r * nb + b;
            quant_block(x, j->type, j->f16, j->q + blk * qb, j->d + blk * db);
        }
    return NULL;
}

static void run_jobs(mat_job *proto, int threads, void *(*fn)(void *)) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t th[64];
    mat_job js[64];
    for (int i = 0; i < threads; i++) {
        js[i] = *proto;
        js[i].r0 = (int)((long long)proto->rows * i / threads);
        js[i].r1 = (int)((long long)proto->rows * (i + 1) / threads);
        pthread_create(&th[i], NULL, fn, &js[i]);
    }
    for (int i = 0; i < threads; i++) pthread_join(th[i], NULL);
}

typedef struct { FILE *f; size_t off; int ok; uint8_t *dev; } writer;

static void put(writer *w, const void *p, size_t n) {
    static const uint8_t zero[ML_ALIGN] = { 0 };
    if (w->ok && n && fwrite(p, 1, n, w->f) != n) w->ok = 0;
    w->off += n;
    const size_t pad = (ML_ALIGN - w->off % ML_ALIGN) % ML_ALIGN;
    if (w->ok && pad && fwrite(zero, 1, pad, w->f) != pad) w->ok = 0;
    w->off += pad;
}

/* threads < 0: draw on the device (krh_gen_blocks) into w->dev */
static void put_mat(writer *w, uint64_t key, int rows, int cols, int type, int f16, float std, int threads) {
    const size_t n = (size_t)rows * cols, nq = type == ML_Q8_0 ? n : n / 2, nd = n / QK * (f16 ? 2 : 4);
    uint8_t *q = malloc(nq), *d = malloc(nd);
    if (!q || !d) { w->ok = 0; free(q); free(d); return; }
    if (threads < 0) {
        uint8_t *dq = w->dev, *dd = w->dev + ((nq + 255) & ~(size_t)255);
        krh_gen_blocks(dq, dd, key, rows, cols, type, f16, std);
        if (krh_copy_d2h(q, dq, nq) != ML_OK || krh_copy_d2h(d, dd, nd) != ML_OK) w->ok = 0;
    } else {
        mat_job j = { key, rows, cols, type, f16, std, q, d, 0, rows };
        run_jobs(&j, threads, mat_rows);
    }
    put(w, q, nq);
    put(w, d, nd);
    free(q);
    free(d);
}

/* n floats: base + scale * N(0,1) */
static void put_vec(writer *w, uint64_t key, int n, float base, float scale) {
    float *v = malloc(sizeof(float) * (size_t)n);
    if (!v) { w->ok = 0; return; }
    for (int i = 0; i < n; i++) v[i] = base + scale * normal_at(key, (uint64_t)i);
    put(w, v, sizeof(float) * (size_t)n);
    free(v);
}

static void wr32(uint8_t *h, int off, uint32_t v) { memcpy(h + off, &v, 4); }
static void wrf(uint8_t *h, int off, float v) { memcpy(h + off, &v, 4); }

ml_status kr_gen_mlb(const char *path, const kr_gen_spec *sp) {
    uint8_t h[256] = { 0 };
    memcpy(h, "MLB1", 4);
    wr32(h, 4, 1);
    wr32(h, 8, (uint32_t)sp->dim); wr32(h, 12, (uint32_t)sp->n_layers); wr32(h, 16, (uint32_t)sp->n_heads);
    wr32(h, 20, (uint32_t)sp->n_kv_heads); wr32(h, 24, (uint32_t)sp->hidden_dim); wr32(h, 28, (uint32_t)sp->vocab);
    wr32(h, 32, (uint32_t)sp->max_seq);
    wrf(h, 36, sp->rope_theta); wrf(h, 40, sp->norm_eps);
    wr32(h, 44, (uint32_t)sp->wtype); wr32(h, 48, sp->shared ? 1u : 0u);
    wr32(h, 52, (uint32_t)sp->rope_type);
    if (sp->rope_type == ML_ROPE_LLAMA3 || sp->rope_type == ML_ROPE_YARN) {
        wrf(h, 56, sp->rope_factor); wrf(h, 60, sp->rope_low_freq_factor); wrf(h, 64, sp->rope_high_freq_factor);
        wr32(h, 68, (uint32_t)sp->rope_orig_max_seq);
    }
    if (sp->rope_type == ML_ROPE_LINEAR) wrf(h, 56, sp->rope_factor);
    if (sp->rope_type == ML_ROPE_YARN) wrf(h, 88, sp->rope_attn_factor);
    const int lflags = sp->layer_sliding || sp->layer_local;
    wr32(h, 92, (uint32_t)sp->sliding_window);
    wr32(h, 96, lflags ? 1u : 0u);
    wrf(h, 100, sp->rope_local_theta);
    wr32(h, 72, sp->wtype == ML_Q4_0 ? sp->q8_mask : 0u);
    wr32(h, 76, sp->qkv_bias ? 1u : 0u);
    wr32(h, 84, sp->qk_norm ? 1u : 0u);
    wr32(h, 108, sp->post_norms ? 1u : 0u);
    wr32(h, 104, (uint32_t)sp->act);
    wrf(h, 112, sp->embed_scale);
    wrf(h, 124, sp->attn_softcap);
    wrf(h, 128, sp->final_softcap);
    wr32(h, 120, sp->scale_f16 ? 1u : 0u);
    ml_config c;
    int shared;
    ml_status st = kr_parse_header(&c, &shared, h);
    if (st != ML_OK) return kr_seterr(st, "generator: invalid model shape");
    uint8_t *dev = NULL;
    if (sp->device) {
        /* room for the largest matrix: quants then scales */
        size_t big = 0;
        const size_t dims[4][2] = { { (size_t)c.vocab, (size_t)c.dim }, { (size_t)c.q_dim, (size_t)c.dim },
                                    { (size_t)c.hidden_dim, (size_t)c.dim }, { (size_t)c.dim, (size_t)c.q_dim } };
        for (int i = 0; i < 4; i++) {
            const size_t n = dims[i][0] * dims[i][1], b = ((n + 255) & ~(size_t)255) + n / QK * 4;
            big = b > big ? b : big;
        }
        st = krh_init();
        if (st != ML_OK) return kr_seterr(st, "%s", krh_last_error());
        dev = krh_alloc(big);
        if (!dev) return kr_seterr(ML_E_NOMEM, "generator: cannot allocate %zu bytes of HBM", big);
    }
    FILE *f = fopen(path, "wb");
    if (!f) { krh_free(dev); return kr_seterr(ML_E_IO, "cannot write %s", path); }
    writer w = { f, 0, 1, dev };
    put(&w, h, sizeof h);
    if (lflags) {   /* one byte a layer after the header (model/mlb.c's order) */
        uint8_t fl[64] = { 0 };
        for (int l = 0; l < c.n_layers && l < 32; l++)
            fl[l] = (uint8_t)(((sp->layer_sliding >> l) & 1u) * ML_LAYER_SLIDING |
                              ((sp->layer_local >> l) & 1u) * ML_LAYER_LOCAL_ROPE);
        if (c.n_layers > 32) w.ok = 0;
        put(&w, fl, (size_t)c.n_layers);
    }
    const int f16 = sp->scale_f16, th = sp->device ? -1 : sp->threads;
    const float sd = sp->std > 0.0f ? sp->std : 0.02f;
    uint64_t s = 0;
#define WT(bits) (c.wtype == ML_Q8_0 || (c.q8_mask & (bits)) ? ML_Q8_0 : ML_Q4_0)
    put_mat(&w, stream_key(sp->seed, s++), c.vocab, c.dim, WT(ML_Q8M_EMB | (shared ? ML_Q8M_CLS : 0)), f16, sd, th);
    for (int l = 0; l < c.n_layers && w.ok; l++) {
        put_vec(&w, stream_key(sp->seed, s++), c.dim, 1.0f, 0.01f);
        put_mat(&w, stream_key(sp->seed, s++), c.q_dim, c.dim, WT(ML_Q8M_QK), f16, sd, th);
        put_mat(&w, stream_key(sp->seed, s++), c.kv_dim, c.dim, WT(ML_Q8M_QK), f16, sd, th);
        put_mat(&w, stream_key(sp->seed, s++), c.kv_dim, c.dim, WT(ML_Q8M_V), f16, sd, th);
        put_mat(&w, stream_key(sp->seed, s++), c.dim, c.q_dim, WT(ML_Q8M_O), f16, sd, th);
        if (c.qkv_bias) {
            put_vec(&w, stream_key(sp->seed, s++), c.q_dim, 0.0f, 0.02f);
            put_vec(&w, stream_key(sp->seed, s++), c.kv_dim, 0.0f, 0.02f);
            put_vec(&w, stream_key(sp->seed, s++), c.kv_dim, 0.0f, 0.02f);
        }
        /* the family norms draw from streams of their own: the other tensors
         * stay those of the same model without them */
        const uint64_t fam = sp->seed ^ 0x3C6EF372FE94F82BULL;
        if (c.qk_norm) {   /* q_norm, k_norm (model/mlb.c's order) */
            put_vec(&w, stream_key(fam, 4 * (uint64_t)l), c.head_dim, 1.0f, 0.1f);
            put_vec(&w, stream_key(fam, 4 * (uint64_t)l + 1), c.head_dim, 1.0f, 0.1f);
        }
        put_vec(&w, stream_key(sp->seed, s++), c.dim, 1.0f, 0.01f);
        put_mat(&w, stream_key(sp->seed, s++), c.hidden_dim, c.dim, WT(ML_Q8M_UP), f16, sd, th);
        put_mat(&w, stream_key(sp->seed, s++), c.dim, c.hidden_dim, WT(ML_Q8M_DOWN), f16, sd, th);
        put_mat(&w, stream_key(sp->seed, s++), c.hidden_dim, c.dim, WT(ML_Q8M_UP), f16, sd, th);
        if (c.post_norms) {   /* post_attn_norm, post_ffn_norm */
            put_vec(&w, stream_key(fam, 4 * (uint64_t)l + 2), c.dim, 1.0f, 0.1f);
            put_vec(&w, stream_key(fam, 4 * (uint64_t)l + 3), c.dim, 1.0f, 0.1f);
        }
    }
    put_vec(&w, stream_key(sp->seed, s++), c.dim, 1.0f, 0.01f);
    if (!shared) put_mat(&w, stream_key(sp->seed, s++), c.vocab, c.dim, WT(ML_Q8M_CLS), f16, sd, th);
#undef WT
    if (fclose(f) != 0) w.ok = 0;
    krh_free(dev);
    return w.ok ? ML_OK : kr_seterr(ML_E_IO, "write failed: %s", path);
}

typedef struct {
    uint64_t key;
    int rows, cols, type;
    uint8_t *q;
    uint16_t *d;
    int r0, r1;
} raw_job;

static void *raw_rows(void *p) {
    raw_job *j = p;
    const int nb = j->cols / QK, qb = j->type == ML_Q8_0 ? QK : QK / 2;
    for (int r = j->r0; r < j->r1; r++)
        for (int b = 0; b < nb; b++) {
            const uint64_t blk = (uint64_t)r * nb + b;
            uint8_t *q = j->q + blk * qb;
            for (int k = 0; k < qb; k += 4) {
                const uint64_t z = draw(j->key, blk * 16 + (uint64_t)k / 4);
                for (int t = 0; t < 4; t++) {
                    const uint32_t u = (uint32_t)(z >> (16 * t)) & 0xffff;
                    q[k + t] = j->type == ML_Q8_0 ? (uint8_t)(int8_t)((int)(u % 255) - 127) : (uint8_t)(u & 0xff);
                }
            }
            const float sc = fabsf(0.01f * normal_at(j->key ^ 0x5555555555555555ULL, blk));
            j->d[blk] = to_f16(sc);
        }
    return NULL;
}

void kr_gen_matrix(void *q, uint16_t *d, int rows, int cols, int type, uint64_t seed, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t th[64];
    raw_job js[64];
    for (int i = 0; i < threads; i++) {
        js[i] = (raw_job){ stream_key(seed, 1000), rows, cols, type, q, d,
                           (int)((long long)rows * i / threads), (int)((long long)rows * (i + 1) / threads) };
        pthread_create(&th[i], NULL, raw_rows, &js[i]);
    }
    for (int i = 0; i < threads; i++) pthread_join(th[i], NULL);
}

void kr_gen_normal(float *x, size_t n, uint64_t seed) {
    const uint64_t key = stream_key(seed, 2000);
    for (size_t i = 0; i < n; i++) x[i] = normal_at(key, i);
}
