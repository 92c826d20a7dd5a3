/* ORACLE — test infrastructure only. Scalar restatement of the reference's
 * kernels (kernels/scalar/k_scalar.c), attention order (ops/ops.c) and forward
 * pass (model/transformer.c). Compiled with -ffp-contract=off like the
 * reference's scalar build, so every float operation rounds where the
 * reference's does. */
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include "kro.h"

/* core/ml.c:39-53 */
uint16_t kro_f32_to_f16(float f) {
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

/* kro_f32_to_f16 over the inputs with bits lo .. lo + n - 1 */
void kro_f32_to_f16_range(uint16_t *out, uint32_t lo, size_t n) {
    for (size_t i = 0; i < n; i++) {
        const uint32_t u = lo + (uint32_t)i;
        float f;
        memcpy(&f, &u, 4);
        out[i] = kro_f32_to_f16(f);
    }
}

/* The check of kro_f32_to_f16: the x86 F16C conversion (vcvtps2ph, IEEE
 * round to nearest even) as the independent reference; NaN inputs must give
 * the quiet NaN 0x7e00 with the input's sign, which F16C does not (it keeps
 * payload bits). Counts mismatches over bit patterns [lo, hi). */
typedef struct { uint64_t lo, hi, bad; } f16_span;

__attribute__((target("f16c"))) static void *f16_scan(void *p) {
    f16_span *sp = p;
    for (uint64_t u = sp->lo; u < sp->hi; u++) {
        const uint32_t b = (uint32_t)u;
        float x;
        memcpy(&x, &b, 4);
        const uint16_t want = isnan(x) ? (uint16_t)(((b >> 16) & 0x8000) | 0x7e00)
                                       : (uint16_t)_cvtss_sh(x, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
        if (kro_f32_to_f16(x) != want) sp->bad++;
    }
    return NULL;
}

uint64_t kro_f32_to_f16_mismatches(uint64_t lo, uint64_t hi, int threads) {
    if (!__builtin_cpu_supports("f16c")) return UINT64_MAX;
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t th[64];
    f16_span sp[64];
    for (int i = 0; i < threads; i++) {
        sp[i].lo = lo + (hi - lo) * (uint64_t)i / (uint64_t)threads;
        sp[i].hi = lo + (hi - lo) * (uint64_t)(i + 1) / (uint64_t)threads;
        sp[i].bad = 0;
        pthread_create(&th[i], NULL, f16_scan, &sp[i]);
    }
    uint64_t bad = 0;
    for (int i = 0; i < threads; i++) { pthread_join(th[i], NULL); bad += sp[i].bad; }
    return bad;
}

/* core/ml.c:55-62 */
float kro_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    if (e == 0) return (sign ? -1.0f : 1.0f) * (float)m * (1.0f / 16777216.0f);
    const uint32_t x = sign | (e == 31 ? 0x7f800000u | (m << 13) : ((e + 112u) << 23) | (m << 13));
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* k_scalar.c:4-17: per row, int32 block dot, then sum += (float)s * wd * xd
 * in block order */
void kro_matvec_q8(float *y, const ml_qtensor *W, const ml_qact *x, int r0, int r1) {
    const int nb = W->cols / QK;
    for (int r = r0; r < r1; r++) {
        const int8_t *wq = W->q + (size_t)r * W->cols;
        const float *wd = W->d + (size_t)r * nb;
        float sum = 0.0f;
        for (int b = 0; b < nb; b++) {
            int32_t s = 0;
            for (int j = 0; j < QK; j++) s += wq[b * QK + j] * x->q[b * QK + j];
            const float t = (float)s * wd[b];
            sum = sum + t * x->d[b];
        }
        y[r] = sum;
    }
}

/* k_scalar.c:19-37: byte j of a block holds elements j (low) and j+16 (high) */
void kro_matvec_q4(float *y, const ml_qtensor *W, const ml_qact *x, int r0, int r1) {
    const int nb = W->cols / QK;
    for (int r = r0; r < r1; r++) {
        const uint8_t *wq = (const uint8_t *)W->q + (size_t)r * nb * (QK / 2);
        const float *wd = W->d + (size_t)r * nb;
        float sum = 0.0f;
        for (int b = 0; b < nb; b++) {
            const uint8_t *p = wq + b * (QK / 2);
            const int8_t *xq = x->q + b * QK;
            int32_t s = 0;
            for (int j = 0; j < QK / 2; j++) {
                s += ((p[j] & 0xF) - 8) * xq[j];
                s += ((p[j] >> 4) - 8) * xq[j + QK / 2];
            }
            const float t = (float)s * wd[b];
            sum = sum + t * x->d[b];
        }
        y[r] = sum;
    }
}

void kro_block_dots(int32_t *s, const ml_qtensor *W, const ml_qact *x, int r0, int r1) {
    const int nb = W->cols / QK;
    for (int r = r0; r < r1; r++)
        for (int b = 0; b < nb; b++) {
            int32_t acc = 0;
            if (W->type == ML_Q8_0) {
                const int8_t *wq = W->q + (size_t)r * W->cols + b * QK;
                for (int j = 0; j < QK; j++) acc += wq[j] * x->q[b * QK + j];
            } else {
                const uint8_t *p = (const uint8_t *)W->q + ((size_t)r * nb + b) * (QK / 2);
                for (int j = 0; j < QK / 2; j++)
                    acc += ((p[j] & 0xF) - 8) * x->q[b * QK + j] + ((p[j] >> 4) - 8) * x->q[b * QK + j + QK / 2];
            }
            s[(size_t)(r - r0) * nb + b] = acc;
        }
}

/* k_scalar.c:39-57 and the rule in docs/file-format.md:133-144 */
void kro_quantize_q8(ml_qact *out, const float *x, int k) {
    for (int b = 0; b < k / QK; b++) {
        const float *xb = x + b * QK;
        float amax = 0.0f;
        for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(xb[j]));
        if (amax < ML_QUANT_TINY) {
            out->d[b] = 0.0f;
            for (int j = 0; j < QK; j++) out->q[b * QK + j] = 0;
            continue;
        }
        const float id = 127.0f / amax;
        out->d[b] = amax / 127.0f;
        for (int j = 0; j < QK; j++) {
            const float m = xb[j] * id;
            float v = truncf(m + copysignf(0.5f, xb[j]));
            v = fminf(fmaxf(v, -127.0f), 127.0f);
            out->q[b * QK + j] = (int8_t)v;
        }
    }
}

/* k_scalar.c:59-64: sequential sum of squares, then (x * inv) * w */
void kro_rmsnorm(float *o, const float *x, const float *w, int n, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss = ss + x[i] * x[i];
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = 0; i < n; i++) o[i] = x[i] * inv * w[i];
}

/* k_scalar.c:66-77 */
void kro_softmax(float *x, int n) {
    float mx = x[0];
    for (int i = 1; i < n; i++) mx = fmaxf(mx, x[i]);
    if (mx == -INFINITY) {
        for (int i = 0; i < n; i++) x[i] = 1.0f / (float)n;
        return;
    }
    float sum = 0.0f;
    for (int i = 0; i < n; i++) { x[i] = kro_expf(x[i] - mx); sum = sum + x[i]; }
    const float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) x[i] *= inv;
}

/* k_scalar.c:100-105, in the C expression's order */
void kro_gelu_mul(float *g, const float *u, int n) {
    for (int i = 0; i < n; i++) {
        const float x = g[i];
        g[i] = 0.5f * x * (1.0f + kro_tanhf(0.7978845608f * (x + 0.044715f * x * x * x))) * u[i];
    }
}

/* ops/ops.c:98-101 */
void kro_softcap_rows(float *x, size_t ld, int rows, int n, float cap) {
    for (int r = 0; r < rows; r++)
        for (int i = 0; i < n; i++) x[(size_t)r * ld + i] = cap * kro_tanhf(x[(size_t)r * ld + i] / cap);
}

/* k_scalar.c:79-94: interleaved pairs (2i, 2i+1) of every head */
static void rope_heads(float *v, const float *c, const float *s, int hd, int nh) {
    for (int h = 0; h < nh; h++) {
        float *p = v + h * hd;
        for (int i = 0; i < hd / 2; i++) {
            const float a = p[2 * i], b = p[2 * i + 1];
            p[2 * i] = a * c[i] - b * s[i];
            p[2 * i + 1] = a * s[i] + b * c[i];
        }
    }
}

void kro_rope(float *q, float *k, const float *cos_t, const float *sin_t, int head_dim, int n_heads, int n_kv_heads) {
    rope_heads(q, cos_t, sin_t, head_dim, n_heads);
    rope_heads(k, cos_t, sin_t, head_dim, n_kv_heads);
}

/* k_scalar.c:96-98: g / (1 + expf(-g)) * u */
void kro_silu_mul(float *g, const float *u, int n) {
    for (int i = 0; i < n; i++) g[i] = g[i] / (1.0f + kro_expf(-g[i])) * u[i];
}

/* k_scalar.c:107-109 */
void kro_add(float *y, const float *x, int n) {
    for (int i = 0; i < n; i++) y[i] += x[i];
}

/* k_scalar.c:111-117 */
void kro_dot_f32(float *s, const float *q, const float *k, size_t ldk, int rows, int n, float scale) {
    for (int t = 0; t < rows; t++, k += ldk) {
        float acc = 0.0f;
        for (int i = 0; i < n; i++) acc = acc + q[i] * k[i];
        s[t] = acc * scale;
    }
}

/* k_scalar.c:119-122 */
void kro_axpy_f32(float *y, const float *a, const float *x, size_t ldx, int rows, int n) {
    for (int t = 0; t < rows; t++, x += ldx)
        for (int i = 0; i < n; i++) y[i] = y[i] + a[t] * x[i];
}

/* core/quant_ref.c:4-19 */
void kro_dequant_row(float *out, const ml_qtensor *W, int row) {
    const int nb = W->cols / QK;
    const float *d = W->d + (size_t)row * nb;
    if (W->type == ML_Q8_0) {
        const int8_t *q = W->q + (size_t)row * W->cols;
        for (int i = 0; i < W->cols; i++) out[i] = q[i] * d[i / QK];
        return;
    }
    const uint8_t *q = (const uint8_t *)W->q + (size_t)row * nb * (QK / 2);
    for (int b = 0; b < nb; b++)
        for (int j = 0; j < QK / 2; j++) {
            const uint8_t v = q[b * (QK / 2) + j];
            out[b * QK + j] = ((v & 0xF) - 8) * d[b];
            out[b * QK + j + QK / 2] = ((v >> 4) - 8) * d[b];
        }
}

/* core/quant_ref.c:21-38 (the amax/7 rule) */
void kro_quantize_row_q4(int8_t *q, float *d, const float *x, int k) {
    for (int b = 0; b < k / QK; b++) {
        const float *xb = x + b * QK;
        float amax = 0.0f;
        for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(xb[j]));
        if (amax < ML_QUANT_TINY) amax = 0.0f;
        const float id = amax != 0.0f ? 7.0f / amax : 0.0f;
        d[b] = amax / 7.0f;
        uint8_t nib[QK];
        for (int j = 0; j < QK; j++) {
            const float m = xb[j] * id;
            float v = truncf(m + copysignf(0.5f, xb[j]));
            v = fminf(fmaxf(v, -8.0f), 7.0f);
            nib[j] = (uint8_t)((int)v + 8);
        }
        for (int j = 0; j < QK / 2; j++) q[b * (QK / 2) + j] = (int8_t)(nib[j] | (nib[j + QK / 2] << 4));
    }
}

/* model/sampler.c:57-61: first index of the maximum */
int kro_argmax(const float *v, int n) {
    int best = 0;
    for (int i = 1; i < n; i++) if (v[i] > v[best]) best = i;
    return best;
}
/* ops/ops.c:81-96: Q8 of a whole row with one scale (the Q8 KV cache's rows
 * and the quantized query heads) */
void kro_quantize_row(int8_t *q, float *d, const float *x, int n) {
    float amax = 0.0f;
    for (int i = 0; i < n; i++) amax = fmaxf(amax, fabsf(x[i]));
    if (amax < ML_QUANT_TINY) {
        *d = 0.0f;
        memset(q, 0, (size_t)n);
        return;
    }
    const float id = 127.0f / amax;
    *d = amax / 127.0f;
    for (int i = 0; i < n; i++) {
        const float m = x[i] * id;
        float v = truncf(m + copysignf(0.5f, x[i]));
        v = fminf(fmaxf(v, -127.0f), 127.0f);
        q[i] = (int8_t)v;
    }
}

/* k_scalar.c:124-129 */
void kro_dot_f16(float *s, const float *q, const uint16_t *k, size_t ldk, int rows, int n, float scale) {
    for (int t = 0; t < rows; t++, k += ldk) {
        float acc = 0.0f;
        for (int i = 0; i < n; i++) acc = acc + q[i] * kro_f16_to_f32(k[i]);
        s[t] = acc * scale;
    }
}

/* k_scalar.c:131-135 */
void kro_axpy_f16(float *y, const float *a, const uint16_t *x, size_t ldx, int rows, int n) {
    for (int t = 0; t < rows; t++, x += ldx)
        for (int i = 0; i < n; i++) y[i] = y[i] + a[t] * kro_f16_to_f32(x[i]);
}

/* k_scalar.c:137-146: exact int32 dot, then (float)sum * (dq * scale) * dk_t */
void kro_dot_q8(float *s, const int8_t *q, float dq, const int8_t *k, const float *dk, size_t ldk, size_t lddk,
                int rows, int n, float scale) {
    const float c = dq * scale;
    for (int t = 0; t < rows; t++) {
        const int8_t *kt = k + (size_t)t * ldk;
        int32_t sum = 0;
        for (int i = 0; i < n; i++) sum += q[i] * kt[i];
        s[t] = (float)sum * c * dk[(size_t)t * lddk];
    }
}

/* k_scalar.c:148-155: w = a_t * dx_t, then y += w * x_t in position order */
void kro_axpy_q8(float *y, const float *a, const int8_t *x, const float *dx, size_t ldx, size_t lddx, int rows,
                 int n) {
    for (int t = 0; t < rows; t++) {
        const int8_t *xt = x + (size_t)t * ldx;
        const float w = a[t] * dx[(size_t)t * lddx];
        for (int i = 0; i < n; i++) y[i] = y[i] + w * (float)xt[i];
    }
}

/* ops/ops.c:169-200 (attend) for the F32 cache, one query head at a time:
 * the 64-position blocks and head grouping of the reference leave each head's
 * operation order as written here (scores per position, softmax over the
 * positions attended, then the V rows added in position order). */
void kro_attention(float *out, const float *q, const ml_kv_layer *kv, float *att, const ml_config *cfg, int pos) {
    const int hd = cfg->head_dim, group = cfg->n_heads / cfg->n_kv_heads;
    const int first = kv->window && pos >= kv->window ? pos + 1 - kv->window : 0;
    const int n = pos + 1 - first;
    const size_t ld = (size_t)cfg->kv_dim, ldd = (size_t)cfg->n_kv_heads;
    /* the Q8 cache: each query head quantized once (ops/ops.c:171-173) */
    int8_t *qq = NULL;
    float *qd = NULL;
    if (kv->kq) {
        qq = malloc((size_t)cfg->q_dim);
        qd = malloc(sizeof(float) * cfg->n_heads);
        if (!qq || !qd) abort();
        for (int h = 0; h < cfg->n_heads; h++) kro_quantize_row(qq + (size_t)h * hd, qd + h, q + (size_t)h * hd, hd);
    }
    for (int h = 0; h < cfg->n_heads; h++) {
        const int g = h / group;
        const size_t off = (size_t)g * hd + (size_t)first * ld, offd = (size_t)first * ldd + g;
        if (kv->k) kro_dot_f32(att, q + (size_t)h * hd, kv->k + off, ld, n, hd, cfg->attn_scale);
        else if (kv->kh) kro_dot_f16(att, q + (size_t)h * hd, kv->kh + off, ld, n, hd, cfg->attn_scale);
        else kro_dot_q8(att, qq + (size_t)h * hd, qd[h], kv->kq + off, kv->kd + offd, ld, ldd, n, hd, cfg->attn_scale);
        if (cfg->attn_softcap > 0.0f) kro_softcap_rows(att, (size_t)n, 1, n, cfg->attn_softcap);   /* ops/ops.c:141 */
        kro_softmax(att, n);
        float *o = out + (size_t)h * hd;
        for (int i = 0; i < hd; i++) o[i] = 0.0f;
        if (kv->v) kro_axpy_f32(o, att, kv->v + off, ld, n, hd);
        else if (kv->vh) kro_axpy_f16(o, att, kv->vh + off, ld, n, hd);
        else kro_axpy_q8(o, att, kv->vq + off, kv->vd + offd, ld, ldd, n, hd);
    }
    free(qq);
    free(qd);
}

/* ---- model ---- */

struct kro_model_data;   /* kro_mlb.c */
int kro_mlb_open(kro_model **m, const char *path);
void kro_mlb_close(kro_model *m);
const ml_config *kro_mlb_config(const kro_model *m);
const ml_qtensor *kro_mlb_tok_emb(const kro_model *m);
const ml_qtensor *kro_mlb_wcls(const kro_model *m);
const float *kro_mlb_final_norm(const kro_model *m);
const ml_layer *kro_mlb_layer(const kro_model *m, int l);

int kro_model_open(kro_model **m, const char *path) { return kro_mlb_open(m, path); }
void kro_model_close(kro_model *m) { kro_mlb_close(m); }
const ml_config *kro_model_config(const kro_model *m) { return kro_mlb_config(m); }

struct kro_state {
    const kro_model *m;
    float *x, *xb, *xb2, *hb, *hb2, *q, *ao, *att, *logits;
    int kv_type;
    float *kcache, *vcache;   /* F32 cache; for F16 / Q8, the current K and V rows (kbuf, vbuf) */
    uint16_t *kh, *vh;        /* F16 cache */
    int8_t *kq, *vq;          /* Q8 cache and its row scales */
    float *kd, *vd;
    float *rope_cos, *rope_sin, *rope_cos_local, *rope_sin_local;
    ml_qact qa_dim, qa_hidden, qa_q;
};

/* model/transformer.c:16-38 */
static double rope_inv_freq(const ml_config *c, int i) {
    const double inv = pow((double)c->rope_theta, -2.0 * i / c->head_dim);
    if (c->rope_type == ML_ROPE_LINEAR) return inv / c->rope_factor;
    if (c->rope_type == ML_ROPE_YARN) {
        const double hd = c->head_dim, orig = c->rope_orig_max_seq, lb = 2.0 * log((double)c->rope_theta);
        const double pi2 = 2.0 * 3.14159265358979323846;
        double lo = floor(hd * log(orig / ((double)c->rope_low_freq_factor * pi2)) / lb);
        double hi = ceil(hd * log(orig / ((double)c->rope_high_freq_factor * pi2)) / lb);
        if (lo < 0.0) lo = 0.0;
        if (hi > hd - 1.0) hi = hd - 1.0;
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

int kro_state_new(kro_state **out, const kro_model *m) { return kro_state_new_kv(out, m, ML_F32); }

/* model/transformer.c:51-166 with kv_type ML_F32, ML_F16 or ML_Q8_0 */
int kro_state_new_kv(kro_state **out, const kro_model *m, int kv_type) {
    const ml_config *c = kro_mlb_config(m);
    if (kv_type != ML_F32 && kv_type != ML_F16 && kv_type != ML_Q8_0) return ML_E_SHAPE;
    kro_state *s = calloc(1, sizeof *s);
    if (!s) return ML_E_NOMEM;
    s->m = m;
    s->kv_type = kv_type;
    const size_t f = sizeof(float), kv = (size_t)c->n_layers * c->max_seq * c->kv_dim;
    const size_t ks = (size_t)c->n_layers * c->max_seq * c->n_kv_heads;
    const size_t half = (size_t)c->max_seq * (c->head_dim / 2);
    s->x = calloc(c->dim, f); s->xb = calloc(c->dim, f); s->xb2 = calloc(c->dim, f);
    s->hb = calloc(c->hidden_dim, f); s->hb2 = calloc(c->hidden_dim, f);
    s->q = calloc(c->q_dim, f); s->ao = calloc(c->q_dim, f);
    s->att = calloc(c->max_seq, f); s->logits = calloc(c->vocab, f);
    if (kv_type == ML_F32) {
        s->kcache = calloc(kv, f); s->vcache = calloc(kv, f);
    } else {
        s->kcache = calloc(c->kv_dim, f); s->vcache = calloc(c->kv_dim, f);
        if (kv_type == ML_F16) {
            s->kh = calloc(kv, 2); s->vh = calloc(kv, 2);
        } else {
            s->kq = calloc(kv, 1); s->vq = calloc(kv, 1); s->kd = calloc(ks, f); s->vd = calloc(ks, f);
        }
        if ((kv_type == ML_F16 && (!s->kh || !s->vh)) || (kv_type == ML_Q8_0 && (!s->kq || !s->vq || !s->kd || !s->vd))) {
            kro_state_free(s);
            return ML_E_NOMEM;
        }
    }
    s->rope_cos = calloc(half, f); s->rope_sin = calloc(half, f);
    s->qa_dim = (ml_qact){ malloc(c->dim), malloc(f * c->dim / QK), c->dim };
    s->qa_hidden = (ml_qact){ malloc(c->hidden_dim), malloc(f * c->hidden_dim / QK), c->hidden_dim };
    s->qa_q = (ml_qact){ malloc(c->q_dim), malloc(f * c->q_dim / QK), c->q_dim };
    if (c->rope_local_theta > 0.0f) { s->rope_cos_local = calloc(half, f); s->rope_sin_local = calloc(half, f); }
    if (!s->kcache || !s->vcache || !s->rope_sin || !s->qa_q.d || (c->rope_local_theta > 0.0f && !s->rope_sin_local)) {
        kro_state_free(s);
        return ML_E_NOMEM;
    }
    /* model/transformer.c:147-162 */
    const int h2 = c->head_dim / 2;
    const double af = c->rope_type == ML_ROPE_YARN ? c->rope_attn_factor : 1.0;
    for (int i = 0; i < h2; i++) {
        const double freq = rope_inv_freq(c, i);
        const double lfreq = s->rope_cos_local ? pow((double)c->rope_local_theta, -2.0 * i / c->head_dim) : 0.0;
        for (int p = 0; p < c->max_seq; p++) {
            const double ang = p * freq;
            s->rope_cos[(size_t)p * h2 + i] = (float)(cos(ang) * af);
            s->rope_sin[(size_t)p * h2 + i] = (float)(sin(ang) * af);
            if (s->rope_cos_local) {
                s->rope_cos_local[(size_t)p * h2 + i] = (float)cos(p * lfreq);
                s->rope_sin_local[(size_t)p * h2 + i] = (float)sin(p * lfreq);
            }
        }
    }
    *out = s;
    return ML_OK;
}

void kro_state_free(kro_state *s) {
    if (!s) return;
    free(s->x); free(s->xb); free(s->xb2); free(s->hb); free(s->hb2); free(s->q); free(s->ao);
    free(s->att); free(s->logits); free(s->kcache); free(s->vcache);
    free(s->kh); free(s->vh); free(s->kq); free(s->vq); free(s->kd); free(s->vd);
    free(s->rope_cos); free(s->rope_sin); free(s->rope_cos_local); free(s->rope_sin_local);
    free(s->qa_dim.q); free(s->qa_dim.d); free(s->qa_hidden.q); free(s->qa_hidden.d);
    free(s->qa_q.q); free(s->qa_q.d);
    free(s);
}

static void matvec(float *y, const ml_qtensor *W, const ml_qact *x) {
    if (W->type == ML_Q8_0) kro_matvec_q8(y, W, x, 0, W->rows);
    else kro_matvec_q4(y, W, x, 0, W->rows);
}

/* model/transformer.c:240-243 */
static void residual_add(const ml_config *c, float *x, float *y, const float *post_norm) {
    if (post_norm) kro_rmsnorm(y, y, post_norm, c->dim, c->norm_eps);
    kro_add(x, y, c->dim);
}

/* model/transformer.c:246-248 */
static void heads_norm(float *x, const float *w, int n, const ml_config *c) {
    for (int h = 0; h < n; h++) kro_rmsnorm(x + (size_t)h * c->head_dim, x + (size_t)h * c->head_dim, w, c->head_dim, c->norm_eps);
}

/* model/transformer.c:191-205 (store_kv): the F16 cache rounds the position's
 * K and V to half precision; the Q8 cache quantizes each KV head's rows */
static void store_kv(kro_state *s, int l, int pos, const float *k, const float *v) {
    if (s->kv_type == ML_F32) return;
    const ml_config *c = kro_mlb_config(s->m);
    const size_t row = (size_t)l * c->max_seq + pos;
    if (s->kv_type == ML_F16) {
        uint16_t *kh = s->kh + row * c->kv_dim, *vh = s->vh + row * c->kv_dim;
        for (int i = 0; i < c->kv_dim; i++) { kh[i] = kro_f32_to_f16(k[i]); vh[i] = kro_f32_to_f16(v[i]); }
        return;
    }
    for (int h = 0; h < c->n_kv_heads; h++) {
        const size_t o = (size_t)h * c->head_dim;
        kro_quantize_row(s->kq + row * c->kv_dim + o, s->kd + row * c->n_kv_heads + h, k + o, c->head_dim);
        kro_quantize_row(s->vq + row * c->kv_dim + o, s->vd + row * c->n_kv_heads + h, v + o, c->head_dim);
    }
}

/* model/transformer.c:169-180 (kv_layer): layer l's view of the cache */
static ml_kv_layer kv_layer(const kro_state *s, int l, int window) {
    const ml_config *c = kro_mlb_config(s->m);
    const size_t rows = (size_t)l * c->max_seq;
    if (s->kv_type == ML_F32)
        return (ml_kv_layer){ s->kcache + rows * c->kv_dim, s->vcache + rows * c->kv_dim, NULL, NULL, NULL, NULL, window,
                              NULL, NULL };
    if (s->kv_type == ML_F16)
        return (ml_kv_layer){ NULL, NULL, NULL, NULL, NULL, NULL, window, s->kh + rows * c->kv_dim, s->vh + rows * c->kv_dim };
    return (ml_kv_layer){ NULL, NULL, s->kq + rows * c->kv_dim, s->vq + rows * c->kv_dim, s->kd + rows * c->n_kv_heads,
                          s->vd + rows * c->n_kv_heads, window, NULL, NULL };
}

/* model/transformer.c:257-306; `cls` = run the classifier. With an F16 or Q8
 * cache the projections write the staging rows, which store_kv converts. */
static void forward(kro_state *s, int token, int pos, int cls) {
    const kro_model *m = s->m;
    const ml_config *c = kro_mlb_config(m);
    kro_dequant_row(s->x, kro_mlb_tok_emb(m), token);
    if (c->embed_scale != 1.0f)
        for (int i = 0; i < c->dim; i++) s->x[i] *= c->embed_scale;
    for (int l = 0; l < c->n_layers; l++) {
        const ml_layer *L = kro_mlb_layer(m, l);
        const size_t row = (size_t)l * c->max_seq;
        const int conv = s->kv_type != ML_F32;
        float *k = conv ? s->kcache : s->kcache + (row + pos) * c->kv_dim;
        float *v = conv ? s->vcache : s->vcache + (row + pos) * c->kv_dim;
        const size_t ro = (size_t)pos * (c->head_dim / 2);
        const float *cs = (L->local_rope ? s->rope_cos_local : s->rope_cos) + ro;
        const float *sn = (L->local_rope ? s->rope_sin_local : s->rope_sin) + ro;
        kro_rmsnorm(s->xb, s->x, L->attn_norm, c->dim, c->norm_eps);
        kro_quantize_q8(&s->qa_dim, s->xb, c->dim);
        matvec(s->q, &L->wq, &s->qa_dim);
        matvec(k, &L->wk, &s->qa_dim);
        matvec(v, &L->wv, &s->qa_dim);
        if (L->bq) { kro_add(s->q, L->bq, c->q_dim); kro_add(k, L->bk, c->kv_dim); kro_add(v, L->bv, c->kv_dim); }
        if (L->q_norm) { heads_norm(s->q, L->q_norm, c->n_heads, c); heads_norm(k, L->k_norm, c->n_kv_heads, c); }
        kro_rope(s->q, k, cs, sn, c->head_dim, c->n_heads, c->n_kv_heads);
        store_kv(s, l, pos, k, v);
        const ml_kv_layer kv = kv_layer(s, l, L->window);
        kro_attention(s->ao, s->q, &kv, s->att, c, pos);
        kro_quantize_q8(&s->qa_q, s->ao, c->q_dim);
        matvec(s->xb2, &L->wo, &s->qa_q);
        residual_add(c, s->x, s->xb2, L->post_attn_norm);
        kro_rmsnorm(s->xb, s->x, L->ffn_norm, c->dim, c->norm_eps);
        kro_quantize_q8(&s->qa_dim, s->xb, c->dim);
        matvec(s->hb, &L->w1, &s->qa_dim);
        matvec(s->hb2, &L->w3, &s->qa_dim);
        if (c->act == ML_ACT_GELU_TANH) kro_gelu_mul(s->hb, s->hb2, c->hidden_dim);   /* act_mul */
        else kro_silu_mul(s->hb, s->hb2, c->hidden_dim);
        kro_quantize_q8(&s->qa_hidden, s->hb, c->hidden_dim);
        matvec(s->xb2, &L->w2, &s->qa_hidden);
        residual_add(c, s->x, s->xb2, L->post_ffn_norm);
    }
    if (!cls) return;
    kro_rmsnorm(s->xb, s->x, kro_mlb_final_norm(m), c->dim, c->norm_eps);
    kro_quantize_q8(&s->qa_dim, s->xb, c->dim);
    matvec(s->logits, kro_mlb_wcls(m), &s->qa_dim);
    if (c->final_softcap > 0.0f) kro_softcap_rows(s->logits, (size_t)c->vocab, 1, c->vocab, c->final_softcap);
}

int kro_forward(kro_state *s, int token, int pos, float *out) {
    const ml_config *c = kro_mlb_config(s->m);
    if (pos < 0 || pos >= c->max_seq || token < 0 || token >= c->vocab) return ML_E_SHAPE;
    forward(s, token, pos, 1);
    if (out) memcpy(out, s->logits, sizeof(float) * c->vocab);
    return ML_OK;
}

/* Batched prefill computes every per-token operation in ml_forward's order
 * (model/transformer.c:381-384), so it is token-by-token forward here. */
int kro_prefill(kro_state *s, const int *tokens, int n, int pos0, float *logits) {
    const ml_config *c = kro_mlb_config(s->m);
    if (n < 0 || pos0 < 0 || pos0 + n > c->max_seq) return ML_E_SHAPE;
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= c->vocab) return ML_E_SHAPE;
    for (int i = 0; i < n; i++) {
        forward(s, tokens[i], pos0 + i, logits != NULL);
        if (logits) memcpy(logits + (size_t)i * c->vocab, s->logits, sizeof(float) * c->vocab);
    }
    return ML_OK;
}

/* app/ml_run.c:369-404 with -T 0 (greedy) and no --eos */
int kro_generate(kro_state *s, const int *prompt, int np, int steps, int *out) {
    const ml_config *c = kro_mlb_config(s->m);
    if (np < 1 || np > c->max_seq) return -1;
    if (steps > c->max_seq) steps = c->max_seq;
    int token = prompt[0], pos = 0, n = 0;
    const int npre = np - 1 < steps - 1 ? np - 1 : steps - 1;
    if (npre > 0) {
        if (kro_prefill(s, prompt, npre, 0, NULL) != ML_OK) return -1;
        for (pos = 0; pos < npre; pos++) out[n++] = prompt[pos + 1];
        token = prompt[npre];
    }
    while (pos < steps) {
        forward(s, token, pos, 1);
        const int next = pos + 1 >= np ? kro_argmax(s->logits, c->vocab) : prompt[pos + 1];
        pos++;
        out[n++] = next;
        token = next;
    }
    return n;
}

const float *kro_state_x(const kro_state *s) { return s->x; }
const void *kro_state_cache(const kro_state *s, const char *name) {
    if (!strcmp(name, "kh")) return s->kh;
    if (!strcmp(name, "vh")) return s->vh;
    if (!strcmp(name, "kq")) return s->kq;
    if (!strcmp(name, "vq")) return s->vq;
    if (!strcmp(name, "kd")) return s->kd;
    if (!strcmp(name, "vd")) return s->vd;
    return NULL;
}

const float *kro_state_kcache(const kro_state *s, int layer) {
    const ml_config *c = kro_mlb_config(s->m);
    return s->kcache + (size_t)layer * c->max_seq * c->kv_dim;
}

const float *kro_state_buffer(const kro_state *s, const char *name) {
    if (!strcmp(name, "x")) return s->x;
    if (!strcmp(name, "q")) return s->q;
    if (!strcmp(name, "ao")) return s->ao;
    if (!strcmp(name, "kcache")) return s->kcache;
    if (!strcmp(name, "vcache")) return s->vcache;
    if (!strcmp(name, "rope_cos")) return s->rope_cos;
    if (!strcmp(name, "rope_sin")) return s->rope_sin;
    return NULL;
}

/* ---- the sampler: model/sampler.c ----
 * Restated from the reference's steps: the penalty once per distinct recent
 * token, temperature, the softmax above, one xorshift64* draw, then the
 * multinomial walk, the top-k cut or the top-p nucleus, each summed one add
 * at a time from +0 in the order the reference sums. Candidates are ordered
 * by (probability descending, id ascending): a total order when the
 * probabilities are numbers, so any correct sort gives the reference's
 * sequence. When they are NaN (a NaN logit, or +inf: inf - inf), all of them
 * are, and the reference's heap and qsort then keep id order; that case is
 * written out where it matters. */
struct kro_sampler {
    kro_sampler_opts o;
    uint64_t rng;
    int vocab, n_recent, recent_at;
    int *recent;
    float *probs;
    int *ids;
};

/* model/sampler.c:6-18 */
int kro_sampler_new(kro_sampler **out, int vocab, const kro_sampler_opts *o) {
    kro_sampler *s = calloc(1, sizeof *s);
    if (!s) return ML_E_NOMEM;
    s->o = *o;
    s->vocab = vocab;
    s->rng = o->seed ? o->seed : 0x9E3779B97F4A7C15ull;
    if (s->o.repeat_last_n < 0) s->o.repeat_last_n = 0;
    s->recent = malloc(sizeof(int) * (size_t)(s->o.repeat_last_n > 0 ? s->o.repeat_last_n : 1));
    s->probs = malloc(sizeof(float) * (size_t)vocab);
    s->ids = malloc(sizeof(int) * (size_t)vocab);
    if (!s->recent || !s->probs || !s->ids) { kro_sampler_free(s); return ML_E_NOMEM; }
    *out = s;
    return ML_OK;
}

void kro_sampler_free(kro_sampler *s) {
    if (!s) return;
    free(s->recent);
    free(s->probs);
    free(s->ids);
    free(s);
}

uint64_t kro_sampler_rng(const kro_sampler *s) { return s->rng; }

/* model/sampler.c:30-35: a ring of the last repeat_last_n ids */
void kro_sampler_accept(kro_sampler *s, int token) {
    const int R = s->o.repeat_last_n;
    if (R <= 0 || token < 0 || token >= s->vocab) return;
    s->recent[s->recent_at] = token;
    s->recent_at = (s->recent_at + 1) % R;
    if (s->n_recent < R) s->n_recent++;
}

/* model/sampler.c:39-48: each distinct id of the ring (below n) once: a
 * positive logit divided by the penalty, any other multiplied */
static void smp_penalize(kro_sampler *s, float *logits, int n) {
    const float rp = s->o.repeat_penalty;
    if (rp == 1.0f || s->n_recent == 0) return;
    for (int i = 0; i < s->n_recent; i++) {
        const int t = s->recent[i];
        if (t >= n) continue;
        int dup = 0;
        for (int j = 0; j < i && !dup; j++) dup = s->recent[j] == t;
        if (dup) continue;
        logits[t] = logits[t] > 0.0f ? logits[t] / rp : logits[t] * rp;
    }
}

/* model/sampler.c:50-55: xorshift64*, the top 24 bits of the product's high
 * word over 2^24 */
static float smp_coin(uint64_t *st) {
    uint64_t x = *st;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *st = x;
    const uint32_t hi = (uint32_t)((x * 0x2545F4914F6CDD1Dull) >> 32);
    return (float)(hi >> 8) / 16777216.0f;
}

static const float *g_sort_p;   /* the probabilities qsort orders ids by */
static int smp_cmp(const void *a, const void *b) {
    const int i = *(const int *)a, j = *(const int *)b;
    const float pi = g_sort_p[i], pj = g_sort_p[j];
    if (pi != pj) return pi > pj ? -1 : 1;
    return i < j ? -1 : i > j;
}

/* the first i < m with thr < p[ids[0]] + ... + p[ids[i]] (one add at a time
 * from +0), or -1; *sum: that partial sum, or the sum of all m */
static int smp_first_above(const float *p, const int *ids, int m, float thr, float *sum) {
    float s = 0.0f;
    for (int i = 0; i < m; i++) {
        s += p[ids ? ids[i] : i];
        if (thr < s) { *sum = s; return i; }
    }
    *sum = s;
    return -1;
}

/* model/sampler.c:155-165 with the draws of :63-70, :84-130 and :132-153 */
int kro_sample(kro_sampler *s, float *logits, int n) {
    smp_penalize(s, logits, n);
    if (s->o.temperature == 0.0f) return kro_argmax(logits, n);
    float *p = s->probs;
    for (int i = 0; i < n; i++) p[i] = logits[i] / s->o.temperature;
    kro_softmax(p, n);
    const float coin = smp_coin(&s->rng);
    const float topp = s->o.topp;
    const int nucleus = topp > 0.0f && topp < 1.0f;
    const int isnan_p = p[0] != p[0];   /* then every probability is NaN */
    if (s->o.topk > 0 && s->o.topk < n) {
        /* :84-130: the k first candidates, their sum, the nucleus cut at
         * topp of that sum, the draw at coin times the kept mass */
        const int k = s->o.topk;
        for (int i = 0; i < n; i++) s->ids[i] = i;
        if (!isnan_p) {
            g_sort_p = p;
            qsort(s->ids, (size_t)n, sizeof(int), smp_cmp);
        }
        float total, cum;
        smp_first_above(p, s->ids, k, INFINITY, &total);
        int last = k - 1;
        if (nucleus) {
            const int i = smp_first_above(p, s->ids, k, topp * total, &cum);
            if (i >= 0) last = i;
            total = cum;
        }
        float c;
        const int j = smp_first_above(p, s->ids, last + 1, coin * total, &c);
        return s->ids[j >= 0 ? j : last];
    }
    if (!nucleus) {   /* :63-70 */
        float c;
        const int j = smp_first_above(p, NULL, n, coin, &c);
        return j >= 0 ? j : n - 1;
    }
    /* :132-153: candidates at or above (1 - topp) / (n - 1), sorted; the
     * nucleus is the shortest prefix whose sum exceeds topp */
    const float cutoff = n > 1 ? (1.0f - topp) / (float)(n - 1) : 0.0f;
    int m = 0;
    for (int i = 0; i < n; i++)
        if (p[i] >= cutoff) s->ids[m++] = i;
    if (m == 0) return kro_argmax(p, n);
    g_sort_p = p;
    qsort(s->ids, (size_t)m, sizeof(int), smp_cmp);
    float cum, c;
    const int i = smp_first_above(p, s->ids, m, topp, &cum);
    const int last = i >= 0 ? i : m - 1;
    const int j = smp_first_above(p, s->ids, last + 1, coin * cum, &c);
    return s->ids[j >= 0 ? j : last];
}

/* app/ml_run.c:361-404 with a sampler: the prompt's ids accepted, every
 * drawn id accepted after its draw; no --eos */
int kro_generate_sampled(kro_state *s, kro_sampler *smp, const int *prompt, int np, int steps, int *out) {
    const ml_config *c = kro_mlb_config(s->m);
    if (np < 1 || np > c->max_seq) return -1;
    for (int i = 0; i < np; i++) kro_sampler_accept(smp, prompt[i]);
    if (steps > c->max_seq) steps = c->max_seq;
    int token = prompt[0], pos = 0, n = 0;
    const int npre = np - 1 < steps - 1 ? np - 1 : steps - 1;
    if (npre > 0) {
        if (kro_prefill(s, prompt, npre, 0, NULL) != ML_OK) return -1;
        for (pos = 0; pos < npre; pos++) out[n++] = prompt[pos + 1];
        token = prompt[npre];
    }
    while (pos < steps) {
        forward(s, token, pos, 1);
        const int sampled = pos + 1 >= np;
        const int next = sampled ? kro_sample(smp, s->logits, c->vocab) : prompt[pos + 1];
        if (sampled) kro_sampler_accept(smp, next);
        pos++;
        out[n++] = next;
        token = next;
    }
    return n;
}
