/* libkrafla_hip.so: the MI355X (gfx950) device layer of the Krafla token loop.
 *
 * Plain C ABI: device pointers, sizes and the reference's own types
 * (krafla_types.h). Three groups of entry points:
 *
 *   1. runtime   device guard, HBM allocation, copies, one stream, graphs
 *   2. fused ops the decode/prefill step as fused HIP kernels on the library
 *                stream, each computing exactly the float operations of the
 *                reference's scalar path (kernels/scalar/k_scalar.c) in its
 *                order, so results are bit-identical
 *   3. op table  the reference's kernel and ops ABI under its own names
 *                (krafla_optable.h), for the ISA=hip binding
 *
 * Ops return void, as the reference's kernels do (docs/kernels.md:50); a
 * launch or device error is kept as a sticky status that krh_sync() and
 * krh_status() report, with the message in krh_last_error().
 */
#ifndef KRAFLA_HIP_H
#define KRAFLA_HIP_H
#include "krafla_types.h"

#ifdef __cplusplus
extern "C" {
#endif

/* A quantized matrix resident in HBM, in the .mlb layout (row-major, one row
 * per output; Q4 byte j of a block = elements j and j+16, docs/file-format.md
 * :121-131). Scales [rows][cols/32] are f32, or f16 when d16 is set (the
 * file's own width; widened exactly on the fly). */
typedef struct {
    const void *q;
    const void *d;
    int rows, cols;
    int type;   /* ML_Q8_0 or ML_Q4_0 */
    int d16;
} krh_mat;

typedef struct krh_graph krh_graph;

/* ---- 1. runtime ---- */

/* Selects device 0 and checks it is gfx950: ML_E_ISA otherwise (the hip
 * counterpart of ml_isa_check, core/isa_check.h:8-9). Idempotent. */
ml_status krh_init(void);
const char *krh_device_arch(void);
/* compute units of device 0 (0 before krh_init) */
int krh_device_cus(void);
/* ML_OK, or the first error since the last krh_clear_error() */
ml_status krh_status(void);
const char *krh_last_error(void);
void krh_clear_error(void);
void *krh_alloc(size_t bytes);          /* HBM, 256-byte aligned; NULL on failure */
void krh_free(void *p);
void *krh_host_alloc(size_t bytes);     /* pinned host memory */
void krh_host_free(void *p);
ml_status krh_copy_h2d(void *dst, const void *src, size_t bytes);   /* synchronous */
ml_status krh_copy_d2h(void *dst, const void *src, size_t bytes);   /* synchronous */
void krh_copy_d2d_async(void *dst, const void *src, size_t bytes);  /* on the library stream */
ml_status krh_sync(void);               /* waits for the library stream */
/* Stream capture into a graph: every op issued between begin and end is
 * recorded, not run; krh_graph_launch replays them. */
ml_status krh_graph_begin(void);
ml_status krh_graph_end(krh_graph **g);
ml_status krh_graph_launch(const krh_graph *g);
void krh_graph_free(krh_graph *g);
/* Events on the library stream, for timing: milliseconds between two marks */
typedef struct krh_timer krh_timer;
krh_timer *krh_timer_new(void);
void krh_timer_mark(krh_timer *t, int which);   /* which = 0 (start) or 1 (stop) */
float krh_timer_ms(krh_timer *t);               /* synchronizes on the stop mark */
void krh_timer_free(krh_timer *t);

/* ---- 2. fused ops (device pointers; `pos` and `tok` point to device ints so a
 *         captured step replays without new arguments) ---- */

/* x[0..cols) = row *tok of emb, dequantized (core/quant_ref.c:4-19),
 * times embed_scale when it is not 1 (model/transformer.c:226-230) */
void krh_embed(float *x, const krh_mat *emb, const int *tok, float embed_scale);

/* o = rmsnorm(x) * w (k_scalar.c:59-64), quantized to Q8_0 blocks into q, d
 * (k_scalar.c:39-57); xb (nullable) receives the float o. ntok rows of n. */
void krh_rmsnorm_q8(int8_t *q, float *d, float *xb, const float *x, const float *w, int n, float eps, int ntok);

/* Q8_0 quantize of ntok rows of n floats (k_scalar.c:39-57) */
void krh_quantize_q8(int8_t *q, float *d, const float *x, int n, int ntok);
/* the same two with the scales transposed: d[b * dld + t] (dld >= ntok), the
 * layout krh_matmul reads */
void krh_rmsnorm_q8_t(int8_t *q, float *d, int dld, float *xb, const float *x, const float *w, int n, float eps,
                      int ntok);
void krh_quantize_q8_t(int8_t *q, float *d, int dld, const float *x, int n, int ntok);

/* y = W x (k_scalar.c:4-37); accumulate != 0: y += W x, the residual add of
 * model/transformer.c:240-243 */
void krh_matvec(float *y, const krh_mat *W, const int8_t *xq, const float *xd, int accumulate);
/* y = W x and r += y in one launch (model/transformer.c:284-287: the
 * projection into a scratch row, then ml_k_add into the residual); r and y
 * do not overlap */
void krh_matvec_residual(float *r, float *y, const krh_mat *W, const int8_t *xq, const float *xd);
/* krh_matvec_residual from a float input x quantized inside the launch, which
 * also stores that Q8_0 of x into xq, xd (W->cols <= 16384): the reference's
 * quantize_q8 of x, product into y and add into r as one launch
 * (model/transformer.c:282-287) */
void krh_matvec_f_residual_keep(float *r, float *y, const krh_mat *W, const float *x, int8_t *xq, float *xd);
/* y[i] = W[i] x for nmat (1..3) matrices of one input length, type and
 * scale kind, in one launch (the ml_matvec calls of model/transformer.c:273-275
 * and :290-291 that share their input) */
void krh_matvec_multi(float *const *y, const krh_mat *const *W, int nmat, const int8_t *xq, const float *xd);
/* the same with a float input x[W->cols], quantized to Q8_0 first
 * (k_scalar.c:39-57) inside the launch */
void krh_matvec_f(float *y, const krh_mat *W, const float *x, int accumulate);
/* the same with x normalized first: y (+)= W q8(rmsnorm(x) * nw)
 * (model/transformer.c:299-303, k_scalar.c:59-64) -- every workgroup runs the
 * norm's ordered sum itself while its weight loads are in flight */
void krh_rmsnorm_matvec(float *y, const krh_mat *W, const float *x, const float *nw, float eps, int accumulate);

/* The attention projections of one layer at position *pos
 * (model/transformer.c:270-281): q = wq x, k = wk x, v = wv x, plus the
 * biases when non-NULL, then RoPE on q and k with the tables' row *pos;
 * k and v go to row *pos of this layer's F32 cache (kc, vc: [max_seq][kv_dim]). */
void krh_matvec_qkv(float *q, float *kc, float *vc, const krh_mat *wq, const krh_mat *wk, const krh_mat *wv,
                    const float *bq, const float *bk, const float *bv, const int8_t *xq, const float *xd,
                    const float *rope_cos, const float *rope_sin, int head_dim, const int *pos);

/* h = silu(w1 x) * (w3 x) (k_scalar.c:96-98; model/transformer.c:291-293) */
void krh_matvec_swiglu(float *h, const krh_mat *w1, const krh_mat *w3, const int8_t *xq, const float *xd);
/* the same, with u = w3 x stored as well (the two ml_matvec outputs and the
 * ml_k_silu_mul of model/transformer.c:290-293, all three effects) */
void krh_matvec_swiglu_keep(float *h, float *u, const krh_mat *w1, const krh_mat *w3, const int8_t *xq,
                            const float *xd);

/* krh_matvec_qkv and krh_matvec_swiglu with their input normalized first
 * (the attention and FFN norms, model/transformer.c:270-271, :288-289): x is
 * the residual stream, nw the norm weight */
void krh_rmsnorm_matvec_qkv(float *q, float *kc, float *vc, const krh_mat *wq, const krh_mat *wk, const krh_mat *wv,
                            const float *bq, const float *bk, const float *bv, const float *x, const float *nw,
                            float eps, const float *rope_cos, const float *rope_sin, int head_dim, const int *pos);
void krh_rmsnorm_matvec_swiglu(float *h, const krh_mat *w1, const krh_mat *w3, const float *x, const float *nw,
                               float eps);
/* The fused-norm launches with every effect of the reference's separate calls
 * (model/transformer.c:270-293): xb receives rmsnorm(x) * nw and xq, xd its
 * Q8_0 (as ml_k_rmsnorm and ml_k_quantize_q8 leave them), u receives w3 x,
 * and k, v go to the rows k, v with RoPE at tables row *pos; dim <= 8192,
 * xb and xq 16-byte aligned */
void krh_rmsnorm_matvec_swiglu_keep(float *h, float *u, const krh_mat *w1, const krh_mat *w3, const float *x,
                                    const float *nw, float eps, float *xb, int8_t *xq, float *xd);
void krh_rmsnorm_matvec_qkv_keep(float *q, float *k, float *v, const krh_mat *wq, const krh_mat *wk,
                                 const krh_mat *wv, const float *bq, const float *bk, const float *bv, const float *x,
                                 const float *nw, float eps, const float *rope_cos, const float *rope_sin,
                                 int head_dim, const int *pos, float *xb, int8_t *xq, float *xd);
/* krh_rmsnorm_matvec_qkv for the F16 cache: k and v go to row *pos of this
 * layer's F16 cache (kc, vc: [max_seq][kv_dim] halves), each value rounded as
 * store_kv rounds it (model/transformer.c:195-197, core/ml.c:39-53) */
void krh_rmsnorm_matvec_qkv_f16(float *q, uint16_t *kc, uint16_t *vc, const krh_mat *wq, const krh_mat *wk,
                                const krh_mat *wv, const float *bq, const float *bk, const float *bv, const float *x,
                                const float *nw, float eps, const float *rope_cos, const float *rope_sin, int head_dim,
                                const int *pos);
/* krh_rmsnorm_matvec_qkv for an F16 or Q8 cache: k and v go to the staging
 * rows k, v [kv_dim] (the state's kbuf, vbuf: model/transformer.c:262-263),
 * which krh_store_kv then converts into the cache */
void krh_rmsnorm_matvec_qkv_stage(float *q, float *k, float *v, const krh_mat *wq, const krh_mat *wk,
                                  const krh_mat *wv, const float *bq, const float *bk, const float *bv, const float *x,
                                  const float *nw, float eps, const float *rope_cos, const float *rope_sin,
                                  int head_dim, const int *pos);

/* Causal GQA attention of one position *pos over this layer's F32 cache
 * (ops/ops.c:169-225): ao [n_heads * head_dim]; aq, ad (nullable) receive its
 * Q8_0 quantization. att: n_heads * max_seq floats of scratch. head_dim % 4
 * == 0, at most 16 query heads per KV head. */
void krh_attention(float *ao, int8_t *aq, float *ad, float *att, const float *q, const float *kc, const float *vc,
                   int n_heads, int n_kv_heads, int head_dim, int max_seq, int window, float scale, const int *pos);
/* krh_attention without the att workspace and without the quantized copy:
 * the score rows live in a static device array of KRH_ATTN_SCRATCH_FLOATS
 * floats per device, so the call allocates nothing (no hipMalloc, no
 * library allocation). No counterpart in the reference: it is for callers
 * that cannot allocate (code under graph capture, serving loops that forbid
 * allocation). n_heads * max_seq must not exceed KRH_ATTN_SCRATCH_FLOATS
 * (ML_E_SHAPE otherwise). Calls that overlap on one device race on the
 * array. Results equal krh_attention's bit for bit. */
#define KRH_ATTN_SCRATCH_FLOATS (1 << 21)
void krh_attention_noalloc(float *ao, const float *q, const float *kc, const float *vc, int n_heads, int n_kv_heads,
                           int head_dim, int max_seq, int window, float scale, const int *pos);
/* The same over one layer's cache of any type (ml_attention, ops/ops.c:124-180):
 * kv (a host struct of device pointers, ops/ops.h:16-22) names the layer's F32
 * rows (k, v), F16 rows (kh, vh) or Q8 rows and row scales (kq, vq, kd, vd),
 * and the window. The Q8 scores quantize each query head with one scale
 * (ops/ops.c:171-173) and take the exact int32 dot (k_scalar.c:137-155). ntok
 * positions *pos0 + t, t < ntok (ml_attention_batch for ntok > 1): ao, q
 * [ntok][q_dim], att [ntok][n_heads][max_seq]; last_pos = *pos0 + ntok - 1
 * sizes the launch (max_seq - 1 when only the device knows *pos0). */
void krh_attention_kv(float *ao, float *att, const float *q, const ml_kv_layer *kv, int n_heads, int n_kv_heads,
                      int head_dim, int max_seq, float scale, const int *pos0, int ntok, int last_pos);
/* Decode over the Q8 cache with row *pos not stored yet: krh_store_kv of the
 * staging rows k_row, v_row [kv_dim] followed by krh_attention_kv (ntok 1),
 * the store done by the score launch itself (the workgroup whose tile holds
 * *pos). Same cache contents and results as the two calls. */
void krh_attention_q8_store(float *ao, float *att, const float *q, const ml_kv_layer *kv, const float *k_row,
                            const float *v_row, int n_heads, int n_kv_heads, int head_dim, int max_seq, float scale,
                            const int *pos);
/* store_kv (model/transformer.c:191-205) of positions *pos0 + t, t < ntok:
 * the staging rows k, v [ntok][n_kv_heads * head_dim] into one layer's cache
 * rows kc, vc [max_seq][kv_dim]. kv_type ML_F16: halves, rounded as
 * core/ml.c:39-53 does; ML_Q8_0: int8, each KV head's row quantized with one
 * scale (ops/ops.c:81-96) into kd, vd [max_seq][n_kv_heads]. */
void krh_store_kv(int kv_type, void *kc, void *vc, float *kd, float *vd, const float *k, const float *v,
                  int n_kv_heads, int head_dim, const int *pos0, int ntok);

/* ---- batched prompt prefill (model/transformer.c:385-425) ---- */

/* Y[t * ldy + r] (+)= W x_t for the T tokens of xq [T][W->cols] with
 * transposed scales xdT[b * ldx + t] (ml_matmul, ops/ops.c:75-79): int8 MFMA
 * per 32-block, each token's float order the matvec's. ldx is a multiple of
 * 128 and >= T; xq must be readable for ldx rows. */
void krh_matmul(float *Y, int ldy, const krh_mat *W, const int8_t *xq, const float *xdT, int ldx, int T,
                int accumulate);
/* krh_matmul over the scales as an ml_qbatch holds them, token rows
 * xd[t * (W->cols / 32) + b] (ops/ops.c:75-79: ml_matmul's X->d, read in
 * place, no transpose launch); xd is read for T rows only. */
void krh_matmul_rows(float *Y, int ldy, const krh_mat *W, const int8_t *xq, const float *xd, int ldx, int T,
                     int accumulate);
/* The FFN's products and activation of a prompt step in one launch
 * (model/transformer.c:410-413: the w1 and w3 ml_matmul calls, then
 * TOK_DOWN_IN's act_mul and quantize_row_t, :353-355): per
 * token t, h = silu(w1 x_t) * (w3 x_t) (k_scalar.c:96-98), quantized to Q8_0
 * (k_scalar.c:39-57) into hq [T][rows] and the transposed scales hdT
 * [rows / 32][ldx], the layout krh_matmul reads. The same bits as two
 * krh_matmul calls and krh_silu_quant; hq, hdT must not overlap xq, xdT.
 * w1, w3: one shape, type and scale width, rows % 32 == 0. */
void krh_matmul_swiglu(int8_t *hq, float *hdT, const krh_mat *w1, const krh_mat *w3, const int8_t *xq,
                       const float *xdT, int ldx, int T);
/* the three attention projections of T tokens at positions pos0.. with bias
 * and RoPE: q [T][q_dim], k and v into cache rows pos0 + t
 * (model/transformer.c:400-402, :335-344) */
void krh_matmul_qkv(float *q, float *kc, float *vc, const krh_mat *wq, const krh_mat *wk, const krh_mat *wv,
                    const float *bq, const float *bk, const float *bv, const int8_t *xq, const float *xdT, int ldx,
                    int T, const float *rope_cos, const float *rope_sin, int head_dim, int pos0);
/* the same for an F16 or Q8 cache: k and v to the staging rows [T][kv_dim] */
void krh_matmul_qkv_stage(float *q, float *k, float *v, const krh_mat *wq, const krh_mat *wk, const krh_mat *wv,
                          const float *bq, const float *bk, const float *bv, const int8_t *xq, const float *xdT,
                          int ldx, int T, const float *rope_cos, const float *rope_sin, int head_dim, int pos0);
/* causal attention of ntok tokens at positions *pos0 + t (ml_attention_batch,
 * ops/ops.c:216-238): ao, q [ntok][q_dim], att [ntok][n_heads][max_seq];
 * last_pos = *pos0 + ntok - 1 (sizes the launch) */
void krh_attention_batch(float *ao, float *att, const float *q, const float *kc, const float *vc, int n_heads,
                         int n_kv_heads, int head_dim, int max_seq, int window, float scale, const int *pos0, int ntok,
                         int last_pos);
/* The batched attention's choice of kernels (no counterpart in the
 * reference): heads of 64 or 128 dims take the register-blocked score and
 * mix kernels when their rows (token, query head) fill at least min_wg
 * workgroups of 64 rows, and the per-token-block kernels below that
 * (default 512). Tests lower it to run the register-blocked kernels on small
 * shapes; the results are the same bits either way. Process-wide. */
void krh_set_attn_rb_min(int min_wg);
/* h = silu(g) * u per token (k_scalar.c:96-98), quantized to Q8_0 with
 * transposed scales dT[b * ldd + t] */
void krh_silu_quant(int8_t *q, float *dT, int ldd, const float *g, const float *u, int n, int ntok);
/* x[t][0..cols) = row tok[t] of emb, dequantized, for ntok tokens */
void krh_embed_batch(float *x, const krh_mat *emb, const int *tok, int ntok, float embed_scale);

/* Greedy pick (model/sampler.c:57-61, ties to the lowest id): *tok = argmax;
 * then, when non-NULL, log[*pos + 1] = *tok and *pos += 1. */
void krh_argmax(int *tok, const float *logits, int n, int *pos, int *log);

/* tok = prompt[*pos] (the prompt resident on the device) */
void krh_take_token(int *tok, const int *prompt, const int *pos);
/* *pos += 1 */
void krh_advance(int *pos);

/* ---- the families' steps (model/transformer.c:240-248) ----
 * q heads [0, n_heads) and k heads [0, n_kv_heads): each RMS-normalized with
 * q_norm / k_norm when they are non-NULL (Qwen3's heads_norm, :246-248;
 * kernels/scalar/k_scalar.c:59-64), then rotated (k_scalar.c:79-94) by row
 * *pos of the tables (head_dim / 2 floats a row). head_dim even, <= 512. */
void krh_heads_norm_rope(float *q, float *k, const float *q_norm, const float *k_norm, const float *cos_t,
                         const float *sin_t, int head_dim, int n_heads, int n_kv_heads, float eps, const int *pos);
/* F32 cache rows: kc[*pos][i] = k[i], vc[*pos][i] = v[i] for i < kv_dim
 * (the reference's projections write them in place, model/transformer.c:263-264) */
void krh_store_rows_f32(float *kc, float *vc, const float *k, const float *v, int kv_dim, const int *pos);
/* ops/ops.c:141: score rows (token t, head h) of att ([ntok][n_heads][max_seq])
 * become cap * tanhf(score / cap) over the positions attended from *pos + t */
void krh_softcap_att(float *att, int n_heads, int max_seq, int window, const int *pos, int ntok, float cap);
/* krh_attention_kv with soft-capped scores (cap > 0, ops/ops.c:141): Gemma 2 */
void krh_attention_kv_softcap(float *ao, float *att, const float *q, const ml_kv_layer *kv, int n_heads,
                              int n_kv_heads, int head_dim, int max_seq, float scale, const int *pos0, int ntok,
                              int last_pos, float cap);
/* y[i] = tanhf of the float with bits lo + i (the device's C-library tanhf; for checks) */
void krh_tanhf_range(float *y, uint32_t lo, size_t n);

/* ---- the device sampler (model/sampler.h:9-35, model/sampler.c) ----
 * The reference's ml_sample on device logits, with its results: the same id,
 * the same penalized logits and the same generator state after each draw
 * (greedy, multinomial, top-k and top-p draws, the repetition penalty). */
typedef struct {            /* ml_sampler_opts (model/sampler.h:9-16): same fields, same order */
    float temperature;      /* 0 = greedy */
    float topp;             /* 0 or 1 = off */
    int topk;               /* 0 = off */
    float repeat_penalty;   /* 1 = off */
    int repeat_last_n;      /* ids the penalty looks back at */
    uint64_t seed;          /* 0: the reference's fixed constant */
} krh_sampler_opts;
typedef struct krh_sampler krh_sampler;
/* ml_sampler_init (model/sampler.c:6-18): device state for ids below vocab */
ml_status krh_sampler_new(krh_sampler **s, int vocab, const krh_sampler_opts *o);
/* ml_sampler_free (:20-28) */
void krh_sampler_free(krh_sampler *s);
/* ml_sampler_accept (:30-35) for n ids in device memory, in order */
void krh_sampler_accept(krh_sampler *s, const int *tokens, int n);
/* ml_sample (:155-165) on device logits[n], n <= vocab (the penalty writes
 * them, as there), then ml_sampler_accept of the id (app/ml_run.c:391-392):
 * *tok = the id; when pos is non-NULL, log[*pos + 1] = id (log non-NULL) and
 * *pos += 1, as krh_argmax does. Stream-ordered; no host synchronization, so
 * it can be captured into a graph. */
void krh_sample(krh_sampler *s, int *tok, float *logits, int n, int *pos, int *log);
/* the generator state (a synchronous read; for checks) */
uint64_t krh_sampler_rng(const krh_sampler *s);

/* ---- the reference's unfused kernels (the ml_k_<op>_hip op table) ----
 * Each computes the scalar kernel of kernels/scalar/k_scalar.c in its float
 * order, on device pointers. */
void krh_rmsnorm(float *o, const float *x, const float *w, int n, float eps);         /* :59-64, n <= 16384 */
void krh_add(float *y, const float *x, int n);                                          /* :107-109 */
/* Measurement op (no reference counterpart): reads the `bytes` (a multiple of
 * 16) at p once with `grid` workgroups; out[grid] receives an XOR fold of
 * each workgroup's words. Times the plain HBM read rate. */
void krh_stream_read(unsigned *out, const void *p, size_t bytes, int grid);
/* Measurement op (no reference counterpart): grid workgroups of 4 waves,
 * each wave iters x 4 int8 MFMAs of 32x32x32 (65,536 int8 operations each)
 * on register operands; out[4 * grid] receives one word per wave. Times the
 * achievable int8 MFMA rate. */
void krh_mfma_rate(int *out, int grid, int iters);
void krh_rope(float *q, float *k, const float *cos_t, const float *sin_t, int head_dim, int n_heads,
              int n_kv_heads);                                                           /* :79-94 */
void krh_silu_mul(float *g, const float *u, int n);                                     /* :96-98 */
void krh_gelu_mul(float *g, const float *u, int n);        /* :100-105, with the C library's tanhf */
void krh_softmax(float *x, int n);                                                      /* :66-77 */
void krh_dot_rows(float *s, const float *q, const float *k, size_t ldk, int rows, int n, float scale); /* :111-117 */
void krh_axpy_rows(float *y, const float *a, const float *x, size_t ldx, int rows, int n);              /* :119-122 */
void krh_quantize_row(int8_t *q, float *d, const float *x, int n);    /* ops/ops.c:81-96: one scale for the row */
/* The same ops over `rows` rows at once, row r of each pointer argument at
 * p + r * ld_p elements (ld_p = 0: one vector shared by every row); each row
 * gets the single call's bits. The batch form of the per-token loops of
 * model/transformer.c:366-376 (token_task). rows <= KRH_ROWS_MAX. */
enum { KRH_ROWS_MAX = 65535 };
void krh_rmsnorm_rows(float *o, size_t ldo, const float *x, size_t ldx, const float *w, size_t ldw, int n,
                      float eps, int rows);
void krh_add_rows(float *y, size_t ldy, const float *x, size_t ldx, int n, int rows);
void krh_rope_rows(float *q, size_t ldq, float *k, size_t ldk, const float *cos_t, size_t ldc, const float *sin_t,
                   size_t lds, int head_dim, int n_heads, int n_kv_heads, int rows);
void krh_silu_mul_rows(float *g, size_t ldg, const float *u, size_t ldu, int n, int rows);
void krh_gelu_mul_rows(float *g, size_t ldg, const float *u, size_t ldu, int n, int rows);
void krh_quantize_row_rows(int8_t *q, size_t ldq, float *d, size_t ldd, const float *x, size_t ldx, int n, int rows);
/* Q8_0 of rows of n floats (k_scalar.c:39-57): q + r*ldq, scales d + r*ldd,
 * x + r*ldx; x 16-byte and q 4-byte aligned, ldx and ldq multiples of 4 */
void krh_quantize_q8_rows(int8_t *q, size_t ldq, float *d, size_t ldd, const float *x, size_t ldx, int n, int rows);
void krh_softcap_rows(float *x, size_t ld, int rows, int n, float cap);    /* ops/ops.c:98-101, the C library's tanhf */
/* *dst = value, in stream order (positions and token ids of op-table calls) */
void krh_set_int(int *dst, int value);

/* ---- synthetic data ---- */
/* Random quantized matrix [rows][cols] on the device: normals of the host
 * generator's stream `key` (include/krafla.h, kr_gen_mlb) times std,
 * quantized per 32-block by the .mlb writer rules; q: rows*cols (Q8) or
 * rows*cols/2 bytes, d: rows*cols/32 scales, f16 when f16 != 0. */
void krh_gen_blocks(void *q, void *d, uint64_t key, int rows, int cols, int type, int f16, float std);

/* ---- self-checks for tests ---- */
/* y[i] = op(a[i], b[i]) as the kernels compute it: expf(a), sqrtf(a), a / b,
 * rmsnorm's 1 / sqrtf(a / b + 1e-5), or the F16 cache's rounding of a (the
 * binary16 bits in the low 16 bits of y[i]) */
enum { KRH_MATH_EXPF = 0, KRH_MATH_SQRT = 1, KRH_MATH_DIV = 2, KRH_MATH_RMS_INV = 3, KRH_MATH_F2H = 4 };
void krh_math_batch(int op, float *y, const float *a, const float *b, size_t n);
/* y[i] = f16 -> f32 of h[i] */
void krh_h2f_batch(float *y, const uint16_t *h, size_t n);
/* s[r*nb+b]: int32 block dots of rows [0, rows) (the exact integer part of
 * the matvec) */
void krh_block_dots(int32_t *s, const krh_mat *W, const int8_t *xq);
/* *out = ((s0 + t[0]) + t[1]) + ... + t[n-1] in fp32, as the rmsnorm and
 * softmax kernels compute their ordered sums (shifted runs with an exact
 * per-run check and a sequential fallback); n in [1, KRH_ORDERED_SUM_MAX].
 * No counterpart in the reference: a self-check of the kernels' summation. */
enum { KRH_ORDERED_SUM_MAX = 8192 };
void krh_ordered_sum(float *out, const float *t, int n, float s0);
/* The same with fewer reads in flight (256 threads; the prefill softmax's
 * form for rows of 2049-4096 scores), n in [1, KRH_ORDERED_SUM_MAX]. */
void krh_ordered_sum_lean(float *out, const float *t, int n, float s0);
/* The same computed by a workgroup of 1024 threads (the decode softmax's),
 * n in [1, KRH_ORDERED_SUM_MAX]. */
void krh_ordered_sum_1024(float *out, const float *t, int n, float s0);
/* The same computed by one wave alone (the batched softmax's single-wave
 * mode), n in [1, KRH_ORDERED_SUM_WAVE_MAX]. */
enum { KRH_ORDERED_SUM_WAVE_MAX = 4096 };
void krh_ordered_sum_wave(float *out, const float *t, int n, float s0);

#ifdef __cplusplus
}
#endif
#endif
