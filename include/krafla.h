/* libkrafla.so: the C host of the MI355X token loop.
 *
 * Loads .mlb models (the reference's format, docs/file-format.md), uploads
 * them once to HBM, and runs Krafla's token loop -- ml_forward, ml_prefill
 * and ml_run's greedy loop (model/transformer.c:257-306, :427-438,
 * app/ml_run.c:369-404) -- as fused HIP kernels through libkrafla_hip.so,
 * with each decode step replayed from a captured graph. Results are the
 * reference scalar build's, bit for bit.
 */
#ifndef KRAFLA_H
#define KRAFLA_H
#include "krafla_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

const char *kr_status_str(ml_status s);   /* core/ml.c:21-33 */
const char *kr_error(void);               /* detail of the last failure */

/* ---- .mlb model ---- */
typedef struct kr_model kr_model;
/* Maps and validates an .mlb file with the reference loader's rules and
 * status codes (model/mlb.c:80-218). */
ml_status kr_model_load(kr_model **m, const char *path);
const ml_config *kr_model_config(const kr_model *m);
/* host views of the tensors (NULL for a layer out of range) */
const ml_layer *kr_model_layer(const kr_model *m, int l);
const ml_qtensor *kr_model_tok_emb(const kr_model *m);
const ml_qtensor *kr_model_wcls(const kr_model *m);
/* Copies every tensor to HBM once (the hip counterpart of ml_model_pack,
 * model/pack_model.h:10). ML_E_NOMEM if HBM is short. */
ml_status kr_model_upload(kr_model *m);
size_t kr_model_device_bytes(const kr_model *m);
/* the device copy of a matrix ("tok_emb", "wcls", or a layer's "wq", "wk",
 * "wv", "wo", "w1", "w2", "w3") or vector ("final_norm", a layer's
 * "attn_norm", "ffn_norm", "bq", "bk", "bv"); NULL before upload */
const krh_mat *kr_model_device_mat(const kr_model *m, int layer, const char *name);
const float *kr_model_device_vec(const kr_model *m, int layer, const char *name);
void kr_model_free(kr_model *m);

/* ---- decoding state (KV cache and activations in HBM) ---- */
typedef struct kr_state kr_state;
/* kv_type: ML_F32, ML_F16 or ML_Q8_0 (ml_state_init, model/transformer.c:51-56);
 * ML_E_SHAPE for any other type, ML_E_NOMEM when HBM runs out. Every model
 * the loader accepts runs: models with q/k-norm, post-norms, GELU or
 * soft-capping take the unfused layer path. */
ml_status kr_state_new(kr_state **s, kr_model *m, int kv_type);
void kr_state_free(kr_state *s);
/* ml_forward: logits of token at pos into logits[vocab] (host memory) */
ml_status kr_forward(kr_state *s, int token, int pos, float *logits);
/* ml_prefill: n tokens from pos0 into the cache; logits [n][vocab] if non-NULL */
ml_status kr_prefill(kr_state *s, const int *tokens, int n, int pos0, float *logits);
/* ml_run's loop (no --eos): prompt of np ids, `steps` positions; out
 * receives the ids ml_run prints (returns their count, or -1). Greedy (-T 0),
 * or drawn by the sampler of kr_state_set_sampler, which accepts the prompt's
 * ids first and each drawn id after its draw (app/ml_run.c:361-392). Times of
 * the prefill and of the decode loop in seconds, if non-NULL. */
int kr_generate(kr_state *s, const int *prompt, int np, int steps, int *out, double *prefill_s, double *decode_s);
/* device address of the residual stream x (dim floats), for tests */
const float *kr_state_x_device(const kr_state *s);
/* device address of an internal buffer by name ("x", "q", "ao", "hb", "att",
 * "logits", "kcache", "vcache", "rope_cos", "rope_sin", "qa_dim", "qd_dim",
 * "qa_q", "qd_q", "qa_hid", "qd_hid", "kd", "vd"), or NULL; for tests. The
 * caches hold floats, halves or int8 by kv_type; kd, vd are the Q8 cache's
 * row scales [n_layers][max_seq][n_kv_heads]. */
const void *kr_state_buffer(const kr_state *s, const char *name);
/* tokens per batched prefill step (ml_state.batch, model/transformer.h:37):
 * 1 = token by token (replays of the decode step), 0 = the default (2048,
 * at most max_seq) */
void kr_state_set_batch(kr_state *s, int batch);
/* the sampler kr_generate draws with (ml_run's -T, -p, --top-k,
 * --repeat-penalty, --repeat-last-n, -s; model/sampler.h:9-16): a new device
 * sampler, its generator seeded and no ids seen; NULL: greedy (the default) */
ml_status kr_state_set_sampler(kr_state *s, const krh_sampler_opts *o);

/* ---- seeded synthetic models ---- */
typedef struct {
    int dim, n_layers, n_heads, n_kv_heads, hidden_dim, vocab, max_seq;
    float rope_theta, norm_eps;
    int wtype;             /* ML_Q8_0 or ML_Q4_0 */
    unsigned q8_mask;      /* Q4 models: ML_Q8M_* classes stored in Q8 */
    int shared;            /* tied classifier */
    int qkv_bias;
    int scale_f16;
    int rope_type;         /* ML_ROPE_NONE or ML_ROPE_LLAMA3 */
    float rope_factor, rope_low_freq_factor, rope_high_freq_factor;
    int rope_orig_max_seq;
    float std;             /* weight and embedding std (0.02) */
    uint64_t seed;
    int threads;
    int device;            /* draw the matrices on the GPU (krh_gen_blocks) */
    int qk_norm;           /* per-head q/k RMSNorm weights (Qwen3) */
    int post_norms;        /* post-attention and post-FFN RMSNorm weights (Gemma 3) */
    int sliding_window;    /* positions a windowed layer attends to; 0: all */
    unsigned layer_sliding, layer_local;   /* per-layer flags (bit l: layer l, at most 32 layers): the
                                            * window applies; RoPE of rope_local_theta. Both 0: no
                                            * flags, the window (if any) in every layer */
    float rope_local_theta;
    float rope_attn_factor; /* yarn (rope_type ML_ROPE_YARN) */
    int act;               /* ML_ACT_SILU or ML_ACT_GELU_TANH */
    float embed_scale;     /* 0: 1 */
    float attn_softcap, final_softcap;   /* 0: off */
} kr_gen_spec;
/* Writes an .mlb: matrices and embedding N(0, std^2), norms 1 + 0.01 N,
 * biases 0.02 N, quantized by the format's rules (docs/file-format.md:133-159). */
ml_status kr_gen_mlb(const char *path, const kr_gen_spec *spec);
/* A matrix for the matvec microbench: Q4 nibbles uniform in [0, 15] with
 * f16 scales |N(0, 0.01)|; Q8 quants uniform in [-127, 127] with the same
 * scales. q: rows*cols (Q8) or rows*cols/2 bytes; d: rows*cols/32 f16. */
void kr_gen_matrix(void *q, uint16_t *d, int rows, int cols, int type, uint64_t seed, int threads);
/* n floats N(0, 1) */
void kr_gen_normal(float *x, size_t n, uint64_t seed);

#ifdef __cplusplus
}
#endif
#endif
