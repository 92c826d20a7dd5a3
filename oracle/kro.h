/* ORACLE — test infrastructure only. A plain-C restatement of the reference's
 * scalar token loop, used by tests/ as the checker of the HIP path and by
 * bench.py's cpu_baseline leg. Nothing in the product links or calls it.
 *
 * Every function follows the reference's scalar build in float operation
 * order (it is compiled with -ffp-contract=off, as the reference is,
 * Makefile:18-22), so its results are the reference's bit for bit. Each
 * definition cites the reference file:line it restates.
 *
 * Pinning (what checks each part; see tests/test_oracle.py):
 *   kro_expf             exhaustively equal to the host libm expf (all 2^32
 *                        inputs) -- the reference calls glibc's expf
 *   kernels              bit-equal to oracle/_ref/libkrafla_ref_scalar.so on
 *                        seeded inputs, plus the reference's known answers
 *                        (tests/test_quant.c:47-70, tests/test_sampler.c:33-40)
 *                        and closed forms (unit-scale matvec = exact int sum)
 *   kro_forward/prefill  logits bit-equal to oracle/_ref/scalar/ml_run
 *                        --dump-logits on generated .mlb models, with the
 *                        F32, F16 and Q8 KV caches (--kv f32|f16|q8)
 *   kro_tanhf            exhaustively equal to the host libm (all 2^32 inputs;
 *                        expm1f too); gelu_mul and softcap bit-equal to the
 *                        reference's scalar kernels
 *   kro_f32_to_f16       exhaustively equal to the x86 F16C conversion (all
 *                        2^32 inputs; NaN -> sign | 0x7e00) and to the
 *                        reference's ml_f32_to_f16
 *   F16/Q8 KV kernels    bit-equal to the reference's scalar kernels on the
 *                        shapes of tests/test_kernels.c:334-426; unit-scale
 *                        dot_q8 = exact int sum; quantize_row's known answers
 *   kro_sample           the same ids, rng state and penalized logits as the
 *                        reference's ml_sample on seeded logits over every
 *                        option path, plus tests/test_sampler.c's answers
 */
#ifndef KRO_H
#define KRO_H
#include "../include/krafla_types.h"

#ifdef __cplusplus
extern "C" {
#endif

float kro_expf(float x);
/* the C library's tanhf and expm1f (fdlibm's algorithm, glibc 2.35), and
 * the count of inputs in [lo, hi) where either differs from the host libm */
float kro_tanhf(float x);
float kro_expm1f(float x);
uint64_t kro_tanhf_mismatches(uint64_t lo, uint64_t hi, int threads);
/* mismatches of got[i] against the host libm's tanhf of the float with bits lo + i */
uint64_t kro_tanhf_check_range(uint64_t lo, const float *got, size_t n, int threads);
/* k_scalar.c:100-105: g = 0.5 x (1 + tanhf(0.7978845608 (x + 0.044715 x^3))) u */
void kro_gelu_mul(float *g, const float *u, int n);
/* ops/ops.c:98-101: x = cap tanhf(x / cap) over rows of n (stride ld) */
void kro_softcap_rows(float *x, size_t ld, int rows, int n, float cap);
/* counts inputs in [lo, hi) (as uint32 bit patterns) where kro_expf differs
 * from the C library's expf; threads > 1 splits the range */
uint64_t kro_expf_mismatches(uint64_t lo, uint64_t hi, int threads);
/* counts i < n where got[i] differs in bits from expf(x[i]) of the C library */
uint64_t kro_expf_check(const float *x, const float *got, size_t n);

/* the same over got[i] = device expf of the input with bits lo + i */
uint64_t kro_expf_check_range(uint64_t lo, const float *got, size_t n, int threads);

uint16_t kro_f32_to_f16(float f);
void kro_f32_to_f16_range(uint16_t *out, uint32_t lo, size_t n);
/* inputs in [lo, hi) where kro_f32_to_f16 differs from the x86 F16C
 * conversion (NaN: the quiet 0x7e00); UINT64_MAX without F16C */
uint64_t kro_f32_to_f16_mismatches(uint64_t lo, uint64_t hi, int threads);
float kro_f16_to_f32(uint16_t h);

/* kernels: same signatures and semantics as kernels/scalar/k_scalar.h:7-24 */
void kro_matvec_q8(float *y, const ml_qtensor *W, const ml_qact *x, int r0, int r1);
void kro_matvec_q4(float *y, const ml_qtensor *W, const ml_qact *x, int r0, int r1);
void kro_quantize_q8(ml_qact *out, const float *x, int k);
void kro_rmsnorm(float *o, const float *x, const float *w, int n, float eps);
void kro_softmax(float *x, int n);
void kro_rope(float *q, float *k, const float *cos_t, const float *sin_t, int head_dim, int n_heads, int n_kv_heads);
void kro_silu_mul(float *g, const float *u, int n);
void kro_add(float *y, const float *x, int n);
void kro_dot_f32(float *s, const float *q, const float *k, size_t ldk, int rows, int n, float scale);
void kro_axpy_f32(float *y, const float *a, const float *x, size_t ldx, int rows, int n);
void kro_dequant_row(float *out, const ml_qtensor *W, int row);
void kro_quantize_row_q4(int8_t *q, float *d, const float *x, int k);
/* int32 block dot products s[r*nb + b] of rows [r0, r1) (exact) */
void kro_block_dots(int32_t *s, const ml_qtensor *W, const ml_qact *x, int r0, int r1);
int kro_argmax(const float *v, int n);
void kro_quantize_row(int8_t *q, float *d, const float *x, int n);
void kro_dot_f16(float *s, const float *q, const uint16_t *k, size_t ldk, int rows, int n, float scale);
void kro_axpy_f16(float *y, const float *a, const uint16_t *x, size_t ldx, int rows, int n);
void kro_dot_q8(float *s, const int8_t *q, float dq, const int8_t *k, const float *dk, size_t ldk, size_t lddk,
                int rows, int n, float scale);
void kro_axpy_q8(float *y, const float *a, const int8_t *x, const float *dx, size_t ldx, size_t lddx, int rows, int n);
/* attention for one position (ops/ops.c:124-180 order) over the cache kv
 * points at: F32 (k, v), F16 (kh, vh) or Q8 (kq, vq, kd, vd) */
void kro_attention(float *out, const float *q, const ml_kv_layer *kv, float *att, const ml_config *cfg, int pos);

/* whole model */
typedef struct kro_model kro_model;
typedef struct kro_state kro_state;
int kro_model_open(kro_model **m, const char *path);
const ml_config *kro_model_config(const kro_model *m);
void kro_model_close(kro_model *m);
int kro_state_new(kro_state **s, const kro_model *m);
/* the same with the KV cache type of ml_state_init: ML_F32, ML_F16, ML_Q8_0 */
int kro_state_new_kv(kro_state **s, const kro_model *m, int kv_type);
void kro_state_free(kro_state *s);
/* logits of token at pos into out[vocab] (model/transformer.c:257-306) */
int kro_forward(kro_state *s, int token, int pos, float *out);
/* n tokens from pos0; logits [n][vocab] if non-NULL (model/transformer.c:427-438) */
int kro_prefill(kro_state *s, const int *tokens, int n, int pos0, float *logits);
/* greedy loop as ml_run does it (app/ml_run.c:373-404): prompt of np ids,
 * run to `steps` positions; out receives the ids ml_run prints */
int kro_generate(kro_state *s, const int *prompt, int np, int steps, int *out);
/* the residual stream x after the last kro_forward */
const float *kro_state_x(const kro_state *s);
const float *kro_state_kcache(const kro_state *s, int layer);
/* internal buffer by name ("x", "q", "ao", "kcache", "vcache", "rope_cos", "rope_sin") */
const float *kro_state_buffer(const kro_state *s, const char *name);
/* the F16 / Q8 cache arrays by name ("kh", "vh", "kq", "vq", "kd", "vd"), or NULL */
const void *kro_state_cache(const kro_state *s, const char *name);

/* the sampler (model/sampler.h:9-35): options as ml_sampler_opts */
typedef struct {
    float temperature, topp;
    int topk;
    float repeat_penalty;
    int repeat_last_n;
    uint64_t seed;
} kro_sampler_opts;
typedef struct kro_sampler kro_sampler;
int kro_sampler_new(kro_sampler **s, int vocab, const kro_sampler_opts *o);   /* model/sampler.c:6-18 */
void kro_sampler_free(kro_sampler *s);
void kro_sampler_accept(kro_sampler *s, int token);                          /* :30-35 */
int kro_sample(kro_sampler *s, float *logits, int n);                        /* :155-165 */
uint64_t kro_sampler_rng(const kro_sampler *s);
/* ml_run's loop with sampling (app/ml_run.c:361-404) */
int kro_generate_sampled(kro_state *s, kro_sampler *smp, const int *prompt, int np, int steps, int *out);

#ifdef __cplusplus
}
#endif
#endif
