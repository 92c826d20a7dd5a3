/* Krafla ABI types, restated so that the hip op table is link-compatible with
 * the reference's callers. Layouts, names and enum values must match the
 * reference field for field:
 *   ml_status, QK, ML_ALIGN, ML_QUANT_TINY, tensor types  core/ml.h:7-22, :67
 *   ml_qtensor, ml_qact, ml_qbatch                         core/ml.h:69-97
 *   ml_config and its enums                                model/mlb.h:9-40
 *   ml_layer, ml_model (pointer members only, see below)   model/mlb.h:42-62
 *   ml_kv_layer                                            ops/ops.h:13-22
 */
#ifndef KRAFLA_TYPES_H
#define KRAFLA_TYPES_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    ML_OK = 0,
    ML_E_IO,
    ML_E_FORMAT,
    ML_E_SHAPE,
    ML_E_NOMEM,
    ML_E_ISA
} ml_status;

#ifndef QK
#define QK 32               /* quantization block size */
#endif
#define ML_ALIGN 64         /* alignment of every tensor array */
#define ML_QUANT_TINY 1e-30f /* blocks with max |x| below this quantize to zero */

enum { ML_F32 = 0, ML_Q8_0 = 1, ML_Q4_0 = 2, ML_F16 = 3 };

/* Quantized weight matrix: q[rows*cols] int8 (Q4: rows*cols/2 bytes, byte j
 * of a block = elements j and j+16), d[rows*cols/QK] f32 scales. */
typedef struct {
    const int8_t *q;
    const float *d;
    int rows, cols;
    uint8_t type;
    const uint8_t *pq;
    const float *pd;
    const uint16_t *dh;
    uint8_t pd16;
} ml_qtensor;

/* Q8_0 activation vector of length n. */
typedef struct {
    int8_t *q;
    float *d;
    int n;
} ml_qact;

/* n Q8_0 activation vectors of length k: token t is q + t*k, d + t*(k/QK). */
typedef struct {
    int8_t *q;
    float *d;
    int n, k;
} ml_qbatch;

typedef struct {
    int dim, n_layers, n_heads, n_kv_heads, hidden_dim, vocab, max_seq, head_dim, kv_dim;
    int q_dim;
    float rope_theta, norm_eps;
    int wtype;
    unsigned q8_mask;
    int qkv_bias;
    int qk_norm;
    int sliding_window;
    int layer_flags;
    float rope_local_theta;
    int act;
    int post_norms;
    float embed_scale;
    float attn_scale;
    int scale_f16;
    float attn_softcap;
    float final_softcap;
    int rope_type, rope_orig_max_seq;
    float rope_factor, rope_low_freq_factor, rope_high_freq_factor;
    float rope_attn_factor;
} ml_config;

enum { ML_ROPE_NONE = 0, ML_ROPE_LLAMA3 = 1, ML_ROPE_LINEAR = 2, ML_ROPE_YARN = 3 };
enum { ML_LAYER_SLIDING = 1, ML_LAYER_LOCAL_ROPE = 2, ML_LAYER_ALL = 3 };
enum { ML_ACT_SILU = 0, ML_ACT_GELU_TANH = 1 };
enum { ML_Q8M_EMB = 1, ML_Q8M_CLS = 2, ML_Q8M_QK = 4, ML_Q8M_V = 8, ML_Q8M_O = 16,
       ML_Q8M_UP = 32, ML_Q8M_DOWN = 64, ML_Q8M_ALL = 127 };

typedef struct {
    const float *attn_norm, *ffn_norm;
    ml_qtensor wq, wk, wv, wo, w1, w2, w3;
    const float *bq, *bk, *bv;
    const float *q_norm, *k_norm;
    const float *post_attn_norm, *post_ffn_norm;
    int window;
    int local_rope;
} ml_layer;

/* One layer of the KV cache, rows [max_seq][kv_dim]: F32 when k is set. */
typedef struct {
    const float *k, *v;
    const int8_t *kq, *vq;
    const float *kd, *vd;
    int window;
    const uint16_t *kh, *vh;
} ml_kv_layer;

#ifdef __cplusplus
}
#endif
#endif
