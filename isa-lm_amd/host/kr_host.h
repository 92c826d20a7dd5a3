/* Internal declarations of the C host library. */
#ifndef KR_HOST_H
#define KR_HOST_H
#include "../../include/krafla.h"
#include "../../include/krafla_hip.h"

struct kr_model {
    ml_config cfg;
    void *map;
    size_t size;
    int shared;
    ml_qtensor tok_emb, wcls;
    const float *final_norm;
    ml_layer *layers;
    /* device copies (kr_model_upload) */
    void *dev;
    size_t dev_bytes;
    krh_mat d_tok_emb, d_wcls;
    const float *d_final_norm;
    struct kr_dev_layer *d_layers;
};

struct kr_dev_layer {
    const float *attn_norm, *ffn_norm, *bq, *bk, *bv;
    const float *q_norm, *k_norm, *post_attn_norm, *post_ffn_norm;   /* NULL unless the model has them */
    krh_mat wq, wk, wv, wo, w1, w2, w3;
};

/* internal to libkrafla.so (not exported) */
#define KR_INTERNAL __attribute__((visibility("hidden")))
KR_INTERNAL ml_status kr_seterr(ml_status s, const char *fmt, ...);
KR_INTERNAL ml_status kr_parse_header(ml_config *cfg, int *shared, const uint8_t *h);
KR_INTERNAL double kr_now(void);

#endif
