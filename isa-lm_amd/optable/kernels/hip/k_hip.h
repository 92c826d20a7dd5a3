/* ISA=hip kernel set: the reference's kernel ABI (kernels/scalar/k_scalar.h:7-24)
 * implemented on one MI355X (gfx950). Pointers are the caller's: addresses
 * inside a registered range (the state arena, the model file) are translated
 * to their HBM copies; any other buffer is staged to the device and back for
 * the call. Rows outside [r0, r1) are left untouched (docs/kernels.md:45). */
#ifndef ML_K_HIP_H
#define ML_K_HIP_H
#include "core/ml.h"

#define ML_HAS_MATVEC_Q8_HIP 1
#define ML_HAS_MATVEC_Q4_HIP 1
#define ML_HAS_QUANTIZE_Q8_HIP 1
#define ML_HAS_RMSNORM_HIP 1
#define ML_HAS_SOFTMAX_HIP 1
#define ML_HAS_ROPE_HIP 1
#define ML_HAS_SILU_MUL_HIP 1
#define ML_HAS_GELU_MUL_HIP 1
#define ML_HAS_ADD_HIP 1
#define ML_HAS_DOT_F32_HIP 1
#define ML_HAS_AXPY_F32_HIP 1

void ml_k_matvec_q8_hip(float *y, const ml_qtensor *W, const ml_qact *x, int r0, int r1);
void ml_k_matvec_q4_hip(float *y, const ml_qtensor *W, const ml_qact *x, int r0, int r1);
void ml_k_quantize_q8_hip(ml_qact *out, const float *x, int k);
void ml_k_rmsnorm_hip(float *o, const float *x, const float *w, int n, float eps);
void ml_k_softmax_hip(float *x, int n);
void ml_k_rope_hip(float *q, float *k, const float *cos_t, const float *sin_t, int head_dim, int n_heads,
                   int n_kv_heads);
void ml_k_silu_mul_hip(float *g, const float *u, int n);
void ml_k_gelu_mul_hip(float *g, const float *u, int n);
void ml_k_add_hip(float *y, const float *x, int n);
void ml_k_dot_f32_hip(float *s, const float *q, const float *k, size_t ldk, int rows, int n, float scale);
void ml_k_axpy_f32_hip(float *y, const float *a, const float *x, size_t ldx, int rows, int n);

/* the backend's status: ML_OK, or the first device or shape error, with a
 * message (ops return void, as the reference's kernels do) */
ml_status ml_hip_status(void);
const char *ml_hip_last_error(void);

#endif
