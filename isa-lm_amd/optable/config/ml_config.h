/* Compile-time kernel binding for ISA=hip: every ml_k_<op> the model and
 * ops code call resolves to the MI355X kernel set (kernels/hip/k_hip.h). The
 * per-row F16/Q8 dot and axpy kernels stay scalar: the reference calls them
 * only from its own attention loop (ops/ops.c), which this backend replaces
 * with device attention over the F32 or Q8 cache (ml_attention in ml_hip.c).
 * The hip counterpart of the reference's config/ml_config.h:41-417. */
#ifndef ML_CONFIG_H
#define ML_CONFIG_H

#include "kernels/scalar/k_scalar.h"
#include "kernels/hip/k_hip.h"

#define ml_k_matvec_q8 ml_k_matvec_q8_hip
#define ml_k_matvec_q4 ml_k_matvec_q4_hip
#define ml_k_quantize_q8 ml_k_quantize_q8_hip
#define ml_k_rmsnorm ml_k_rmsnorm_hip
#define ml_k_softmax ml_k_softmax_hip
#define ml_k_rope ml_k_rope_hip
#define ml_k_silu_mul ml_k_silu_mul_hip
#define ml_k_gelu_mul ml_k_gelu_mul_hip
#define ml_k_add ml_k_add_hip
#define ml_k_dot_f32 ml_k_dot_f32_hip
#define ml_k_axpy_f32 ml_k_axpy_f32_hip
#define ml_k_dot_f16 ml_k_dot_f16_scalar
#define ml_k_axpy_f16 ml_k_axpy_f16_scalar
#define ml_k_dot_q8 ml_k_dot_q8_scalar
#define ml_k_axpy_q8 ml_k_axpy_q8_scalar

/* no CPU row-interleaved layout: the weights stay in the file's layout in HBM */
#define ML_PACK_G 0
#define ML_PACK_Q8_OFFSET 0
#define ML_PACK_Q8 0
#define ML_PACK_Q4_XOR 0
#define ML_PACK_D16 0

#define ML_ISA_NAME "hip"

#define ML_STR_(x) #x
#define ML_STR(x) ML_STR_(x)

#endif
