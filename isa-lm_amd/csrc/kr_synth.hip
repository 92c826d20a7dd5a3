// Synthetic quantized matrices generated on the device, for the large
// benchmark models (an 8.5 GB model takes minutes on a few host cores).
//
// The random streams are the host generator's (isa-lm_amd/host/kr_gen.c):
// element i of a matrix is normal i of the stream `key`, drawn as Box-Muller
// pairs in double from splitmix64 of a Weyl sequence, times std, then
// quantized per 32-block by the .mlb writer rules (docs/file-format.md:
// 133-159). The double log/sqrt/sin/cos are kr_normal.h's, evaluated from
// IEEE arithmetic alone, so the device writes the host generator's bytes.
#include "kr_internal.h"
#include "kr_numerics.h"

namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

#define KR_NORMAL_FN static __device__ inline
#include "kr_normal.h"

__device__ __forceinline__ void normal_pair(uint64_t key, uint64_t j, float *a, float *b) {
    krn_pair(mix64(key + (j + 1) * 0x9E3779B97F4A7C15ULL), a, b);
}

// One thread per 32-block: the same float operations as the host writer.
__global__ void __launch_bounds__(256) k_gen_blocks(uint8_t *q, uint8_t *d, uint64_t key, int rows, int cols, int type,
                                                    int f16, float std) {
    const int nb = cols / KR_QK;
    const size_t blk = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= (size_t)rows * nb) return;
    const size_t r = blk / nb, b = blk - r * nb;
    const uint64_t base = (uint64_t)r * cols + (uint64_t)b * KR_QK;
    float x[KR_QK];
    for (int k = 0; k < KR_QK; k += 2) normal_pair(key, (base + k) >> 1, &x[k], &x[k + 1]);
    float amax = 0.0f;
    for (int k = 0; k < KR_QK; k++) {
        x[k] = kr_fmul(x[k], std);
        amax = fmaxf(amax, fabsf(x[k]));
    }
    const float lim = type == ML_Q8_0 ? 127.0f : 7.0f, lo = type == ML_Q8_0 ? -127.0f : -8.0f;
    float dv = amax < KR_QUANT_TINY ? 0.0f : kr_fdiv(amax, lim);
    if (f16) {
        const __half h = __float2half_rn(dv);
        dv = __half2float(h);
        ((uint16_t *)d)[blk] = __half_as_ushort(h);
    } else {
        ((float *)d)[blk] = dv;
    }
    const float id = dv != 0.0f ? (f16 ? kr_fdiv(1.0f, dv) : kr_fdiv(lim, amax)) : 0.0f;
    int v[KR_QK];
    for (int k = 0; k < KR_QK; k++) {
        float t = truncf(kr_fadd(kr_fmul(x[k], id), copysignf(0.5f, x[k])));
        t = fminf(fmaxf(t, lo), lim);
        v[k] = (int)t;
    }
    if (type == ML_Q8_0) {
        uint8_t *o = q + blk * KR_QK;
        for (int k = 0; k < KR_QK; k++) o[k] = (uint8_t)(int8_t)v[k];
    } else {
        uint8_t *o = q + blk * (KR_QK / 2);
        for (int k = 0; k < KR_QK / 2; k++) o[k] = (uint8_t)((v[k] + 8) | ((v[k + KR_QK / 2] + 8) << 4));
    }
}

}  // namespace

extern "C" void krh_gen_blocks(void *q, void *d, uint64_t key, int rows, int cols, int type, int f16, float std) {
    if (rows <= 0 || cols <= 0 || cols % KR_QK || (type != ML_Q8_0 && type != ML_Q4_0)) {
        kr_fail(ML_E_SHAPE, "gen_blocks shape", hipSuccess);
        return;
    }
    const size_t n = (size_t)rows * (cols / KR_QK);
    hipLaunchKernelGGL(k_gen_blocks, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, kr_stream(), (uint8_t *)q,
                       (uint8_t *)d, key, rows, cols, type, f16, std);
    kr_check_launch("gen_blocks");
}
