/*
 * Row math of the q/k prologue: RMS QK-norm with a per-dim gain, then RoPE as a rotation by -θ of the pairs
 * (i, i + 64) (model/kernels/qk_row.cuh:25-41; inference/modeling_nanochat.py:37-45).
 *
 * A row (one head of one token, 128 dims) is 8 consecutive lanes of a wave. Lane g = lane % 8 holds dims
 * [8g, 8g + 8) in x1 and their rotation partners [64 + 8g, 64 + 8g + 8) in x2, one 16-byte load each.
 *
 * Rounding rule (bit-exact with the CPU oracle): every product and sum is one fp32 rounding, nothing contracted;
 * Σx² is the fixed tree (i, i+64), then within the lane (e, e+4), (e, e+2), (e, e+1), then across lanes xor 4, 2,
 * 1; r = 1 / sqrt(Σx²/128 + FLT_EPSILON) with correctly rounded sqrt and division; n = (x r) g;
 * y1 = n1 c + n2 s, y2 = n2 c - n1 s. The reference's CUDA path uses rsqrtf and a different lane tree instead
 * (qk_row.cuh:25-30): this is the build's documented rule, not a copy of that one.
 */
#pragma once

#include "common.h"

#define NC_ROW_LANES 8

/* 1 / sqrt(mean(x²) + FLT_EPSILON) of this lane's row, in the fixed tree. */
__device__ __forceinline__ float row_rstd(const float *x1, const float *x2) {
#pragma clang fp contract(off)
    float s[8];
#pragma unroll
    for (int e = 0; e < 8; e++) s[e] = x1[e] * x1[e] + x2[e] * x2[e];
#pragma unroll
    for (int e = 0; e < 4; e++) s[e] = s[e] + s[e + 4];
    s[0] = s[0] + s[2];
    s[1] = s[1] + s[3];
    float t = s[0] + s[1];
    t = t + shfl_xor_f(t, 4);
    t = t + shfl_xor_f(t, 2);
    t = t + shfl_xor_f(t, 1);
    return 1.0f / sqrtf(t / 128.0f + 1.1920928955078125e-07f);
}

/* x1, x2 <- bf16-valued rows after norm, gain and rotation (fp32 holding the rounded bf16 values). */
__device__ __forceinline__ void row_norm_rope(float *x1, float *x2, const float *g1, const float *g2, const float *c,
                                              const float *s) {
#pragma clang fp contract(off)
    const float r = row_rstd(x1, x2);
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float n1 = (x1[e] * r) * g1[e];
        const float n2 = (x2[e] * r) * g2[e];
        const float y1 = n1 * c[e] + n2 * s[e];
        const float y2 = n2 * c[e] - n1 * s[e];
        x1[e] = bf16_to_f32(f32_to_bf16(y1));
        x2[e] = bf16_to_f32(f32_to_bf16(y2));
    }
}

/* Per-(token, kv head) absmax quantisation of this lane's 16 values of the row: returns the row's scale
 * (max|x| / 448, one correctly rounded division) and writes the lane's e4m3fn codes, 8 per 64-bit word:
 * c1 = dims [8g, 8g+8), c2 = dims [64+8g, 64+8g+8), byte e = dim 8g+e. A zero row gives scale 0 and codes 0. */
__device__ __forceinline__ float row_quantize(const float *x1, const float *x2, uint64_t *c1, uint64_t *c2) {
#pragma clang fp contract(off)
    float a = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) a = fmaxf(a, fmaxf(fabsf(x1[e]), fabsf(x2[e])));
    a = fmaxf(a, shfl_xor_f(a, 4));
    a = fmaxf(a, shfl_xor_f(a, 2));
    a = fmaxf(a, shfl_xor_f(a, 1));
    const float scale = a / NC_FP8_MAX;
    uint64_t w1 = 0, w2 = 0;
    if (scale != 0.0f) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            w1 |= (uint64_t)f32_to_e4m3(x1[e] / scale) << (8 * e);
            w2 |= (uint64_t)f32_to_e4m3(x2[e] / scale) << (8 * e);
        }
    }
    *c1 = w1;
    *c2 = w2;
    return scale;
}
