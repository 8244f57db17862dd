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
    t = t + xor8_f<4>(t);
    t = t + xor8_f<2>(t);
    t = t + xor8_f<1>(t);
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
 * c1 = dims [8g, 8g+8), c2 = dims [64+8g, 64+8g+8), byte e = dim 8g+e. A zero row gives scale 0 and codes 0.
 * Each code is the e4m3fn rounding (nearest, ties to even) of the correctly rounded quotient x / scale. */
__device__ __forceinline__ float row_quantize_exact(const float *x1, const float *x2, uint64_t *c1, uint64_t *c2) {
#pragma clang fp contract(off)
    float a = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) a = fmaxf(a, fmaxf(fabsf(x1[e]), fabsf(x2[e])));
    a = fmaxf(a, xor8_f<4>(a));
    a = fmaxf(a, xor8_f<2>(a));
    a = fmaxf(a, xor8_f<1>(a));
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

/* x / scale for |x| <= 448 scale, scale a normal number: r = 1 / scale correctly rounded, q0 = x r, and one FMA
 * correction q0 + (x - q0 scale) r, which is the correctly rounded quotient (Markstein's theorem: r within half an
 * ulp of 1 / scale, q0 within an ulp of the quotient, the residual exact by FMA); the sign restores -0 / scale. */
__device__ __forceinline__ float quotient(float x, float scale, float r) {
#pragma clang fp contract(off)
    const float q0 = x * r;
    return __builtin_copysignf(fmaf(fmaf(-q0, scale, x), r, q0), x);
}

/* Four codes of the hardware e4m3fn conversion, which rounds like f32_to_e4m3 for every non-NaN input. */
__device__ __forceinline__ uint32_t e4m3x4(float q0, float q1, float q2, float q3) {
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q2, q3, __builtin_amdgcn_cvt_pk_fp8_f32(q0, q1, 0, false), true);
}

/* row_quantize_exact's results with one division per lane instead of 16 and hardware conversions: for a row of
 * finite values whose scale is a normal number every quotient is x / scale bit for bit and finite (so the
 * conversion never sees a NaN); other rows (a NaN or infinity, a subnormal scale) take row_quantize_exact. The
 * row's max |x| is the integer maximum of the magnitudes' bit patterns, which orders finite floats. */
__device__ __forceinline__ float row_quantize(const float *x1, const float *x2, uint64_t *c1, uint64_t *c2) {
#pragma clang fp contract(off)
    uint32_t m = 0;
#pragma unroll
    for (int e = 0; e < 8; e++)
        m = max(m, max(__float_as_uint(x1[e]) & 0x7fffffffu, __float_as_uint(x2[e]) & 0x7fffffffu));
    m = max(m, xor8_u32<4>(m));
    m = max(m, xor8_u32<2>(m));
    m = max(m, xor8_u32<1>(m));
    const float scale = __uint_as_float(m) / NC_FP8_MAX; /* not used when m is not finite */
    if (m >= 0x7f800000u || scale < 0x1p-126f) return row_quantize_exact(x1, x2, c1, c2);
    const float r = 1.0f / scale;
    float q1[8], q2[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        q1[e] = quotient(x1[e], scale, r);
        q2[e] = quotient(x2[e], scale, r);
    }
    *c1 = e4m3x4(q1[0], q1[1], q1[2], q1[3]) | (uint64_t)e4m3x4(q1[4], q1[5], q1[6], q1[7]) << 32;
    *c2 = e4m3x4(q2[0], q2[1], q2[2], q2[3]) | (uint64_t)e4m3x4(q2[4], q2[5], q2[6], q2[7]) << 32;
    return scale;
}
