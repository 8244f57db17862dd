/*
 * Shared by every kernel file of the MI355X (gfx950) fp8-KV decode path: types, the HIP error policy, bf16 and
 * OCP e4m3fn rounding, 16-byte vector access and wave64 lane exchanges.
 *
 * Precision rules: code that must match the CPU oracle bit for bit (the append's row math and quantisation) lives
 * in functions that open with `#pragma clang fp contract(off)`, so no a*b+c is fused; `/` and `sqrtf` are
 * correctly rounded (hipcc's default -fhip-fp32-correctly-rounded-divide-sqrt). Attention code may contract.
 */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#define NC_WAVE 64
#define NC_HEAD_DIM 128
#define NC_HALF 64

typedef uint16_t bf16_t; /* bf16 storage: the high half of an fp32 */

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

/* A failed HIP runtime call aborts with its file and line: a launch that did not happen must never look like a
 * result (the reference's policy, model/kernels/decode.cu:47-53). Argument errors are returned, not aborted. */
#define NC_HIP_CHECK(call) nc_hip_check((call), #call, __FILE__, __LINE__)
static inline void nc_hip_check(hipError_t e, const char *call, const char *file, int line) {
    if (e == hipSuccess) return;
    fprintf(stderr, "%s:%d: %s: %s\n", file, line, call, hipGetErrorString(e));
    abort();
}

/* After a kernel launch: a launch error (bad configuration, no device) aborts like a failed call. */
#define NC_LAUNCH_CHECK() NC_HIP_CHECK(hipGetLastError())

/* Host-side argument errors: the message of the last failed entry point (per thread), status < 0. */
int nc_fail(const char *fmt, ...);
#define NC_REQUIRE(cond, ...) \
    do {                      \
        if (!(cond)) return nc_fail(__VA_ARGS__); \
    } while (0)

/* ------------------------------------------------------------------------------------------ bf16 */

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

/* fp32 -> bf16 by gfx950's v_cvt_pk_bf16_f32: round to nearest even, a NaN's upper 16 bits kept with the quiet bit
 * set. On this GPU it equals the integer rule ((u + 0x7fff + bit 16 of u) >> 16; a NaN gives (u >> 16) | 0x40) for
 * all 2^32 inputs, in both halves and with or without IEEE mode (tests/test_gpu_bf16_rounding.py). */
typedef float nc_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 nc_bf16x2 __attribute__((ext_vector_type(2)));

/* Two fp32 as packed bf16 bits: lo in bits 0-15, hi in bits 16-31 (one instruction). */
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(nc_f32x2{lo, hi}, nc_bf16x2));
}

__device__ __forceinline__ uint32_t f32_to_bf16(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }

/* 8 bf16 (one 16-byte load) as fp32. */
__device__ __forceinline__ void load_bf16x8(const bf16_t *p, float *v) {
    const u32x4 u = *reinterpret_cast<const u32x4 *>(p);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[2 * i] = __uint_as_float(u[i] << 16);
        v[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    }
}

/* 8 fp32 rounded to bf16, one 16-byte store. */
__device__ __forceinline__ void store_bf16x8(bf16_t *p, const float *v) {
    u32x4 u;
#pragma unroll
    for (int i = 0; i < 4; i++) u[i] = f32x2_to_bf16x2(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<u32x4 *>(p) = u;
}

/* ------------------------------------------------------------------------------------------ OCP e4m3fn */

#define NC_FP8_MAX 448.0f

/* fp32 -> e4m3fn code, round to nearest even, no saturation (|x| > 464, inf, NaN give 0x7f | sign): the same
 * function as torch's float32 -> float8_e4m3fn cast. Normal results re-bias the exponent (127 -> 7) and round the
 * mantissa to 3 bits in integer arithmetic; subnormal results count 2^-9 steps with v_rndne. */
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
#pragma clang fp contract(off)
    const uint32_t u = __float_as_uint(x);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7fffffffu;
    uint32_t code;
    if (a >= 0x7f800000u) {
        code = 0x7fu;
    } else if (a >= 0x3c800000u) { /* >= 2^-6 */
        const uint32_t v = a - (120u << 23);
        code = (v + 0x7ffffu + ((v >> 20) & 1u)) >> 20;
        if (code > 0x7eu) code = 0x7fu;
    } else {
        code = (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);
    }
    return code | sign;
}

/* ------------------------------------------------------------------------------------------ lane exchanges */

__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, NC_WAVE); }

/* v of lane (lane ^ MASK), MASK 1, 2 or 4: exchanges inside 8-lane rows as DPP moves (VALU latency, no LDS
 * round trip): quad_perm [1,0,3,2] and [2,3,0,1]; for 4, row_shl:4 (lane + 4) where lane bit 2 is clear and
 * row_shr:4 (lane - 4) where it is set, both inside the lane's 16-lane DPP row. */
template <int MASK> __device__ __forceinline__ uint32_t xor8_u32(uint32_t v) {
    static_assert(MASK == 1 || MASK == 2 || MASK == 4, "exchanges inside 8-lane rows");
    const int i = (int)v;
    if constexpr (MASK == 1) {
        return (uint32_t)__builtin_amdgcn_mov_dpp(i, 0xB1, 0xf, 0xf, false);
    } else if constexpr (MASK == 2) {
        return (uint32_t)__builtin_amdgcn_mov_dpp(i, 0x4E, 0xf, 0xf, false);
    } else {
        const int up = __builtin_amdgcn_mov_dpp(i, 0x104, 0xf, 0xf, false);
        const int dn = __builtin_amdgcn_mov_dpp(i, 0x114, 0xf, 0xf, false);
        return (uint32_t)((__lane_id() & 4) ? dn : up);
    }
}
template <int MASK> __device__ __forceinline__ float xor8_f(float v) {
    return __uint_as_float(xor8_u32<MASK>(__float_as_uint(v)));
}
