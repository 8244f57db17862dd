/*
 * Row kernels of the decoder's layer body: the residual add fused with the RMS norm, the MLP's ReLU^2, and the
 * value-embedding mix.
 * Reference: the slot GEMM's RESID epilogue (out = bf16(s + res)) with k_rstd (r = rsqrt(Σ x² / K + FLT_EPSILON)),
 * and the RELU2 epilogue (bf16(relu(p) p)), model/kernels/decode.cu:107-123,169-184,447-456; the model's norm,
 * model/modeling.py:47-49. Here the weight GEMMs are library GEMMs, so these run as their own bandwidth-bound
 * passes: a (row) workgroup loads the row once into registers.
 *
 * add_rms_norm: x_out = bf16(x + delta) (delta NULL: x_out = x), y = bf16(x_out * r), r = 1 / sqrt(Σ x_out² / d +
 * FLT_EPSILON) over the rounded x_out, Σ in fp32 (thread partials, then a fixed wave and workgroup tree).
 *
 * value_embed (a value-embedding layer's v, reference: attn_prologue, model/kernels/decode.cu:476-493;
 * inference/modeling_nanochat.py:85-88): per row, n = bf16(x r) exactly as add_rms_norm (the same sums), per kv head
 * g = 2 sigmoid(Σ_c n_c gate[h][c]) (fp32, a fixed lane order), then v = bf16(v + g ve[token]) in the projection
 * row, in place (fp32 product and sum, one rounding). One workgroup per row: the normed row in LDS, a wave per head.
 */
#include "common.h"

#define RN_THREADS 256
#define RN_MAX_CHUNKS 4 /* 8-element chunks per thread: d <= 8192 */

/* x_out may alias x (in-place residual update): each thread reads and writes only its own chunks. */
__global__ void __launch_bounds__(RN_THREADS) k_add_rms_norm(const bf16_t *x, const bf16_t *__restrict__ delta,
                                                             bf16_t *x_out, bf16_t *__restrict__ y, int d) {
    __shared__ float part[RN_THREADS / NC_WAVE];
    const int row = blockIdx.x, tid = threadIdx.x, chunks = d / 8;
    const size_t base = (size_t)row * d;
    float v[RN_MAX_CHUNKS][8];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < RN_MAX_CHUNKS; k++) {
        const int c = tid + k * RN_THREADS;
        if (c >= chunks) break;
        load_bf16x8(x + base + 8 * c, v[k]);
        if (delta) {
            float dv[8];
            load_bf16x8(delta + base + 8 * c, dv);
#pragma unroll
            for (int e = 0; e < 8; e++) v[k][e] = bf16_to_f32(f32_to_bf16(v[k][e] + dv[e]));
            if (x_out) store_bf16x8(x_out + base + 8 * c, v[k]);
        } else if (x_out && x_out != x) {
            store_bf16x8(x_out + base + 8 * c, v[k]);
        }
#pragma unroll
        for (int e = 0; e < 8; e++) ss += v[k][e] * v[k][e];
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss += shfl_xor_f(ss, m);
    if ((tid & (NC_WAVE - 1)) == 0) part[tid / NC_WAVE] = ss;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < RN_THREADS / NC_WAVE; w++) total += part[w];
    const float r = 1.0f / sqrtf(total / (float)d + 1.1920928955078125e-07f);
#pragma unroll
    for (int k = 0; k < RN_MAX_CHUNKS; k++) {
        const int c = tid + k * RN_THREADS;
        if (c >= chunks) break;
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = v[k][e] * r;
        store_bf16x8(y + base + 8 * c, o);
    }
}

/* x[r] = bf16(e r), e = table[tok[r]] (fp32 or bf16), r = 1 / sqrt(Σ e² / d + FLT_EPSILON), Σ in fp32 in
 * k_add_rms_norm's order; a token outside [0, vocab) gives a zero row. */
template <bool FP32>
__global__ void __launch_bounds__(RN_THREADS) k_embed_norm(const void *table, const int32_t *tok, long long vocab,
                                                           bf16_t *x, int d) {
    __shared__ float part[RN_THREADS / NC_WAVE];
    const int row = blockIdx.x, tid = threadIdx.x, chunks = d / 8;
    const int t = tok[row];
    bf16_t *dst = x + (size_t)row * d;
    if (t < 0 || t >= vocab) {
        for (int c = tid; c < chunks; c += RN_THREADS) reinterpret_cast<u32x4 *>(dst)[c] = u32x4{0u, 0u, 0u, 0u};
        return;
    }
    float v[RN_MAX_CHUNKS][8];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < RN_MAX_CHUNKS; k++) {
        const int c = tid + k * RN_THREADS;
        if (c >= chunks) break;
        if constexpr (FP32) {
            const f32x4 *src = reinterpret_cast<const f32x4 *>((const float *)table + (size_t)t * d + 8 * c);
            const f32x4 a = src[0], b = src[1];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                v[k][e] = a[e];
                v[k][4 + e] = b[e];
            }
        } else {
            load_bf16x8((const bf16_t *)table + (size_t)t * d + 8 * c, v[k]);
        }
#pragma unroll
        for (int e = 0; e < 8; e++) ss += v[k][e] * v[k][e];
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss += shfl_xor_f(ss, m);
    if ((tid & (NC_WAVE - 1)) == 0) part[tid / NC_WAVE] = ss;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < RN_THREADS / NC_WAVE; w++) total += part[w];
    const float r = 1.0f / sqrtf(total / (float)d + 1.1920928955078125e-07f);
#pragma unroll
    for (int k = 0; k < RN_MAX_CHUNKS; k++) {
        const int c = tid + k * RN_THREADS;
        if (c >= chunks) break;
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = v[k][e] * r;
        store_bf16x8(dst + 8 * c, o);
    }
}

/* x = bf16(lr x + l0 x0): the two products and their sum each rounded to fp32, then one bf16 rounding. */
__global__ void __launch_bounds__(RN_THREADS) k_mix(bf16_t *x, const bf16_t *x0, long long n8, float lr, float l0) {
#pragma clang fp contract(off)
    const long long stride = (long long)gridDim.x * RN_THREADS;
    for (long long c = (long long)blockIdx.x * RN_THREADS + threadIdx.x; c < n8; c += stride) {
        float a[8], b[8];
        load_bf16x8(x + 8 * c, a);
        load_bf16x8(x0 + 8 * c, b);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float p = lr * a[e], q = l0 * b[e];
            a[e] = p + q;
        }
        store_bf16x8(x + 8 * c, a);
    }
}

#define VE_MAX_HEADS 64

__global__ void __launch_bounds__(RN_THREADS) k_value_embed(bf16_t *qkv, long long row_stride, const bf16_t *x,
                                                            long long x_stride, const int32_t *tok, const bf16_t *ve,
                                                            long long vocab, const float *gate, int d, int hq,
                                                            int hkv) {
    __shared__ float part[RN_THREADS / NC_WAVE];
    __shared__ float nrow[8 * RN_THREADS * RN_MAX_CHUNKS];
    __shared__ float g[VE_MAX_HEADS];
    const int row = blockIdx.x, tid = threadIdx.x, chunks = d / 8, lane = tid & (NC_WAVE - 1);
    const int t = tok[row];
    if (t < 0 || t >= vocab) return; /* no table row: v stays as projected */
    const bf16_t *xr = x + (size_t)row * x_stride;
    float v[RN_MAX_CHUNKS][8];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < RN_MAX_CHUNKS; k++) {
        const int c = tid + k * RN_THREADS;
        if (c >= chunks) break;
        load_bf16x8(xr + 8 * c, v[k]);
#pragma unroll
        for (int e = 0; e < 8; e++) ss += v[k][e] * v[k][e];
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss += shfl_xor_f(ss, m);
    if (lane == 0) part[tid / NC_WAVE] = ss;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < RN_THREADS / NC_WAVE; w++) total += part[w];
    const float r = 1.0f / sqrtf(total / (float)d + 1.1920928955078125e-07f);
#pragma unroll
    for (int k = 0; k < RN_MAX_CHUNKS; k++) {
        const int c = tid + k * RN_THREADS;
        if (c >= chunks) break;
#pragma unroll
        for (int e = 0; e < 8; e++) nrow[8 * c + e] = bf16_to_f32(f32_to_bf16(v[k][e] * r));
    }
    __syncthreads();
    for (int h = tid / NC_WAVE; h < hkv; h += RN_THREADS / NC_WAVE) {
        const float *gh = gate + (size_t)h * d;
        float dot = 0.f;
        for (int c = lane; c < d; c += NC_WAVE) dot += nrow[c] * gh[c];
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) dot += shfl_xor_f(dot, m);
        if (lane == 0) g[h] = 2.0f / (1.0f + expf(-dot));
    }
    __syncthreads();
    bf16_t *vr = qkv + (size_t)row * row_stride + (size_t)(hq + hkv) * NC_HEAD_DIM;
    const bf16_t *er = ve + (size_t)t * hkv * NC_HEAD_DIM;
    for (int c = tid; c < hkv * NC_HEAD_DIM / 8; c += RN_THREADS) {
#pragma clang fp contract(off)
        float vv[8], ev[8];
        load_bf16x8(vr + 8 * c, vv);
        load_bf16x8(er + 8 * c, ev);
        const float gh = g[(8 * c) / NC_HEAD_DIM];
#pragma unroll
        for (int e = 0; e < 8; e++) vv[e] = vv[e] + gh * ev[e];
        store_bf16x8(vr + 8 * c, vv);
    }
}

__global__ void __launch_bounds__(RN_THREADS) k_relu2(const bf16_t *in, bf16_t *out, /* may be in */
                                                      long long n8) {
    const long long stride = (long long)gridDim.x * RN_THREADS;
    for (long long c = (long long)blockIdx.x * RN_THREADS + threadIdx.x; c < n8; c += stride) {
        float v[8];
        load_bf16x8(in + 8 * c, v);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float p = fmaxf(v[e], 0.f);
            v[e] = p * p;
        }
        store_bf16x8(out + 8 * c, v);
    }
}

extern "C" int nc_add_rms_norm_bf16(const void *x, const void *delta, void *x_out, void *y, int rows, int d,
                                    void *stream) {
    NC_REQUIRE(rows >= 0 && d > 0 && d % 8 == 0 && d <= 8 * RN_THREADS * RN_MAX_CHUNKS,
               "nc_add_rms_norm_bf16: rows %d, d %d (d a multiple of 8, at most %d)", rows, d,
               8 * RN_THREADS * RN_MAX_CHUNKS);
    if (rows == 0) return 0;
    NC_REQUIRE(x && y, "nc_add_rms_norm_bf16: null pointer");
    NC_REQUIRE(((uintptr_t)x | (uintptr_t)delta | (uintptr_t)x_out | (uintptr_t)y) % 16 == 0,
               "nc_add_rms_norm_bf16: 16-byte alignment");
    hipLaunchKernelGGL(k_add_rms_norm, dim3(rows), dim3(RN_THREADS), 0, (hipStream_t)stream, (const bf16_t *)x,
                       (const bf16_t *)delta, (bf16_t *)x_out, (bf16_t *)y, d);
    NC_LAUNCH_CHECK();
    return 0;
}

extern "C" int nc_relu2_bf16(const void *in, void *out, long long n, void *stream) {
    NC_REQUIRE(n >= 0 && n % 8 == 0, "nc_relu2_bf16: n = %lld must be a non-negative multiple of 8", n);
    if (n == 0) return 0;
    NC_REQUIRE(in && out, "nc_relu2_bf16: null pointer");
    NC_REQUIRE(((uintptr_t)in | (uintptr_t)out) % 16 == 0, "nc_relu2_bf16: 16-byte alignment");
    const long long n8 = n / 8;
    long long blocks = (n8 + RN_THREADS - 1) / RN_THREADS;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(k_relu2, dim3((unsigned)blocks), dim3(RN_THREADS), 0, (hipStream_t)stream, (const bf16_t *)in,
                       (bf16_t *)out, n8);
    NC_LAUNCH_CHECK();
    return 0;
}

extern "C" int nc_value_embed_bf16(void *qkv, long long row_stride, const void *x, long long x_stride,
                                   const int32_t *tok, const void *ve, long long vocab, const float *gate, int rows,
                                   int d, int hq, int hkv, void *stream) {
    NC_REQUIRE(rows >= 0 && d > 0 && d % 8 == 0 && d <= 8 * RN_THREADS * RN_MAX_CHUNKS,
               "nc_value_embed_bf16: rows %d, d %d (d a multiple of 8, at most %d)", rows, d,
               8 * RN_THREADS * RN_MAX_CHUNKS);
    NC_REQUIRE(hq > 0 && hkv > 0 && hkv <= VE_MAX_HEADS && hq % hkv == 0,
               "nc_value_embed_bf16: hq %d, hkv %d (hkv <= %d dividing hq)", hq, hkv, VE_MAX_HEADS);
    NC_REQUIRE(row_stride >= (long long)(hq + 2 * hkv) * NC_HEAD_DIM && row_stride % 8 == 0 && x_stride >= d &&
                   x_stride % 8 == 0,
               "nc_value_embed_bf16: row_stride %lld, x_stride %lld", row_stride, x_stride);
    NC_REQUIRE(vocab > 0, "nc_value_embed_bf16: vocab %lld", vocab);
    if (rows == 0) return 0;
    NC_REQUIRE(qkv && x && tok && ve && gate, "nc_value_embed_bf16: null pointer");
    NC_REQUIRE(((uintptr_t)qkv | (uintptr_t)x | (uintptr_t)ve) % 16 == 0, "nc_value_embed_bf16: 16-byte alignment");
    hipLaunchKernelGGL(k_value_embed, dim3(rows), dim3(RN_THREADS), 0, (hipStream_t)stream, (bf16_t *)qkv, row_stride,
                       (const bf16_t *)x, x_stride, tok, (const bf16_t *)ve, vocab, gate, d, hq, hkv);
    NC_LAUNCH_CHECK();
    return 0;
}

extern "C" int nc_embed_rms_norm(const void *table, int table_fp32, long long vocab, const int32_t *tok, int rows,
                                 int d, void *x, void *stream) {
    NC_REQUIRE(rows >= 0 && d > 0 && d % 8 == 0 && d <= 8 * RN_THREADS * RN_MAX_CHUNKS,
               "nc_embed_rms_norm: rows %d, d %d (d a multiple of 8, at most %d)", rows, d,
               8 * RN_THREADS * RN_MAX_CHUNKS);
    NC_REQUIRE(vocab > 0, "nc_embed_rms_norm: vocab %lld", vocab);
    if (rows == 0) return 0;
    NC_REQUIRE(table && tok && x, "nc_embed_rms_norm: null pointer");
    NC_REQUIRE(((uintptr_t)table | (uintptr_t)x) % 16 == 0, "nc_embed_rms_norm: 16-byte alignment");
    if (table_fp32)
        hipLaunchKernelGGL(k_embed_norm<true>, dim3(rows), dim3(RN_THREADS), 0, (hipStream_t)stream, table, tok,
                           vocab, (bf16_t *)x, d);
    else
        hipLaunchKernelGGL(k_embed_norm<false>, dim3(rows), dim3(RN_THREADS), 0, (hipStream_t)stream, table, tok,
                           vocab, (bf16_t *)x, d);
    NC_LAUNCH_CHECK();
    return 0;
}

extern "C" int nc_mix_bf16(void *x, const void *x0, long long n, float lr, float l0, void *stream) {
    NC_REQUIRE(n >= 0 && n % 8 == 0, "nc_mix_bf16: n = %lld must be a non-negative multiple of 8", n);
    if (n == 0) return 0;
    NC_REQUIRE(x && x0, "nc_mix_bf16: null pointer");
    NC_REQUIRE(((uintptr_t)x | (uintptr_t)x0) % 16 == 0, "nc_mix_bf16: 16-byte alignment");
    const long long n8 = n / 8;
    long long blocks = (n8 + RN_THREADS - 1) / RN_THREADS;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(k_mix, dim3((unsigned)blocks), dim3(RN_THREADS), 0, (hipStream_t)stream, (bf16_t *)x,
                       (const bf16_t *)x0, n8, lr, l0);
    NC_LAUNCH_CHECK();
    return 0;
}
