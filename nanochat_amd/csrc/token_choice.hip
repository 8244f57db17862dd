/*
 * Greedy token choice: per row, the column of the largest fp32 logit, the lowest column among exact ties
 * (reference: the packed-key argmax of the slot GEMM's EPI_ARGMAX epilogue, model/kernels/decode.cu:90-96,189-230).
 *
 * The key of a (score, column) pair is the score's IEEE bits mapped to an unsigned order (negatives inverted,
 * positives above them) in the high word and ~column in the low word, so one unsigned 64-bit max gives the largest
 * score and, on a tie, the lowest column. One 256-thread workgroup per row: 16-byte loads, a per-thread max, a
 * wave max by xor shuffles, then the four waves through LDS. HBM-bound: 4 B per logit.
 */
#include "common.h"

#define TC_THREADS 256

__device__ __forceinline__ unsigned long long choice_key(float score, uint32_t col) {
    const uint32_t bits = __float_as_uint(score);
    const uint32_t ordered = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
    return ((unsigned long long)ordered << 32) | (0xffffffffu - col);
}

__device__ __forceinline__ unsigned long long max_u64(unsigned long long a, unsigned long long b) { return a > b ? a : b; }

__global__ void __launch_bounds__(TC_THREADS) k_argmax(const float *__restrict__ logits, int cols, long long ld,
                                                       int32_t *__restrict__ out) {
    __shared__ unsigned long long part[TC_THREADS / NC_WAVE];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float *x = logits + (size_t)row * ld;
    unsigned long long best = 0;
    const int vec = (cols / 4) * 4;
    if ((((uintptr_t)x) & 15) == 0) {
        for (int c = 4 * tid; c < vec; c += 4 * TC_THREADS) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(x + c);
#pragma unroll
            for (int e = 0; e < 4; e++) best = max_u64(best, choice_key(v[e], c + e));
        }
    } else {
        for (int c = tid; c < vec; c += TC_THREADS) best = max_u64(best, choice_key(x[c], c));
    }
    for (int c = vec + tid; c < cols; c += TC_THREADS) best = max_u64(best, choice_key(x[c], c));
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const unsigned long long o = ((unsigned long long)__shfl_xor((unsigned)(best >> 32), d, NC_WAVE) << 32) |
                                     __shfl_xor((unsigned)best, d, NC_WAVE);
        best = max_u64(best, o);
    }
    if ((tid & (NC_WAVE - 1)) == 0) part[tid / NC_WAVE] = best;
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < TC_THREADS / NC_WAVE; w++) best = max_u64(best, part[w]);
        out[row] = (int32_t)(0xffffffffu - (uint32_t)best);
    }
}

extern "C" int nc_argmax_f32(const float *logits, int rows, int cols, long long ld, int32_t *out, void *stream) {
    NC_REQUIRE(rows >= 0 && cols > 0 && ld >= cols, "nc_argmax_f32: rows %d, cols %d, ld %lld", rows, cols, ld);
    if (rows == 0) return 0;
    NC_REQUIRE(logits && out, "nc_argmax_f32: null pointer");
    hipLaunchKernelGGL(k_argmax, dim3(rows), dim3(TC_THREADS), 0, (hipStream_t)stream, logits, cols, ld, out);
    NC_LAUNCH_CHECK();
    return 0;
}
