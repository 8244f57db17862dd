/* GPU probe for tests/test_gpu_bf16_rounding.py (test infrastructure): the library's bf16 rounding helpers
 * (nanochat_amd/csrc/common.h: f32x2_to_bf16x2, the packed v_cvt_pk_bf16_f32, and f32_to_bf16) against the integer
 * round-to-nearest-even rule with quiet NaNs, ((u + 0x7fff + bit 16 of u) >> 16, a NaN giving (u >> 16) | 0x40),
 * over all 2^32 fp32 bit patterns. Each result is written to memory by its own kernel and a fourth kernel compares
 * them, so no compiler folding relates the two. Built twice by build_probes.py: with the library's default flags
 * and with prefill_attn.hip's -mno-amdgpu-ieee -fno-honor-nans. */
#include "../../nanochat_amd/csrc/common.h"

namespace {

constexpr uint32_t PAIRS = 1u << 27; /* pairs of patterns per round: 16 rounds cover 2^32 */
constexpr uint32_t BLOCK = 256;

__global__ void k_packed(uint32_t base, uint32_t *out) {
    const uint32_t t = blockIdx.x * BLOCK + threadIdx.x, u = base + 2 * t;
    out[t] = f32x2_to_bf16x2(__uint_as_float(u), __uint_as_float(u + 1));
}

__global__ void k_scalar(uint32_t base, uint32_t *out) {
    const uint32_t t = blockIdx.x * BLOCK + threadIdx.x, u = base + 2 * t;
    out[t] = f32_to_bf16(__uint_as_float(u)) | (f32_to_bf16(__uint_as_float(u + 1)) << 16);
}

__device__ uint32_t integer_rule(uint32_t u) {
    const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16, quiet = (u >> 16) | 0x40u;
    return ((u & 0x7fffffffu) > 0x7f800000u ? quiet : rounded) & 0xffffu;
}

__global__ void k_rule(uint32_t base, uint32_t *out) {
    const uint32_t t = blockIdx.x * BLOCK + threadIdx.x, u = base + 2 * t;
    out[t] = integer_rule(u) | (integer_rule(u + 1) << 16);
}

/* per block: the number of differing pairs and the first differing pair's index (or ~0) */
__global__ void k_compare(const uint32_t *a, const uint32_t *b, uint32_t *count, uint32_t *first) {
    __shared__ uint32_t c[BLOCK], f[BLOCK];
    const uint32_t t = blockIdx.x * BLOCK + threadIdx.x;
    const bool differ = a[t] != b[t];
    c[threadIdx.x] = differ;
    f[threadIdx.x] = differ ? t : 0xffffffffu;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t s = 0, m = 0xffffffffu;
        for (uint32_t i = 0; i < BLOCK; i++) {
            s += c[i];
            m = f[i] < m ? f[i] : m;
        }
        count[blockIdx.x] = s;
        first[blockIdx.x] = m;
    }
}

}  // namespace

/* Differing pairs for the packed and the scalar helper over all 2^32 patterns; first_bad: the first differing
 * pattern (or ~0). Returns 0, or -1 on a HIP error (message to stderr). */
extern "C" int bf16_probe(unsigned long long *packed_bad, unsigned long long *scalar_bad, uint32_t *first_bad) {
    const uint32_t blocks = PAIRS / BLOCK;
    uint32_t *hw = nullptr, *sc = nullptr, *rule = nullptr, *cnt = nullptr, *fst = nullptr;
    uint32_t *hc = new uint32_t[blocks], *hf = new uint32_t[blocks];
    int rc = 0;
    *packed_bad = *scalar_bad = 0;
    *first_bad = 0xffffffffu;
    if (hipMalloc(&hw, (size_t)PAIRS * 4) != hipSuccess || hipMalloc(&sc, (size_t)PAIRS * 4) != hipSuccess ||
        hipMalloc(&rule, (size_t)PAIRS * 4) != hipSuccess || hipMalloc(&cnt, blocks * 4) != hipSuccess ||
        hipMalloc(&fst, blocks * 4) != hipSuccess) {
        fprintf(stderr, "bf16_probe: hipMalloc failed\n");
        rc = -1;
    }
    for (uint32_t r = 0; r < 16 && rc == 0; r++) {
        const uint32_t base = r << 28;
        hipLaunchKernelGGL(k_packed, dim3(blocks), dim3(BLOCK), 0, 0, base, hw);
        hipLaunchKernelGGL(k_scalar, dim3(blocks), dim3(BLOCK), 0, 0, base, sc);
        hipLaunchKernelGGL(k_rule, dim3(blocks), dim3(BLOCK), 0, 0, base, rule);
        for (int which = 0; which < 2 && rc == 0; which++) {
            hipLaunchKernelGGL(k_compare, dim3(blocks), dim3(BLOCK), 0, 0, which ? sc : hw, rule, cnt, fst);
            if (hipDeviceSynchronize() != hipSuccess || hipMemcpy(hc, cnt, blocks * 4, hipMemcpyDeviceToHost) ||
                hipMemcpy(hf, fst, blocks * 4, hipMemcpyDeviceToHost)) {
                fprintf(stderr, "bf16_probe: HIP error in round %u\n", r);
                rc = -1;
                break;
            }
            for (uint32_t i = 0; i < blocks; i++) {
                (which ? *scalar_bad : *packed_bad) += hc[i];
                if (hc[i] && *first_bad == 0xffffffffu) *first_bad = base + 2 * hf[i];
            }
        }
    }
    hipFree(hw);
    hipFree(sc);
    hipFree(rule);
    hipFree(cnt);
    hipFree(fst);
    delete[] hc;
    delete[] hf;
    return rc;
}
