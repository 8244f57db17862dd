/*
 * Token choice of a decode step's slots.
 *
 * nc_argmax_f32, greedy: per row, the column of the largest fp32 logit, the lowest column among exact ties
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

/* ------------------------------------------------------------------------------------------ sampling head */
/*
 * nc_choose_tokens: every active slot's next token by its temperature, top_p, seed and (for a masked slot) its
 * allowed rows, then the commit (reference: the ARGMAX epilogue with CHOICE, k_nucleus and k_commit,
 * model/kernels/decode.cu:170-230,360-404,676-689; host rules inference/decoder.py:28-40):
 *   T == 0     the largest raw logit over the allowed rows (lowest row on ties);
 *   T > 0      Gumbel-max: the largest z / T + g(seed, pos - first, row), z = c tanh(s / c) (c <= 0: z = s), which
 *              samples softmax(z / T) (arXiv 1411.0030 §2);
 *   top_p < 1  (T > 0) nucleus (arXiv 1904.09751 §3.1): e = exp(z / T - max), keep e >= e*, e* the least e with
 *              sum(e' <= e*) > (1 - top_p) sum(e) (bisection on the IEEE bits of e* in [0, 1], fp32 sums in a fixed
 *              order), then Gumbel-max over the kept rows;
 *   alt        the best allowed row but `lazy` (none for a nucleus slot), for a host that rejects the lazy row;
 *   commit     tokens = the choice's row (-1: no allowed row), alt_tokens likewise, pos += 1.
 * The noise: Philox4x32-10 (Salmon et al., SC '11: "Parallel random numbers: as easy as 1, 2, 3") at counter
 * (row, i, 0, 0) and key (seed low, seed high); the top 52 bits r of its first two words give u = (2r + 1) 2^-53,
 * g = float(-log(-log(u))) in double (decode.cu:98-105's transform).
 *
 * k_choose: a grid of B x P workgroups of 512 threads; workgroup (b, p) scans rows [p L, (p + 1) L) of slot b and
 * writes its best and alternative keys to the workspace. A nucleus slot needs whole-row reductions: k_nucleus, one
 * 512-thread workgroup per slot, keeps the slot's e values in registers (up to 128 per thread: vocabularies up to
 * 65536; up to 131072 with spills) so that the bisection's ~30 passes are register sums and block reductions, and
 * writes the slot's key.
 * k_commit then folds each slot's P keys and commits. Sampling is ALU-bound (10 Philox rounds and two double logs
 * per row); greedy is HBM-bound on 4 B per logit.
 */

#define CH_THREADS 512
#define CH_WAVES (CH_THREADS / NC_WAVE)
#define CH_ROWS_PER_THREAD 16 /* rows a thread scans on the non-nucleus paths: P = ceil(vocab / (512 x 16)) */
#define CH_MAX_PARTS 64

struct ChooseArgs {
    const float *logits;
    long long ld;
    int B, vocab, parts, span;               /* workgroups per slot, rows per workgroup */
    const unsigned long long *active;        /* [2][words]: active slots, then masked slots; null: all, none */
    int words;
    const uint32_t *allow;                   /* [B][allow_words]: a masked slot's allowed rows */
    int allow_words;
    const float *temperature, *top_p;        /* [B] */
    const unsigned long long *seed;          /* [B] */
    const int32_t *first;                    /* [B] */
    int32_t *pos;                            /* [B]: the input's position; += 1 by the commit */
    float softcap;
    int lazy;
    unsigned long long *keys;                /* [B][parts][2]: best, alternative */
    int32_t *tokens, *alt_tokens;            /* [B] */
};

__device__ __forceinline__ bool slot_bit(const unsigned long long *mask, int b) { return (mask[b >> 6] >> (b & 63)) & 1ull; }

/* Philox4x32-10 (SC '11): (hi0, lo0) = M0 c0, (hi1, lo1) = M1 c2, c = (hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0); the key
 * advances by the Weyl increments between rounds. Returns the first two output words. */
__device__ __forceinline__ void philox_2(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0, uint32_t k1,
                                         uint32_t &o0, uint32_t &o1) {
#pragma unroll
    for (int r = 0; r < 10; r++) {
        const uint32_t lo0 = 0xD2511F53u * c0, hi0 = __umulhi(0xD2511F53u, c0);
        const uint32_t lo1 = 0xCD9E8D57u * c2, hi1 = __umulhi(0xCD9E8D57u, c2);
        const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
        c0 = n0, c1 = lo1, c2 = n2, c3 = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    o0 = c0;
    o1 = c1;
}

__device__ __forceinline__ float gumbel_noise(unsigned long long seed, uint32_t i, uint32_t row) {
    uint32_t x0, x1;
    philox_2(row, i, 0u, 0u, (uint32_t)seed, (uint32_t)(seed >> 32), x0, x1);
    const unsigned long long r = (((unsigned long long)x0 << 32) | x1) >> 12;
    const double u = (2.0 * (double)r + 1.0) * 0x1p-53;
    return (float)-log(-log(u));
}

__device__ __forceinline__ float capped(float s, float c) { return c > 0.f ? c * tanhf(s / c) : s; }

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long v, int d) {
    return ((unsigned long long)__shfl_xor((unsigned)(v >> 32), d, NC_WAVE) << 32) | __shfl_xor((unsigned)v, d, NC_WAVE);
}

/* Block reductions over CH_WAVES waves, result in every thread; fixed order (xor tree, then waves in order). */
__device__ unsigned long long block_max_u64(unsigned long long v, unsigned long long *sh) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v = max_u64(v, shfl_xor_u64(v, d));
    __syncthreads();
    if ((threadIdx.x & (NC_WAVE - 1)) == 0) sh[threadIdx.x / NC_WAVE] = v;
    __syncthreads();
    unsigned long long r = sh[0];
    for (int w = 1; w < CH_WAVES; w++) r = max_u64(r, sh[w]);
    return r;
}

__device__ __forceinline__ bool row_allowed(const uint32_t *allow, int r) { return !allow || ((allow[r >> 5] >> (r & 31)) & 1u); }

/* A nucleus slot, one workgroup of NU_THREADS: its e values stay in registers (PER per thread, row
 * r = k NU_THREADS + thread), so the ~30 bisection passes are ALU and block sums only. Rows past the vocabulary hold
 * e = 0, which no pass counts above a positive threshold. */
#define NU_THREADS 512 /* 2 waves per SIMD: up to 256 VGPRs, room for 128 e values per thread */
#define NU_WAVES (NU_THREADS / NC_WAVE)

__device__ float nu_block_max(float v, float *sh) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, shfl_xor_f(v, d));
    __syncthreads();
    if ((threadIdx.x & (NC_WAVE - 1)) == 0) sh[threadIdx.x / NC_WAVE] = v;
    __syncthreads();
    float r = sh[0];
    for (int w = 1; w < NU_WAVES; w++) r = fmaxf(r, sh[w]);
    return r;
}

__device__ float nu_block_sum(float v, float *sh) {
#pragma clang fp contract(off)
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v = v + shfl_xor_f(v, d);
    __syncthreads();
    if ((threadIdx.x & (NC_WAVE - 1)) == 0) sh[threadIdx.x / NC_WAVE] = v;
    __syncthreads();
    float r = sh[0];
    for (int w = 1; w < NU_WAVES; w++) r = r + sh[w];
    return r;
}

__device__ unsigned long long nu_block_max_u64(unsigned long long v, unsigned long long *sh) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v = max_u64(v, shfl_xor_u64(v, d));
    __syncthreads();
    if ((threadIdx.x & (NC_WAVE - 1)) == 0) sh[threadIdx.x / NC_WAVE] = v;
    __syncthreads();
    unsigned long long r = sh[0];
    for (int w = 1; w < NU_WAVES; w++) r = max_u64(r, sh[w]);
    return r;
}


template <int PER>
__global__ void __launch_bounds__(NU_THREADS) k_nucleus(ChooseArgs a) {
#pragma clang fp contract(off)
    __shared__ float fsh[NU_WAVES];
    __shared__ unsigned long long ksh[NU_WAVES];
    const int b = blockIdx.x, tid = threadIdx.x;
    if (a.active && !slot_bit(a.active, b)) return;
    const float T = a.temperature ? a.temperature[b] : 0.f, P = a.top_p ? a.top_p[b] : 1.f;
    if (!(T > 0.f && P < 1.f)) return;
    const bool masked = a.active && slot_bit(a.active + a.words, b);
    const uint32_t *allow = masked ? a.allow + (size_t)b * a.allow_words : nullptr;
    const float *s = a.logits + (size_t)b * a.ld;
    const uint32_t i = (uint32_t)(a.pos[b] - (a.first ? a.first[b] : 0));
    float zt[PER];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int r = k * NU_THREADS + tid;
        zt[k] = (r < a.vocab && row_allowed(allow, r)) ? capped(s[r], a.softcap) / T : -INFINITY;
        m = fmaxf(m, zt[k]);
    }
    m = nu_block_max(m, fsh);
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        zt[k] = zt[k] == -INFINITY ? 0.f : expf(zt[k] - m); /* zt now holds e */
        sum = sum + zt[k];
    }
    const float drop = (1.f - P) * nu_block_sum(sum, fsh);
    uint32_t lo = 0u, hi = __float_as_uint(1.f); /* the least bits u with C(u) > drop; C(1) is the whole sum */
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        const float x = __uint_as_float(mid);
        float below = 0.f;
#pragma unroll
        for (int k = 0; k < PER; k++) below = below + (zt[k] <= x ? zt[k] : 0.f);
        if (nu_block_sum(below, fsh) > drop) hi = mid; else lo = mid + 1;
    }
    const float least = __uint_as_float(lo);
    /* the kept rows as bit masks (static register indices), then Gumbel-max over their set bits */
    constexpr int WORDS = (PER + 63) / 64;
    unsigned long long best = 0;
#pragma unroll
    for (int wd = 0; wd < WORDS; wd++) {
        unsigned long long kept = 0;
#pragma unroll
        for (int k = wd * 64; k < (wd + 1) * 64 && k < PER; k++)
            kept |= (unsigned long long)(zt[k] >= least && zt[k] > 0.f) << (k - wd * 64);
        while (kept) {
            const int k = wd * 64 + __builtin_ctzll(kept);
            kept &= kept - 1;
            const int r = k * NU_THREADS + tid;
            const float score = capped(s[r], a.softcap) / T + gumbel_noise(a.seed[b], i, (uint32_t)r);
            best = max_u64(best, choice_key(score, (uint32_t)r));
        }
    }
    best = nu_block_max_u64(best, ksh);
    if (tid == 0) {
        unsigned long long *out = a.keys + (size_t)b * a.parts * 2;
        out[0] = best;
        out[1] = 0ull;
    }
}

__global__ void __launch_bounds__(CH_THREADS) k_choose(ChooseArgs a) {
#pragma clang fp contract(off)
    __shared__ unsigned long long ksh[CH_WAVES];
    const int b = blockIdx.x / a.parts, p = blockIdx.x % a.parts;
    if (a.active && !slot_bit(a.active, b)) return;
    const bool masked = a.active && slot_bit(a.active + a.words, b);
    const uint32_t *allow = masked ? a.allow + (size_t)b * a.allow_words : nullptr;
    const float T = a.temperature ? a.temperature[b] : 0.f, P = a.top_p ? a.top_p[b] : 1.f;
    const float *s = a.logits + (size_t)b * a.ld;
    const uint32_t i = (uint32_t)(a.pos[b] - (a.first ? a.first[b] : 0));
    unsigned long long *out = a.keys + ((size_t)b * a.parts + p) * 2;
    if (T > 0.f && P < 1.f) { /* k_nucleus writes part 0 */
        if (threadIdx.x == 0 && p > 0) out[0] = out[1] = 0ull;
        return;
    }
    unsigned long long best = 0, alt = 0;
    const int r1 = min(a.vocab, (p + 1) * a.span);
    for (int r = p * a.span + threadIdx.x; r < r1; r += CH_THREADS) {
        if (!row_allowed(allow, r)) continue;
        const float score = T > 0.f ? capped(s[r], a.softcap) / T + gumbel_noise(a.seed[b], i, (uint32_t)r) : s[r];
        const unsigned long long key = choice_key(score, (uint32_t)r);
        best = max_u64(best, key);
        if (r != a.lazy) alt = max_u64(alt, key);
    }
    best = block_max_u64(best, ksh);
    alt = block_max_u64(alt, ksh);
    if (threadIdx.x == 0) out[0] = best, out[1] = alt;
}

__global__ void k_commit(ChooseArgs a) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= a.B || (a.active && !slot_bit(a.active, b))) return;
    unsigned long long best = 0, alt = 0;
    const unsigned long long *k = a.keys + (size_t)b * a.parts * 2;
    for (int p = 0; p < a.parts; p++) best = max_u64(best, k[2 * p]), alt = max_u64(alt, k[2 * p + 1]);
    a.tokens[b] = (int32_t)(0xffffffffu - (uint32_t)best);
    a.alt_tokens[b] = (int32_t)(0xffffffffu - (uint32_t)alt);
    a.pos[b] += 1;
}

static int choose_parts(int vocab) {
    const int per = CH_THREADS * CH_ROWS_PER_THREAD;
    const int parts = (vocab + per - 1) / per;
    return parts < 1 ? 1 : (parts > CH_MAX_PARTS ? CH_MAX_PARTS : parts);
}

extern "C" long long nc_choose_workspace_bytes(int B, int vocab) {
    if (B <= 0 || vocab <= 0) return 0;
    return (long long)((size_t)B * choose_parts(vocab) * 2 * sizeof(unsigned long long));
}

extern "C" int nc_choose_tokens(const float *logits, int B, int vocab, long long ld, const unsigned long long *active,
                                const uint32_t *allow, const float *temperature, const float *top_p,
                                const unsigned long long *seed, const int32_t *first, int32_t *pos, float softcap,
                                int lazy, int32_t *tokens, int32_t *alt_tokens, void *workspace,
                                long long workspace_bytes, void *stream) {
    NC_REQUIRE(B >= 0 && vocab > 0 && ld >= vocab, "nc_choose_tokens: B %d, vocab %d, ld %lld", B, vocab, ld);
    NC_REQUIRE(vocab <= 256 * NU_THREADS, "nc_choose_tokens: vocab %d exceeds %d", vocab, 256 * NU_THREADS);
    if (B == 0) return 0;
    NC_REQUIRE(logits && pos && tokens && alt_tokens && workspace, "nc_choose_tokens: null argument");
    NC_REQUIRE(!active || allow, "nc_choose_tokens: a slot mask needs the allowed-row masks (allow)");
    NC_REQUIRE((temperature && seed) || !temperature, "nc_choose_tokens: sampling needs seeds");
    const long long need = nc_choose_workspace_bytes(B, vocab);
    NC_REQUIRE(workspace_bytes >= need, "nc_choose_tokens: workspace %lld bytes, %lld needed", workspace_bytes, need);
    NC_REQUIRE((uintptr_t)workspace % 16 == 0, "nc_choose_tokens: workspace must be 16-byte aligned");
    ChooseArgs a = {};
    a.logits = logits; a.ld = ld; a.B = B; a.vocab = vocab;
    a.parts = choose_parts(vocab);
    a.span = (vocab + a.parts - 1) / a.parts;
    a.active = active; a.words = (B + 63) / 64;
    a.allow = allow; a.allow_words = (vocab + 31) / 32;
    a.temperature = temperature; a.top_p = top_p; a.seed = seed; a.first = first; a.pos = pos;
    a.softcap = softcap; a.lazy = lazy;
    a.keys = (unsigned long long *)workspace;
    a.tokens = tokens; a.alt_tokens = alt_tokens;
    hipLaunchKernelGGL(k_choose, dim3((unsigned)(B * a.parts)), dim3(CH_THREADS), 0, (hipStream_t)stream, a);
    NC_LAUNCH_CHECK();
    if (temperature && top_p) { /* nucleus slots (temperature > 0, top_p < 1), if any: chosen on the device */
        const int per = (vocab + NU_THREADS - 1) / NU_THREADS;
        if (per <= 16)
            hipLaunchKernelGGL(k_nucleus<16>, dim3(B), dim3(NU_THREADS), 0, (hipStream_t)stream, a);
        else if (per <= 32)
            hipLaunchKernelGGL(k_nucleus<32>, dim3(B), dim3(NU_THREADS), 0, (hipStream_t)stream, a);
        else if (per <= 64)
            hipLaunchKernelGGL(k_nucleus<64>, dim3(B), dim3(NU_THREADS), 0, (hipStream_t)stream, a);
        else if (per <= 128)
            hipLaunchKernelGGL(k_nucleus<128>, dim3(B), dim3(NU_THREADS), 0, (hipStream_t)stream, a);
        else /* past 65536 rows the values spill to scratch: slower, the same result */
            hipLaunchKernelGGL(k_nucleus<256>, dim3(B), dim3(NU_THREADS), 0, (hipStream_t)stream, a);
        NC_LAUNCH_CHECK();
    }
    hipLaunchKernelGGL(k_commit, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, (hipStream_t)stream, a);
    NC_LAUNCH_CHECK();
    return 0;
}
