/*
 * Split-K flash-decode over the fp8 paged cache (reference: k_attn, model/kernels/decode.cu:567-675, which reads a
 * bf16 contiguous cache with one block per (head, slot) and no split).
 *
 * Work: one wave per (split, kv head, sequence). A split is `split_pages` consecutive 16-key pages of the
 * sequence's key range [max(p - window, 0), p], p = ctx_len - 1 (the query's own key, appended first, is read
 * back from the cache). All G = Hq / Hkv query heads of the kv head ride in the same wave, so every fp8 byte is
 * read from HBM once.
 *
 * Per step the wave takes two pages (32 keys):
 *   scores  Sᵀ[16 keys][16 heads] = K[16][128] · Qᵀ, 4 v_mfma_f32_16x16x32_bf16 per page. The A operand is the
 *           K tile as loaded (lane: key lane%16, 32 contiguous bytes at dims 32 (lane/16)), fp8 -> bf16 exact by
 *           v_cvt_scalef32_pk_bf16_fp8; B is q (bf16) with head = lane%16 (zero past G). Lane (j = lane/16,
 *           n = lane%16) receives the scores of keys 4j..4j+3 for head n.
 *   softmax fp32 online softmax in base 2 (scores pre-scaled by k_scale · sm_scale · log2 e); the running max of
 *           a head is shared by its four lanes (xor 16, 32), the running sum stays per lane until the end.
 *   values  Oᵀ[16 dims][16 heads] += Vᵀ[16 dims][32 keys] · Pᵀ, 8 MFMAs (one per 16 output dims). Pᵀ is the
 *           lane's own 8 probabilities times v_scale, rounded to bf16 (as the reference's torch path feeds bf16
 *           probabilities to PV, inference/modeling_nanochat.py:55); Vᵀ comes straight from the quad-transposed
 *           V tile: lane (j, n) loads the 32 bytes of dims 8n..8n+7, keys 4j..4j+3, and dword bb is one
 *           MFMA's 4 keys of dim 8n+bb. The accumulator lane holds head n, so the softmax rescale is lane-local.
 * Loads for the next step are issued before the current step's math (register double buffer).
 *
 * A split writes its unnormalised Oᵀ, max and sum to the workspace; k_merge combines the splits of each
 * (sequence, query head) with weights exp2(m_s - max m) (decode.cu:547-548's rescale, 0 for an empty state).
 * A sequence with a single split is normalised and written by the attention wave itself.
 *
 * Roofline: HBM. Per (token, kv head) the kernel reads 128 B of K, 128 B of V and two fp32 scales: 264 B.
 */
#include "layout.h"

#define DEC_THREADS 64
#define DEC_TARGET_WAVES 4096 /* ~4 waves per SIMD on 256 CUs: enough loads in flight to cover HBM latency */
#define DEC_MAX_G 16

struct DecodeArgs {
    const bf16_t *q;          /* [B][hq][128] */
    const uint8_t *k_cache, *v_cache;
    const float *k_scale, *v_scale;
    const int32_t *block_table;
    int max_blocks, num_blocks;
    const int32_t *ctx_len;   /* [B] */
    int window;               /* keys before the query; < 0: all */
    int hq, hkv, group;
    float score_scale;        /* sm_scale * log2(e) */
    bf16_t *out;              /* [B][hq][128] */
    float *ws_o;              /* [B][hq][max_splits][128] */
    float *ws_ml;             /* [B][hq][max_splits][2] */
    int max_splits, split_pages;
    int max_ctx;              /* ctx_len is clamped to it: the grid and the workspace are sized by it */
};

struct KeyRange {
    int ctx, p, begin, first_page, last_page, n_splits;
};

__device__ __forceinline__ KeyRange key_range(const DecodeArgs &a, int b) {
    KeyRange r;
    r.ctx = min(a.ctx_len[b], a.max_ctx);
    if (r.ctx <= 0) {
        r.n_splits = 0;
        return r;
    }
    r.p = r.ctx - 1;
    r.begin = (a.window < 0 || r.p <= a.window) ? 0 : r.p - a.window;
    r.first_page = r.begin / NC_PAGE;
    r.last_page = r.p / NC_PAGE;
    r.n_splits = (r.last_page - r.first_page + a.split_pages) / a.split_pages;
    return r;
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

/* 8 fp8 codes (two dwords, byte order = element order) -> 8 bf16, exact. */
__device__ __forceinline__ bf16x8 fp8x8_to_bf16(uint32_t w0, uint32_t w1) {
    const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false);
    const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true);
    const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false);
    const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true);
    return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

/* 8 fp8 codes -> 8 fp16, exact (every e4m3fn value is an fp16 value). */
__device__ __forceinline__ f16x8 fp8x8_to_f16(uint32_t w0, uint32_t w1) {
    const f16x2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false);
    const f16x2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true);
    const f16x2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false);
    const f16x2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true);
    return f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

/* One page's fragments for this lane: K row bytes, V quad bytes, the 4 keys' scales. */
struct Page {
    u32x4 k0, k1, v0, v1;
    f32x4 ks, vs;
};

__device__ __forceinline__ void load_page(const DecodeArgs &a, int blk, int h, int n, int j, Page &pg) {
    const size_t tile = tile_offset(blk, h, a.hkv);
    const uint8_t *kp = a.k_cache + tile + n * NC_HEAD_DIM + j * 32;
    const uint8_t *vp = a.v_cache + tile + j * 512 + n * 32;
    pg.k0 = *reinterpret_cast<const u32x4 *>(kp);
    pg.k1 = *reinterpret_cast<const u32x4 *>(kp + 16);
    pg.v0 = *reinterpret_cast<const u32x4 *>(vp);
    pg.v1 = *reinterpret_cast<const u32x4 *>(vp + 16);
    const size_t s = scale_offset(blk, h, a.hkv) + 4 * j;
    pg.ks = *reinterpret_cast<const f32x4 *>(a.k_scale + s);
    pg.vs = *reinterpret_cast<const f32x4 *>(a.v_scale + s);
}

/* Sᵀ of one page: keys 4j..4j+3 of the page for head n (lane-wise). */
__device__ __forceinline__ f32x4 page_scores(const Page &pg, const bf16x8 *qop) {
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16(pg.k0[0], pg.k0[1]), qop[0], s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16(pg.k0[2], pg.k0[3]), qop[1], s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16(pg.k1[0], pg.k1[1]), qop[2], s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16(pg.k1[2], pg.k1[3]), qop[3], s, 0, 0, 0);
    return s;
}

__device__ __forceinline__ uint32_t v_dword(const Page &pg, int bb) { return bb < 4 ? pg.v0[bb] : pg.v1[bb - 4]; }

/* 2^e as fp32 for e in [-126, 127] (exponent bits only). */
__device__ __forceinline__ float exp2i(int e) { return __uint_as_float((uint32_t)(e + 127) << 23); }

__global__ void __launch_bounds__(DEC_THREADS) k_decode(DecodeArgs a) {
    const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x, n = lane & 15, j = lane >> 4;
    const KeyRange r = key_range(a, b);
    if (r.n_splits == 0) {
        if (split == 0 && n < a.group) { /* no keys: a zero row */
            bf16_t *o = a.out + ((size_t)b * a.hq + h * a.group + n) * NC_HEAD_DIM + j * 32;
            const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int c = 0; c < 4; c++) reinterpret_cast<u32x4 *>(o)[c] = z;
        }
        return;
    }
    if (split >= r.n_splits) return;
    const int pg_begin = r.first_page + split * a.split_pages;
    const int npg = min(a.split_pages, r.last_page + 1 - pg_begin); /* 1..64 pages */

    bf16x8 qop[4];
    if (n < a.group) {
        const u32x4 *qp = reinterpret_cast<const u32x4 *>(a.q + ((size_t)b * a.hq + h * a.group + n) * NC_HEAD_DIM +
                                                         j * 32);
#pragma unroll
        for (int c = 0; c < 4; c++) qop[c] = __builtin_bit_cast(bf16x8, qp[c]);
    } else {
#pragma unroll
        for (int c = 0; c < 4; c++) qop[c] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
    }
    /* lane i holds the block of the split's page i (-1: none), read back by v_readlane */
    const int my_blk = lane < npg ? lookup_block(a.block_table, a.max_blocks, a.num_blocks, b, pg_begin + lane) : -1;

    f32x4 o[8];
#pragma unroll
    for (int bb = 0; bb < 8; bb++) o[bb] = f32x4{0.f, 0.f, 0.f, 0.f};
    /* running softmax max m and per-lane sum l (probability units); o is held in units of 2^(e_ref - 126),
     * e_ref the largest v_scale exponent seen, so that p * v_scale * 2^(126 - e_ref) <= 1 fits fp16 */
    float m = -INFINITY, l = 0.f;
    int e_ref = 0;

    int blk0 = __builtin_amdgcn_readlane(my_blk, 0);
    int blk1 = npg > 1 ? __builtin_amdgcn_readlane(my_blk, 1) : -1;
    Page c0, c1;
    load_page(a, max(blk0, 0), h, n, j, c0);
    load_page(a, blk1 >= 0 ? blk1 : max(blk0, 0), h, n, j, c1);

    const int steps = (npg + 1) >> 1;
    for (int st = 0; st < steps; st++) {
        /* the next step's pages, always loaded (the last step re-reads its own last page) so the wait before
         * this step's math leaves exactly those loads in flight */
        const int i0 = min(2 * st + 2, npg - 1), i1 = min(2 * st + 3, npg - 1);
        const int nb0 = __builtin_amdgcn_readlane(my_blk, i0), nb1 = __builtin_amdgcn_readlane(my_blk, i1);
        Page n0, n1;
        load_page(a, max(nb0, 0), h, n, j, n0);
        load_page(a, max(nb1, 0), h, n, j, n1);

        const f32x4 s0 = page_scores(c0, qop), s1 = page_scores(c1, qop);
        const int base = (pg_begin + 2 * st) * NC_PAGE + 4 * j; /* key of (page 0, i = 0) for this lane */
        const int lo = r.begin - base, hi = r.p - base;         /* valid i of page 0 in [lo, hi], page 1 -16 */
        float sv[8], vsv[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const bool ok0 = blk0 >= 0 && i >= lo && i <= hi;
            const bool ok1 = blk1 >= 0 && i + NC_PAGE >= lo && i + NC_PAGE <= hi;
            sv[i] = ok0 ? s0[i] * (c0.ks[i] * a.score_scale) : -INFINITY;
            sv[4 + i] = ok1 ? s1[i] * (c1.ks[i] * a.score_scale) : -INFINITY;
            vsv[i] = ok0 ? c0.vs[i] : 0.f;
            vsv[4 + i] = ok1 ? c1.vs[i] : 0.f;
        }
        float mx = sv[0], vmax = vsv[0];
#pragma unroll
        for (int i = 1; i < 8; i++) {
            mx = fmaxf(mx, sv[i]);
            vmax = fmaxf(vmax, vsv[i]);
        }
        mx = fmaxf(mx, shfl_xor_f(mx, 16));
        mx = fmaxf(mx, shfl_xor_f(mx, 32));
        vmax = fmaxf(vmax, shfl_xor_f(vmax, 16));
        vmax = fmaxf(vmax, shfl_xor_f(vmax, 32));
        const float m_new = fmaxf(m, mx);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m - m_use);
        const int e_new = max(e_ref, (int)(__float_as_uint(vmax) >> 23));
        const float w = exp2i(126 - e_new);                          /* p * vs * w <= 1 */
        const float rescale = alpha * exp2i(max(e_ref - e_new, -126)); /* old units -> new units */
        e_ref = e_new;
        float pv[8], ps = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            pv[i] = __builtin_amdgcn_exp2f(sv[i] - m_use);
            ps += pv[i];
        }
        l = l * alpha + ps;
        m = m_new;
        f16x8 pop;
#pragma unroll
        for (int i = 0; i < 8; i++) pop[i] = (_Float16)(pv[i] * (vsv[i] * w));
        if (!__all(rescale == 1.0f)) {
#pragma unroll
            for (int bb = 0; bb < 8; bb++) o[bb] *= rescale;
        }
#pragma unroll
        for (int bb = 0; bb < 8; bb++)
            o[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fp8x8_to_f16(v_dword(c0, bb), v_dword(c1, bb)), pop, o[bb],
                                                           0, 0, 0);
        c0 = n0;
        c1 = n1;
        blk0 = 2 * st + 2 < npg ? nb0 : -1;
        blk1 = 2 * st + 3 < npg ? nb1 : -1;
    }

    l += shfl_xor_f(l, 16);
    l += shfl_xor_f(l, 32);
    if (n >= a.group) return;
    const int head = h * a.group + n;
    const float unit = exp2i(e_ref - 126); /* o * unit: Σ p v in value units */
    /* lane (j, n) holds dims (4j + i) * 8 + bb of head n: 8 contiguous dims per i */
    if (r.n_splits == 1) {
        bf16_t *dst = a.out + ((size_t)b * a.hq + head) * NC_HEAD_DIM;
        const float inv = unit / l;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float v[8];
#pragma unroll
            for (int bb = 0; bb < 8; bb++) v[bb] = o[bb][i] * inv;
            store_bf16x8(dst + (4 * j + i) * 8, v);
        }
        return;
    }
    const size_t slot = ((size_t)b * a.hq + head) * a.max_splits + split;
    float *dst = a.ws_o + slot * NC_HEAD_DIM;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f32x4 lo4 = {o[0][i] * unit, o[1][i] * unit, o[2][i] * unit, o[3][i] * unit};
        f32x4 hi4 = {o[4][i] * unit, o[5][i] * unit, o[6][i] * unit, o[7][i] * unit};
        reinterpret_cast<f32x4 *>(dst + (4 * j + i) * 8)[0] = lo4;
        reinterpret_cast<f32x4 *>(dst + (4 * j + i) * 8)[1] = hi4;
    }
    if (j == 0) {
        a.ws_ml[2 * slot] = m;
        a.ws_ml[2 * slot + 1] = l;
    }
}

/* One wave per (query head, sequence): thread t combines dims 2t, 2t+1 over the splits. */
__global__ void __launch_bounds__(DEC_THREADS) k_merge(DecodeArgs a) {
    const int head = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    const KeyRange r = key_range(a, b);
    if (r.n_splits <= 1) return;
    const size_t base = ((size_t)b * a.hq + head) * a.max_splits;
    const float *ml = a.ws_ml + 2 * base;
    float mmax = -INFINITY;
    for (int s = 0; s < r.n_splits; s++) mmax = fmaxf(mmax, ml[2 * s]);
    float sum = 0.f, acc0 = 0.f, acc1 = 0.f;
    for (int s = 0; s < r.n_splits; s++) {
        const float w = ml[2 * s] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml[2 * s] - mmax);
        sum += w * ml[2 * s + 1];
        const f32x2 v = *reinterpret_cast<const f32x2 *>(a.ws_o + (base + s) * NC_HEAD_DIM + 2 * t);
        acc0 += w * v[0];
        acc1 += w * v[1];
    }
    const float inv = 1.0f / sum;
    bf16_t *dst = a.out + ((size_t)b * a.hq + head) * NC_HEAD_DIM + 2 * t;
    *reinterpret_cast<uint32_t *>(dst) = f32_to_bf16(acc0 * inv) | (f32_to_bf16(acc1 * inv) << 16);
}

/* Waves the split plan aims for; NC_DECODE_TARGET_WAVES overrides it (a tuning knob, read once). */
static int target_waves() {
    static const int waves = [] {
        const char *e = getenv("NC_DECODE_TARGET_WAVES");
        const int v = e ? atoi(e) : 0;
        return v > 0 ? v : DEC_TARGET_WAVES;
    }();
    return waves;
}

/* The split plan, a function of the shape only so the workspace size is known before the call. */
static void decode_plan(int B, int hkv, int max_ctx, int *split_pages, int *max_splits) {
    const int pages = (max_ctx + NC_PAGE - 1) / NC_PAGE + 1; /* +1: a window can start mid-page */
    long long units = (long long)B * hkv;
    int per_seq = (int)((target_waves() + units - 1) / units);
    if (per_seq < 1) per_seq = 1;
    int sp = (pages + per_seq - 1) / per_seq;
    sp = sp < 2 ? 2 : (sp + 1) & ~1; /* whole two-page steps */
    if (sp > 64) sp = 64;          /* one lane per page holds the split's block ids */
    *split_pages = sp;
    *max_splits = (pages + sp - 1) / sp;
}

extern "C" long long nc_decode_workspace_bytes(int B, int hq, int hkv, int max_ctx) {
    if (B <= 0 || hq <= 0 || hkv <= 0 || max_ctx <= 0) return 0;
    int sp, ms;
    decode_plan(B, hkv, max_ctx, &sp, &ms);
    if (ms <= 1) return 0;
    return (long long)B * hq * ms * (NC_HEAD_DIM + 2) * (long long)sizeof(float);
}

extern "C" int nc_decode_attn_fp8(const void *q, const uint8_t *k_cache, const uint8_t *v_cache,
                                  const float *k_scale, const float *v_scale, const int32_t *block_table,
                                  int max_blocks, int num_blocks, const int32_t *ctx_len, int window, int B, int hq,
                                  int hkv, int max_ctx, float sm_scale, void *out, void *workspace,
                                  long long workspace_bytes, void *stream) {
    NC_REQUIRE(B >= 0, "B = %d < 0", B);
    if (B == 0) return 0;
    NC_REQUIRE(hkv > 0 && hq > 0 && hq % hkv == 0, "hq = %d must be a positive multiple of hkv = %d", hq, hkv);
    NC_REQUIRE(hq / hkv <= DEC_MAX_G, "hq / hkv = %d exceeds %d query heads per kv head", hq / hkv, DEC_MAX_G);
    NC_REQUIRE(max_blocks > 0 && num_blocks > 0, "max_blocks %d, num_blocks %d must be positive", max_blocks,
               num_blocks);
    NC_REQUIRE(block_table || (long long)B * max_blocks <= num_blocks,
               "contiguous cache: %d sequences x %d blocks exceed the %d blocks", B, max_blocks, num_blocks);
    NC_REQUIRE(max_ctx > 0 && max_ctx <= max_blocks * NC_PAGE, "max_ctx %d outside [1, %d]", max_ctx,
               max_blocks * NC_PAGE);
    NC_REQUIRE(q && k_cache && v_cache && k_scale && v_scale && ctx_len && out, "null argument");
    NC_REQUIRE(((uintptr_t)q | (uintptr_t)out | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)k_scale |
                (uintptr_t)v_scale | (uintptr_t)workspace) % 16 == 0, "tensors must be 16-byte aligned");
    const long long need = nc_decode_workspace_bytes(B, hq, hkv, max_ctx);
    NC_REQUIRE(workspace_bytes >= need && (need == 0 || workspace), "workspace %lld bytes, %lld needed",
               workspace_bytes, need);
    DecodeArgs a = {};
    a.q = (const bf16_t *)q; a.k_cache = k_cache; a.v_cache = v_cache; a.k_scale = k_scale; a.v_scale = v_scale;
    a.block_table = block_table; a.max_blocks = max_blocks; a.num_blocks = num_blocks; a.ctx_len = ctx_len;
    a.window = window; a.hq = hq; a.hkv = hkv; a.group = hq / hkv;
    a.score_scale = sm_scale * 1.4426950408889634f;
    a.out = (bf16_t *)out;
    a.max_ctx = max_ctx;
    decode_plan(B, hkv, max_ctx, &a.split_pages, &a.max_splits);
    a.ws_o = (float *)workspace;
    a.ws_ml = a.ws_o ? a.ws_o + (size_t)B * hq * a.max_splits * NC_HEAD_DIM : nullptr;
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(k_decode, dim3(a.max_splits, hkv, B), dim3(DEC_THREADS), 0, s, a);
    NC_LAUNCH_CHECK();
    if (a.max_splits > 1) {
        hipLaunchKernelGGL(k_merge, dim3(hq, B), dim3(DEC_THREADS), 0, s, a);
        NC_LAUNCH_CHECK();
    }
    return 0;
}
