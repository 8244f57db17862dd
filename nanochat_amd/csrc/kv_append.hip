/*
 * The fp8 KV cache's write side and its gather:
 *   nc_kv_append_fp8  fused append: per row of the fused projection, q and k through QK-norm + RoPE (q to q_out
 *                     in bf16), k and v quantised per (token, kv head) to e4m3fn + fp32 scale and written to
 *                     the row's page (reference: k_prologue, model/kernels/decode.cu:550-565, which writes bf16)
 *   nc_kv_store_fp8   quantise-and-store of K/V rows that are already final (no norm, no rotation), e.g. a
 *                     cache filled from another model's keys (DynamicCache.update,
 *                     inference/modeling_nanochat.py:95-96)
 *   qkp_forward       the training-side q/k prologue, same signature as model/kernels/qk_prologue.cu:111-118
 *   nc_kv_gather_fp8  each sequence's cached codes and scales in the canonical row-major layout
 *
 * A row item is 8 lanes (qk_row.h); a 256-thread workgroup handles 32 items. These kernels move a few hundred
 * bytes per row: they are launch-latency bound, not HBM bound, and are written for exactness, not speed.
 */
#include <stdarg.h>
#include <string.h>

#include "layout.h"
#include "qk_row.h"

#define APPEND_THREADS 256
#define ITEMS_PER_BLOCK (APPEND_THREADS / NC_ROW_LANES)

static __thread char nc_error[512];

int nc_fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(nc_error, sizeof nc_error, fmt, ap);
    va_end(ap);
    return -1;
}

extern "C" const char *nc_last_error(void) { return nc_error; }

extern "C" int nc_abi_version(void) { return 1; }

struct AppendArgs {
    const bf16_t *qkv;        /* fused mode: [n][row_stride], q heads then k heads then v heads */
    const bf16_t *k_rows;     /* store mode: [n][row_stride] kv heads */
    const bf16_t *v_rows;
    long long row_stride;
    int n;
    const int32_t *pos, *seq;
    const float *q_gain, *k_gain, *cos, *sin;
    int rope_len;
    int hq, hkv;
    bf16_t *q_out;            /* fused mode: [n][hq][128] */
    int32_t *ctx_out;         /* fused mode, optional: [n] pos + 1, the context length after the append */
    uint8_t *cache;           /* [num_blocks][hkv][4224] tiles */
    const int32_t *block_table;
    int max_blocks, num_blocks, num_seqs;
    int fused;                /* 1: norm + rope q and k, write q_out; 0: store rows as given */
};

/* The 4 x 4 byte transpose of a quad's V codes: lane r of 4 items (8 lanes apart) holds dword w = bytes of dims
 * 4c..4c+3 of token r; it returns the dword of dim 4c + r over tokens 0..3 (the quad-transposed layout), in two
 * exchanges (partner r ^ 2, then r ^ 1). */
__device__ __forceinline__ uint32_t quad_transpose(uint32_t w, int r) {
    const uint32_t x = (uint32_t)__shfl_xor((int)w, 16, NC_WAVE);
    const uint32_t w1 = r < 2 ? (w & 0xffffu) | (x << 16) : (x >> 16) | (w & 0xffff0000u);
    const uint32_t y = (uint32_t)__shfl_xor((int)w1, 8, NC_WAVE);
    return (r & 1) ? ((y >> 8) & 0x00ff00ffu) | (w1 & 0xff00ff00u) : (w1 & 0x00ff00ffu) | ((y & 0x00ff00ffu) << 8);
}

/* The least and the largest of v over the 4 items of a quad (lanes 8 and 16 apart). */
__device__ __forceinline__ int quad_min(int v) {
    v = min(v, __shfl_xor(v, 8, NC_WAVE));
    return min(v, __shfl_xor(v, 16, NC_WAVE));
}
__device__ __forceinline__ int quad_max(int v) {
    v = max(v, __shfl_xor(v, 8, NC_WAVE));
    return max(v, __shfl_xor(v, 16, NC_WAVE));
}

/* Items are (row quad, head, row r within the quad), 8 lanes each (qk_row.h). Fused: heads [0, hq) are q,
 * [hq, hq + hkv) k, then v. Store: [0, hkv) k, then v. The 4 rows of a quad sit in 4 consecutive items of one wave
 * (lanes 8 r + lane % 8 of a 32-lane half), so when they are the 4 positions of one quad of one page, in order (a
 * prefill's rows), their V codes are transposed between the items and written as dwords instead of bytes. A row
 * whose position, sequence or page is out of range writes no cache byte; its q_out row is NaN. */
__global__ void __launch_bounds__(APPEND_THREADS) k_append(AppendArgs a) {
    const int heads = a.fused ? a.hq + 2 * a.hkv : 2 * a.hkv;
    const long long item = (long long)blockIdx.x * ITEMS_PER_BLOCK + threadIdx.x / NC_ROW_LANES;
    if (item >= (((long long)a.n + 3) / 4) * heads * 4) return; /* whole quads of items leave together */
    const int g = threadIdx.x % NC_ROW_LANES, r = (int)(item & 3);
    const int head = (int)((item >> 2) % heads), row = (int)((item >> 2) / heads) * 4 + r;
    const bool live = row < a.n;
    const int rowc = live ? row : a.n - 1; /* a quad's rows past n load row n - 1 and write nothing */

    const bool is_q = a.fused && head < a.hq;
    const int kv = a.fused ? head - a.hq : head; /* [0, hkv) k, [hkv, 2 hkv) v */
    const bool is_v = !is_q && kv >= a.hkv;
    const int h = is_v ? kv - a.hkv : kv;

    /* the row's 256 bytes first: their round trip overlaps the position and page lookups */
    const bf16_t *x;
    if (a.fused)
        x = a.qkv + (size_t)rowc * a.row_stride + (size_t)head * NC_HEAD_DIM;
    else
        x = (is_v ? a.v_rows : a.k_rows) + (size_t)rowc * a.row_stride + (size_t)h * NC_HEAD_DIM;
    float x1[8], x2[8];
    load_bf16x8(x + 8 * g, x1);
    load_bf16x8(x + NC_HALF + 8 * g, x2);

    const int p = a.pos[rowc], s = a.seq[rowc];
    if (live && a.ctx_out && head == 0 && g == 0) a.ctx_out[row] = p + 1; /* never aliases pos (host check) */
    bool ok = live && p >= 0 && s >= 0 && s < a.num_seqs;
    if (a.fused) ok = ok && p < a.rope_len;
    const int blk = ok ? lookup_block(a.block_table, a.max_blocks, a.num_blocks, s, p / NC_PAGE) : -1;
    const int t = p % NC_PAGE;

    if (!is_v) {
        if (is_q && !live) return;
        if (is_q && !ok) {
            const u32x4 nan = {0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u};
            bf16_t *y = a.q_out + ((size_t)row * a.hq + head) * NC_HEAD_DIM;
            *reinterpret_cast<u32x4 *>(y + 8 * g) = nan;
            *reinterpret_cast<u32x4 *>(y + NC_HALF + 8 * g) = nan;
            return;
        }
        if (!is_q && blk < 0) return;
        if (a.fused) {
            const float *gain = is_q ? a.q_gain : a.k_gain;
            float g1[8], g2[8], c[8], sn[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                g1[e] = gain[8 * g + e];
                g2[e] = gain[NC_HALF + 8 * g + e];
                c[e] = a.cos[(size_t)p * NC_HALF + 8 * g + e];
                sn[e] = a.sin[(size_t)p * NC_HALF + 8 * g + e];
            }
            row_norm_rope(x1, x2, g1, g2, c, sn);
        }
        if (is_q) {
            bf16_t *y = a.q_out + ((size_t)row * a.hq + head) * NC_HEAD_DIM;
            store_bf16x8(y + 8 * g, x1);
            store_bf16x8(y + NC_HALF + 8 * g, x2);
            return;
        }
        uint64_t c1, c2;
        const float scale = row_quantize(x1, x2, &c1, &c2);
        uint8_t *tile = a.cache + tile_offset(blk, h, a.hkv);
        write_codes(tile, t, g, c1, c2, false);
        if (g == 0) reinterpret_cast<float *>(tile + NC_TILE_KS)[t] = scale;
        return;
    }

    /* v: every item of the quad is here (one head per quad), so the exchanges below see all four */
    uint64_t c1, c2;
    const float scale = row_quantize(x1, x2, &c1, &c2);
    /* the quad is whole when its 4 rows name the same block and position quad, row r at position 4 q + r */
    const int qb = blk >= 0 && (p & 3) == r ? blk : -1, qp = p >> 2;
    const bool whole = quad_min(qb) >= 0 && quad_min(qb) == quad_max(qb) && quad_min(qp) == quad_max(qp);
    const uint32_t d0 = quad_transpose((uint32_t)c1, r), d1 = quad_transpose((uint32_t)(c1 >> 32), r);
    const uint32_t d2 = quad_transpose((uint32_t)c2, r), d3 = quad_transpose((uint32_t)(c2 >> 32), r);
    if (blk < 0) return;
    uint8_t *tile = a.cache + tile_offset(blk, h, a.hkv);
    if (whole) {
        /* dims 8g + r, 8g + 4 + r and their partners 64 apart: one dword of 4 keys each */
        const int t0 = t & ~3;
        *reinterpret_cast<uint32_t *>(tile + v_byte(t0, 8 * g + r)) = d0;
        *reinterpret_cast<uint32_t *>(tile + v_byte(t0, 8 * g + 4 + r)) = d1;
        *reinterpret_cast<uint32_t *>(tile + v_byte(t0, NC_HALF + 8 * g + r)) = d2;
        *reinterpret_cast<uint32_t *>(tile + v_byte(t0, NC_HALF + 8 * g + 4 + r)) = d3;
    } else {
        write_codes(tile, t, g, c1, c2, true);
    }
    if (g == 0) reinterpret_cast<float *>(tile + NC_TILE_VS)[t] = scale;
}

static int check_cache_args(int n, int hkv, int max_blocks, int num_blocks, int num_seqs, const void *cache,
                            const void *block_table) {
    NC_REQUIRE(n >= 0, "n = %d < 0", n);
    NC_REQUIRE(hkv > 0, "hkv = %d must be positive", hkv);
    NC_REQUIRE(max_blocks > 0 && num_blocks > 0 && num_seqs > 0, "max_blocks %d, num_blocks %d, num_seqs %d must "
               "be positive", max_blocks, num_blocks, num_seqs);
    NC_REQUIRE(block_table || (long long)num_seqs * max_blocks <= num_blocks,
               "contiguous cache: %d sequences x %d blocks exceed the %d blocks", num_seqs, max_blocks, num_blocks);
    NC_REQUIRE(cache, "null cache pointer");
    NC_REQUIRE((uintptr_t)cache % 16 == 0, "cache must be 16-byte aligned");
    return 0;
}

static void launch_append(const AppendArgs &a, hipStream_t stream) {
    const int heads = a.fused ? a.hq + 2 * a.hkv : 2 * a.hkv;
    const long long items = (((long long)a.n + 3) / 4) * heads * 4; /* whole quads of rows */
    if (items == 0) return;
    const unsigned blocks = (unsigned)((items + ITEMS_PER_BLOCK - 1) / ITEMS_PER_BLOCK);
    hipLaunchKernelGGL(k_append, dim3(blocks), dim3(APPEND_THREADS), 0, stream, a);
    NC_LAUNCH_CHECK();
}

extern "C" int nc_kv_append_fp8(const void *qkv, long long row_stride, int n, const int32_t *pos,
                                const int32_t *seq, const float *q_gain, const float *k_gain, const float *cos,
                                const float *sin, int rope_len, int hq, int hkv, void *q_out, uint8_t *cache,
                                const int32_t *block_table, int max_blocks, int num_blocks, int num_seqs,
                                int32_t *ctx_out, void *stream) {
    int rc = check_cache_args(n, hkv, max_blocks, num_blocks, num_seqs, cache, block_table);
    if (rc) return rc;
    NC_REQUIRE(hq > 0 && hq % hkv == 0, "hq = %d must be a positive multiple of hkv = %d", hq, hkv);
    NC_REQUIRE(row_stride >= (long long)(hq + 2 * hkv) * NC_HEAD_DIM && row_stride % 8 == 0,
               "row_stride %lld must hold (hq + 2 hkv) * 128 elements and keep 16-byte alignment", row_stride);
    NC_REQUIRE(rope_len > 0, "rope_len = %d", rope_len);
    NC_REQUIRE(n == 0 || (qkv && pos && seq && q_gain && k_gain && cos && sin && q_out), "null argument");
    NC_REQUIRE(((uintptr_t)qkv | (uintptr_t)q_out) % 16 == 0, "qkv and q_out must be 16-byte aligned");
    NC_REQUIRE(!ctx_out || ctx_out + n <= pos || pos + n <= ctx_out, "ctx_out must not overlap pos");
    AppendArgs a = {};
    a.qkv = (const bf16_t *)qkv; a.row_stride = row_stride; a.n = n; a.pos = pos; a.seq = seq;
    a.q_gain = q_gain; a.k_gain = k_gain; a.cos = cos; a.sin = sin; a.rope_len = rope_len;
    a.hq = hq; a.hkv = hkv; a.q_out = (bf16_t *)q_out; a.ctx_out = ctx_out;
    a.cache = cache;
    a.block_table = block_table; a.max_blocks = max_blocks; a.num_blocks = num_blocks; a.num_seqs = num_seqs;
    a.fused = 1;
    launch_append(a, (hipStream_t)stream);
    return 0;
}

extern "C" int nc_kv_store_fp8(const void *k, const void *v, long long row_stride, int n, const int32_t *pos,
                               const int32_t *seq, int hkv, uint8_t *cache, const int32_t *block_table,
                               int max_blocks, int num_blocks, int num_seqs, void *stream) {
    int rc = check_cache_args(n, hkv, max_blocks, num_blocks, num_seqs, cache, block_table);
    if (rc) return rc;
    NC_REQUIRE(row_stride >= (long long)hkv * NC_HEAD_DIM && row_stride % 8 == 0,
               "row_stride %lld must hold hkv * 128 elements and keep 16-byte alignment", row_stride);
    NC_REQUIRE(n == 0 || (k && v && pos && seq), "null argument");
    NC_REQUIRE(((uintptr_t)k | (uintptr_t)v) % 16 == 0, "k and v must be 16-byte aligned");
    AppendArgs a = {};
    a.k_rows = (const bf16_t *)k; a.v_rows = (const bf16_t *)v; a.row_stride = row_stride; a.n = n;
    a.pos = pos; a.seq = seq; a.hkv = hkv;
    a.cache = cache;
    a.block_table = block_table; a.max_blocks = max_blocks; a.num_blocks = num_blocks; a.num_seqs = num_seqs;
    a.fused = 0;
    launch_append(a, (hipStream_t)stream);
    return 0;
}

/* ------------------------------------------------------------------------------------------ qkp_forward */

/* Training-layout prologue: q, k are (B, T, H, 128) column blocks of the fused projection (token stride 3 H 128);
 * outputs contiguous (B, T, H, 128); position of token p is p % T; items [0, rows) q, [rows, 2 rows) k. */
__global__ void __launch_bounds__(APPEND_THREADS) k_qk_prologue(const bf16_t *q, const bf16_t *k, const float *gq,
                                                                const float *gk, bf16_t *qo, bf16_t *ko,
                                                                const float *cos, const float *sin, long long rows,
                                                                int H, int T) {
    const long long item = (long long)blockIdx.x * ITEMS_PER_BLOCK + threadIdx.x / NC_ROW_LANES;
    if (item >= 2 * rows) return;
    const int g = threadIdx.x % NC_ROW_LANES;
    const bool is_q = item < rows;
    const long long r = is_q ? item : item - rows;
    const long long token = r / H;
    const int head = (int)(r % H), p = (int)(token % T);
    const bf16_t *x = (is_q ? q : k) + token * 3 * H * NC_HEAD_DIM + (long long)head * NC_HEAD_DIM;
    const float *gain = is_q ? gq : gk;
    float x1[8], x2[8], g1[8], g2[8], c[8], sn[8];
    load_bf16x8(x + 8 * g, x1);
    load_bf16x8(x + NC_HALF + 8 * g, x2);
#pragma unroll
    for (int e = 0; e < 8; e++) {
        g1[e] = gain[8 * g + e];
        g2[e] = gain[NC_HALF + 8 * g + e];
        c[e] = cos[(size_t)p * NC_HALF + 8 * g + e];
        sn[e] = sin[(size_t)p * NC_HALF + 8 * g + e];
    }
    row_norm_rope(x1, x2, g1, g2, c, sn);
    bf16_t *y = (is_q ? qo : ko) + r * NC_HEAD_DIM;
    store_bf16x8(y + 8 * g, x1);
    store_bf16x8(y + NC_HALF + 8 * g, x2);
}

/* model/kernels/qk_prologue.cu:111-118: same arguments and meaning (rows = B T H; cos, sin [T][64] fp32). */
extern "C" void qkp_forward(const void *q, const void *k, const void *gq, const void *gk, void *qo, void *ko,
                            const void *cos, const void *sin, long long rows, int H, int T, void *stream) {
    if (rows <= 0) return;
    const unsigned blocks = (unsigned)((2 * rows + ITEMS_PER_BLOCK - 1) / ITEMS_PER_BLOCK);
    hipLaunchKernelGGL(k_qk_prologue, dim3(blocks), dim3(APPEND_THREADS), 0, (hipStream_t)stream,
                       (const bf16_t *)q, (const bf16_t *)k, (const float *)gq, (const float *)gk, (bf16_t *)qo,
                       (bf16_t *)ko, (const float *)cos, (const float *)sin, rows, H, T);
    NC_LAUNCH_CHECK();
}

/* ------------------------------------------------------------------------------------------ gather */

/* One 256-thread workgroup per (16-position tile, kv head, sequence): thread (t = tid / 16, c = tid % 16) moves
 * 8 bytes of key t's K row and V row (dims 8c..8c+7) to the canonical layout; positions past ctx_len are zeroed. */
__global__ void __launch_bounds__(256) k_gather(const uint8_t *cache, const int32_t *block_table, int max_blocks,
                                                int num_blocks, const int32_t *ctx_len, int hkv, int max_ctx,
                                                uint8_t *k_out, uint8_t *v_out, float *ks_out, float *vs_out) {
    const int page = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int t = threadIdx.x / 16, c = threadIdx.x % 16;
    const int pos = page * NC_PAGE + t;
    if (pos >= max_ctx) return;
    const int ctx = ctx_len[b];
    const int blk = pos < ctx ? lookup_block(block_table, max_blocks, num_blocks, b, page) : -1;
    uint64_t kw = 0, vw = 0;
    float ks = 0.0f, vs = 0.0f;
    if (blk >= 0) {
        const uint8_t *tile = cache + tile_offset(blk, h, hkv);
        kw = *reinterpret_cast<const uint64_t *>(tile + k_byte(t, 8 * c));
#pragma unroll
        for (int e = 0; e < 8; e++) vw |= (uint64_t)tile[v_byte(t, 8 * c + e)] << (8 * e);
        ks = reinterpret_cast<const float *>(tile + NC_TILE_KS)[t];
        vs = reinterpret_cast<const float *>(tile + NC_TILE_VS)[t];
    }
    const size_t row = ((size_t)b * hkv + h) * max_ctx + pos;
    *reinterpret_cast<uint64_t *>(k_out + row * NC_HEAD_DIM + 8 * c) = kw;
    *reinterpret_cast<uint64_t *>(v_out + row * NC_HEAD_DIM + 8 * c) = vw;
    if (c == 0) {
        ks_out[row] = ks;
        vs_out[row] = vs;
    }
}

extern "C" int nc_kv_gather_fp8(const uint8_t *cache, const int32_t *block_table, int max_blocks, int num_blocks,
                                const int32_t *ctx_len, int B, int hkv, int max_ctx, uint8_t *k_out, uint8_t *v_out,
                                float *ks_out, float *vs_out, void *stream) {
    int rc = check_cache_args(B, hkv, max_blocks, num_blocks, B > 0 ? B : 1, cache, block_table);
    if (rc) return rc;
    NC_REQUIRE(max_ctx >= 0 && max_ctx <= max_blocks * NC_PAGE, "max_ctx %d outside [0, %d]", max_ctx,
               max_blocks * NC_PAGE);
    if (B == 0 || max_ctx == 0) return 0;
    NC_REQUIRE(ctx_len && k_out && v_out && ks_out && vs_out, "null argument");
    const dim3 grid((max_ctx + NC_PAGE - 1) / NC_PAGE, hkv, B);
    hipLaunchKernelGGL(k_gather, grid, dim3(256), 0, (hipStream_t)stream, cache, block_table, max_blocks,
                       num_blocks, ctx_len, hkv, max_ctx, k_out, v_out, ks_out, vs_out);
    NC_LAUNCH_CHECK();
    return 0;
}
