/*
 * Split-K flash-decode over the fp8 paged cache (reference: k_attn, model/kernels/decode.cu:567-675, which reads a
 * bf16 contiguous cache with one block per (head, slot) and no split).
 *
 * Schedule: a persistent grid of W single-wave workgroups (the device's resident capacity). The work is the
 * flattened list of (sequence b, kv head h, page) triples over every sequence's key range [max(p - window, 0), p]
 * (p = ctx_len - 1; the query's own key, appended first, is read back from the cache). Each wave takes an equal
 * contiguous slice of it, computed in the kernel from the live context lengths, so a ragged batch stays balanced.
 * A slice is processed as pieces, one per segment (b, h) it touches. All G = Hq / Hkv query heads of a kv head
 * ride in the same wave, so every fp8 byte is read from HBM once.
 * The piece plan (nc_decode_step_fp8_pieces) instead cuts every segment into fixed pieces set by its own length
 * (piece_len) and rounds the slice ends to piece boundaries, so a sequence's bits do not depend on the batch.
 *
 * Per page (16 keys) a wave computes
 *   scores  Sᵀ[16 keys][16 heads] = K[16][128] · Qᵀ, 4 v_mfma_f32_16x16x32_bf16. A is the K tile as loaded (lane:
 *           key lane%16, dims 32 (lane/16) .. + 31, its fragments of the tile's parts 0 and 1), fp8 -> bf16 exact by
 *           v_cvt_scalef32_pk_bf16_fp8; B is q (bf16), head = lane%16 (zero past G). Lane (j = lane/16,
 *           n = lane%16) receives keys 4j..4j+3 for head n.
 *   softmax fp32, base 2 (scores times k_scale · sm_scale · log2 e). The reference max m of a head moves only
 *           when a score exceeds it by more than 8 (a rare wave-uniform branch that rescales), so p <= 2^8 and the
 *           steady state has no cross-lane traffic; sums stay per lane until the end.
 *   values  Oᵀ[16 dims][16 heads] += Vᵀ[16 dims][16 keys] · Pᵀ, 8 v_mfma_f32_16x16x16_f16. Pᵀ is the lane's own
 *           4 probabilities times v_scale times 2^(126 - e_ref), e_ref the largest v_scale exponent seen (so the
 *           factor is <= 256 and fits fp16 with 11-bit precision; bf16 probabilities measurably miss the
 *           benchmark's max-error bound on outlier data). Vᵀ comes straight from the quad-transposed V tile:
 *           lane (j, n) holds the 32 bytes of dims 8n..8n+7 for keys 4j..4j+3 (its fragments of parts 2 and 3);
 *           dword bb is one MFMA's A operand.
 *           The accumulator lane holds head n, so rescales are lane-local.
 * DEC_DEPTH page buffers rotate in registers (DEC_DEPTH - 1 pages in flight while one is computed), one wave per
 * SIMD: with two, the older wave wins issue arbitration and the younger finishes its equal share ~1.6x later. A
 * page is six nontemporal loads per lane; each code load of the wave reads one contiguous 1 KiB part of the tile.
 *
 * A piece covering its whole segment writes the normalised bf16 output. Otherwise it writes (Σ p v, max, sum) to a
 * workspace slot, and k_merge, launched next, combines a segment's slots with weights exp2(m_s - max m)
 * (decode.cu:547-548's rescale). The merge is a second kernel on purpose: the eight XCDs' L2 caches are not
 * coherent with each other, so a piece's partials reach a merging wave on another XCD only through device-scope
 * (write-through) stores, whose acknowledgements the in-order memory counter puts ahead of the next pages' loads.
 * An in-kernel merge built that way (the last piece to arrive at a per-segment counter merges) was measured: about
 * 3 µs slower per config-3 call with the partials written as they finish, 1 µs slower with them held in registers
 * until the end of the wave, than this launch.
 *
 * The fused step (nc_decode_step_fp8) is the append and the attention of a decode step in these two launches
 * instead of three (reference: k_prologue's append, decode.cu:550-565, then k_attn). Every piece builds its q
 * rows from the projection (QK-norm, gain, RoPE, the row math of k_append, so bit-identical) while its first pages
 * load, and the piece that ends a segment also quantises the new key and value (after its first page, off the
 * critical path), patches them into its registers for the last page and stores them in the cache after its pages:
 * that page is read by no other wave, so the new key needs no ordering between waves.
 *
 * Roofline: HBM. Per (token, kv head) the kernel reads 128 B of K, 128 B of V and two fp32 scales: 264 B.
 */
#include <algorithm>

#include "decode_scratch.h"
#include "layout.h"
#include "qk_row.h"


#define DEC_THREADS 64
#define DEC_MAX_G 16
#define DEC_MAX_WAVES 8192  /* workspace slots are sized for this many waves */
#define DEC_MERGE_DIRECT 8  /* pieces of a segment k_merge reads in its first round trip */
#define DEC_PIECES_MIN 32   /* fixed pieces of a segment at most: this many ... */
#define DEC_PIECES_MAX 256  /* ... or, for longer contexts, enough for 16-page pieces, up to this many */
#define DEC_MIN_CHUNK 8     /* pages per wave at least: fewer pieces to merge on small problems */
#define DEC_LAZY 8.0f       /* log2 headroom before the softmax reference moves */
#define DEC_M_INIT -3.0e38f /* finite "no score yet": exp2(m - m') = 0, never NaN */
#define DEC_DEPTH 4         /* page buffers per wave: 3 pages (12.4 KiB) in flight while one is computed */
/* DEC_DEPTH 4 is the depth built and tested. The ring's rotation and clamped loads work for any depth, and 5 or 6
 * buffers fit in registers at one wave per SIMD, but measured 1-2 us slower per call on configs 2, 3 and 5. */
static_assert(DEC_DEPTH == 4, "the page ring is 4 buffers deep");

/* Schedule units (page equivalents, measured on config 3 by sweeping these values) of a piece start (the
 * segment's context length and block ids: two dependent round trips) and of a segment's end (the fused step's q
 * rows and the append's quantisation; the same in both entry points, so that they split the work alike and give
 * bit-identical outputs). */
#ifndef DEC_UNITS_START
#define DEC_UNITS_START 3
#endif
#ifndef DEC_UNITS_END
#define DEC_UNITS_END 10
#endif
#ifndef DEC_WAVES_PER_SIMD
#define DEC_WAVES_PER_SIMD 1 /* one wave per SIMD: no older/younger wave competing for issue on a SIMD */
#endif

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

struct DecodeArgs {
    const bf16_t *q;          /* [B][hq][128] */
    uint8_t *cache;           /* [num_blocks][hkv][4224] tiles; written only by the fused step's append */
    const int32_t *block_table;
    int max_blocks, num_blocks;
    const int32_t *ctx_len;   /* [B]; the fused step: the positions */
    /* the fused step: q and the new key/value come from the projection rows (null: q is given) */
    const bf16_t *qkv;        /* [B][row_stride]: hq q heads, hkv k heads, hkv v heads */
    long long row_stride;
    const float *q_gain, *k_gain; /* [128] */
    const float *cos, *sin;   /* [rope_len][64] */
    int rope_len;
    int32_t *pos_out;         /* optional [B]: pos + 1, the next step's positions (never aliases the positions) */
    int window;               /* keys before the query; < 0: all */
    int B, hq, hkv, group;
    float score_scale;        /* sm_scale * log2(e) */
    bf16_t *out;              /* [B][hq][128] */
    float *ws_o;              /* [slots][group][128]: the pieces' Σ p v (slot layout at merge_slot) */
    float *ws_ml;             /* [slots][group][2]: their max and sum */
    int2 *ws_desc;            /* [S]: each segment's piece count and first piece's wave */
    int max_ctx;              /* ctx_len is clamped to it */
    int unit_start, unit_end; /* schedule units a non-empty segment costs before its first and after its last page */
    int piece_pages;          /* 0: pieces cut by the balanced split; > 0: fixed pieces (piece_len) */
    int piece_slots;          /* fixed pieces: the most pieces of a segment (piece_slots_for), its slots apart */
    int merge_groups;         /* k_merge's groups of 16 G lanes per segment */
};

/* The key range of sequence b: pages [first, last] (none if last < first), keys [begin, p]. */
struct SeqRange {
    int first, last, begin, p;
};

/* The context length of a sequence whose ctx_len entry is v: v clamped to [0, max_ctx]. The fused step's entry is
 * a position p, giving p + 1, 0 for p < 0, and -1 (no append, a NaN output row) for p at or past max_ctx or
 * rope_len. */
__device__ __forceinline__ int seq_ctx_of(const DecodeArgs &a, int v) {
    if (!a.qkv) return max(min(v, a.max_ctx), 0);
    if (v < 0) return 0;
    return (v >= a.max_ctx || v >= a.rope_len) ? -1 : v + 1;
}

/* seq_ctx_of sequence b's entry. */
__device__ __forceinline__ int seq_ctx(const DecodeArgs &a, int b) { return seq_ctx_of(a, a.ctx_len[b]); }

/* The key range of a sequence of context length ctx (seq_ctx). */
__device__ __forceinline__ SeqRange seq_range_of(const DecodeArgs &a, int ctx) {
    SeqRange r;
    if (ctx <= 0) {
        r.first = 0, r.last = -1, r.begin = 0, r.p = -1;
        return r;
    }
    r.p = ctx - 1;
    r.begin = (a.window < 0 || r.p <= a.window) ? 0 : r.p - a.window;
    r.first = r.begin / NC_PAGE;
    r.last = r.p / NC_PAGE;
    return r;
}

__device__ __forceinline__ int pages_of(const DecodeArgs &a, int ctx) {
    const SeqRange r = seq_range_of(a, ctx);
    return r.last - r.first + 1;
}

/* Schedule units of one segment of a sequence of context length ctx: its pages plus the fixed costs of starting a
 * piece there and of ending the segment (the fused step's append), in page equivalents, so that the waves that
 * carry them get fewer pages; an empty sequence costs nothing. */
__device__ __forceinline__ int units_of(const DecodeArgs &a, int ctx) {
    const int pg = pages_of(a, ctx);
    return pg > 0 ? pg + a.unit_start + a.unit_end : 0;
}

/* Fixed pieces: a segment of `pages` pages is cut into pieces of max(piece_pages, ceil(pages / piece_slots)) pages
 * from its first page on (at most piece_slots pieces, each with its own workspace slot). A function of the segment's
 * own length and of max_ctx (piece_slots_for) only: its output bits do not depend on the batch. */
__device__ __forceinline__ int piece_len(const DecodeArgs &a, int pages) {
    return max(a.piece_pages, (pages + a.piece_slots - 1) / a.piece_slots);
}

/* A k_decode wave's context lengths: seq_ctx of every sequence, in LDS when the batch fits (read from memory once
 * per wave, in schedule_total), else from memory each time. */
#define DEC_LDS_SEQS 2048

__device__ __forceinline__ int ctx_at(const DecodeArgs &a, const int *lds, int b) {
    return lds ? lds[b] : seq_ctx(a, b);
}

/* The contexts a k_decode wave schedules from. A batch of at most 64 stays in registers: lane l holds sequence l's
 * context, schedule units and inclusive unit sum, read back by readlane; a larger batch keeps its contexts in LDS
 * (lds, up to DEC_LDS_SEQS) or reads them from memory. */
struct Ctx {
    const int *lds;
    int c, units, incl;
    bool regs;
};

__device__ __forceinline__ int ctx_of(const DecodeArgs &a, const Ctx &cx, int b) {
    return cx.regs ? __builtin_amdgcn_readlane(cx.c, b) : ctx_at(a, cx.lds, b);
}

/* The inclusive prefix sum of v over the wave's 64 lanes. */
__device__ __forceinline__ int wave_inclusive_sum(int v, int lane) {
    (void)lane; /* DPP: row_shr 1, 2, 4, 8 inside each 16-lane row, then row_bcast15 / row_bcast31 across rows */
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false); /* row 0's total into row 1, row 2's into 3 */
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false); /* rows 0-1's total into rows 2 and 3 */
    return v;
}

/* 8 fp8 codes (two dwords, byte order = element order) -> 8 bf16, exact. */
__device__ __forceinline__ bf16x8 fp8x8_to_bf16(uint32_t w0, uint32_t w1) {
    const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false);
    const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true);
    const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false);
    const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true);
    return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

/* 4 fp8 codes -> 4 fp16, exact (every e4m3fn value is an fp16 value). */
__device__ __forceinline__ f16x4 fp8x4_to_f16(uint32_t w) {
    const f16x2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false);
    const f16x2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true);
    return f16x4{a[0], a[1], b[0], b[1]};
}

/* 2^e as fp32 for e in [-126, 127] (exponent bits only). */
__device__ __forceinline__ float exp2i(int e) { return __uint_as_float((uint32_t)(e + 127) << 23); }

/* One page's fragments for this lane: K row bytes, V quad bytes, the 4 keys' scales, and the block (-1: none). */
struct Page {
    u32x4 k0, k1, v0, v1;
    f32x4 ks, vs;
    int blk;
};

/* Each code load reads one 1 KB part of the tile, the lanes' fragments in lane order. The loads are nontemporal:
 * a page is read once per step, and streamed this way a cold cache moves about 12 % faster than with plain loads
 * (the 256 MB memory-side cache cannot hold a model's cache between two steps of a layer anyway). */
__device__ __forceinline__ void load_page(const DecodeArgs &a, int blk, int h, int n, int j, Page &pg) {
    pg.blk = blk;
    const int at = blk < 0 ? 0 : blk;
    const uint8_t *tile = a.cache + tile_offset(at, h, a.hkv);
    const uint8_t *fp = tile + (n + 16 * j) * 16;
    pg.k0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(fp));
    pg.k1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(fp + NC_TILE_PART));
    pg.v0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(fp + 2 * NC_TILE_PART));
    pg.v1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(fp + 3 * NC_TILE_PART));
    pg.ks = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(tile + NC_TILE_KS + 16 * j));
    pg.vs = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(tile + NC_TILE_VS + 16 * j));
}

/* The online-softmax state of one piece, lane (j, n): head n's reference max m, this lane's partial sum l, the
 * v_scale exponent reference and Oᵀ (dims (4j + i) * 8 + bb of head n in o[bb][i], units 2^(e_ref - 126)). */
struct State {
    f32x4 o[8];
    float m, l, w, vlim;
    int e_ref;
};

__device__ __forceinline__ void state_init(State &st) {
#pragma unroll
    for (int bb = 0; bb < 8; bb++) st.o[bb] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.m = DEC_M_INIT;
    st.l = 0.f;
    st.e_ref = 0;
    st.w = exp2i(126);
    st.vlim = exp2i(-126);
}

/* The fused step's new key and value (codes and scales in LDS, key t = p % 16 of the last page): t >= 0 when
 * the piece appends. */
/* Staged partial results: a piece that is a part of its segment leaves (Σ p v, max, sum) here, not in the
 * workspace, while the wave still streams pages: stores issued between page loads hold up those loads' waits (the
 * memory counter completes in order; measured: 10 µs on a config-5 layer cut into 8 pieces per segment). They go
 * to the workspace when the stage is full and at the end of the wave. */
#define DEC_PART_FLOATS 6144 /* 24 KB: pieces of G (128 + 2) floats each, 11 at G = 4, 2 at G = 16 */
#define DEC_PART_MAX 32

struct StepLds {
    bf16_t q[DEC_MAX_G][NC_HEAD_DIM];
    uint8_t codes[2][NC_HEAD_DIM]; /* new key, new value */
    float scale[2];
    int blk;                       /* their block, -1: none */
    int part_slot[DEC_PART_MAX];   /* their merge slots */
    float part[DEC_PART_FLOATS];   /* piece i at i G 130: o [G][128] (value units), then (max, sum) [G][2] */
};

/* Put the new key and value into a page loaded before they were stored: lane (j, n) holds K row n, dims 32 j..,
 * and the V codes of dims 8 n.. for keys 4 j..4 j + 3. */
__device__ __forceinline__ void apply_patch(Page &pg, const StepLds &sm, int t, int n, int j) {
    if (n == t) {
        pg.k0 = *reinterpret_cast<const u32x4 *>(&sm.codes[0][32 * j]);
        pg.k1 = *reinterpret_cast<const u32x4 *>(&sm.codes[0][32 * j + 16]);
    }
    if (j == (t >> 2)) {
        const u32x2 v = *reinterpret_cast<const u32x2 *>(&sm.codes[1][8 * n]);
        const int sh = 8 * (t & 3);
        const uint32_t keep = ~(0xffu << sh);
#pragma unroll
        for (int bb = 0; bb < 4; bb++) {
            pg.v0[bb] = (pg.v0[bb] & keep) | (((v[0] >> (8 * bb)) & 0xffu) << sh);
            pg.v1[bb] = (pg.v1[bb] & keep) | (((v[1] >> (8 * bb)) & 0xffu) << sh);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            pg.ks[i] = i == (t & 3) ? sm.scale[0] : pg.ks[i];
            pg.vs[i] = i == (t & 3) ? sm.scale[1] : pg.vs[i];
        }
    }
}

/* Attend one page: pg its page number in the sequence. */
__device__ __forceinline__ void attend_page(const DecodeArgs &a, Page pg, int page, const SeqRange &sr,
                                            const bf16x8 *qop, int lane, int patch_t, const StepLds &sm, State &st) {
    const int j = lane >> 4;
    if (patch_t >= 0 && page == sr.last) apply_patch(pg, sm, patch_t, lane & 15, j);
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16(pg.k0[0], pg.k0[1]), qop[0], s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16(pg.k0[2], pg.k0[3]), qop[1], s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16(pg.k1[0], pg.k1[1]), qop[2], s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16(pg.k1[2], pg.k1[3]), qop[3], s, 0, 0, 0);
    float x[4], vs[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        x[i] = s[i] * (pg.ks[i] * a.score_scale);
        vs[i] = pg.vs[i];
    }
    /* partial pages (window start, the last key, a missing block) mask keys outside [begin, p] */
    const bool partial = pg.blk < 0 || (page == sr.first && (sr.begin & (NC_PAGE - 1))) ||
                         (page == sr.last && (sr.p & (NC_PAGE - 1)) != NC_PAGE - 1);
    if (partial) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int key = page * NC_PAGE + 4 * j + i;
            const bool ok = pg.blk >= 0 && key >= sr.begin && key <= sr.p;
            x[i] = ok ? x[i] : -INFINITY;
            vs[i] = ok ? vs[i] : 0.f;
        }
    }
    const float xm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    if (__any(xm > st.m + DEC_LAZY)) { /* rare: move the reference max to the exact max, rescale */
        float mx = fmaxf(xm, shfl_xor_f(xm, 16));
        mx = fmaxf(mx, shfl_xor_f(mx, 32));
        const float m_new = fmaxf(st.m, mx);
        const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
        st.l *= alpha;
#pragma unroll
        for (int bb = 0; bb < 8; bb++) st.o[bb] *= alpha;
        st.m = m_new;
    }
    const float vm = fmaxf(fmaxf(vs[0], vs[1]), fmaxf(vs[2], vs[3]));
    if (__any(vm >= st.vlim)) { /* rare: a larger v_scale exponent, rescale the units of o */
        float vx = fmaxf(vm, shfl_xor_f(vm, 16));
        vx = fmaxf(vx, shfl_xor_f(vx, 32));
        const int e_new = max(st.e_ref, (int)(__float_as_uint(vx) >> 23));
        const float r = exp2i(max(st.e_ref - e_new, -126));
#pragma unroll
        for (int bb = 0; bb < 8; bb++) st.o[bb] *= r;
        st.e_ref = e_new;
        st.w = exp2i(max(126 - e_new, -126));
        st.vlim = exp2i(min(e_new - 126, 127));
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = __builtin_amdgcn_exp2f(x[i] - st.m);
    st.l += (p[0] + p[1]) + (p[2] + p[3]);
    const f16x4 pp = {(_Float16)(p[0] * (vs[0] * st.w)), (_Float16)(p[1] * (vs[1] * st.w)),
                      (_Float16)(p[2] * (vs[2] * st.w)), (_Float16)(p[3] * (vs[3] * st.w))};
#pragma unroll
    for (int bb = 0; bb < 8; bb++) {
        const uint32_t vd = bb < 4 ? pg.v0[bb] : pg.v1[bb - 4];
        st.o[bb] = __builtin_amdgcn_mfma_f32_16x16x16f16(fp8x4_to_f16(vd), pp, st.o[bb], 0, 0, 0);
    }
}

/* ------------------------------------------------------------------------------------------ fused step rows */

#define DEC_Q_PASSES ((DEC_MAX_G + 7) / 8) /* 8-lane rows per wave pass: the G q heads */

/* A piece's q rows in the 8-lane row layout of qk_row.h (lane g = lane % 8 holds dims [8g, 8g + 8) and
 * [64 + 8g, 64 + 8g + 8)): row ri = 8 pass + lane / 8 is q head h G + ri for ri < G; with the q gains and the
 * position's rotation table entries. Loaded after the block ids, so the page loads wait for the ids alone. */
struct QRows {
    u32x4 lo[DEC_Q_PASSES], hi[DEC_Q_PASSES];
    f32x4 qg[4], cs[2], sn[2];
};

/* The appending piece's new key and value rows (lanes 0-7: the k head, lanes 8-15: the v head; the other lanes
 * repeat the k head), the k gains and the new key's block (table entry, unchecked). */
struct KvRows {
    u32x4 lo, hi;
    f32x4 kg[4];
    int blk;
};

__device__ __forceinline__ void load_qrows(const DecodeArgs &a, int b, int h, int p, int lane, QRows &qr) {
    const int g = lane & 7, G = a.group;
    const bf16_t *row = a.qkv + (size_t)b * a.row_stride;
#pragma unroll
    for (int ps = 0; ps < DEC_Q_PASSES; ps++) {
        const int ri = min(8 * ps + (lane >> 3), G - 1); /* unused rows read a valid one */
        const u32x4 *src = reinterpret_cast<const u32x4 *>(row + (size_t)(h * G + ri) * NC_HEAD_DIM);
        qr.lo[ps] = src[g];
        qr.hi[ps] = src[8 + g];
    }
    const f32x4 *qg = reinterpret_cast<const f32x4 *>(a.q_gain);
    const f32x4 *cp = reinterpret_cast<const f32x4 *>(a.cos + (size_t)p * NC_HALF);
    const f32x4 *sp = reinterpret_cast<const f32x4 *>(a.sin + (size_t)p * NC_HALF);
#pragma unroll
    for (int i = 0; i < 2; i++) {
        qr.qg[i] = qg[2 * g + i];
        qr.qg[2 + i] = qg[16 + 2 * g + i];
        qr.cs[i] = cp[2 * g + i];
        qr.sn[i] = sp[2 * g + i];
    }
}

template <bool TABLE>
__device__ __forceinline__ void load_kvrows(const DecodeArgs &a, int b, int h, int p, int lane, KvRows &kr) {
    const int g = lane & 7;
    const int head = (lane >> 3) == 1 ? a.hq + a.hkv + h : a.hq + h;
    const u32x4 *src = reinterpret_cast<const u32x4 *>(a.qkv + (size_t)b * a.row_stride + (size_t)head * NC_HEAD_DIM);
    kr.lo = src[g];
    kr.hi = src[8 + g];
    const f32x4 *kg = reinterpret_cast<const f32x4 *>(a.k_gain);
#pragma unroll
    for (int i = 0; i < 2; i++) {
        kr.kg[i] = kg[2 * g + i];
        kr.kg[2 + i] = kg[16 + 2 * g + i];
    }
    /* the new key's page: p < max_ctx keeps it in the table (contiguous: computed in build_kv). The index gets a
     * zero the compiler cannot see through, so the entry stays a per-lane value: read as a uniform one it would
     * be moved to a scalar register here, and the wait for it would hold the first page loads behind every row
     * load (1 us per fused piece); only build_kv, after the first page, reads it. */
    if constexpr (TABLE) {
        int opaque_zero;
        asm volatile("v_mov_b32 %0, 0" : "=v"(opaque_zero));
        kr.blk = a.block_table[(size_t)b * a.max_blocks + p / NC_PAGE + opaque_zero];
    } else {
        kr.blk = 0;
    }
}

__device__ __forceinline__ void unpack_bf16x8(const u32x4 u, float *v) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[2 * i] = __uint_as_float(u[i] << 16);
        v[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    }
}

__device__ __forceinline__ void rope_entries(const QRows &qr, float *c, float *s) {
#pragma unroll
    for (int e = 0; e < 8; e++) {
        c[e] = qr.cs[e / 4][e % 4];
        s[e] = qr.sn[e / 4][e % 4];
    }
}

/* Norm, gain and rotate the piece's q rows (k_append's row math, so bit-identical to its q_out) into this lane's
 * MFMA operand (head n, dims 32 j..) through LDS. */
__device__ __forceinline__ void build_q(const DecodeArgs &a, const QRows &qr, int lane, bf16x8 *qop, StepLds &sm) {
    const int g = lane & 7, G = a.group;
    float c[8], s[8], g1[8], g2[8];
    rope_entries(qr, c, s);
#pragma unroll
    for (int e = 0; e < 8; e++) {
        g1[e] = qr.qg[e / 4][e % 4];
        g2[e] = qr.qg[2 + e / 4][e % 4];
    }
    __syncthreads(); /* the previous piece's reads of sm.q are done */
#pragma unroll
    for (int ps = 0; ps < DEC_Q_PASSES; ps++) {
        if (8 * ps >= G) break;
        const int ri = 8 * ps + (lane >> 3);
        if (ri >= G) continue; /* whole 8-lane rows: the row reductions stay inside active lanes */
        float x1[8], x2[8];
        unpack_bf16x8(qr.lo[ps], x1);
        unpack_bf16x8(qr.hi[ps], x2);
        row_norm_rope(x1, x2, g1, g2, c, s);
        store_bf16x8(&sm.q[ri][8 * g], x1);
        store_bf16x8(&sm.q[ri][NC_HALF + 8 * g], x2);
    }
    __syncthreads();
    const int n = lane & 15, j = lane >> 4;
#pragma unroll
    for (int cc = 0; cc < 4; cc++)
        qop[cc] = n < G ? *reinterpret_cast<const bf16x8 *>(&sm.q[n][32 * j + 8 * cc])
                        : __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
}

/* The appending piece's new key (norm, gain, rotation) and value, quantised into LDS (codes, scales, block) for
 * the last page's patch and for store_new_kv. Lanes 0-15 work, two 8-lane rows. */
__device__ __forceinline__ void build_kv(const DecodeArgs &a, int b, int p, const QRows &qr, const KvRows &kr,
                                         int lane, StepLds &sm) {
    const int g = lane & 7, is_v = lane >> 3;
    if (lane < 16) {
        float x1[8], x2[8];
        unpack_bf16x8(kr.lo, x1);
        unpack_bf16x8(kr.hi, x2);
        if (!is_v) {
            float c[8], s[8], g1[8], g2[8];
            rope_entries(qr, c, s);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                g1[e] = kr.kg[e / 4][e % 4];
                g2[e] = kr.kg[2 + e / 4][e % 4];
            }
            row_norm_rope(x1, x2, g1, g2, c, s);
        }
        uint64_t c1, c2;
        const float scale = row_quantize(x1, x2, &c1, &c2);
        *reinterpret_cast<uint64_t *>(&sm.codes[is_v][8 * g]) = c1;
        *reinterpret_cast<uint64_t *>(&sm.codes[is_v][NC_HALF + 8 * g]) = c2;
        if (g == 0) sm.scale[is_v] = scale;
        if (lane == 0) {
            const int blk = a.block_table ? kr.blk : b * a.max_blocks + p / NC_PAGE;
            sm.blk = (blk >= 0 && blk < a.num_blocks) ? blk : -1;
        }
    }
    __syncthreads(); /* the codes are in LDS before the last page's patch reads them */
}

/* The fused step's cache write of the new key and value (codes and scales from LDS, the bytes k_append writes),
 * after the piece: nothing in this kernel reads them from memory (the piece used them from LDS), and stores
 * issued before page loads would hold up those loads' waits (the memory counter completes in order). Lane l
 * writes dims 2l and 2l + 1. */
__device__ __forceinline__ void store_new_kv(const DecodeArgs &a, int h, int p, int lane, const StepLds &sm) {
    const int blk = sm.blk, t = p % NC_PAGE;
    if (blk < 0) return;
    uint8_t *tile = a.cache + tile_offset(blk, h, a.hkv);
    const int d = 2 * lane;
    *reinterpret_cast<uint16_t *>(tile + k_byte(t, d)) = *reinterpret_cast<const uint16_t *>(&sm.codes[0][d]);
    tile[v_byte(t, d)] = sm.codes[1][d];
    tile[v_byte(t, d + 1)] = sm.codes[1][d + 1];
    if (lane < 2) reinterpret_cast<float *>(tile + (lane ? NC_TILE_VS : NC_TILE_KS))[t] = sm.scale[lane];
}

/* The table entry of page `page` of sequence b (TABLE: loaded from an index clamped into the table, always in
 * bounds; contiguous: computed), and its check: the block, or -1 when the page or the block is out of range. Split
 * so that a wave can issue the entry's load, then other loads, and wait for the entry alone. */
template <bool TABLE>
__device__ __forceinline__ int block_entry(const DecodeArgs &a, int b, int page) {
    const int pc = min(max(page, 0), a.max_blocks - 1);
    if constexpr (TABLE) return a.block_table[(size_t)b * a.max_blocks + pc];
    return b * a.max_blocks + pc;
}

__device__ __forceinline__ int block_checked(const DecodeArgs &a, int entry, int page) {
    return (page >= 0 && page < a.max_blocks && entry >= 0 && entry < a.num_blocks) ? entry : -1;
}

/* One window of at most 64 pages [base, base + nw) of segment (b, h): lane i's entry is page base + i's. The first
 * window of a fused piece also builds q once its pages are in flight, and the appending piece's key and value after
 * its first page (before the last). */
__device__ void finish_piece(const DecodeArgs &a, int b, int h, int w, int piece, bool whole, int lane, State &st,
                             StepLds &sm, int &np);

/* Fixed pieces: at the first page of the next piece (page number next_cut), finish the piece before it into its
 * merge slot and start the next one from a fresh state. */
__device__ __forceinline__ void cut_piece(const DecodeArgs &a, int b, int h, int page, const SeqRange &sr, int lane,
                                          int &next_cut, State &st, StepLds &sm, int &np) {
    if (page != next_cut) return;
    const int len = piece_len(a, sr.last - sr.first + 1);
    finish_piece(a, b, h, 0, (page - sr.first) / len - 1, false, lane, st, sm, np);
    state_init(st);
    next_cut += len;
}

template <bool FUSED, bool FIRST>
__device__ __forceinline__ void stream_window(const DecodeArgs &a, int b, int h, int base, int nw, int entry,
                                              const SeqRange &sr, bool app, const QRows &qr, const KvRows &kr,
                                              bf16x8 *qop, int lane, StepLds &sm, State &st, int &next_cut,
                                              int &np) {
    const int n = lane & 15, j = lane >> 4;
    const int patch_t = FUSED && app ? sr.p % NC_PAGE : -1;
    const int ids = lane < nw ? block_checked(a, entry, base + lane) : -1;
    const int last = __builtin_amdgcn_readfirstlane(nw - 1);
    Page r[DEC_DEPTH];
#pragma unroll
    for (int i = 0; i < DEC_DEPTH - 1; i++) {
        __builtin_amdgcn_sched_barrier(0);
        load_page(a, __builtin_amdgcn_readlane(ids, min(i, last)), h, n, j, r[i]);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (FUSED && FIRST) {
        build_q(a, qr, lane, qop, sm);
        if (app && nw == 1 && sr.p / NC_PAGE == base) build_kv(a, b, sr.p, qr, kr, lane, sm); /* the only page */
        __builtin_amdgcn_sched_barrier(0);
    }
    /* sched_barrier keeps each reload after the math that frees its buffer: with the live ranges apart the buffers
     * keep their registers across iterations (no copies of in-flight loads, no vmcnt(0)). Loads are unconditional
     * (clamped to the last page) so the counted waits stay exact. */
    for (int k = 0; k < nw; k += DEC_DEPTH) {
#pragma unroll
        for (int u = 0; u < DEC_DEPTH; u++) {
            load_page(a, __builtin_amdgcn_readlane(ids, min(k + u + DEC_DEPTH - 1, last)), h, n, j,
                      r[(u + DEC_DEPTH - 1) % DEC_DEPTH]);
            __builtin_amdgcn_sched_barrier(0);
            if (u == 0 || k + u < nw) {
                if (a.piece_pages > 0) cut_piece(a, b, h, base + k + u, sr, lane, next_cut, st, sm, np);
                attend_page(a, r[u], base + k + u, sr, qop, lane, patch_t, sm, st);
            }
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (FUSED && FIRST) {
                if (app && k == 0 && u == 0 && !(nw == 1 && sr.p / NC_PAGE == base)) {
                    build_kv(a, b, sr.p, qr, kr, lane, sm); /* after the first page, before the last */
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    }
}

/* The pages [pg_lo, pg_lo + npg) of segment (b, h), DEC_DEPTH buffers in rotation: DEC_DEPTH - 1 pages are in
 * flight while one is computed. The first window's block ids load first, the fused step's rows behind them (every
 * piece loads both row sets: unconditional loads keep every wait a counted one), so its page loads wait for the
 * ids alone. */
template <bool FUSED, bool TABLE>
__device__ __forceinline__ void attend_run(const DecodeArgs &a, int b, int h, int pg_lo, int npg, const SeqRange &sr,
                                           bool app, bf16x8 *qop, int lane, StepLds &sm, State &st, int &np) {
    /* fixed pieces: the first cut after the run's first page */
    int next_cut = a.piece_pages > 0 ? pg_lo + piece_len(a, sr.last - sr.first + 1) : -1;
    QRows qr;
    KvRows kr;
    const int entry = block_entry<TABLE>(a, b, pg_lo + lane);
    if constexpr (FUSED) {
        load_qrows(a, b, h, sr.p, lane, qr);
        load_kvrows<TABLE>(a, b, h, sr.p, lane, kr);
    }
    __builtin_amdgcn_sched_barrier(0);
    stream_window<FUSED, true>(a, b, h, pg_lo, min(64, npg), entry, sr, app, qr, kr, qop, lane, sm, st, next_cut,
                               np);
    for (int win = 64; win < npg; win += 64) {
        const int e = block_entry<TABLE>(a, b, pg_lo + win + lane);
        __builtin_amdgcn_sched_barrier(0);
        stream_window<FUSED, false>(a, b, h, pg_lo + win, min(64, npg - win), e, sr, app, qr, kr, qop, lane, sm,
                                    st, next_cut, np);
    }
}

/* The workspace slot of piece i of segment s, made by wave w. Fixed pieces: s * piece_slots + i. Pieces cut
 * by the balanced split (piece i is the i-th wave to touch the segment): the first DEC_MERGE_DIRECT sit together
 * at s * DEC_MERGE_DIRECT + i; later ones at S * DEC_MERGE_DIRECT + w + s (unique: a wave's pieces lie in
 * consecutive segments and the waves' slices are in segment order, so w + s never repeats). */
__device__ __forceinline__ size_t merge_slot(const DecodeArgs &a, int s, int i, int w) {
    const int S = a.B * a.hkv;
    if (a.piece_pages > 0) return (size_t)s * a.piece_slots + i;
    return i < DEC_MERGE_DIRECT ? (size_t)s * DEC_MERGE_DIRECT + i : (size_t)S * DEC_MERGE_DIRECT + w + s;
}

/* The staged pieces to their workspace slots (slot [G][128] of ws_o, [G][2] of ws_ml, both contiguous per slot). */
__device__ void flush_parts(const DecodeArgs &a, int lane, StepLds &sm, int &np) {
    __syncthreads(); /* the stage's writes before other lanes' reads */
    const int G = a.group, per = G * (NC_HEAD_DIM + 2);
    for (int i = 0; i < np; i++) {
        const size_t slot = (size_t)sm.part_slot[i];
        const f32x4 *src = reinterpret_cast<const f32x4 *>(&sm.part[i * per]);
        f32x4 *dst = reinterpret_cast<f32x4 *>(a.ws_o + slot * G * NC_HEAD_DIM);
        for (int v = lane; v < G * NC_HEAD_DIM / 4; v += NC_WAVE) dst[v] = src[v];
        if (lane < 2 * G) a.ws_ml[slot * G * 2 + lane] = sm.part[i * per + G * NC_HEAD_DIM + lane];
    }
    __syncthreads(); /* the reads done before the stage is reused */
    np = 0;
}

/* Finish piece `piece` of segment (b, h), wave w: the whole segment writes the normalised bf16 output; a part of it
 * stages (Σ p v in value units, max, sum) for its merge slot, which k_merge combines. Lane (j, n) holds dims
 * (4 j + i) 8 + bb of head n. */
__device__ void finish_piece(const DecodeArgs &a, int b, int h, int w, int piece, bool whole, int lane, State &st,
                             StepLds &sm, int &np) {
    const int n = lane & 15, j = lane >> 4, G = a.group;
    float l = st.l;
    l += shfl_xor_f(l, 16);
    l += shfl_xor_f(l, 32);
    const float unit = exp2i(st.e_ref - 126); /* o * unit: Σ p v in value units */
    if (whole) {
        if (n >= G) return;
        bf16_t *dst = a.out + ((size_t)b * a.hq + h * G + n) * NC_HEAD_DIM;
        const float inv = l > 0.f ? unit / l : 0.f; /* 0: every block of the segment was missing */
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float v[8];
#pragma unroll
            for (int bb = 0; bb < 8; bb++) v[bb] = st.o[bb][i] * inv;
            store_bf16x8(dst + (4 * j + i) * 8, v);
        }
        return;
    }
    const int per = G * (NC_HEAD_DIM + 2);
    if ((np + 1) * per > DEC_PART_FLOATS || np == DEC_PART_MAX) flush_parts(a, lane, sm, np);
    const int at = np * per;
    if (n < G) {
        float *o = &sm.part[at + n * NC_HEAD_DIM];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const f32x4 lo = {st.o[0][i] * unit, st.o[1][i] * unit, st.o[2][i] * unit, st.o[3][i] * unit};
            const f32x4 hi = {st.o[4][i] * unit, st.o[5][i] * unit, st.o[6][i] * unit, st.o[7][i] * unit};
            reinterpret_cast<f32x4 *>(o + (4 * j + i) * 8)[0] = lo;
            reinterpret_cast<f32x4 *>(o + (4 * j + i) * 8)[1] = hi;
        }
        if (j == 0) {
            sm.part[at + G * NC_HEAD_DIM + 2 * n] = st.m;
            sm.part[at + G * NC_HEAD_DIM + 2 * n + 1] = l;
        }
    }
    if (lane == 0) sm.part_slot[np] = (int)merge_slot(a, b * a.hkv + h, piece, w);
    np++; /* flush_parts' barrier orders these stage writes before its reads */
}

/* Schedule units of the whole batch: every wave derives the same value from the live context lengths (the first
 * 64 entries already loaded, raw0 in lane b) and keeps them in lds (if not null) or, for a batch of at most 64, in
 * cx's lanes; wave b % W writes sequence b's row if it is empty (zeros, or NaN for the fused step's
 * positions out of range) and its next position to pos_out: sequence w's (own_pos, in lane w % 64) after its pages
 * (put_own_pos), any later ones (a batch larger than the grid) here. 32-bit: the host bounds the total. */
__device__ int schedule_total(const DecodeArgs &a, int w, int W, int lane, int *lds, int &own_pos, int raw0,
                              Ctx &cx) {
    int total = 0;
    for (int base = 0; base < a.B; base += 64) {
        const int b = base + lane;
        const int raw = b < a.B ? (base == 0 ? raw0 : a.ctx_len[b]) : 0;
        const int c = b < a.B ? seq_ctx_of(a, raw) : 0;
        const int pg = units_of(a, c);
        if (lds && b < a.B) lds[b] = c;
        if (a.pos_out && b < a.B && b % W == w) {
            if (b == w) own_pos = raw + 1;
            else a.pos_out[b] = raw + 1;
        }
        if (b < a.B && pg == 0 && b % W == w) {
            for (int hh = 0; hh < a.hkv; hh++) a.ws_desc[b * a.hkv + hh] = make_int2(0, 0); /* nothing to merge */
            const uint32_t f = c < 0 ? 0x7fc07fc0u : 0u;
            const u32x4 z = {f, f, f, f};
            for (int r = 0; r < a.hq * NC_HEAD_DIM / 8; r++)
                reinterpret_cast<u32x4 *>(a.out + (size_t)b * a.hq * NC_HEAD_DIM)[r] = z;
        }
        const int incl = wave_inclusive_sum(pg, lane);
        if (cx.regs) cx.c = c, cx.units = pg, cx.incl = incl;
        total += __builtin_amdgcn_readlane(incl, 63);
    }
    return total * a.hkv;
}

/* The fused step's next position of sequence w, held since schedule_total: stored after the wave's pages, so that
 * the store's acknowledgement holds up none of their waits (the memory counter completes in order). */
__device__ __forceinline__ void put_own_pos(const DecodeArgs &a, int w, int lane, int own_pos) {
    if (a.pos_out && w < a.B && lane == (w & 63)) a.pos_out[w] = own_pos;
}

/* The segment holding unit u of the flattened list: sequence b, kv head h and the segment's first unit. */
__device__ __forceinline__ void find_segment(const DecodeArgs &a, const Ctx &cx, int u, int lane, int &b, int &h,
                                             int &seg_base) {
    int carry = 0, units_b = 0;
    b = -1;
    if (cx.regs) { /* the sums schedule_total left in the lanes */
        const unsigned long long hit = __ballot(lane < a.B && cx.incl * a.hkv > u);
        const int first = hit ? __builtin_ctzll(hit) : 0;
        b = first;
        units_b = __builtin_amdgcn_readlane(cx.units, first);
        carry = __builtin_amdgcn_readlane(cx.incl - cx.units, first) * a.hkv;
    }
    for (int base = 0; base < a.B && b < 0; base += 64) {
        const int bb = base + lane;
        const int pg = bb < a.B ? units_of(a, ctx_at(a, cx.lds, bb)) : 0;
        const int incl = wave_inclusive_sum(pg, lane);
        const unsigned long long hit = __ballot(bb < a.B && carry + incl * a.hkv > u);
        if (hit) {
            const int first = __builtin_ctzll(hit);
            b = base + first;
            units_b = __builtin_amdgcn_readlane(pg, first);
            carry += __builtin_amdgcn_readlane(incl - pg, first) * a.hkv;
        } else {
            carry += __builtin_amdgcn_readlane(incl, 63) * a.hkv;
        }
    }
    const int into = u - carry; /* offset inside sequence b */
    h = into / units_b;
    seg_base = u - into % units_b;
}

/* Fixed pieces: the piece boundary nearest to unit u. A segment's boundaries are its first unit, the units of its
 * pieces' first pages after the first (its start units go with its first piece) and its end (its end units go with
 * its last piece). Every wave rounds a shared slice end alike, so the snapped slices still tile the list. */
__device__ __forceinline__ int snap_unit(const DecodeArgs &a, const Ctx &cx, int u, int lane) {
    int b, h, seg_base;
    find_segment(a, cx, u, lane, b, h, seg_base);
    const int pages = pages_of(a, ctx_of(a, cx, b)), len = piece_len(a, pages), np = (pages + len - 1) / len;
    const int units = pages + a.unit_start + a.unit_end;
    const int k = min(max((u - seg_base - a.unit_start + len / 2) / len, 0), np); /* numerator >= -unit_start */
    const int at = u - seg_base < a.unit_start ? 0 : k;
    return seg_base + (at == 0 ? 0 : at == np ? units : a.unit_start + at * len);
}

template <bool FUSED, bool TABLE>
__global__ void __launch_bounds__(DEC_THREADS) k_decode(DecodeArgs a) {
    __shared__ StepLds sm;
    __shared__ int ctx_lds[DEC_LDS_SEQS];
    const int w = blockIdx.x, W = gridDim.x, lane = threadIdx.x, n = lane & 15, j = lane >> 4;
    /* the first 64 context entries, loaded before anything else: their round trip overlaps the wave's set-up */
    const int raw0 = lane < a.B ? a.ctx_len[lane] : 0;
    int *const lds = a.B > 64 && a.B <= DEC_LDS_SEQS ? ctx_lds : nullptr;
    Ctx cx;
    cx.lds = lds, cx.c = 0, cx.units = 0, cx.incl = 0, cx.regs = a.B <= 64;

    int np = 0; /* staged pieces (one wave: a register) */
    int own_pos = 0;
    const int total = schedule_total(a, w, W, lane, lds, own_pos, raw0, cx);
    __syncthreads(); /* lds complete before other lanes' reads */
    const int chunk = max((total + W - 1) / W, DEC_MIN_CHUNK);
    int start = w * chunk;
    if (start >= total) {
        put_own_pos(a, w, lane, own_pos);
        return;
    }
    int end = min(start + chunk, total);
    if (a.piece_pages > 0) { /* whole fixed pieces: both ends at the nearest piece boundary */
        start = snap_unit(a, cx, start, lane);
        end = end >= total ? total : snap_unit(a, cx, end, lane);
        if (start >= end) {
            put_own_pos(a, w, lane, own_pos);
            return;
        }
    }
    int remaining = end - start;

    /* the segment holding `start`: sequence b, kv head h, its first unit seg_base */
    int b, h, seg_base;
    find_segment(a, cx, start, lane, b, h, seg_base);
    int off = start - seg_base;

    while (remaining > 0) {
        const SeqRange sr = seq_range_of(a, ctx_of(a, cx, b));
        const int seg_pages = sr.last - sr.first + 1;
        /* this slice takes units [off, off + take) of the segment; its pages are [lo, hi) */
        const int units = seg_pages + a.unit_start + a.unit_end;
        const int take = min(units - off, remaining);
        const int lo = max(off - a.unit_start, 0), hi = min(off + take - a.unit_start, seg_pages);
        /* the waves holding the segment's first and last pages: piece i of the segment is wave w_first + i */
        const int page0 = seg_base + a.unit_start;
        const int w_first = page0 / chunk, pieces = (page0 + seg_pages - 1) / chunk - w_first + 1;
        remaining -= take;
        off = 0;
        seg_base += units;
        if (hi > lo) {
            /* the piece this run ends with (finished after it) and the segment's piece count; fixed pieces from
             * the segment's first page, else one per wave (piece i of the segment is wave w_first + i) */
            const int len = a.piece_pages > 0 ? piece_len(a, seg_pages) : 0;
            const int piece = len ? (hi - 1) / len : w - w_first;
            const int seg_pieces = len ? (seg_pages + len - 1) / len : pieces;
            const bool whole = seg_pieces == 1;
            bf16x8 qop[4]; /* the fused step builds it in attend_run */
            if constexpr (!FUSED) {
                if (n < a.group) {
                    const u32x4 *qp = reinterpret_cast<const u32x4 *>(
                        a.q + ((size_t)b * a.hq + h * a.group + n) * NC_HEAD_DIM + j * 32);
#pragma unroll
                    for (int c = 0; c < 4; c++) qop[c] = __builtin_bit_cast(bf16x8, qp[c]);
                } else {
#pragma unroll
                    for (int c = 0; c < 4; c++) qop[c] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
                }
            }
            State st;
            state_init(st);
            attend_run<FUSED, TABLE>(a, b, h, sr.first + lo, hi - lo, sr, hi == seg_pages, qop, lane, sm, st, np);
            finish_piece(a, b, h, w, piece, whole, lane, st, sm, np);
            if (lo == 0 && lane == 0) a.ws_desc[b * a.hkv + h] = make_int2(seg_pieces, len ? 0 : w_first);
            if (FUSED && hi == seg_pages) store_new_kv(a, h, sr.p, lane, sm);
        }
        if (++h == a.hkv) {
            h = 0;
            do {
                b++;
            } while (remaining > 0 && b < a.B && pages_of(a, ctx_of(a, cx, b)) == 0);
            if (b >= a.B) break;
        }
    }
    flush_parts(a, lane, sm, np); /* after the last pages: these stores hold up no wait */
    put_own_pos(a, w, lane, own_pos);
}

/* One workgroup per segment s = (b, h) = blockIdx.x combines the pieces of a segment that more than one wave
 * touched, weights exp2(m_k - max m) as decode.cu:547-548's rescale. A thread holds head n, dims 8 c..8 c + 8 (16
 * lanes per head) of one of Q = merge_groups groups of 16 G lanes. Group q folds, in order, pieces 8 q..8 q + 7,
 * then 8 (q + Q)..8 (q + Q) + 7, and so on; group 0 then folds the groups' results in order: a fixed order for a
 * given piece count, head group and Q, so the bits depend on nothing else. The balanced split launches
 * MERGE_GROUPS groups, and past DEC_LONG_CTX as many as its longest possible segment fills (up to
 * 1024 / (16 G)); fixed pieces launch as many as the longest segment at max_ctx fills
 * (ceil(pieces / 8), at most 1024 / (16 G)), so every segment of at most 8 Q pieces folds in one round whatever Q
 * is, and Q depends on max_ctx alone, not on the batch. The kernel is latency-bound: the first round's slots do not
 * depend on the segment's descriptor (fixed pieces: s * piece_slots + i; the balanced split's first
 * DEC_MERGE_DIRECT: s * DEC_MERGE_DIRECT + i), so they load together with it, unconditionally (a predicate per slot
 * puts each load behind a branch and a wait), one round trip for up to 8 Q fixed pieces (8 for the balanced split,
 * every segment of config 3). THREADS: 256, or 1024 where the groups need more lanes. */
#define MERGE_LANES 16
#define MERGE_THREADS 256      /* the workgroup where the groups fit in 256 lanes */
#define MERGE_THREADS_MAX 1024 /* otherwise (head groups of 5 or more, long contexts): up to 1024 / (16 G) groups */
#define MERGE_GROUPS 4
#define DEC_LONG_CTX 16384     /* the balanced split's merge takes more groups from this max_ctx on */

struct MergeAcc {
    float m, l, o[8];
};

__device__ __forceinline__ void merge_fold(MergeAcc &r, float m_k, float l_k, const float *o_k) {
    const float m_new = fmaxf(r.m, m_k);
    const float a_old = __builtin_amdgcn_exp2f(r.m - m_new), a_new = __builtin_amdgcn_exp2f(m_k - m_new);
    r.l = r.l * a_old + l_k * a_new;
#pragma unroll
    for (int e = 0; e < 8; e++) r.o[e] = r.o[e] * a_old + o_k[e] * a_new;
    r.m = m_new;
}

/* Pieces base..base + 7 (those below `pieces`) of segment s into r: slots from merge_slot, or, with `spec`, the
 * first round's fixed slots loaded before the piece count is known (every one of them inside the workspace). */
__device__ __forceinline__ void merge_round(const DecodeArgs &a, int s, int2 d, int base, int n, int c,
                                            MergeAcc &r) {
    f32x2 ml[DEC_MERGE_DIRECT];
    f32x4 ov[DEC_MERGE_DIRECT][2];
#pragma unroll
    for (int k = 0; k < DEC_MERGE_DIRECT; k++) {
        if (base + k < d.x) {
            const size_t slot = merge_slot(a, s, base + k, d.y + base + k) * a.group + n;
            ml[k] = *reinterpret_cast<const f32x2 *>(a.ws_ml + 2 * slot);
            const f32x4 *src = reinterpret_cast<const f32x4 *>(a.ws_o + slot * NC_HEAD_DIM + 8 * c);
            ov[k][0] = src[0];
            ov[k][1] = src[1];
        }
    }
#pragma unroll
    for (int k = 0; k < DEC_MERGE_DIRECT; k++) {
        if (base + k < d.x) {
            const float o_k[8] = {ov[k][0][0], ov[k][0][1], ov[k][0][2], ov[k][0][3],
                                  ov[k][1][0], ov[k][1][1], ov[k][1][2], ov[k][1][3]};
            merge_fold(r, ml[k][0], ml[k][1], o_k);
        }
    }
}

template <int THREADS>
__global__ void __launch_bounds__(THREADS) k_merge(DecodeArgs a) {
    __shared__ MergeAcc grp[THREADS];
    const int s = blockIdx.x, b = s / a.hkv, h = s % a.hkv, t = threadIdx.x, G = a.group;
    const int row = G * MERGE_LANES, Q = a.merge_groups, q = t / row, n = (t % row) / MERGE_LANES,
              c = t % MERGE_LANES;
    const int2 d = a.ws_desc[s];
    /* the first round's slots, loaded with the descriptor: slot(i) needs no d where spec holds */
    const bool fixed = a.piece_pages > 0;
    const bool spec = q < Q && (fixed ? DEC_MERGE_DIRECT * (q + 1) <= a.piece_slots : q == 0);
    f32x2 ml[DEC_MERGE_DIRECT];
    f32x4 ov[DEC_MERGE_DIRECT][2];
    if (spec) {
#pragma unroll
        for (int k = 0; k < DEC_MERGE_DIRECT; k++) {
            const int i = DEC_MERGE_DIRECT * q + k;
            const size_t slot = ((size_t)s * (fixed ? a.piece_slots : DEC_MERGE_DIRECT) + i) * G + n;
            ml[k] = *reinterpret_cast<const f32x2 *>(a.ws_ml + 2 * slot);
            const f32x4 *src = reinterpret_cast<const f32x4 *>(a.ws_o + slot * NC_HEAD_DIM + 8 * c);
            ov[k][0] = src[0];
            ov[k][1] = src[1];
        }
    }
    const int pieces = d.x;
    if (pieces <= 1) return; /* one piece: k_decode wrote the output; none: an empty sequence's zero row */
    MergeAcc r;
    r.m = DEC_M_INIT, r.l = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) r.o[e] = 0.f;
    if (q < Q) {
        if (spec) {
#pragma unroll
            for (int k = 0; k < DEC_MERGE_DIRECT; k++) {
                if (DEC_MERGE_DIRECT * q + k < pieces) {
                    const float o_k[8] = {ov[k][0][0], ov[k][0][1], ov[k][0][2], ov[k][0][3],
                                          ov[k][1][0], ov[k][1][1], ov[k][1][2], ov[k][1][3]};
                    merge_fold(r, ml[k][0], ml[k][1], o_k);
                }
            }
        } else if (DEC_MERGE_DIRECT * q < pieces) {
            merge_round(a, s, d, DEC_MERGE_DIRECT * q, n, c, r);
        }
        for (int base = DEC_MERGE_DIRECT * (q + Q); base < pieces; base += DEC_MERGE_DIRECT * Q)
            merge_round(a, s, d, base, n, c, r);
    }
    grp[t] = r;
    __syncthreads();
    if (q != 0) return;
    for (int g = 1; g < Q && DEC_MERGE_DIRECT * g < pieces; g++) {
        const MergeAcc &o = grp[g * row + t];
        merge_fold(r, o.m, o.l, o.o);
    }
    const float inv = r.l > 0.f ? 1.0f / r.l : 0.f;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = r.o[e] * inv;
    store_bf16x8(a.out + ((size_t)b * a.hq + h * G + n) * NC_HEAD_DIM + 8 * c, v);
}

/* Resident single-wave workgroups of k_decode on the current device (cached per device). */
static int decode_waves() {
    static int cached[64];
    int dev = 0;
    NC_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) dev = 0;
    if (!cached[dev]) {
        int per_cu = 0, cus = 0;
        int per_cu_fused = 0;
        const void *kernels[4] = {(const void *)k_decode<false, false>, (const void *)k_decode<false, true>,
                                  (const void *)k_decode<true, false>, (const void *)k_decode<true, true>};
        per_cu = 1 << 30;
        for (const void *k : kernels) { /* one grid size for all: the same schedule */
            NC_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu_fused, k, DEC_THREADS, 0));
            if (per_cu_fused < per_cu) per_cu = per_cu_fused;
        }
        NC_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        /* CDNA: 4 SIMDs per CU. Resident waves beyond DEC_WAVES_PER_SIMD per SIMD are not used: a second wave on
         * a SIMD loses issue arbitration to the older one and finishes its equal share last. */
        if (per_cu > 4 * DEC_WAVES_PER_SIMD) per_cu = 4 * DEC_WAVES_PER_SIMD;
        const int w = per_cu * cus;
        cached[dev] = w < 1 ? 1 : (w > DEC_MAX_WAVES ? DEC_MAX_WAVES : w);
    }
    return cached[dev];
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

/* The most fixed pieces of a segment for contexts up to max_ctx: DEC_PIECES_MIN, or enough to cut the longest
 * segment (ceil(max_ctx / 16) pages) into 16-page pieces, at most DEC_PIECES_MAX. A function of max_ctx alone, so
 * a sequence's pieces do not depend on the batch; from 8192 keys on, long segments get more, shorter pieces (and
 * so more waves) instead of 32 long ones. */
static int piece_slots_for(int max_ctx) {
    const long long pages = ((long long)max_ctx + NC_PAGE - 1) / NC_PAGE;
    return (int)std::min<long long>(DEC_PIECES_MAX, std::max<long long>(DEC_PIECES_MIN, (pages + 15) / 16));
}

/* Partial-result slots: for the balanced split the first DEC_MERGE_DIRECT pieces of every segment, then one per
 * (wave, segment) offset; for fixed pieces piece_slots_for(max_ctx) per segment. */
static size_t balanced_slots(size_t S) { return S * DEC_MERGE_DIRECT + DEC_MAX_WAVES + S; }
static size_t merge_slots(size_t S, int max_ctx, bool fixed) {
    return fixed ? S * (size_t)piece_slots_for(max_ctx) : balanced_slots(S);
}
static long long workspace_bytes(size_t S, size_t G, size_t slots) {
    return (long long)(align256(slots * G * NC_HEAD_DIM * sizeof(float)) + align256(slots * G * 2 * sizeof(float)) +
                       S * sizeof(int2));
}

extern "C" long long nc_decode_workspace_bytes(int B, int hq, int hkv, int max_ctx) {
    if (B <= 0 || hq <= 0 || hkv <= 0 || max_ctx <= 0 || hq % hkv) return 0;
    const size_t S = (size_t)B * hkv, G = hq / hkv;
    return std::max(workspace_bytes(S, G, merge_slots(S, max_ctx, false)),
                    workspace_bytes(S, G, merge_slots(S, max_ctx, true)));
}

/* Checks shared by both entry points, then the launch of k_decode<FUSED, TABLE>. */
static int decode_launch(DecodeArgs &a, bool fused, const void *out, const void *workspace, long long workspace_bytes,
                         int max_ctx, float sm_scale, void *stream) {
    const int B = a.B, hq = a.hq, hkv = a.hkv;
    NC_REQUIRE(hkv > 0 && hq > 0 && hq % hkv == 0, "hq = %d must be a positive multiple of hkv = %d", hq, hkv);
    NC_REQUIRE(hq / hkv <= DEC_MAX_G, "hq / hkv = %d exceeds %d query heads per kv head", hq / hkv, DEC_MAX_G);
    NC_REQUIRE(a.max_blocks > 0 && a.num_blocks > 0, "max_blocks %d, num_blocks %d must be positive", a.max_blocks,
               a.num_blocks);
    NC_REQUIRE(a.block_table || (long long)B * a.max_blocks <= a.num_blocks,
               "contiguous cache: %d sequences x %d blocks exceed the %d blocks", B, a.max_blocks, a.num_blocks);
    NC_REQUIRE(max_ctx > 0 && max_ctx <= a.max_blocks * NC_PAGE, "max_ctx %d outside [1, %d]", max_ctx,
               a.max_blocks * NC_PAGE);
    NC_REQUIRE(a.cache && a.ctx_len && out && workspace, "null argument");
    NC_REQUIRE(((uintptr_t)out | (uintptr_t)a.cache | (uintptr_t)workspace) % 16 == 0,
               "tensors must be 16-byte aligned");
    const bool fixed = a.piece_pages > 0;
    const size_t S = (size_t)B * hkv, slots = merge_slots(S, max_ctx, fixed);
    const long long need = ::workspace_bytes(S, (size_t)(hq / hkv), slots);
    NC_REQUIRE(workspace_bytes >= need, "workspace %lld bytes, %lld needed", workspace_bytes, need);
    /* the kernel's schedule counts units in 32 bits: every segment's pages plus its start and end units */
    NC_REQUIRE((long long)B * hkv * ((long long)a.max_blocks + DEC_UNITS_START + DEC_UNITS_END) < (1ll << 31),
               "%d sequences x %d kv heads x %d pages exceed the schedule's 2^31 units", B, hkv, a.max_blocks);
    a.group = hq / hkv;
    a.score_scale = sm_scale * 1.4426950408889634f;
    a.out = (bf16_t *)out;
    a.max_ctx = max_ctx;
    a.piece_slots = piece_slots_for(max_ctx);
    unsigned char *ws = (unsigned char *)workspace;
    a.ws_o = (float *)ws;
    ws += align256(slots * a.group * NC_HEAD_DIM * sizeof(float));
    a.ws_ml = (float *)ws;
    ws += align256(slots * a.group * 2 * sizeof(float));
    a.ws_desc = (int2 *)ws;
    a.unit_start = DEC_UNITS_START;
    a.unit_end = DEC_UNITS_END;
    const int W = decode_waves();
    const dim3 grid(W), block(DEC_THREADS);
    hipStream_t st = (hipStream_t)stream;
    if (fused && a.block_table) hipLaunchKernelGGL((k_decode<true, true>), grid, block, 0, st, a);
    else if (fused) hipLaunchKernelGGL((k_decode<true, false>), grid, block, 0, st, a);
    else if (a.block_table) hipLaunchKernelGGL((k_decode<false, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((k_decode<false, false>), grid, block, 0, st, a);
    NC_LAUNCH_CHECK();
    /* the groups. The balanced split: MERGE_GROUPS (in 1024-lane workgroups for head groups of 5 or more, where 256
     * lanes hold fewer), and past DEC_LONG_CTX as many as its longest possible segment fills. Fixed pieces: as many
     * as the pieces of the longest segment at max_ctx fill (ceil(max_ctx / 16) pages at most), up to
     * MERGE_THREADS_MAX lanes, so that a segment of up to 8 Q pieces folds in one round trip. 1024-lane workgroups
     * only where 256 lanes cannot hold the groups. */
    const int row = a.group * MERGE_LANES;
    int groups = std::min(MERGE_GROUPS, MERGE_THREADS_MAX / row);
    if (!fixed && max_ctx > DEC_LONG_CTX) {
        /* long contexts: a segment can span up to ceil(pages / DEC_MIN_CHUNK) + 1 waves, so as many groups as that
         * fills (fewer dependent rounds for one long sequence); shorter contexts keep the groups above */
        const long long pages = ((long long)max_ctx + NC_PAGE - 1) / NC_PAGE;
        const long long most = (pages + DEC_MIN_CHUNK - 1) / DEC_MIN_CHUNK + 1;
        groups = (int)std::max<long long>(groups, std::min<long long>((most + DEC_MERGE_DIRECT - 1) / DEC_MERGE_DIRECT,
                                                                      MERGE_THREADS_MAX / row));
    }
    if (fixed) {
        const long long pages = ((long long)max_ctx + NC_PAGE - 1) / NC_PAGE;
        const int most = (int)std::min<long long>(a.piece_slots, (pages + a.piece_pages - 1) / a.piece_pages);
        groups = std::max(1, std::min((most + DEC_MERGE_DIRECT - 1) / DEC_MERGE_DIRECT, MERGE_THREADS_MAX / row));
    }
    a.merge_groups = groups;
    const int threads = (groups * row + NC_WAVE - 1) / NC_WAVE * NC_WAVE;
    if (threads <= MERGE_THREADS) hipLaunchKernelGGL(k_merge<MERGE_THREADS>, dim3((unsigned)S), dim3(threads), 0, st, a);
    else hipLaunchKernelGGL(k_merge<MERGE_THREADS_MAX>, dim3((unsigned)S), dim3(threads), 0, st, a);
    NC_LAUNCH_CHECK();
    return 0;
}

extern "C" int nc_decode_attn_fp8(const void *q, const uint8_t *cache, const int32_t *block_table, int max_blocks,
                                  int num_blocks, const int32_t *ctx_len, int window, int B, int hq, int hkv,
                                  int max_ctx, float sm_scale, void *out, void *workspace, long long workspace_bytes,
                                  void *stream) {
    NC_REQUIRE(B >= 0, "B = %d < 0", B);
    if (B == 0) return 0;
    NC_REQUIRE(q && (uintptr_t)q % 16 == 0, "q must be a 16-byte aligned pointer");
    DecodeArgs a = {};
    a.q = (const bf16_t *)q; a.cache = const_cast<uint8_t *>(cache); /* not written without qkv */
    a.block_table = block_table; a.max_blocks = max_blocks; a.num_blocks = num_blocks; a.ctx_len = ctx_len;
    a.window = window; a.B = B; a.hq = hq; a.hkv = hkv;
    return decode_launch(a, false, out, workspace, workspace_bytes, max_ctx, sm_scale, stream);
}

/* The fused step's checks and launch, shared by the workspace, fixed-piece and static-scratch entry points. */
static int decode_step(const void *qkv, long long row_stride, const int32_t *pos, int32_t *pos_out,
                       const float *q_gain, const float *k_gain, const float *cos, const float *sin, int rope_len,
                       uint8_t *cache, const int32_t *block_table, int max_blocks, int num_blocks, int window, int B,
                       int hq, int hkv, int max_ctx, float sm_scale, int piece_pages, void *out, void *workspace,
                       long long workspace_bytes, void *stream) {
    NC_REQUIRE(B >= 0, "B = %d < 0", B);
    if (B == 0) return 0;
    NC_REQUIRE(hkv > 0 && hq > 0 && hq % hkv == 0, "hq = %d must be a positive multiple of hkv = %d", hq, hkv);
    NC_REQUIRE(row_stride >= (long long)(hq + 2 * hkv) * NC_HEAD_DIM && row_stride % 8 == 0,
               "row_stride %lld must hold (hq + 2 hkv) * 128 elements and keep 16-byte alignment", row_stride);
    NC_REQUIRE(rope_len > 0, "rope_len = %d", rope_len);
    NC_REQUIRE(qkv && pos && q_gain && k_gain && cos && sin, "null argument");
    NC_REQUIRE(((uintptr_t)qkv | (uintptr_t)q_gain | (uintptr_t)k_gain | (uintptr_t)cos | (uintptr_t)sin) % 16 == 0,
               "qkv, gains and rotary tables must be 16-byte aligned");
    const char *o = (const char *)out, *x = (const char *)qkv;
    NC_REQUIRE(!out || o + (size_t)B * hq * NC_HEAD_DIM * 2 <= x || x + (size_t)B * row_stride * 2 <= o,
               "out must not overlap qkv");
    NC_REQUIRE(!pos_out || pos_out + B <= pos || pos + B <= pos_out, "pos_out must not overlap pos");
    DecodeArgs a = {};
    a.cache = cache;
    a.block_table = block_table; a.max_blocks = max_blocks; a.num_blocks = num_blocks; a.ctx_len = pos;
    a.pos_out = pos_out;
    a.qkv = (const bf16_t *)qkv; a.row_stride = row_stride; a.q_gain = q_gain; a.k_gain = k_gain;
    a.cos = cos; a.sin = sin; a.rope_len = rope_len;
    a.window = window; a.B = B; a.hq = hq; a.hkv = hkv;
    a.piece_pages = piece_pages;
    return decode_launch(a, true, out, workspace, workspace_bytes, max_ctx, sm_scale, stream);
}

extern "C" int nc_decode_step_fp8(const void *qkv, long long row_stride, const int32_t *pos, int32_t *pos_out,
                                  const float *q_gain, const float *k_gain, const float *cos, const float *sin,
                                  int rope_len, uint8_t *cache, const int32_t *block_table, int max_blocks,
                                  int num_blocks, int window, int B, int hq, int hkv, int max_ctx, float sm_scale,
                                  void *out, void *workspace, long long workspace_bytes, void *stream) {
    return decode_step(qkv, row_stride, pos, pos_out, q_gain, k_gain, cos, sin, rope_len, cache, block_table,
                       max_blocks, num_blocks, window, B, hq, hkv, max_ctx, sm_scale, 0, out, workspace,
                       workspace_bytes, stream);
}

extern "C" int nc_decode_step_fp8_pieces(const void *qkv, long long row_stride, const int32_t *pos, int32_t *pos_out,
                                         const float *q_gain, const float *k_gain, const float *cos,
                                         const float *sin, int rope_len, uint8_t *cache, const int32_t *block_table,
                                         int max_blocks, int num_blocks, int window, int B, int hq, int hkv,
                                         int max_ctx, float sm_scale, int piece_pages, void *out, void *workspace,
                                         long long workspace_bytes, void *stream) {
    NC_REQUIRE(piece_pages >= 1 && piece_pages <= 1 << 16, "piece_pages = %d outside [1, 65536]", piece_pages);
    return decode_step(qkv, row_stride, pos, pos_out, q_gain, k_gain, cos, sin, rope_len, cache, block_table,
                       max_blocks, num_blocks, window, B, hq, hkv, max_ctx, sm_scale, piece_pages, out, workspace,
                       workspace_bytes, stream);
}

/* ------------------------------------------------------------------------------------------------------------
 * The fused step without a workspace argument, for callers that cannot allocate (code under graph capture, tight
 * serving loops): the partial results and the segments' piece descriptors live in a static device array of
 * NC_DECODE_SCRATCH_BYTES (decode_scratch.hip, a code object of its own, so only devices on which this entry runs
 * hold it, until the process ends), passed to the kernel like the workspace of nc_decode_step_fp8. No value needs
 * to start at zero: k_decode writes every segment's descriptor and every piece's partial before k_merge reads them,
 * so what earlier calls left there does not matter. Calls share their device's array, so two calls that may
 * overlap on one device (two streams) race; calls in one stream do not. */
extern "C" int nc_decode_step_fp8_noalloc(const void *qkv, long long row_stride, const int32_t *pos,
                                          int32_t *pos_out, const float *q_gain, const float *k_gain,
                                          const float *cos, const float *sin, int rope_len, uint8_t *cache,
                                          const int32_t *block_table, int max_blocks, int num_blocks, int window,
                                          int B, int hq, int hkv, int max_ctx, float sm_scale, void *out,
                                          void *stream) {
    /* the balanced split's partial results (this entry does not take fixed pieces) */
    const long long need = B > 0 && hq > 0 && hkv > 0 && hq % hkv == 0 && max_ctx > 0
                               ? workspace_bytes((size_t)B * hkv, (size_t)(hq / hkv), balanced_slots((size_t)B * hkv))
                               : 0;
    NC_REQUIRE(need <= NC_DECODE_SCRATCH_BYTES,
               "%d sequences of %d / %d heads need %lld bytes of partial results, the static scratch holds %lld", B,
               hq, hkv, need, NC_DECODE_SCRATCH_BYTES);
    if (B <= 0 || need == 0) /* nothing to launch: the shared checks report a bad B or head count */
        return decode_step(qkv, row_stride, pos, pos_out, q_gain, k_gain, cos, sin, rope_len, cache, block_table,
                           max_blocks, num_blocks, window, B, hq, hkv, max_ctx, sm_scale, 0, out, nullptr, 0, stream);
    return decode_step(qkv, row_stride, pos, pos_out, q_gain, k_gain, cos, sin, rope_len, cache, block_table,
                       max_blocks, num_blocks, window, B, hq, hkv, max_ctx, sm_scale, 0, out, nc_decode_scratch(),
                       NC_DECODE_SCRATCH_BYTES, stream);
}
