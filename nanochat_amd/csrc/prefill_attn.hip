/*
 * Chunked-prefill attention over the fp8 paged cache (reference: dec_prefill, model/kernels/decode.cu:1039-1051,
 * whose rows each run k_attn, decode.cu:567-675, as one single-query block: no K/V reuse across rows).
 *
 * Rows: n query rows (bf16 q [n][Hq][128], the append's q_out), row r at position pos[r] of sequence seq[r]. As in
 * the reference (decode.cu:859-863) every row's key and value are appended before any row attends, so row r
 * reads keys [max(pos - window, 0), pos] of its sequence from the cache, its own and its chunk's earlier keys
 * included. Rows may come in any order and from any sequences; the kernel is fastest when a sequence's rows are
 * consecutive.
 *
 * Work: one workgroup of 4 waves (one per SIMD) per (kv head h, tile of 8 R consecutive rows), R = floor(16 / G)
 * rows per 16-column MFMA block, G = Hq / Hkv. A wave holds 2 blocks; column n of a block is (row n / G, query
 * head h G + n % G), so the G heads of a row share every key read. The workgroup walks the pages of the union key
 * range of its rows in pairs; its four waves consume the same pair from LDS. Two workgroups share a CU (256
 * VGPRs and 72 KB of LDS each), so the two waves of a SIMD belong to different workgroups: no barrier ties their
 * phases together, and one workgroup's set-up and epilogue overlap the other's page loop (short key ranges:
 * 1.3x the speed of 8-wave workgroups, one per CU).
 *
 * Per page pair (32 keys) a wave computes, for each of its 2 blocks,
 *   scores  Sᵀ[16 keys][16 columns] per page = K · Qᵀ on fp8 MFMAs: v_mfma_scale_f32_16x16x128_f8f6f4 takes the
 *           page's e4m3 K codes as they are (A: key lane % 16, dims 32 (lane / 16) .. + 31, all 128 dims in one
 *           instruction) against q split into two e4m3 terms, q 2^e = hi + lo (hi = e4m3(q 2^e), lo = e4m3 of the
 *           exact remainder: about 8 significant bits, bf16's precision), with e per column chosen so |q| 2^e <
 *           256; the MFMA's E8M0 B-scale 2^-e undoes it. Two 32-cycle MFMAs per page and block, the same MFMA time
 *           as four bf16 ones, and no K conversion;
 *   softmax fp32 base 2, lazy reference max per column (moves only when a score exceeds it by more than 8);
 *   values  Oᵀ[16 dims][16 columns] += Vᵀ[16 dims][32 keys] · Pᵀ, 8 v_mfma_f32_16x16x32_f16. The lane's k slots
 *           8j..8j+7 are keys 4j..4j+3 of the first page then of the second, which is where the score MFMAs left
 *           this lane's probabilities: Pᵀ is built in registers, no exchange. P carries v_scale and a running
 *           power of two (as in decode): fp16 with headroom, V codes fp8 -> fp16 exact.
 * Roofline: MFMA (the dense bf16/fp16 peak; the fp8 score MFMAs run at twice that rate over twice the work).
 *
 * K/V staging: a ring of PF_RING page-pair slots in LDS, filled by global_load_lds_dwordx4 (lane i of a DMA lands
 * at slot + 16 i: the tile's fragment-major parts arrive as they lie, and the read back is a contiguous,
 * conflict-free ds_read_b128 per fragment). Each wave issues 2 of a pair's 8 fragment loads from a scalar tile
 * base, the last wave also the pair's scales; the waves meet at a barrier every PF_BATCH pairs, where the ring's
 * freed slots are refilled. Block ids are staged in LDS per chunk of PF_IDS pages.
 *
 * Software pipeline: iteration k runs the softmax of pair k (VALU), then one burst of 24 MFMAs at raised wave
 * priority (s_setprio 1): the scores of pair k + 1 and the values of pair k. A wave's VALU work does not issue
 * under its own MFMAs on gfx950 (measured: an MFMA plus 4 independent v_mul cost their sum), but it does under the
 * other wave's on the same SIMD: each wave alternates one VALU stretch and one MFMA stretch, and the two waves of a
 * SIMD fill each other's. (Scores first, then the softmax, made the softmax wait out its own wave's score MFMAs:
 * config 4 8-12 % slower.)
 *
 * Compiled without IEEE mode and NaN semantics (build.py): the maxima of the lazy-max and scale checks need no
 * NaN-quieting canonicalisations then (2-5 % faster, same bits on finite inputs).
 */
#include "layout.h"

#define PF_WAVES 4         /* per workgroup, one per SIMD; two workgroups per CU */
#define PF_THREADS (PF_WAVES * NC_WAVE)
#define PF_BLOCKS 2        /* 16-column MFMA blocks per wave */
#define PF_RING 6          /* page-pair slots (50.7 KB; 3-4 % faster than 8 slots with the fragment-major tiles) */
#define PF_BATCH 2         /* pairs between barriers: the ring is refilled PF_BATCH pairs at a time, and the waves of
                              a SIMD drift up to PF_BATCH pairs apart (3 % faster than a barrier every pair) */
#define PF_PAIR_BYTES (2 * NC_TILE_BYTES)
#define PF_IDS 1024        /* block ids staged per chunk of a segment's pages */
#define PF_BAND 32         /* CUs per XCD: units per band of the unit order */
#define PF_LAZY 8.0f
#define PF_LW_MAX 64 /* the largest power of two folded into p (keeps p w and l finite for zero value scales) */
#define PF_M_INIT -3.0e38f
#define PF_NO_KEY 0x40000000

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) unsigned char lds_u8;

struct PrefillArgs {
    const bf16_t *q;        /* [n][hq][128] */
    int n;
    const uint8_t *cache;   /* [num_blocks][hkv][4224] tiles */
    int max_blocks, num_blocks, num_seqs;
    int window;             /* keys before the query; < 0: all */
    int hq, hkv, group, rows_per_block;
    float score_scale;      /* sm_scale * log2(e) */
    bf16_t *out;            /* [n][hq][128] */
    int tiles;              /* row tiles per kv head */
    int units_per_xcd;
};

__device__ __forceinline__ bf16x8 pf_fp8x8_to_bf16(uint32_t w0, uint32_t w1) {
    const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false);
    const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true);
    const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false);
    const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true);
    return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

/* Dword bb of the V fragments of both pages -> 8 fp16 (keys 4j..4j+3 of the first page, then of the second). */
__device__ __forceinline__ f16x8 pf_v_operand(uint32_t wa, uint32_t wb) {
    const f16x2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(wa, 1.0f, false);
    const f16x2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(wa, 1.0f, true);
    const f16x2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(wb, 1.0f, false);
    const f16x2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(wb, 1.0f, true);
    return f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

__device__ __forceinline__ float pf_exp2i(int e) { return __uint_as_float((uint32_t)(e + 127) << 23); }

__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v = min(v, __shfl_xor(v, d, 64));
    return v;
}

__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v = max(v, __shfl_xor(v, d, 64));
    return v;
}

template <int N> __device__ __forceinline__ void pf_wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

/* A ring slot holds a page pair as [A: K 2 KiB, V 2 KiB][B: K, V][A: K and V scales 128 B][B: scales]. Its 8
 * fragments of 1 KiB (per page the tile's four contiguous parts: K bytes 0-15 / 16-31 of every lane, V bytes
 * 0-15 / 16-31) are spread over the waves, 2 each; the last wave also loads both pages' scales with one dword DMA
 * of all 64 lanes (lane l: page l / 32, bytes 4 (l % 32) of its scales). No DMA runs under a partial exec mask:
 * the compiler may merge two exec-masked DMAs of different LDS destinations into one whose M0 (the destination,
 * which must be wave-uniform) comes from a divergent value. Per-lane byte offsets within a tile are fixed for the
 * whole loop; the tile base is wave-uniform. */
#define PF_FRAGS (8 / PF_WAVES)         /* fragments per wave and pair */
#define PF_SLOT_SCALES (4 * NC_TILE_V)  /* 8192: both pages' scales */
#define PF_SCALE_WAVE (PF_WAVES - 1)
struct PfDma {
    uint32_t frag[PF_FRAGS];
    int page[PF_FRAGS], part[PF_FRAGS];
    uint32_t scale; /* the scale DMA's lane offset within its page's tile */
    int scale_page;
};

__device__ __forceinline__ PfDma dma_plan(int wv, int lane) {
    const int n = lane & 15, j = lane >> 4;
    PfDma d;
#pragma unroll
    for (int i = 0; i < PF_FRAGS; i++) {
        const int f = wv * PF_FRAGS + i;
        d.page[i] = f >> 2;
        d.part[i] = f & 3;
        d.frag[i] = d.part[i] * NC_TILE_PART + 16 * (n + 16 * j);
    }
    d.scale_page = lane >> 5;
    d.scale = NC_TILE_KS + 4 * (lane & 31);
    return d;
}

__device__ __forceinline__ void dma_pair(const PrefillArgs &a, int blk0, int blk1, int h, const PfDma &d, int wv,
                                         unsigned char *slot) {
    blk0 = blk0 < 0 ? 0 : blk0; /* no block: load block 0, masked later */
    blk1 = blk1 < 0 ? 0 : blk1;
    const uint8_t *t0 = a.cache + ((size_t)blk0 * a.hkv + h) * NC_TILE_BYTES;
    const uint8_t *t1 = a.cache + ((size_t)blk1 * a.hkv + h) * NC_TILE_BYTES;
#pragma unroll
    for (int i = 0; i < PF_FRAGS; i++)
        __builtin_amdgcn_global_load_lds((d.page[i] ? t1 : t0) + d.frag[i],
                                         slot + d.page[i] * 2 * NC_TILE_V + d.part[i] * 1024, 16, 0, 0);
    if (wv == PF_SCALE_WAVE) /* wave-uniform */
        __builtin_amdgcn_global_load_lds((d.scale_page ? t1 : t0) + d.scale, slot + PF_SLOT_SCALES, 4, 0, 0);
}

/* Wait until at most this wave's DMAs of its last N pairs are in flight. */
template <int N> __device__ __forceinline__ void pf_wait_pairs(int wv) {
    if (wv == PF_SCALE_WAVE)
        pf_wait_vmcnt<(PF_FRAGS + 1) * N>();
    else
        pf_wait_vmcnt<PF_FRAGS * N>();
}

/* K fragments of a pair for the score MFMAs: dims 32j.. of key n, both pages. */
struct PfKeys {
    u32x4 a0, a1, b0, b1;
};

/* V quad fragments of a pair for the value MFMAs (dims 8n.. of keys 4j..4j+3, both pages), and the K and V scales
 * of keys 4j..4j+3 of both pages. */
struct PfVals {
    u32x4 a0, a1, b0, b1, ks_a, ks_b, vs_a, vs_b;
};

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const lds_u8 *)(const unsigned char *)p;
}

/* The keys of slot_k, the block ids of pair `pair_k` and of pair `pair_dma` (the next refill). Inline ds_reads with
 * their own lgkmcnt wait: as plain LDS loads the compiler would precede them with s_waitcnt vmcnt(0) (it cannot
 * tell them from the ring's in-flight DMA writes) and drain the ring. */
__device__ __forceinline__ void read_keys(const unsigned char *slot_k, const int *ids, int pair_k, int pair_dma,
                                          int lane, PfKeys &k, u32x2 &ids_k, u32x2 &ids_dma) {
    const uint32_t mk = lds_addr(slot_k) + 16 * lane;
    asm volatile(
        "ds_read_b128 %0, %6\n"
        "ds_read_b128 %1, %6 offset:1024\n"
        "ds_read_b128 %2, %6 offset:4096\n"
        "ds_read_b128 %3, %6 offset:5120\n"
        "ds_read_b64 %4, %7\n"
        "ds_read_b64 %5, %8\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(k.a0), "=&v"(k.a1), "=&v"(k.b0), "=&v"(k.b1), "=&v"(ids_k), "=&v"(ids_dma)
        : "v"(mk), "v"(lds_addr(ids + 2 * pair_k)), "v"(lds_addr(ids + 2 * pair_dma))
        : "memory");
}

/* The scales of slot_v (the pair whose softmax runs this step) and two pairs' block ids: what the softmax reads. */
__device__ __forceinline__ void read_scales(const unsigned char *slot_v, const int *ids, int pair_k, int pair_dma,
                                            int lane, PfVals &v, u32x2 &ids_k, u32x2 &ids_dma) {
    const uint32_t sv = lds_addr(slot_v) + PF_SLOT_SCALES + 16 * (lane >> 4);
    asm volatile(
        "ds_read_b128 %0, %6\n"
        "ds_read_b128 %1, %6 offset:128\n"
        "ds_read_b128 %2, %6 offset:64\n"
        "ds_read_b128 %3, %6 offset:192\n"
        "ds_read_b64 %4, %7\n"
        "ds_read_b64 %5, %8\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v.ks_a), "=&v"(v.ks_b), "=&v"(v.vs_a), "=&v"(v.vs_b), "=&v"(ids_k), "=&v"(ids_dma)
        : "v"(sv), "v"(lds_addr(ids + 2 * pair_k)), "v"(lds_addr(ids + 2 * pair_dma))
        : "memory");
}

/* The value fragments of slot_v and the key fragments of slot_k: what the step's MFMA burst reads. Read after the
 * softmax, so the fragments are not live across it. */
__device__ __forceinline__ void read_frags(const unsigned char *slot_v, const unsigned char *slot_k, int lane,
                                           PfVals &v, PfKeys &k) {
    const uint32_t mv = lds_addr(slot_v) + 16 * lane, mk = lds_addr(slot_k) + 16 * lane;
    asm volatile(
        "ds_read_b128 %0, %8\n"
        "ds_read_b128 %1, %8 offset:1024\n"
        "ds_read_b128 %2, %8 offset:4096\n"
        "ds_read_b128 %3, %8 offset:5120\n"
        "ds_read_b128 %4, %9 offset:2048\n"
        "ds_read_b128 %5, %9 offset:3072\n"
        "ds_read_b128 %6, %9 offset:6144\n"
        "ds_read_b128 %7, %9 offset:7168\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(k.a0), "=&v"(k.a1), "=&v"(k.b0), "=&v"(k.b1), "=&v"(v.a0), "=&v"(v.a1), "=&v"(v.b0), "=&v"(v.b1)
        : "v"(mk), "v"(mv)
        : "memory");
}

/* The online-softmax state of a wave's 4 blocks, lane (j, n): column n's reference max m[bl] and this lane's
 * partial sum l[bl]; Oᵀ in o[bl][bb][i] = dim 8 (4j + i) + bb of column n. Both carry the factor w = 2^lw,
 * lw = min(126 - e_ref, PF_LW_MAX) with e_ref the largest v_scale exponent so far: p w v_scale < 2^9 stays in
 * fp16 for the value MFMAs, and w folds into the exponent, p w = exp2(s k_scale score_scale - m + lw). */
struct PfState {
    f32x4 o[PF_BLOCKS][8];
    float m[PF_BLOCKS], l[PF_BLOCKS];
    float mo[PF_BLOCKS];   /* lw - m: t = s k_scale score_scale + mo = log2(p w) */
    /* per column, like m: a column's state follows its own keys only, so its result does not depend on the rows
     * that share its wave */
    float vlim[PF_BLOCKS]; /* 2^(e_ref - 126): a v_scale at or above it raises e_ref */
    int e_ref[PF_BLOCKS];  /* the largest v_scale exponent (biased) among the column's keys so far */
    float lazy[PF_BLOCKS]; /* PF_LAZY + lw */
    int lw[PF_BLOCKS];     /* log2 w = min(126 - e_ref, PF_LW_MAX) */
};

/* A wave's view of the segment being attended: per column the key range [lo, hi] (lo > hi: masked throughout),
 * and the wave-uniform bounds under which a page pair needs no mask. */
struct PfCols {
    int lo[PF_BLOCKS], hi[PF_BLOCKS];
    int max_lo, min_hi; /* over the wave's columns of the segment */
    int seg_lo, seg_hi; /* the workgroup's union key range */
    bool masked_always; /* a column of another sequence sits in this wave */
    bool active;        /* the wave has a column of the segment */
};

/* q of one block as the fp8 score operand: q 2^e = hi + lo in e4m3, e per column; scale = the E8M0 byte of 2^-e. */
struct PfQ8 {
    i32x8 hi, lo;
    int scale;
};

typedef short pf_i16x2 __attribute__((ext_vector_type(2)));

/* 32 bf16 of q (this lane's dims 32j .. 32j+31 of its column) -> the two e4m3 terms (exact for a bf16 value whose low
 * term stays in e4m3's normal range: 4 + 4 significant bits); the column's exponent from its absmax over the four
 * lanes holding it (xor 16, 32). A zero column gives zero terms. A column holding an infinity or a NaN (the append's
 * q rows past the rotary table) sets `bad` on its four lanes and gives zero terms: no NaN enters the MFMAs of a
 * kernel compiled without NaN semantics. The test is on the bf16 bits (exponent all ones), which that compilation
 * cannot fold away. */
__device__ PfQ8 quantize_q(const u32x4 (&u)[4], bool &bad) {
#pragma clang fp contract(off)
    uint32_t nonfinite = 0;
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int i = 0; i < 4; i++)
            nonfinite |= ((u[c][i] & 0x7f80u) == 0x7f80u) | ((u[c][i] & 0x7f800000u) == 0x7f800000u);
    nonfinite |= (uint32_t)__shfl_xor((int)nonfinite, 16, 64);
    nonfinite |= (uint32_t)__shfl_xor((int)nonfinite, 32, 64);
    bad = nonfinite != 0;
    const uint32_t keep = bad ? 0u : 0xffffffffu;
    float x[32];
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            x[8 * c + 2 * i] = __uint_as_float((u[c][i] << 16) & keep);
            x[8 * c + 2 * i + 1] = __uint_as_float(u[c][i] & 0xffff0000u & keep);
        }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[i]));
    amax = fmaxf(amax, shfl_xor_f(amax, 16));
    amax = fmaxf(amax, shfl_xor_f(amax, 32));
    /* amax in [2^ea, 2^(ea+1)): with e = 7 - ea, |q| 2^e < 2^8 <= 448 */
    const int ea = amax > 0.f ? (int)((__float_as_uint(amax) >> 23) & 0xffu) - 127 : 0;
    const int e = max(min(7 - ea, 127), -126);
    const float up = __uint_as_float((uint32_t)(e + 127) << 23);
    PfQ8 q;
    q.scale = max(min(127 - e, 254), 0);
    /* the hardware conversions (round to nearest even; |v| < 256 is in range): byte b of a dword is element b */
#pragma unroll
    for (int w = 0; w < 8; w++) {
        float v[4];
#pragma unroll
        for (int b = 0; b < 4; b++) v[b] = x[4 * w + b] * up; /* exact: a power of two */
        pf_i16x2 h = {0, 0}, l = {0, 0};
        h = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(h, v[0], v[1], 1.0f, false);
        h = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(h, v[2], v[3], 1.0f, true);
        const uint32_t hu = __builtin_bit_cast(uint32_t, h);
        const f32x2 d01 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hu, 1.0f, false);
        const f32x2 d23 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hu, 1.0f, true);
        /* the remainders v - hi are exact in fp32 */
        l = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(l, v[0] - d01[0], v[1] - d01[1], 1.0f, false);
        l = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(l, v[2] - d23[0], v[3] - d23[1], 1.0f, true);
        q.hi[w] = (int)hu;
        q.lo[w] = __builtin_bit_cast(int, l);
    }
    return q;
}

/* Scores of a pair for every block: s[bl][0] page A, s[bl][1] page B, lane (j, n) keys 4j..4j+3 of column n. */
__device__ __forceinline__ void pair_scores(const PfKeys &k, const PfQ8 *q8, f32x4 (*s)[2]) {
    const i32x8 ka = __builtin_bit_cast(i32x8, u32x8{k.a0[0], k.a0[1], k.a0[2], k.a0[3], k.a1[0], k.a1[1], k.a1[2],
                                                     k.a1[3]});
    const i32x8 kb = __builtin_bit_cast(i32x8, u32x8{k.b0[0], k.b0[1], k.b0[2], k.b0[3], k.b1[0], k.b1[1], k.b1[2],
                                                     k.b1[3]});
#pragma unroll
    for (int bl = 0; bl < PF_BLOCKS; bl++) {
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        f32x4 sa = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ka, q8[bl].hi, z, 0, 0, 0, 127, 0, q8[bl].scale);
        f32x4 sb = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(kb, q8[bl].hi, z, 0, 0, 0, 127, 0, q8[bl].scale);
        s[bl][0] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ka, q8[bl].lo, sa, 0, 0, 0, 127, 0, q8[bl].scale);
        s[bl][1] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(kb, q8[bl].lo, sb, 0, 0, 0, 127, 0, q8[bl].scale);
    }
}

/* Softmax of a pair whose scores are s (keys of pages page0, page0 + 1 with blocks ida, idb) and whose scales are
 * v's: t = s k_scale score_scale - m + lw, so exp2(t) = p w; pp receives Pᵀ = p w v_scale in fp16, the value MFMAs'
 * B operand. */
__device__ __forceinline__ void pair_softmax(const PrefillArgs &a, const f32x4 (*s)[2], const PfVals &v, int ida,
                                             int idb, int page0, const PfCols &c, int j, PfState &st,
                                             f16x8 (&pp)[PF_BLOCKS]) {
    float ksc[8], vs[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        ksc[i] = __uint_as_float(v.ks_a[i]) * a.score_scale;
        ksc[4 + i] = __uint_as_float(v.ks_b[i]) * a.score_scale;
        vs[i] = __uint_as_float(v.vs_a[i]);
        vs[4 + i] = __uint_as_float(v.vs_b[i]);
    }
    float t[PF_BLOCKS][8];
#pragma unroll
    for (int bl = 0; bl < PF_BLOCKS; bl++)
#pragma unroll
        for (int i = 0; i < 8; i++) t[bl][i] = __builtin_fmaf(s[bl][i >> 2][i & 3], ksc[i], st.mo[bl]);
    /* masks: wave-uniform test, per-lane keys only on pairs that need it */
    const int key0 = page0 * NC_PAGE + 4 * j;
    const bool fast = ida >= 0 && idb >= 0 && !c.masked_always && page0 * NC_PAGE >= c.max_lo &&
                      page0 * NC_PAGE + 2 * NC_PAGE - 1 <= c.min_hi;
    unsigned ok[PF_BLOCKS];
    float vm[PF_BLOCKS]; /* the largest v_scale among the keys each column keeps (this lane's 8) */
    {
        const float vmax = fmaxf(fmaxf(fmaxf(vs[0], vs[1]), fmaxf(vs[2], vs[3])),
                                 fmaxf(fmaxf(vs[4], vs[5]), fmaxf(vs[6], vs[7])));
#pragma unroll
        for (int bl = 0; bl < PF_BLOCKS; bl++) {
            ok[bl] = 0xffu;
            vm[bl] = vmax; /* a pair on the fast path: every column keeps every key */
        }
    }
    if (!fast) {
#pragma unroll
        for (int bl = 0; bl < PF_BLOCKS; bl++) vm[bl] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int key = key0 + (i < 4 ? i : NC_PAGE + i - 4);
            const bool pg_ok = i < 4 ? ida >= 0 : idb >= 0;
            const bool in_seg = pg_ok && key >= c.seg_lo && key <= c.seg_hi;
            vs[i] = in_seg ? vs[i] : 0.f;
#pragma unroll
            for (int bl = 0; bl < PF_BLOCKS; bl++) {
                const bool keep = in_seg && key >= c.lo[bl] && key <= c.hi[bl];
                ok[bl] &= ~((keep ? 0u : 1u) << i);
                t[bl][i] = keep ? t[bl][i] : -INFINITY;
                vm[bl] = fmaxf(vm[bl], keep ? vs[i] : 0.f);
            }
        }
    }
    bool need[PF_BLOCKS], any_need = false;
#pragma unroll
    for (int bl = 0; bl < PF_BLOCKS; bl++) {
        const float tm = fmaxf(fmaxf(fmaxf(t[bl][0], t[bl][1]), fmaxf(t[bl][2], t[bl][3])),
                               fmaxf(fmaxf(t[bl][4], t[bl][5]), fmaxf(t[bl][6], t[bl][7])));
        need[bl] = tm > st.lazy[bl];
        any_need |= need[bl];
    }
    if (__any(any_need)) {
        /* rare: a column whose score passed its lazy bound moves its reference max to its exact max over its keys
         * so far; the others keep m, mo, o, l and t bit for bit */
#pragma unroll
        for (int bl = 0; bl < PF_BLOCKS; bl++) {
            int cn = need[bl] ? 1 : 0; /* the column's decision: any of its 4 lanes */
            cn |= __shfl_xor(cn, 16, 64);
            cn |= __shfl_xor(cn, 32, 64);
            float xm = -INFINITY;
#pragma unroll
            for (int i = 0; i < 8; i++)
                xm = fmaxf(xm, (ok[bl] >> i) & 1 ? s[bl][i >> 2][i & 3] * ksc[i] : -INFINITY);
            xm = fmaxf(xm, shfl_xor_f(xm, 16));
            xm = fmaxf(xm, shfl_xor_f(xm, 32));
            const float m_new = fmaxf(st.m[bl], xm);
            const float alpha = cn ? __builtin_amdgcn_exp2f(st.m[bl] - m_new) : 1.f; /* x 1: exact */
            st.l[bl] *= alpha;
#pragma unroll
            for (int bb = 0; bb < 8; bb++) st.o[bl][bb] *= alpha;
            st.m[bl] = cn ? m_new : st.m[bl];
            st.mo[bl] = cn ? (float)st.lw[bl] - m_new : st.mo[bl];
            /* every column's t again, by the fast path's FMA (the same bits where mo did not move); mo through an
             * empty asm, so the compiler does not keep the unmasked FMA results alive across the masked path to
             * reuse them here */
            float mo_b = st.mo[bl];
            asm volatile("" : "+v"(mo_b));
#pragma unroll
            for (int i = 0; i < 8; i++)
                t[bl][i] = (ok[bl] >> i) & 1 ? __builtin_fmaf(s[bl][i >> 2][i & 3], ksc[i], mo_b) : -INFINITY;
        }
    }
    bool vneed = false;
#pragma unroll
    for (int bl = 0; bl < PF_BLOCKS; bl++) vneed |= vm[bl] >= st.vlim[bl];
    if (__any(vneed)) {
        /* rare: a column met a larger v_scale exponent: its w = 2^lw drops, and its o, l and t follow. The others
         * have d = 0: x 1 and + 0 keep their bits (mo and t are never -0: round-to-nearest differences and FMAs of
         * a nonzero mo give +0) */
#pragma unroll
        for (int bl = 0; bl < PF_BLOCKS; bl++) {
            float vx = fmaxf(vm[bl], shfl_xor_f(vm[bl], 16));
            vx = fmaxf(vx, shfl_xor_f(vx, 32));
            const int e_new = max(st.e_ref[bl], (int)(__float_as_uint(vx) >> 23));
            const int lw_new = min(126 - e_new, PF_LW_MAX), d = lw_new - st.lw[bl];
            const float r = pf_exp2i(max(d, -126));
#pragma unroll
            for (int bb = 0; bb < 8; bb++) st.o[bl][bb] *= r;
            st.l[bl] *= r;
            st.mo[bl] += (float)d;
#pragma unroll
            for (int i = 0; i < 8; i++) t[bl][i] += (float)d;
            st.lw[bl] = lw_new;
            st.lazy[bl] = PF_LAZY + (float)lw_new;
            st.e_ref[bl] = e_new;
            st.vlim[bl] = pf_exp2i(min(e_new - 126, 127));
        }
    }
#pragma unroll
    for (int bl = 0; bl < PF_BLOCKS; bl++) {
        float p[8];
#pragma unroll
        for (int i = 0; i < 8; i++) p[i] = __builtin_amdgcn_exp2f(t[bl][i]);
        st.l[bl] += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
#pragma unroll
        for (int i = 0; i < 8; i++) pp[bl][i] = (_Float16)(p[i] * vs[i]);
    }
}

/* The value MFMAs of a pair: Oᵀ += Vᵀ Pᵀ, V's fp8 codes converted exactly to fp16. */
__device__ __forceinline__ void pair_values(const PfVals &v, const f16x8 (&pp)[PF_BLOCKS], PfState &st) {
#pragma unroll
    for (int bb = 0; bb < 8; bb++) {
        const uint32_t wa = bb < 4 ? v.a0[bb] : v.a1[bb - 4];
        const uint32_t wb = bb < 4 ? v.b0[bb] : v.b1[bb - 4];
        const f16x8 va = pf_v_operand(wa, wb);
#pragma unroll
        for (int bl = 0; bl < PF_BLOCKS; bl++)
            st.o[bl][bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pp[bl], st.o[bl][bb], 0, 0, 0);
    }
}

__device__ __forceinline__ bool row_valid(const PrefillArgs &a, int p, int s) {
    return p >= 0 && s >= 0 && s < a.num_seqs;
}

/* Bit k of bits: tile row k's q holds an infinity or a NaN. */
__device__ __forceinline__ bool row_bad(const unsigned *bits, int k) { return (bits[k >> 5] >> (k & 31)) & 1u; }

/* The first key of a row at position p. */
__device__ __forceinline__ int key_lo(const PrefillArgs &a, int p) {
    return (a.window < 0 || p <= a.window) ? 0 : p - a.window;
}

__global__ void __launch_bounds__(PF_THREADS, 2)
    k_prefill(PrefillArgs a, const int32_t *__restrict__ pos, const int32_t *__restrict__ seq,
              const int32_t *__restrict__ block_table) {
    __shared__ __attribute__((aligned(16))) unsigned char ring[PF_RING * PF_PAIR_BYTES];
    __shared__ __attribute__((aligned(16))) int ids[PF_IDS];
    __shared__ int2 rows_ps[PF_WAVES * PF_BLOCKS * 16]; /* the tile's (position, sequence) pairs */
    __shared__ unsigned rows_bad[PF_WAVES * PF_BLOCKS * 16 / 32]; /* rows whose q is not finite */

    /* XCD-aware unit order: workgroup b runs on XCD b % 8, which takes a contiguous range of units, so the row
     * tiles of one (sequence, kv head) -- the readers of the same pages -- share an L2. Within the range, every
     * second band of PF_BAND units (one workgroup per CU of the XCD) runs in reverse: the two workgroups that share
     * a CU then hold tiles from opposite ends of a band, whose key ranges differ most in a causal prefill, and the
     * slots turn over at different times (16 x 2047 causal rows, G = 1: 1.14x the speed of the plain order). A
     * trailing partial band keeps its order. */
    const int li = blockIdx.x >> 3, band = li / PF_BAND, lpos = li % PF_BAND;
    const bool flip = (band & 1) && (band + 1) * PF_BAND <= a.units_per_xcd;
    const int unit = (blockIdx.x & 7) * a.units_per_xcd + band * PF_BAND + (flip ? PF_BAND - 1 - lpos : lpos);
    if (li >= a.units_per_xcd || unit >= a.hkv * a.tiles) return;
    const int h = unit / a.tiles, tile = unit % a.tiles;
    /* the wave index is wave-uniform: readfirstlane lets the compiler keep what derives from it in scalars */
    const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, n = lane & 15,
              j = lane >> 4;
    const int G = a.group, R = a.rows_per_block, TR = PF_WAVES * PF_BLOCKS * R;
    const int row0 = tile * TR;

    /* this lane's q operands: column n of block bl is row row0 + (wv PF_BLOCKS + bl) R + n / G, head h G + n % G */
    PfQ8 q8[PF_BLOCKS];
    unsigned qbad = 0; /* bit bl: this lane's column of block bl is a used row whose q is not finite */
#pragma unroll
    for (int bl = 0; bl < PF_BLOCKS; bl++) {
        const int r = row0 + (wv * PF_BLOCKS + bl) * R + n / G;
        const bool used = n < R * G && r < a.n;
        const bf16_t *qr = a.q + ((size_t)(used ? r : 0) * a.hq + h * G + n % G) * NC_HEAD_DIM + 32 * j;
        u32x4 u[4];
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
            u[kk] = used ? *reinterpret_cast<const u32x4 *>(qr + 8 * kk) : u32x4{0u, 0u, 0u, 0u};
        bool bad;
        q8[bl] = quantize_q(u, bad);
        qbad |= (used && bad) ? 1u << bl : 0u;
    }

    PfState st;
#pragma unroll
    for (int bl = 0; bl < PF_BLOCKS; bl++) {
#pragma unroll
        for (int bb = 0; bb < 8; bb++) st.o[bl][bb] = f32x4{0.f, 0.f, 0.f, 0.f};
        st.m[bl] = PF_M_INIT;
        st.l[bl] = 0.f;
    }
#pragma unroll
    for (int bl = 0; bl < PF_BLOCKS; bl++) {
        st.e_ref[bl] = 0;
        st.vlim[bl] = pf_exp2i(-126);
        st.lw[bl] = PF_LW_MAX;
        st.lazy[bl] = PF_LAZY + (float)PF_LW_MAX;
    }
#pragma unroll
    for (int bl = 0; bl < PF_BLOCKS; bl++) st.mo[bl] = (float)PF_LW_MAX - PF_M_INIT;

    /* the tile's positions and sequences, read once into LDS ((-1, -1) past the rows) */
    for (int k = tid; k < TR; k += PF_THREADS) {
        const int r = row0 + k;
        rows_ps[k] = r < a.n ? make_int2(pos[r], seq[r]) : make_int2(-1, -1);
    }
    if (tid < PF_WAVES * PF_BLOCKS * 16 / 32) rows_bad[tid] = 0u; /* every word: TR need not be a multiple of 32 */
    __syncthreads();
    /* rows whose q is not finite: attended by no segment (like invalid rows), NaN rows at the end */
#pragma unroll
    for (int bl = 0; bl < PF_BLOCKS; bl++) {
        const int k = (wv * PF_BLOCKS + bl) * R + n / G;
        if ((qbad >> bl) & 1u && j == 0) atomicOr(&rows_bad[k >> 5], 1u << (k & 31));
    }
    __syncthreads();

    /* rows of the tile still to attend, 4 per lane (row0 + lane + 64 i); every wave derives the same segments */
    unsigned pend = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int k = lane + 64 * i;
        if (k < TR && row_valid(a, rows_ps[k].x, rows_ps[k].y) && !row_bad(rows_bad, k)) pend |= 1u << i;
    }

    for (;;) {
        /* a sequence with rows still to attend: its rows form the segment */
        int s = -1;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const unsigned long long bal = __ballot((pend >> i) & 1);
            if (s < 0 && bal) {
                const int src = __builtin_ctzll(bal);
                s = __shfl((pend >> i) & 1 ? rows_ps[lane + 64 * i].y : -1, src, 64);
            }
        }
        s = __builtin_amdgcn_readfirstlane(s);
        if (s < 0) break;
        int lo = PF_NO_KEY, hi = -1;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int k = lane + 64 * i;
            if ((pend >> i) & 1 && rows_ps[k].y == s) {
                const int p = rows_ps[k].x;
                lo = min(lo, key_lo(a, p));
                hi = max(hi, p);
                pend &= ~(1u << i);
            }
        }
        lo = __builtin_amdgcn_readfirstlane(wave_min_i(lo));
        hi = __builtin_amdgcn_readfirstlane(wave_max_i(hi));

        PfCols c;
        int wmax_lo = -1, wmin_hi = PF_NO_KEY;
        bool other = false, mine = false;
#pragma unroll
        for (int bl = 0; bl < PF_BLOCKS; bl++) {
            const int r = row0 + (wv * PF_BLOCKS + bl) * R + n / G;
            const bool used = n < R * G && r < a.n;
            const int2 ps = used ? rows_ps[r - row0] : make_int2(-1, -1);
            const int p = ps.x, sq = ps.y;
            const bool ok = used && row_valid(a, p, sq) && !row_bad(rows_bad, r - row0), in_seg = ok && sq == s;
            other |= ok && !in_seg;
            mine |= in_seg;
            c.lo[bl] = in_seg ? key_lo(a, p) : (ok ? PF_NO_KEY : 0);
            c.hi[bl] = in_seg ? p : (ok ? -1 : PF_NO_KEY);
            if (in_seg) {
                wmax_lo = max(wmax_lo, key_lo(a, p));
                wmin_hi = min(wmin_hi, p);
            }
        }
        c.max_lo = __builtin_amdgcn_readfirstlane(wave_max_i(wmax_lo));
        c.min_hi = __builtin_amdgcn_readfirstlane(wave_min_i(wmin_hi));
        c.masked_always = __any(other);
        c.active = __any(mine);
        c.seg_lo = lo;
        c.seg_hi = hi;

        /* pairs start at even pages whatever the segment's first key: a column meets its keys in the same pairs,
         * slots and sum trees whichever rows share its workgroup (pages before lo are masked) */
        const int first = (lo / NC_PAGE) & ~1, npages = hi / NC_PAGE - first + 1;
        for (int cb = 0; cb < npages; cb += PF_IDS) {
            const int cp = min(PF_IDS, npages - cb), npairs = (cp + 1) / 2;
            __syncthreads(); /* the previous chunk's ring and ids are no longer read */
            for (int e = tid; e < 2 * npairs; e += PF_THREADS)
                ids[e] = e < cp ? lookup_block(block_table, a.max_blocks, a.num_blocks, s, first + cb + e) : -1;
            __syncthreads();
            const PfDma dp = dma_plan(wv, lane);
            /* the ring: pair p in slot p % PF_RING; pairs 0..PRO - 1 in flight before step 0, and the batch starting
             * at step k (k % PF_BATCH == 0) refills the slots of pairs k - PF_BATCH .. k - 1 with pairs
             * k + PRO .. k + PF_RING - 1 (past the end: the last pair again) */
            constexpr int PRO = PF_RING - PF_BATCH;
            static_assert(PF_RING >= 2 * PF_BATCH + 1, "ring depth for the batch");
            int pro[PRO][2];
#pragma unroll
            for (int k = 0; k < PRO; k++) {
                pro[k][0] = __builtin_amdgcn_readfirstlane(ids[2 * min(k, npairs - 1)]);
                pro[k][1] = __builtin_amdgcn_readfirstlane(ids[2 * min(k, npairs - 1) + 1]);
            }
#pragma unroll
            for (int k = 0; k < PRO; k++) {
                __builtin_amdgcn_sched_barrier(0);
                dma_pair(a, pro[k][0], pro[k][1], h, dp, wv, ring + k * PF_PAIR_BYTES);
            }
            __builtin_amdgcn_sched_barrier(0);
            /* pipeline fill: the scores of pair 0 */
            pf_wait_pairs<PRO - 1>(wv); /* this wave's DMAs of pair 0 have landed */
            __builtin_amdgcn_s_barrier();                      /* everyone's have */
            __builtin_amdgcn_sched_barrier(0);
            PfKeys kf;
            u32x2 ids_cur, ids_dma;
            read_keys(ring, ids, 0, min(PF_RING - 1, npairs - 1), lane, kf, ids_cur, ids_dma);
            f32x4 s0[PF_BLOCKS][2], s1[PF_BLOCKS][2];
            if (c.active) pair_scores(kf, q8, s0);
            __builtin_amdgcn_sched_barrier(0);
            /* iteration k: the scores of pair k + 1 into one buffer while pair k's softmax and values read the other
             * (unrolled twice so the buffers swap without copies) */
            auto step = [&](int k, f32x4 (*s_cur)[2], f32x4 (*s_next)[2]) {
                if (k % PF_BATCH == 0) {
                    /* this wave's DMAs of pairs <= k + PF_BATCH have landed (later ones may fly) */
                    pf_wait_pairs<PF_RING - 1 - 2 * PF_BATCH>(wv);
                    __builtin_amdgcn_s_barrier(); /* everyone's have; the slots of pairs < k are free */
                    __builtin_amdgcn_sched_barrier(0);
                }
                PfVals vf;
                u32x2 ids_next;
                read_scales(ring + (k % PF_RING) * PF_PAIR_BYTES, ids, min(k + 1, npairs - 1), min(k + 1, npairs - 1),
                            lane, vf, ids_next, ids_dma);
                __builtin_amdgcn_sched_barrier(0);
                if (c.active) {
                    /* the softmax of pair k, then all of the step's MFMAs in one burst at raised priority: the
                     * scores of pair k + 1 (past the end: the clamped refill, unused) and the values of pair k */
                    f16x8 pp[PF_BLOCKS];
                    pair_softmax(a, s_cur, vf, __builtin_amdgcn_readfirstlane((int)ids_cur[0]),
                                 __builtin_amdgcn_readfirstlane((int)ids_cur[1]), first + cb + 2 * k, c, j, st, pp);
                    __builtin_amdgcn_sched_barrier(0);
                    read_frags(ring + (k % PF_RING) * PF_PAIR_BYTES, ring + ((k + 1) % PF_RING) * PF_PAIR_BYTES, lane,
                               vf, kf);
                    __builtin_amdgcn_sched_barrier(0);
                    __builtin_amdgcn_s_setprio(1);
                    pair_scores(kf, q8, s_next);
                    pair_values(vf, pp, st);
                    __builtin_amdgcn_s_setprio(0);
                }
                if (k % PF_BATCH == 0) {
                    /* the freed slots take pairs k + PRO.. after the step's work (the ring holds them PRO pairs
                     * ahead, so they are not late): issued before it, the block-id reads and DMA burst held up the
                     * step's own LDS reads and softmax */
                    u32x2 id[PF_BATCH];
#pragma unroll
                    for (int bb = 0; bb < PF_BATCH; bb++) {
                        const uint32_t at = lds_addr(ids + 2 * min(k + PRO + bb, npairs - 1));
                        asm volatile("ds_read_b64 %0, %1" : "=v"(id[bb]) : "v"(at) : "memory");
                    }
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
                    for (int bb = 0; bb < PF_BATCH; bb++) {
                        asm volatile("" : "+v"(id[bb]));
                        dma_pair(a, __builtin_amdgcn_readfirstlane((int)id[bb][0]),
                                 __builtin_amdgcn_readfirstlane((int)id[bb][1]), h, dp, wv,
                                 ring + ((k + PRO + bb) % PF_RING) * PF_PAIR_BYTES);
                    }
                }
                ids_cur = ids_next;
                __builtin_amdgcn_sched_barrier(0);
            };
            for (int k = 0; k < npairs; k += 2) {
                step(k, s0, s1);
                if (k + 1 < npairs) step(k + 1, s1, s0);
            }
            pf_wait_vmcnt<0>(); /* the clamped refills past the last pair */
        }
    }

    /* normalise and store; rows with an invalid position or sequence get zeros, other rows whose q (the G heads of
     * this kv head) is not finite NaN (as the decode step's rows past the rotary table) */
#pragma unroll
    for (int bl = 0; bl < PF_BLOCKS; bl++) {
        float l = st.l[bl];
        l += shfl_xor_f(l, 16);
        l += shfl_xor_f(l, 32);
        const int r = row0 + (wv * PF_BLOCKS + bl) * R + n / G;
        if (!(n < R * G && r < a.n)) continue;
        const int2 ps = rows_ps[r - row0];
        const bool valid = row_valid(a, ps.x, ps.y), nan_row = valid && row_bad(rows_bad, r - row0);
        const bool zero = !(valid && l > 0.f); /* +0, not o * 0 (which keeps signs) */
        const float inv = zero ? 0.f : 1.0f / l; /* o and l both carry w */
        bf16_t *dst = a.out + ((size_t)r * a.hq + h * G + n % G) * NC_HEAD_DIM;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float v[8];
#pragma unroll
            for (int bb = 0; bb < 8; bb++) v[bb] = zero ? 0.f : st.o[bl][bb][i] * inv;
            u32x4 bits;
#pragma unroll
            for (int c = 0; c < 4; c++) bits[c] = f32x2_to_bf16x2(v[2 * c], v[2 * c + 1]);
            if (nan_row) bits = u32x4{0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u};
            *reinterpret_cast<u32x4 *>(dst + (4 * j + i) * 8) = bits;
        }
    }
}

extern "C" int nc_prefill_attn_fp8(const void *q, const int32_t *pos, const int32_t *seq, int n,
                                   const uint8_t *cache, const int32_t *block_table, int max_blocks, int num_blocks,
                                   int num_seqs, int window, int hq, int hkv, float sm_scale, void *out,
                                   void *stream) {
    NC_REQUIRE(n >= 0, "nc_prefill_attn_fp8: n = %d < 0", n);
    NC_REQUIRE(hq > 0 && hkv > 0 && hq % hkv == 0 && hq / hkv <= 16,
               "nc_prefill_attn_fp8: need hq %% hkv == 0 and 1 <= hq / hkv <= 16 (hq %d, hkv %d)", hq, hkv);
    NC_REQUIRE(max_blocks > 0 && num_blocks > 0 && num_seqs > 0,
               "nc_prefill_attn_fp8: max_blocks %d, num_blocks %d, num_seqs %d must be positive", max_blocks,
               num_blocks, num_seqs);
    NC_REQUIRE((long long)num_blocks * hkv * NC_TILE_BYTES < (1ll << 47), "nc_prefill_attn_fp8: pool too large");
    NC_REQUIRE(block_table || (long long)num_seqs * max_blocks <= num_blocks,
               "nc_prefill_attn_fp8: a contiguous cache needs num_seqs * max_blocks <= num_blocks");
    if (n == 0) return 0;
    NC_REQUIRE(q && pos && seq && cache && out, "nc_prefill_attn_fp8: null pointer");
    NC_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)out & 15) == 0 && ((uintptr_t)cache & 15) == 0,
               "nc_prefill_attn_fp8: q, out and cache must be 16-byte aligned");
    PrefillArgs a;
    a.q = static_cast<const bf16_t *>(q);
    a.n = n;
    a.cache = cache;
    a.max_blocks = max_blocks;
    a.num_blocks = num_blocks;
    a.num_seqs = num_seqs;
    a.window = window;
    a.hq = hq;
    a.hkv = hkv;
    a.group = hq / hkv;
    a.rows_per_block = 16 / a.group;
    a.score_scale = sm_scale * 1.4426950408889634f;
    a.out = static_cast<bf16_t *>(out);
    const int tr = PF_WAVES * PF_BLOCKS * a.rows_per_block;
    a.tiles = (n + tr - 1) / tr;
    const long long units = (long long)hkv * a.tiles;
    NC_REQUIRE(units <= (1ll << 30), "nc_prefill_attn_fp8: too many rows");
    a.units_per_xcd = (int)((units + 7) / 8);
    hipLaunchKernelGGL(k_prefill, dim3(8 * a.units_per_xcd), dim3(PF_THREADS), 0, (hipStream_t)stream, a, pos, seq,
                       block_table);
    NC_LAUNCH_CHECK();
    return 0;
}
