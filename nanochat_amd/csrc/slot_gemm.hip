/*
 * The decode step's weight GEMMs (the reference's slot GEMM, model/kernels/decode.cu:107-123,169-184,292-338):
 * out[b][r] = epilogue(Σ_k W[r][k] x[b][k]) for the M rows x of a decode batch (M is the batch, 1..a few hundred)
 * against a weight matrix W [N][K] in nn.Linear layout, bf16 operands, fp32 accumulation.
 *
 * At decode batch sizes the GEMM is a stream of W through the chip: W is read once from HBM and every byte meets all
 * M rows of x, which stay L2-resident. The work unit is an output tile of NT weight rows x MT batch rows over the full
 * K, so the epilogue sees complete sums and the result is deterministic (no split-K atomics):
 *
 *   - K is walked in 64-column chunks through an LDS ring of up to 8 slots; each chunk's NT + MT rows of 128 bytes
 *     arrive by global_load_lds_dwordx4 (8 whole rows per instruction), shared evenly by the 4 waves, at a swizzled
 *     position so the fragment reads (ds_read_b128) are bank-conflict free;
 *   - the 4 waves split the tile as WN x 4 / WN over W rows and batch rows and multiply with
 *     v_mfma_f32_16x16x32_bf16 (A = 16 W rows, B = 16 x rows: Yᵀ tiles); per step a wave waits for its own DMAs,
 *     meets the others at one barrier, refills the slots everyone has finished, reads the next chunk's fragments
 *     while this chunk's MFMAs run, and settles them. A step covers two chunks where the ring is 6 or more slots
 *     deep (half the barriers and waits; the decode-step GEMMs 4-16 % faster with the same bits). The loop moves
 *     about 50 GB/s into each CU whatever issues the loads (4 or 8 extra DMA-only waves were no faster, nor W loaded
 *     straight into registers), so the time is the bytes reaching the busiest CU, (NT + MT) K 2 per tile;
 *   - the RMS norm of the input rows is fused: the same x fragments feed one more MFMA per 16 rows, x·xᵀ, whose
 *     diagonal is Σ x² of each row, so r = 1 / sqrt(Σ x² / K + FLT_EPSILON) (model/modeling.py:47-49, decode.cu:448-456)
 *     scales the sums in the epilogue instead of a separate normalised copy of x (the reference's RELU2 epilogue,
 *     p = s r, decode.cu:171-175);
 *   - units are ordered so the MT-row slices of one weight tile run on one XCD (workgroup b on XCD b % 8 takes a
 *     contiguous range), so W is fetched from HBM once and re-read from that XCD's L2.
 *
 * Epilogues (decode.cu:169-184): STORE bf16(s); NORM_STORE bf16(s r); RESID bf16(s + res) (one rounding, res may be
 * out: an in-place residual update); RELU2_NORM bf16(relu(p) p) with p = s r; NORM_F32 fp32 s r (the lm_head's
 * logits for nc_argmax_f32).
 */
#include "common.h"
#include <algorithm>

#define SG_THREADS 256
#define SG_WAVES 4
#define SG_CHUNK 64                 /* K columns per ring slot: 128 bytes of every row */
#define SG_LDS_BUDGET (128 * 1024) /* ring bytes per workgroup */
#define SG_MAX_DEPTH 8             /* ring slots: deeper rings measured no faster */
#define SG_GROUP 2                 /* chunks per barrier where the ring is deep enough (2 measured faster than 1, 4) */

enum { SG_STORE = 0, SG_NORM_STORE = 1, SG_RESID = 2, SG_RELU2_NORM = 3, SG_NORM_F32 = 4 };

typedef __attribute__((address_space(3))) unsigned char sg_lds_u8;

struct SlotGemmArgs {
    const bf16_t *w;   /* [n][k] */
    const bf16_t *x;   /* [m][k] */
    void *out;         /* [m][n] bf16 (fp32 for NORM_F32) */
    const bf16_t *res; /* [m][n] RESID's addend, may equal out */
    int n, k, m;
    int n_tiles, m_slices, units_per_xcd;
    const unsigned char *pf; /* read by the pf_wgs workgroups past the tiles' (null: none) */
    long long pf_bytes;
    int pf_wgs;
};

/* The 4 waves as WN (over W rows) x 4/WN (over batch rows): the split that reads the fewest fragments per wave
 * (per chunk a wave reads its NT/WN W rows and MT/(4/WN) x rows from LDS); ties to the larger WN. */
__host__ __device__ constexpr int sg_reads(int nt, int mt, int wn) {
    return (nt / 16) % wn || (mt / 16) % (4 / wn) ? 1 << 20 : nt / 16 / wn + mt / 16 / (4 / wn);
}
__host__ __device__ constexpr int sg_waves_n(int nt, int mt) {
    return sg_reads(nt, mt, 4) <= sg_reads(nt, mt, 2) && sg_reads(nt, mt, 4) <= sg_reads(nt, mt, 1)
               ? 4
               : (sg_reads(nt, mt, 2) <= sg_reads(nt, mt, 1) ? 2 : 1);
}

/* Ring geometry of an NT x MT tile: a slot holds the chunk's NT W rows then MT x rows, 128 bytes each. */
__host__ __device__ constexpr int sg_slot_bytes(int nt, int mt) { return (nt + mt) * 128; }
__host__ __device__ constexpr int sg_depth(int nt, int mt) {
    return SG_LDS_BUDGET / sg_slot_bytes(nt, mt) > SG_MAX_DEPTH ? SG_MAX_DEPTH : SG_LDS_BUDGET / sg_slot_bytes(nt, mt);
}
/* Chunks per barrier: G (even, or 1) with D >= 2 G + 2, so the ring keeps at least 2 chunks in flight past a step. */
__host__ __device__ constexpr int sg_group(int d) { return d >= 2 * SG_GROUP + 2 ? SG_GROUP : (d >= 6 ? 2 : 1); }

template <int N> __device__ __forceinline__ void sg_wait_vmcnt() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

__device__ __forceinline__ uint32_t sg_lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const sg_lds_u8 *)(const unsigned char *)p;
}

/* 16 bytes of LDS; completion is waited for by sg_ds_wait (the compiler does not see the read in flight). */
__device__ __forceinline__ bf16x8 sg_ds_read(uint32_t addr) {
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
    return __builtin_bit_cast(bf16x8, v);
}
__device__ __forceinline__ void sg_ds_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
/* Orders every use of v after the preceding sg_ds_wait. */
__device__ __forceinline__ void sg_after_wait(bf16x8 &v) { asm volatile("" : "+v"(v)); }

/* This wave's DMA instructions of a chunk: instruction wv + SG_WAVES d lands at dst + 1024 (wv + SG_WAVES d). (A
 * function, not a lambda: clang drops the host stub of a kernel template whose lambda calls this builtin.) */
template <int DPW>
__device__ __forceinline__ void sg_dma(const unsigned char *const *src, size_t off, unsigned char *dst, int wv) {
#pragma unroll
    for (int d = 0; d < DPW; d++)
        __builtin_amdgcn_global_load_lds(src[d] + off, dst + 1024 * (wv + SG_WAVES * d), 16, 0, 0);
}

/* A prefetch workgroup's part of [pf, pf + pf_bytes): whole 64 KiB blocks b = wg, wg + pf_wgs, ... read with 16
 * loads in flight per lane and discarded, so that the bytes sit in the memory-side cache for the next kernel (the
 * next GEMM's weights). Plain loads: the nontemporal hint would keep them out of that cache. */
__device__ __forceinline__ void sg_prefetch(const SlotGemmArgs &a) {
    constexpr int U = 16;
    constexpr long long BLOCK = (long long)SG_THREADS * 16 * U;
    const long long blocks = a.pf_bytes / BLOCK;
    u32x4 acc = u32x4{0u, 0u, 0u, 0u};
    for (long long b = (long long)blockIdx.x - 8 * a.units_per_xcd; b < blocks; b += a.pf_wgs) {
        const unsigned char *p = a.pf + b * BLOCK + (long long)threadIdx.x * 16;
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = *reinterpret_cast<const u32x4 *>(p + (long long)u * SG_THREADS * 16);
#pragma unroll
        for (int u = 0; u < U; u++) acc |= v[u];
    }
    asm volatile("" ::"v"(acc[0]), "v"(acc[1]), "v"(acc[2]), "v"(acc[3])); /* the loads stay */
}

/*
 * LDS layout of a slot: row r (W rows 0..NT-1, then x rows) at 128 r; its 16-byte piece p (k columns 8p..8p+7 of
 * the chunk) at position p ^ (r & 7), so the fragment reads below are bank-conflict free. DMA instruction i of a
 * chunk moves rows 8i..8i+7: lane l lands at slot + 1024 i + 16 l (row 8i + l/8, position l % 8) and therefore
 * fetches piece (l % 8) ^ (row & 7) of its row -- every instruction reads 8 whole 128-byte row segments.
 */
template <int NT, int MT, int EPI>
__global__ void __launch_bounds__(SG_THREADS) k_slot_gemm(SlotGemmArgs a) {
    constexpr int ROWS = NT + MT, DMAS = ROWS / 8, DPW = DMAS / SG_WAVES; /* DMA instructions per chunk, per wave */
    constexpr int SLOT = sg_slot_bytes(NT, MT), D = sg_depth(NT, MT), G = sg_group(D);
    constexpr int WN = sg_waves_n(NT, MT), WM = SG_WAVES / WN; /* waves over W rows x batch rows */
    constexpr int TNW = NT / 16 / WN, TMW = MT / 16 / WM;     /* 16x16 tiles per wave */
    constexpr int TSQ = (TMW + WN - 1) / WN; /* batch tiles whose Σ x² this wave computes (shared with its row) */
    constexpr bool NORM = EPI == SG_NORM_STORE || EPI == SG_RELU2_NORM || EPI == SG_NORM_F32;
    static_assert(DMAS % SG_WAVES == 0 && NT % (16 * WN) == 0 && MT % (16 * WM) == 0, "tile shape");
    static_assert(D >= 3, "ring depth");
    __shared__ __attribute__((aligned(1024))) unsigned char ring[D * SLOT];

    if ((int)blockIdx.x >= 8 * a.units_per_xcd) { /* a prefetch workgroup (nc_slot_gemm_bf16_prefetch) */
        sg_prefetch(a);
        return;
    }
    const int unit = (blockIdx.x & 7) * a.units_per_xcd + (blockIdx.x >> 3);
    if (unit >= a.n_tiles * a.m_slices) return;
    const int nt = unit / a.m_slices, ms = unit % a.m_slices;
    const int row0 = nt * NT, m0 = ms * MT;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
    const int j = lane >> 4, n = lane & 15;
    const int wn = wv % WN, wm = wv / WN;
    const int chunks = a.k / SG_CHUNK;
    const size_t ld = (size_t)a.k;

    /* this wave's DMA sources: instruction i = wv + SG_WAVES d of every chunk; x rows past m repeat row m - 1 */
    const unsigned char *src[DPW];
#pragma unroll
    for (int d = 0; d < DPW; d++) {
        const int r = 8 * (wv + SG_WAVES * d) + (lane >> 3);
        const int piece = (lane & 7) ^ (r & 7);
        const bf16_t *row = r < NT ? a.w + (size_t)(row0 + r) * ld : a.x + (size_t)min(m0 + r - NT, a.m - 1) * ld;
        src[d] = reinterpret_cast<const unsigned char *>(row) + 16 * piece;
    }
    /* chunk c (clamped to the last) into ring slot `slot` */
    auto dma = [&](int c, int slot) {
        sg_dma<DPW>(src, (size_t)min(c, chunks - 1) * (SG_CHUNK * 2), ring + slot * SLOT, wv);
    };

    /* this wave's fragment addresses within a slot: W row tile t, x row tile u, k half h: piece 4h + j of row n */
    uint32_t fw[TNW][2], fx[TMW][2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
        for (int t = 0; t < TNW; t++) {
            const int r = 16 * (wn * TNW + t) + n;
            fw[t][h] = sg_lds_addr(ring) + 128 * r + 16 * ((4 * h + j) ^ (r & 7));
        }
#pragma unroll
        for (int u = 0; u < TMW; u++) {
            const int r = NT + 16 * (wm * TMW + u) + n;
            fx[u][h] = sg_lds_addr(ring) + 128 * r + 16 * ((4 * h + j) ^ (r & 7));
        }
    }

    f32x4 acc[TNW][TMW];
    f32x4 sq[TSQ];
#pragma unroll
    for (int t = 0; t < TNW; t++)
#pragma unroll
        for (int u = 0; u < TMW; u++) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < TSQ; q++) sq[q] = f32x4{0.f, 0.f, 0.f, 0.f};

    /* fragment reads of a chunk's slot (completed by the next sg_ds_wait) */
    auto read = [&](int c, bf16x8 (&wf)[TNW][2], bf16x8 (&xf)[TMW][2]) {
        const uint32_t so = (uint32_t)((c % D) * SLOT);
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll
            for (int t = 0; t < TNW; t++) wf[t][h] = sg_ds_read(fw[t][h] + so);
#pragma unroll
            for (int u = 0; u < TMW; u++) xf[u][h] = sg_ds_read(fx[u][h] + so);
        }
    };
    auto settle = [&](bf16x8 (&wf)[TNW][2], bf16x8 (&xf)[TMW][2]) {
        sg_ds_wait();
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll
            for (int t = 0; t < TNW; t++) sg_after_wait(wf[t][h]);
#pragma unroll
            for (int u = 0; u < TMW; u++) sg_after_wait(xf[u][h]);
        }
    };
    auto multiply = [&](const bf16x8 (&wf)[TNW][2], const bf16x8 (&xf)[TMW][2]) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll
            for (int t = 0; t < TNW; t++)
#pragma unroll
                for (int u = 0; u < TMW; u++)
                    acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[t][h], xf[u][h], acc[t][u], 0, 0, 0);
            if constexpr (NORM) {
                /* this wave's batch tiles u = q WN + wn, picked by selects (no dynamic register indexing, no branch);
                 * past TMW the product is computed and ignored */
#pragma unroll
                for (int q = 0; q < TSQ; q++) {
                    bf16x8 v = xf[q * WN < TMW ? q * WN : TMW - 1][h];
#pragma unroll
                    for (int w = 1; w < WN; w++)
                        if (q * WN + w < TMW) v = wn == w ? xf[q * WN + w][h] : v;
                    sq[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v, v, sq[q], 0, 0, 0);
                }
            }
        }
    };
    /* one iteration, straight-line code (fragments in flight never cross a branch, where the compiler could copy
     * their registers before the data lands): once every wave has settled chunk c's fragments (the barrier), slot
     * c % D takes chunk c + D; chunk c + 1's fragments are read while chunk c's MFMAs run, then settle. Past the
     * end the chunk indices clamp to the last chunk, which the refill then rewrites with the same bytes. */
    auto step = [&](int c, const bf16x8 (&wf)[TNW][2], const bf16x8 (&xf)[TMW][2], bf16x8 (&wn_)[TNW][2],
                    bf16x8 (&xn_)[TMW][2]) {
        sg_wait_vmcnt<DPW * (D - 2)>(); /* this wave's DMAs of chunk c + 1 have landed */
        __builtin_amdgcn_s_barrier();   /* everyone's have, and everyone has settled chunk c's reads */
        __builtin_amdgcn_sched_barrier(0);
        read(min(c + 1, chunks - 1), wn_, xn_);
        dma(c + D, c % D);
        multiply(wf, xf);
        settle(wn_, xn_);
        __builtin_amdgcn_sched_barrier(0);
    };

    bf16x8 wa[TNW][2], xa[TMW][2], wb[TNW][2], xb[TMW][2];
    if (G > 1 && chunks % 2 == 0) {
        /* G chunks per barrier (fewer barriers and waits, the same MFMAs in the same order): step c (a multiple of
         * G) multiplies chunks c..c+G-1 and reads c+1..c+G, once everyone's DMAs of those have landed and everyone
         * has settled its reads of chunks c-G+1..c, whose slots then take chunks c-G+1+D..c+D. The slots of chunks
         * D-G+1..D-1 start empty. The last step may hold fewer than G chunks (pairs past the end are skipped; their
         * reads and waits stay inside the branch). */
#pragma unroll
        for (int c = 0; c <= D - G; c++) dma(c, c);
        sg_wait_vmcnt<DPW * (D - G)>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        read(0, wa, xa);
        settle(wa, xa);
        for (int c = 0; c < chunks; c += G) {
            sg_wait_vmcnt<DPW * (D - 2 * G)>(); /* this wave's DMAs of chunks c + 1..c + G have landed */
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < G; i += 2) {
                if (i == 0 || c + i < chunks) {
                    read(c + i + 1, wb, xb);
                    if (i == 0) { /* the refills after the first reads: a burst of DMAs holds up what follows it */
#pragma unroll
                        for (int k = 1; k <= G; k++) dma(c - G + k + D, (c - G + k + D) % D);
                    }
                    multiply(wa, xa);
                    settle(wb, xb);
                    __builtin_amdgcn_sched_barrier(0);
                    read(min(c + i + 2, chunks - 1), wa, xa);
                    multiply(wb, xb);
                    settle(wa, xa);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < D; c++) dma(c, c); /* chunks 0..D-1 in flight (the slot of chunk D is that of chunk 0) */
        sg_wait_vmcnt<DPW * (D - 1)>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        read(0, wa, xa);
        settle(wa, xa);
        for (int c = 0; c < chunks; c += 2) {
            step(c, wa, xa, wb, xb);
            if (c + 1 < chunks) step(c + 1, wb, xb, wa, xa);
        }
    }
    sg_wait_vmcnt<0>(); /* the clamped refills past the last chunk land before the ring is reused or released */

    /* the rows' Σ x², each computed by one wave of its batch slice: x·xᵀ's diagonal, row n's in lane (n / 4, n),
     * element n % 4; exchanged through LDS (the ring is free: every wave is past its last read) */
    float rstd[TMW];
    if constexpr (NORM) {
        float *ss = reinterpret_cast<float *>(ring);
        __syncthreads();
#pragma unroll
        for (int q = 0; q < TSQ; q++) {
            const int u = q * WN + wn;
            if (u < TMW && j == (n >> 2)) ss[16 * (wm * TMW + u) + n] = sq[q][n & 3];
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < TMW; u++)
            rstd[u] = 1.0f / sqrtf(ss[16 * (wm * TMW + u) + n] / (float)a.k + 1.1920928955078125e-07f);
    } else {
#pragma unroll
        for (int u = 0; u < TMW; u++) rstd[u] = 1.f;
    }

    const int N = a.n;
#pragma unroll
    for (int u = 0; u < TMW; u++) {
        const int b = m0 + 16 * (wm * TMW + u) + n;
        const float r = rstd[u];
        if (b >= a.m) continue;
#pragma unroll
        for (int t = 0; t < TNW; t++) {
            const f32x4 s = acc[t][u];
            const int col = row0 + 16 * (wn * TNW + t) + 4 * j;
            const size_t at = (size_t)b * N + col;
            if constexpr (EPI == SG_NORM_F32) {
                *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(a.out) + at) = s * r;
            } else {
                float v[4];
                if constexpr (EPI == SG_RESID) {
                    const u32x2 rr = *reinterpret_cast<const u32x2 *>(a.res + at);
                    v[0] = s[0] + bf16_to_f32(rr[0] & 0xffffu);
                    v[1] = s[1] + bf16_to_f32(rr[0] >> 16);
                    v[2] = s[2] + bf16_to_f32(rr[1] & 0xffffu);
                    v[3] = s[3] + bf16_to_f32(rr[1] >> 16);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float p = s[i] * r;
                        v[i] = EPI == SG_RELU2_NORM ? fmaxf(p, 0.f) * p : p;
                    }
                }
                const u32x2 o = {f32x2_to_bf16x2(v[0], v[1]), f32x2_to_bf16x2(v[2], v[3])};
                *reinterpret_cast<u32x2 *>(reinterpret_cast<bf16_t *>(a.out) + at) = o;
            }
        }
    }
}

/* ------------------------------------------------------------------------------------------------ large M */

/*
 * The same GEMM for many rows (prefill chunks: M in the thousands), where it is MFMA-bound instead of a stream of W:
 * a workgroup of 8 waves owns a 256 x-row x 256 W-row output tile over the full K (complete sums, deterministic), and
 * each wave a 128 x-row x 64 W-row part of it. Every output element is computed by the same instruction
 * (v_mfma_f32_16x16x32_bf16, A = 16 W rows, B = 16 x rows), in the same order of 32-column K steps, as
 * k_slot_gemm computes it, and the norm's Σ x² the same way (x·xᵀ's diagonal over the same steps): the result of a
 * row does not depend on M, on the tile, or on which of the two kernels ran.
 *
 * K is walked in 64-column chunks through a 2-slot LDS ring (64 KB a slot: the tile's 256 W rows and 256 x rows of
 * 128 bytes, the swizzled layout and DMA of k_slot_gemm), chunk c in slot c & 1. Per chunk a wave reads the second
 * half's fragments while the first half's MFMAs run, then meets the others at the chunk's one barrier (everyone's
 * DMAs of chunk c + 1 have landed, everyone is done reading chunk c), reads the next chunk's first half and runs the
 * second half's MFMAs with the DMAs of chunk c + 2 (into chunk c's slot) issued one between each group of 4: every
 * LDS read is in flight behind MFMAs, and the DMAs no longer stall the MFMAs behind the memory queue. Rows past m or
 * n read the last row (clamped) and are not stored. The tile leaves through LDS, half at a time, as whole rows.
 *
 * Tiles are ordered XCD-aware (workgroup b on XCD b % 8 takes a contiguous range) and, within it, in groups of
 * RG_GROUP x-row tiles that sweep the W tiles, so neighbouring workgroups share x and W rows in L2.
 */
#define RG_THREADS 512
#define RG_WAVES 8
#define RG_BM 256 /* x rows per tile */
#define RG_BN 256 /* W rows per tile */
#define RG_GROUP 4
#define RG_MIN_M 512 /* nc_slot_gemm_bf16 takes this kernel from this many rows on (automatic tile) */
#define RG_SROW (RG_BN + 4) /* floats per staged output row: 65 x 16 bytes, so 16 lanes' 16-byte writes of 16 rows
                             * land on 16 different bank groups */

struct RowsGemmArgs {
    const bf16_t *w, *x;
    void *out;
    const bf16_t *res;
    int n, k, m;
    int n_tiles, m_tiles, units_per_xcd;
};

/* 16 bytes of LDS at addr + OFF (an immediate: tile offsets need no registers of their own). */
template <int OFF> __device__ __forceinline__ bf16x8 rg_ds_read(uint32_t addr) {
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return __builtin_bit_cast(bf16x8, v);
}

/* One 16-byte-per-lane DMA into LDS (a function, not a builtin call inside the kernel's lambdas: clang has dropped
 * the host stub of kernel templates whose lambdas call this builtin). */
__device__ __forceinline__ void rg_dma1(const unsigned char *src, unsigned char *dst) {
    __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}

/* One of four fragments by a wave-uniform index, as selects on values (an indexed array here ends up in scratch). */
__device__ __forceinline__ bf16x8 rg_pick4(int w, bf16x8 f0, bf16x8 f1, bf16x8 f2, bf16x8 f3) {
    return w == 0 ? f0 : (w == 1 ? f1 : (w == 2 ? f2 : f3));
}

template <int EPI>
__global__ void __launch_bounds__(RG_THREADS) k_rows_gemm(RowsGemmArgs a) {
    constexpr int ROWS = RG_BN + RG_BM, SLOT = ROWS * 128, DPW = ROWS / 8 / RG_WAVES; /* 8 DMAs per wave a chunk */
    constexpr int WM = 2, WN = 4;                                  /* waves over x rows x W rows */
    constexpr int TM = RG_BM / 16 / WM, TN = RG_BN / 16 / WN;     /* 8 x tiles, 4 W tiles per wave */
    constexpr int TSQ = TM / WN;                                   /* x tiles whose Σ x² this wave computes */
    constexpr bool NORM = EPI == SG_NORM_STORE || EPI == SG_RELU2_NORM || EPI == SG_NORM_F32;
    /* the epilogue stages half the tile (128 x rows of fp32, rows RG_SROW floats apart) where the ring was */
    constexpr int STAGE = RG_BM / 2 * RG_SROW * 4, LDS = STAGE > 2 * SLOT ? STAGE : 2 * SLOT;
    __shared__ __attribute__((aligned(1024))) unsigned char ring[LDS];

    const int unit = (blockIdx.x & 7) * a.units_per_xcd + (blockIdx.x >> 3);
    if (unit >= a.n_tiles * a.m_tiles) return;
    const int per_group = RG_GROUP * a.n_tiles, group = unit / per_group, first_m = group * RG_GROUP;
    const int gsz = min(a.m_tiles - first_m, RG_GROUP), in_group = unit % per_group;
    const int mt = first_m + in_group % gsz, ntl = in_group / gsz;
    const int row0 = ntl * RG_BN, m0 = mt * RG_BM;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
    const int j = lane >> 4, n = lane & 15;
    const int wn = wv % WN, wm = wv / WN;
    const int chunks = a.k / SG_CHUNK;
    const size_t ld = (size_t)a.k;

    /* DMA instruction i = wv + RG_WAVES d of a chunk moves slot rows 8i..8i+7 (W rows first, then x rows) */
    /* as 32-bit byte offsets from W or x (each under 2 GiB): instructions d < DPW / 2 move W rows, the rest x rows */
    static_assert(RG_BN == RG_BM && DPW % 2 == 0, "W rows fill the first half of a chunk's DMA instructions");
    uint32_t soff[DPW];
#pragma unroll
    for (int d = 0; d < DPW; d++) {
        const int r = 8 * (wv + RG_WAVES * d) + (lane >> 3);
        const int piece = (lane & 7) ^ (r & 7);
        const size_t row = r < RG_BN ? (size_t)min(row0 + r, a.n - 1) : (size_t)min(m0 + r - RG_BN, a.m - 1);
        soff[d] = (uint32_t)(row * ld * 2 + 16 * piece);
    }
    const unsigned char *wb = reinterpret_cast<const unsigned char *>(a.w);
    const unsigned char *xb = reinterpret_cast<const unsigned char *>(a.x);
    auto dma1 = [&](int c, int slot, int d) { /* DMA instruction d of chunk c (clamped to the last) */
        const unsigned char *base = (d < DPW / 2 ? wb : xb) + (size_t)min(c, chunks - 1) * (SG_CHUNK * 2);
        rg_dma1(base + soff[d], ring + slot * SLOT + 1024 * (wv + RG_WAVES * d));
    };
    auto dma = [&](int c, int slot) {
#pragma unroll
        for (int d = 0; d < DPW; d++) dma1(c, slot, d);
    };

    /* fragment rows: W tile t row 16 (wn TN + t) + n, x tile u row RG_BN + 16 (wm TM + u) + n; a row's swizzle
     * (piece ^ (row & 7)) is n & 7 for every tile, so one base address per half and operand, tiles 2048 B apart */
    uint32_t bw[2], bx[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t swz = 16 * ((4 * h + j) ^ (n & 7));
        bw[h] = sg_lds_addr(ring) + 128 * (16 * wn * TN + n) + swz;
        bx[h] = sg_lds_addr(ring) + 128 * (RG_BN + 16 * wm * TM + n) + swz;
    }

    f32x4 acc[TN][TM];
    f32x4 sq[TSQ];
#pragma unroll
    for (int t = 0; t < TN; t++)
#pragma unroll
        for (int u = 0; u < TM; u++) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < TSQ; q++) sq[q] = f32x4{0.f, 0.f, 0.f, 0.f};

    /* half h of chunk c's fragments (completed by the next sg_ds_wait) */
    auto read = [&](int c, int h, bf16x8 (&wf)[TN], bf16x8 (&xf)[TM]) {
        const uint32_t so = (uint32_t)((c & 1) * SLOT), aw = bw[h] + so, ax = bx[h] + so;
        static_assert(TN == 4 && TM == 8, "the reads below are unrolled for 4 W and 8 x tiles");
        wf[0] = rg_ds_read<0>(aw);
        wf[1] = rg_ds_read<2048>(aw);
        wf[2] = rg_ds_read<4096>(aw);
        wf[3] = rg_ds_read<6144>(aw);
        xf[0] = rg_ds_read<0>(ax);
        xf[1] = rg_ds_read<2048>(ax);
        xf[2] = rg_ds_read<4096>(ax);
        xf[3] = rg_ds_read<6144>(ax);
        xf[4] = rg_ds_read<8192>(ax);
        xf[5] = rg_ds_read<10240>(ax);
        xf[6] = rg_ds_read<12288>(ax);
        xf[7] = rg_ds_read<14336>(ax);
    };
    auto settle = [&](bf16x8 (&wf)[TN], bf16x8 (&xf)[TM]) {
        sg_ds_wait();
#pragma unroll
        for (int t = 0; t < TN; t++) sg_after_wait(wf[t]);
#pragma unroll
        for (int u = 0; u < TM; u++) sg_after_wait(xf[u]);
    };
    auto multiply = [&](const bf16x8 (&wf)[TN], const bf16x8 (&xf)[TM]) {
#pragma unroll
        for (int t = 0; t < TN; t++)
#pragma unroll
            for (int u = 0; u < TM; u++)
                acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[t], xf[u], acc[t][u], 0, 0, 0);
        if constexpr (NORM) {
#pragma unroll
            for (int q = 0; q < TSQ; q++) { /* x tile q WN + wn, picked by selects (wn is wave-uniform) */
                bf16x8 v = xf[q * WN];
#pragma unroll
                for (int w = 1; w < WN; w++) v = wn == w ? xf[q * WN + w] : v;
                sq[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v, v, sq[q], 0, 0, 0);
            }
        }
    };

    /* the MFMAs of one half in 8 groups of 4 (W tile g / 2, x tiles 4 (g % 2) .. + 3), the same order as multiply */
    auto multiply_group = [&](int g, const bf16x8 (&wf)[TN], const bf16x8 (&xf)[TM]) {
#pragma unroll
        for (int uu = 0; uu < 4; uu++) {
            f32x4 &d = acc[g / 2][4 * (g % 2) + uu];
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[g / 2], xf[4 * (g % 2) + uu], d, 0, 0, 0);
        }
    };
    auto multiply_norm = [&](const bf16x8 (&xf)[TM]) {
        if constexpr (NORM) {
            static_assert(WN == 4, "x tile q WN + wn of 4");
#pragma unroll
            for (int q = 0; q < TSQ; q++) {
                const bf16x8 v = rg_pick4(wn, xf[q * WN], xf[q * WN + 1], xf[q * WN + 2], xf[q * WN + 3]);
                sq[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v, v, sq[q], 0, 0, 0);
            }
        }
    };
    static_assert(DPW == 8, "one DMA instruction per group of 4 MFMAs");

    /* Chunk c lives in slot c & 1. Per chunk: the second half's reads go out, the first half's MFMAs run, the reads
     * settle; then one barrier (everyone's DMAs of chunk c + 1 have landed, everyone is done reading chunk c), the
     * DMAs of chunk c + 2 go into chunk c's slot, the next chunk's first-half reads go out and the second half's
     * MFMAs run. Every LDS read is in flight behind MFMAs; the barrier is the only exposed step. */
    bf16x8 w0[TN], x0[TM], w1[TN], x1[TM];
    dma(0, 0);
    sg_wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    dma(1, 1);
    read(0, 0, w0, x0);
    settle(w0, x0);
    for (int c = 0; c < chunks; c++) {
        read(c, 1, w1, x1);
        __builtin_amdgcn_sched_barrier(0);
        multiply(w0, x0);
        __builtin_amdgcn_sched_barrier(0);
        settle(w1, x1);
        sg_wait_vmcnt<0>();           /* this wave's DMAs of chunk c + 1 have landed */
        __builtin_amdgcn_s_barrier(); /* everyone's have, and everyone is past its reads of chunk c */
        __builtin_amdgcn_sched_barrier(0);
        multiply_norm(x1); /* no read is in flight here */
        read(min(c + 1, chunks - 1), 0, w0, x0);
        {
            /* the DMAs of chunk c + 2 (past the end: the last chunk again) into chunk c's slot, one between each
             * group of 4 MFMAs: issued all at once they hold up the MFMAs behind the memory queue */
#pragma unroll
            for (int g = 0; g < 8; g++) {
                __builtin_amdgcn_sched_barrier(0);
                dma1(c + 2, c & 1, g);
                multiply_group(g, w1, x1);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        settle(w0, x0);
    }
    sg_wait_vmcnt<0>();

    float rstd[TM];
    if constexpr (NORM) {
        float *ss = reinterpret_cast<float *>(ring);
        __syncthreads(); /* every wave is past its last read of the ring */
#pragma unroll
        for (int q = 0; q < TSQ; q++)
            if (j == (n >> 2)) ss[16 * (wm * TM + q * WN + wn) + n] = sq[q][n & 3];
        __syncthreads();
#pragma unroll
        for (int u = 0; u < TM; u++)
            rstd[u] = 1.0f / sqrtf(ss[16 * (wm * TM + u) + n] / (float)a.k + 1.1920928955078125e-07f);
    } else {
#pragma unroll
        for (int u = 0; u < TM; u++) rstd[u] = 1.f;
    }

    /* The tile leaves in two passes of 128 x rows (the waves of one x-row half each): those waves stage their values
     * before rounding -- s, s r or relu(s r) s r, and for RESID s alone -- in LDS, then all 512 threads write
     * whole output rows, 16 bytes each, coalesced (RESID adds res there, one rounding as before). */
    const int N = a.n;
    float *stage = reinterpret_cast<float *>(ring);
#pragma unroll
    for (int pass = 0; pass < WM; pass++) {
        __syncthreads(); /* the ring (or the previous pass's stage) is free */
        if (wm == pass) {
#pragma unroll
            for (int u = 0; u < TM; u++) {
                const float r = rstd[u];
#pragma unroll
                for (int t = 0; t < TN; t++) {
                    f32x4 v = acc[t][u];
                    if constexpr (EPI != SG_RESID && EPI != SG_STORE) {
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const float pv = v[i] * r;
                            v[i] = EPI == SG_RELU2_NORM ? fmaxf(pv, 0.f) * pv : pv;
                        }
                    }
                    *reinterpret_cast<f32x4 *>(stage + (16 * u + n) * RG_SROW + 16 * (wn * TN + t) + 4 * j) = v;
                }
            }
        }
        __syncthreads();
        const int b0 = m0 + pass * (RG_BM / WM);
        if constexpr (EPI == SG_NORM_F32) {
            /* 4 fp32 per 16 bytes: 64 per row */
            for (int i = threadIdx.x; i < RG_BM / WM * 64; i += RG_THREADS) {
                const int rr = i >> 6, c4 = (i & 63) * 4, b = b0 + rr, col = row0 + c4;
                if (b < a.m && col < N)
                    *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(a.out) + (size_t)b * N + col) =
                        *reinterpret_cast<const f32x4 *>(stage + rr * RG_SROW + c4);
            }
        } else {
            /* 8 bf16 per 16 bytes: 32 per row */
            for (int i = threadIdx.x; i < RG_BM / WM * 32; i += RG_THREADS) {
                const int rr = i >> 5, c8 = (i & 31) * 8, b = b0 + rr, col = row0 + c8;
                if (b >= a.m || col >= N) continue;
                const f32x4 lo = *reinterpret_cast<const f32x4 *>(stage + rr * RG_SROW + c8);
                const f32x4 hi = *reinterpret_cast<const f32x4 *>(stage + rr * RG_SROW + c8 + 4);
                float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                const size_t at = (size_t)b * N + col;
                if constexpr (EPI == SG_RESID) {
                    const u32x4 rr4 = *reinterpret_cast<const u32x4 *>(a.res + at);
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        v[2 * e] = v[2 * e] + bf16_to_f32(rr4[e] & 0xffffu);
                        v[2 * e + 1] = v[2 * e + 1] + bf16_to_f32(rr4[e] >> 16);
                    }
                }
                u32x4 o;
#pragma unroll
                for (int e = 0; e < 4; e++) o[e] = f32x2_to_bf16x2(v[2 * e], v[2 * e + 1]);
                *reinterpret_cast<u32x4 *>(reinterpret_cast<bf16_t *>(a.out) + at) = o;
            }
        }
    }
}

/* ------------------------------------------------------------------------------------------------ host side */

typedef void (*SgKernel)(SlotGemmArgs);

template <int NT, int MT> static SgKernel sg_pick_epi(int epi) {
    switch (epi) {
    case SG_STORE: return k_slot_gemm<NT, MT, SG_STORE>;
    case SG_NORM_STORE: return k_slot_gemm<NT, MT, SG_NORM_STORE>;
    case SG_RESID: return k_slot_gemm<NT, MT, SG_RESID>;
    case SG_RELU2_NORM: return k_slot_gemm<NT, MT, SG_RELU2_NORM>;
    default: return k_slot_gemm<NT, MT, SG_NORM_F32>;
    }
}

/* The tiles built: NT W rows x MT batch rows per workgroup (NT + MT a multiple of 32, so the 4 waves share a
 * chunk's DMAs evenly). */
static const int SG_TILES[][2] = {{32, 32}, {64, 32}, {32, 64}, {64, 64}, {32, 128}, {64, 128}, {128, 64}, {128, 128}};

static SgKernel sg_pick(int nt, int mt, int epi) {
    if (nt == 32 && mt == 32) return sg_pick_epi<32, 32>(epi);
    if (nt == 64 && mt == 32) return sg_pick_epi<64, 32>(epi);
    if (nt == 32 && mt == 64) return sg_pick_epi<32, 64>(epi);
    if (nt == 64 && mt == 64) return sg_pick_epi<64, 64>(epi);
    if (nt == 32 && mt == 128) return sg_pick_epi<32, 128>(epi);
    if (nt == 64 && mt == 128) return sg_pick_epi<64, 128>(epi);
    if (nt == 128 && mt == 64) return sg_pick_epi<128, 64>(epi);
    if (nt == 128 && mt == 128) return sg_pick_epi<128, 128>(epi);
    return nullptr;
}

/* The automatic tile: a workgroup moves (NT + MT) rows of K into its CU, and a CU fills at a roughly fixed rate, so
 * the time is about (units per CU) x (NT + MT); among the tiles dividing n, the least of ceil(units / 256) x
 * (NT + MT), ties to the larger tile (less re-reading of W and x through L2). */
static void sg_auto_tile(int n, int m, int &nt, int &mt) {
    long long best = -1;
    nt = mt = 0;
    for (const auto &t : SG_TILES) {
        if (n % t[0] || (t[1] > 32 && t[1] / 2 >= m)) continue;
        const long long units = (long long)(n / t[0]) * ((m + t[1] - 1) / t[1]);
        const long long cost = ((units + 255) / 256) * (t[0] + t[1]);
        if (best < 0 || cost < best || (cost == best && t[0] * t[1] > nt * mt)) {
            best = cost;
            nt = t[0];
            mt = t[1];
        }
    }
}

/* Compute units of the current device (cached per device). */
static int sg_device_cus() {
    static int cached[64];
    int dev = 0;
    NC_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) dev = 0;
    if (!cached[dev]) {
        int cus = 0;
        NC_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        cached[dev] = cus > 0 ? cus : 1;
    }
    return cached[dev];
}

static int slot_gemm(const void *w, int n, int k, const void *x, int m, int epi, void *out, const void *res, int nt,
                     int mt, const void *prefetch, long long prefetch_bytes, void *stream) {
    NC_REQUIRE(n > 0 && k > 0 && m >= 0, "nc_slot_gemm_bf16: n %d, k %d, m %d", n, k, m);
    NC_REQUIRE(n % 32 == 0 && k % SG_CHUNK == 0, "nc_slot_gemm_bf16: n = %d must be a multiple of 32 and k = %d of %d",
               n, k, SG_CHUNK);
    NC_REQUIRE(epi >= SG_STORE && epi <= SG_NORM_F32, "nc_slot_gemm_bf16: unknown epilogue %d", epi);
    NC_REQUIRE((long long)n * k * 2 < (1LL << 31) && (long long)m * k * 2 < (1LL << 31),
               "nc_slot_gemm_bf16: W (%d x %d) and x (%d x %d) must each stay under 2 GiB", n, k, m, k);
    if (m == 0) return 0;
    NC_REQUIRE(w && x && out, "nc_slot_gemm_bf16: null pointer");
    NC_REQUIRE(epi != SG_RESID || res, "nc_slot_gemm_bf16: RESID needs res");
    NC_REQUIRE(((uintptr_t)w | (uintptr_t)x | (uintptr_t)out | (uintptr_t)res) % 16 == 0,
               "nc_slot_gemm_bf16: 16-byte alignment");
    if (nt == 0 && mt == 0 && m >= RG_MIN_M) { /* many rows: the MFMA-bound tile (the same results) */
        RowsGemmArgs r;
        r.w = (const bf16_t *)w;
        r.x = (const bf16_t *)x;
        r.out = out;
        r.res = (const bf16_t *)res;
        r.n = n;
        r.k = k;
        r.m = m;
        r.n_tiles = (n + RG_BN - 1) / RG_BN;
        r.m_tiles = (m + RG_BM - 1) / RG_BM;
        const long long units = (long long)r.n_tiles * r.m_tiles;
        r.units_per_xcd = (int)((units + 7) / 8);
        void (*kern)(RowsGemmArgs) = epi == SG_STORE        ? k_rows_gemm<SG_STORE>
                                     : epi == SG_NORM_STORE ? k_rows_gemm<SG_NORM_STORE>
                                     : epi == SG_RESID      ? k_rows_gemm<SG_RESID>
                                     : epi == SG_RELU2_NORM ? k_rows_gemm<SG_RELU2_NORM>
                                                            : k_rows_gemm<SG_NORM_F32>;
        hipLaunchKernelGGL(kern, dim3(8 * r.units_per_xcd), dim3(RG_THREADS), 0, (hipStream_t)stream, r);
        NC_LAUNCH_CHECK();
        return 0;
    }
    if (nt == 0 && mt == 0) sg_auto_tile(n, m, nt, mt);
    const SgKernel kern = sg_pick(nt, mt, epi);
    NC_REQUIRE(kern && n % nt == 0, "nc_slot_gemm_bf16: tile %d x %d is not available for n = %d", nt, mt, n);
    SlotGemmArgs a;
    a.w = (const bf16_t *)w;
    a.x = (const bf16_t *)x;
    a.out = out;
    a.res = (const bf16_t *)res;
    a.n = n;
    a.k = k;
    a.m = m;
    a.n_tiles = n / nt;
    a.m_slices = (m + mt - 1) / mt;
    const long long units = (long long)a.n_tiles * a.m_slices;
    a.units_per_xcd = (int)((units + 7) / 8);
    /* prefetch workgroups on the compute units the tiles leave idle, behind the tiles in dispatch order */
    a.pf = (const unsigned char *)prefetch;
    a.pf_bytes = prefetch ? prefetch_bytes : 0;
    a.pf_wgs = a.pf_bytes >= 65536 ? std::max(0, sg_device_cus() - 8 * a.units_per_xcd) : 0;
    hipLaunchKernelGGL(kern, dim3(8 * a.units_per_xcd + a.pf_wgs), dim3(SG_THREADS), 0, (hipStream_t)stream, a);
    NC_LAUNCH_CHECK();
    return 0;
}

extern "C" int nc_slot_gemm_bf16(const void *w, int n, int k, const void *x, int m, int epi, void *out,
                                 const void *res, int nt, int mt, void *stream) {
    return slot_gemm(w, n, k, x, m, epi, out, res, nt, mt, nullptr, 0, stream);
}

extern "C" int nc_slot_gemm_bf16_prefetch(const void *w, int n, int k, const void *x, int m, int epi, void *out,
                                          const void *res, int nt, int mt, const void *prefetch,
                                          long long prefetch_bytes, void *stream) {
    NC_REQUIRE(prefetch_bytes >= 0 && (prefetch || prefetch_bytes == 0) && (uintptr_t)prefetch % 16 == 0,
               "nc_slot_gemm_bf16_prefetch: prefetch %p of %lld bytes", prefetch, prefetch_bytes);
    return slot_gemm(w, n, k, x, m, epi, out, res, nt, mt, prefetch, prefetch_bytes, stream);
}
