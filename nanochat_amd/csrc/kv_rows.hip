/*
 * Position rows of the fp8 cache: the bytes of any positions [at, at + n) of one sequence, every kv head, in one or
 * more layers' pools, moved between the page tiles and a flat row layout, position-granular (any at, any n).
 *
 * Row layout, uint8 [layers][n][hkv][264]: per (layer, position, kv head) one 264-byte row
 *   [0, 128)    K codes, dims 0..127
 *   [128, 256)  V codes, dims 0..127 (the tile's quad transposition undone)
 *   [256, 260)  K scale fp32
 *   [260, 264)  V scale fp32
 * so a position is exactly its algorithmic bytes and a run of positions is contiguous per layer. The decoder
 * handle's prompt store keeps prompts in this layout in pinned host memory, at any position (the reference stores
 * bf16 rows [L][n][C] per position, model/kernels/decode.cu:1053-1075).
 *
 * One wave per row: lanes 0-31 move a dword of K codes each (one 128-B line per row), lanes 32-63 four V dims each
 * (four bytes of the tile, 4 bytes apart), lanes 0 and 1 the two scales. Byte-movement kernels: HBM / launch bound.
 */
#include "layout.h"

#define ROW_BYTES 264
#define ROWS_PER_BLOCK 4

struct RowArgs {
    uint8_t *cache;       /* pool of layer 0; layer l's at + l * pool_bytes */
    long long pool_bytes;
    const int32_t *block_table;
    int max_blocks, num_blocks;
    int seq, at, n, hkv;
    long long rows;       /* layers * n * hkv */
    uint8_t *flat;        /* [layers][n][hkv][264] */
};

/* The tile and token of row r (layer, position at + i, kv head h), or null when its block is missing. */
__device__ __forceinline__ uint8_t *row_tile(const RowArgs &a, long long r, int *t) {
    const int h = (int)(r % a.hkv);
    const long long li = r / a.hkv;
    const int i = (int)(li % a.n), l = (int)(li / a.n);
    const int pos = a.at + i;
    *t = pos % NC_PAGE;
    const int blk = lookup_block(a.block_table, a.max_blocks, a.num_blocks, a.seq, pos / NC_PAGE);
    return blk < 0 ? nullptr : a.cache + (size_t)l * a.pool_bytes + tile_offset(blk, h, a.hkv);
}

/* Tile -> rows; a missing block gives a zero row. */
__global__ void __launch_bounds__(ROWS_PER_BLOCK * NC_WAVE) k_rows_export(RowArgs a) {
    const long long r = (long long)blockIdx.x * ROWS_PER_BLOCK + threadIdx.x / NC_WAVE;
    if (r >= a.rows) return;
    const int lane = threadIdx.x % NC_WAVE;
    int t;
    const uint8_t *tile = row_tile(a, r, &t);
    uint8_t *dst = a.flat + r * ROW_BYTES;
    uint32_t word = 0;
    if (tile) {
        if (lane < 32) {
            word = *reinterpret_cast<const uint32_t *>(tile + k_byte(t, 4 * lane));
        } else {
            const int d = 4 * (lane - 32);
#pragma unroll
            for (int e = 0; e < 4; e++) word |= (uint32_t)tile[v_byte(t, d + e)] << (8 * e);
        }
    }
    reinterpret_cast<uint32_t *>(dst)[lane] = word;
    if (lane < 2) {
        const float s = tile ? reinterpret_cast<const float *>(tile + (lane ? NC_TILE_VS : NC_TILE_KS))[t] : 0.0f;
        reinterpret_cast<float *>(dst + 2 * NC_HEAD_DIM)[lane] = s;
    }
}

/* Rows -> tile; a missing block is not written. Only the row's own bytes of the tile change. */
__global__ void __launch_bounds__(ROWS_PER_BLOCK * NC_WAVE) k_rows_import(RowArgs a) {
    const long long r = (long long)blockIdx.x * ROWS_PER_BLOCK + threadIdx.x / NC_WAVE;
    if (r >= a.rows) return;
    const int lane = threadIdx.x % NC_WAVE;
    int t;
    uint8_t *tile = row_tile(a, r, &t);
    if (!tile) return;
    const uint8_t *src = a.flat + r * ROW_BYTES;
    const uint32_t word = reinterpret_cast<const uint32_t *>(src)[lane];
    if (lane < 32) {
        *reinterpret_cast<uint32_t *>(tile + k_byte(t, 4 * lane)) = word;
    } else {
        const int d = 4 * (lane - 32);
#pragma unroll
        for (int e = 0; e < 4; e++) tile[v_byte(t, d + e)] = (uint8_t)(word >> (8 * e));
    }
    if (lane < 2)
        reinterpret_cast<float *>(tile + (lane ? NC_TILE_VS : NC_TILE_KS))[t] =
            reinterpret_cast<const float *>(src + 2 * NC_HEAD_DIM)[lane];
}

static int row_args(RowArgs &a, const void *cache, long long pool_bytes, int layers, const int32_t *block_table,
                    int max_blocks, int num_blocks, int num_seqs, int seq, int at, int n, int hkv, const void *flat) {
    NC_REQUIRE(layers > 0 && hkv > 0 && n >= 0, "layers %d, hkv %d, n %d", layers, hkv, n);
    NC_REQUIRE(max_blocks > 0 && num_blocks > 0 && num_seqs > 0, "max_blocks %d, num_blocks %d, num_seqs %d must be "
               "positive", max_blocks, num_blocks, num_seqs);
    NC_REQUIRE(block_table || (long long)num_seqs * max_blocks <= num_blocks,
               "contiguous cache: %d sequences x %d blocks exceed the %d blocks", num_seqs, max_blocks, num_blocks);
    NC_REQUIRE(seq >= 0 && seq < num_seqs, "sequence %d outside [0, %d)", seq, num_seqs);
    NC_REQUIRE(at >= 0 && (long long)at + n <= (long long)max_blocks * NC_PAGE,
               "positions [%d, %lld) outside the sequence's %d positions", at, (long long)at + n, max_blocks * NC_PAGE);
    const long long pool_min = (long long)num_blocks * hkv * NC_TILE_BYTES;
    NC_REQUIRE(layers == 1 || (pool_bytes >= pool_min && pool_bytes % 16 == 0),
               "pool_bytes %lld: at least %lld and a multiple of 16 for %d layers", pool_bytes, pool_min, layers);
    NC_REQUIRE(cache && (n == 0 || flat), "null argument");
    NC_REQUIRE((uintptr_t)cache % 16 == 0 && (uintptr_t)flat % 8 == 0,
               "cache must be 16-byte and rows 8-byte aligned");
    a.cache = (uint8_t *)const_cast<void *>(cache);
    a.pool_bytes = pool_bytes;
    a.block_table = block_table;
    a.max_blocks = max_blocks;
    a.num_blocks = num_blocks;
    a.seq = seq;
    a.at = at;
    a.n = n;
    a.hkv = hkv;
    a.rows = (long long)layers * n * hkv;
    a.flat = (uint8_t *)const_cast<void *>(flat);
    return 0;
}

static void launch_rows(void (*kernel)(RowArgs), const RowArgs &a, void *stream) {
    if (a.rows == 0) return;
    const long long blocks = (a.rows + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK;
    hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(ROWS_PER_BLOCK * NC_WAVE), 0, (hipStream_t)stream, a);
    NC_LAUNCH_CHECK();
}

extern "C" int nc_kv_export_fp8(const uint8_t *cache, long long pool_bytes, int layers, const int32_t *block_table,
                                int max_blocks, int num_blocks, int num_seqs, int seq, int at, int n, int hkv,
                                uint8_t *rows, void *stream) {
    RowArgs a = {};
    const int rc = row_args(a, cache, pool_bytes, layers, block_table, max_blocks, num_blocks, num_seqs, seq, at, n,
                            hkv, rows);
    if (rc) return rc;
    launch_rows(k_rows_export, a, stream);
    return 0;
}

extern "C" int nc_kv_import_fp8(const uint8_t *rows, int layers, uint8_t *cache, long long pool_bytes,
                                const int32_t *block_table, int max_blocks, int num_blocks, int num_seqs, int seq,
                                int at, int n, int hkv, void *stream) {
    RowArgs a = {};
    const int rc = row_args(a, cache, pool_bytes, layers, block_table, max_blocks, num_blocks, num_seqs, seq, at, n,
                            hkv, rows);
    if (rc) return rc;
    launch_rows(k_rows_import, a, stream);
    return 0;
}
