/*
 * The fp8 KV cache's layout in HBM, shared by the append, gather, decode and prefill kernels.
 *
 * A cache is a pool of blocks; a block holds PAGE (16) consecutive positions of one sequence for every kv head.
 * For block `blk` and kv head `h` the (blk, h) tile is 2 KiB of K codes and 2 KiB of V codes, at byte
 * (blk * Hkv + h) * 2048 of each pool:
 *   K tile: row-major, key t (0..15) dim d at t * 128 + d. A wave reads a tile as 64 lanes x 32 contiguous bytes
 *           (lane's key = lane % 16, dims 32 * (lane / 16) ..), the A operand of a 16x16x32 MFMA per 8 dims.
 *   V tile: quad-transposed, key t dim d at (t / 4) * 512 + d * 4 + t % 4, so the 4 keys of a quad sit in one
 *           dword per dim: the layout the PV MFMA's A operand (Vᵀ, keys contiguous per lane) reads directly.
 * Scales are fp32, one per (block, kv head, key) for K and for V: [num_blocks][Hkv][16].
 *
 * A sequence's page i is block_table[seq * max_blocks + i]; with no table (contiguous mode) it is block
 * seq * max_blocks + i, i.e. each sequence owns max_blocks consecutive blocks.
 */
#pragma once

#include "common.h"

#define NC_PAGE 16
#define NC_TILE_BYTES (NC_PAGE * NC_HEAD_DIM)

/* Byte offset of the (blk, h) tile in a K or V pool. */
__device__ __forceinline__ size_t tile_offset(int blk, int h, int hkv) {
    return ((size_t)blk * hkv + h) * NC_TILE_BYTES;
}

/* Index of the first scale of the (blk, h) tile. */
__device__ __forceinline__ size_t scale_offset(int blk, int h, int hkv) { return ((size_t)blk * hkv + h) * NC_PAGE; }

/* Byte of key t, dim d within a V tile. */
__device__ __forceinline__ int v_byte(int t, int d) { return (t >> 2) * 512 + d * 4 + (t & 3); }

/* The block of page `page` of sequence `seq`, or -1 when the page or the block is out of range. */
__device__ __forceinline__ int lookup_block(const int32_t *block_table, int max_blocks, int num_blocks, int seq,
                                            int page) {
    if (page < 0 || page >= max_blocks) return -1;
    const int blk = block_table ? block_table[(size_t)seq * max_blocks + page] : seq * max_blocks + page;
    return (blk >= 0 && blk < num_blocks) ? blk : -1;
}
