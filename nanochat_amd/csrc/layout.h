/*
 * The fp8 KV cache's layout in HBM, shared by the append, gather, decode and prefill kernels.
 *
 * A cache is one pool of blocks; a block holds PAGE (16) consecutive positions of one sequence for every kv head.
 * Block `blk`, kv head `h` is one contiguous 4224-byte tile at byte (blk * Hkv + h) * 4224 of the pool:
 *   [0, 2048)     K codes, row-major: key t (0..15), dim d at t * 128 + d. A wave reads them as 64 lanes x 32
 *                 contiguous bytes (lane's key = lane % 16, dims 32 (lane / 16) ..), the A operand of 16x16x32
 *                 MFMAs.
 *   [2048, 4096)  V codes, quad-transposed: key t, dim d at 2048 + (t / 4) * 512 + d * 4 + t % 4, so the 4 keys
 *                 of a quad sit in one dword per dim: the A operand (Vᵀ, keys contiguous per lane) of the PV MFMA.
 *   [4096, 4160)  K scales, fp32 [16]
 *   [4160, 4224)  V scales, fp32 [16]
 * 4224 B = 16 positions x 264 B: the tile holds exactly the algorithmic bytes of a (page, kv head), and a page
 * of decode attention is one contiguous read (separate K, V and scale pools measured ~20 % slower on MI355X:
 * four scattered DRAM/TLB streams per page instead of one).
 *
 * A sequence's page i is block_table[seq * max_blocks + i]; with no table (contiguous mode) it is block
 * seq * max_blocks + i, i.e. each sequence owns max_blocks consecutive blocks.
 */
#pragma once

#include "common.h"

#define NC_PAGE 16
#define NC_TILE_BYTES 4224
#define NC_TILE_V 2048
#define NC_TILE_KS 4096
#define NC_TILE_VS 4160

/* Byte offset of the (blk, h) tile in the pool. */
__device__ __forceinline__ size_t tile_offset(int blk, int h, int hkv) {
    return ((size_t)blk * hkv + h) * NC_TILE_BYTES;
}

/* Byte of key t, dim d within a tile's V region. */
__device__ __forceinline__ int v_byte(int t, int d) { return NC_TILE_V + (t >> 2) * 512 + d * 4 + (t & 3); }

/* The block of page `page` of sequence `seq`, or -1 when the page or the block is out of range. */
__device__ __forceinline__ int lookup_block(const int32_t *block_table, int max_blocks, int num_blocks, int seq,
                                            int page) {
    if (page < 0 || page >= max_blocks) return -1;
    const int blk = block_table ? block_table[(size_t)seq * max_blocks + page] : seq * max_blocks + page;
    return (blk >= 0 && blk < num_blocks) ? blk : -1;
}

/* Write this lane's 16 codes of a quantised row into the tile's K region (row-major) or V region
 * (quad-transposed). */
__device__ __forceinline__ void write_codes(uint8_t *tile, int t, int g, uint64_t c1, uint64_t c2, bool is_v) {
    if (!is_v) {
        *reinterpret_cast<uint64_t *>(tile + t * NC_HEAD_DIM + 8 * g) = c1;
        *reinterpret_cast<uint64_t *>(tile + t * NC_HEAD_DIM + NC_HALF + 8 * g) = c2;
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            tile[v_byte(t, 8 * g + e)] = (uint8_t)(c1 >> (8 * e));
            tile[v_byte(t, NC_HALF + 8 * g + e)] = (uint8_t)(c2 >> (8 * e));
        }
    }
}
