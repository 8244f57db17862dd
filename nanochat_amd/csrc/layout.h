/*
 * The fp8 KV cache's layout in HBM, shared by the append, gather, decode and prefill kernels.
 *
 * A cache is one pool of blocks; a block holds PAGE (16) consecutive positions of one sequence for every kv head.
 * Block `blk`, kv head `h` is one contiguous 4224-byte tile at byte (blk * Hkv + h) * 4224 of the pool, laid out
 * by the 16-byte fragments a wave's lanes hold for the MFMAs, lane f's fragment of part P at P * 1024 + 16 f:
 *   [0, 2048)     K codes, parts 0 and 1: key t (0..15), dim d at ((d / 16) % 2) * 1024 + (t + 16 (d / 32)) * 16
 *                 + d % 16. Lane f = t + 16 c holds key t's dims 32 c .. 32 c + 31 (16 in each part), the A operand
 *                 of 16x16x32 MFMAs.
 *   [2048, 4096)  V codes, parts 2 and 3, quad-transposed: key t, dim d at 2048 + ((d / 4) % 2) * 1024
 *                 + (d / 8 + 16 (t / 4)) * 16 + (d % 4) * 4 + t % 4. Lane f = n + 16 q holds dims 8 n .. 8 n + 7
 *                 of keys 4 q .. 4 q + 3, one dword per dim (the 4 keys of a quad), the A operand (Vᵀ) of the PV
 *                 MFMAs.
 *   [4096, 4160)  K scales, fp32 [16]
 *   [4160, 4224)  V scales, fp32 [16]
 * 4224 B = 16 positions x 264 B: the tile holds exactly the algorithmic bytes of a (page, kv head), and a page
 * of decode attention is one contiguous read (separate K, V and scale pools measured ~20 % slower on MI355X:
 * four scattered DRAM/TLB streams per page instead of one). With the fragments in lane order each of a wave's four
 * code loads reads 1 KB contiguous (eight whole 128-byte lines), which is what lets nontemporal loads stream at
 * full rate: loads that each cover half of every line they touch (a row-major K) streamed slower with the hint
 * than without it.
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

#define NC_TILE_PART 1024 /* one 16-byte fragment per lane of a wave */

/* Byte of key t, dim d within a tile's K region. */
__device__ __forceinline__ int k_byte(int t, int d) {
    return ((d >> 4) & 1) * NC_TILE_PART + (t + 16 * (d >> 5)) * 16 + (d & 15);
}

/* Byte of key t, dim d within a tile's V region. */
__device__ __forceinline__ int v_byte(int t, int d) {
    return NC_TILE_V + ((d >> 2) & 1) * NC_TILE_PART + ((d >> 3) + 16 * (t >> 2)) * 16 + (d & 3) * 4 + (t & 3);
}

/* The block of page `page` of sequence `seq`, or -1 when the page or the block is out of range. */
__device__ __forceinline__ int lookup_block(const int32_t *block_table, int max_blocks, int num_blocks, int seq,
                                            int page) {
    if (page < 0 || page >= max_blocks) return -1;
    const int blk = block_table ? block_table[(size_t)seq * max_blocks + page] : seq * max_blocks + page;
    return (blk >= 0 && blk < num_blocks) ? blk : -1;
}

/* Write this lane's 16 codes of a quantised row (dims 8 g .. 8 g + 7 and 64 + 8 g ..) into the tile's K region
 * (8 dims of a key are 8 contiguous bytes) or V region (quad-transposed). */
__device__ __forceinline__ void write_codes(uint8_t *tile, int t, int g, uint64_t c1, uint64_t c2, bool is_v) {
    if (!is_v) {
        *reinterpret_cast<uint64_t *>(tile + k_byte(t, 8 * g)) = c1;
        *reinterpret_cast<uint64_t *>(tile + k_byte(t, NC_HALF + 8 * g)) = c2;
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            tile[v_byte(t, 8 * g + e)] = (uint8_t)(c1 >> (8 * e));
            tile[v_byte(t, NC_HALF + 8 * g + e)] = (uint8_t)(c2 >> (8 * e));
        }
    }
}
