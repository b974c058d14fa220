/*
 * tile.h -- the MFMA tile layout of a quantised matrix (prefill GEMM operand).
 *
 * The expert table keeps every matrix twice: in the GGML layout the reference
 * reads (row-major super-blocks, kernels.c:416-431) and, repacked once at
 * upload, in this tile layout.  A tile is 32 rows x one super-block (256
 * columns).  Its 64 lane records are what the 64 lanes of a wave need for one
 * MFMA K step over those rows: lane l = n + 32 h holds row n's half h
 * (columns 128h .. 128h+127):
 *   Q6_K record, 28 dwords: ql dwords 16h .. 16h+15, qh dwords 8h .. 8h+7,
 *                           scale dwords 2h, 2h+1, d (low 16 bits), 0
 *   Q4_K record, 20 dwords: header dwords 0..3 (d, dmin, 12 scale bytes),
 *                           qs dwords 16h .. 16h+15
 * Dword q of lane l is at tile + 1024 (q / 4) + 16 l + 4 (q % 4): one 16-byte
 * load per lane per slice (7 slices for Q6_K, 5 for Q4_K), each a contiguous
 * kilobyte per wave.  Tile (g, kb) of a matrix with nkb super-blocks per row is
 * at (g * nkb + kb) * TL_BYTES(q6).
 */
#ifndef ROASTER_TILE_H
#define ROASTER_TILE_H

#include <stddef.h>

#define TL_ROWS 32
#define TL_Q6_BYTES (64 * 28 * 4)         /* 7168 */
#define TL_Q4_BYTES (64 * 20 * 4)         /* 5120 */
#define TL_BYTES(q6) ((q6) ? TL_Q6_BYTES : TL_Q4_BYTES)
#define TL_SLICES(q6) ((q6) ? 7 : 5)      /* 16-byte slices per record = loads per lane */

static inline size_t tl_mat_bytes(int q6, size_t rows, size_t cols)
{
    return rows / TL_ROWS * (cols / 256) * (size_t)TL_BYTES(q6);
}

#endif
