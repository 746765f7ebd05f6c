// The device layout of a Q4_K weight matrix (host upload, synthetic
// generation and every Q4_K kernel agree on it through these helpers).
//
// Rows are taken 16 at a time ("a tile", padded with zero rows to a whole
// tile).  For tile t and block b (256 weights of each row) one contiguous unit
// of 16 × 144 = 2304 bytes holds:
//   bytes   0 ..  255   the 16 rows' 16-byte block headers (f16 d, f16 dmin,
//                       12 bytes of packed 6-bit scales and mins), row r at 16r;
//   bytes 256 .. 2303   their quants: the 32 bytes of quant group g (0..3) of
//                       row r at 256 + (16g + r)·32, byte i holding weight
//                       64g + i in its low nibble and weight 64g + 32 + i in its
//                       high nibble, as ggml's block_q4_K does, except that the
//                       high nibble is stored XOR 8.
// Lane 16g + r of a wave reads group g of row r: a wave's two 16-byte loads per
// lane cover the unit's 2048 quant bytes once, contiguously.  Masked with
// 0xf0, a stored byte is 16·(q − 8) as a signed 8-bit integer, which the int8
// matrix cores take as it is; masked with 0x0f it is the low weight's q.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace q4kt {

constexpr size_t kTile = 16;
constexpr size_t kUnit = kTile * 144;

__host__ __device__ inline size_t tiles(size_t rows) { return (rows + kTile - 1) / kTile; }
__host__ __device__ inline size_t bytes(size_t rows, size_t cols) { return tiles(rows) * (cols / 256) * kUnit; }
__host__ __device__ inline size_t unit(size_t tile, size_t b, size_t nb) { return (tile * nb + b) * kUnit; }
__host__ __device__ inline size_t meta_off(size_t r) { return r * 16; }
__host__ __device__ inline size_t qs_off(size_t g, size_t r) { return kTile * 16 + (g * kTile + r) * 32; }

// The stored form of a ggml quant byte, and back (the same XOR).
__host__ __device__ inline uint8_t stored(uint8_t byte) { return byte ^ 0x80u; }

// Places one ggml block_q4_K (144 bytes: d, dmin, scales[12], qs[128]) of
// row `row`, block `b` into the tiled matrix.
__host__ __device__ inline void place(uint8_t *dst, size_t nb, size_t row, size_t b, const uint8_t *blk) {
    uint8_t *u = dst + unit(row / kTile, b, nb);
    const size_t r = row % kTile;
    for (int i = 0; i < 16; i++) u[meta_off(r) + i] = blk[i];
    for (int g = 0; g < 4; g++)
        for (int i = 0; i < 32; i++) u[qs_off(g, r) + i] = stored(blk[16 + 32 * g + i]);
}

}  // namespace q4kt
