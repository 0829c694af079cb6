/* Q8_0 weights: the block format, the f16 scale conversions and the cooked
 * 16-row tile layout the LM head is stored in (reference include/fg_quant.h,
 * src/quant.c).  Same names, arguments and results as the reference.
 *
 * Q8_0 block (34 bytes): f16 scale d (little-endian), 32 int8 quants; the
 * values are d * q.  Cooked layout, per tile of FG_Q8_0_COOK_ROWS rows:
 *   [0, quant_offset)             scales, [block][tile_row] as f16
 *   [quant_offset, tile_bytes)    quants, [tile_row][block][32] as int8
 * with quant_offset = align64(16 * blocks * 2) and tile_bytes =
 * align64(quant_offset + 16 * blocks * 32); rows past the last real row of
 * the final tile are zero.  The device products over this layout are in
 * fg_sampler_hip.h (fg_hip_dense_q8_0_cooked). */
#ifndef FG_QUANT_H
#define FG_QUANT_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FG_QK8_0 32u
#define FG_Q8_0_BLOCK_BYTES 34u
#define FG_Q8_0_COOK_ALIGNMENT 64u
#define FG_Q8_0_COOK_ROWS 16u

/* IEEE binary16 <-> binary32: exact widening; narrowing rounds to nearest
 * even, overflows to infinity, and maps NaN to the quiet NaN 0x7e00 with the
 * input's sign (src/quant.c:10-24). */
float fg_f16_to_f32(uint16_t value);
uint16_t fg_f32_to_f16(float value);

/* values / 32 blocks: d = max|x| / 127 (as f16), q = round(x / d) with
 * halves away from zero, q = 0 when d = 0 (src/quant.c:26-33). */
void fg_quantize_q8_0(const float *input, void *output, uint64_t values);
/* output[i] = f16(d) * q (src/quant.c:45-47). */
void fg_dequantize_q8_0(const void *input, float *output, uint64_t values);

/* Tile and matrix sizes of the cooked layout; 0 when input_width is 0 or
 * not a multiple of 32 (or rows is 0). */
uint64_t fg_q8_0_cooked_tile_bytes(uint32_t input_width);
uint64_t fg_q8_0_cooked_matrix_bytes(uint32_t input_width, uint32_t rows);
/* Packed rows (row-major Q8_0 blocks) <-> cooked tiles; false on bad sizes
 * or a too-small output (src/quant.c:96, 98-113). */
bool fg_cook_q8_0_rows(const void *input, void *output, uint64_t output_bytes,
                       uint32_t input_width, uint32_t rows);
bool fg_uncook_q8_0_rows(const void *input, void *output, uint64_t output_bytes,
                         uint32_t input_width, uint32_t rows);

#ifdef __cplusplus
}
#endif

#endif
