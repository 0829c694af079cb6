/* Q8_0 blocks, f16 scales and the cooked tile layout (reference
 * src/quant.c:10-113). */
#include "fg_quant.h"

#include <math.h>
#include <string.h>

static uint32_t f32_bits(float v)
{
    uint32_t b;
    memcpy(&b, &v, sizeof b);
    return b;
}

static float bits_f32(uint32_t b)
{
    float v;
    memcpy(&v, &b, sizeof v);
    return v;
}

float fg_f16_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exponent = (h >> 10) & 0x1fu;
    const uint32_t fraction = h & 0x3ffu;
    if (exponent == 0x1fu)
        return bits_f32(sign | 0x7f800000u | (fraction << 13));
    if (exponent)
        return bits_f32(sign | ((exponent + 112u) << 23) | (fraction << 13));
    /* zero or subnormal: fraction * 2^-24, exact in binary32 */
    const float magnitude = (float)fraction * 0x1p-24f;
    return sign ? -magnitude : magnitude;
}

uint16_t fg_f32_to_f16(float value)
{
    const uint32_t b = f32_bits(value);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    const uint32_t exponent = (b >> 23) & 0xffu;
    const uint32_t fraction = b & 0x7fffffu;
    if (exponent == 0xffu)
        return (uint16_t)(sign | (fraction ? 0x7e00u : 0x7c00u));
    const int32_t e = (int32_t)exponent - 112; /* binary16 biased exponent */
    if (e >= 31)
        return (uint16_t)(sign | 0x7c00u);
    /* Normal results round the 23-bit fraction to 10 bits; results below
     * the normal range shift the full significand further. */
    const uint32_t significand = e > 0 ? fraction : (fraction | (exponent ? 0x800000u : 0u));
    const uint32_t shift = e > 0 ? 13u : (uint32_t)(14 - e);
    if (shift > 24u)
        return sign;
    uint32_t half = significand >> shift;
    const uint32_t rest = significand & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1u);
    if (rest > halfway || (rest == halfway && (half & 1u)))
        half++;
    if (e > 0)
        half += (uint32_t)e << 10; /* the carry of a rounded-up fraction bumps the exponent */
    return (uint16_t)(sign | half);
}

void fg_quantize_q8_0(const float *input, void *output, uint64_t values)
{
    uint8_t *out = output;
    for (uint64_t b = 0; b < values / FG_QK8_0; b++) {
        const float *x = input + b * FG_QK8_0;
        float amax = 0.0f;
        for (uint32_t i = 0; i < FG_QK8_0; i++)
            amax = fmaxf(amax, fabsf(x[i]));
        const float d = amax / 127.0f;
        const float inv = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t h = fg_f32_to_f16(d);
        uint8_t *block = out + b * FG_Q8_0_BLOCK_BYTES;
        block[0] = (uint8_t)h;
        block[1] = (uint8_t)(h >> 8);
        for (uint32_t i = 0; i < FG_QK8_0; i++)
            block[2 + i] = (uint8_t)(int8_t)roundf(x[i] * inv);
    }
}

void fg_dequantize_q8_0(const void *input, float *output, uint64_t values)
{
    const uint8_t *in = input;
    for (uint64_t b = 0; b < values / FG_QK8_0; b++) {
        const uint8_t *block = in + b * FG_Q8_0_BLOCK_BYTES;
        const float d = fg_f16_to_f32((uint16_t)(block[0] | (block[1] << 8)));
        for (uint32_t i = 0; i < FG_QK8_0; i++)
            output[b * FG_QK8_0 + i] = d * (float)(int8_t)block[2 + i];
    }
}

static uint64_t align64(uint64_t v)
{
    return (v + FG_Q8_0_COOK_ALIGNMENT - 1u) & ~(uint64_t)(FG_Q8_0_COOK_ALIGNMENT - 1u);
}

static uint64_t quant_offset(uint64_t blocks)
{
    return align64(FG_Q8_0_COOK_ROWS * blocks * 2u);
}

uint64_t fg_q8_0_cooked_tile_bytes(uint32_t input_width)
{
    if (!input_width || input_width % FG_QK8_0)
        return 0;
    const uint64_t blocks = input_width / FG_QK8_0;
    return align64(quant_offset(blocks) + FG_Q8_0_COOK_ROWS * blocks * FG_QK8_0);
}

uint64_t fg_q8_0_cooked_matrix_bytes(uint32_t input_width, uint32_t rows)
{
    const uint64_t tile = fg_q8_0_cooked_tile_bytes(input_width);
    const uint64_t tiles = ((uint64_t)rows + FG_Q8_0_COOK_ROWS - 1u) / FG_Q8_0_COOK_ROWS;
    if (!tile || !rows || tiles > UINT64_MAX / tile)
        return 0;
    return tiles * tile;
}

/* Byte addresses of row `row`, block `block` in the cooked layout. */
static void cooked_at(uint64_t tile_bytes, uint64_t blocks, uint32_t row, uint64_t block,
                      uint64_t *scale_at, uint64_t *quants_at)
{
    const uint64_t tile = (uint64_t)(row / FG_Q8_0_COOK_ROWS) * tile_bytes;
    const uint64_t r = row % FG_Q8_0_COOK_ROWS;
    *scale_at = tile + (block * FG_Q8_0_COOK_ROWS + r) * 2u;
    *quants_at = tile + quant_offset(blocks) + (r * blocks + block) * FG_QK8_0;
}

bool fg_cook_q8_0_rows(const void *input, void *output, uint64_t output_bytes,
                       uint32_t input_width, uint32_t rows)
{
    const uint64_t tile_bytes = fg_q8_0_cooked_tile_bytes(input_width);
    const uint64_t required = fg_q8_0_cooked_matrix_bytes(input_width, rows);
    if (!input || !output || !required || output_bytes < required)
        return false;
    const uint64_t blocks = input_width / FG_QK8_0;
    const uint8_t *src = input;
    uint8_t *dst = output;
    memset(dst, 0, (size_t)required);
    for (uint32_t row = 0; row < rows; row++) {
        for (uint64_t block = 0; block < blocks; block++) {
            const uint8_t *b = src + ((uint64_t)row * blocks + block) * FG_Q8_0_BLOCK_BYTES;
            uint64_t s, q;
            cooked_at(tile_bytes, blocks, row, block, &s, &q);
            memcpy(dst + s, b, 2u);
            memcpy(dst + q, b + 2, FG_QK8_0);
        }
    }
    return true;
}

bool fg_uncook_q8_0_rows(const void *input, void *output, uint64_t output_bytes,
                         uint32_t input_width, uint32_t rows)
{
    const uint64_t tile_bytes = fg_q8_0_cooked_tile_bytes(input_width);
    if (!input || !output || !tile_bytes || !fg_q8_0_cooked_matrix_bytes(input_width, rows))
        return false;
    const uint64_t blocks = input_width / FG_QK8_0;
    if (output_bytes < blocks * FG_Q8_0_BLOCK_BYTES * rows)
        return false;
    const uint8_t *src = input;
    uint8_t *dst = output;
    for (uint32_t row = 0; row < rows; row++) {
        for (uint64_t block = 0; block < blocks; block++) {
            uint8_t *b = dst + ((uint64_t)row * blocks + block) * FG_Q8_0_BLOCK_BYTES;
            uint64_t s, q;
            cooked_at(tile_bytes, blocks, row, block, &s, &q);
            memcpy(b, src + s, 2u);
            memcpy(b + 2, src + q, FG_QK8_0);
        }
    }
    return true;
}
