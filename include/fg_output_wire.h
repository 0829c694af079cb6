/* Wire messages of the sampling path: the output owner (rank 4) receives one
 * 40-byte output config per token (the sampler controls and the draw) and
 * answers with a 16-byte output result (the token and its logit).  Big-endian
 * fields, the same names, layouts, checks and errors as the reference:
 *   fg_output_config / fg_output_result   include/fg_protocol.h:461-481
 *   fg_output_config_encode / _decode     src/protocol.c:1160-1166
 *   fg_output_result_encode / _decode     src/protocol.c:1275-1279
 * and two batch helpers with no reference counterpart, for an owner that
 * samples many rows per launch: fg_output_configs_batch builds the rows'
 * controls and uniforms for fg_sampler_hip_set_configs /
 * fg_sampler_hip_sample, fg_output_results_encode_batch answers each row. */
#ifndef FG_OUTPUT_WIRE_H
#define FG_OUTPUT_WIRE_H

#include <stdint.h>

#include "fg.h"
#include "fg_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

#define FG_OUTPUT_CONFIG_BYTES 40u
#define FG_OUTPUT_RESULT_BYTES 16u
#define FG_OUTPUT_CONFIG_FLAG_SPLIT 1u    /* greedy rows: vocabulary-split head */
#define FG_OUTPUT_CONFIG_FLAG_SPLIT_4 2u  /* with FLAG_SPLIT: four ways, else two */
#define FG_OUTPUT_WIRE_RANKS 8u           /* FG_RANK_COUNT, reference include/fg.h:13 */
#define FG_OUTPUT_WIRE_OWNER 4u           /* the output owner's rank */
#define FG_OUTPUT_WIRE_SESSIONS 2u        /* FG_DECODE_BATCH_MAX_SLOTS */
#define FG_OUTPUT_WIRE_VOCAB 248320u      /* FG_Q38_VOCAB_SIZE: bound on result tokens */

typedef struct fg_output_result {
    uint8_t source_rank;
    uint8_t destination_rank;
    uint32_t token_index;
    uint32_t token;
    float logit;
} fg_output_result;

typedef struct fg_output_config {
    uint8_t source_rank;
    uint8_t destination_rank;
    uint8_t flags;
    uint8_t session_slot; /* owner session whose sampling history this token belongs to */
    uint32_t token_index;
    fg_sampler_config sampler;
    float uniform;
} fg_output_config;

/* Checks the route (source < 8, destination 4, session < 2), the sampler
 * (fg_sampler_config_validate unless every control is 0) and the draw
 * (finite, in [0, 1)) and writes the 40 bytes.  FG_ERR_ARGUMENT for a NULL
 * buffer, FG_ERR_FORMAT for a config that fails a check. */
fg_status fg_output_config_encode(uint8_t output[FG_OUTPUT_CONFIG_BYTES],
                                  const fg_output_config *config, fg_error *err);
/* FG_ERR_FORMAT for a size other than 40, unknown flag bits, FLAG_SPLIT_4
 * without FLAG_SPLIT, or a decoded config that fails the encoder's checks. */
fg_status fg_output_config_decode(fg_output_config *config, const uint8_t *payload,
                                  uint32_t bytes, fg_error *err);
/* Checks source 4, destination < 8, token < FG_OUTPUT_WIRE_VOCAB and a finite
 * logit, and writes the 16 bytes (bytes 2-3 zero). */
fg_status fg_output_result_encode(uint8_t output[FG_OUTPUT_RESULT_BYTES],
                                  const fg_output_result *result, fg_error *err);
/* FG_ERR_FORMAT for a size other than 16, nonzero bytes 2-3, or a result
 * that fails the encoder's checks. */
fg_status fg_output_result_decode(fg_output_result *result, const uint8_t *payload,
                                  uint32_t bytes, fg_error *err);

/* Row r of a batch takes configs[r].sampler and configs[r].uniform.  A
 * config whose controls are all 0 (the wire's "no controls", which the
 * decoder lets through unvalidated) becomes fg_sampler_config_greedy.
 * FG_ERR_ARGUMENT for NULL pointers or rows == 0. */
fg_status fg_output_configs_batch(const fg_output_config *configs, uint32_t rows,
                                  fg_sampler_config *samplers, float *uniforms, fg_error *err);
/* Encodes row r's answer to configs[r] (source 4, destination the config's
 * source, its token index, tokens[r], logits[r]) at output + 16 r.  A row
 * whose row_status (NULL: all 0) is not 0 is skipped: its 16 bytes are
 * zeroed and *answered (when not NULL) counts only the encoded rows.
 * FG_ERR_FORMAT if an encoded row fails fg_output_result_encode's checks. */
fg_status fg_output_results_encode_batch(uint8_t *output, const fg_output_config *configs,
                                         const uint32_t *tokens, const float *logits,
                                         const int32_t *row_status, uint32_t rows,
                                         uint32_t *answered, fg_error *err);

#ifdef __cplusplus
}
#endif

#endif
