/* Vocabulary-split greedy output: the LM-head rows are divided over 2 or 4
 * ranks, each reduces its slice of the logits to one (value, id) finalist,
 * and the output owner combines the finalists into the token.
 *
 * Host side (same names, arguments and results as the reference):
 *   fg_output_better / fg_output_combine       include/fg_output.h:38-40
 *   fg_output_split_way_for_rank / _rank / _span include/fg_protocol.h:488-490
 *   fg_output_split_combine_finalists          restates the combine step of
 *                                              src/runtime.c:2440-2466
 * Device side (batched over decode rows): fg_sampler_hip.h,
 * fg_hip_output_slice_* and fg_hip_output_split_combine. */
#ifndef FG_OUTPUT_SPLIT_H
#define FG_OUTPUT_SPLIT_H

#include <stdbool.h>
#include <stdint.h>

#include "fg.h"

#ifdef __cplusplus
extern "C" {
#endif

#define FG_OUTPUT_SPLIT_FIRST_ROWS 140048u  /* rows kept by the owner in the 2-way split */
#define FG_OUTPUT_SPLIT_WAYS_MIN 2u
#define FG_OUTPUT_SPLIT_WAYS_MAX 4u
#define FG_OUTPUT_SPLIT_OWNER_RANK 4u       /* fg_output_owner_rank, include/fg_output.h:15 */
#define FG_OUTPUT_SPLIT_VOCAB 248320u       /* FG_Q38_VOCAB_SIZE */

/* Total order of (value, id) finalists (src/output.c:484-492): a padding id
 * (0xffffffff) loses to any real one; a non-finite value beats a finite one
 * and two non-finite values go to the lower id; otherwise the larger value,
 * then the lower id. */
bool fg_output_better(float left, uint32_t left_id, float right, uint32_t right_id);
/* The better of the two (right when neither is better); NULL outputs skipped. */
void fg_output_combine(float left, uint32_t left_id, float right, uint32_t right_id,
                       float *value, uint32_t *id);

/* Way index of `rank` in a `ways`-way split: 2-way {4, 0}, 4-way {4, 0, 1, 2}.
 * False for a rank that owns no slice or an unsupported `ways`. */
bool fg_output_split_way_for_rank(uint32_t ways, uint32_t rank, uint32_t *way);
/* Inverse of the above; UINT32_MAX for an invalid (ways, way). */
uint32_t fg_output_split_rank(uint32_t ways, uint32_t way);
/* Vocabulary rows of a way: 2-way [0, 140048) and [140048, 248320); 4-way
 * quarters of 248320.  (0, 0) for an invalid (ways, way). */
void fg_output_split_span(uint32_t ways, uint32_t way, uint32_t *first_row, uint32_t *rows);

/* The owner's combine: its own finalist and `remote_count` remote ones, each
 * with the rank that sent it.  FG_ERR_MISMATCH if a remote rank owns no slice,
 * a remote id is outside that rank's span, or the result is non-finite or
 * not below FG_OUTPUT_SPLIT_VOCAB; otherwise *token (and *logit if non-NULL). */
fg_status fg_output_split_combine_finalists(uint32_t ways, float local_value, uint32_t local_id,
                                            const float *remote_value, const uint32_t *remote_id,
                                            const uint8_t *remote_rank, uint32_t remote_count,
                                            uint32_t *token, float *logit, fg_error *err);

#ifdef __cplusplus
}
#endif

#endif
