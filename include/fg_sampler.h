/* Host sampler API, drop-in for the reference's include/fg_sampler.h:1-34.
 *
 * The declarations below are the reference's public surface, unchanged, so
 * callers (reference src/output.c:708-752, src/runtime.c:4622, src/api.c:1613,
 * src/decode_batch.c:147) link against this library without edits.  The
 * implementation is flash-gordon_amd/src/sampler.c. */
#ifndef FLASH_GORDON_SAMPLER_H
#define FLASH_GORDON_SAMPLER_H

#include "fg.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Per-request controls (reference include/fg_sampler.h:6-15). */
typedef struct fg_sampler_config {
    float temperature;
    float top_p;
    uint32_t top_k;
    float presence_penalty;
    float frequency_penalty;
    float repetition_penalty;
    float min_p;
    uint64_t seed;
} fg_sampler_config;

/* xorshift64* stream state, one per request (include/fg_sampler.h:17-19). */
typedef struct fg_sampler_state {
    uint64_t state;
} fg_sampler_state;

/* Presets: greedy T=0,k=1 / defaults T=1,p=.95,k=20 (src/sampler.c:8-22). */
void fg_sampler_config_greedy(fg_sampler_config *config);
void fg_sampler_config_defaults(fg_sampler_config *config);
/* Range checks; FG_ERR_ARGUMENT "invalid sampler controls" (src/sampler.c:24-38). */
fg_status fg_sampler_config_validate(const fg_sampler_config *config, fg_error *err);
/* Seed 0 selects the default seed (src/sampler.c:62-65). */
void fg_sampler_state_init(fg_sampler_state *state, uint64_t seed);
/* Next uniform in [0,1) with 24 bits (src/sampler.c:67-73). */
float fg_sampler_uniform(fg_sampler_state *state);
/* Top-k / top-p / temperature draw over <=64 candidates (src/sampler.c:80-122). */
fg_status fg_sampler_select(const fg_sampler_config *config,
                            const float *scores, const uint32_t *ids, uint32_t count,
                            float uniform, uint32_t *token, float *logit, fg_error *err);
/* presence != 0 || frequency != 0 || repetition != 1 (src/sampler.c:40-44). */
bool fg_sampler_penalties_active(const fg_sampler_config *config);
/* In-place penalties from a dense count table (src/sampler.c:46-60). */
void fg_sampler_apply_penalties(float *scores, const uint32_t *ids,
                                const uint32_t *counts, uint32_t count,
                                const fg_sampler_config *config);

#ifdef __cplusplus
}
#endif

#endif
