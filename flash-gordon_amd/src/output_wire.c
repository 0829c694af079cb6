/* Output-owner wire messages of the sampling path (reference
 * include/fg_protocol.h:461-481, src/protocol.c:1160-1166, 1275-1279). */
#include "fg_output_wire.h"

#include <math.h>
#include <string.h>

static void store_be32(uint8_t *p, uint32_t v)
{
    p[0] = (uint8_t)(v >> 24);
    p[1] = (uint8_t)(v >> 16);
    p[2] = (uint8_t)(v >> 8);
    p[3] = (uint8_t)v;
}

static uint32_t load_be32(const uint8_t *p)
{
    return ((uint32_t)p[0] << 24) | ((uint32_t)p[1] << 16) | ((uint32_t)p[2] << 8) | p[3];
}

static void store_be_f32(uint8_t *p, float v)
{
    uint32_t bits;
    memcpy(&bits, &v, sizeof bits);
    store_be32(p, bits);
}

static float load_be_f32(const uint8_t *p)
{
    const uint32_t bits = load_be32(p);
    float v;
    memcpy(&v, &bits, sizeof v);
    return v;
}

static int controls_all_zero(const fg_sampler_config *s)
{
    return s->temperature == 0.0f && s->top_p == 0.0f && s->top_k == 0u &&
           s->presence_penalty == 0.0f && s->frequency_penalty == 0.0f &&
           s->repetition_penalty == 0.0f && s->min_p == 0.0f;
}

/* src/protocol.c:1160 (validate_output_config). */
static fg_status check_config(const fg_output_config *c, fg_error *err)
{
    if (!c || c->source_rank >= FG_OUTPUT_WIRE_RANKS || c->destination_rank != FG_OUTPUT_WIRE_OWNER ||
        c->session_slot >= FG_OUTPUT_WIRE_SESSIONS) {
        fg_error_set(err, FG_ERR_FORMAT, "invalid output config route");
        return FG_ERR_FORMAT;
    }
    if (!controls_all_zero(&c->sampler) && fg_sampler_config_validate(&c->sampler, err) != FG_OK)
        return FG_ERR_FORMAT;
    if (!isfinite(c->uniform) || c->uniform < 0.0f || c->uniform >= 1.0f) {
        fg_error_set(err, FG_ERR_FORMAT, "invalid output config sampler draw");
        return FG_ERR_FORMAT;
    }
    return FG_OK;
}

fg_status fg_output_config_encode(uint8_t output[FG_OUTPUT_CONFIG_BYTES],
                                  const fg_output_config *config, fg_error *err)
{
    if (!output) {
        fg_error_set(err, FG_ERR_ARGUMENT, "output config buffer is null");
        return FG_ERR_ARGUMENT;
    }
    const fg_status st = check_config(config, err);
    if (st != FG_OK)
        return st;
    output[0] = config->source_rank;
    output[1] = config->destination_rank;
    output[2] = config->flags;
    output[3] = config->session_slot;
    store_be32(output + 4, config->token_index);
    store_be_f32(output + 8, config->sampler.temperature);
    store_be_f32(output + 12, config->sampler.top_p);
    store_be32(output + 16, config->sampler.top_k);
    store_be_f32(output + 20, config->uniform);
    store_be_f32(output + 24, config->sampler.presence_penalty);
    store_be_f32(output + 28, config->sampler.frequency_penalty);
    store_be_f32(output + 32, config->sampler.repetition_penalty);
    store_be_f32(output + 36, config->sampler.min_p);
    return FG_OK;
}

fg_status fg_output_config_decode(fg_output_config *config, const uint8_t *payload,
                                  uint32_t bytes, fg_error *err)
{
    if (!config || !payload) {
        fg_error_set(err, FG_ERR_ARGUMENT, "invalid output config input");
        return FG_ERR_ARGUMENT;
    }
    const uint8_t flags = bytes == FG_OUTPUT_CONFIG_BYTES ? payload[2] : 0u;
    const uint8_t known = FG_OUTPUT_CONFIG_FLAG_SPLIT | FG_OUTPUT_CONFIG_FLAG_SPLIT_4;
    if (bytes != FG_OUTPUT_CONFIG_BYTES || (flags & ~known) ||
        ((flags & FG_OUTPUT_CONFIG_FLAG_SPLIT_4) && !(flags & FG_OUTPUT_CONFIG_FLAG_SPLIT))) {
        fg_error_set(err, FG_ERR_FORMAT, "invalid output config size or reserved bytes");
        return FG_ERR_FORMAT;
    }
    memset(config, 0, sizeof *config);
    config->source_rank = payload[0];
    config->destination_rank = payload[1];
    config->flags = flags;
    config->session_slot = payload[3];
    config->token_index = load_be32(payload + 4);
    config->sampler.temperature = load_be_f32(payload + 8);
    config->sampler.top_p = load_be_f32(payload + 12);
    config->sampler.top_k = load_be32(payload + 16);
    config->uniform = load_be_f32(payload + 20);
    config->sampler.presence_penalty = load_be_f32(payload + 24);
    config->sampler.frequency_penalty = load_be_f32(payload + 28);
    config->sampler.repetition_penalty = load_be_f32(payload + 32);
    config->sampler.min_p = load_be_f32(payload + 36);
    return check_config(config, err);
}

/* src/protocol.c:1275 (validate_output_result). */
static fg_status check_result(const fg_output_result *r, fg_error *err)
{
    if (!r || r->source_rank != FG_OUTPUT_WIRE_OWNER || r->destination_rank >= FG_OUTPUT_WIRE_RANKS ||
        r->token >= FG_OUTPUT_WIRE_VOCAB || !isfinite(r->logit)) {
        fg_error_set(err, FG_ERR_FORMAT, "invalid output result");
        return FG_ERR_FORMAT;
    }
    return FG_OK;
}

fg_status fg_output_result_encode(uint8_t output[FG_OUTPUT_RESULT_BYTES],
                                  const fg_output_result *result, fg_error *err)
{
    if (!output) {
        fg_error_set(err, FG_ERR_ARGUMENT, "output result buffer is null");
        return FG_ERR_ARGUMENT;
    }
    const fg_status st = check_result(result, err);
    if (st != FG_OK)
        return st;
    output[0] = result->source_rank;
    output[1] = result->destination_rank;
    output[2] = 0u;
    output[3] = 0u;
    store_be32(output + 4, result->token_index);
    store_be32(output + 8, result->token);
    store_be_f32(output + 12, result->logit);
    return FG_OK;
}

fg_status fg_output_result_decode(fg_output_result *result, const uint8_t *payload,
                                  uint32_t bytes, fg_error *err)
{
    if (!result || !payload) {
        fg_error_set(err, FG_ERR_ARGUMENT, "invalid output result input");
        return FG_ERR_ARGUMENT;
    }
    if (bytes != FG_OUTPUT_RESULT_BYTES || payload[2] || payload[3]) {
        fg_error_set(err, FG_ERR_FORMAT, "invalid output result size or reserved bytes");
        return FG_ERR_FORMAT;
    }
    memset(result, 0, sizeof *result);
    result->source_rank = payload[0];
    result->destination_rank = payload[1];
    result->token_index = load_be32(payload + 4);
    result->token = load_be32(payload + 8);
    result->logit = load_be_f32(payload + 12);
    return check_result(result, err);
}

fg_status fg_output_configs_batch(const fg_output_config *configs, uint32_t rows,
                                  fg_sampler_config *samplers, float *uniforms, fg_error *err)
{
    if (!configs || !samplers || !uniforms || !rows) {
        fg_error_set(err, FG_ERR_ARGUMENT, "invalid output config batch");
        return FG_ERR_ARGUMENT;
    }
    for (uint32_t r = 0; r < rows; r++) {
        if (controls_all_zero(&configs[r].sampler))
            fg_sampler_config_greedy(&samplers[r]);
        else
            samplers[r] = configs[r].sampler;
        uniforms[r] = configs[r].uniform;
    }
    return FG_OK;
}

fg_status fg_output_results_encode_batch(uint8_t *output, const fg_output_config *configs,
                                         const uint32_t *tokens, const float *logits,
                                         const int32_t *row_status, uint32_t rows,
                                         uint32_t *answered, fg_error *err)
{
    if (answered)
        *answered = 0u;
    if (!output || !configs || !tokens || !logits || !rows) {
        fg_error_set(err, FG_ERR_ARGUMENT, "invalid output result batch");
        return FG_ERR_ARGUMENT;
    }
    uint32_t n = 0u;
    for (uint32_t r = 0; r < rows; r++) {
        uint8_t *at = output + (size_t)FG_OUTPUT_RESULT_BYTES * r;
        if (row_status && row_status[r] != 0) {
            memset(at, 0, FG_OUTPUT_RESULT_BYTES);
            continue;
        }
        const fg_output_result res = {
            .source_rank = FG_OUTPUT_WIRE_OWNER,
            .destination_rank = configs[r].source_rank,
            .token_index = configs[r].token_index,
            .token = tokens[r],
            .logit = logits[r],
        };
        const fg_status st = fg_output_result_encode(at, &res, err);
        if (st != FG_OK)
            return st;
        n++;
    }
    if (answered)
        *answered = n;
    return FG_OK;
}
