/* Host implementation of the fg_sampler.h API (C17).
 *
 * Written from the reference's behaviour in src/sampler.c; every function
 * cites the lines whose semantics it reproduces.  The arithmetic order is part
 * of the contract (bit-exact token ids), so each formula keeps the reference's
 * evaluation order and precision:
 *   - penalties are f32 with one IEEE division and no contraction;
 *   - the softmax / top-p / draw sums are sequential f64 sums in sorted order.
 * Build with -ffp-contract=off. */
#include "fg_sampler.h"

#include <math.h>
#include <string.h>

#define FG_SAMPLER_MAX_CANDIDATES 64u

/* Seed used when the caller passes 0 (src/sampler.c:6). */
static const uint64_t default_seed = UINT64_C(0x9e3779b97f4a7c15);

static void config_fill(fg_sampler_config *config, float temperature, float top_p,
                        uint32_t top_k)
{
    config->temperature = temperature;
    config->top_p = top_p;
    config->top_k = top_k;
    config->presence_penalty = 0.0f;
    config->frequency_penalty = 0.0f;
    config->repetition_penalty = 1.0f;
    config->min_p = 0.0f;
    config->seed = default_seed;
}

/* src/sampler.c:8-14 */
void fg_sampler_config_greedy(fg_sampler_config *config)
{
    if (config != NULL)
        config_fill(config, 0.0f, 1.0f, 1u);
}

/* src/sampler.c:16-22 */
void fg_sampler_config_defaults(fg_sampler_config *config)
{
    if (config != NULL)
        config_fill(config, 1.0f, 0.95f, 20u);
}

static bool finite_in(float value, float lo, float hi)
{
    return isfinite(value) && value >= lo && value <= hi;
}

/* src/sampler.c:24-38: T finite >= 0; 0 < top_p <= 1; 1 <= top_k <= 64;
 * presence/frequency finite in [-2, 2]; repetition finite > 0; min_p == 0. */
fg_status fg_sampler_config_validate(const fg_sampler_config *config, fg_error *err)
{
    bool ok = config != NULL;
    if (ok) {
        ok = isfinite(config->temperature) && config->temperature >= 0.0f;
        ok = ok && isfinite(config->top_p) && config->top_p > 0.0f && config->top_p <= 1.0f;
        ok = ok && config->top_k >= 1u && config->top_k <= FG_SAMPLER_MAX_CANDIDATES;
        ok = ok && finite_in(config->presence_penalty, -2.0f, 2.0f);
        ok = ok && finite_in(config->frequency_penalty, -2.0f, 2.0f);
        ok = ok && isfinite(config->repetition_penalty) && config->repetition_penalty > 0.0f;
        ok = ok && isfinite(config->min_p) && config->min_p == 0.0f;
    }
    if (!ok) {
        fg_error_set(err, FG_ERR_ARGUMENT, "invalid sampler controls");
        return FG_ERR_ARGUMENT;
    }
    return FG_OK;
}

/* src/sampler.c:40-44 */
bool fg_sampler_penalties_active(const fg_sampler_config *config)
{
    if (config == NULL)
        return false;
    return config->presence_penalty != 0.0f || config->frequency_penalty != 0.0f ||
           config->repetition_penalty != 1.0f;
}

/* src/sampler.c:46-60.  For a candidate whose token was seen c > 0 times:
 *   repetition != 1:  s = s > 0 ? s / rep : s * rep
 *   then              s = s - (freq * (float)c + pres)      (all f32). */
void fg_sampler_apply_penalties(float *scores, const uint32_t *ids,
                                const uint32_t *counts, uint32_t count,
                                const fg_sampler_config *config)
{
    if (scores == NULL || ids == NULL || counts == NULL || config == NULL)
        return;
    const float rep = config->repetition_penalty;
    const float freq = config->frequency_penalty;
    const float pres = config->presence_penalty;
    for (uint32_t i = 0; i < count; i++) {
        const uint32_t seen = counts[ids[i]];
        if (seen == 0u)
            continue;
        float s = scores[i];
        if (rep != 1.0f)
            s = (s > 0.0f) ? s / rep : s * rep;
        const float scaled = freq * (float)seen;
        const float total = scaled + pres;
        scores[i] = s - total;
    }
}

/* src/sampler.c:62-65 */
void fg_sampler_state_init(fg_sampler_state *state, uint64_t seed)
{
    if (state != NULL)
        state->state = seed != 0u ? seed : default_seed;
}

/* src/sampler.c:67-73: xorshift64* (12, 25, 27; multiplier 2685821657736338717),
 * top 24 bits of the product scaled by 2^-24. */
float fg_sampler_uniform(fg_sampler_state *state)
{
    uint64_t x = state->state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    state->state = x;
    const uint64_t mixed = x * UINT64_C(2685821657736338717);
    const double scale = 1.0 / 16777216.0;
    return (float)((double)(mixed >> 40) * scale);
}

/* Candidate order of src/sampler.c:75-78: larger score first, then lower id. */
static bool ranks_before(float a, uint32_t a_id, float b, uint32_t b_id)
{
    if (a > b)
        return true;
    if (a < b)
        return false;
    return a_id < b_id;
}

static fg_status select_error(fg_error *err, fg_status code, const char *message)
{
    fg_error_set(err, code, "%s", message);
    return code;
}

/* src/sampler.c:80-122.  Steps: (1) validate; (2) stable order of the finite
 * candidates; (3) T == 0 -> first; (4) untempered softmax over the first
 * min(top_k, kept); (5) top-p cutoff on its running sum; (6) tempered softmax
 * over the cutoff; (7) clamp the uniform; (8) inverse-CDF draw. */
fg_status fg_sampler_select(const fg_sampler_config *config,
                            const float *scores, const uint32_t *ids, uint32_t count,
                            float uniform, uint32_t *token, float *logit, fg_error *err)
{
    if (fg_sampler_config_validate(config, err) != FG_OK || scores == NULL ||
        ids == NULL || count == 0u || count > FG_SAMPLER_MAX_CANDIDATES ||
        token == NULL || logit == NULL) {
        if (err != NULL && err->message[0] == '\0')
            fg_error_set(err, FG_ERR_ARGUMENT, "invalid sampler candidates");
        return (err != NULL && err->code != FG_OK) ? err->code : FG_ERR_ARGUMENT;
    }

    /* Insertion into a sorted index list; equal keys keep arrival order. */
    uint32_t order[FG_SAMPLER_MAX_CANDIDATES];
    uint32_t kept = 0u;
    for (uint32_t i = 0; i < count; i++) {
        if (!isfinite(scores[i]))
            continue;
        uint32_t slot = kept++;
        while (slot > 0u) {
            const uint32_t prev = order[slot - 1u];
            if (!ranks_before(scores[i], ids[i], scores[prev], ids[prev]))
                break;
            order[slot] = prev;
            slot--;
        }
        order[slot] = i;
    }
    if (kept == 0u)
        return select_error(err, FG_ERR_FORMAT, "sampler received no finite candidates");

    if (config->temperature == 0.0f) {
        *token = ids[order[0]];
        *logit = scores[order[0]];
        return FG_OK;
    }

    const uint32_t limit = config->top_k < kept ? config->top_k : kept;
    const double top = (double)scores[order[0]];
    double raw_sum = 0.0;
    for (uint32_t i = 0; i < limit; i++)
        raw_sum += exp((double)scores[order[i]] - top);
    if (!(raw_sum > 0.0) || !isfinite(raw_sum))
        return select_error(err, FG_ERR_FORMAT, "sampler raw softmax failed");

    uint32_t cutoff = limit;
    double mass = 0.0;
    for (uint32_t i = 0; i < limit; i++) {
        mass += exp((double)scores[order[i]] - top) / raw_sum;
        if (mass >= (double)config->top_p) {
            cutoff = i + 1u;
            break;
        }
    }

    const double temperature = (double)config->temperature;
    const double top_scaled = (double)scores[order[0]] / temperature;
    double tempered_sum = 0.0;
    for (uint32_t i = 0; i < cutoff; i++)
        tempered_sum += exp((double)scores[order[i]] / temperature - top_scaled);
    if (!(tempered_sum > 0.0) || !isfinite(tempered_sum))
        return select_error(err, FG_ERR_FORMAT, "sampler temperature softmax failed");

    float u = uniform;
    if (!isfinite(u) || u < 0.0f)
        u = 0.0f;
    if (u >= 1.0f)
        u = nextafterf(1.0f, 0.0f);
    const double target = (double)u * tempered_sum;

    uint32_t pick = cutoff - 1u;
    double running = 0.0;
    for (uint32_t i = 0; i < cutoff; i++) {
        running += exp((double)scores[order[i]] / temperature - top_scaled);
        if (target < running) {
            pick = i;
            break;
        }
    }
    *token = ids[order[pick]];
    *logit = scores[order[pick]];
    return FG_OK;
}
