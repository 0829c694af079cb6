/* C17 test of the host sampler API (include/fg_sampler.h) in
 * libfg_sampler_hip.so: presets, validation bounds, draws and penalties on the
 * known answers of the reference's tests/test_sampler.c:9-55.  Exit 0 = pass. */
#include "fg_sampler.h"

#include <math.h>
#include <stdio.h>

static int failures;
#define EXPECT(x)                                                        \
    do {                                                                 \
        if (!(x)) {                                                      \
            fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #x); \
            failures++;                                                  \
        }                                                                \
    } while (0)

static fg_status validate(fg_sampler_config c)
{
    fg_error err = {0};
    return fg_sampler_config_validate(&c, &err);
}

int main(void)
{
    fg_sampler_config c;
    fg_sampler_config_defaults(&c);
    EXPECT(c.temperature == 1.0f && c.top_p == 0.95f && c.top_k == 20u);
    EXPECT(validate(c) == FG_OK);
    fg_sampler_config v = c;
    v.presence_penalty = 2.0f;
    v.frequency_penalty = -2.0f;
    EXPECT(validate(v) == FG_OK);
    v.presence_penalty = 2.01f;
    EXPECT(validate(v) == FG_ERR_ARGUMENT);
    v = c;
    v.frequency_penalty = -2.01f;
    EXPECT(validate(v) == FG_ERR_ARGUMENT);
    v = c;
    v.repetition_penalty = 0.0f;
    EXPECT(validate(v) == FG_ERR_ARGUMENT);
    v = c;
    v.min_p = 0.1f;
    EXPECT(validate(v) == FG_ERR_ARGUMENT);
    v = c;
    v.top_k = 65u;
    EXPECT(validate(v) == FG_ERR_ARGUMENT);
    v.top_k = 0u;
    EXPECT(validate(v) == FG_ERR_ARGUMENT);
    v = c;
    v.top_p = 0.0f;
    EXPECT(validate(v) == FG_ERR_ARGUMENT);
    v.top_p = NAN;
    EXPECT(validate(v) == FG_ERR_ARGUMENT);

    fg_error err = {0};
    EXPECT(fg_sampler_config_validate(NULL, &err) == FG_ERR_ARGUMENT && err.code == FG_ERR_ARGUMENT);

    fg_sampler_config_greedy(&c);
    EXPECT(c.temperature == 0.0f && c.top_k == 1u && !fg_sampler_penalties_active(&c));

    const float scores[] = {5.0f, 4.0f, 3.0f};
    const uint32_t ids[] = {9u, 3u, 1u};
    uint32_t tok = 0;
    float logit = 0;
    c.temperature = 1.0f;
    c.top_p = 1.0f;
    c.top_k = 3u;
    EXPECT(fg_sampler_select(&c, scores, ids, 3u, 0.8f, &tok, &logit, &err) == FG_OK && tok == 3u);
    c.temperature = 0.1f;
    EXPECT(fg_sampler_select(&c, scores, ids, 3u, 0.8f, &tok, &logit, &err) == FG_OK && tok == 9u);
    c.top_p = 0.5f;
    EXPECT(fg_sampler_select(&c, scores, ids, 3u, 0.99f, &tok, &logit, &err) == FG_OK && tok == 9u);
    c.top_p = 1.0f;
    c.temperature = 0.01f;
    EXPECT(fg_sampler_select(&c, scores, ids, 3u, 0.99f, &tok, &logit, &err) == FG_OK && tok == 9u);
    const float tied[] = {1.0f, 1.0f};
    const uint32_t tied_ids[] = {8u, 2u};
    c.temperature = 0.0f;
    c.top_k = 1u;
    EXPECT(fg_sampler_select(&c, tied, tied_ids, 2u, 0.5f, &tok, &logit, &err) == FG_OK && tok == 2u);
    const float none[] = {NAN, INFINITY};
    fg_error e2 = {0};
    EXPECT(fg_sampler_select(&c, none, tied_ids, 2u, 0.5f, &tok, &logit, &e2) == FG_ERR_FORMAT);
    fg_error e3 = {0};
    EXPECT(fg_sampler_select(&c, scores, ids, 0u, 0.5f, &tok, &logit, &e3) == FG_ERR_ARGUMENT);

    fg_sampler_state a, b;
    fg_sampler_state_init(&a, 42u);
    fg_sampler_state_init(&b, 42u);
    for (int i = 0; i < 4; i++) {
        const float x = fg_sampler_uniform(&a);
        EXPECT(x == fg_sampler_uniform(&b) && x >= 0.0f && x < 1.0f);
    }

    c.presence_penalty = 1.0f;
    c.frequency_penalty = 0.5f;
    c.repetition_penalty = 2.0f;
    EXPECT(fg_sampler_penalties_active(&c));
    float pen[] = {4.0f, -4.0f, 3.0f};
    const uint32_t pen_ids[] = {1u, 2u, 3u};
    const uint32_t counts[] = {0u, 2u, 3u, 0u};
    fg_sampler_apply_penalties(pen, pen_ids, counts, 3u, &c);
    EXPECT(pen[0] == 0.0f && pen[1] == -10.5f && pen[2] == 3.0f);

    if (failures == 0)
        printf("test_fg_sampler: ok\n");
    return failures ? 1 : 0;
}
