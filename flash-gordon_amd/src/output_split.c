/* Vocabulary-split finalist order, layout and combine (reference
 * src/output.c:484-497, src/protocol.c:23-44 and 93-105,
 * src/runtime.c:2440-2466). */
#include "fg_output_split.h"

#include <math.h>

bool fg_output_better(float left, uint32_t left_id, float right, uint32_t right_id)
{
    const bool lpad = left_id == UINT32_MAX, rpad = right_id == UINT32_MAX;
    if (lpad || rpad)
        return rpad && !lpad;
    const bool lnf = !isfinite(left), rnf = !isfinite(right);
    if (lnf != rnf)
        return lnf;
    if (lnf)
        return left_id < right_id;
    if (left != right)
        return left > right;
    return left_id < right_id;
}

void fg_output_combine(float left, uint32_t left_id, float right, uint32_t right_id,
                       float *value, uint32_t *id)
{
    const bool take_left = fg_output_better(left, left_id, right, right_id);
    if (value)
        *value = take_left ? left : right;
    if (id)
        *id = take_left ? left_id : right_id;
}

/* Ranks by way: the owner first, then ranks 0, 1, 2. */
static const uint32_t split_ranks[FG_OUTPUT_SPLIT_WAYS_MAX] = {FG_OUTPUT_SPLIT_OWNER_RANK, 0u, 1u, 2u};

static bool ways_supported(uint32_t ways)
{
    return ways == FG_OUTPUT_SPLIT_WAYS_MIN || ways == FG_OUTPUT_SPLIT_WAYS_MAX;
}

bool fg_output_split_way_for_rank(uint32_t ways, uint32_t rank, uint32_t *way)
{
    if (!ways_supported(ways))
        return false;
    for (uint32_t w = 0; w < ways; w++) {
        if (split_ranks[w] == rank) {
            if (way)
                *way = w;
            return true;
        }
    }
    return false;
}

uint32_t fg_output_split_rank(uint32_t ways, uint32_t way)
{
    return ways_supported(ways) && way < ways ? split_ranks[way] : UINT32_MAX;
}

void fg_output_split_span(uint32_t ways, uint32_t way, uint32_t *first_row, uint32_t *rows)
{
    uint32_t first = 0u, count = 0u;
    if (ways == FG_OUTPUT_SPLIT_WAYS_MIN && way < ways) {
        first = way ? FG_OUTPUT_SPLIT_FIRST_ROWS : 0u;
        count = way ? FG_OUTPUT_SPLIT_VOCAB - FG_OUTPUT_SPLIT_FIRST_ROWS : FG_OUTPUT_SPLIT_FIRST_ROWS;
    } else if (ways == FG_OUTPUT_SPLIT_WAYS_MAX && way < ways) {
        const uint32_t quarter = FG_OUTPUT_SPLIT_VOCAB / FG_OUTPUT_SPLIT_WAYS_MAX;
        first = way * quarter;
        count = way + 1u == ways ? FG_OUTPUT_SPLIT_VOCAB - first : quarter;
    }
    if (first_row)
        *first_row = first;
    if (rows)
        *rows = count;
}

fg_status fg_output_split_combine_finalists(uint32_t ways, float local_value, uint32_t local_id,
                                            const float *remote_value, const uint32_t *remote_id,
                                            const uint8_t *remote_rank, uint32_t remote_count,
                                            uint32_t *token, float *logit, fg_error *err)
{
    if (!token || (remote_count && (!remote_value || !remote_id || !remote_rank))) {
        fg_error_set(err, FG_ERR_ARGUMENT, "invalid output split combine arguments");
        return FG_ERR_ARGUMENT;
    }
    float best = local_value;
    uint32_t best_id = local_id;
    for (uint32_t i = 0; i < remote_count; i++) {
        uint32_t way = 0u, first = 0u, rows = 0u;
        if (!fg_output_split_way_for_rank(ways, remote_rank[i], &way)) {
            fg_error_set(err, FG_ERR_MISMATCH,
                         "output partial from rank %u which owns no slice in the %u-way split",
                         remote_rank[i], ways);
            return FG_ERR_MISMATCH;
        }
        fg_output_split_span(ways, way, &first, &rows);
        if (remote_id[i] < first || remote_id[i] - first >= rows) {
            fg_error_set(err, FG_ERR_MISMATCH, "output partial id %u is outside rank %u slice %u..%u",
                         remote_id[i], remote_rank[i], first, first + rows);
            return FG_ERR_MISMATCH;
        }
        fg_output_combine(remote_value[i], remote_id[i], best, best_id, &best, &best_id);
    }
    if (best_id >= FG_OUTPUT_SPLIT_VOCAB || !isfinite(best)) {
        fg_error_set(err, FG_ERR_MISMATCH, "invalid combined output finalist");
        return FG_ERR_MISMATCH;
    }
    *token = best_id;
    if (logit)
        *logit = best;
    return FG_OK;
}
