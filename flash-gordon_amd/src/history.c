/* Output-history payload codec (reference src/protocol.c:1328-1366). */
#include "fg_history.h"

#include <stddef.h>

static void put_be32(uint8_t *p, uint32_t v)
{
    p[0] = (uint8_t)(v >> 24);
    p[1] = (uint8_t)(v >> 16);
    p[2] = (uint8_t)(v >> 8);
    p[3] = (uint8_t)v;
}

static uint32_t get_be32(const uint8_t *p)
{
    return ((uint32_t)p[0] << 24) | ((uint32_t)p[1] << 16) | ((uint32_t)p[2] << 8) | p[3];
}

fg_status fg_output_history_encode_vocab(uint8_t *output, uint32_t capacity, uint32_t *bytes,
                                         const fg_output_history *history, uint32_t vocab,
                                         fg_error *err)
{
    if (!output || !bytes || !history || history->count > FG_OUTPUT_HISTORY_NATIVE_CONTEXT ||
        (history->count && !history->tokens) ||
        history->session_slot >= FG_OUTPUT_HISTORY_MAX_SLOTS) {
        fg_error_set(err, FG_ERR_ARGUMENT, "invalid output history");
        return FG_ERR_ARGUMENT;
    }
    const uint64_t required = FG_OUTPUT_HISTORY_HEADER_BYTES + (uint64_t)history->count * 4u;
    if (required > capacity || required > FG_OUTPUT_HISTORY_MAX_FRAME_BYTES) {
        fg_error_set(err, FG_ERR_LIMIT, "output history buffer is too small");
        return FG_ERR_LIMIT;
    }
    put_be32(output, history->count);
    output[4] = history->session_slot;
    output[5] = output[6] = output[7] = 0u;
    for (uint32_t i = 0; i < history->count; i++) {
        if (history->tokens[i] >= vocab) {
            fg_error_set(err, FG_ERR_FORMAT, "output history token is outside vocabulary");
            return FG_ERR_FORMAT;
        }
        put_be32(output + FG_OUTPUT_HISTORY_HEADER_BYTES + 4u * i, history->tokens[i]);
    }
    *bytes = (uint32_t)required;
    return FG_OK;
}

fg_status fg_output_history_encode(uint8_t *output, uint32_t capacity, uint32_t *bytes,
                                   const fg_output_history *history, fg_error *err)
{
    return fg_output_history_encode_vocab(output, capacity, bytes, history,
                                          FG_OUTPUT_HISTORY_Q38_VOCAB, err);
}

fg_status fg_output_history_decode_vocab(fg_output_history *history, uint32_t *storage,
                                         uint32_t capacity, const uint8_t *payload,
                                         uint32_t bytes, uint32_t vocab, fg_error *err)
{
    if (!history || !payload || bytes < FG_OUTPUT_HISTORY_HEADER_BYTES) {
        fg_error_set(err, FG_ERR_ARGUMENT, "invalid output history input");
        return FG_ERR_ARGUMENT;
    }
    const uint32_t count = get_be32(payload);
    const uint8_t slot = payload[4];
    const uint32_t reserved = ((uint32_t)payload[5] << 16) | ((uint32_t)payload[6] << 8) | payload[7];
    const uint64_t required = FG_OUTPUT_HISTORY_HEADER_BYTES + (uint64_t)count * 4u;
    if (reserved || slot >= FG_OUTPUT_HISTORY_MAX_SLOTS ||
        count > FG_OUTPUT_HISTORY_NATIVE_CONTEXT || count > capacity || required != bytes ||
        (count && !storage)) {
        fg_error_set(err, FG_ERR_FORMAT, "invalid output history size or reserved bytes");
        return FG_ERR_FORMAT;
    }
    for (uint32_t i = 0; i < count; i++) {
        const uint32_t token = get_be32(payload + FG_OUTPUT_HISTORY_HEADER_BYTES + 4u * i);
        if (token >= vocab) {
            fg_error_set(err, FG_ERR_FORMAT, "output history token is outside vocabulary");
            return FG_ERR_FORMAT;
        }
        storage[i] = token;
    }
    history->tokens = storage;
    history->count = count;
    history->session_slot = slot;
    return FG_OK;
}

fg_status fg_output_history_decode(fg_output_history *history, uint32_t *storage,
                                   uint32_t capacity, const uint8_t *payload, uint32_t bytes,
                                   fg_error *err)
{
    return fg_output_history_decode_vocab(history, storage, capacity, payload, bytes,
                                          FG_OUTPUT_HISTORY_Q38_VOCAB, err);
}
