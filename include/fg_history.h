/* Output-history wire format (FG_MSG_OUTPUT_HISTORY payload) and its host
 * codec: the token history a session sends to the rank that samples, from
 * which the sampler's per-row count table is rebuilt.
 *
 * Payload layout (big-endian), reference src/protocol.c:1328-1365:
 *   u32 count | u8 session_slot | 3 zero bytes | count x u32 token
 *
 * The same names and rules as the reference (include/fg_protocol.h:566-571,
 * 757-759): tokens must be below the vocabulary (FG_Q38_VOCAB_SIZE in the
 * reference; the _vocab forms take it as a parameter), count at most
 * FG_NATIVE_CONTEXT, session_slot below FG_DECODE_BATCH_MAX_SLOTS.  The
 * device-side decoder that builds count tables straight from payloads is
 * fg_hip_history_build_wire (fg_sampler_hip.h). */
#ifndef FG_HISTORY_H
#define FG_HISTORY_H

#include <stdint.h>

#include "fg.h"

#ifdef __cplusplus
extern "C" {
#endif

#define FG_OUTPUT_HISTORY_HEADER_BYTES 8u
#define FG_OUTPUT_HISTORY_NATIVE_CONTEXT 262144u   /* FG_NATIVE_CONTEXT, include/fg.h:25 */
#define FG_OUTPUT_HISTORY_MAX_SLOTS 2u             /* FG_DECODE_BATCH_MAX_SLOTS */
#define FG_OUTPUT_HISTORY_MAX_FRAME_BYTES (64u * 1024u * 1024u) /* FG_MAX_FRAME_BYTES */
#define FG_OUTPUT_HISTORY_Q38_VOCAB 248320u         /* FG_Q38_VOCAB_SIZE */
#define FG_OUTPUT_HISTORY_MAX_BYTES \
    (FG_OUTPUT_HISTORY_HEADER_BYTES + FG_OUTPUT_HISTORY_NATIVE_CONTEXT * 4u)

typedef struct fg_output_history {
    const uint32_t *tokens;
    uint32_t count;
    /* Owner session the history belongs to; 0 is the legacy path. */
    uint8_t session_slot;
} fg_output_history;

/* Writes the payload of `history` into output[capacity]; *bytes = its size.
 * FG_ERR_ARGUMENT: null pointers, count > FG_OUTPUT_HISTORY_NATIVE_CONTEXT,
 * session_slot >= FG_OUTPUT_HISTORY_MAX_SLOTS, or count > 0 with no tokens.
 * FG_ERR_LIMIT: capacity (or the frame limit) too small.  FG_ERR_FORMAT: a
 * token >= vocab.  Replaces fg_output_history_encode, src/protocol.c:1328. */
fg_status fg_output_history_encode(uint8_t *output, uint32_t capacity, uint32_t *bytes,
                                   const fg_output_history *history, fg_error *err);
fg_status fg_output_history_encode_vocab(uint8_t *output, uint32_t capacity, uint32_t *bytes,
                                         const fg_output_history *history, uint32_t vocab,
                                         fg_error *err);

/* Parses a payload of `bytes` bytes; tokens go to storage[capacity] and
 * history->tokens points there.  FG_ERR_ARGUMENT: null pointers or fewer
 * than the header's bytes.  FG_ERR_FORMAT: nonzero reserved bytes, a bad
 * slot, a count above the context, above `capacity` or not matching
 * `bytes`, or a token >= vocab.  Replaces fg_output_history_decode,
 * src/protocol.c:1348. */
fg_status fg_output_history_decode(fg_output_history *history, uint32_t *storage,
                                   uint32_t capacity, const uint8_t *payload, uint32_t bytes,
                                   fg_error *err);
fg_status fg_output_history_decode_vocab(fg_output_history *history, uint32_t *storage,
                                         uint32_t capacity, const uint8_t *payload,
                                         uint32_t bytes, uint32_t vocab, fg_error *err);

#ifdef __cplusplus
}
#endif

#endif
