/* MI355X (gfx950) token-sampling path: the C ABI.
 *
 * Plain C, plain pointers and sizes.  Every device pointer below is a HIP
 * device address owned by the caller; `stream` is a hipStream_t passed as
 * void* (NULL = the null stream).  All launches are stream-ordered and return
 * without synchronising.  Invalid arguments return FG_ERR_ARGUMENT with a
 * message and launch nothing, as the reference's Vulkan wrappers do
 * (src/vk.c:1812-1818, 2240-2248, 2260).  No C++ exception crosses this ABI.
 *
 * Two layers are exported:
 *
 *  1. Unit kernels that replace the reference's three GPU entry points one for
 *     one (same arguments, same output counts, same error behaviour), so a
 *     port of src/output.c:681-756 can swap the Vulkan ladder for HIP:
 *        fg_hip_apply_penalties   <- fg_vk_apply_penalties  include/fg_vk.h:324-327
 *        fg_hip_argmax_reduce     <- fg_vk_argmax_reduce    include/fg_vk.h:509-512
 *        fg_hip_topk_select       <- fg_vk_topk_select      include/fg_vk.h:494-499
 *
 *  2. The batched sampler, which replaces the per-row orchestration of
 *     fg_output_sample (src/output.c:702-756: penalties -> argmax | top-k ->
 *     readback -> fg_sampler_select -> history increment) with one fused
 *     launch over many rows that ends in a token id per row on the device.
 */
#ifndef FLASH_GORDON_SAMPLER_HIP_H
#define FLASH_GORDON_SAMPLER_HIP_H

#include "fg_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Padding id written by top-k / argmax for slots with no finite candidate
 * (shaders/fg_topk_select.comp:16, fg_argmax_reduce.comp:15). */
#define FG_HIP_INVALID_ID 0xffffffffu
/* Largest top_k and largest log-prob count per row (src/sampler.c:27). */
#define FG_HIP_MAX_TOPK 64u

/* ------------------------------------------------------------------------ */
/* 1. Unit kernels                                                           */
/* ------------------------------------------------------------------------ */

/* In-place penalties over `values` logits from a dense u32 count table of the
 * same length (identity token ids).  Replaces fg_vk_apply_penalties
 * (src/vk.c:1808-1823, shaders/fg_apply_penalties.comp).  Rounds as the C
 * formula of src/sampler.c:55-58: s' = rep(s) - (freq*(float)c + pres).
 * Errors: values == 0, NULL pointers, non-finite penalty, repetition <= 0. */
fg_status fg_hip_apply_penalties(float *logits, const uint32_t *counts, uint32_t values,
                                 float presence_penalty, float frequency_penalty,
                                 float repetition_penalty, void *stream, fg_error *err);

/* One argmax step: the best (value, id) of each 4096-element slice is written
 * to out_*[slice]; *output_count = ceil(count / 4096).  Call repeatedly until
 * one remains (src/output.c:565, 728-733).  Order: real ids before padding,
 * non-finite before finite (lower id first), then larger value, then lower id
 * (shaders/fg_argmax_reduce.comp:14-24).  in_ids == NULL means ids 0..count-1.
 * Replaces fg_vk_argmax_reduce (src/vk.c:2260). */
fg_status fg_hip_argmax_reduce(float *output_scores, uint32_t *output_ids,
                               const float *input_scores, const uint32_t *input_ids,
                               uint32_t count, uint32_t *output_count,
                               void *stream, fg_error *err);

/* One top-k step: each 1024-element tile yields its exact top min(k, tile)
 * finite candidates by the order-preserving float key (NaN/Inf excluded,
 * +0 above -0, lower position first on ties), padded with (-inf,
 * FG_HIP_INVALID_ID); *output_count = ceil(count/1024) * k.  Call repeatedly
 * until output_count <= k (src/output.c:681-700).  The reference leaves the
 * order inside a tile unspecified (include/fg_vk.h:492-493); here the
 * selected entries keep their tile order, so equal keys stay in position
 * order and the ladder's fixed point is the exact top-k by (key desc, id
 * asc).  in_ids == NULL means ids 0..count-1.  Errors: k outside [1, 64],
 * count == 0.  Replaces fg_vk_topk_select (src/vk.c:2237-2258). */
fg_status fg_hip_topk_select(float *output_scores, uint32_t *output_ids,
                             const float *input_scores, const uint32_t *input_ids,
                             uint32_t count, uint32_t k, uint32_t *output_count,
                             void *stream, fg_error *err);

/* Top-512 per 4096-value tile: output tile g holds the tile's entries in
 * the order of shaders/fg_topk_reduce_v2.comp:9 (non-finite first, then
 * larger score, ties to the lower id; padding id 0xffffffff last), the first
 * min(512, n_g) of them, the rest of its 512 slots (-inf, 0xffffffff).
 * *output_count = 512 per tile, or count when one tile holds fewer than 512.
 * Outputs must hold *output_count entries.  in_ids == NULL means ids
 * 0..count-1.  Errors: count == 0, null pointers ("invalid top-k reduction
 * dispatch").  Replaces fg_vk_topk_reduce (src/vk.c:2235); the caller
 * iterates it as the reference does (src/qsa.c:839-851). */
fg_status fg_hip_topk_reduce(float *output_scores, uint32_t *output_ids,
                             const float *input_scores, const uint32_t *input_ids,
                             uint32_t count, uint32_t *output_count, void *stream,
                             fg_error *err);

/* The whole QSA top-512 scan in one launch (no counterpart entry point in
 * the reference, which iterates fg_vk_topk_reduce, src/qsa.c:839-851): the
 * top min(count, 512) entries of the input in the comparator order of
 * fg_hip_topk_reduce, sorted, as the reference's loop leaves them;
 * *output_count = min(count, 512).  in_ids == NULL means ids 0..count-1.
 * `workspace`: fg_hip_topk_reduce_all_workspace_bytes(count) bytes of
 * device memory, 256-byte aligned, zero before the first call with it.
 * Bytes 4-7 and 16-19 hold a barrier generation and a call counter that
 * calls advance; each call returns the rest of the first 98,368 bytes
 * (counters and tables) to zero and writes what else it reads.  Calls that share a workspace must not
 * overlap.
 * FG_ERR_LIMIT when the count's 4096-entry tiles are more than 1024 or more
 * workgroups than the device holds at once (262,144 scores are 64 tiles).
 * Errors: count == 0, null pointers. */
uint64_t fg_hip_topk_reduce_all_workspace_bytes(uint32_t count);
fg_status fg_hip_topk_reduce_all(float *output_scores, uint32_t *output_ids,
                                 const float *input_scores, const uint32_t *input_ids,
                                 uint32_t count, void *workspace, uint32_t *output_count,
                                 void *stream, fg_error *err);

/* Dense history count tables from token lists, one launch, stream-ordered,
 * no synchronisation: for each row r, counts[r*stride .. +vocab) is cleared
 * and then incremented once per id in ids[offsets[r] .. offsets[r+1])
 * (device memory).  Replaces fg_output_history_reset (src/output.c:601-617)
 * for many rows at once, with its per-row outcome in row_status[r] (device
 * int32): FG_OK; FG_ERR_FORMAT when an id is outside the vocabulary (the
 * reference's "history token %u is outside vocabulary": the row holds the
 * counts of the ids before it, as the reference's table does); or
 * FG_ERR_ARGUMENT for more than FG_NATIVE_CONTEXT (262,144) ids (counts left
 * as they were).  Calls on different streams touch only their own buffers.
 * Errors: null pointers, rows == 0, stride < vocab. */
fg_status fg_hip_history_build(uint32_t *counts, uint64_t counts_stride, uint32_t vocab,
                               const uint32_t *ids, const uint64_t *offsets,
                               uint32_t rows, int32_t *row_status, void *stream,
                               fg_error *err);

/* The same count tables straight from FG_MSG_OUTPUT_HISTORY payloads
 * (fg_history.h): row r's payload is payloads[offsets[r] .. offsets[r+1])
 * (device memory, big-endian, any alignment).  Each payload is checked as
 * fg_output_history_decode_vocab checks it, against `vocab`; row_status[r]
 * gets FG_OK, FG_ERR_ARGUMENT (shorter than the header) or FG_ERR_FORMAT,
 * and row_slot[r] (optional) the session slot.  A valid row's counts are
 * cleared and incremented per token (saturating); an invalid row's counts
 * are left as they were, as the reference leaves the history when decoding
 * fails (src/runtime.c:2696-2702 then src/output.c:601-617).  Stream-ordered,
 * no synchronisation.  Errors: null pointers, rows == 0, stride < vocab. */
fg_status fg_hip_history_build_wire(uint32_t *counts, uint64_t counts_stride, uint32_t vocab,
                                    const uint8_t *payloads, const uint64_t *offsets,
                                    uint32_t rows, int32_t *row_status, uint8_t *row_slot,
                                    void *stream, fg_error *err);

/* ------------------------------------------------------------------------ */
/* 2. Batched sampler                                                        */
/* ------------------------------------------------------------------------ */

typedef struct fg_sampler_hip fg_sampler_hip;

/* Extension flag for fg_sampler_hip_set_configs: accept top_k == 0, meaning
 * "no top-k": fg_sampler_select (src/sampler.c:80-122) over every finite
 * logit of the row (nucleus over the whole vocabulary).  The reference
 * rejects top_k == 0 (src/sampler.c:27); without this flag so does this
 * library.  Such rows are finished in the fused pass when the cut falls
 * inside the row's 64 best logits, otherwise by a second kernel launched on
 * the same stream (histogram descent over the whole row). */
#define FG_SAMPLER_HIP_ALLOW_FULL_VOCAB 1u

/* Creates a sampler for rows of `vocab` logits and up to `max_rows` rows per
 * call.  Allocates the device workspace once (candidate lists, row counters);
 * the calls below allocate nothing.  Uses the current HIP device.  Reads the
 * tuning variables FG_HIP_TARGET_GROUPS, FG_HIP_PAIRED, FG_HIP_FRONT_SHARE,
 * FG_HIP_PACE, FG_HIP_FINISHER and FG_HIP_FINISHER_WAIT_US (launch geometry
 * and hand-off only; results do not depend on them). */
fg_status fg_sampler_hip_create(fg_sampler_hip **out, uint32_t vocab, uint32_t max_rows,
                                fg_error *err);
void fg_sampler_hip_destroy(fg_sampler_hip *sampler);

/* No counterpart in the reference (its per-token dispatches wait on a host
 * fence, src/output.c:702-756): the wait limit of the finisher hand-off of
 * later fg_sampler_hip_sample calls, in microseconds (default 100000).  In
 * that hand-off one workgroup of each row waits, on the device, for the
 * row's other workgroups (it is used only when the whole launch fits on the
 * device at once); a row whose wait passes the limit gets row_status
 * FG_ERR_UNAVAILABLE and token 0xffffffff instead of a token.  0 makes
 * every such row that is not complete at the first look report it (a
 * host-side way to exercise that path). */
fg_status fg_sampler_hip_set_wait_limit(fg_sampler_hip *sampler, uint64_t wait_us, fg_error *err);

/* Validates each row's controls as fg_sampler_config_validate does and keeps
 * them for later fg_sampler_hip_sample calls.  Row r of a batch uses
 * configs[r].  Launches nothing itself: up to 64 configured rows travel in
 * the arguments of the next sample launch (which also writes them to the
 * sampler's device table), more as the arguments of small fill kernels
 * launched first by the next call that reads the controls (sample or
 * history_increment), on that call's stream.  So the call never waits for
 * the device, needs no staging copy, and an owner loop that sets every
 * row's controls before every sample, as the reference ships them with
 * every token (src/protocol.c:1158-1166), costs one launch per step.
 * `stream` is unused (kept for the signature); launches that read the
 * controls must be on one stream. */
fg_status fg_sampler_hip_set_configs(fg_sampler_hip *sampler, const fg_sampler_config *configs,
                                     uint32_t rows, uint32_t flags, void *stream,
                                     fg_error *err);

typedef struct fg_sampler_hip_batch {
    const float *logits;        /* rows x logits_stride f32, read only */
    uint64_t logits_stride;     /* elements between rows, >= vocab */
    const uint32_t *counts;     /* rows x counts_stride u32 history counts, or NULL */
    uint64_t counts_stride;     /* elements between rows, >= vocab */
    const float *uniforms;      /* one uniform per row (unused by greedy rows) */
    uint32_t rows;              /* 1 .. max_rows */
    uint32_t *tokens;           /* out: chosen id per row */
    float *token_logits;        /* out (optional): penalised, untempered logit of the id */
    int32_t *row_status;        /* out (optional): fg_status per row */
    float *penalised;           /* out (optional): rows x vocab penalised logits */
    uint32_t logprobs;          /* 0 .. 64 top log-probs per row */
    float *logprob_values;      /* out: rows x logprobs, s/T - logsumexp(s/T) */
    uint32_t *logprob_ids;      /* out: rows x logprobs */
} fg_sampler_hip_batch;

/* Samples one token per row in one launch (two when a row has top_k == 0).
 * Per row, with the row's config:
 *   penalties (when fg_sampler_penalties_active and counts != NULL),
 *   T == 0: argmax with the reference's greedy order; a non-finite winner sets
 *           row_status FG_ERR_MISMATCH (no penalties, src/output.c:593) or
 *           FG_ERR_FORMAT (penalties, src/output.c:736-740);
 *   T  > 0: exact top_k by float key, then fg_sampler_select's arithmetic on
 *           those candidates with the row's uniform (src/sampler.c:80-122);
 *           top_k == 0 (extension) runs the same rule over the whole row
 *           (FG_ERR_LIMIT only if that search finds no element, which a
 *           row with a finite logit does not produce).
 * Log-probs: the first `logprobs` of the row's max(top_k, logprobs) best
 * candidates ordered by (value desc, id asc), lp = s/T - logsumexp_j(s_j/T)
 * over the finite penalised logits of the row (T == 0 uses T = 1).
 * Rows are independent.  One call at a time per sampler: calls on different
 * streams that overlap on one sampler race on its workspace. */
fg_status fg_sampler_hip_sample(fg_sampler_hip *sampler, const fg_sampler_hip_batch *batch,
                                void *stream, fg_error *err);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  fg_sampler_hip_set_configs + fg_sampler_hip_sample in
 * one call, with no sampler object: the same kernels and the same results,
 * but the controls travel as kernel arguments and the workspace is a
 * file-scope device array of FG_SAMPLER_HIP_STATIC_BYTES bytes per GPU
 * (allocated when the library loads, held until the process ends).  Allocates
 * nothing and never waits for the device.  configs[r] are row r's controls
 * (host memory, read before return); flags as for set_configs.  At most
 * FG_SAMPLER_HIP_STATIC_MAX_ROWS rows (more: FG_ERR_LIMIT).  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (different
 * streams, or another thread) race and must be serialised by the caller. */
#define FG_SAMPLER_HIP_STATIC_MAX_ROWS 256u
#define FG_SAMPLER_HIP_STATIC_BYTES 2856960u
fg_status fg_sampler_hip_sample_static(uint32_t vocab, const fg_sampler_config *configs,
                                       uint32_t flags, const fg_sampler_hip_batch *batch,
                                       void *stream, fg_error *err);

/* Launch geometry of fg_sampler_hip_sample, for tests and tuning (no
 * counterpart in the reference, whose per-tile dispatches have a fixed
 * shape, shaders/fg_topk_select.comp).  Each row is split into `chunks`
 * workgroups of four waves; wave i = chunk * 4 + w streams elements
 * [begin, end) of its row, slices of `wave_elems` for chunks < split and
 * `wave_elems_b` after.  split < chunks: the row's chunks are divided between
 * the grid's two dispatch halves. */
typedef struct fg_sampler_hip_geometry {
    uint32_t chunks;
    uint32_t split;
    uint32_t wave_elems;
    uint32_t wave_elems_b;
    uint32_t pace; /* 1: waves step their issue priority down as they progress */
} fg_sampler_hip_geometry;

#define FG_SAMPLER_HIP_ROWS_NUCLEUS 1u     /* some row is a whole-row nucleus (top_k 0) */
#define FG_SAMPLER_HIP_ROWS_UNLIKE_COST 2u /* rows differ in whether penalties apply */

/* The geometry a sampler created now (same environment) uses for `rows` rows
 * of `vocab` logits with the given FG_SAMPLER_HIP_ROWS_* traits.  Host only:
 * no device is needed.  FG_ERR_ARGUMENT on invalid arguments. */
fg_status fg_sampler_hip_plan(uint32_t vocab, uint32_t rows, uint32_t traits,
                              fg_sampler_hip_geometry *out, fg_error *err);

/* Which row and chunk workgroup `block` of such a launch takes, and the
 * element range [begin, end) of its wave `wave` (0-3).  Host only. */
fg_status fg_sampler_hip_block(const fg_sampler_hip_geometry *g, uint32_t vocab, uint32_t rows,
                               uint32_t block, uint32_t wave, uint32_t *row, uint32_t *chunk,
                               uint32_t *begin, uint32_t *end, fg_error *err);

/* After a draw, adds 1 (saturating) to counts[r*stride + tokens[r]] for every
 * row whose config has penalties active and whose row_status is FG_OK (or
 * row_status == NULL).  Replaces fg_output_history_increment as called at
 * src/output.c:752. */
fg_status fg_sampler_hip_history_increment(fg_sampler_hip *sampler, uint32_t *counts,
                                           uint64_t counts_stride, const uint32_t *tokens,
                                           const int32_t *row_status, uint32_t rows,
                                           void *stream, fg_error *err);

/* ---- Q8_0 matrix-vector products over cooked weights (fg_quant.h) ----
 * output[t*rows + r] = scale * sum_i w(r, i) * input[t*in + i] for t <
 * tokens, r < rows, w the cooked Q8_0 rows (ceil(rows/16) tiles of
 * fg_q8_0_cooked_tile_bytes(in) bytes, 16-byte aligned; so is input).  Sums
 * are f32 in the device's own order (within 1e-5 of the exact product's sum
 * of magnitudes).  Errors: in == 0, in % 32, in > 8192, tokens == 0, rows
 * == 0, null or unaligned pointers ("invalid cooked Q8_0 dense dispatch").
 * Replaces fg_vk_dense_q8_0_f32 for cooked weights (src/vk.c:1451-1453). */
fg_status fg_hip_dense_q8_0_cooked(float *output, const void *weights, const float *input,
                                   uint32_t in, uint32_t rows, uint32_t tokens, float scale,
                                   void *stream, fg_error *err);

/* ---- vocabulary-split greedy output (fg_output_split.h has the layout) ----
 * A rank holding vocabulary rows [first_row, first_row + rows) of the LM head
 * reduces its logits to one (value, id) finalist per decode row; the output
 * owner gathers the finalists and combines them.  Greedy only, as in the
 * reference (src/runtime.c:2399-2401). */
typedef struct fg_hip_output_slice fg_hip_output_slice;

/* Mirrors fg_output_slice_create (src/output.c:234-258) without the model:
 * `vocab` is the full vocabulary, `ways` 2 or 4 (or 1), the slice non-empty and
 * inside [0, vocab), and `max_batch_rows` (1..65535) the most decode rows
 * one call reduces.  `ways` 1 (an extension) is the whole head on one GPU.  FG_ERR_ARGUMENT ("invalid output slice arguments") otherwise;
 * FG_ERR_OOM when the workspace cannot be allocated. */
fg_status fg_hip_output_slice_create(fg_hip_output_slice **out, uint32_t vocab, uint32_t ways,
                                     uint32_t first_row, uint32_t rows,
                                     uint32_t max_batch_rows, fg_error *err);
void fg_hip_output_slice_destroy(fg_hip_output_slice *slice);
/* ways of the slice, 0 for NULL (fg_output_slice_ways, src/output.c:318). */
uint32_t fg_hip_output_slice_ways(const fg_hip_output_slice *slice);

/* The reduction half of fg_output_slice_run (src/output.c:320-344) for
 * batch_rows decode rows: logits[r*stride + i], i < rows, is the logit of
 * vocabulary id first_row + i.  values[r], ids[r] receive the row's best
 * (value, id) in fg_output_better's order; row_status[r] is FG_OK, or
 * FG_ERR_MISMATCH when that value is non-finite ("invalid output slice
 * finalist"), or FG_ERR_UNAVAILABLE (value -inf, id 0xffffffff) when the
 * step's tagged hand-off waited past the slice's wait limit (see
 * fg_hip_output_slice_reduce_combine).  One launch; calls on one slice must
 * not overlap (they share its workspace). */
fg_status fg_hip_output_slice_reduce(fg_hip_output_slice *slice, const float *logits,
                                     uint64_t stride, uint32_t batch_rows, float *values,
                                     uint32_t *ids, int32_t *row_status, void *stream,
                                     fg_error *err);

/* fg_hip_output_slice_reduce and fg_hip_output_split_combine in one launch:
 * the owner's step of src/runtime.c:2440-2466 (its own slice reduced, then
 * combined with the finalists the other ranks sent) for a slice of 2 or 4
 * ways.  part_*[r*ways + i] for i >= 1 and span_first/span_rows are as for
 * fg_hip_output_split_combine (part_*[r*ways + 0] is not read: the own
 * finalist is computed here); tokens/logits_out (may be NULL)/row_status as
 * there.  No counterpart entry point in the reference, whose owner runs the
 * two halves back to back.  When the step's grid fits the device at once
 * and the slice's ids are below 2^18, the slice's chunks hand their bests to
 * the row's last chunk through tagged words; otherwise one workgroup streams
 * each row.  A row whose finishing chunk waited past the slice's wait limit
 * gets status FG_ERR_UNAVAILABLE and token 0xffffffff.  Replays of a
 * captured launch are exact: the words' epochs live on the device. */
fg_status fg_hip_output_slice_reduce_combine(
    fg_hip_output_slice *slice, const float *logits, uint64_t stride, uint32_t batch_rows,
    const float *part_values, const uint32_t *part_ids, const uint8_t *part_ranks,
    const uint32_t *span_first, const uint32_t *span_rows, uint32_t *tokens, float *logits_out,
    int32_t *row_status, void *stream, fg_error *err);

/* The tagged hand-off's wait limit for the slice's steps, in microseconds
 * (initially FG_HIP_FINISHER_WAIT_US or 100,000; at most 42,000,000; 0 gives
 * up at the first poll that finds a word missing).  No counterpart in the
 * reference. */
fg_status fg_hip_output_slice_set_wait_limit(fg_hip_output_slice *slice, uint64_t wait_us,
                                             fg_error *err);

/* fg_output_slice_run_hidden (src/output.c:367-383): its dense product
 * (output_slice_reduce, src/output.c:320-344) fused with its reduction: weights are the slice's cooked rows
 * (its first_row must be a multiple of 16), hidden[t*in ..] the inputs of
 * tokens t < tokens (<= max_batch_rows).  values/ids/row_status as
 * fg_hip_output_slice_reduce over the logits fg_hip_dense_q8_0_cooked would
 * write, bit for bit; logits (may be NULL) receives those logits too.  Ways
 * 1 (an extension: the whole head on one GPU) is allowed at create. */
fg_status fg_hip_output_slice_run_dense(fg_hip_output_slice *slice, const void *weights,
                                        const float *hidden, uint32_t in, uint32_t tokens,
                                        float scale, float *values, uint32_t *ids,
                                        int32_t *row_status, float *logits, void *stream,
                                        fg_error *err);

/* fg_output_sample (src/output.c:702-756) fused with the LM head it samples
 * from, for `tokens` hidden vectors: per token t, the logits
 * fg_hip_dense_q8_0_cooked would write (never stored), penalties over
 * counts[t*counts_stride + id] when fg_sampler_penalties_active(configs[t])
 * and counts != NULL (the C rounding of fg_sampler_apply_penalties), then
 * T == 0: the argmax (the greedy order of fg_output_better; a non-finite
 * winner sets row_status FG_ERR_FORMAT with penalties, FG_ERR_MISMATCH
 * without, and token 0xffffffff), or T > 0: the exact top_k (1..64) and
 * fg_sampler_select with uniforms[t].  out_tokens[t], out_logits[t] (the
 * penalised, untempered logit) and row_status[t] as fg_sampler_hip_sample
 * writes them for those logits.  Whole-head slices only (ways 1, first_row
 * 0, rows == vocab); configs are host memory, validated as
 * fg_sampler_config_validate does (FG_ERR_ARGUMENT, "invalid sampler
 * controls").  One launch per two tokens; calls on one slice must not
 * overlap.  The history increment stays a separate step
 * (fg_sampler_hip_history_increment, or the caller's own). */
fg_status fg_hip_output_slice_run_dense_sampled(
    fg_hip_output_slice *slice, const void *weights, const float *hidden, uint32_t in,
    uint32_t tokens, float scale, const fg_sampler_config *configs, const uint32_t *counts,
    uint64_t counts_stride, const float *uniforms, uint32_t *out_tokens, float *out_logits,
    int32_t *row_status, void *stream, fg_error *err);

/* The owner's combine (src/runtime.c:2440-2466) for `rows` decode rows:
 * part_*[r*ways + 0] is the owner's own finalist, part_*[r*ways + i] (i >= 1)
 * the one rank part_ranks[r*ways + i] sent.  span_first/span_rows (host
 * arrays of `ways` entries, by way) give each way's vocabulary rows, as
 * fg_output_split_span does for the reference vocabulary; they must tile
 * [0, vocab).  Ranks map to ways as fg_output_split_way_for_rank.  Per row:
 * tokens[r] and logits_out[r] (may be NULL) get the combined finalist and
 * row_status[r] FG_OK, or FG_ERR_MISMATCH (token 0xffffffff) when a rank owns
 * no slice, an id is outside its rank's span, or the result is non-finite or
 * >= vocab. */
fg_status fg_hip_output_split_combine(uint32_t *tokens, float *logits_out, int32_t *row_status,
                                      const float *part_values, const uint32_t *part_ids,
                                      const uint8_t *part_ranks, uint32_t rows, uint32_t ways,
                                      uint32_t vocab, const uint32_t *span_first,
                                      const uint32_t *span_rows, void *stream, fg_error *err);

#ifdef __cplusplus
}
#endif

#endif
