/* CPU oracle for the token-sampling path.  TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain C17 restatement of the reference's sampling semantics,
 * used by tests/ to check the HIP path and by bench.py's cpu_baseline leg as
 * the timed CPU baseline.  The product library never links, loads or calls it.
 *
 * Each function cites the reference lines it restates (paths relative to the
 * reference checkout).  How each one is pinned (golden vectors, compiled
 * reference, closed forms, brute force) is stated next to it; the tests in
 * tests/test_oracle.py carry those checks. */
#ifndef FG_ORACLE_H
#define FG_ORACLE_H

#include <stdint.h>

#define FGO_INVALID_ID 0xffffffffu

typedef struct fgo_config {
    float temperature;
    float top_p;
    uint32_t top_k;            /* 1..64, or 0 = whole-row nucleus (extension) */
    float presence;
    float frequency;
    float repetition;
} fgo_config;

/* Per-row result of fgo_sample_rows. */
typedef struct fgo_result {
    uint32_t token;
    float logit;
    int32_t status;            /* fg_status value */
    uint32_t cutoff;           /* top-p cutoff used by the draw (0 for greedy) */
    double margin;             /* distance of the draw / top-p test from a boundary */
} fgo_result;

/* Random123 Philox4x32-10 (Salmon et al., SC'11).  Pinned by the published
 * known-answer vectors. */
void fgo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* xorshift64* uniform, src/sampler.c:67-73.  Pinned against the compiled
 * reference (oracle/_ref). */
float fgo_xorshift_uniform(uint64_t *state);

/* Order-preserving key, shaders/fg_topk_select.comp:27-31 (NaN/Inf -> 0). */
uint32_t fgo_float_key(float value);

/* Penalties over a row with identity ids.  fgo_penalties_c restates
 * src/sampler.c:46-60 (pinned against the compiled reference and the
 * tests/test_sampler.c:48-53 vector); fgo_penalties_glsl restates
 * shaders/fg_apply_penalties.comp:13-18 ((s - f*c) - p rounding). */
void fgo_penalties_c(float *scores, const uint32_t *counts, uint32_t n,
                     float presence, float frequency, float repetition);
void fgo_penalties_glsl(float *scores, const uint32_t *counts, uint32_t n,
                        float presence, float frequency, float repetition);

/* Greedy order of src/output.c:484-492 / shaders/fg_argmax_reduce.comp:14-24.
 * Returns 1 when (a, aid) ranks before (b, bid). */
int fgo_greedy_before(float a, uint32_t aid, float b, uint32_t bid);

/* One fg_vk_argmax_reduce step (4096-element slices); returns slice count.
 * ids NULL = identity.  Pinned by brute force + tests/test_fg_vk.c:1340-1342. */
uint32_t fgo_argmax_reduce_step(float *out_scores, uint32_t *out_ids,
                                const float *in_scores, const uint32_t *in_ids,
                                uint32_t count);

/* One fg_vk_topk_select step (1024-element tiles, k per tile) in the
 * reference's output order (shaders/fg_topk_select.comp:33-123); returns
 * tiles*k.  ids NULL = identity.  Pinned by tests/test_fg_vk.c:1274-1338 and
 * by comparing each tile's set with a full sort. */
uint32_t fgo_topk_select_step(float *out_scores, uint32_t *out_ids,
                              const float *in_scores, const uint32_t *in_ids,
                              uint32_t count, uint32_t k);

/* Exact top-k of a row by (key desc, id asc), the fixed point of the
 * reference's select ladder (src/output.c:681-700).  Output sorted, padded
 * with (-inf, FGO_INVALID_ID); returns the number of finite entries. */
uint32_t fgo_topk_row(const float *scores, uint32_t n, uint32_t k,
                      float *out_scores, uint32_t *out_ids);

/* fg_sampler_select arithmetic (src/sampler.c:80-122) over `count`
 * candidates; count may exceed 64 (whole-row nucleus extension) and top_k 0
 * means "all".  Returns an fg_status value; *cutoff and *margin describe the
 * top-p cut and how close the f64 running sums came to a decision boundary
 * (relative).  Pinned against the compiled reference on random candidate
 * sets and the tests/test_sampler.c:31-46 vectors. */
int32_t fgo_select(float temperature, float top_p, uint32_t top_k,
                   const float *scores, const uint32_t *ids, uint32_t count,
                   float uniform, uint32_t *token, float *logit,
                   uint32_t *cutoff, double *margin);

/* Whole-row sampling as the HIP batch path defines it (fg_sampler_hip.h):
 * penalties (if active and counts != NULL) -> greedy argmax (T == 0) or
 * exact top-k + select (T > 0; top_k == 0 = nucleus over the whole row), plus
 * `logprobs` top log-probs.  Follows src/output.c:702-756.  penalised_out
 * (optional) receives rows x n penalised logits.  Returns 0. */
int fgo_sample_rows(const fgo_config *configs, const float *logits, uint64_t logits_stride,
                    const uint32_t *counts, uint64_t counts_stride, uint32_t n,
                    const float *uniforms, uint32_t rows, uint32_t logprobs,
                    fgo_result *results, float *lp_values, uint32_t *lp_ids,
                    float *penalised_out, uint32_t threads);

/* ---- synthetic inputs (the benchmark's configs) ------------------------- */

/* Uniform in (0,1) from a Philox word: ((x >> 8) + 0.5) * 2^-24. */
double fgo_u01(uint32_t word);
/* One per-row uniform for the draw: (x >> 8) * 2^-24, x = Philox(row, 0xD8A7). */
void fgo_gen_uniforms(float *out, uint32_t rows, uint32_t seed, uint32_t config_id);
/* rows x n logits.  kind 0: N(0, sigma^2); 1: Student-t(nu) * sigma;
 * 2: N(0, sigma^2) rounded to multiples of 0.25 and clamped to [-16, 16];
 * 3: rows alternate N(0, sigma^2) / N(0, sigma2^2).  Box-Muller on Philox
 * counter (row, element/4), key (seed, config_id). */
void fgo_gen_logits(float *out, uint64_t stride, uint32_t rows, uint32_t n, int kind,
                    double sigma, double sigma2, double nu, uint32_t seed,
                    uint32_t config_id);
/* Zipf(s) history ids over ranks 1..n mapped through a seeded permutation;
 * `per_row` ids per row written to ids[rows*per_row]. */
void fgo_gen_zipf_ids(uint32_t *ids, uint32_t rows, uint32_t per_row, uint32_t n,
                      double s, uint32_t seed, uint32_t config_id);
/* Uniform history ids over [0, n). */
void fgo_gen_uniform_ids(uint32_t *ids, uint32_t rows, uint32_t per_row, uint32_t n,
                         uint32_t seed, uint32_t config_id);
/* Dense count tables from per-row id lists (saturating, src/output.c:601-617). */
void fgo_build_counts(uint32_t *counts, uint64_t stride, uint32_t rows, uint32_t n,
                      const uint32_t *ids, uint32_t per_row);

#endif
