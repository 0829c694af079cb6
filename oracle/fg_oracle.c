/* CPU oracle for the token-sampling path.  TEST INFRASTRUCTURE ONLY: used by
 * tests/ as the checker and by bench.py's cpu_baseline leg; the product never
 * links it.  Build: oracle/Makefile (-O2 -ffp-contract=off, no fast-math). */
#include "fg_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

enum { ST_OK = 0, ST_ARGUMENT = 2, ST_FORMAT = 4, ST_MISMATCH = 5 };

/* ---- Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11) ------------------ */

void fgo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4])
{
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int round = 0; round < 10; round++) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n1 = (uint32_t)p1;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        const uint32_t n3 = (uint32_t)p0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* ---- xorshift64*: src/sampler.c:67-73 ----------------------------------- */

float fgo_xorshift_uniform(uint64_t *state)
{
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return (float)((double)((x * UINT64_C(2685821657736338717)) >> 40) * (1.0 / 16777216.0));
}

/* ---- keys and orders ----------------------------------------------------- */

static uint32_t f2u(float v) { uint32_t u; memcpy(&u, &v, 4); return u; }

/* shaders/fg_topk_select.comp:27-31 */
uint32_t fgo_float_key(float value)
{
    if (!isfinite(value))
        return 0u;
    const uint32_t bits = f2u(value);
    return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}

/* src/output.c:484-492 */
int fgo_greedy_before(float a, uint32_t aid, float b, uint32_t bid)
{
    const int a_pad = aid == FGO_INVALID_ID, b_pad = bid == FGO_INVALID_ID;
    if (a_pad || b_pad)
        return !a_pad && b_pad;
    const int a_bad = !isfinite(a), b_bad = !isfinite(b);
    if (a_bad || b_bad)
        return a_bad != b_bad ? a_bad : aid < bid;
    return a > b || (a == b && aid < bid);
}

/* (key desc, id asc): the top-k ladder's order (see fgo_topk_row). */
static int key_before(uint32_t ka, uint32_t ida, uint32_t kb, uint32_t idb)
{
    return ka > kb || (ka == kb && ida < idb);
}

/* src/sampler.c:75-78 */
static int value_before(float a, uint32_t aid, float b, uint32_t bid)
{
    if (a != b)
        return a > b;
    return aid < bid;
}

/* ---- penalties ------------------------------------------------------------ */

/* src/sampler.c:46-60 with ids[i] = i. */
void fgo_penalties_c(float *scores, const uint32_t *counts, uint32_t n,
                     float presence, float frequency, float repetition)
{
    for (uint32_t i = 0; i < n; i++) {
        const uint32_t c = counts[i];
        if (c == 0u)
            continue;
        float s = scores[i];
        if (repetition != 1.0f)
            s = s > 0.0f ? s / repetition : s * repetition;
        s -= frequency * (float)c + presence;
        scores[i] = s;
    }
}

/* shaders/fg_apply_penalties.comp:13-18: value - frequency*count - presence,
 * evaluated left to right. */
void fgo_penalties_glsl(float *scores, const uint32_t *counts, uint32_t n,
                        float presence, float frequency, float repetition)
{
    for (uint32_t i = 0; i < n; i++) {
        const uint32_t c = counts[i];
        if (c == 0u)
            continue;
        float s = scores[i];
        if (repetition != 1.0f)
            s = s > 0.0f ? s / repetition : s * repetition;
        const float fc = frequency * (float)c;
        const float t = s - fc;
        scores[i] = t - presence;
    }
}

/* ---- argmax step: shaders/fg_argmax_reduce.comp:26-56 --------------------- */

uint32_t fgo_argmax_reduce_step(float *out_scores, uint32_t *out_ids,
                                const float *in_scores, const uint32_t *in_ids,
                                uint32_t count)
{
    const uint32_t groups = (count + 4095u) / 4096u;
    for (uint32_t g = 0; g < groups; g++) {
        float best = -INFINITY;
        uint32_t best_id = FGO_INVALID_ID;
        const uint32_t end = (g + 1u) * 4096u < count ? (g + 1u) * 4096u : count;
        for (uint32_t i = g * 4096u; i < end; i++) {
            const uint32_t id = in_ids ? in_ids[i] : i;
            if (fgo_greedy_before(in_scores[i], id, best, best_id)) {
                best = in_scores[i];
                best_id = id;
            }
        }
        out_scores[g] = best;
        out_ids[g] = best_id;
    }
    return groups;
}

/* ---- top-k step: shaders/fg_topk_select.comp ------------------------------ */

/* Per 1024 tile: the exact top min(k, available) finite entries by (key desc,
 * position asc), emitted in tile order, then padding.  The reference's radix
 * search (fg_topk_select.comp:45-77) picks the same set; its in-tile order is
 * unspecified, this build keeps tile order. */
uint32_t fgo_topk_select_step(float *out_scores, uint32_t *out_ids,
                              const float *in_scores, const uint32_t *in_ids,
                              uint32_t count, uint32_t k)
{
    const uint32_t tiles = (count + 1023u) / 1024u;
    for (uint32_t t = 0; t < tiles; t++) {
        const uint32_t base = t * 1024u;
        const uint32_t avail = count - base < 1024u ? count - base : 1024u;
        const uint32_t limit = k < avail ? k : avail;
        unsigned char chosen[1024];
        memset(chosen, 0, sizeof chosen);
        /* Select greedily `limit` times the best unchosen finite entry. */
        for (uint32_t r = 0; r < limit; r++) {
            int best = -1;
            for (uint32_t i = 0; i < avail; i++) {
                const float v = in_scores[base + i];
                if (chosen[i] || !isfinite(v))
                    continue;
                if (best < 0 || key_before(fgo_float_key(v), i, fgo_float_key(in_scores[base + best]),
                                           (uint32_t)best))
                    best = (int)i;
            }
            if (best < 0)
                break;
            chosen[best] = 1;
        }
        uint32_t o = 0;
        for (uint32_t i = 0; i < avail; i++) {
            if (!chosen[i])
                continue;
            out_scores[t * k + o] = in_scores[base + i];
            out_ids[t * k + o] = in_ids ? in_ids[base + i] : base + i;
            o++;
        }
        for (; o < k; o++) {
            out_scores[t * k + o] = -INFINITY;
            out_ids[t * k + o] = FGO_INVALID_ID;
        }
    }
    return tiles * k;
}

/* ---- exact row top-k ------------------------------------------------------ */

/* Insertion into a sorted list of at most k (key desc, id asc). */
uint32_t fgo_topk_row(const float *scores, uint32_t n, uint32_t k,
                      float *out_scores, uint32_t *out_ids)
{
    uint32_t keys[1024];
    uint32_t ids[1024];
    if (k > 1024u)
        k = 1024u;
    uint32_t have = 0;
    for (uint32_t i = 0; i < n; i++) {
        const float v = scores[i];
        if (!isfinite(v))
            continue;
        const uint32_t key = fgo_float_key(v);
        if (have == k && !key_before(key, i, keys[k - 1u], ids[k - 1u]))
            continue;
        uint32_t at = have < k ? have++ : k - 1u;
        while (at > 0u && key_before(key, i, keys[at - 1u], ids[at - 1u])) {
            keys[at] = keys[at - 1u];
            ids[at] = ids[at - 1u];
            at--;
        }
        keys[at] = key;
        ids[at] = i;
    }
    for (uint32_t j = 0; j < k; j++) {
        if (j < have) {
            out_scores[j] = scores[ids[j]];
            out_ids[j] = ids[j];
        } else {
            out_scores[j] = -INFINITY;
            out_ids[j] = FGO_INVALID_ID;
        }
    }
    return have;
}

/* ---- fg_sampler_select arithmetic: src/sampler.c:80-122 ------------------- */

typedef struct { float v; uint32_t id; } cand_t;

static int cand_cmp(const void *a, const void *b)
{
    const cand_t *x = a, *y = b;
    if (value_before(x->v, x->id, y->v, y->id))
        return -1;
    if (value_before(y->v, y->id, x->v, x->id))
        return 1;
    return 0;
}

static double rel_gap(double a, double b, double scale)
{
    return fabs(a - b) / scale;
}

int32_t fgo_select(float temperature, float top_p, uint32_t top_k,
                   const float *scores, const uint32_t *ids, uint32_t count,
                   float uniform, uint32_t *token, float *logit,
                   uint32_t *cutoff_out, double *margin_out)
{
    *cutoff_out = 0;
    *margin_out = INFINITY;
    cand_t *c = malloc((size_t)(count ? count : 1u) * sizeof *c);
    if (!c)
        return ST_ARGUMENT;
    uint32_t kept = 0;
    for (uint32_t i = 0; i < count; i++)
        if (isfinite(scores[i])) {
            c[kept].v = scores[i];
            c[kept].id = ids[i];
            kept++;
        }
    /* ids are unique, so any sort by (value desc, id asc) equals the
     * reference's stable insertion sort (src/sampler.c:88-96). */
    qsort(c, kept, sizeof *c, cand_cmp);
    if (kept == 0u) {
        free(c);
        return ST_FORMAT;
    }
    if (temperature == 0.0f) {
        *token = c[0].id;
        *logit = c[0].v;
        free(c);
        return ST_OK;
    }
    const uint32_t limit = (top_k != 0u && top_k < kept) ? top_k : kept;
    const double max_raw = c[0].v;
    double sum = 0.0;
    for (uint32_t i = 0; i < limit; i++)
        sum += exp((double)c[i].v - max_raw);
    if (!(sum > 0.0) || !isfinite(sum)) {
        free(c);
        return ST_FORMAT;
    }
    double cumulative = 0.0, margin = INFINITY;
    uint32_t cutoff = limit;
    for (uint32_t i = 0; i < limit; i++) {
        cumulative += exp((double)c[i].v - max_raw) / sum;
        const double g = rel_gap(cumulative, (double)top_p, 1.0);
        if (g < margin)
            margin = g;
        if (cumulative >= top_p) {
            cutoff = i + 1u;
            break;
        }
    }
    const double t = (double)temperature;
    const double max_temp = (double)c[0].v / t;
    double temp_sum = 0.0;
    for (uint32_t i = 0; i < cutoff; i++)
        temp_sum += exp((double)c[i].v / t - max_temp);
    if (!(temp_sum > 0.0) || !isfinite(temp_sum)) {
        free(c);
        return ST_FORMAT;
    }
    if (!isfinite(uniform) || uniform < 0.0f)
        uniform = 0.0f;
    if (uniform >= 1.0f)
        uniform = nextafterf(1.0f, 0.0f);
    const double draw = (double)uniform * temp_sum;
    double chosen = 0.0;
    uint32_t selected = cutoff - 1u;
    for (uint32_t i = 0; i < cutoff; i++) {
        chosen += exp((double)c[i].v / t - max_temp);
        const double g = rel_gap(chosen, draw, temp_sum);
        if (g < margin)
            margin = g;
        if (draw < chosen) {
            selected = i;
            break;
        }
    }
    *token = c[selected].id;
    *logit = c[selected].v;
    *cutoff_out = cutoff;
    *margin_out = margin;
    free(c);
    return ST_OK;
}

/* ---- whole rows ----------------------------------------------------------- */

static int penalties_active(const fgo_config *c)
{
    return c->presence != 0.0f || c->frequency != 0.0f || c->repetition != 1.0f;
}

typedef struct {
    const fgo_config *configs;
    const float *logits;
    uint64_t lstride;
    const uint32_t *counts;
    uint64_t cstride;
    uint32_t n;
    const float *uniforms;
    uint32_t rows;
    uint32_t logprobs;
    fgo_result *results;
    float *lp_values;
    uint32_t *lp_ids;
    float *penalised_out;
    uint32_t first, step;
} job_t;

static void sample_one(const job_t *j, uint32_t r, float *row)
{
    const fgo_config *cfg = &j->configs[r];
    const uint32_t n = j->n;
    fgo_result *res = &j->results[r];
    memcpy(row, j->logits + (uint64_t)r * j->lstride, (size_t)n * 4u);
    const int pen = j->counts != NULL && penalties_active(cfg);
    if (pen)
        fgo_penalties_c(row, j->counts + (uint64_t)r * j->cstride, n,
                        cfg->presence, cfg->frequency, cfg->repetition);
    if (j->penalised_out)
        memcpy(j->penalised_out + (uint64_t)r * n, row, (size_t)n * 4u);
    res->cutoff = 0;
    res->margin = INFINITY;
    if (cfg->temperature == 0.0f) {
        /* src/output.c:560-599 (no penalties) and :728-741 (penalties). */
        float best = -INFINITY;
        uint32_t best_id = FGO_INVALID_ID;
        for (uint32_t i = 0; i < n; i++)
            if (fgo_greedy_before(row[i], i, best, best_id)) {
                best = row[i];
                best_id = i;
            }
        res->token = best_id;
        res->logit = best;
        res->status = (best_id == FGO_INVALID_ID || !isfinite(best))
                          ? (pen ? ST_FORMAT : ST_MISMATCH) : ST_OK;
    } else if (cfg->top_k == 0u) {
        /* Whole-row nucleus: fg_sampler_select over every finite logit. */
        uint32_t *ids = malloc((size_t)n * 4u);
        for (uint32_t i = 0; i < n; i++)
            ids[i] = i;
        res->status = fgo_select(cfg->temperature, cfg->top_p, 0u, row, ids, n,
                                 j->uniforms[r], &res->token, &res->logit,
                                 &res->cutoff, &res->margin);
        free(ids);
    } else {
        /* src/output.c:746-751: exact top-k, then fg_sampler_select. */
        float cs[64];
        uint32_t ci[64];
        fgo_topk_row(row, n, cfg->top_k, cs, ci);
        res->status = fgo_select(cfg->temperature, cfg->top_p, cfg->top_k, cs, ci,
                                 cfg->top_k, j->uniforms[r], &res->token, &res->logit,
                                 &res->cutoff, &res->margin);
    }
    if (res->status != ST_OK) {
        res->token = FGO_INVALID_ID;
    }
    if (j->logprobs) {
        const uint32_t L = j->logprobs;
        const uint32_t kk = cfg->temperature > 0.0f && cfg->top_k > L ? cfg->top_k : L;
        float cs[64];
        uint32_t ci[64];
        const uint32_t have = fgo_topk_row(row, n, kk, cs, ci);
        cand_t c[64];
        for (uint32_t i = 0; i < have; i++) {
            c[i].v = cs[i];
            c[i].id = ci[i];
        }
        qsort(c, have, sizeof c[0], cand_cmp);
        const double t = cfg->temperature > 0.0f ? (double)cfg->temperature : 1.0;
        double m = -INFINITY;
        for (uint32_t i = 0; i < n; i++)
            if (isfinite(row[i]) && (double)row[i] / t > m)
                m = (double)row[i] / t;
        double z = 0.0;
        for (uint32_t i = 0; i < n; i++)
            if (isfinite(row[i]))
                z += exp((double)row[i] / t - m);
        const double lse = m + log(z);
        for (uint32_t i = 0; i < L; i++) {
            float *v = &j->lp_values[(uint64_t)r * L + i];
            uint32_t *id = &j->lp_ids[(uint64_t)r * L + i];
            if (i < have) {
                *v = (float)((double)c[i].v / t - lse);
                *id = c[i].id;
            } else {
                *v = -INFINITY;
                *id = FGO_INVALID_ID;
            }
        }
    }
}

static void *worker(void *arg)
{
    const job_t *j = arg;
    float *row = malloc((size_t)j->n * 4u);
    if (!row)
        return NULL;
    for (uint32_t r = j->first; r < j->rows; r += j->step)
        sample_one(j, r, row);
    free(row);
    return NULL;
}

int fgo_sample_rows(const fgo_config *configs, const float *logits, uint64_t logits_stride,
                    const uint32_t *counts, uint64_t counts_stride, uint32_t n,
                    const float *uniforms, uint32_t rows, uint32_t logprobs,
                    fgo_result *results, float *lp_values, uint32_t *lp_ids,
                    float *penalised_out, uint32_t threads)
{
    if (threads == 0u)
        threads = 1u;
    if (threads > 256u)
        threads = 256u;
    job_t jobs[256];
    pthread_t tid[256];
    for (uint32_t t = 0; t < threads; t++) {
        jobs[t] = (job_t){configs, logits, logits_stride, counts, counts_stride, n, uniforms,
                          rows, logprobs, results, lp_values, lp_ids, penalised_out, t, threads};
    }
    if (threads == 1u) {
        worker(&jobs[0]);
        return 0;
    }
    for (uint32_t t = 0; t < threads; t++)
        pthread_create(&tid[t], NULL, worker, &jobs[t]);
    for (uint32_t t = 0; t < threads; t++)
        pthread_join(tid[t], NULL);
    return 0;
}

/* ---- synthetic inputs ------------------------------------------------------ */

double fgo_u01(uint32_t word)
{
    return ((double)(word >> 8) + 0.5) * (1.0 / 16777216.0);
}

static void philox_words(uint32_t a, uint32_t b, uint32_t c, uint32_t seed, uint32_t cfg,
                         uint32_t out[4])
{
    const uint32_t ctr[4] = {a, b, c, 0x5A4D504Cu};
    const uint32_t key[2] = {seed, cfg};
    fgo_philox4x32_10(ctr, key, out);
}

void fgo_gen_uniforms(float *out, uint32_t rows, uint32_t seed, uint32_t config_id)
{
    for (uint32_t r = 0; r < rows; r++) {
        uint32_t w[4];
        philox_words(r, 0xD8A7u, 0u, seed, config_id, w);
        out[r] = (float)((double)(w[0] >> 8) * (1.0 / 16777216.0));
    }
}

static void box_muller(const uint32_t w[4], double z[4])
{
    const double two_pi = 6.283185307179586476925286766559;
    for (int p = 0; p < 2; p++) {
        const double u1 = fgo_u01(w[2 * p]), u2 = fgo_u01(w[2 * p + 1]);
        const double r = sqrt(-2.0 * log(u1));
        z[2 * p] = r * cos(two_pi * u2);
        z[2 * p + 1] = r * sin(two_pi * u2);
    }
}

void fgo_gen_logits(float *out, uint64_t stride, uint32_t rows, uint32_t n, int kind,
                    double sigma, double sigma2, double nu, uint32_t seed,
                    uint32_t config_id)
{
    for (uint32_t r = 0; r < rows; r++) {
        float *row = out + (uint64_t)r * stride;
        const double s = (kind == 3 && (r & 1u)) ? sigma2 : sigma;
        for (uint32_t q = 0; q < (n + 3u) / 4u; q++) {
            uint32_t w[4];
            double z[4];
            philox_words(r, q, 0u, seed, config_id, w);
            box_muller(w, z);
            if (kind == 1) {
                /* Student-t(nu) = Z / sqrt(chi2_nu / nu); element e takes its
                 * chi-square from the first nu (<= 4) normals of counter word
                 * 1 + e. */
                const int dof = (int)nu;
                for (int e = 0; e < 4 && q * 4u + (uint32_t)e < n; e++) {
                    uint32_t w2[4];
                    double g[4];
                    philox_words(r, q, 1u + (uint32_t)e, seed, config_id, w2);
                    box_muller(w2, g);
                    double chi = 0.0;
                    for (int d = 0; d < dof && d < 4; d++)
                        chi += g[d] * g[d];
                    row[q * 4u + (uint32_t)e] = (float)(s * z[e] / sqrt(chi / nu));
                }
                continue;
            }
            for (int e = 0; e < 4 && q * 4u + (uint32_t)e < n; e++) {
                double v = s * z[e];
                if (kind == 2) {
                    v = nearbyint(v / 0.25) * 0.25;
                    if (v > 16.0) v = 16.0;
                    if (v < -16.0) v = -16.0;
                }
                row[q * 4u + (uint32_t)e] = (float)v;
            }
        }
    }
}

/* Seeded Fisher-Yates permutation of 0..n-1 (rank -> token id). */
static uint32_t *permutation(uint32_t n, uint32_t seed, uint32_t cfg)
{
    uint32_t *p = malloc((size_t)n * 4u);
    if (!p)
        return NULL;
    for (uint32_t i = 0; i < n; i++)
        p[i] = i;
    for (uint32_t i = n - 1u; i > 0u; i--) {
        uint32_t w[4];
        philox_words(i, 0xF15Eu, 0u, seed, cfg, w);
        const uint64_t j = ((uint64_t)w[0] * (uint64_t)(i + 1u)) >> 32;
        const uint32_t t = p[i];
        p[i] = p[j];
        p[j] = t;
    }
    return p;
}

void fgo_gen_zipf_ids(uint32_t *ids, uint32_t rows, uint32_t per_row, uint32_t n,
                      double s, uint32_t seed, uint32_t config_id)
{
    double *cdf = malloc((size_t)n * sizeof *cdf);
    uint32_t *perm = permutation(n, seed, config_id);
    if (!cdf || !perm) {
        free(cdf);
        free(perm);
        return;
    }
    double acc = 0.0;
    for (uint32_t k = 0; k < n; k++) {
        acc += pow((double)(k + 1u), -s);
        cdf[k] = acc;
    }
    for (uint32_t k = 0; k < n; k++)
        cdf[k] /= acc;
    for (uint32_t r = 0; r < rows; r++)
        for (uint32_t i = 0; i < per_row; i++) {
            uint32_t w[4];
            philox_words(r, i, 0x21Fu, seed, config_id, w);
            const double u = fgo_u01(w[0]);
            uint32_t lo = 0, hi = n - 1u;
            while (lo < hi) {
                const uint32_t mid = lo + (hi - lo) / 2u;
                if (cdf[mid] < u)
                    lo = mid + 1u;
                else
                    hi = mid;
            }
            ids[(uint64_t)r * per_row + i] = perm[lo];
        }
    free(cdf);
    free(perm);
}

void fgo_gen_uniform_ids(uint32_t *ids, uint32_t rows, uint32_t per_row, uint32_t n,
                         uint32_t seed, uint32_t config_id)
{
    for (uint32_t r = 0; r < rows; r++)
        for (uint32_t i = 0; i < per_row; i++) {
            uint32_t w[4];
            philox_words(r, i, 0x0E1Du, seed, config_id, w);
            ids[(uint64_t)r * per_row + i] = (uint32_t)(((uint64_t)w[0] * n) >> 32);
        }
}

void fgo_build_counts(uint32_t *counts, uint64_t stride, uint32_t rows, uint32_t n,
                      const uint32_t *ids, uint32_t per_row)
{
    for (uint32_t r = 0; r < rows; r++) {
        uint32_t *c = counts + (uint64_t)r * stride;
        memset(c, 0, (size_t)n * 4u);
        for (uint32_t i = 0; i < per_row; i++) {
            const uint32_t id = ids[(uint64_t)r * per_row + i];
            if (id < n && c[id] != UINT32_MAX)
                c[id]++;
        }
    }
}
