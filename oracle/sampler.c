/* CPU restatement of crates/mivi-model/src/sampler.rs (Sampler::sample and
 * its helpers). TEST INFRASTRUCTURE ONLY: the checker for the device
 * sampler, never part of the product.
 *
 * Pinned by the reference's own tests (sampler.rs:322-404, restated in
 * tests/test_oracle_sampler.py): the seed-0 fallback, argmax, zero
 * temperature with penalties, top-p reaching past the first 1024 tokens,
 * min-p thresholds, and the penalty arithmetic; plus closed forms
 * (xorshift64* by hand, categorical frequencies against the probabilities).
 * Tie order inside the top-p sort is unspecified in the reference
 * (sort_unstable_by, sampler.rs:178-184); this restatement sorts ties by
 * index ("parity unpinned" for tied probabilities at the sampled position). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* sampler.rs:6-13 */
#define OR_FALLBACK_SEED 0x853c49e6748fea9bULL
#define OR_XORSHIFT_MUL 0x2545F4914F6CDD1DULL

uint64_t or_sampler_seed(uint64_t seed) { return seed == 0 ? OR_FALLBACK_SEED : seed; } /* sampler.rs:54-57 */

/* sampler.rs:70-77, xorshift64* (Vigna 2014) */
float or_random_f32(uint64_t* state) {
    uint64_t s = *state;
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    *state = s;
    const uint64_t r = (s * OR_XORSHIFT_MUL) >> 32;
    return (float)(r >> 8) / 16777216.0f;
}

/* sampler.rs:219-257 */
void or_apply_penalties(float* l, size_t n, const uint32_t* recent, size_t nr, float rep, float presence,
                        float frequency) {
    for (size_t i = 0; i < nr; i++) {
        const uint32_t tok = recent[i];
        if ((size_t)tok >= n) continue;
        int seen = 0;
        for (size_t k = 0; k < i; k++)
            if (recent[k] == tok) seen = 1;
        if (seen) continue;
        size_t count = 0;
        for (size_t k = 0; k < nr; k++) count += recent[k] == tok;
        if (rep > 0.0f && rep != 1.0f) {
            if (l[tok] > 0.0f) l[tok] /= rep;
            else l[tok] *= rep;
        }
        if (presence != 0.0f) l[tok] -= presence;
        if (frequency != 0.0f) l[tok] -= frequency * (float)count;
    }
}

/* sampler.rs:260-276 */
void or_apply_min_p(float* l, size_t n, float min_p) {
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (l[i] > mx && isfinite(l[i])) mx = l[i];
    if (!isfinite(mx)) return;
    const float thr = mx + logf(min_p);
    for (size_t i = 0; i < n; i++)
        if (l[i] < thr) l[i] = -INFINITY;
}

static int desc_f32(const void* a, const void* b) {
    const float x = *(const float*)a, y = *(const float*)b;
    return x > y ? -1 : x < y ? 1 : 0;
}

/* sampler.rs:287-301: the k-th largest value (inputs without NaN) is the cutoff */
void or_apply_top_k(float* l, size_t n, size_t k) {
    float* s = (float*)malloc(n * sizeof(float));
    memcpy(s, l, n * sizeof(float));
    qsort(s, n, sizeof(float), desc_f32);
    const float cutoff = s[k - 1];
    free(s);
    for (size_t i = 0; i < n; i++)
        if (l[i] < cutoff) l[i] = -INFINITY;
}

typedef struct {
    uint32_t idx;
    float p;
} or_cand;

static int desc_cand(const void* a, const void* b) {
    const or_cand *x = (const or_cand*)a, *y = (const or_cand*)b;
    if (x->p > y->p) return -1;
    if (x->p < y->p) return 1;
    return x->idx < y->idx ? -1 : x->idx > y->idx ? 1 : 0;
}

/* sampler.rs:137-148 */
static uint32_t sample_categorical(const float* p, size_t n, uint64_t* rng) {
    const float r = or_random_f32(rng);
    float cum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        cum += p[i];
        if (r <= cum) return (uint32_t)i;
    }
    return n ? (uint32_t)(n - 1) : 0;
}

/* sampler.rs:150-215 (the quickselect window loop only bounds the sort; the
 * nucleus is the shortest descending prefix reaching top_p) */
static uint32_t sample_top_p(const float* p, size_t n, float top_p, uint64_t* rng) {
    const float cutoff = (n > 1 && top_p < 1.0f) ? (1.0f - top_p) / ((float)n - 1.0f) : 0.0f;
    or_cand* s = (or_cand*)malloc((n ? n : 1) * sizeof(or_cand));
    size_t m = 0;
    for (size_t i = 0; i < n; i++)
        if (p[i] >= cutoff && p[i] > 0.0f && isfinite(p[i])) s[m++] = (or_cand){(uint32_t)i, p[i]};
    if (m == 0) {
        free(s);
        return or_argmax(p, n);
    }
    qsort(s, m, sizeof(or_cand), desc_cand);
    float mass = 0.0f;
    size_t cut = m;
    for (size_t i = 0; i < m; i++) {
        mass += s[i].p;
        if (mass >= top_p) {
            cut = i + 1;
            break;
        }
    }
    const float r = or_random_f32(rng) * mass;
    float cum = 0.0f;
    uint32_t out = s[0].idx;
    for (size_t i = 0; i < cut; i++) {
        cum += s[i].p;
        if (cum >= r) {
            out = s[i].idx;
            break;
        }
    }
    free(s);
    return out;
}

/* sampler.rs:91-135 Sampler::sample: logits are modified in place */
uint32_t or_sample(float* l, size_t n, const uint32_t* recent, size_t nr, const or_sampler_config* c,
                   uint64_t* rng) {
    if (nr > 0 && ((c->repetition_penalty > 0.0f && c->repetition_penalty != 1.0f) || c->presence_penalty != 0.0f ||
                   c->frequency_penalty != 0.0f))
        or_apply_penalties(l, n, recent, nr, c->repetition_penalty, c->presence_penalty, c->frequency_penalty);
    if (c->temperature <= 0.0f) return or_argmax(l, n);
    const float inv = 1.0f / c->temperature; /* sampler.rs:279-285 */
    for (size_t i = 0; i < n; i++) l[i] *= inv;
    if (c->min_p > 0.0f && c->min_p < 1.0f) or_apply_min_p(l, n, c->min_p);
    if (c->top_k > 0 && (size_t)c->top_k < n) or_apply_top_k(l, n, c->top_k);
    or_softmax(l, n);
    if (c->top_p < 1.0f) return sample_top_p(l, n, c->top_p, rng);
    return sample_categorical(l, n, rng);
}
