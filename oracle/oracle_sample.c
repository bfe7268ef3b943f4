/*
 * oracle_sample.c — TEST INFRASTRUCTURE ONLY: the reference's sampler (crates/core/src/sample.rs) restated in C, the
 * checker for the device sampler. Never linked into the product.
 *
 * Rng (sample.rs:15-51): xoshiro256** (Blackman & Vigna) seeded by four splitmix64 outputs; f32() = (next >> 40) *
 * 2^-24. Sampler::process (sample.rs:181-236): candidates sorted by logit descending, ties by id ascending (the
 * first top_k of them when 0 < top_k < vocab), softmax at the temperature from the top candidate (sequential f32
 * sum in that order), top-p (keep while the mass before a candidate is below top_p), min-p (keep while p >= min_p *
 * p[0]), renormalise (sequential sum). draw (sample.rs:239-251), write_dense (259-265), accept_or_resample
 * (272-303). expf is the platform libm's, as Rust's f32::exp on Linux.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* ------------------------------------------------------------------------------------------------ Rng */

void or_rng_seed(uint64_t seed, uint64_t s[4]) {
    uint64_t x = seed;
    for (int i = 0; i < 4; i++) { /* splitmix64 */
        x += 0x9E3779B97F4A7C15ull;
        uint64_t z = x;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        s[i] = z ^ (z >> 31);
    }
}

static inline uint64_t rotl(uint64_t v, int k) { return (v << k) | (v >> (64 - k)); }

uint64_t or_rng_next(uint64_t s[4]) {
    const uint64_t result = rotl(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return result;
}

float or_rng_f32(uint64_t s[4]) { return (float)(or_rng_next(s) >> 40) * (1.0f / 16777216.0f); }

/* -------------------------------------------------------------------------------------------- Sampler */

struct or_sampler {
    aq_sampler_config cfg;
    uint64_t rng[4];
    uint32_t *idx;
    float *probs;
    size_t n, vocab;
};

or_sampler *or_sampler_new(const aq_sampler_config *cfg, size_t vocab) {
    or_sampler *sp = (or_sampler *)calloc(1, sizeof(or_sampler));
    sp->cfg = *cfg;
    or_rng_seed(cfg->seed, sp->rng);
    sp->idx = (uint32_t *)calloc(vocab + 1, sizeof(uint32_t));
    sp->probs = (float *)calloc(vocab + 1, sizeof(float));
    sp->vocab = vocab;
    return sp;
}

void or_sampler_free(or_sampler *sp) {
    if (!sp) return;
    free(sp->idx);
    free(sp->probs);
    free(sp);
}

void or_sampler_reseed(or_sampler *sp, uint64_t seed) {
    sp->cfg.seed = seed;
    or_rng_seed(seed, sp->rng);
}

void or_sampler_rng(const or_sampler *sp, uint64_t out[4]) { memcpy(out, sp->rng, sizeof sp->rng); }

int or_sampler_is_greedy(const or_sampler *sp) { return !sp || sp->cfg.temperature <= 0.0f; }

static const float *g_cmp_logits; /* the comparator's logits (qsort has no context argument) */

/* sample.rs:196: b's logit against a's (partial_cmp; unordered counts as equal), then the lower id first */
static int by_logit_desc(const void *pa, const void *pb) {
    const uint32_t a = *(const uint32_t *)pa, b = *(const uint32_t *)pb;
    const float la = g_cmp_logits[a], lb = g_cmp_logits[b];
    if (lb > la) return 1;
    if (lb < la) return -1;
    return a < b ? -1 : (a > b ? 1 : 0);
}

/* model.rs:505-513 argmax: the first maximum */
static uint32_t argmax_first(const float *v, size_t n) {
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return (uint32_t)best;
}

size_t or_sampler_process(or_sampler *sp, const float *logits) {
    const aq_sampler_config *cfg = &sp->cfg;
    if (cfg->temperature <= 0.0f) {
        sp->idx[0] = argmax_first(logits, sp->vocab);
        sp->probs[0] = 1.0f;
        sp->n = 1;
        return 1;
    }
    const size_t vocab = sp->vocab;
    for (size_t i = 0; i < vocab; i++) sp->idx[i] = (uint32_t)i;
    const size_t n_cand = (cfg->top_k > 0 && cfg->top_k < vocab) ? cfg->top_k : vocab;
    /* select_nth + sort of the first n_cand under a total order (no NaN) = the first n_cand of a full sort */
    g_cmp_logits = logits;
    qsort(sp->idx, vocab, sizeof(uint32_t), by_logit_desc);
    const float inv_t = 1.0f / cfg->temperature;
    const float m = logits[sp->idx[0]] * inv_t;
    float sum = 0.0f;
    for (size_t i = 0; i < n_cand; i++) {
        const float e = expf(logits[sp->idx[i]] * inv_t - m);
        sp->probs[i] = e;
        sum += e;
    }
    for (size_t i = 0; i < n_cand; i++) sp->probs[i] /= sum;
    size_t n = n_cand;
    if (cfg->top_p < 1.0f) {
        float cum = 0.0f;
        n = 0;
        while (n < n_cand && cum < cfg->top_p) {
            cum += sp->probs[n];
            n++;
        }
        if (n < 1) n = 1;
    }
    if (cfg->min_p > 0.0f) {
        const float thr = cfg->min_p * sp->probs[0];
        size_t keep = 1;
        while (keep < n && sp->probs[keep] >= thr) keep++;
        n = keep;
    }
    float s = 0.0f;
    for (size_t i = 0; i < n; i++) s += sp->probs[i];
    for (size_t i = 0; i < n; i++) sp->probs[i] /= s;
    sp->n = n;
    return n;
}

size_t or_sampler_kept(const or_sampler *sp, uint32_t *ids, float *probs) {
    if (ids) memcpy(ids, sp->idx, sp->n * sizeof(uint32_t));
    if (probs) memcpy(probs, sp->probs, sp->n * sizeof(float));
    return sp->n;
}

uint32_t or_sampler_draw(or_sampler *sp) {
    const float u = or_rng_f32(sp->rng);
    float cum = 0.0f;
    for (size_t i = 0; i < sp->n; i++) {
        cum += sp->probs[i];
        if (u < cum) return sp->idx[i];
    }
    return sp->idx[sp->n - 1];
}

uint32_t or_sampler_sample(or_sampler *sp, const float *logits) {
    or_sampler_process(sp, logits);
    return or_sampler_draw(sp);
}

void or_sampler_write_dense(const or_sampler *sp, float *out) {
    memset(out, 0, sp->vocab * sizeof(float));
    for (size_t i = 0; i < sp->n; i++) out[sp->idx[i]] = sp->probs[i];
}

int or_sampler_accept_or_resample(or_sampler *sp, const float *target, const float *q, uint32_t d, uint32_t *tok) {
    or_sampler_process(sp, target);
    if (sp->cfg.temperature <= 0.0f) {
        *tok = sp->idx[0];
        return sp->idx[0] == d;
    }
    float pd = 0.0f;
    for (size_t i = 0; i < sp->n; i++)
        if (sp->idx[i] == d) {
            pd = sp->probs[i];
            break;
        }
    const float qd = q[d];
    const float u = or_rng_f32(sp->rng);
    if (qd > 0.0f && (pd >= qd || u < pd / qd)) {
        *tok = d;
        return 1;
    }
    float sum = 0.0f;
    for (size_t i = 0; i < sp->n; i++) {
        const float r = fmaxf(sp->probs[i] - q[sp->idx[i]], 0.0f);
        sp->probs[i] = r;
        sum += r;
    }
    if (sum <= 0.0f) {
        or_sampler_process(sp, target);
        *tok = or_sampler_draw(sp);
        return 0;
    }
    for (size_t i = 0; i < sp->n; i++) sp->probs[i] /= sum;
    *tok = or_sampler_draw(sp);
    return 0;
}
