/* The reference's token sampler (dwim inference/sampler.rs), restated in C
 * as the checker of the device's.  TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Everything is f32 in the reference's order of operations, its exp the C
 * library's expf (Rust's f32::exp on Linux calls it). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* sampler.rs:136-146: xorshift64*, uniform in [0, 1) (24 bits) */
float or_xorshift_next(uint64_t *state) {
    uint64_t s = *state;
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    *state = s;
    const uint64_t bits = s * 0x2545F4914F6CDD1DULL;
    return (float)(bits >> 40) / (float)(1ULL << 24);
}

/* sampler.rs:29-38: the generator starts from max(seed, 1) */
void or_sampler_init(or_sampler *s, float temperature, size_t top_k, float top_p, float min_p, uint64_t seed) {
    s->temperature = temperature;
    s->top_k = top_k;
    s->top_p = top_p;
    s->min_p = min_p;
    s->rng = seed > 1 ? seed : 1;
}

/* sampler.rs:84-133 (candidates): the top k in one pass over the logits,
 * kept in order (an equal logit goes after those already kept, and one
 * equal to the k-th is not taken: the first index wins), then at a nonzero
 * temperature their softmax, cut to top_p and min_p.  Writes the kept tokens
 * and probabilities (at most min(top_k, len) of each) and returns how many;
 * *total is their probabilities' sum (1 at temperature zero). */
size_t or_sampler_candidates(const or_sampler *s, const float *logits, size_t len, uint32_t *tokens, float *probs,
                             float *total) {
    size_t k = s->top_k < 1 ? 1 : s->top_k > len ? len : s->top_k;
    uint32_t *ct = malloc(sizeof(uint32_t) * (k + 1));
    float *cl = malloc(sizeof(float) * (k + 1));
    size_t n = 0;
    for (size_t token = 0; token < len; token++) {
        const float logit = logits[token];
        if (n == k && logit <= cl[k - 1]) continue;
        /* partition_point(|l| l >= logit): the first kept entry below it */
        size_t at = 0;
        while (at < n && cl[at] >= logit) at++;
        memmove(ct + at + 1, ct + at, sizeof(uint32_t) * (n - at));
        memmove(cl + at + 1, cl + at, sizeof(float) * (n - at));
        ct[at] = (uint32_t)token;
        cl[at] = logit;
        if (n < k) n++;
    }
    size_t kept_n;
    if (s->temperature == 0.0f) {
        tokens[0] = ct[0];
        probs[0] = 1.0f;
        *total = 1.0f;
        kept_n = 1;
    } else {
        const float max = cl[0];
        float sum = 0.0f;
        for (size_t i = 0; i < n; i++) {
            probs[i] = expf((cl[i] - max) / s->temperature);
            sum += probs[i];
        }
        for (size_t i = 0; i < n; i++) probs[i] /= sum;
        const float floor_ = s->min_p * probs[0];
        float kept = 0.0f;
        size_t m = 0;
        while (m < n && kept < s->top_p && probs[m] >= floor_) {
            kept += probs[m];
            m++;
        }
        for (size_t i = 0; i < m; i++) tokens[i] = ct[i];
        *total = kept;
        kept_n = m;
    }
    free(ct);
    free(cl);
    return kept_n;
}

/* sampler.rs:40-51 (sample) */
uint32_t or_sample(or_sampler *s, const float *logits, size_t len) {
    uint32_t *tokens = malloc(sizeof(uint32_t) * (len ? len : 1));
    float *probs = malloc(sizeof(float) * (len ? len : 1));
    float total;
    const size_t n = or_sampler_candidates(s, logits, len, tokens, probs, &total);
    const float r = or_xorshift_next(&s->rng) * total;
    float acc = 0.0f;
    uint32_t pick = tokens[n - 1];
    for (size_t i = 0; i < n; i++) {
        acc += probs[i];
        if (r < acc) {
            pick = tokens[i];
            break;
        }
    }
    free(tokens);
    free(probs);
    return pick;
}

/* sampler.rs:53-81 (verify): the draft is kept with the probability sample
 * would pick it; otherwise another kept token is picked in proportion to
 * the rest's probabilities.  *accepted says which. */
uint32_t or_sampler_verify(or_sampler *s, const float *logits, size_t len, uint32_t draft, int *accepted) {
    uint32_t *tokens = malloc(sizeof(uint32_t) * (len ? len : 1));
    float *probs = malloc(sizeof(float) * (len ? len : 1));
    float total;
    const size_t n = or_sampler_candidates(s, logits, len, tokens, probs, &total);
    float p = 0.0f;
    for (size_t i = 0; i < n; i++)
        if (tokens[i] == draft) {
            p = probs[i];
            break;
        }
    uint32_t pick = draft;
    *accepted = 0;
    if (p >= total || or_xorshift_next(&s->rng) * total < p) {
        *accepted = 1;
    } else {
        const float r = or_xorshift_next(&s->rng) * (total - p);
        float acc = 0.0f;
        uint32_t last = draft;
        int found = 0;
        for (size_t i = 0; i < n && !found; i++) {
            if (tokens[i] == draft) continue;
            acc += probs[i];
            if (r < acc) {
                pick = tokens[i];
                found = 1;
            }
            last = tokens[i];
        }
        if (!found) pick = last;
    }
    free(tokens);
    free(probs);
    return pick;
}
