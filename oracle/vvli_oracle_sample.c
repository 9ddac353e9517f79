/*
 * vvli_oracle_sample.c -- CPU restatement of VVLI's token sampler
 * (src/generator.zig:14-23 Options, 65-127 Sampler, 338-463 helpers) and of the
 * sampled generation loop (generateGreedyMeasuredInternal, :221-293).
 * TEST INFRASTRUCTURE ONLY: reference results for the GPU sampling kernel.
 *
 * The random stream is Zig's std.Random.DefaultPrng (Xoshiro256, the
 * xoshiro256++ generator of Blackman and Vigna, seeded by four SplitMix64
 * outputs) and Random.float(f32) (23 random mantissa bits, the exponent from
 * the leading zeros of the remaining bits). Zig's standard library is not in
 * the reference tree; these are restated from their published algorithms.
 * Pinned: SplitMix64 against its published first outputs for seed 0;
 * xoshiro256++ against Blackman and Vigna's published known-answer vector
 * (state {1, 2, 3, 4}); float(f32) by closed forms on that stream; the
 * deterministic steps (penalties, candidates, probabilities, top-p cut, the
 * cumulative pick) against the reference's own tests (src/generator.zig:
 * 491-512) and closed forms.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "vvli_oracle.h"

uint64_t orc_splitmix64_next(uint64_t* s) {
    *s += 0x9e3779b97f4a7c15ull;
    uint64_t z = *s;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

void orc_prng_seed(uint64_t state[4], uint64_t seed) {
    uint64_t sm = seed;
    for (int i = 0; i < 4; ++i) state[i] = orc_splitmix64_next(&sm);
}

static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

uint64_t orc_prng_next(uint64_t s[4]) {
    /* xoshiro256++ */
    const uint64_t result = rotl64(s[0] + s[3], 23) + s[0];
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return result;
}

float orc_prng_float(uint64_t s[4]) {
    /* Random.float(f32): mantissa = low 23 bits; exponent 126 - leading zeros
     * of the 64-bit draw, extended by further draws while they are zero. */
    const uint64_t r = orc_prng_next(s);
    uint32_t lz = r ? (uint32_t)__builtin_clzll(r) : 64;
    if (lz >= 41) {
        const uint64_t r2 = orc_prng_next(s);
        lz = 41 + (r2 ? (uint32_t)__builtin_clzll(r2) : 64);
        if (lz == 41 + 64) {
            const uint32_t r3 = (uint32_t)orc_prng_next(s) | 0x7ffu; /* the low 32 bits of one more draw */
            lz += (uint32_t)__builtin_clz(r3);
        }
    }
    const uint32_t bits = ((126u - lz) << 23) | (uint32_t)(r & 0x7fffffu);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

int orc_sampling_validate(const orc_sampling* o) {
    /* validateSamplingOptions, src/generator.zig:329-333 */
    if (o->temperature < 0.0f || isnan(o->temperature)) return ORC_INVALID_SAMPLING;
    if (o->top_p <= 0.0f || o->top_p > 1.0f || isnan(o->top_p)) return ORC_INVALID_SAMPLING;
    if (o->repeat_penalty < 1.0f || isnan(o->repeat_penalty)) return ORC_INVALID_SAMPLING;
    return ORC_OK;
}

void orc_build_repeat_counts(uint16_t* counts, size_t n, const uint32_t* prompt, size_t n_prompt,
                             const uint32_t* generated, size_t n_generated, const orc_sampling* o) {
    /* buildRepeatCounts, src/generator.zig:335-351 */
    memset(counts, 0, n * sizeof(uint16_t));
    if (o->repeat_penalty <= 1.0f || o->repeat_last_n == 0) return;
    const size_t total = n_prompt + n_generated;
    const size_t start = total > o->repeat_last_n ? total - o->repeat_last_n : 0;
    for (size_t i = start; i < total; ++i) {
        const uint32_t tok = i < n_prompt ? prompt[i] : generated[i - n_prompt];
        if (tok >= n) continue;
        if (counts[tok] != 0xffff) counts[tok] += 1;
    }
}

/* buildCandidates (src/generator.zig:367-389) with insertTopCandidate /
 * bubbleCandidateUp (:396-421): the `limit` highest finite adjusted logits in
 * descending order; among equal logits the lower id stays first. With no limit
 * (top_k == 0 or >= n) the reference sorts all candidates with an unstable
 * sort; this restatement keeps ids ascending within equal logits there too. */
typedef struct {
    float score;
    uint32_t id;
} orc_cand;

static int cand_desc(const void* a, const void* b) {
    const orc_cand* x = (const orc_cand*)a;
    const orc_cand* y = (const orc_cand*)b;
    if (x->score != y->score) return x->score > y->score ? -1 : 1;
    return x->id < y->id ? -1 : (x->id > y->id);
}

size_t orc_build_candidates(uint32_t* ids, float* scores, const float* logits, const uint16_t* counts, size_t n,
                            const orc_sampling* o) {
    const size_t limit = (o->top_k == 0 || o->top_k >= n) ? n : o->top_k;
    size_t count = 0;
    if (limit == n) { /* every finite candidate, sorted */
        orc_cand* c = (orc_cand*)malloc((n ? n : 1) * sizeof(orc_cand));
        if (!c) return 0;
        for (size_t i = 0; i < n; ++i) {
            const float s = orc_adjusted_logit(logits[i], counts[i], o->repeat_penalty);
            if (!isfinite(s)) continue;
            c[count].score = s;
            c[count].id = (uint32_t)i;
            ++count;
        }
        qsort(c, count, sizeof(orc_cand), cand_desc);
        for (size_t i = 0; i < count; ++i) ids[i] = c[i].id, scores[i] = c[i].score;
        free(c);
        return count;
    }
    for (size_t i = 0; i < n; ++i) {
        const float s = orc_adjusted_logit(logits[i], counts[i], o->repeat_penalty);
        if (!isfinite(s)) continue;
        if (count < limit) {
            ids[count] = (uint32_t)i;
            scores[count] = s;
            ++count;
        } else {
            if (s <= scores[count - 1]) continue;
            ids[count - 1] = (uint32_t)i;
            scores[count - 1] = s;
        }
        for (size_t j = count - 1; j > 0 && scores[j] > scores[j - 1]; --j) {
            const float ts = scores[j];
            scores[j] = scores[j - 1];
            scores[j - 1] = ts;
            const uint32_t ti = ids[j];
            ids[j] = ids[j - 1];
            ids[j - 1] = ti;
        }
    }
    return count;
}

size_t orc_prepare_probabilities(float* probs, const float* scores, size_t count, const orc_sampling* o) {
    /* prepareProbabilities, src/generator.zig:428-449 */
    if (count == 0) return 0;
    const float temperature = o->temperature > 1e-6f ? o->temperature : 1e-6f;
    const float max_logit = scores[0];
    float total = 0.0f;
    for (size_t i = 0; i < count; ++i) {
        const float p = expf((scores[i] - max_logit) / temperature);
        probs[i] = isfinite(p) ? p : 0.0f;
        total += probs[i];
    }
    if (total <= 0.0f || !isfinite(total)) return 1;
    if (o->top_p >= 1.0f) return count;
    float cumulative = 0.0f;
    for (size_t i = 0; i < count; ++i) {
        cumulative += probs[i];
        if (cumulative / total >= o->top_p) return i + 1;
    }
    return count;
}

uint32_t orc_sample_candidate(const uint32_t* ids, const float* probs, size_t count, float random_unit) {
    /* sampleCandidate, src/generator.zig:451-463 */
    float total = 0.0f;
    for (size_t i = 0; i < count; ++i) total += probs[i];
    if (total <= 0.0f || !isfinite(total)) return ids[0];
    const float target = (random_unit < 0.99999994f ? random_unit : 0.99999994f) * total;
    float cumulative = 0.0f;
    for (size_t i = 0; i < count; ++i) {
        cumulative += probs[i];
        if (target <= cumulative) return ids[i];
    }
    return ids[count - 1];
}

int orc_sampler_next(const float* logits, size_t n, const uint32_t* prompt, size_t n_prompt,
                     const uint32_t* generated, size_t n_generated, const orc_sampling* o, uint64_t prng[4],
                     uint32_t* token_out) {
    /* Sampler.next, src/generator.zig:93-120 */
    int rc = orc_sampling_validate(o);
    if (rc) return rc;
    uint16_t* counts = (uint16_t*)malloc(n * sizeof(uint16_t));
    uint32_t* ids = (uint32_t*)malloc(n * sizeof(uint32_t));
    float* scores = (float*)malloc(n * sizeof(float));
    float* probs = (float*)malloc(n * sizeof(float));
    if (!counts || !ids || !scores || !probs) {
        free(counts), free(ids), free(scores), free(probs);
        return ORC_OUT_OF_MEMORY;
    }
    orc_build_repeat_counts(counts, n, prompt, n_prompt, generated, n_generated, o);
    if (o->temperature <= 0.0f) {
        *token_out = orc_greedy_with_penalties(logits, counts, n, o->repeat_penalty);
    } else {
        const size_t c = orc_build_candidates(ids, scores, logits, counts, n, o);
        if (c == 0) {
            *token_out = (uint32_t)orc_argmax(logits, n);
        } else {
            const size_t k = orc_prepare_probabilities(probs, scores, c, o);
            if (k == 0) {
                *token_out = ids[0];
            } else {
                *token_out = orc_sample_candidate(ids, probs, k, orc_prng_float(prng));
            }
        }
    }
    free(counts), free(ids), free(scores), free(probs);
    return ORC_OK;
}

int orc_generate_sampled(orc_runner* r, size_t vocab, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                         int64_t eos, const orc_sampling* o, uint32_t* out_tokens, uint32_t* n_out) {
    /* generateGreedyMeasuredInternal's loop (src/generator.zig:230-280) with the
     * Sampler; the seed 0 maps to 0x9e3779b97f4a7c15 as in Sampler.init (:75). */
    if (!r || !prompt || !o || !out_tokens || !n_out) return ORC_NULL_ARG;
    if (n_prompt == 0) return ORC_EMPTY_PROMPT;
    int rc = orc_sampling_validate(o);
    if (rc) return rc;
    float* logits = (float*)malloc(vocab * sizeof(float));
    if (!logits) return ORC_OUT_OF_MEMORY;
    uint32_t pos = 0;
    for (uint32_t i = 0; i < n_prompt; ++i)
        if ((rc = orc_forward_token(r, prompt[i], pos++, logits, NULL))) goto done;
    uint64_t prng[4];
    orc_prng_seed(prng, o->seed ? o->seed : 0x9e3779b97f4a7c15ull);
    uint32_t produced = 0;
    while (produced < max_new) {
        uint32_t next;
        if ((rc = orc_sampler_next(logits, vocab, prompt, n_prompt, out_tokens, produced, o, prng, &next))) goto done;
        out_tokens[produced++] = next;
        if (eos >= 0 && (int64_t)next == eos) break;
        if ((rc = orc_forward_token(r, next, pos++, logits, NULL))) goto done;
    }
    *n_out = produced;
done:
    free(logits);
    return rc;
}
