/* binade_chain_model.c -- CPU model of the whole-vocabulary sampler's
 * running-sum algorithm (sample_full_kernel in vvli_amd/csrc/sample.hip),
 * checked against one-after-another f32 sums. Test infrastructure only.
 *
 * The reference adds the candidates' probabilities in order in f32
 * (prepareProbabilities / sampleCandidate, src/generator.zig:428-463). The
 * kernel computes the same sums in parallel: while the running sum c = m * u
 * stays in one binade (u = 2^(e-23), 2^23 <= m < 2^24), fl(c + p) =
 * u * (m + round(p / u)) with ties to an even result; the tentative integer
 * sums (ties rounded down) and the tie corrections (parity changes along the
 * ties) come out of one scan of (sum, tie summary) pairs; the first candidate
 * whose exact sum leaves the binade is added as a plain f32 add and the chunk
 * resumes after it. This file restates that structure -- NT threads of E
 * candidates, chunks held across restarts, windows that start at 1024 after a
 * restart and double -- as sequential C, and compares every sum bit for bit.
 *
 * Build flags plant mistakes that must be caught: -DDROP_FLIP (the scan
 * operator does not shift the later run's parities), -DDROP_INPUT_FLIP (the
 * window's starting parity is ignored), -DDROP_TIES (ties rounded down, no
 * correction).
 *
 * Usage: binade_chain_model [cases] -> prints a summary, exit 0 iff every
 * case matches.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define NT 1024
#define E 8
#define CAP (1u << 30)
#define HAS (1u << 29)
#define W0 1024u

static uint32_t sadd(uint32_t a, uint32_t b) {
    const uint32_t s = a + b;
    return s > CAP ? CAP : s;
}
static float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
/* Tie summary: count of parity changes (bits 0-28), has (29), first (30), last (31). */
static uint32_t comb(uint32_t a, uint32_t b) {
    if (!(a & HAS)) return b;
    if (!(b & HAS)) return a;
    const uint32_t cnt = (a & (HAS - 1)) + (b & (HAS - 1)) + ((a >> 31) != ((b >> 30) & 1u));
    return cnt | HAS | (a & (1u << 30)) | (b & (1u << 31));
}
static uint32_t leaf(uint32_t par) { return HAS | (par << 30) | (par << 31); }
static uint32_t flip(uint32_t y, uint32_t par) { return (par && (y & HAS)) ? y ^ (3u << 30) : y; }
typedef struct {
    uint32_t s, y;
} pair_t;
static pair_t op(pair_t a, pair_t b) {
#ifdef DROP_FLIP
    const pair_t r = {sadd(a.s, b.s), comb(a.y, b.y)};
#else
    const pair_t r = {sadd(a.s, b.s), comb(a.y, flip(b.y, a.s & 1u))};
#endif
    return r;
}

static uint32_t tl[NT][E], mv[NT][E], ties[NT];
static pair_t loc[NT], ex[NT];

static long chain(const float* p, uint32_t n, float* out) {
    float c = 0.0f;
    uint32_t pos = 0, width = W0;
    long iters = 0;
    for (uint32_t cbase = 0; cbase < n; cbase += NT * E) {
        const uint32_t cend = cbase + NT * E < n ? cbase + NT * E : n;
        while (pos < cend) {
            ++iters;
            const uint32_t wend = pos + width < cend ? pos + width : cend;
            const uint32_t bits = f2u(c);
            const int normal = c >= 7.88860905e-31f;
            const int e = (int)((bits >> 23) & 255u) - 127;
            const uint32_t m = (bits & 0x7fffffu) | 0x800000u;
            const float scale = normal ? u2f((uint32_t)(150 - e) << 23) : 0.0f;
            const float ulp = normal ? u2f((uint32_t)(104 + e) << 23) : 0.0f;
            for (int t = 0; t < NT; ++t) { /* per thread: tentative sums, ties, tie summary */
                uint32_t run = 0, y = 0, tb = 0;
                for (int i = 0; i < E; ++i) {
                    const uint32_t j = cbase + (uint32_t)t * E + (uint32_t)i;
                    const int act = normal && j >= pos && j < wend;
                    const float x = fminf((j < n ? p[j] : 0.0f) * scale, 33554432.0f);
                    const float fl = floorf(x), fr = x - fl;
#ifdef DROP_TIES
                    const int tie = 0;
                    const uint32_t q = act ? (uint32_t)fl + (fr > 0.5f ? 1u : 0u) : 0u;
#else
                    const int tie = act && fr == 0.5f;
                    const uint32_t q = act ? (uint32_t)fl + (fr > 0.5f ? 1u : 0u) : 0u;
#endif
                    tb |= (uint32_t)tie << i;
                    run = sadd(run, q);
                    tl[t][i] = run;
                    if (tie) y = comb(y, leaf(run & 1u));
                }
                loc[t].s = run, loc[t].y = y, ties[t] = tb;
            }
            pair_t acc = {0, 0};
            for (int t = 0; t < NT; ++t) ex[t] = acc, acc = op(acc, loc[t]);
            uint32_t stop = 0xffffffffu, prev_stop = 0;
            float p_stop = 0.0f, last = 0.0f;
            for (int t = 0; t < NT; ++t) { /* per thread: corrected sums, first crossing */
#ifdef DROP_INPUT_FLIP
                const uint32_t yin = comb(leaf(0), ex[t].y);
#else
                const uint32_t yin = comb(leaf(0), flip(ex[t].y, m & 1u));
#endif
                uint32_t corr = yin & (HAS - 1), lp = yin >> 31;
                const uint32_t mb = sadd(m, ex[t].s);
                uint32_t prev = sadd(mb, corr);
                for (int i = 0; i < E; ++i) {
                    const uint32_t j = cbase + (uint32_t)t * E + (uint32_t)i;
                    const int act = normal && j >= pos && j < wend;
                    const uint32_t tt = sadd(mb, tl[t][i]);
                    if ((ties[t] >> i) & 1u) {
                        const uint32_t par = tt & 1u;
                        corr += par != lp;
                        lp = par;
                    }
                    mv[t][i] = sadd(tt, corr);
                    const uint32_t fl = (uint32_t)floorf(fminf((j < n ? p[j] : 0.0f) * scale, 33554432.0f));
                    if (act && j < stop && sadd(prev, fl) >= (1u << 24)) stop = j, prev_stop = prev, p_stop = p[j];
                    if (act && j == wend - 1) last = (float)mv[t][i] * ulp;
                    prev = mv[t][i];
                }
            }
            if (!normal) stop = pos, p_stop = p[pos];
            const uint32_t done = stop < wend ? stop : wend;
            for (uint32_t j = pos; j < done; ++j) out[j] = (float)mv[(j - cbase) / E][(j - cbase) % E] * ulp;
            if (stop < wend) {
                const float cp = stop == pos ? c : (float)prev_stop * ulp;
                volatile float cn = cp + p_stop; /* the plain f32 add */
                c = cn;
                out[stop] = c;
                const uint32_t d = 2 * (stop - pos + 1);
                width = d < W0 ? W0 : (d > NT * E ? NT * E : d);
                pos = stop + 1;
            } else {
                c = last;
                width = 2 * width > NT * E ? NT * E : 2 * width;
                pos = wend;
            }
        }
    }
    return iters;
}

static uint64_t rs = 88172645463325252ull;
static double rnd(void) {
    rs ^= rs << 13, rs ^= rs >> 7, rs ^= rs << 17;
    return (double)(rs >> 11) * (1.0 / 9007199254740992.0);
}
static int desc(const void* a, const void* b) {
    const float x = *(const float*)a, y = *(const float*)b;
    return x < y ? 1 : (x > y ? -1 : 0);
}

int main(int argc, char** argv) {
    const int cases = argc > 1 ? atoi(argv[1]) : 200;
    static float p[170000], out[170000], ref[170000];
    int bad = 0;
    long ties_seen = 0;
    for (int cs = 0; cs < cases; ++cs) {
        const uint32_t n = 1 + (uint32_t)(rnd() * (cs % 3 == 0 ? 160000 : cs % 3 == 1 ? 20000 : 3000));
        const int kind = cs % 8;
        const float temp = (float)(0.05 + rnd() * 2.0), sc = (float)(rnd() * 5.0);
        const int z = 10 + cs % 5;
        for (uint32_t i = 0; i < n; ++i) { /* scores */
            float s;
            if (kind == 1) s = (float)(0.01 * rnd());                          /* flat */
            else if (kind == 3) s = rnd() < 0.5 ? 0.0f : (float)(-rnd() * 3); /* many equal */
            else if (kind == 4) s = (float)(-fabs(rnd() * 40));                /* long tail */
            else s = (float)(sc * (rnd() * 2 - 1));
            p[i] = s;
        }
        qsort(p, n, 4, desc);
        const float s0 = p[0];
        for (uint32_t i = 0; i < n; ++i) { /* probabilities, descending */
            float v = expf((p[i] - s0) / temp);
            if (kind == 2) v = ldexpf(1.0f, -(int)(rnd() * 26)) * (rnd() < 0.5 ? 1.0f : 1.5f); /* dyadic */
            if (kind == 5) v = (float)(int)(rnd() * 4) * 0.25f + ldexpf(1.0f, -(int)(rnd() * 24));
            if (kind == 6) v = 1.0f - (float)i / (float)n * 0.5f;
            if (kind == 7) v = 1.0f - ldexpf(1.0f, z - 24); /* a run of exact ties in [2^z, 2^(z+1)) */
            p[i] = isfinite(v) ? v : 0.0f;
        }
        if (kind == 2 || kind == 5) qsort(p, n, 4, desc);
        if (kind != 5) p[0] = 1.0f; /* exp(0): the first candidate */
        volatile float c = 0.0f;
        for (uint32_t i = 0; i < n; ++i) {
            if (i > 0) { /* count the ties the inputs exercise */
                const int e = (int)floor(log2((double)c));
                const double x = (double)p[i] / ldexp(1.0, e - 23);
                ties_seen += (x - floor(x) == 0.5);
            }
            c = c + p[i];
            ref[i] = c;
        }
        chain(p, n, out);
        for (uint32_t i = 0; i < n; ++i)
            if (f2u(out[i]) != f2u(ref[i])) {
                if (bad < 5) printf("case %d (kind %d, n %u): sum %u is %.9g, sequential %.9g\n", cs, kind, n, i, out[i], ref[i]);
                ++bad;
                break;
            }
    }
    printf("%d cases, %d mismatched, %ld ties in the inputs\n", cases, bad, ties_seen);
    return bad != 0;
}
