/*
 * vvli_oracle.c -- CPU restatement of VVLI's dense-decoder forward pass.
 *
 * TEST INFRASTRUCTURE ONLY: reference results for the parity tests and the
 * timed CPU baseline. The product library never links or calls this file. See vvli_oracle.h for the
 * pinning status of each function.
 *
 * Built with -ffp-contract=off so that `acc + a*b` stays an unfused multiply
 * and add, as Zig's strict float mode keeps vector `acc += a * b`; the scalar
 * tails use fmaf() where the reference calls @mulAdd.
 */
#define _GNU_SOURCE
#include "vvli_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#define MAX_LANES 16
#define MAX_WORKERS 64 /* src/llm.zig:11 max_worker_threads */
#define ALIGN_BYTES 64 /* src/tensor.zig:8 data_alignment_bytes */

/* ------------------------------------------------------------------------ */
/* scalar conversions: src/llm.zig:791-803                                   */
/* ------------------------------------------------------------------------ */

float orc_bf16_to_f32(uint16_t bits) {
    uint32_t u = (uint32_t)bits << 16; /* src/llm.zig:791-793 */
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t orc_f32_to_bf16(float value) {
    /* src/llm.zig:799-803: round to nearest even, no NaN special case. */
    uint32_t bits;
    memcpy(&bits, &value, 4);
    uint32_t rounded = bits + 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)(rounded >> 16);
}

float orc_f16_to_f32(uint16_t bits) {
    /* src/llm.zig:795-797 (@floatCast of an f16): IEEE binary16 decode. */
    uint32_t sign = (uint32_t)(bits >> 15) << 31;
    uint32_t exp = (bits >> 10) & 0x1f;
    uint32_t man = bits & 0x3ff;
    uint32_t out;
    if (exp == 0) {
        if (man == 0) {
            out = sign;
        } else { /* subnormal: renormalise */
            int e = -1;
            do {
                man <<= 1;
                e++;
            } while ((man & 0x400) == 0);
            man &= 0x3ff;
            out = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        out = sign | 0x7f800000u | (man << 13);
    } else {
        out = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &out, 4);
    return f;
}

static inline float weight_at(const void* w, uint32_t kind, size_t i) {
    /* src/llm.zig:289-294 WeightSlice.at */
    return kind == 1 ? orc_bf16_to_f32(((const uint16_t*)w)[i]) : ((const float*)w)[i];
}

/* ------------------------------------------------------------------------ */
/* config & layout                                                           */
/* ------------------------------------------------------------------------ */

static inline size_t head_dim(const orc_config* c) { return c->hidden / c->heads; } /* src/llm.zig:229-231 */
static inline size_t kv_dim(const orc_config* c) { return c->kv_heads * head_dim(c); } /* :233-235 */

int orc_config_validate(const orc_config* c) {
    /* src/llm.zig:195-216 (dense branch) */
    if (!c) return ORC_NULL_ARG;
    if (c->vocab == 0 || c->hidden == 0 || c->inter == 0 || c->layers == 0 || c->heads == 0 || c->kv_heads == 0 ||
        c->max_pos == 0)
        return ORC_INVALID_CONFIG;
    if (c->hidden % c->heads != 0) return ORC_INVALID_CONFIG;
    if (c->heads % c->kv_heads != 0) return ORC_INVALID_CONFIG;
    if (head_dim(c) % 2 != 0) return ORC_INVALID_CONFIG;
    if (c->weight_kind > 1 || c->rope_layout > 1) return ORC_INVALID_CONFIG;
    return ORC_OK;
}

size_t orc_parameter_count(const orc_config* c) {
    /* src/llm.zig:241-276, dense, no qk_norm */
    size_t h = c->hidden, kv = kv_dim(c), inter = c->inter;
    size_t bias = c->qkv_bias ? h + kv + kv : 0;
    size_t layer = h + h * h + bias + kv * h + kv * h + h * h + h + 3 * inter * h;
    size_t total = (size_t)c->vocab * h + (size_t)c->layers * layer + h;
    if (!c->tie) total += (size_t)c->vocab * h;
    return total;
}

static inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

static size_t take(size_t* cursor, size_t elem_align, size_t len) {
    /* src/llm.zig:1490-1493 addAligned / :1495-1497 alignStorageCursor */
    *cursor = align_up(*cursor, elem_align);
    size_t start = *cursor;
    *cursor += len;
    return start;
}

size_t orc_layout(const orc_config* c, orc_layer_offsets* layers, size_t* embed, size_t* final_norm,
                  size_t* lm_head) {
    /* src/llm.zig:488-522 assignSlices; elements per 64-B line (:1499-1504). */
    size_t ea = ALIGN_BYTES / (c->weight_kind == 1 ? 2 : 4);
    size_t h = c->hidden, kv = kv_dim(c), inter = c->inter;
    size_t cur = 0;
    size_t e = take(&cur, ea, (size_t)c->vocab * h);
    if (embed) *embed = e;
    for (uint32_t l = 0; l < c->layers; ++l) {
        orc_layer_offsets o;
        o.input_norm = take(&cur, ea, h);
        o.q = take(&cur, ea, h * h);
        o.q_bias = c->qkv_bias ? take(&cur, ea, h) : (size_t)-1;
        o.k = take(&cur, ea, kv * h);
        o.k_bias = c->qkv_bias ? take(&cur, ea, kv) : (size_t)-1;
        o.v = take(&cur, ea, kv * h);
        o.v_bias = c->qkv_bias ? take(&cur, ea, kv) : (size_t)-1;
        o.o = take(&cur, ea, h * h);
        o.post_norm = take(&cur, ea, h);
        o.gate = take(&cur, ea, inter * h);
        o.up = take(&cur, ea, inter * h);
        o.down = take(&cur, ea, h * inter);
        if (layers) layers[l] = o;
    }
    size_t fn = take(&cur, ea, h);
    if (final_norm) *final_norm = fn;
    size_t lm = c->tie ? (size_t)-1 : take(&cur, ea, (size_t)c->vocab * h);
    if (lm_head) *lm_head = lm;
    return cur;
}

size_t orc_storage_element_count(const orc_config* c) {
    /* src/llm.zig:814-837 */
    return orc_layout(c, NULL, NULL, NULL, NULL);
}

void orc_fill_deterministic(void* blob, size_t n, uint32_t weight_kind) {
    /* src/llm.zig:466-477: value i = ((i % 251) - 125) * 0.001 (bf16: RNE). */
    for (size_t i = 0; i < n; ++i) {
        float v = (float)((int32_t)(i % 251) - 125) * 0.001f;
        if (weight_kind == 1)
            ((uint16_t*)blob)[i] = orc_f32_to_bf16(v);
        else
            ((float*)blob)[i] = v;
    }
}

/* ------------------------------------------------------------------------ */
/* dot products: src/llm.zig:1433-1466                                       */
/* One simd_lanes-wide accumulator (acc += a*b, unfused), in-order lane      */
/* reduction (@reduce(.Add)), then an fma tail (@mulAdd).                    */
/* ------------------------------------------------------------------------ */

#define DEFINE_DOTS(L)                                                             \
    static float dot_f32_##L(const float* a, const float* b, size_t n) {           \
        float acc[L];                                                              \
        for (int l = 0; l < L; ++l) acc[l] = 0.0f;                                 \
        size_t i = 0;                                                              \
        for (; i + L <= n; i += L)                                                 \
            for (int l = 0; l < L; ++l) acc[l] = acc[l] + a[i + l] * b[i + l];     \
        float sum = 0.0f;                                                          \
        for (int l = 0; l < L; ++l) sum = sum + acc[l];                            \
        for (; i < n; ++i) sum = fmaf(a[i], b[i], sum);                            \
        return sum;                                                                \
    }                                                                              \
    static float dot_bf16_##L(const uint16_t* a, const float* b, size_t n) {       \
        float acc[L];                                                              \
        for (int l = 0; l < L; ++l) acc[l] = 0.0f;                                 \
        size_t i = 0;                                                              \
        for (; i + L <= n; i += L)                                                 \
            for (int l = 0; l < L; ++l) {                                          \
                uint32_t u = (uint32_t)a[i + l] << 16;                             \
                float w;                                                           \
                memcpy(&w, &u, 4);                                                 \
                acc[l] = acc[l] + w * b[i + l];                                    \
            }                                                                      \
        float sum = 0.0f;                                                          \
        for (int l = 0; l < L; ++l) sum = sum + acc[l];                            \
        for (; i < n; ++i) sum = fmaf(orc_bf16_to_f32(a[i]), b[i], sum);           \
        return sum;                                                                \
    }                                                                              \
    static float sum_squares_##L(const float* v, size_t n) {                       \
        float acc[L];                                                              \
        for (int l = 0; l < L; ++l) acc[l] = 0.0f;                                 \
        size_t i = 0;                                                              \
        for (; i + L <= n; i += L)                                                 \
            for (int l = 0; l < L; ++l) acc[l] = acc[l] + v[i + l] * v[i + l];     \
        float sum = 0.0f;                                                          \
        for (int l = 0; l < L; ++l) sum = sum + acc[l];                            \
        for (; i < n; ++i) sum = fmaf(v[i], v[i], sum);                            \
        return sum;                                                                \
    }

DEFINE_DOTS(1)
DEFINE_DOTS(4)
DEFINE_DOTS(8)
DEFINE_DOTS(16)

float orc_dot_f32(const float* a, const float* b, size_t n, int lanes) {
    switch (lanes) {
        case 1: return dot_f32_1(a, b, n);
        case 4: return dot_f32_4(a, b, n);
        case 8: return dot_f32_8(a, b, n);
        default: return dot_f32_16(a, b, n);
    }
}

float orc_dot_bf16(const uint16_t* a, const float* b, size_t n, int lanes) {
    switch (lanes) {
        case 1: return dot_bf16_1(a, b, n);
        case 4: return dot_bf16_4(a, b, n);
        case 8: return dot_bf16_8(a, b, n);
        default: return dot_bf16_16(a, b, n);
    }
}

static float sum_squares(const float* v, size_t n, int lanes) {
    /* src/llm.zig:1421-1431 */
    switch (lanes) {
        case 1: return sum_squares_1(v, n);
        case 4: return sum_squares_4(v, n);
        case 8: return sum_squares_8(v, n);
        default: return sum_squares_16(v, n);
    }
}

/* ------------------------------------------------------------------------ */
/* linear: src/llm.zig:1228-1285                                             */
/* ------------------------------------------------------------------------ */

static void linear_range(float* out, const void* w, uint32_t kind, size_t cols, const float* x, const void* bias,
                         size_t start, size_t end, int lanes) {
    /* src/llm.zig:1271-1275 linearRange: out[r] = dotRow(r, x) + bias[r] (or + 0.0) */
    for (size_t r = start; r < end; ++r) {
        float d = kind == 1 ? orc_dot_bf16((const uint16_t*)w + r * cols, x, cols, lanes)
                            : orc_dot_f32((const float*)w + r * cols, x, cols, lanes);
        out[r] = d + (bias ? weight_at(bias, kind, r) : 0.0f);
    }
}

void orc_linear(float* out, const void* w, uint32_t weight_kind, size_t rows, size_t cols, const float* x,
                const void* bias, int lanes) {
    linear_range(out, w, weight_kind, cols, x, bias, 0, rows, lanes);
}

void orc_matmul_blocked(float* out, const float* a, size_t m, size_t k, const float* b, size_t n, int lanes) {
    /* src/tensor.zig:683-733; matmul_col_unroll = 4 (src/tensor.zig:14). A
     * Vec of `lanes` f32 is an array here: acc[l] = acc[l] + av * b[..+l]. */
    const size_t vec = (size_t)lanes, panel = vec * 4;
    float acc[4][64];
    for (size_t row = 0; row < m; ++row) {
        const float* ar = a + row * k;
        float* orow = out + row * n;
        size_t col = 0;
        for (; col + panel <= n; col += panel) {
            for (int v = 0; v < 4; ++v)
                for (size_t l = 0; l < vec; ++l) acc[v][l] = 0.0f;
            for (size_t p = 0; p < k; ++p) {
                const float av = ar[p];
                const float* bb = b + p * n + col;
                for (int v = 0; v < 4; ++v)
                    for (size_t l = 0; l < vec; ++l) acc[v][l] = acc[v][l] + av * bb[v * vec + l];
            }
            for (int v = 0; v < 4; ++v)
                for (size_t l = 0; l < vec; ++l) orow[col + v * vec + l] = acc[v][l];
        }
        for (; col + vec <= n; col += vec) {
            for (size_t l = 0; l < vec; ++l) acc[0][l] = 0.0f;
            for (size_t p = 0; p < k; ++p) {
                const float av = ar[p];
                for (size_t l = 0; l < vec; ++l) acc[0][l] = acc[0][l] + av * b[p * n + col + l];
            }
            for (size_t l = 0; l < vec; ++l) orow[col + l] = acc[0][l];
        }
        for (; col < n; ++col) {
            float sum = 0.0f;
            for (size_t p = 0; p < k; ++p) sum = fmaf(ar[p], b[p * n + col], sum);
            orow[col] = sum;
        }
    }
}

typedef struct linear_job {
    float* out;
    const void* w;
    uint32_t kind;
    size_t cols;
    const float* x;
    const void* bias;
    size_t start, end;
    int lanes;
} linear_job;

static void* linear_worker(void* arg) {
    /* src/llm.zig:1267-1269 linearWorker */
    linear_job* j = (linear_job*)arg;
    linear_range(j->out, j->w, j->kind, j->cols, j->x, j->bias, j->start, j->end, j->lanes);
    return NULL;
}

static size_t resolve_worker_count(size_t rows, int threads, int min_rows) {
    /* src/llm.zig:1277-1285 resolveWorkerCount */
    if (rows == 0) return 1;
    long requested = threads == 0 ? sysconf(_SC_NPROCESSORS_ONLN) : threads;
    if (requested <= 1) return 1;
    size_t mr = min_rows > 1 ? (size_t)min_rows : 1;
    size_t useful = rows / mr;
    if (useful < 1) useful = 1;
    size_t w = (size_t)requested < useful ? (size_t)requested : useful;
    if (w > MAX_WORKERS) w = MAX_WORKERS;
    return w < 1 ? 1 : w;
}

int orc_linear_threaded(float* out, const void* w, uint32_t weight_kind, size_t rows, size_t cols, const float* x,
                        const void* bias, int lanes, int threads, int min_rows) {
    /* src/llm.zig:1228-1256 linearInto: spawn workers-1 threads over
     * contiguous row ranges, run the last range on the caller, join all. */
    size_t workers = resolve_worker_count(rows, threads, min_rows);
    if (workers == 1) {
        linear_range(out, w, weight_kind, cols, x, bias, 0, rows, lanes);
        return ORC_OK;
    }
    pthread_t tid[MAX_WORKERS];
    linear_job jobs[MAX_WORKERS];
    size_t per = (rows + workers - 1) / workers;
    size_t spawned = 0;
    for (; spawned + 1 < workers; ++spawned) {
        size_t s = spawned * per;
        size_t e = s + per < rows ? s + per : rows;
        jobs[spawned] = (linear_job){out, w, weight_kind, cols, x, bias, s, e, lanes};
        if (pthread_create(&tid[spawned], NULL, linear_worker, &jobs[spawned]) != 0) {
            for (size_t i = 0; i < spawned; ++i) pthread_join(tid[i], NULL);
            return ORC_THREAD_SPAWN_FAILED;
        }
    }
    size_t s = spawned * per;
    linear_range(out, w, weight_kind, cols, x, bias, s < rows ? s : rows, rows, lanes);
    for (size_t i = 0; i < spawned; ++i) pthread_join(tid[i], NULL);
    return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* elementwise ops                                                           */
/* ------------------------------------------------------------------------ */

void orc_rmsnorm(float* out, const float* x, const void* w, uint32_t kind, size_t n, float eps, int lanes) {
    /* src/llm.zig:1287-1300: ms = sumSquares/n; s = 1/sqrt(ms+eps); out = x*w*s */
    float ms = sum_squares(x, n, lanes) / (float)n;
    float scale = 1.0f / sqrtf(ms + eps);
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * weight_at(w, kind, i) * scale;
}

static void rotate_pair(float* v, size_t first, size_t second, size_t dim_index, float dim_f, float pos_f,
                        float theta, const float* inv_freq_table) {
    /* src/llm.zig:1360-1371 rotatePair */
    float inv_freq;
    if (inv_freq_table) {
        inv_freq = inv_freq_table[dim_index / 2];
    } else {
        float exponent = (float)dim_index / dim_f;
        inv_freq = 1.0f / powf(theta, exponent);
    }
    float angle = pos_f * inv_freq;
    float c = cosf(angle), s = sinf(angle);
    float x0 = v[first], x1 = v[second];
    v[first] = x0 * c - x1 * s;
    v[second] = x0 * s + x1 * c;
}

int orc_llama3_inv_freq(uint32_t head_dim, float theta, float factor, float low_freq_factor, float high_freq_factor,
                        uint32_t original_max_pos, float* out) {
    /* Llama-3 scaling (as in HF transformers' _compute_llama3_parameters, f32
     * tensors): base table 1/powf(theta, 2i/hd) as rotatePair computes it
     * (src/llm.zig:1360-1366); band edges old/low and old/high; linear blend
     * in the middle band. */
    if (head_dim == 0 || (head_dim & 1u) || !(factor > 0.0f) || !(low_freq_factor > 0.0f) ||
        !(high_freq_factor > low_freq_factor) || original_max_pos == 0)
        return ORC_INVALID_CONFIG;
    const float old_ctx = (float)original_max_pos;
    const float lo_edge = old_ctx / low_freq_factor, hi_edge = old_ctx / high_freq_factor;
    const float twopi = (float)(2.0 * 3.14159265358979323846);
    for (uint32_t i = 0; 2 * i < head_dim; ++i) {
        float base = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
        float wl = twopi / base;
        if (wl > lo_edge) {
            out[i] = base / factor;
        } else if (wl < hi_edge) {
            out[i] = base;
        } else {
            float sm = (old_ctx / wl - low_freq_factor) / (high_freq_factor - low_freq_factor);
            out[i] = (1.0f - sm) * base / factor + sm * base;
        }
    }
    return ORC_OK;
}

void orc_rope(float* values, size_t heads, size_t hd, size_t pos, float theta, uint32_t layout,
              const float* inv_freq) {
    /* src/llm.zig:1337-1358 applyRoPE. interleaved pairs (i, i+1) with
     * dim index i; split_half pairs (i, i+hd/2) with dim index 2i. */
    float pos_f = (float)pos, dim_f = (float)hd;
    for (size_t h = 0; h < heads; ++h) {
        float* hs = values + h * hd;
        if (layout == 0) {
            for (size_t i = 0; i < hd; i += 2) rotate_pair(hs, i, i + 1, i, dim_f, pos_f, theta, inv_freq);
        } else {
            size_t half = hd / 2;
            for (size_t i = 0; i < half; ++i) rotate_pair(hs, i, i + half, i * 2, dim_f, pos_f, theta, inv_freq);
        }
    }
}

void orc_softmax(float* v, size_t n) {
    /* src/llm.zig:1408-1419 softmaxInPlace */
    float mx = v[0];
    for (size_t i = 1; i < n; ++i) mx = fmaxf(mx, v[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        v[i] = expf(v[i] - mx);
        sum += v[i];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; ++i) v[i] *= inv;
}

static void add_scaled(float* out, const float* values, float scale, size_t n, int lanes) {
    /* src/llm.zig:1398-1406: vector part out + v*s (unfused), tail @mulAdd */
    size_t i = 0;
    size_t L = (size_t)(lanes < 1 ? 1 : lanes);
    for (; i + L <= n; i += L)
        for (size_t l = 0; l < L; ++l) out[i + l] = out[i + l] + values[i + l] * scale;
    for (; i < n; ++i) out[i] = fmaf(values[i], scale, out[i]);
}

void orc_attention(float* out, const float* q, const float* keys, const float* values, size_t heads,
                   size_t kv_heads, size_t hd, size_t pos, float* scores, int lanes) {
    /* src/llm.zig:1302-1335 computeAttentionInto. keys/values hold rows t of
     * width kv_heads*hd for t = 0..pos. */
    size_t group = heads / kv_heads;
    size_t kvw = kv_heads * hd;
    float inv_sqrt = 1.0f / sqrtf((float)hd);
    memset(out, 0, heads * hd * sizeof(float));
    for (size_t qh = 0; qh < heads; ++qh) {
        size_t kvh = qh / group;
        const float* qs = q + qh * hd;
        for (size_t t = 0; t <= pos; ++t) scores[t] = orc_dot_f32(qs, keys + t * kvw + kvh * hd, hd, lanes) * inv_sqrt;
        orc_softmax(scores, pos + 1);
        float* oh = out + qh * hd;
        memset(oh, 0, hd * sizeof(float));
        for (size_t t = 0; t <= pos; ++t) add_scaled(oh, values + t * kvw + kvh * hd, scores[t], hd, lanes);
    }
}

void orc_silu_mul(float* out, const float* gate, const float* up, size_t n) {
    /* src/llm.zig:1382-1387 */
    for (size_t i = 0; i < n; ++i) {
        float g = gate[i];
        out[i] = (g / (1.0f + expf(-g))) * up[i];
    }
}

void orc_add(float* out, const float* a, const float* b, size_t n) {
    /* src/llm.zig:1389-1396 */
    for (size_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

size_t orc_argmax(const float* logits, size_t n) {
    /* src/llm.zig:778-789: first index of the strict maximum */
    size_t best = 0;
    float bv = logits[0];
    for (size_t i = 1; i < n; ++i)
        if (logits[i] > bv) {
            bv = logits[i];
            best = i;
        }
    return best;
}

/* ------------------------------------------------------------------------ */
/* runner: src/llm.zig:539-776                                               */
/* ------------------------------------------------------------------------ */

struct orc_runner {
    orc_config c;
    const void* blob;
    size_t blob_elems;
    uint32_t max_seq;
    int threads, lanes;
    orc_layer_offsets* lo;
    size_t embed, final_norm, lm_head;
    float* keys;   /* [layer][max_seq][kv] (src/llm.zig:603-605) */
    float* values;
    float *x, *residual, *norm, *q, *k, *v, *attn, *proj, *gate, *up, *ff, *scores, *logits;
    float* inv_freq; /* optional table override */
};

static void* aligned_floats(size_t n) {
    void* p = NULL;
    if (posix_memalign(&p, ALIGN_BYTES, (n ? n : 1) * sizeof(float)) != 0) return NULL;
    return p;
}

void orc_runner_destroy(orc_runner* r) {
    if (!r) return;
    free(r->lo);
    free(r->keys);
    free(r->values);
    float* bufs[] = {r->x, r->residual, r->norm, r->q, r->k, r->v, r->attn, r->proj,
                     r->gate, r->up, r->ff, r->scores, r->logits, r->inv_freq};
    for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); ++i) free(bufs[i]);
    free(r);
}

int orc_runner_create(const orc_config* c, const void* blob, size_t blob_elems, uint32_t max_seq_len, int threads,
                      int lanes, orc_runner** out) {
    if (!c || !blob || !out) return ORC_NULL_ARG;
    *out = NULL;
    int rc = orc_config_validate(c);
    if (rc) return rc;
    /* src/llm.zig:545-548 KVCache.init */
    if (max_seq_len == 0 || max_seq_len > c->max_pos) return ORC_INVALID_CONFIG;
    orc_runner* r = (orc_runner*)calloc(1, sizeof(orc_runner));
    if (!r) return ORC_OUT_OF_MEMORY;
    r->c = *c;
    r->blob = blob;
    r->blob_elems = blob_elems;
    r->max_seq = max_seq_len;
    r->threads = threads;
    r->lanes = lanes;
    r->lo = (orc_layer_offsets*)calloc(c->layers, sizeof(orc_layer_offsets));
    if (!r->lo) {
        orc_runner_destroy(r);
        return ORC_OUT_OF_MEMORY;
    }
    size_t need = orc_layout(c, r->lo, &r->embed, &r->final_norm, &r->lm_head);
    if (blob_elems < need) { /* the blob must cover every slice */
        orc_runner_destroy(r);
        return ORC_INVALID_WEIGHT;
    }
    size_t h = c->hidden, kv = kv_dim(c), inter = c->inter;
    size_t kvlen = (size_t)c->layers * max_seq_len * kv;
    r->keys = (float*)aligned_floats(kvlen);
    r->values = (float*)aligned_floats(kvlen);
    r->x = aligned_floats(h);
    r->residual = aligned_floats(h);
    r->norm = aligned_floats(h);
    r->q = aligned_floats(h);
    r->k = aligned_floats(kv);
    r->v = aligned_floats(kv);
    r->attn = aligned_floats(h);
    r->proj = aligned_floats(h);
    r->gate = aligned_floats(inter);
    r->up = aligned_floats(inter);
    r->ff = aligned_floats(inter);
    r->scores = aligned_floats(max_seq_len);
    r->logits = aligned_floats(c->vocab);
    if (!r->keys || !r->values || !r->x || !r->residual || !r->norm || !r->q || !r->k || !r->v || !r->attn ||
        !r->proj || !r->gate || !r->up || !r->ff || !r->scores || !r->logits) {
        orc_runner_destroy(r);
        return ORC_OUT_OF_MEMORY;
    }
    orc_kv_clear(r);
    *out = r;
    return ORC_OK;
}

void orc_kv_clear(orc_runner* r) {
    /* src/llm.zig:576-579 KVCache.clear */
    size_t kvlen = (size_t)r->c.layers * r->max_seq * kv_dim(&r->c);
    memset(r->keys, 0, kvlen * sizeof(float));
    memset(r->values, 0, kvlen * sizeof(float));
}

int orc_set_rope_table(orc_runner* r, const float* inv_freq, uint32_t n) {
    if (!r) return ORC_NULL_ARG;
    free(r->inv_freq);
    r->inv_freq = NULL;
    if (!inv_freq) return ORC_OK;
    if (n != head_dim(&r->c) / 2) return ORC_INVALID_CONFIG;
    r->inv_freq = (float*)malloc(n * sizeof(float));
    if (!r->inv_freq) return ORC_OUT_OF_MEMORY;
    memcpy(r->inv_freq, inv_freq, n * sizeof(float));
    return ORC_OK;
}

static const void* wptr(const orc_runner* r, size_t off) {
    return r->c.weight_kind == 1 ? (const void*)((const uint16_t*)r->blob + off)
                                 : (const void*)((const float*)r->blob + off);
}

static int linear(orc_runner* r, float* out, size_t w_off, size_t rows, size_t cols, const float* x,
                  size_t bias_off) {
    const void* bias = bias_off == (size_t)-1 ? NULL : wptr(r, bias_off);
    return orc_linear_threaded(out, wptr(r, w_off), r->c.weight_kind, rows, cols, x, bias, r->lanes, r->threads, 64);
}

static int forward_layer(orc_runner* r, uint32_t l, uint32_t pos) {
    /* src/llm.zig:732-766 forwardLayer */
    const orc_config* c = &r->c;
    const orc_layer_offsets* o = &r->lo[l];
    size_t h = c->hidden, kv = kv_dim(c), hd = head_dim(c), inter = c->inter;
    int rc;
    memcpy(r->residual, r->x, h * sizeof(float));
    orc_rmsnorm(r->norm, r->x, wptr(r, o->input_norm), c->weight_kind, h, c->rms_eps, r->lanes);
    if ((rc = linear(r, r->q, o->q, h, h, r->norm, o->q_bias))) return rc;
    if ((rc = linear(r, r->k, o->k, kv, h, r->norm, o->k_bias))) return rc;
    if ((rc = linear(r, r->v, o->v, kv, h, r->norm, o->v_bias))) return rc;
    orc_rope(r->q, c->heads, hd, pos, c->rope_theta, c->rope_layout, r->inv_freq);
    orc_rope(r->k, c->kv_heads, hd, pos, c->rope_theta, c->rope_layout, r->inv_freq);
    float* kl = r->keys + (size_t)l * r->max_seq * kv;
    float* vl = r->values + (size_t)l * r->max_seq * kv;
    memcpy(kl + (size_t)pos * kv, r->k, kv * sizeof(float));
    memcpy(vl + (size_t)pos * kv, r->v, kv * sizeof(float));
    orc_attention(r->attn, r->q, kl, vl, c->heads, c->kv_heads, hd, pos, r->scores, r->lanes);
    if ((rc = linear(r, r->proj, o->o, h, h, r->attn, (size_t)-1))) return rc; /* no o_bias in the blob */
    orc_add(r->x, r->residual, r->proj, h);
    memcpy(r->residual, r->x, h * sizeof(float));
    orc_rmsnorm(r->norm, r->x, wptr(r, o->post_norm), c->weight_kind, h, c->rms_eps, r->lanes);
    if ((rc = linear(r, r->gate, o->gate, inter, h, r->norm, (size_t)-1))) return rc;
    if ((rc = linear(r, r->up, o->up, inter, h, r->norm, (size_t)-1))) return rc;
    orc_silu_mul(r->ff, r->gate, r->up, inter);
    if ((rc = linear(r, r->proj, o->down, h, inter, r->ff, (size_t)-1))) return rc;
    orc_add(r->x, r->residual, r->proj, h);
    return ORC_OK;
}

static int forward_current(orc_runner* r, uint32_t pos, float* logits_out, float* hidden_out) {
    /* src/llm.zig:720-730 forwardCurrentEmbedding */
    const orc_config* c = &r->c;
    int rc;
    for (uint32_t l = 0; l < c->layers; ++l) {
        if ((rc = forward_layer(r, l, pos))) return rc;
        if (hidden_out) memcpy(hidden_out + (size_t)l * c->hidden, r->x, c->hidden * sizeof(float));
    }
    orc_rmsnorm(r->norm, r->x, wptr(r, r->final_norm), c->weight_kind, c->hidden, c->rms_eps, r->lanes);
    size_t head = c->tie ? r->embed : r->lm_head; /* src/llm.zig:410-412 logitsMatrix */
    if ((rc = linear(r, r->logits, head, c->vocab, c->hidden, r->norm, (size_t)-1))) return rc;
    if (logits_out) memcpy(logits_out, r->logits, (size_t)c->vocab * sizeof(float));
    return ORC_OK;
}

int orc_forward_token(orc_runner* r, uint32_t token, uint32_t pos, float* logits_out, float* hidden_out) {
    /* src/llm.zig:702-709 forwardToken + copyEmbeddingToken (:1373-1380) */
    if (!r) return ORC_NULL_ARG;
    if (token >= r->c.vocab) return ORC_INVALID_TOKEN;
    if (pos >= r->max_seq) return ORC_CONTEXT_FULL;
    size_t h = r->c.hidden;
    size_t start = r->embed + (size_t)token * h;
    for (size_t i = 0; i < h; ++i) r->x[i] = weight_at(r->blob, r->c.weight_kind, start + i);
    return forward_current(r, pos, logits_out, hidden_out);
}

int orc_forward_embedding(orc_runner* r, const float* embedding, uint32_t pos, float* logits_out,
                          float* hidden_out) {
    /* src/llm.zig:711-718 forwardEmbedding */
    if (!r || !embedding) return ORC_NULL_ARG;
    if (pos >= r->max_seq) return ORC_CONTEXT_FULL;
    memcpy(r->x, embedding, r->c.hidden * sizeof(float));
    return forward_current(r, pos, logits_out, hidden_out);
}

/* ------------------------------------------------------------------------ */
/* prompt pass: the prompt loop of src/generator.zig:243-251 (one           */
/* forwardToken per prompt token) with its loops interchanged so that a     */
/* weight row is read once per block of tokens instead of once per token.   */
/* Every value is computed by the same functions in the same order as       */
/* orc_forward_token computes it for that token, so the KV rows and the     */
/* last token's logits are bit-identical to the token loop's (only the      */
/* work order across tokens and rows differs). A token's attention reads    */
/* rows 0..its pos, all written before any attention of the layer runs.     */
/* ------------------------------------------------------------------------ */

#define PF_TOKEN_BLOCK 16

typedef struct pf_linear_job {
    const orc_runner* r;
    float* out; /* [n][rows] */
    size_t w_off, bias_off, rows, cols;
    const float* x; /* [n][cols] */
    size_t n;
    size_t row0, row1;
} pf_linear_job;

static void* pf_linear_worker(void* arg) {
    pf_linear_job* j = (pf_linear_job*)arg;
    const orc_runner* r = j->r;
    const uint32_t kind = r->c.weight_kind;
    const void* w = kind == 1 ? (const void*)((const uint16_t*)r->blob + j->w_off)
                              : (const void*)((const float*)r->blob + j->w_off);
    const void* bias = j->bias_off == (size_t)-1 ? NULL
                       : (kind == 1 ? (const void*)((const uint16_t*)r->blob + j->bias_off)
                                    : (const void*)((const float*)r->blob + j->bias_off));
    for (size_t t0 = 0; t0 < j->n; t0 += PF_TOKEN_BLOCK) {
        size_t t1 = t0 + PF_TOKEN_BLOCK < j->n ? t0 + PF_TOKEN_BLOCK : j->n;
        for (size_t row = j->row0; row < j->row1; ++row)
            for (size_t t = t0; t < t1; ++t) /* linear_range's expression for one row */
                j->out[t * j->rows + row] =
                    (kind == 1 ? orc_dot_bf16((const uint16_t*)w + row * j->cols, j->x + t * j->cols, j->cols, r->lanes)
                               : orc_dot_f32((const float*)w + row * j->cols, j->x + t * j->cols, j->cols, r->lanes)) +
                    (bias ? weight_at(bias, kind, row) : 0.0f);
    }
    return NULL;
}

static int pf_threads(const orc_runner* r) {
    long t = r->threads == 0 ? sysconf(_SC_NPROCESSORS_ONLN) : r->threads;
    return t < 1 ? 1 : (t > MAX_WORKERS ? MAX_WORKERS : (int)t);
}

static int pf_linear(const orc_runner* r, float* out, size_t w_off, size_t rows, size_t cols, const float* x, size_t n,
                     size_t bias_off) {
    int nt = pf_threads(r);
    pthread_t tid[MAX_WORKERS];
    pf_linear_job jobs[MAX_WORKERS];
    size_t per = (rows + (size_t)nt - 1) / (size_t)nt;
    int spawned = 0;
    for (int i = 0; i < nt; ++i) {
        size_t a = (size_t)i * per, b = a + per < rows ? a + per : rows;
        jobs[i] = (pf_linear_job){r, out, w_off, bias_off, rows, cols, x, n, a < rows ? a : rows, b};
    }
    for (; spawned + 1 < nt; ++spawned)
        if (pthread_create(&tid[spawned], NULL, pf_linear_worker, &jobs[spawned]) != 0) {
            for (int i = 0; i < spawned; ++i) pthread_join(tid[i], NULL);
            return ORC_THREAD_SPAWN_FAILED;
        }
    pf_linear_worker(&jobs[nt - 1]);
    for (int i = 0; i < spawned; ++i) pthread_join(tid[i], NULL);
    return ORC_OK;
}

typedef struct pf_attn_job {
    const orc_runner* r;
    float* attn;     /* [n][h] */
    const float* q;  /* [n][h], rotated */
    const float* kl; /* this layer's cache */
    const float* vl;
    size_t n, start, first, stride;
    float* scores;   /* max_seq floats of this worker */
} pf_attn_job;

static void* pf_attn_worker(void* arg) {
    pf_attn_job* j = (pf_attn_job*)arg;
    const orc_config* c = &j->r->c;
    size_t h = c->hidden, hd = head_dim(c);
    for (size_t t = j->first; t < j->n; t += j->stride)
        orc_attention(j->attn + t * h, j->q + t * h, j->kl, j->vl, c->heads, c->kv_heads, hd, j->start + t, j->scores,
                      j->r->lanes);
    return NULL;
}

int orc_prefill(orc_runner* r, const uint32_t* tokens, uint32_t n, uint32_t start_pos, float* logits_out) {
    if (!r || !tokens) return ORC_NULL_ARG;
    if (n == 0) return ORC_EMPTY_PROMPT;
    if ((uint64_t)start_pos + n > r->max_seq) return ORC_CONTEXT_FULL;
    const orc_config* c = &r->c;
    for (uint32_t i = 0; i < n; ++i)
        if (tokens[i] >= c->vocab) return ORC_INVALID_TOKEN;
    size_t h = c->hidden, kv = kv_dim(c), hd = head_dim(c), inter = c->inter;
    int nt = pf_threads(r);
    float* x = aligned_floats((size_t)n * h);
    float* res = aligned_floats((size_t)n * h);
    float* nrm = aligned_floats((size_t)n * h);
    float* q = aligned_floats((size_t)n * h);
    float* k = aligned_floats((size_t)n * kv);
    float* v = aligned_floats((size_t)n * kv);
    float* attn = aligned_floats((size_t)n * h);
    float* proj = aligned_floats((size_t)n * h);
    float* gate = aligned_floats((size_t)n * inter);
    float* up = aligned_floats((size_t)n * inter);
    float* scores = aligned_floats((size_t)nt * r->max_seq);
    float* bufs[] = {x, res, nrm, q, k, v, attn, proj, gate, up, scores};
    int rc = ORC_OK;
    for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); ++i)
        if (!bufs[i]) rc = ORC_OUT_OF_MEMORY;
    for (uint32_t t = 0; rc == ORC_OK && t < n; ++t) { /* copyEmbeddingToken (src/llm.zig:1373-1380) */
        size_t start = r->embed + (size_t)tokens[t] * h;
        for (size_t i = 0; i < h; ++i) x[t * h + i] = weight_at(r->blob, c->weight_kind, start + i);
    }
    for (uint32_t l = 0; rc == ORC_OK && l < c->layers; ++l) { /* forwardLayer (src/llm.zig:732-766) per token */
        const orc_layer_offsets* o = &r->lo[l];
        memcpy(res, x, (size_t)n * h * sizeof(float));
        for (uint32_t t = 0; t < n; ++t)
            orc_rmsnorm(nrm + t * h, x + t * h, wptr(r, o->input_norm), c->weight_kind, h, c->rms_eps, r->lanes);
        if ((rc = pf_linear(r, q, o->q, h, h, nrm, n, o->q_bias))) break;
        if ((rc = pf_linear(r, k, o->k, kv, h, nrm, n, o->k_bias))) break;
        if ((rc = pf_linear(r, v, o->v, kv, h, nrm, n, o->v_bias))) break;
        float* kl = r->keys + (size_t)l * r->max_seq * kv;
        float* vl = r->values + (size_t)l * r->max_seq * kv;
        for (uint32_t t = 0; t < n; ++t) {
            orc_rope(q + t * h, c->heads, hd, start_pos + t, c->rope_theta, c->rope_layout, r->inv_freq);
            orc_rope(k + t * kv, c->kv_heads, hd, start_pos + t, c->rope_theta, c->rope_layout, r->inv_freq);
            memcpy(kl + (size_t)(start_pos + t) * kv, k + t * kv, kv * sizeof(float));
            memcpy(vl + (size_t)(start_pos + t) * kv, v + t * kv, kv * sizeof(float));
        }
        {
            pthread_t tid[MAX_WORKERS];
            pf_attn_job jobs[MAX_WORKERS];
            int spawned = 0;
            for (int i = 0; i < nt; ++i)
                jobs[i] = (pf_attn_job){r, attn, q, kl, vl, n, start_pos, (size_t)i, (size_t)nt,
                                        scores + (size_t)i * r->max_seq};
            for (; spawned + 1 < nt; ++spawned)
                if (pthread_create(&tid[spawned], NULL, pf_attn_worker, &jobs[spawned]) != 0) {
                    rc = ORC_THREAD_SPAWN_FAILED;
                    break;
                }
            if (rc == ORC_OK) pf_attn_worker(&jobs[nt - 1]);
            for (int i = 0; i < spawned; ++i) pthread_join(tid[i], NULL);
            if (rc) break;
        }
        if ((rc = pf_linear(r, proj, o->o, h, h, attn, n, (size_t)-1))) break;
        for (uint32_t t = 0; t < n; ++t) orc_add(x + t * h, res + t * h, proj + t * h, h);
        memcpy(res, x, (size_t)n * h * sizeof(float));
        for (uint32_t t = 0; t < n; ++t)
            orc_rmsnorm(nrm + t * h, x + t * h, wptr(r, o->post_norm), c->weight_kind, h, c->rms_eps, r->lanes);
        if ((rc = pf_linear(r, gate, o->gate, inter, h, nrm, n, (size_t)-1))) break;
        if ((rc = pf_linear(r, up, o->up, inter, h, nrm, n, (size_t)-1))) break;
        for (uint32_t t = 0; t < n; ++t) orc_silu_mul(gate + t * inter, gate + t * inter, up + t * inter, inter);
        if ((rc = pf_linear(r, proj, o->down, h, inter, gate, n, (size_t)-1))) break;
        for (uint32_t t = 0; t < n; ++t) orc_add(x + t * h, res + t * h, proj + t * h, h);
    }
    if (rc == ORC_OK) { /* the last token's forwardCurrentEmbedding tail (src/llm.zig:727-728) */
        memcpy(r->x, x + (size_t)(n - 1) * h, h * sizeof(float));
        orc_rmsnorm(r->norm, r->x, wptr(r, r->final_norm), c->weight_kind, h, c->rms_eps, r->lanes);
        size_t head = c->tie ? r->embed : r->lm_head;
        rc = linear(r, r->logits, head, c->vocab, h, r->norm, (size_t)-1);
        if (rc == ORC_OK && logits_out) memcpy(logits_out, r->logits, (size_t)c->vocab * sizeof(float));
    }
    for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); ++i) free(bufs[i]);
    return rc;
}

int orc_kv_read(const orc_runner* r, uint32_t layer, uint32_t pos, float* k_out, float* v_out) {
    if (!r) return ORC_NULL_ARG;
    if (layer >= r->c.layers || pos >= r->max_seq) return ORC_INVALID_CONFIG;
    size_t kv = kv_dim(&r->c);
    size_t off = ((size_t)layer * r->max_seq + pos) * kv;
    if (k_out) memcpy(k_out, r->keys + off, kv * sizeof(float));
    if (v_out) memcpy(v_out, r->values + off, kv * sizeof(float));
    return ORC_OK;
}

/* Overwrite n consecutive cache rows pos.. of one layer (k, v: n * kv floats
 * each), so that a test can continue from another implementation's cache. */
int orc_kv_write(orc_runner* r, uint32_t layer, uint32_t pos, uint32_t n, const float* k, const float* v) {
    if (!r || !k || !v) return ORC_NULL_ARG;
    if (layer >= r->c.layers || pos > r->max_seq || n > r->max_seq - pos) return ORC_INVALID_CONFIG;
    size_t kv = kv_dim(&r->c);
    size_t off = ((size_t)layer * r->max_seq + pos) * kv;
    memcpy(r->keys + off, k, (size_t)n * kv * sizeof(float));
    memcpy(r->values + off, v, (size_t)n * kv * sizeof(float));
    return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* generator: src/generator.zig:142-175, 221-293                             */
/* ------------------------------------------------------------------------ */

static int64_t now_ns(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (int64_t)ts.tv_sec * 1000000000LL + ts.tv_nsec;
}

int orc_generate_greedy(orc_runner* r, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new, int64_t eos,
                        uint32_t* out_tokens, uint32_t* n_out, orc_stats* stats) {
    /* generateGreedyMeasuredInternal with a greedy sampler: prefill is one
     * forwardToken per prompt token; each decode step takes argmax, emits it,
     * stops on EOS, else forwards it (the last token is forwarded too). */
    if (!r || !out_tokens || !n_out) return ORC_NULL_ARG;
    if (n_prompt == 0 || !prompt) return ORC_EMPTY_PROMPT;
    int rc;
    int64_t t0 = now_ns();
    uint32_t pos = 0;
    for (uint32_t i = 0; i < n_prompt; ++i) {
        if ((rc = orc_forward_token(r, prompt[i], pos, NULL, NULL))) return rc;
        pos++;
    }
    int64_t t1 = now_ns();
    uint32_t produced = 0;
    while (produced < max_new) {
        uint32_t next = (uint32_t)orc_argmax(r->logits, r->c.vocab);
        out_tokens[produced++] = next;
        if (eos >= 0 && next == (uint32_t)eos) break;
        if ((rc = orc_forward_token(r, next, pos, NULL, NULL))) return rc;
        pos++;
    }
    int64_t t2 = now_ns();
    *n_out = produced;
    if (stats) {
        stats->prompt_tokens = n_prompt;
        stats->generated_tokens = produced;
        stats->prefill_ns = t1 - t0;
        stats->decode_ns = t2 - t1;
        stats->total_ns = t2 - t0;
    }
    return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* sampler pieces: src/generator.zig:376-379 adjustedLogit, :362-374         */
/* ------------------------------------------------------------------------ */

float orc_adjusted_logit(float logit, uint16_t repeat_count, float repeat_penalty) {
    if (repeat_count == 0 || repeat_penalty <= 1.0f) return logit;
    return logit < 0.0f ? logit * repeat_penalty : logit / repeat_penalty;
}

uint32_t orc_greedy_with_penalties(const float* logits, const uint16_t* counts, size_t n, float repeat_penalty) {
    uint32_t best = 0;
    float bl = orc_adjusted_logit(logits[0], counts[0], repeat_penalty);
    for (size_t i = 1; i < n; ++i) {
        float s = orc_adjusted_logit(logits[i], counts[i], repeat_penalty);
        if (s > bl) {
            bl = s;
            best = (uint32_t)i;
        }
    }
    return best;
}
