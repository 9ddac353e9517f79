/*
 * vvli_oracle_moe.c -- CPU restatement of a mixture-of-experts decoder step
 * (OLMoE form). TEST INFRASTRUCTURE ONLY: reference results for the GPU
 * MoE runner; nothing in the product path links or calls it.
 *
 * The reference has no MoE forward pass: Config carries num_experts /
 * num_experts_per_tok / qk_norm (src/llm.zig:86-88,119-133) and the runner
 * rejects such configs (src/llm.zig:218-223,426). The semantics here are
 * those of HF transformers' OLMoE (transformers/models/olmoe/modeling_olmoe.py
 * in transformers 5.15):
 *   q = q_norm(q_proj(x)), k = k_norm(k_proj(x)): RMSNorm over the full q
 *     (width hidden) and the full k (width kv), weight * (x * 1/sqrt(mean+eps));
 *   split-half RoPE, causal attention as the dense path;
 *   router: logits = W_r . norm(x); softmax in f32; top-k by probability
 *     (ties: lower expert index first); no renormalisation of the k weights;
 *   experts: act = silu(gate) * up from the fused [2I][H] gate|up matrix,
 *     out_e = W_down,e . act; moe = sum over the selected experts in
 *     ascending expert index of (out_e * weight_e); x = residual + moe.
 * The ops (linear, attention, RoPE, SiLU*up, add) are the dense oracle's
 * restatements of the reference (vvli_oracle.c); only the composition above is
 * new. Pinned by tests/test_moe.py against HF OlmoeForCausalLM golden
 * fixtures (tests/golden/make_moe_golden.py) and by closed-form routing cases.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "vvli_oracle.h"

#define MOE_ALIGN_BYTES 64

static inline size_t m_head_dim(const orc_config* c) { return c->hidden / c->heads; }
static inline size_t m_kv_dim(const orc_config* c) { return c->kv_heads * m_head_dim(c); }

static size_t m_take(size_t* cursor, size_t elem_align, size_t len) {
    *cursor = (*cursor + elem_align - 1) / elem_align * elem_align;
    size_t at = *cursor;
    *cursor += len;
    return at;
}

static inline float m_weight_at(const void* w, uint32_t kind, size_t i) {
    if (kind == 1) return orc_bf16_to_f32(((const uint16_t*)w)[i]);
    return ((const float*)w)[i];
}

size_t orc_moe_layout(const orc_moe_config* mc, orc_moe_layer_offsets* layers, size_t* embed, size_t* final_norm,
                      size_t* lm_head) {
    const orc_config* c = &mc->base;
    const size_t none = (size_t)-1;
    const size_t ea = MOE_ALIGN_BYTES / (c->weight_kind == 1 ? 2 : 4);
    const size_t h = c->hidden, kv = m_kv_dim(c), inter = c->inter, e = mc->experts;
    size_t cur = 0;
    *embed = m_take(&cur, ea, (size_t)c->vocab * h);
    for (uint32_t l = 0; l < c->layers; ++l) {
        orc_moe_layer_offsets* o = &layers[l];
        o->input_norm = m_take(&cur, ea, h);
        o->q = m_take(&cur, ea, h * h);
        o->q_bias = c->qkv_bias ? m_take(&cur, ea, h) : none;
        o->k = m_take(&cur, ea, kv * h);
        o->k_bias = c->qkv_bias ? m_take(&cur, ea, kv) : none;
        o->v = m_take(&cur, ea, kv * h);
        o->v_bias = c->qkv_bias ? m_take(&cur, ea, kv) : none;
        o->q_norm = mc->qk_norm ? m_take(&cur, ea, h) : none;
        o->k_norm = mc->qk_norm ? m_take(&cur, ea, kv) : none;
        o->o = m_take(&cur, ea, h * h);
        o->post_norm = m_take(&cur, ea, h);
        o->router = m_take(&cur, ea, e * h);
        o->gate_up = m_take(&cur, ea, e * 2 * inter * h);
        o->down = m_take(&cur, ea, e * h * inter);
    }
    *final_norm = m_take(&cur, ea, h);
    *lm_head = c->tie ? none : m_take(&cur, ea, (size_t)c->vocab * h);
    return cur;
}

void orc_moe_rmsnorm(float* out, const float* x, const void* w, uint32_t kind, size_t n, float eps) {
    /* OlmoeRMSNorm: variance = mean(x^2) in f32; weight * (x * rsqrt(variance + eps)) */
    float ss = 0.f;
    for (size_t i = 0; i < n; ++i) ss += x[i] * x[i];
    const float s = 1.0f / sqrtf(ss / (float)n + eps);
    for (size_t i = 0; i < n; ++i) out[i] = m_weight_at(w, kind, i) * (x[i] * s);
}

void orc_moe_route(const float* logits, size_t n, size_t top_k, uint32_t* idx, float* weights) {
    /* OlmoeTopKRouter: softmax(logits, f32) -> topk; no renormalisation. */
    float mx = -INFINITY;
    for (size_t i = 0; i < n; ++i) mx = logits[i] > mx ? logits[i] : mx;
    float* p = (float*)malloc(n * sizeof(float));
    unsigned char* used = (unsigned char*)calloc(n, 1);
    if (!p || !used) {
        free(p);
        free(used);
        for (size_t k = 0; k < top_k; ++k) idx[k] = 0, weights[k] = 0.f;
        return;
    }
    float sum = 0.f;
    for (size_t i = 0; i < n; ++i) {
        p[i] = expf(logits[i] - mx);
        sum += p[i];
    }
    for (size_t i = 0; i < n; ++i) p[i] = p[i] / sum;
    for (size_t k = 0; k < top_k; ++k) {
        size_t best = n;
        for (size_t i = 0; i < n; ++i) {
            if (used[i]) continue;
            if (best == n || p[i] > p[best]) best = i; /* strict >: the lower index wins a tie */
        }
        used[best] = 1;
        idx[k] = (uint32_t)best;
        weights[k] = p[best];
    }
    free(p);
    free(used);
}

struct orc_moe_runner {
    orc_moe_config c;
    const void* blob;
    uint32_t max_seq;
    int threads, lanes;
    orc_moe_layer_offsets* lo;
    size_t embed, final_norm, lm_head;
    float *keys, *values;
    float *x, *residual, *norm, *q, *k, *v, *attn, *proj, *router, *gu, *act, *eout, *moe, *scores, *logits;
    uint32_t* idx;
    float* rw;
};

static float* m_floats(size_t n) { return (float*)calloc(n ? n : 1, sizeof(float)); }

void orc_moe_runner_destroy(orc_moe_runner* r) {
    if (!r) return;
    float* bufs[] = {r->keys, r->values, r->x, r->residual, r->norm, r->q, r->k, r->v, r->attn, r->proj,
                     r->router, r->gu, r->act, r->eout, r->moe, r->scores, r->logits, r->rw};
    for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); ++i) free(bufs[i]);
    free(r->idx);
    free(r->lo);
    free(r);
}

int orc_moe_runner_create(const orc_moe_config* mc, const void* blob, size_t blob_elems, uint32_t max_seq_len,
                          int threads, int lanes, orc_moe_runner** out) {
    if (!mc || !blob || !out) return ORC_NULL_ARG;
    *out = NULL;
    const orc_config* c = &mc->base;
    int rc = orc_config_validate(c);
    if (rc) return rc;
    if (mc->experts == 0 || mc->top_k == 0 || mc->top_k > mc->experts) return ORC_INVALID_CONFIG;
    if (max_seq_len == 0 || max_seq_len > c->max_pos) return ORC_INVALID_CONFIG;
    orc_moe_runner* r = (orc_moe_runner*)calloc(1, sizeof(orc_moe_runner));
    if (!r) return ORC_OUT_OF_MEMORY;
    r->c = *mc;
    r->blob = blob;
    r->max_seq = max_seq_len;
    r->threads = threads;
    r->lanes = lanes;
    r->lo = (orc_moe_layer_offsets*)calloc(c->layers, sizeof(orc_moe_layer_offsets));
    if (!r->lo) {
        orc_moe_runner_destroy(r);
        return ORC_OUT_OF_MEMORY;
    }
    if (orc_moe_layout(mc, r->lo, &r->embed, &r->final_norm, &r->lm_head) > blob_elems) {
        orc_moe_runner_destroy(r);
        return ORC_INVALID_WEIGHT;
    }
    const size_t h = c->hidden, kv = m_kv_dim(c), inter = c->inter;
    const size_t kvlen = (size_t)c->layers * max_seq_len * kv;
    r->keys = m_floats(kvlen);
    r->values = m_floats(kvlen);
    r->x = m_floats(h);
    r->residual = m_floats(h);
    r->norm = m_floats(h);
    r->q = m_floats(h);
    r->k = m_floats(kv);
    r->v = m_floats(kv);
    r->attn = m_floats(h);
    r->proj = m_floats(h);
    r->router = m_floats(mc->experts);
    r->gu = m_floats(2 * inter);
    r->act = m_floats(inter);
    r->eout = m_floats(h);
    r->moe = m_floats(h);
    r->scores = m_floats(max_seq_len);
    r->logits = m_floats(c->vocab);
    r->rw = m_floats(mc->top_k);
    r->idx = (uint32_t*)calloc(mc->top_k, sizeof(uint32_t));
    if (!r->keys || !r->values || !r->x || !r->residual || !r->norm || !r->q || !r->k || !r->v || !r->attn ||
        !r->proj || !r->router || !r->gu || !r->act || !r->eout || !r->moe || !r->scores || !r->logits || !r->rw ||
        !r->idx) {
        orc_moe_runner_destroy(r);
        return ORC_OUT_OF_MEMORY;
    }
    *out = r;
    return ORC_OK;
}

static const void* m_w(const orc_moe_runner* r, size_t off) {
    return r->c.base.weight_kind == 1 ? (const void*)((const uint16_t*)r->blob + off)
                                      : (const void*)((const float*)r->blob + off);
}

static int m_linear(orc_moe_runner* r, float* out, size_t w_off, size_t rows, size_t cols, const float* x,
                    size_t bias_off) {
    const void* bias = bias_off == (size_t)-1 ? NULL : m_w(r, bias_off);
    return orc_linear_threaded(out, m_w(r, w_off), r->c.base.weight_kind, rows, cols, x, bias, r->lanes,
                               r->threads, 64);
}

static int m_forward_layer(orc_moe_runner* r, uint32_t l, uint32_t pos) {
    const orc_config* c = &r->c.base;
    const orc_moe_layer_offsets* o = &r->lo[l];
    const uint32_t kind = c->weight_kind;
    const size_t h = c->hidden, kv = m_kv_dim(c), hd = m_head_dim(c), inter = c->inter;
    int rc;
    memcpy(r->residual, r->x, h * sizeof(float));
    orc_moe_rmsnorm(r->norm, r->x, m_w(r, o->input_norm), kind, h, c->rms_eps);
    if ((rc = m_linear(r, r->q, o->q, h, h, r->norm, o->q_bias))) return rc;
    if ((rc = m_linear(r, r->k, o->k, kv, h, r->norm, o->k_bias))) return rc;
    if ((rc = m_linear(r, r->v, o->v, kv, h, r->norm, o->v_bias))) return rc;
    if (r->c.qk_norm) {
        orc_moe_rmsnorm(r->q, r->q, m_w(r, o->q_norm), kind, h, c->rms_eps);
        orc_moe_rmsnorm(r->k, r->k, m_w(r, o->k_norm), kind, kv, c->rms_eps);
    }
    orc_rope(r->q, c->heads, hd, pos, c->rope_theta, c->rope_layout, NULL);
    orc_rope(r->k, c->kv_heads, hd, pos, c->rope_theta, c->rope_layout, NULL);
    float* kl = r->keys + (size_t)l * r->max_seq * kv;
    float* vl = r->values + (size_t)l * r->max_seq * kv;
    memcpy(kl + (size_t)pos * kv, r->k, kv * sizeof(float));
    memcpy(vl + (size_t)pos * kv, r->v, kv * sizeof(float));
    orc_attention(r->attn, r->q, kl, vl, c->heads, c->kv_heads, hd, pos, r->scores, r->lanes);
    if ((rc = m_linear(r, r->proj, o->o, h, h, r->attn, (size_t)-1))) return rc;
    orc_add(r->x, r->residual, r->proj, h);
    memcpy(r->residual, r->x, h * sizeof(float));
    orc_moe_rmsnorm(r->norm, r->x, m_w(r, o->post_norm), kind, h, c->rms_eps);
    if ((rc = m_linear(r, r->router, o->router, r->c.experts, h, r->norm, (size_t)-1))) return rc;
    orc_moe_route(r->router, r->c.experts, r->c.top_k, r->idx, r->rw);
    if ((rc = orc_moe_experts(r->moe, r->blob, kind, o->gate_up, o->down, r->norm, h, inter, r->c.experts,
                              r->c.top_k, r->idx, r->rw, r->lanes, r->threads, 0)))
        return rc;
    orc_add(r->x, r->residual, r->moe, h);
    return ORC_OK;
}

/* W rows [rows][cols] of the blob (f32 or bf16) as the f32 [cols][rows]
 * matrix B of tensor.zig's out = x . B. */
static float* m_transposed_f32(const void* blob, uint32_t kind, size_t off, size_t rows, size_t cols) {
    float* t = (float*)malloc(rows * cols * sizeof(float));
    if (!t) return NULL;
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) t[c * rows + r] = m_weight_at(blob, kind, off + r * cols + c);
    return t;
}

int orc_moe_experts(float* moe, const void* blob, uint32_t kind, size_t gate_up, size_t down, const float* x,
                    size_t hidden, size_t inter, size_t experts, size_t top_k, const uint32_t* idx,
                    const float* weights, int lanes, int threads, int matmul) {
    const size_t h = hidden;
    float* gu = m_floats(2 * inter);
    float* act = m_floats(inter);
    float* eout = m_floats(h);
    int rc = (gu && act && eout) ? ORC_OK : ORC_OUT_OF_MEMORY;
    memset(moe, 0, h * sizeof(float));
    /* ascending expert index, the order of the reference implementation's index_add */
    for (size_t e = 0; e < experts && rc == ORC_OK; ++e) {
        int slot = -1;
        for (size_t k = 0; k < top_k; ++k)
            if (idx[k] == e) slot = (int)k;
        if (slot < 0) continue;
        const size_t gu_off = gate_up + e * 2 * inter * h, d_off = down + e * h * inter;
        if (!matmul) {
            const void* wgu = kind == 1 ? (const void*)((const uint16_t*)blob + gu_off)
                                        : (const void*)((const float*)blob + gu_off);
            const void* wd = kind == 1 ? (const void*)((const uint16_t*)blob + d_off)
                                       : (const void*)((const float*)blob + d_off);
            if ((rc = orc_linear_threaded(gu, wgu, kind, 2 * inter, h, x, NULL, lanes, threads, 64))) break;
            orc_silu_mul(act, gu, gu + inter, inter);
            if ((rc = orc_linear_threaded(eout, wd, kind, h, inter, act, NULL, lanes, threads, 64))) break;
        } else {  /* src/tensor.zig:297-325 matmul -> matmulBlocked, one row of activations */
            float* bgu = m_transposed_f32(blob, kind, gu_off, 2 * inter, h);
            float* bd = m_transposed_f32(blob, kind, d_off, h, inter);
            if (!bgu || !bd) {
                free(bgu);
                free(bd);
                rc = ORC_OUT_OF_MEMORY;
                break;
            }
            orc_matmul_blocked(gu, x, 1, h, bgu, 2 * inter, lanes);
            orc_silu_mul(act, gu, gu + inter, inter);
            orc_matmul_blocked(eout, act, 1, inter, bd, h, lanes);
            free(bgu);
            free(bd);
        }
        const float w = weights[slot];
        for (size_t i = 0; i < h; ++i) moe[i] = moe[i] + eout[i] * w;
    }
    free(gu);
    free(act);
    free(eout);
    return rc;
}

int orc_moe_forward_token(orc_moe_runner* r, uint32_t token, uint32_t pos, float* logits_out, float* hidden_out,
                          uint32_t* experts_out) {
    if (!r) return ORC_NULL_ARG;
    const orc_config* c = &r->c.base;
    if (token >= c->vocab) return ORC_INVALID_TOKEN;
    if (pos >= r->max_seq) return ORC_CONTEXT_FULL;
    const size_t h = c->hidden;
    for (size_t i = 0; i < h; ++i) r->x[i] = m_weight_at(r->blob, c->weight_kind, r->embed + (size_t)token * h + i);
    int rc;
    for (uint32_t l = 0; l < c->layers; ++l) {
        if ((rc = m_forward_layer(r, l, pos))) return rc;
        if (hidden_out) memcpy(hidden_out + (size_t)l * h, r->x, h * sizeof(float));
        if (experts_out) memcpy(experts_out + (size_t)l * r->c.top_k, r->idx, r->c.top_k * sizeof(uint32_t));
    }
    orc_moe_rmsnorm(r->norm, r->x, m_w(r, r->final_norm), c->weight_kind, h, c->rms_eps);
    const size_t head = c->tie ? r->embed : r->lm_head;
    if ((rc = m_linear(r, r->logits, head, c->vocab, h, r->norm, (size_t)-1))) return rc;
    if (logits_out) memcpy(logits_out, r->logits, (size_t)c->vocab * sizeof(float));
    return ORC_OK;
}

int orc_moe_kv_read(const orc_moe_runner* r, uint32_t layer, uint32_t pos, float* k_out, float* v_out) {
    if (!r) return ORC_NULL_ARG;
    const size_t kv = m_kv_dim(&r->c.base);
    if (layer >= r->c.base.layers || pos >= r->max_seq) return ORC_INVALID_CONFIG;
    const size_t off = ((size_t)layer * r->max_seq + pos) * kv;
    if (k_out) memcpy(k_out, r->keys + off, kv * sizeof(float));
    if (v_out) memcpy(v_out, r->values + off, kv * sizeof(float));
    return ORC_OK;
}
