// model.hip -- the C ABI of include/vvli_gpu.h: device-resident model, the
// token step, and the greedy generation loop.
//
// Device memory of one model (one HIP stream per model):
//   blob      weights, byte-identical to the host blob (OwnedModel layout)
//   k, v      f32 KV cache [layer][max_seq][kv_dim] (KVCache, src/llm.zig:539-606)
//   rope_cs   (cos, sin) of pos * inv_freq for every position, f32
//   x, qkv, attn, ff, logits   f32 activations (Scratch, src/llm.zig:608-686)
//   part, counters             decode-attention split partials
//   keys, state, prompt, out   argmax keys and the device-side step state
// One token step = embed, per layer {qkv GEMV, attention, o GEMV + residual,
// gate/up GEMV + SwiGLU, down GEMV + residual}, logits GEMV, argmax. It reads
// the token and position from `state`, so it is captured once into a HIP
// graph and replayed; generation chains the steps on the device.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstring>
#include <mutex>
#include <vector>

#include "internal.hpp"
#include "vvli_host.h"
#include "kernels.hpp"

using namespace vvli;

struct vvli_gpu_model {
    vvli_gpu_config cfg{};
    uint32_t max_seq = 0;
    int device = 0;
    hipStream_t stream = nullptr;
    BlobLayout layout;
    size_t ebytes = 2;
    char* blob = nullptr;
    float* kcache = nullptr;
    float* vcache = nullptr;
    float* rope_cs = nullptr;
    float* x = nullptr;
    float* qkv = nullptr;
    float* attn = nullptr;
    float* ff = nullptr;
    float* logits = nullptr;
    float* hidden = nullptr;
    float* part = nullptr;
    uint32_t* counters = nullptr;
    unsigned long long* keys = nullptr;
    uint32_t nkeys = 0;
    StepState* state = nullptr;
    uint32_t* prompt = nullptr;
    uint32_t* out_tokens = nullptr;
    uint32_t out_cap = 0;
    StepState* h_state = nullptr;  // pinned
    uint32_t nsplit = 1;
    hipGraphExec_t graph = nullptr;
    std::vector<float> inv_freq;
    // Persistent decode step (bf16 only).
    bool mk_ok = false;
    uint32_t path = 0;  // 0 auto, 1 per-kernel graph, 2 persistent
    uint32_t mk_blocks = 0;
    size_t mk_lds = 0;
    uint32_t mk_glds_off1 = 0, mk_glds_tiles1 = 0, mk_glds_off2 = 0, mk_glds_tiles = 0, mk_glds_park = 0;
    uint32_t mk_nsplit = 1;
    DecodeLayer* mk_layers = nullptr;
    DecodeGemv* mk_gemv = nullptr;  // [layers * 4 + 1] phase descriptors
    unsigned long long* mk_tw = nullptr;  // tagged activations (DecodeStepParams tx .. step_word)
    size_t mk_tw_words = 0;
    uint32_t* mk_err = nullptr;           // device error word
    uint32_t mk_epoch = 1;                // epoch of the next launch's first phase
    uint32_t* h_err = nullptr;    // pinned
    bool mk_pending = false;      // a persistent launch ran since the last error check
    uint32_t mk_inject = 0;       // test hook: the mk_inject-th next persistent launch starts flagged
    hipEvent_t mk_ev0 = nullptr, mk_ev1 = nullptr;  // around the last timed persistent launch
    bool mk_timed = false;
    HostStepOut* h_out = nullptr;  // pinned: result of the last single-step launch
    float* h_logits = nullptr;     // pinned [vocab]: forward_token_view's logits (allocated on first use)
    uint32_t mk_host_seq = 0;      // sequence number of the last single step (launch or resident request)
    // Resident single steps (vvli_gpu_set_resident): the launch stays on the
    // stream between forward_token calls and takes the next request from
    // h_mbox, for up to res_linger_us of idle time.
    HostMailbox* h_mbox = nullptr;  // pinned (allocated on first use)
    uint32_t res_linger_us = 0;     // 0: off
    bool res_active = false;        // a resident launch may still be running
    uint32_t res_left = 0;          // requests it can still take
    // Mixture-of-experts model (vvli_gpu_moe_model_create).
    bool moe = false;
    MoeLayout moe_layout;
    float* moe_router = nullptr;   // [E] router logits
    uint32_t* moe_idx = nullptr;   // [top_k] selected experts
    float* moe_w = nullptr;        // [top_k] their probabilities
    uint32_t* moe_ticket = nullptr;  // router completion ticket (zero between launches)
    // On-device sampling (vvli_gpu_generate with temperature > 0 or a repeat penalty).
    uint32_t* sample_counts = nullptr;        // [vocab] repeat counts of the window
    unsigned long long* sample_prng = nullptr;  // xoshiro256++ state [4]
    unsigned long long* sample_cand = nullptr;  // two-stage top-k survivors
    uint32_t* sample_nf = nullptr;              // finite counts of the vocab slices
    void* sample_full = nullptr;                // whole-vocabulary candidates (limits over 1024)
    hipGraphExec_t graph_sample = nullptr;    // token step ending in the sampler
    // Batched prefill (bf16 only): chunk buffers, allocated on first use.
    bool pf_ok = false;
    uint32_t prefill_path = 0;  // 0 auto, 1 token loop, 2 batched
    uint32_t pf_rows = 0;       // rows per chunk the buffers hold
    float* pf_x = nullptr;      // [rows][H] residual stream
    float* pf_qkv = nullptr;    // [rows][H + 2 kv]
    float* pf_attn = nullptr;   // [rows][H]
    float* pf_scale = nullptr;  // [rows] RMS scales
    float* pf_ahl = nullptr;    // GEMM activations split hi | lo (gemm_split_elems bf16)
    float* pf_ahl2 = nullptr;   // split planes written by attention (o_proj's A) and SwiGLU (down's A)
    float* pf_gu = nullptr;     // gate/up split-K sums for short chunks ([pf_gu_rows][2I])
    float* pf_part = nullptr;   // K-split partial sums of q|k|v, o_proj and down (gemm_part_elems)
    uint32_t pf_gu_rows = 0;
    void* pf_kvp = nullptr;     // packed K/V tiles of one layer for the attention kernel
    size_t pf_kvp_bytes = 0;
    // MoE prefill, per (row, slot) pair of a chunk (pf_rows * top_k pairs).
    uint32_t* pf_eidx = nullptr;   // expert of each pair
    float* pf_ew = nullptr;        // its router probability
    uint32_t* pf_grows = nullptr;  // grouped pair -> row
    uint32_t* pf_ppos = nullptr;   // pair -> grouped position
    uint4* pf_tiles = nullptr;     // grouped GEMM tile table
    uint16_t* pf_ehl = nullptr;    // gate/up input planes over the grouped pairs
    uint16_t* pf_eact = nullptr;   // SwiGLU planes (the down GEMM's input)
    float* pf_eout = nullptr;      // [pairs][H] expert outputs
};

namespace {

#define HIP_TRY(expr)                                                                                   \
    do {                                                                                                \
        hipError_t e_ = (expr);                                                                         \
        if (e_ != hipSuccess)                                                                           \
            return set_error(e_ == hipErrorOutOfMemory ? VVLI_OUT_OF_MEMORY : VVLI_HIP_ERROR, "%s: %s", \
                             #expr, hipGetErrorString(e_));                                             \
    } while (0)

#define LAUNCH(expr) HIP_TRY(expr)
#define RESIDENT_STOP(m)                       \
    do {                                       \
        const int rs_ = resident_stop(m);      \
        if (rs_) return rs_;                   \
    } while (0)

const void* wslice(const vvli_gpu_model* m, size_t off) {
    return off == kNone ? nullptr : static_cast<const void*>(m->blob + off * m->ebytes);
}

int init_once() {
    static std::once_flag flag;
    static hipError_t err = hipSuccess;
    std::call_once(flag, [] {
        err = gemv_init_attributes();
        if (err == hipSuccess) err = moe_gemv_init_attributes();
    });
    HIP_TRY(err);
    return VVLI_OK;
}

// inv_freq[i] = 1 / pow(theta, 2i / hd) in f32 (rotatePair, src/llm.zig:1360-1363),
// then (cos, sin) of the f32 angle pos * inv_freq for every position.
int upload_rope(vvli_gpu_model* m) {
    const uint32_t hd = head_dim(m->cfg), half = hd / 2;
    if (m->inv_freq.empty()) {
        m->inv_freq.resize(half);
        for (uint32_t i = 0; i < half; ++i) {
            const float exponent = static_cast<float>(2 * i) / static_cast<float>(hd);
            m->inv_freq[i] = 1.0f / powf(m->cfg.rope_theta, exponent);
        }
    }
    std::vector<float> cs(static_cast<size_t>(m->max_seq) * hd);
    for (uint32_t p = 0; p < m->max_seq; ++p) {
        const float pos_f = static_cast<float>(p);
        for (uint32_t i = 0; i < half; ++i) {
            const float angle = pos_f * m->inv_freq[i];
            cs[(static_cast<size_t>(p) * half + i) * 2] = cosf(angle);
            cs[(static_cast<size_t>(p) * half + i) * 2 + 1] = sinf(angle);
        }
    }
    HIP_TRY(hipMemcpy(m->rope_cs, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice));
    return VVLI_OK;
}

int check_kernel_shapes(const vvli_gpu_config& c) {
    const uint32_t hd = head_dim(c), e = c.weight_kind == VVLI_WEIGHT_BF16 ? 8 : 4;
    if (hd % 4 != 0 || hd > 128)
        return set_error(VVLI_INVALID_CONFIG, "head_dim %u: GPU kernels need a multiple of 4 up to 128", hd);
    if (kv_group(c) > 16) return set_error(VVLI_INVALID_CONFIG, "GQA group %u > 16", kv_group(c));
    if (c.hidden % e != 0 || c.inter % e != 0)
        return set_error(VVLI_INVALID_CONFIG, "hidden/intermediate must be multiples of %u", e);
    return VVLI_OK;
}

int enqueue_logits(vvli_gpu_model* m, hipStream_t s, const SampleArgs* smp = nullptr);

// Slices of the attention half of a layer (dense and MoE blobs share it).
struct AttnSlices {
    size_t input_norm, q, q_bias, k, k_bias, v, v_bias, q_norm, k_norm, o;
};

// input RMSNorm + q/k/v (+ bias) [+ q/k RMSNorm] + RoPE + KV append +
// attention + o_proj with the residual add, for layer l.
int enqueue_attention_half(vvli_gpu_model* m, hipStream_t s, uint32_t l, const AttnSlices& L) {
    const vvli_gpu_config& c = m->cfg;
    const int kind = static_cast<int>(c.weight_kind);
    const uint32_t H = c.hidden, kv = kv_dim(c), hd = head_dim(c);
    float* q = m->qkv;
    float* kn = m->qkv + H;
    float* vn = m->qkv + H + kv;
    const uint32_t rplain = gemv_rows_per_block(kGemvPlain);
    const bool stack = (H % rplain == 0) && (kv % rplain == 0);
    // 1. input RMSNorm + q/k/v projections (+ bias).
    GemvArgs g;
    g.x = m->x;
    g.norm_w = wslice(m, L.input_norm);
    g.eps = c.rms_eps;
    g.K = H;
    if (stack) {
        g.w[0] = wslice(m, L.q);
        g.w[1] = wslice(m, L.k);
        g.w[2] = wslice(m, L.v);
        g.bias[0] = wslice(m, L.q_bias);
        g.bias[1] = wslice(m, L.k_bias);
        g.bias[2] = wslice(m, L.v_bias);
        g.out[0] = q;
        g.out[1] = kn;
        g.out[2] = vn;
        g.rows[0] = H;
        g.rows[1] = kv;
        g.rows[2] = kv;
        LAUNCH(launch_gemv(kind, kGemvPlain, g, s));
    } else {
        const size_t wo[3] = {L.q, L.k, L.v}, bo[3] = {L.q_bias, L.k_bias, L.v_bias};
        float* outs[3] = {q, kn, vn};
        const uint32_t rows[3] = {H, kv, kv};
        for (int i = 0; i < 3; ++i) {
            GemvArgs gi = g;
            gi.w[0] = wslice(m, wo[i]);
            gi.bias[0] = wslice(m, bo[i]);
            gi.out[0] = outs[i];
            gi.rows[0] = rows[i];
            LAUNCH(launch_gemv(kind, kGemvPlain, gi, s));
        }
    }
    // 2. RoPE + KV append + attention.
    AttnArgs a;
    a.q = q;
    a.k_new = kn;
    a.v_new = vn;
    a.kcache = m->kcache + static_cast<size_t>(l) * m->max_seq * kv;
    a.vcache = m->vcache + static_cast<size_t>(l) * m->max_seq * kv;
    a.pos = &m->state->pos;
    a.rope_cs = m->rope_cs;
    a.part = m->part;
    a.counters = m->counters;
    a.out = m->attn;
    a.heads = c.heads;
    a.kv_heads = c.kv_heads;
    a.hd = hd;
    a.nsplit = m->nsplit;
    a.rope_layout = c.rope_layout;
    a.scale = 1.0f / sqrtf(static_cast<float>(hd));  // src/llm.zig:1313
    if (L.q_norm != kNone) {  // QK-norm over the full q and k (MoE models that carry it)
        a.q_norm = static_cast<const uint16_t*>(wslice(m, L.q_norm));
        a.k_norm = static_cast<const uint16_t*>(wslice(m, L.k_norm));
        a.norm_eps = c.rms_eps;
    }
    LAUNCH(launch_attn_decode(a, s));
    // 3. x += Wo . attn
    GemvArgs go;
    go.w[0] = wslice(m, L.o);
    go.out[0] = m->x;
    go.rows[0] = H;
    go.x = m->attn;
    go.K = H;
    LAUNCH(launch_gemv(kind, kGemvResid, go, s));
    return VVLI_OK;
}

// Router + top-k + selected experts + weighted combine into x (MoE layer l).
int enqueue_moe_ffn(vvli_gpu_model* m, hipStream_t s, uint32_t l) {
    const vvli_gpu_config& c = m->cfg;
    const MoeLayerSlices& L = m->moe_layout.layers[l];
    const uint32_t H = c.hidden, I = c.inter, E = c.num_experts, K = c.experts_per_tok;
    auto w16 = [&](size_t off) { return static_cast<const uint16_t*>(wslice(m, off)); };
    MoeRouterArgs ra;
    ra.w = w16(L.router), ra.x = m->x, ra.norm_w = w16(L.post_norm), ra.eps = c.rms_eps;
    ra.H = H, ra.E = E, ra.top_k = K, ra.logits = m->moe_router, ra.ticket = m->moe_ticket;
    ra.idx = m->moe_idx, ra.weight = m->moe_w;
    LAUNCH(launch_moe_router(ra, s));
    MoeGemvArgs gu;
    gu.w = w16(L.gate_up), gu.experts = m->moe_idx, gu.top_k = K, gu.rows_per_slot = I, gu.K = H;
    gu.x = m->x, gu.x_len = H, gu.norm_w = w16(L.post_norm), gu.eps = c.rms_eps, gu.out = m->ff;
    LAUNCH(launch_moe_gemv(kGemvGateUp, gu, s));
    MoeGemvArgs gd;
    gd.w = w16(L.down), gd.experts = m->moe_idx, gd.top_k = K, gd.rows_per_slot = H, gd.K = I;
    gd.x = m->ff, gd.x_len = K * I;
    LAUNCH(launch_moe_down(gd, m->x, m->moe_w, s));
    return VVLI_OK;
}

// The layers, final norm and logits of one step (embedding already in x);
// the step ends in the greedy finish, or in the sampler when smp is given.
int enqueue_body(vvli_gpu_model* m, hipStream_t s, float* hidden_dbg, const SampleArgs* smp = nullptr) {
    const vvli_gpu_config& c = m->cfg;
    const int kind = static_cast<int>(c.weight_kind);
    const uint32_t H = c.hidden, I = c.inter;
    int rc;
    for (uint32_t l = 0; l < c.layers; ++l) {
        if (m->moe) {
            const MoeLayerSlices& L = m->moe_layout.layers[l];
            const AttnSlices as{L.input_norm, L.q, L.q_bias, L.k, L.k_bias, L.v, L.v_bias, L.q_norm, L.k_norm, L.o};
            if ((rc = enqueue_attention_half(m, s, l, as))) return rc;
            if ((rc = enqueue_moe_ffn(m, s, l))) return rc;
        } else {
            const LayerSlices& L = m->layout.layers[l];
            const AttnSlices as{L.input_norm, L.q, L.q_bias, L.k, L.k_bias, L.v, L.v_bias, kNone, kNone, L.o};
            if ((rc = enqueue_attention_half(m, s, l, as))) return rc;
            // 4. post-attention RMSNorm + gate/up + SwiGLU.
            GemvArgs gu;
            gu.w[0] = wslice(m, L.gate);
            gu.w_up = wslice(m, L.up);
            gu.out[0] = m->ff;
            gu.rows[0] = I;
            gu.x = m->x;
            gu.norm_w = wslice(m, L.post_norm);
            gu.eps = c.rms_eps;
            gu.K = H;
            LAUNCH(launch_gemv(kind, kGemvGateUp, gu, s));
            // 5. x += Wd . ff
            GemvArgs gd;
            gd.w[0] = wslice(m, L.down);
            gd.out[0] = m->x;
            gd.rows[0] = H;
            gd.x = m->ff;
            gd.K = I;
            LAUNCH(launch_gemv(kind, kGemvResid, gd, s));
        }
        if (hidden_dbg)
            HIP_TRY(hipMemcpyAsync(hidden_dbg + static_cast<size_t>(l) * H, m->x, H * sizeof(float),
                                   hipMemcpyDeviceToDevice, s));
    }
    return enqueue_logits(m, s, smp);
}

// Final RMSNorm + logits + argmax (or sampler) of the hidden state in x.
int enqueue_logits(vvli_gpu_model* m, hipStream_t s, const SampleArgs* smp) {
    const vvli_gpu_config& c = m->cfg;
    const int kind = static_cast<int>(c.weight_kind);
    const uint32_t H = c.hidden;
    // logitsMatrix: lm_head, or the embedding when tied (src/llm.zig:410-412).
    GemvArgs gl;
    gl.w[0] = wslice(m, c.tie ? m->layout.embed : m->layout.lm_head);
    gl.out[0] = m->logits;
    gl.rows[0] = c.vocab;
    gl.x = m->x;
    gl.norm_w = wslice(m, m->layout.final_norm);
    gl.eps = c.rms_eps;
    gl.K = H;
    gl.block_keys = m->keys;
    LAUNCH(launch_gemv(kind, kGemvLogits, gl, s));
    if (smp) LAUNCH(launch_sample(*smp, s));
    else LAUNCH(launch_argmax_finish(m->keys, m->nkeys, m->logits, m->state, m->prompt, m->out_tokens, m->out_cap, s));
    return VVLI_OK;
}

int enqueue_step(vvli_gpu_model* m, hipStream_t s, float* hidden_dbg, const SampleArgs* smp = nullptr) {
    LAUNCH(launch_embed(static_cast<int>(m->cfg.weight_kind), wslice(m, m->layout.embed), m->state, m->x,
                        m->cfg.hidden, s));
    return enqueue_body(m, s, hidden_dbg, smp);
}

int ensure_graph(vvli_gpu_model* m) {
    if (m->graph) return VVLI_OK;
    hipGraph_t g = nullptr;
    HIP_TRY(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_step(m, m->stream, nullptr);
    hipError_t e = hipStreamEndCapture(m->stream, &g);
    if (rc != VVLI_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    HIP_TRY(e);
    e = hipGraphInstantiate(&m->graph, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    HIP_TRY(e);
    return VVLI_OK;
}

// The token step ending in the sampler; options are kernel arguments, so the
// graph is captured again for every generate call.
int capture_sample_graph(vvli_gpu_model* m, const SampleArgs& sa) {
    if (m->graph_sample) {
        (void)hipGraphExecDestroy(m->graph_sample);
        m->graph_sample = nullptr;
    }
    hipGraph_t g = nullptr;
    HIP_TRY(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_step(m, m->stream, nullptr, &sa);
    hipError_t e = hipStreamEndCapture(m->stream, &g);
    if (rc != VVLI_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    HIP_TRY(e);
    e = hipGraphInstantiate(&m->graph_sample, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    HIP_TRY(e);
    return VVLI_OK;
}

// validateSamplingOptions (src/generator.zig:329-333) plus the device limit:
// a repeat window that fits 16-bit counts.
int validate_sampling(const vvli_gpu_sampling& o, uint32_t vocab) {
    if (o.temperature < 0.0f || std::isnan(o.temperature))
        return set_error(VVLI_INVALID_SAMPLING, "temperature %g", o.temperature);
    if (o.top_p <= 0.0f || o.top_p > 1.0f || std::isnan(o.top_p))
        return set_error(VVLI_INVALID_SAMPLING, "top_p %g not in (0, 1]", o.top_p);
    if (o.repeat_penalty < 1.0f || std::isnan(o.repeat_penalty))
        return set_error(VVLI_INVALID_SAMPLING, "repeat_penalty %g < 1", o.repeat_penalty);
    (void)vocab;
    if (o.repeat_last_n > 65535) return set_error(VVLI_INVALID_SAMPLING, "repeat_last_n %u > 65535", o.repeat_last_n);
    return VVLI_OK;
}

void prng_seed(uint64_t seed, uint64_t out[4]) {
    // DefaultPrng.init: four SplitMix64 outputs; Sampler.init maps seed 0 to
    // 0x9e3779b97f4a7c15 (src/generator.zig:70-75).
    uint64_t x = seed ? seed : 0x9e3779b97f4a7c15ull;
    for (int i = 0; i < 4; ++i) {
        x += 0x9e3779b97f4a7c15ull;
        uint64_t z = x;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        out[i] = z ^ (z >> 31);
    }
}

// Auto picks the persistent step where it is available (bf16 weights): on the
// Llama-3.2-1B decode benchmark it measures 1178 tok/s against the per-kernel
// graph's 921.
bool use_persistent(const vvli_gpu_model* m) { return m->mk_ok && m->path != 1; }

// Width of the persistent step's feed-forward activation (the down phase's
// input): the intermediate size, or top_k expert widths in an MoE model.
uint32_t mk_ff_width(const vvli_gpu_config& c) { return c.num_experts ? c.experts_per_tok * c.inter : c.inter; }

// Offsets (in words) of the tagged activation arrays inside mk_tw.
struct TaggedLayout {
    size_t tx, tqkv, tattn, tff, ml, acc, keys, copied, step, rl, total;
};
TaggedLayout tagged_layout(const vvli_gpu_config& c, uint32_t nsplit, uint32_t blocks) {
    const size_t H = c.hidden, kv = kv_dim(c), G = c.heads / c.kv_heads, hd = head_dim(c);
    TaggedLayout t{};
    size_t cur = 0;
    auto take = [&](size_t n) {
        const size_t at = cur;
        cur += (n + 15) / 16 * 16;  // 128-byte aligned arrays
        return at;
    };
    t.tx = take(2 * H);
    t.tqkv = take(H + 2 * kv);
    t.tattn = take(H);
    t.tff = take(mk_ff_width(c));
    t.ml = take(static_cast<size_t>(c.kv_heads) * nsplit * G * 2);
    t.acc = take(static_cast<size_t>(c.kv_heads) * nsplit * G * hd);
    t.keys = take(static_cast<size_t>(blocks) * 8 * 2);
    t.copied = take(blocks);
    t.step = take(1);
    t.rl = take(c.num_experts);  // MoE router logits
    t.total = cur;
    return t;
}

// One step of a single-step call (forward_token): its token and position go
// in the launch arguments, and the result comes back in m->h_out.
struct SingleStep {
    uint32_t token, pos;
    bool resident = false;  // stay for the next requests (h_mbox)
    bool logits = false;    // resident: the first step writes its logits to h_logits
};
// Steps one resident launch can take (its epochs are reserved at launch), and
// the longest idle wait between requests (well inside the other blocks'
// bounded step-word polls, which last seconds).
constexpr uint32_t kResidentSteps = 4096;
constexpr uint32_t kMaxResidentLingerUs = 100000;

int run_persistent(vvli_gpu_model* m, uint32_t n_steps, int64_t eos, unsigned long long* timing = nullptr,
                   uint32_t timing_stride = 0, float* hidden_dbg = nullptr, const SingleStep* single = nullptr) {
    const vvli_gpu_config& c = m->cfg;
    // Epochs only grow; before they would wrap, clear every tag (stale words
    // then carry epoch 0, which no phase uses).
    const uint64_t need = static_cast<uint64_t>(n_steps) * decode_step_phases_per_step(c.layers) + 1;
    if (static_cast<uint64_t>(m->mk_epoch) + need >= 0xffffffffull) {
        HIP_TRY(hipMemsetAsync(m->mk_tw, 0, m->mk_tw_words * sizeof(unsigned long long), m->stream));
        m->mk_epoch = 1;
    }
    DecodeStepParams p{};
    p.vocab = c.vocab;
    p.hidden = c.hidden;
    p.inter = mk_ff_width(c);
    p.layers = c.layers;
    p.heads = c.heads;
    p.kv_heads = c.kv_heads;
    p.hd = head_dim(c);
    p.kvdim = kv_dim(c);
    p.rope_layout = c.rope_layout;
    p.max_seq = m->max_seq;
    p.eps = c.rms_eps;
    p.scale = 1.0f / sqrtf(static_cast<float>(p.hd));
    p.embed = static_cast<const uint16_t*>(wslice(m, m->layout.embed));
    p.final_norm = static_cast<const uint16_t*>(wslice(m, m->layout.final_norm));
    p.lm_head = static_cast<const uint16_t*>(wslice(m, c.tie ? m->layout.embed : m->layout.lm_head));
    p.layer = m->mk_layers;
    p.gemv = m->mk_gemv;
    p.kcache = m->kcache;
    p.vcache = m->vcache;
    p.rope_cs = m->rope_cs;
    const TaggedLayout tl = tagged_layout(c, m->mk_nsplit, m->mk_blocks);
    p.tx = m->mk_tw + tl.tx;
    p.tqkv = m->mk_tw + tl.tqkv;
    p.tattn = m->mk_tw + tl.tattn;
    p.tff = m->mk_tw + tl.tff;
    p.tpart_ml = m->mk_tw + tl.ml;
    p.tpart_acc = m->mk_tw + tl.acc;
    p.tkeys = m->mk_tw + tl.keys;
    p.tcopied = m->mk_tw + tl.copied;
    p.step_word = m->mk_tw + tl.step;
    p.logits = m->logits;
    p.state = m->state;
    p.prompt = m->prompt;
    p.out_tokens = m->out_tokens;
    p.out_cap = m->out_cap;
    p.error = m->mk_err;
    p.epoch0 = m->mk_epoch;
    p.nsplit = m->mk_nsplit;
    p.min_chunk = 64;
    p.n_steps = n_steps;
    p.eos = eos;
    p.timing = timing;
    p.timing_stride = timing_stride;
    p.timing_slots = timing_stride >= 16u * decode_step_phases_per_step(c.layers) ? 16u : 1u;
    p.table_lds_offset = static_cast<uint32_t>(decode_step_table_offset(c.hidden, mk_ff_width(c), p.hd));
    p.g_lds_offset1 = m->mk_glds_off1;
    p.g_lds_tiles1 = m->mk_glds_tiles1;
    p.g_lds_offset2 = m->mk_glds_off2;
    p.g_lds_tiles = m->mk_glds_tiles;
    p.g_lds_park = m->mk_glds_park;
    p.hidden_dbg = hidden_dbg;
    if (m->moe) p.experts = c.num_experts, p.top_k = c.experts_per_tok, p.trl = m->mk_tw + tl.rl;
    if (single) {
        p.init_step = 1;
        p.init_token = single->token;
        p.init_pos = single->pos;
        p.host_out = m->h_out;
        p.host_seq = ++m->mk_host_seq;
        if (p.host_seq == 0) p.host_seq = m->mk_host_seq = 1;  // 0 is what h_out holds before any launch
        if (single->resident) {
            p.mbox = m->h_mbox;
            p.linger_ticks = m->res_linger_us * 100u;  // s_memrealtime runs at 100 MHz
            p.host_logits = m->h_logits;
            p.init_logits = single->logits ? 1u : 0u;
        }
    }
    m->mk_epoch += static_cast<uint32_t>(need);
    // The error word is zero here unless a launch of an unchecked sequence
    // (the sampled generation loop) failed: its blocks then leave at once, and
    // the check that reports the flag clears it (persistent_error_rc).
    if (m->mk_inject && --m->mk_inject == 0)
        HIP_TRY(hipMemsetAsync(m->mk_err, kDecodeErrInjected, 1, m->stream));
    // Single steps go untimed: the two event records cost a per-token caller
    // about 8 us per call.
    if (!single) HIP_TRY(hipEventRecord(m->mk_ev0, m->stream));
    HIP_TRY(launch_decode_step(p, m->mk_blocks, m->mk_lds, m->stream));
    if (!single) HIP_TRY(hipEventRecord(m->mk_ev1, m->stream));
    m->mk_pending = true;
    if (!single) m->mk_timed = true;
    return VVLI_OK;
}

// The device error word of the last persistent launch, once it is in h_err.
// A raised flag is reported once and cleared, so the next launch starts
// with it down.
static int persistent_error_rc(vvli_gpu_model* m, uint32_t e) {
    if (e == 0) return VVLI_OK;
    HIP_TRY(hipMemsetAsync(m->mk_err, 0, sizeof(uint32_t), m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return set_error(VVLI_HIP_ERROR, "persistent decode step stopped: device error %u (%s)", e,
                     e == kDecodeErrTimeout ? "input wait timed out"
                                            : (e == kDecodeErrState ? "invalid step state" : "injected by test hook"));
}

int check_persistent_error(vvli_gpu_model* m) {
    if (!m->mk_pending) return VVLI_OK;
    m->mk_pending = false;
    HIP_TRY(hipMemcpyAsync(m->h_err, m->mk_err, sizeof(uint32_t),
                           hipMemcpyDeviceToHost, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return persistent_error_rc(m, *m->h_err);
}

// Outputs of a single-step persistent launch: the argmax (and error word)
// from pinned host memory, which the step's finishing thread wrote -- no
// copy -- and the logits when asked for, behind one synchronisation.
int read_single(vvli_gpu_model* m, float* logits_out, uint32_t* argmax_out) {
    if (logits_out)
        HIP_TRY(hipMemcpyAsync(logits_out, m->logits, static_cast<size_t>(m->cfg.vocab) * sizeof(float),
                               hipMemcpyDeviceToHost, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    const volatile HostStepOut* h = m->h_out;
    if (h->seq == m->mk_host_seq && h->error == 0) {
        m->mk_pending = false;
        if (argmax_out) *argmax_out = h->argmax;
        return VVLI_OK;
    }
    // The blocks left before the end of the step: the device word says why.
    const int rc = check_persistent_error(m);
    if (rc) return rc;
    return set_error(VVLI_HIP_ERROR, "persistent decode step ended without its result");
}

// ---------------------------------------------------------------------------
// Resident single steps. forward_token hands the running launch its request
// through pinned host memory (token, position, whether to write the logits,
// then the sequence number) and spins on the step's report in h_out; the
// step writes its logits straight to h_logits when asked. A launch that has
// ended (no request within the linger time, kResidentSteps taken, or an
// error) is found by a stream query: after an error the device word says
// why, else the request goes out with a new launch.
// ---------------------------------------------------------------------------
// Coherent (fine-grained) pinned memory: the device's stores reach it while
// its launch runs, and its loads see the host's stores.
static int alloc_pinned(void** p, size_t bytes) {
    if (*p) return VVLI_OK;
    if (hipHostMalloc(p, bytes, hipHostMallocCoherent) != hipSuccess) {
        *p = nullptr;
        return set_error(VVLI_OUT_OF_MEMORY, "hipHostMalloc of %zu bytes failed", bytes);
    }
    std::memset(*p, 0, bytes);
    return VVLI_OK;
}

// Ends a resident launch that may still be waiting for a request (every
// other entry point calls this before it touches the stream or the model).
int resident_stop(vvli_gpu_model* m) {
    if (!m->res_active) return VVLI_OK;
    m->res_active = false;
    volatile HostMailbox* mb = m->h_mbox;
    mb->cmd = 1;
    std::atomic_thread_fence(std::memory_order_release);
    mb->seq = ++m->mk_host_seq;  // the request it waits for: leave
    HIP_TRY(hipStreamSynchronize(m->stream));
    return check_persistent_error(m);
}

static int resident_launch(vvli_gpu_model* m, uint32_t token, uint32_t pos, bool logits) {
    SingleStep one{token, pos};
    one.resident = true;
    one.logits = logits;
    const int rc = run_persistent(m, kResidentSteps, -1, nullptr, 0, nullptr, &one);
    if (rc) return rc;
    m->res_active = true;
    m->res_left = kResidentSteps - 1;
    return VVLI_OK;
}

static int forward_resident(vvli_gpu_model* m, uint32_t token, uint32_t pos, float* logits_out,
                            uint32_t* argmax_out) {
    const vvli_gpu_config& c = m->cfg;
    int rc = alloc_pinned(reinterpret_cast<void**>(&m->h_mbox), sizeof(HostMailbox));
    if (rc) return rc;
    const bool want = logits_out != nullptr;
    // Every resident launch gets the logits buffer, so any request can ask for them.
    if ((rc = alloc_pinned(reinterpret_cast<void**>(&m->h_logits), static_cast<size_t>(c.vocab) * sizeof(float))))
        return rc;
    if (m->mk_host_seq >= 0xfffffff0u) {  // sequence numbers restart (0 is never a request's)
        if ((rc = resident_stop(m))) return rc;
        m->mk_host_seq = 0;
        m->h_out->seq = 0;
    }
    bool sent = false;
    if (m->res_active && m->res_left > 0) {
        volatile HostMailbox* mb = m->h_mbox;
        mb->token = token;
        mb->pos = pos | (want ? 0x80000000u : 0u);
        mb->cmd = 0;
        std::atomic_thread_fence(std::memory_order_release);
        mb->seq = ++m->mk_host_seq;
        --m->res_left;
        sent = true;
    } else {
        if ((rc = resident_stop(m))) return rc;  // a launch with no requests left
        if ((rc = resident_launch(m, token, pos, want))) return rc;
    }
    const volatile HostStepOut* h = m->h_out;
    // (m->mk_host_seq: the request's number; a relaunch below gives it a new one.)
    for (uint32_t spins = 1; h->seq != m->mk_host_seq; ++spins) {
        if ((spins & 255u) != 0) continue;
        const hipError_t q = hipStreamQuery(m->stream);
        if (q == hipErrorNotReady) continue;
        if (q != hipSuccess) HIP_TRY(q);
        if (h->seq == m->mk_host_seq) break;
        // The launch has ended without this step's report.
        m->res_active = false;
        if ((rc = check_persistent_error(m))) return rc;
        if (!sent) return set_error(VVLI_HIP_ERROR, "persistent decode step ended without its result");
        // It left before taking the request: a new launch carries it.
        if ((rc = resident_launch(m, token, pos, want))) return rc;
        sent = false;
    }
    std::atomic_thread_fence(std::memory_order_acquire);
    if (argmax_out) *argmax_out = h->argmax;
    if (logits_out && logits_out != m->h_logits)
        std::memcpy(logits_out, m->h_logits, static_cast<size_t>(c.vocab) * sizeof(float));
    return VVLI_OK;
}

// The step's outputs. Without logits, the argmax and (after a persistent
// launch) the error word come back behind one synchronisation; with the
// logits, the error word is read after them (measured per call at Llama-1B:
// 798 against 808 us with the argmax only, but 864-870 against 857 us when
// the small copies share the logits copy's batch).
int read_outputs(vvli_gpu_model* m, float* logits_out, uint32_t* argmax_out) {
    const bool merged = m->mk_pending && !logits_out;
    if (merged)
        HIP_TRY(hipMemcpyAsync(m->h_err, m->mk_err, sizeof(uint32_t), hipMemcpyDeviceToHost, m->stream));
    if (logits_out)
        HIP_TRY(hipMemcpyAsync(logits_out, m->logits, static_cast<size_t>(m->cfg.vocab) * sizeof(float),
                               hipMemcpyDeviceToHost, m->stream));
    if (argmax_out)
        HIP_TRY(hipMemcpyAsync(m->h_state, m->state, sizeof(StepState), hipMemcpyDeviceToHost, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    if (merged) {
        m->mk_pending = false;
        const int rc = persistent_error_rc(m, *m->h_err);
        if (rc) return rc;
    } else {
        const int rc = check_persistent_error(m);
        if (rc) return rc;
    }
    if (argmax_out) *argmax_out = m->h_state->argmax;
    return VVLI_OK;
}

// ---------------------------------------------------------------------------
// Batched prefill: every prompt row of a chunk through each layer at once
// (prefill.hip). Same KV rows and last logits as the token loop, within the
// f32 tolerance; bf16 weights and head_dim 32 / 64 / 128.
// ---------------------------------------------------------------------------
constexpr uint32_t kPrefillChunk = 2048;  // rows per pass; bounds the chunk buffers

bool prefill_supported(const vvli_gpu_config& c) {
    const uint32_t hd = head_dim(c);
    return c.weight_kind == VVLI_WEIGHT_BF16 && (hd == 32 || hd == 64 || hd == 128);
}

bool use_batched_prefill(const vvli_gpu_model* m) {
    return m->prefill_path != 1 && prefill_supported(m->cfg);
}

int ensure_prefill_buffers(vvli_gpu_model* m) {
    if (m->pf_scale) return VVLI_OK;
    const vvli_gpu_config& c = m->cfg;
    const size_t rows = std::min(m->max_seq, kPrefillChunk);
    const size_t H = c.hidden, kv = kv_dim(c), I = c.inter;
    float** bufs[] = {&m->pf_x, &m->pf_qkv, &m->pf_attn, &m->pf_scale, &m->pf_ahl, &m->pf_ahl2};
    const size_t split = (gemm_split_elems(static_cast<uint32_t>(rows), static_cast<uint32_t>(std::max(H, I))) + 1) / 2;
    const size_t sizes[] = {rows * H, rows * (H + 2 * kv), rows * H, rows, split, split};
    for (int i = 0; i < 6; ++i) {
        hipError_t e = hipMalloc(reinterpret_cast<void**>(bufs[i]), sizes[i] * sizeof(float));
        if (e != hipSuccess) {
            for (float** b : bufs) {
                if (*b) (void)hipFree(*b);
                *b = nullptr;
            }
            return set_error(e == hipErrorOutOfMemory ? VVLI_OUT_OF_MEMORY : VVLI_HIP_ERROR,
                             "prefill buffers (%zu rows): %s", rows, hipGetErrorString(e));
        }
    }
    const size_t kvp = prefill_kv_pack_bytes(static_cast<uint32_t>(m->max_seq), c.kv_heads, head_dim(c));
    hipError_t e = hipMalloc(&m->pf_kvp, kvp);
    if (e != hipSuccess) {
        for (float** b : bufs) {
            (void)hipFree(*b);
            *b = nullptr;
        }
        m->pf_kvp = nullptr;
        return set_error(e == hipErrorOutOfMemory ? VVLI_OUT_OF_MEMORY : VVLI_HIP_ERROR,
                         "prefill K/V tiles (%zu bytes): %s", kvp, hipGetErrorString(e));
    }
    m->pf_kvp_bytes = kvp;
    m->pf_rows = static_cast<uint32_t>(rows);
    e = hipMalloc(reinterpret_cast<void**>(&m->pf_part), gemm_part_elems() * sizeof(float));
    if (e != hipSuccess) {
        m->pf_part = nullptr;  // split GEMMs then add their partial sums atomically
        (void)hipGetLastError();
    }
    if (m->moe) return VVLI_OK;
    const uint32_t gu_rows = std::min<uint32_t>(m->pf_rows, gemm_gateup_split_rows(c.inter));
    if (gu_rows > 0 && hipMalloc(reinterpret_cast<void**>(&m->pf_gu), static_cast<size_t>(gu_rows) * 2 * I *
                                                                          sizeof(float)) == hipSuccess)
        m->pf_gu_rows = gu_rows;
    else
        m->pf_gu = nullptr;  // short chunks then run gate/up unsplit
    return VVLI_OK;
}

int ensure_moe_prefill_buffers(vvli_gpu_model* m) {
    if (m->pf_eout) return VVLI_OK;
    const vvli_gpu_config& c = m->cfg;
    const size_t n = static_cast<size_t>(m->pf_rows) * c.experts_per_tok;
    void** bufs[] = {reinterpret_cast<void**>(&m->pf_eidx), reinterpret_cast<void**>(&m->pf_ew),
                     reinterpret_cast<void**>(&m->pf_grows), reinterpret_cast<void**>(&m->pf_ppos),
                     reinterpret_cast<void**>(&m->pf_tiles), reinterpret_cast<void**>(&m->pf_ehl),
                     reinterpret_cast<void**>(&m->pf_eact), reinterpret_cast<void**>(&m->pf_eout)};
    const size_t tiles = 1 + grouped_gemm_max_tiles(static_cast<uint32_t>(n), c.num_experts);
    const size_t bytes[] = {n * 4, n * 4, n * 4, n * 4, tiles * sizeof(uint4), gemm_split_elems(static_cast<uint32_t>(n), c.hidden) * 2,
                            gemm_split_elems(static_cast<uint32_t>(n), c.inter) * 2, n * c.hidden * sizeof(float)};
    for (int i = 0; i < 8; ++i) {
        hipError_t e = hipMalloc(bufs[i], bytes[i]);
        if (e != hipSuccess) {
            for (void** b : bufs) {
                if (*b) (void)hipFree(*b);
                *b = nullptr;
            }
            return set_error(e == hipErrorOutOfMemory ? VVLI_OUT_OF_MEMORY : VVLI_HIP_ERROR,
                             "MoE prefill buffers (%zu pairs): %s", n, hipGetErrorString(e));
        }
    }
    return VVLI_OK;
}

// Mixture-of-experts half of a prefill layer for the chunk's P rows: route
// every row, group the (row, slot) pairs by expert, run the experts' gate/up
// and down as grouped GEMMs over their rows, combine into pf_x.
int enqueue_prefill_moe_ffn(vvli_gpu_model* m, uint32_t l, uint32_t P, hipStream_t s, uint32_t o_splits) {
    const vvli_gpu_config& c = m->cfg;
    const MoeLayerSlices& L = m->moe_layout.layers[l];
    const uint32_t H = c.hidden, I = c.inter, E = c.num_experts, K = c.experts_per_tok, n = P * K;
    auto w16 = [&](size_t off) { return static_cast<const uint16_t*>(wslice(m, off)); };
    // (completes x with o_proj's K-split partial sums first, when it split)
    LAUNCH(launch_row_rms(m->pf_x, H, P, c.rms_eps, m->pf_scale, s, m->pf_part, o_splits));
    MoeRouteRowsArgs ra;
    ra.w = w16(L.router), ra.x = m->pf_x, ra.row_scale = m->pf_scale, ra.norm_w = w16(L.post_norm);
    ra.rows = P, ra.H = H, ra.E = E, ra.top_k = K, ra.idx = m->pf_eidx, ra.weight = m->pf_ew;
    LAUNCH(launch_moe_route_rows(ra, s));
    LAUNCH(launch_moe_group(m->pf_eidx, P, K, E, grouped_gemm_tile_rows(), m->pf_grows, m->pf_ppos, m->pf_tiles, s));
    // act = silu(norm(x_row) . Wg_e^T) * (norm(x_row) . Wu_e^T) per pair, as split planes
    GemmArgs gu;
    gu.a = m->pf_x, gu.lda = H, gu.a_rows = m->pf_grows, gu.row_scale = m->pf_scale, gu.norm_w = w16(L.post_norm);
    gu.w[0] = w16(L.gate_up), gu.w_up = w16(L.gate_up) + static_cast<size_t>(I) * H;
    gu.w_expert = static_cast<size_t>(2) * I * H;
    gu.seg_end[0] = gu.seg_end[1] = gu.seg_end[2] = I;
    gu.M = n, gu.N = I, gu.K = H;
    gu.a_hl = m->pf_ehl;
    gu.out_hl = m->pf_eact, gu.out_plane = static_cast<size_t>(n) * gemm_kp(I);
    gu.tiles = m->pf_tiles, gu.max_tiles = grouped_gemm_max_tiles(n, E);
    LAUNCH(launch_gemm_grouped(kGemmGateUp, gu, s));
    // out_pair = act . Wd_e^T
    GemmArgs gd;
    gd.w[0] = w16(L.down), gd.w_expert = static_cast<size_t>(H) * I;
    gd.seg_end[0] = gd.seg_end[1] = gd.seg_end[2] = H;
    gd.out = m->pf_eout, gd.ldo = H, gd.M = n, gd.N = H, gd.K = I;
    gd.a_hl = m->pf_eact, gd.a_ready = true, gd.a_plane = static_cast<size_t>(n) * gemm_kp(I);
    gd.tiles = m->pf_tiles, gd.max_tiles = gu.max_tiles;
    LAUNCH(launch_gemm_grouped(kGemmPlain, gd, s));
    LAUNCH(launch_moe_combine(m->pf_eout, m->pf_ppos, m->pf_eidx, m->pf_ew, P, K, H, m->pf_x, s));
    return VVLI_OK;
}

// Prompt tokens are already in m->prompt[start .. start + n). Leaves the KV
// rows of those positions, the last row's logits and argmax, and the step
// state as the token loop leaves it (next position start + n, next token the
// argmax; with `counting` the argmax is out_tokens[0]).
int enqueue_prefill_batched(vvli_gpu_model* m, uint32_t start, uint32_t n, uint32_t last_token, uint32_t counting) {
    int rc = ensure_prefill_buffers(m);
    if (rc) return rc;
    if (m->moe && (rc = ensure_moe_prefill_buffers(m))) return rc;
    const vvli_gpu_config& c = m->cfg;
    hipStream_t s = m->stream;
    const uint32_t H = c.hidden, kv = kv_dim(c), I = c.inter, hd = head_dim(c), ldqkv = H + 2 * kv;
    const uint16_t* embed = static_cast<const uint16_t*>(wslice(m, m->layout.embed));
    auto w16 = [&](size_t off) { return static_cast<const uint16_t*>(wslice(m, off)); };
    // K-split GEMMs leave partial sums in pf_part for their consumer (the
    // next row RMS pass, or the RoPE pass for q|k|v), which adds them in split
    // order: pend = the splits of the Resid GEMM whose sums x still lacks
    // (0: the GEMM did not leave any).
    // (Up to 8 splits: with more, the partial sums cost more traffic than the
    // atomic adds they replace -- measured at 128 rows, where down splits 32
    // ways: 3.11 ms with atomics, 3.30 ms with partial sums.)
    auto use_part = [&](int mode, GemmArgs& g) {
        const uint32_t sp = m->pf_part ? gemm_splits(mode, g) : 1u;
        g.part = (sp > 1 && sp <= 8) ? m->pf_part : nullptr;
        return g.part ? sp : 0u;
    };
    for (uint32_t c0 = 0; c0 < n; c0 += m->pf_rows) {
        const uint32_t P = std::min(m->pf_rows, n - c0);
        const uint32_t pos0 = start + c0;
        uint32_t pend = 0;
        LAUNCH(launch_prefill_embed(embed, m->prompt + pos0, P, H, m->pf_x, s));
        for (uint32_t l = 0; l < c.layers; ++l) {
            AttnSlices L;
            if (m->moe) {
                const MoeLayerSlices& M = m->moe_layout.layers[l];
                L = AttnSlices{M.input_norm, M.q, M.q_bias, M.k, M.k_bias, M.v, M.v_bias, M.q_norm, M.k_norm, M.o};
            } else {
                const LayerSlices& D = m->layout.layers[l];
                L = AttnSlices{D.input_norm, D.q, D.q_bias, D.k, D.k_bias, D.v, D.v_bias, kNone, kNone, D.o};
            }
            float* kc = m->kcache + static_cast<size_t>(l) * m->max_seq * kv;
            float* vc = m->vcache + static_cast<size_t>(l) * m->max_seq * kv;
            // input RMSNorm into the q|k|v GEMM's A planes (+ bias in the GEMM)
            GemmArgs gq;
            if (row_norm_split_fits(H)) {
                LAUNCH(launch_row_norm_split(m->pf_x, H, P, c.rms_eps, w16(L.input_norm), m->pf_part, pend,
                                             reinterpret_cast<uint16_t*>(m->pf_ahl),
                                             static_cast<size_t>(P) * gemm_kp(H), s));
                gq.a_ready = true, gq.a_plane = static_cast<size_t>(P) * gemm_kp(H);
            } else {
                LAUNCH(launch_row_rms(m->pf_x, H, P, c.rms_eps, m->pf_scale, s, m->pf_part, pend));
                gq.row_scale = m->pf_scale, gq.norm_w = w16(L.input_norm);
            }
            pend = 0;
            gq.a = m->pf_x, gq.lda = H;
            gq.w[0] = w16(L.q), gq.w[1] = w16(L.k), gq.w[2] = w16(L.v);
            gq.bias[0] = w16(L.q_bias), gq.bias[1] = w16(L.k_bias), gq.bias[2] = w16(L.v_bias);
            gq.seg_end[0] = H, gq.seg_end[1] = H + kv, gq.seg_end[2] = H + 2 * kv;
            gq.out = m->pf_qkv, gq.ldo = ldqkv, gq.M = P, gq.N = ldqkv, gq.K = H;
            gq.a_hl = reinterpret_cast<uint16_t*>(m->pf_ahl);
            const uint32_t q_splits = use_part(kGemmPlain, gq);
            LAUNCH(launch_gemm_bf16(kGemmPlain, gq, s));
            // RoPE on q and k, k/v appended at positions pos0 ..
            PrefillRopeArgs ra{m->pf_qkv, ldqkv, P, pos0, c.heads, c.kv_heads, hd, kv, c.rope_layout,
                               m->rope_cs, kc, vc};
            if (q_splits > 1) ra.part = m->pf_part, ra.splits = q_splits;
            if (L.q_norm != kNone) ra.q_norm = w16(L.q_norm), ra.k_norm = w16(L.k_norm), ra.norm_eps = c.rms_eps;
            // The MFMA attention writes o_proj's split planes itself (heads * hd = H, a multiple of 32).
            const bool fused_o = !prefill_attn_vector;
            if (fused_o) ra.kv_pack = m->pf_kvp, ra.kv_pack_bytes = m->pf_kvp_bytes;
            LAUNCH(launch_prefill_rope_kv(ra, s));
            PrefillAttnArgs aa{m->pf_qkv, ldqkv, kc, vc, m->pf_attn, H, P, pos0, c.heads, c.kv_heads, kv,
                               1.0f / sqrtf(static_cast<float>(hd))};
            aa.kv_pack = m->pf_kvp, aa.kv_pack_bytes = m->pf_kvp_bytes, aa.new_rows_packed = fused_o;
            if (fused_o) aa.out_hl = reinterpret_cast<uint16_t*>(m->pf_ahl2), aa.out_plane = m->pf_rows * gemm_kp(H);
            LAUNCH(launch_prefill_attn(aa, hd, s));
            // x += attn . Wo^T
            GemmArgs go;
            go.a = m->pf_attn, go.lda = H, go.w[0] = w16(L.o);
            go.seg_end[0] = go.seg_end[1] = go.seg_end[2] = H;
            go.out = m->pf_x, go.ldo = H, go.M = P, go.N = H, go.K = H;
            go.a_hl = reinterpret_cast<uint16_t*>(fused_o ? m->pf_ahl2 : m->pf_ahl);
            if (fused_o) go.a_ready = true, go.a_plane = m->pf_rows * gemm_kp(H);
            pend = use_part(kGemmResid, go);
            LAUNCH(launch_gemm_bf16(kGemmResid, go, s));
            if (m->moe) {
                if ((rc = enqueue_prefill_moe_ffn(m, l, P, s, pend))) return rc;
                pend = 0;
                continue;
            }
            const LayerSlices& D = m->layout.layers[l];
            // post-attention RMSNorm into the gate/up GEMM's A planes (+ SwiGLU in the GEMM)
            GemmArgs gu;
            if (row_norm_split_fits(H)) {
                LAUNCH(launch_row_norm_split(m->pf_x, H, P, c.rms_eps, w16(D.post_norm), m->pf_part, pend,
                                             reinterpret_cast<uint16_t*>(m->pf_ahl),
                                             static_cast<size_t>(P) * gemm_kp(H), s));
                gu.a_ready = true, gu.a_plane = static_cast<size_t>(P) * gemm_kp(H);
            } else {
                LAUNCH(launch_row_rms(m->pf_x, H, P, c.rms_eps, m->pf_scale, s, m->pf_part, pend));
                gu.row_scale = m->pf_scale, gu.norm_w = w16(D.post_norm);
            }
            pend = 0;
            gu.a = m->pf_x, gu.lda = H;
            gu.w[0] = w16(D.gate), gu.w_up = w16(D.up);
            gu.seg_end[0] = gu.seg_end[1] = gu.seg_end[2] = I;
            gu.M = P, gu.N = I, gu.K = H;
            gu.a_hl = reinterpret_cast<uint16_t*>(m->pf_ahl);
            // SwiGLU written as the down GEMM's split planes.
            gu.out_hl = reinterpret_cast<uint16_t*>(m->pf_ahl2), gu.out_plane = m->pf_rows * gemm_kp(I);
            if (P <= m->pf_gu_rows) gu.gu_acc = m->pf_gu;
            LAUNCH(launch_gemm_bf16(kGemmGateUp, gu, s));
            // x += ff . Wd^T
            GemmArgs gd;
            gd.w[0] = w16(D.down);
            gd.seg_end[0] = gd.seg_end[1] = gd.seg_end[2] = H;
            gd.out = m->pf_x, gd.ldo = H, gd.M = P, gd.N = H, gd.K = I;
            gd.a_hl = reinterpret_cast<uint16_t*>(m->pf_ahl2);
            gd.a_ready = true, gd.a_plane = m->pf_rows * gemm_kp(I);
            pend = use_part(kGemmResid, gd);
            LAUNCH(launch_gemm_bf16(kGemmResid, gd, s));
        }
        if (pend > 1)  // the last down projection's partial sums (the scale computed with them is unused)
            LAUNCH(launch_row_rms(m->pf_x, H, P, c.rms_eps, m->pf_scale, s, m->pf_part, pend));
        if (c0 + P == n)
            HIP_TRY(hipMemcpyAsync(m->x, m->pf_x + static_cast<size_t>(P - 1) * H, H * sizeof(float),
                                   hipMemcpyDeviceToDevice, s));
    }
    // State of the token loop after its last prompt step, then that step's logits.
    LAUNCH(launch_set_state(m->state, last_token, start + n - 1, start + n, counting, s));
    return enqueue_logits(m, s);
}

void free_model(vvli_gpu_model* m) {
    if (!m) return;
    (void)hipSetDevice(m->device);
    if (m->graph) (void)hipGraphExecDestroy(m->graph);
    if (m->graph_sample) (void)hipGraphExecDestroy(m->graph_sample);
    void* bufs[] = {m->blob, m->kcache, m->vcache, m->rope_cs, m->x, m->qkv, m->attn, m->ff, m->logits,
                    m->hidden, m->part, m->counters, m->keys, m->state, m->prompt, m->out_tokens,
                    m->mk_layers, m->mk_gemv, m->mk_tw, m->mk_err, m->pf_x, m->pf_qkv, m->pf_attn,
                    m->pf_scale, m->pf_ahl, m->pf_ahl2, m->pf_gu, m->pf_part, m->pf_kvp, m->pf_eidx, m->pf_ew, m->pf_grows, m->pf_ppos, m->pf_tiles, m->pf_ehl, m->pf_eact,
                    m->pf_eout, m->moe_router, m->moe_idx, m->moe_w, m->moe_ticket, m->sample_counts,
                    m->sample_prng, m->sample_cand, m->sample_nf, m->sample_full};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    if (m->h_state) (void)hipHostFree(m->h_state);
    if (m->h_err) (void)hipHostFree(m->h_err);
    if (m->h_out) (void)hipHostFree(m->h_out);
    if (m->h_mbox) (void)hipHostFree(m->h_mbox);
    if (m->h_logits) (void)hipHostFree(m->h_logits);
    if (m->mk_ev0) (void)hipEventDestroy(m->mk_ev0);
    if (m->mk_ev1) (void)hipEventDestroy(m->mk_ev1);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    delete m;
}

template <typename T>
int dmalloc(T** p, size_t count) {
    HIP_TRY(hipMalloc(reinterpret_cast<void**>(p), (count ? count : 1) * sizeof(T)));
    return VVLI_OK;
}

// host_blob == nullptr: the device blob is zeroed and filled by the caller.
int create_impl(const vvli_gpu_config* cfg, uint32_t max_seq_len, const void* host_blob, size_t blob_elems,
                vvli_gpu_model** out, bool moe, bool blob_from_device = false) {
    if (!cfg || (!host_blob && !blob_from_device) || !out)
        return set_error(VVLI_NULL_ARG, "NULL argument to vvli_gpu_model_create");
    *out = nullptr;
    int rc = validate_config(*cfg, !moe);
    if (rc) return rc;
    if ((rc = check_kernel_shapes(*cfg))) return rc;
    if (moe) {
        if (cfg->num_experts == 0) return set_error(VVLI_INVALID_CONFIG, "MoE model with num_experts = 0");
        if (cfg->weight_kind != VVLI_WEIGHT_BF16) return set_error(VVLI_UNSUPPORTED_DTYPE, "MoE models need bf16 weights");
        if (cfg->num_experts > 256 || cfg->experts_per_tok > static_cast<uint32_t>(kMaxTopK))
            return set_error(VVLI_INVALID_CONFIG, "MoE kernels take up to 256 experts and top-%d", kMaxTopK);
        if (static_cast<size_t>(cfg->experts_per_tok) * cfg->inter * sizeof(float) > 150 * 1024)
            return set_error(VVLI_INVALID_CONFIG, "experts_per_tok * intermediate must fit LDS (%u * %u)",
                             cfg->experts_per_tok, cfg->inter);
    }
    if (max_seq_len == 0 || max_seq_len > cfg->max_pos)  // KVCache.init, src/llm.zig:548
        return set_error(VVLI_INVALID_CONFIG, "max_seq_len %u not in 1..%u", max_seq_len, cfg->max_pos);
    if ((rc = init_once())) return rc;

    auto* m = new vvli_gpu_model();
    m->cfg = *cfg;
    m->max_seq = max_seq_len;
    m->moe = moe;
    if (moe) {
        m->moe_layout = compute_moe_layout(*cfg);
        m->layout.embed = m->moe_layout.embed;
        m->layout.final_norm = m->moe_layout.final_norm;
        m->layout.lm_head = m->moe_layout.lm_head;
        m->layout.total = m->moe_layout.total;
    } else {
        m->layout = compute_layout(*cfg);
    }
    m->ebytes = elem_bytes(*cfg);
    if (!blob_from_device && blob_elems < m->layout.total) {
        free_model(m);
        return set_error(VVLI_INVALID_WEIGHT, "blob has %zu elements, layout needs %zu", blob_elems, m->layout.total);
    }
    (void)hipGetDevice(&m->device);
    const uint32_t H = cfg->hidden, kv = kv_dim(*cfg), hd = head_dim(*cfg);
    const size_t kvlen = static_cast<size_t>(cfg->layers) * max_seq_len * kv;
    m->nsplit = attn_nsplit(max_seq_len, hd);
    m->nkeys = gemv_num_keys(cfg->vocab);
    // Persistent step: bf16 only, one 512-thread block per CU if it fits
    // (MoE: head_dim 64 or 128).
    if (cfg->weight_kind == VVLI_WEIGHT_BF16 && (!moe || decode_step_moe_supported(hd))) {
        int cus = 0, bpc = 0;
        m->mk_lds = decode_step_lds_bytes(H, mk_ff_width(*cfg), cfg->layers, hd);
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, m->device) == hipSuccess &&
            m->mk_lds <= 160 * 1024 && decode_step_max_blocks(hd, m->mk_lds, &bpc, moe) == hipSuccess && bpc >= 1 &&
            cus > 0 && static_cast<uint64_t>(max_seq_len) * kv * sizeof(float) < (1ull << 31)) {  // 32-bit KV offsets
            m->mk_ok = true;
            m->mk_blocks = static_cast<uint32_t>(cus);
            // Splits per kv head (<= kMaxSplitMk): every split of a head waits for
            // the others' partials, so all kv_heads * nsplit units hold a block at once.
            m->mk_nsplit = std::max<uint32_t>(
                1, std::min<uint32_t>(std::min<uint32_t>(64, (max_seq_len + 63) / 64), m->mk_blocks / cfg->kv_heads));
            // The rest of the CU's LDS holds gate/up tiles (VVLI_DECODE_GLDS=0: off;
            // MoE: none, the experts are known only once the gate/up phase routes).
            const char* env = getenv("VVLI_DECODE_GLDS");
            uint32_t off1 = 0, n1 = 0, off2 = 0, park = 0;
            size_t lds2 = m->mk_lds;
            const uint32_t tiles = (moe || (env && env[0] == '0'))
                                       ? 0
                                       : decode_step_glds_plan(H, cfg->inter, hd, &lds2, &off1, &n1, &off2, &park);
            if (tiles > 0 && decode_step_max_blocks(hd, lds2, &bpc, moe) == hipSuccess && bpc >= 1) {
                m->mk_glds_off1 = off1;
                m->mk_glds_tiles1 = n1;
                m->mk_glds_off2 = off2;
                m->mk_glds_tiles = tiles;
                m->mk_glds_park = park;
                m->mk_lds = lds2;
            } else {
                (void)decode_step_max_blocks(hd, m->mk_lds, &bpc, moe);  // restore the attribute for the smaller size
            }
        }
        (void)hipGetLastError();
    }
    const size_t part_floats = attn_part_floats(cfg->heads, cfg->kv_heads, hd, m->nsplit);
    const uint32_t nkeys_alloc = std::max<uint32_t>(m->nkeys, m->mk_blocks * 8);
    m->out_cap = max_seq_len + 1;
#define TRY_ALLOC(expr)         \
    if ((rc = (expr)) != 0) {   \
        free_model(m);          \
        return rc;              \
    }
    TRY_ALLOC(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) == hipSuccess
                  ? 0
                  : set_error(VVLI_HIP_ERROR, "hipStreamCreate failed"));
    TRY_ALLOC(dmalloc(&m->blob, m->layout.total * m->ebytes));
    TRY_ALLOC(dmalloc(&m->kcache, kvlen));
    TRY_ALLOC(dmalloc(&m->vcache, kvlen));
    TRY_ALLOC(dmalloc(&m->rope_cs, static_cast<size_t>(max_seq_len) * hd));
    TRY_ALLOC(dmalloc(&m->x, H));
    TRY_ALLOC(dmalloc(&m->qkv, H + 2 * kv));
    TRY_ALLOC(dmalloc(&m->attn, H));
    TRY_ALLOC(dmalloc(&m->ff, static_cast<size_t>(cfg->inter) * (moe ? cfg->experts_per_tok : 1)));
    if (moe) {
        TRY_ALLOC(dmalloc(&m->moe_router, cfg->num_experts));
        TRY_ALLOC(dmalloc(&m->moe_idx, cfg->experts_per_tok));
        TRY_ALLOC(dmalloc(&m->moe_w, cfg->experts_per_tok));
        TRY_ALLOC(dmalloc(&m->moe_ticket, 1));
    }
    TRY_ALLOC(dmalloc(&m->logits, cfg->vocab));
    TRY_ALLOC(dmalloc(&m->hidden, static_cast<size_t>(cfg->layers) * H));
    TRY_ALLOC(dmalloc(&m->part, part_floats));
    TRY_ALLOC(dmalloc(&m->counters, cfg->kv_heads));
    TRY_ALLOC(dmalloc(&m->keys, nkeys_alloc));
    if (m->mk_ok) {
        m->mk_tw_words = tagged_layout(*cfg, m->mk_nsplit, m->mk_blocks).total;
        TRY_ALLOC(dmalloc(&m->mk_tw, m->mk_tw_words));
        TRY_ALLOC(dmalloc(&m->mk_err, 32));
        TRY_ALLOC(dmalloc(&m->mk_layers, cfg->layers));
        TRY_ALLOC(dmalloc(&m->mk_gemv, static_cast<size_t>(cfg->layers) * 4 + 1));
        TRY_ALLOC(hipEventCreate(&m->mk_ev0) == hipSuccess && hipEventCreate(&m->mk_ev1) == hipSuccess
                      ? 0
                      : set_error(VVLI_HIP_ERROR, "hipEventCreate failed"));
        TRY_ALLOC(hipHostMalloc(reinterpret_cast<void**>(&m->h_err), sizeof(uint32_t), hipHostMallocDefault) ==
                          hipSuccess
                      ? 0
                      : set_error(VVLI_OUT_OF_MEMORY, "hipHostMalloc failed"));
        TRY_ALLOC(hipHostMalloc(reinterpret_cast<void**>(&m->h_out), sizeof(HostStepOut), hipHostMallocCoherent) ==
                          hipSuccess
                      ? 0
                      : set_error(VVLI_OUT_OF_MEMORY, "hipHostMalloc failed"));
        std::memset(m->h_out, 0, sizeof(HostStepOut));
    }
    TRY_ALLOC(dmalloc(&m->state, 1));
    TRY_ALLOC(dmalloc(&m->prompt, max_seq_len));
    TRY_ALLOC(dmalloc(&m->out_tokens, m->out_cap));
    TRY_ALLOC(hipHostMalloc(reinterpret_cast<void**>(&m->h_state), sizeof(StepState), hipHostMallocDefault) ==
                      hipSuccess
                  ? 0
                  : set_error(VVLI_OUT_OF_MEMORY, "hipHostMalloc failed"));
    auto fail_hip = [&](hipError_t e, const char* what) {
        return e == hipSuccess ? 0 : set_error(VVLI_HIP_ERROR, "%s: %s", what, hipGetErrorString(e));
    };
    if (host_blob) {
        TRY_ALLOC(fail_hip(hipMemcpy(m->blob, host_blob, m->layout.total * m->ebytes, hipMemcpyHostToDevice),
                           "blob upload"));
    } else {
        TRY_ALLOC(fail_hip(hipMemset(m->blob, 0, m->layout.total * m->ebytes), "blob clear"));
    }
    TRY_ALLOC(fail_hip(hipMemset(m->kcache, 0, kvlen * sizeof(float)), "kv clear"));
    TRY_ALLOC(fail_hip(hipMemset(m->vcache, 0, kvlen * sizeof(float)), "kv clear"));
    TRY_ALLOC(fail_hip(hipMemset(m->counters, 0, cfg->kv_heads * sizeof(uint32_t)), "counters"));
    TRY_ALLOC(fail_hip(hipMemset(m->state, 0, sizeof(StepState)), "state"));
    if (moe) {
        TRY_ALLOC(fail_hip(hipMemset(m->moe_idx, 0, cfg->experts_per_tok * sizeof(uint32_t)), "expert ids"));
        TRY_ALLOC(fail_hip(hipMemset(m->moe_ticket, 0, sizeof(uint32_t)), "router ticket"));
    }
    if (m->mk_tw) {
        TRY_ALLOC(fail_hip(hipMemset(m->mk_tw, 0, m->mk_tw_words * sizeof(unsigned long long)), "tag clear"));
        TRY_ALLOC(fail_hip(hipMemset(m->mk_err, 0, 32 * sizeof(uint32_t)), "error clear"));
    }
    TRY_ALLOC(upload_rope(m));
    if (m->mk_ok) {
        std::vector<DecodeLayer> dl(cfg->layers);
        auto w = [&](size_t off) { return static_cast<const uint16_t*>(wslice(m, off)); };
        const size_t IH = static_cast<size_t>(cfg->inter) * H;
        for (uint32_t l = 0; l < cfg->layers; ++l) {
            if (moe) {  // gate = the fused gate|up of expert 0, up = its up rows
                const MoeLayerSlices& L = m->moe_layout.layers[l];
                dl[l] = DecodeLayer{w(L.input_norm), w(L.q), w(L.q_bias), w(L.k), w(L.k_bias), w(L.v),
                                    w(L.v_bias),     w(L.o), w(L.post_norm), w(L.gate_up), w(L.gate_up) + IH,
                                    w(L.down),       w(L.router), w(L.q_norm), w(L.k_norm)};
                continue;
            }
            const LayerSlices& L = m->layout.layers[l];
            dl[l] = DecodeLayer{w(L.input_norm), w(L.q), w(L.q_bias), w(L.k), w(L.k_bias), w(L.v), w(L.v_bias),
                                w(L.o),          w(L.post_norm), w(L.gate), w(L.up), w(L.down),
                                nullptr,         nullptr,        nullptr};
        }
        TRY_ALLOC(fail_hip(hipMemcpy(m->mk_layers, dl.data(), dl.size() * sizeof(DecodeLayer), hipMemcpyHostToDevice),
                           "layer table"));
        // GEMV phase descriptors: per layer qkv, o (+residual), gate/up, down (+residual); then logits.
        std::vector<DecodeGemv> dg(static_cast<size_t>(cfg->layers) * 4 + 1, DecodeGemv{});
        const TaggedLayout tl = tagged_layout(*cfg, m->mk_nsplit, m->mk_blocks);
        unsigned long long* q = m->mk_tw + tl.tqkv;
        unsigned long long* x_in = m->mk_tw + tl.tx;       // layer input (written by D)
        unsigned long long* x_mid = m->mk_tw + tl.tx + H;  // after attention (written by O)
        for (uint32_t l = 0; l < cfg->layers; ++l) {
            const DecodeLayer& L = dl[l];
            DecodeGemv& gq = dg[l * 4 + 0];
            gq.w0 = L.q, gq.w1 = L.k, gq.w2 = L.v;
            gq.b0 = L.q_bias, gq.b1 = L.k_bias, gq.b2 = L.v_bias;
            gq.o0 = q, gq.o1 = q + H, gq.o2 = q + H + kv;
            gq.r0 = H, gq.r1 = kv, gq.r2 = kv;
            gq.K = H;
            DecodeGemv& go = dg[l * 4 + 1];
            go.w0 = L.o, go.o0 = x_mid, go.r0 = H, go.K = H;
            DecodeGemv& gg = dg[l * 4 + 2];
            gg.w0 = L.gate, gg.w_up = L.up, gg.o0 = m->mk_tw + tl.tff, gg.r0 = cfg->inter, gg.K = H;
            DecodeGemv& gd = dg[l * 4 + 3];
            gd.w0 = L.down, gd.o0 = x_in, gd.r0 = H, gd.K = cfg->inter;
            // Down rows are long (inter) and few (hidden): split each row in
            // two halves so that every wave of the grid streams.
            gd.split = (cfg->inter % 16 == 0 && cfg->inter >= 2 * H) ? 1u : 0u;
            if (moe) {  // routed experts: top_k slots of inter rows / columns
                gg.moe = 1, gg.r_slot = cfg->inter, gg.w_expert = 2 * IH, gg.r0 = cfg->experts_per_tok * cfg->inter;
                gd.moe = 2, gd.r_slot = cfg->experts_per_tok, gd.w_expert = IH, gd.split = 0;
            }
        }
        DecodeGemv& gl = dg[static_cast<size_t>(cfg->layers) * 4];
        gl.w0 = static_cast<const uint16_t*>(wslice(m, cfg->tie ? m->layout.embed : m->layout.lm_head));
        gl.plain = m->logits, gl.r0 = cfg->vocab, gl.K = H;
        TRY_ALLOC(fail_hip(hipMemcpy(m->mk_gemv, dg.data(), dg.size() * sizeof(DecodeGemv), hipMemcpyHostToDevice),
                           "gemv table"));
    }
    TRY_ALLOC(fail_hip(hipDeviceSynchronize(), "create sync"));
#undef TRY_ALLOC
    *out = m;
    return VVLI_OK;
}

int64_t now_ns();

// generateGreedyMeasured on the persistent step: one launch for the prompt
// (token-at-a-time, as the reference), one for the decode steps; the device
// feeds each argmax back as the next token and stops on EOS.
int generate_persistent(vvli_gpu_model* m, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new, int64_t eos,
                        bool batched, uint32_t* out_tokens, uint32_t* n_out, vvli_gpu_stats* stats) {
    const uint32_t avail = m->max_seq - n_prompt;  // positions left for decode forwards
    if (eos < 0 && static_cast<uint64_t>(n_prompt) + max_new > m->max_seq)
        return set_error(VVLI_CONTEXT_FULL, "prompt %u + %u new tokens > max_seq_len %u", n_prompt, max_new, m->max_seq);
    const int64_t t0 = now_ns();
    HIP_TRY(hipMemcpyAsync(m->prompt, prompt, n_prompt * sizeof(uint32_t), hipMemcpyHostToDevice, m->stream));
    int rc;
    if (batched) {
        rc = enqueue_prefill_batched(m, 0, n_prompt, prompt[n_prompt - 1], 1);
    } else {
        HIP_TRY(launch_set_state(m->state, prompt[0], 0, n_prompt, 1, m->stream));
        rc = run_persistent(m, n_prompt, eos);
    }
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(m->h_state, m->state, sizeof(StepState), hipMemcpyDeviceToHost, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    if ((rc = check_persistent_error(m))) return rc;
    const int64_t t1 = now_ns();
    uint32_t produced = 0;
    if (max_new > 0) {
        const bool first_is_eos = eos >= 0 && static_cast<int64_t>(m->h_state->argmax) == eos;
        const uint32_t steps = std::min(max_new, avail);
        if (!first_is_eos && steps > 0) {
            if ((rc = run_persistent(m, steps, eos))) return rc;
        }
        HIP_TRY(hipMemcpyAsync(m->h_state, m->state, sizeof(StepState), hipMemcpyDeviceToHost, m->stream));
        HIP_TRY(hipStreamSynchronize(m->stream));
        if ((rc = check_persistent_error(m))) return rc;
        produced = std::min(m->h_state->n_out, max_new);
        HIP_TRY(hipMemcpyAsync(out_tokens, m->out_tokens, produced * sizeof(uint32_t), hipMemcpyDeviceToHost,
                               m->stream));
        HIP_TRY(hipStreamSynchronize(m->stream));
        const bool hit_eos = eos >= 0 && produced > 0 && static_cast<int64_t>(out_tokens[produced - 1]) == eos;
        if (produced < max_new && !hit_eos)
            return set_error(VVLI_CONTEXT_FULL, "decode reached max_seq_len %u after %u tokens", m->max_seq, produced);
    }
    const int64_t t2 = now_ns();
    *n_out = produced;
    if (stats) {
        stats->prompt_tokens = n_prompt;
        stats->generated_tokens = produced;
        stats->prefill_ns = t1 - t0;
        stats->decode_ns = t2 - t1;
        stats->total_ns = t2 - t0;
    }
    return VVLI_OK;
}

// generateGreedyMeasured with Options (src/generator.zig:221-293): the prompt
// token by token (or batched), then Sampler.next on the device after every
// forward; the sampled token is forwarded, the last one too.
int generate_sampled(vvli_gpu_model* m, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new, int64_t eos,
                     bool batched, const vvli_gpu_sampling& o, uint32_t* out_tokens, uint32_t* n_out,
                     vvli_gpu_stats* stats) {
    const vvli_gpu_config& c = m->cfg;
    if (eos < 0 && static_cast<uint64_t>(n_prompt) + max_new > m->max_seq)
        return set_error(VVLI_CONTEXT_FULL, "prompt %u + %u new tokens > max_seq_len %u", n_prompt, max_new, m->max_seq);
    int rc;
    if (!m->sample_counts && (rc = dmalloc(&m->sample_counts, c.vocab))) return rc;
    if (!m->sample_prng && (rc = dmalloc(&m->sample_prng, 4))) return rc;
    if (!m->sample_cand && (rc = dmalloc(&m->sample_cand, sample_cand_elems(c.vocab)))) return rc;
    if (!m->sample_nf && (rc = dmalloc(&m->sample_nf, sample_nf_elems(c.vocab)))) return rc;
    const uint32_t limit = (o.top_k == 0 || o.top_k > c.vocab) ? c.vocab : o.top_k;
    const bool full = o.temperature > 0.0f && limit > static_cast<uint32_t>(kMaxSampleTopK);
    if (full && !m->sample_full) {
        const size_t bytes = sample_full_bytes(c.vocab);
        if (bytes == 0) return set_error(VVLI_HIP_ERROR, "sort storage size query failed");
        HIP_TRY(hipMalloc(&m->sample_full, bytes));
    }
    const bool penalty = o.repeat_penalty > 1.0f && o.repeat_last_n > 0;
    SampleArgs sa;
    sa.logits = m->logits;
    sa.vocab = c.vocab;
    sa.counts = penalty ? m->sample_counts : nullptr;
    sa.temperature = o.temperature;
    sa.top_p = o.top_p;
    sa.repeat_penalty = o.repeat_penalty;
    sa.top_k = (o.top_k == 0 || o.top_k > c.vocab) ? c.vocab : o.top_k;
    sa.repeat_last_n = o.repeat_last_n;
    sa.prng = m->sample_prng;
    sa.cand_buf = m->sample_cand;
    sa.cand_nf = m->sample_nf;
    sa.full = m->sample_full;
    sa.state = m->state;
    sa.prompt = m->prompt;
    sa.n_prompt = n_prompt;
    sa.out_tokens = m->out_tokens;
    sa.out_cap = m->out_cap;
    // Persistent step where available: each token is one single-step launch
    // (the step leaves the logits, token = argmax and pos + 1 in the state;
    // counting is off, so it appends nothing) and the sampler then replaces the
    // token without advancing pos. Else the captured step + sampler graph.
    const bool persistent = use_persistent(m);
    SampleArgs after_step = sa;
    after_step.advance_pos = 0;
    // The whole-vocabulary sampler (a library sort among its launches) is not
    // captured: the per-kernel path then replays the plain step graph and
    // samples after it, as the persistent path does.
    const bool eager_sampler = persistent || full;
    if (!persistent && full && (rc = ensure_graph(m))) return rc;
    if (!eager_sampler && (rc = capture_sample_graph(m, sa))) return rc;
    const int64_t t0 = now_ns();
    HIP_TRY(hipMemcpyAsync(m->prompt, prompt, n_prompt * sizeof(uint32_t), hipMemcpyHostToDevice, m->stream));
    if (batched) {
        if ((rc = enqueue_prefill_batched(m, 0, n_prompt, prompt[n_prompt - 1], 0))) return rc;
    } else if (persistent) {
        HIP_TRY(launch_set_state(m->state, prompt[0], 0, n_prompt, 0, m->stream));
        if ((rc = run_persistent(m, n_prompt, -1))) return rc;
    } else {
        if ((rc = ensure_graph(m))) return rc;
        HIP_TRY(launch_set_state(m->state, prompt[0], 0, n_prompt, 0, m->stream));
        for (uint32_t i = 0; i < n_prompt; ++i) HIP_TRY(hipGraphLaunch(m->graph, m->stream));
    }
    HIP_TRY(hipStreamSynchronize(m->stream));
    if (persistent && (rc = check_persistent_error(m))) return rc;
    const int64_t t1 = now_ns();
    auto forward_and_sample = [&]() -> int {
        if (!eager_sampler) {
            HIP_TRY(hipGraphLaunch(m->graph_sample, m->stream));
            return VVLI_OK;
        }
        if (persistent) {
            int r = run_persistent(m, 1, -1);
            if (r) return r;
        } else {
            HIP_TRY(hipGraphLaunch(m->graph, m->stream));
        }
        HIP_TRY(launch_sample(after_step, m->stream));
        return VVLI_OK;
    };
    // Sampler.init: PRNG state, repeat counts of the prompt's window.
    uint64_t st4[4];
    prng_seed(o.seed, st4);
    HIP_TRY(hipMemcpy(m->sample_prng, st4, sizeof(st4), hipMemcpyHostToDevice));
    if (penalty) HIP_TRY(launch_sample_counts(m->sample_counts, c.vocab, m->prompt, n_prompt, o.repeat_last_n, m->stream));
    uint32_t produced = 0;
    if (max_new > 0) {
        SampleArgs first = sa;  // the first token comes from the prompt's last logits
        first.advance_pos = 0;
        HIP_TRY(launch_sample(first, m->stream));
        if (eos < 0) {
            for (uint32_t i = 0; i < max_new; ++i)
                if ((rc = forward_and_sample())) return rc;
            produced = max_new;
        } else {
            uint32_t pos = n_prompt;
            while (produced < max_new) {
                HIP_TRY(hipMemcpyAsync(m->h_state, m->state, sizeof(StepState), hipMemcpyDeviceToHost, m->stream));
                HIP_TRY(hipStreamSynchronize(m->stream));
                const uint32_t next = m->h_state->argmax;
                ++produced;
                if (static_cast<int64_t>(next) == eos) break;
                if (pos >= m->max_seq) return set_error(VVLI_CONTEXT_FULL, "pos %u >= max_seq_len", pos);
                if ((rc = forward_and_sample())) return rc;
                ++pos;
            }
        }
        HIP_TRY(hipMemcpyAsync(out_tokens, m->out_tokens, produced * sizeof(uint32_t), hipMemcpyDeviceToHost,
                               m->stream));
    }
    HIP_TRY(hipStreamSynchronize(m->stream));
    if (persistent && (rc = check_persistent_error(m))) return rc;
    const int64_t t2 = now_ns();
    *n_out = produced;
    if (stats) {
        stats->prompt_tokens = n_prompt;
        stats->generated_tokens = produced;
        stats->prefill_ns = t1 - t0;
        stats->decode_ns = t2 - t1;
        stats->total_ns = t2 - t0;
    }
    return VVLI_OK;
}

int64_t now_ns() {
    return std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

}  // namespace

extern "C" {

int vvli_gpu_model_create(const vvli_gpu_config* cfg, uint32_t max_seq_len, const void* host_blob, size_t blob_elems,
                          vvli_gpu_model** out) {
    clear_error();
    return create_impl(cfg, max_seq_len, host_blob, blob_elems, out, false);
}

}  // extern "C"

namespace {

// Places one tensor of a mapped checkpoint into the device blob: same-dtype
// tensors are copied straight from the file bytes, others go through a
// staging buffer and the conversion kernel, in chunks.
struct DeviceSink {
    vvli_gpu_model* m;
    void* staging = nullptr;
    size_t staging_bytes = 0;
};

int device_put(void* ctx, size_t dst, const uint8_t* raw, TensorSrc src, size_t n) {
    auto* d = static_cast<DeviceSink*>(ctx);
    vvli_gpu_model* m = d->m;
    const uint32_t kind = m->cfg.weight_kind;
    char* out = m->blob + dst * m->ebytes;
    const bool same = (kind == VVLI_WEIGHT_F32 && src == kSrcF32) || (kind == VVLI_WEIGHT_BF16 && src == kSrcBF16);
    if (same) {
        HIP_TRY(hipMemcpyAsync(out, raw, n * m->ebytes, hipMemcpyHostToDevice, m->stream));
        return VVLI_OK;
    }
    const size_t sb = src == kSrcF32 ? 4 : 2;
    if (!d->staging) {
        d->staging_bytes = 64ull << 20;
        HIP_TRY(hipMalloc(&d->staging, d->staging_bytes));
    }
    const size_t per = d->staging_bytes / sb;
    for (size_t off = 0; off < n; off += per) {
        const size_t cnt = std::min(per, n - off);
        // Stream order keeps the next chunk's copy behind this chunk's kernel.
        HIP_TRY(hipMemcpyAsync(d->staging, raw + off * sb, cnt * sb, hipMemcpyHostToDevice, m->stream));
        HIP_TRY(launch_convert(d->staging, static_cast<uint32_t>(src), out + off * m->ebytes, kind, cnt, m->stream));
    }
    return VVLI_OK;
}

int finish_device_load(vvli_gpu_model* m, DeviceSink& sink, int rc, vvli_gpu_model** out) {
    hipError_t e = hipStreamSynchronize(m->stream);
    if (sink.staging) (void)hipFree(sink.staging);
    if (rc == VVLI_OK && e != hipSuccess) rc = set_error(VVLI_HIP_ERROR, "device load: %s", hipGetErrorString(e));
    if (rc != VVLI_OK) {
        free_model(m);
        return rc;
    }
    *out = m;
    return VVLI_OK;
}

}  // namespace

extern "C" {

int vvli_gpu_model_create_from_safetensors(const vvli_gpu_config* cfg, uint32_t max_seq_len, const void* bytes,
                                           size_t len, vvli_host_progress_fn progress, void* user,
                                           vvli_gpu_model** out) {
    clear_error();
    if (!cfg || !bytes || !out) return set_error(VVLI_NULL_ARG, "NULL argument to vvli_gpu_model_create_from_safetensors");
    vvli_gpu_model* m = nullptr;
    int rc = create_impl(cfg, max_seq_len, nullptr, 0, &m, false, true);
    if (rc) return rc;
    DeviceSink sink{m};
    rc = load_safetensors_into(*cfg, bytes, len, device_put, &sink, progress, user);
    return finish_device_load(m, sink, rc, out);
}

int vvli_gpu_model_create_from_gguf(const void* bytes, size_t len, uint32_t weight_kind, uint32_t max_seq_len,
                                    vvli_host_progress_fn progress, void* user, vvli_gpu_config* cfg_out,
                                    vvli_gpu_model** out) {
    clear_error();
    if (!bytes || !out) return set_error(VVLI_NULL_ARG, "NULL argument to vvli_gpu_model_create_from_gguf");
    vvli_gpu_config cfg;
    int rc = gguf_config(bytes, len, weight_kind, cfg);
    if (rc) return rc;
    vvli_gpu_model* m = nullptr;
    if ((rc = create_impl(&cfg, max_seq_len, nullptr, 0, &m, false, true))) return rc;
    DeviceSink sink{m};
    rc = load_gguf_into(cfg, bytes, len, device_put, &sink, progress, user);
    if (rc == VVLI_OK && cfg_out) *cfg_out = cfg;
    return finish_device_load(m, sink, rc, out);
}

int vvli_gpu_read_weights(vvli_gpu_model* m, uint64_t elem_offset, uint64_t n, void* out) {
    if (!m || !out) return set_error(VVLI_NULL_ARG, "NULL argument to vvli_gpu_read_weights");
    if (elem_offset > m->layout.total || n > m->layout.total - elem_offset)
        return set_error(VVLI_INVALID_CONFIG, "weights [%llu, +%llu) outside the blob of %zu elements",
                         static_cast<unsigned long long>(elem_offset), static_cast<unsigned long long>(n),
                         m->layout.total);
    HIP_TRY(hipSetDevice(m->device));
    RESIDENT_STOP(m);
    HIP_TRY(hipMemcpy(out, m->blob + elem_offset * m->ebytes, n * m->ebytes, hipMemcpyDeviceToHost));
    return VVLI_OK;
}

int vvli_gpu_moe_model_create(const vvli_gpu_config* cfg, uint32_t max_seq_len, const void* host_blob,
                              size_t blob_elems, vvli_gpu_model** out) {
    clear_error();
    return create_impl(cfg, max_seq_len, host_blob, blob_elems, out, true);
}

int vvli_gpu_model_destroy(vvli_gpu_model* model) {
    if (!model) return set_error(VVLI_NULL_ARG, "model is NULL");
    (void)hipSetDevice(model->device);
    (void)resident_stop(model);
    (void)hipStreamSynchronize(model->stream);
    free_model(model);
    return VVLI_OK;
}

int vvli_gpu_kv_clear(vvli_gpu_model* m) {
    if (!m) return set_error(VVLI_NULL_ARG, "model is NULL");
    HIP_TRY(hipSetDevice(m->device));
    RESIDENT_STOP(m);
    const size_t kvlen = static_cast<size_t>(m->cfg.layers) * m->max_seq * kv_dim(m->cfg);
    HIP_TRY(hipMemsetAsync(m->kcache, 0, kvlen * sizeof(float), m->stream));
    HIP_TRY(hipMemsetAsync(m->vcache, 0, kvlen * sizeof(float), m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return VVLI_OK;
}

int vvli_gpu_set_rope_table(vvli_gpu_model* m, const float* inv_freq, uint32_t n) {
    if (!m) return set_error(VVLI_NULL_ARG, "model is NULL");
    HIP_TRY(hipSetDevice(m->device));
    RESIDENT_STOP(m);
    const uint32_t half = head_dim(m->cfg) / 2;
    if (inv_freq && n != half) return set_error(VVLI_INVALID_CONFIG, "rope table needs %u entries, got %u", half, n);
    if (inv_freq)
        m->inv_freq.assign(inv_freq, inv_freq + n);
    else
        m->inv_freq.clear();
    HIP_TRY(hipStreamSynchronize(m->stream));
    return upload_rope(m);
}

int vvli_gpu_forward_token(vvli_gpu_model* m, uint32_t token, uint32_t pos, float* logits_out, uint32_t* argmax_out) {
    if (!m) return set_error(VVLI_NULL_ARG, "model is NULL");
    if (token >= m->cfg.vocab) return set_error(VVLI_INVALID_TOKEN, "token %u >= vocab %u", token, m->cfg.vocab);
    if (pos >= m->max_seq) return set_error(VVLI_CONTEXT_FULL, "pos %u >= max_seq_len %u", pos, m->max_seq);
    HIP_TRY(hipSetDevice(m->device));
    if (use_persistent(m)) {
        if (m->res_linger_us) return forward_resident(m, token, pos, logits_out, argmax_out);
        const SingleStep one{token, pos};
        int rc = run_persistent(m, 1, -1, nullptr, 0, nullptr, &one);
        if (rc) return rc;
        return read_single(m, logits_out, argmax_out);
    }
    int rc = ensure_graph(m);
    if (rc) return rc;
    HIP_TRY(launch_set_state(m->state, token, pos, 0, 0, m->stream));
    HIP_TRY(hipGraphLaunch(m->graph, m->stream));
    return read_outputs(m, logits_out, argmax_out);
}

int vvli_gpu_forward_token_view(vvli_gpu_model* m, uint32_t token, uint32_t pos, const float** logits_view,
                                uint32_t* argmax_out) {
    if (!m || !logits_view) return set_error(VVLI_NULL_ARG, "NULL argument to vvli_gpu_forward_token_view");
    if (!m->h_logits) {
        HIP_TRY(hipSetDevice(m->device));
        if (hipHostMalloc(reinterpret_cast<void**>(&m->h_logits), static_cast<size_t>(m->cfg.vocab) * sizeof(float),
                          hipHostMallocCoherent) != hipSuccess) {
            m->h_logits = nullptr;
            return set_error(VVLI_OUT_OF_MEMORY, "hipHostMalloc of the logits view failed");
        }
    }
    // A copy into pinned memory is a direct DMA (measured per call at
    // Llama-1B: 793-803 against 817-855 us into pageable memory).
    const int rc = vvli_gpu_forward_token(m, token, pos, m->h_logits, argmax_out);
    if (rc) return rc;
    *logits_view = m->h_logits;
    return VVLI_OK;
}

int vvli_gpu_set_decode_path(vvli_gpu_model* m, uint32_t path) {
    if (!m) return set_error(VVLI_NULL_ARG, "model is NULL");
    if (path > 2) return set_error(VVLI_INVALID_CONFIG, "decode path %u not in 0..2", path);
    if (path == 2 && !m->mk_ok)
        return set_error(VVLI_INVALID_CONFIG, "persistent decode step unavailable (bf16 weights, fits one CU)");
    HIP_TRY(hipSetDevice(m->device));
    RESIDENT_STOP(m);
    m->path = path;
    return VVLI_OK;
}

int vvli_gpu_set_resident(vvli_gpu_model* m, uint32_t linger_us) {
    if (!m) return set_error(VVLI_NULL_ARG, "model is NULL");
    if (linger_us > kMaxResidentLingerUs)
        return set_error(VVLI_INVALID_CONFIG, "linger %u us over %u", linger_us, kMaxResidentLingerUs);
    HIP_TRY(hipSetDevice(m->device));
    RESIDENT_STOP(m);
    m->res_linger_us = linger_us;
    return VVLI_OK;
}

int vvli_gpu_set_prefill_path(vvli_gpu_model* m, uint32_t path) {
    if (!m) return set_error(VVLI_NULL_ARG, "model is NULL");
    if (path > 2) return set_error(VVLI_INVALID_CONFIG, "prefill path %u not in 0..2", path);
    if (path == 2 && !prefill_supported(m->cfg))
        return set_error(VVLI_INVALID_CONFIG, "batched prefill needs bf16 weights and head_dim 32, 64 or 128");
    m->prefill_path = path;
    return VVLI_OK;
}

int vvli_gpu_forward_embedding(vvli_gpu_model* m, const float* embedding, uint32_t pos, float* logits_out,
                               uint32_t* argmax_out) {
    if (!m || !embedding) return set_error(VVLI_NULL_ARG, "NULL argument to vvli_gpu_forward_embedding");
    if (pos >= m->max_seq) return set_error(VVLI_CONTEXT_FULL, "pos %u >= max_seq_len %u", pos, m->max_seq);
    HIP_TRY(hipSetDevice(m->device));
    RESIDENT_STOP(m);
    HIP_TRY(hipMemcpyAsync(m->x, embedding, m->cfg.hidden * sizeof(float), hipMemcpyHostToDevice, m->stream));
    HIP_TRY(launch_set_state(m->state, 0, pos, 0, 0, m->stream));
    int rc = enqueue_body(m, m->stream, nullptr);
    if (rc) return rc;
    return read_outputs(m, logits_out, argmax_out);
}

int vvli_gpu_forward_token_debug(vvli_gpu_model* m, uint32_t token, uint32_t pos, float* logits_out,
                                 float* hidden_out) {
    if (!m) return set_error(VVLI_NULL_ARG, "model is NULL");
    if (token >= m->cfg.vocab) return set_error(VVLI_INVALID_TOKEN, "token %u >= vocab %u", token, m->cfg.vocab);
    if (pos >= m->max_seq) return set_error(VVLI_CONTEXT_FULL, "pos %u >= max_seq_len %u", pos, m->max_seq);
    HIP_TRY(hipSetDevice(m->device));
    RESIDENT_STOP(m);
    HIP_TRY(launch_set_state(m->state, token, pos, 0, 0, m->stream));
    // The path forward_token takes: the persistent step's down-projection
    // phases write the residual rows, or the per-kernel step runs eagerly.
    int rc = use_persistent(m) ? run_persistent(m, 1, -1, nullptr, 0, m->hidden) : enqueue_step(m, m->stream, m->hidden);
    if (rc) return rc;
    if (hidden_out)
        HIP_TRY(hipMemcpyAsync(hidden_out, m->hidden, static_cast<size_t>(m->cfg.layers) * m->cfg.hidden * sizeof(float),
                               hipMemcpyDeviceToHost, m->stream));
    return read_outputs(m, logits_out, nullptr);
}

int vvli_gpu_profile_step(vvli_gpu_model* m, uint32_t token, uint32_t pos, float* ms_out, uint32_t cap,
                          uint32_t* n_out) {
    if (!m || !ms_out || !n_out) return set_error(VVLI_NULL_ARG, "NULL argument to vvli_gpu_profile_step");
    if (token >= m->cfg.vocab) return set_error(VVLI_INVALID_TOKEN, "token %u >= vocab %u", token, m->cfg.vocab);
    if (pos >= m->max_seq) return set_error(VVLI_CONTEXT_FULL, "pos %u >= max_seq_len %u", pos, m->max_seq);
    HIP_TRY(hipSetDevice(m->device));
    RESIDENT_STOP(m);
    HIP_TRY(launch_set_state(m->state, token, pos, 0, 0, m->stream));
    std::vector<std::pair<hipEvent_t, hipEvent_t>> evs;
    g_launch_events = &evs;
    int rc = enqueue_step(m, m->stream, nullptr);
    g_launch_events = nullptr;
    hipError_t e = hipStreamSynchronize(m->stream);
    uint32_t n = 0;
    if (rc == VVLI_OK && e == hipSuccess) {
        for (size_t i = 0; i < evs.size() && n < cap; ++i, ++n) {
            float ms = 0.f;
            e = hipEventElapsedTime(&ms, evs[i].first, evs[i].second);
            if (e != hipSuccess) break;
            ms_out[n] = ms;
        }
    }
    for (auto& ev : evs) {
        (void)hipEventDestroy(ev.first);
        (void)hipEventDestroy(ev.second);
    }
    if (rc) return rc;
    HIP_TRY(e);
    *n_out = n;
    return VVLI_OK;
}

int vvli_gpu_profile_persistent(vvli_gpu_model* m, uint32_t token, uint32_t pos, uint64_t* ticks_out,
                                uint32_t stride, uint32_t* n_blocks) {
    if (!m || !ticks_out || !n_blocks) return set_error(VVLI_NULL_ARG, "NULL argument to vvli_gpu_profile_persistent");
    if (!m->mk_ok) return set_error(VVLI_INVALID_CONFIG, "persistent decode step unavailable for this model");
    if (token >= m->cfg.vocab) return set_error(VVLI_INVALID_TOKEN, "token %u >= vocab %u", token, m->cfg.vocab);
    if (pos >= m->max_seq) return set_error(VVLI_CONTEXT_FULL, "pos %u >= max_seq_len %u", pos, m->max_seq);
    HIP_TRY(hipSetDevice(m->device));
    RESIDENT_STOP(m);
    const size_t n = static_cast<size_t>(m->mk_blocks + 1) * stride;
    unsigned long long* d = nullptr;
    HIP_TRY(hipMalloc(reinterpret_cast<void**>(&d), n * sizeof(unsigned long long)));
    hipError_t e = hipMemsetAsync(d, 0, n * sizeof(unsigned long long), m->stream);
    int rc = e == hipSuccess ? VVLI_OK : set_error(VVLI_HIP_ERROR, "memset: %s", hipGetErrorString(e));
    if (!rc) rc = launch_set_state(m->state, token, pos, 0, 0, m->stream) == hipSuccess ? VVLI_OK
                                                                                       : set_error(VVLI_HIP_ERROR, "set_state");
    if (!rc) rc = run_persistent(m, 1, -1, d, stride);
    if (!rc) {
        e = hipMemcpyAsync(ticks_out, d, n * sizeof(unsigned long long), hipMemcpyDeviceToHost, m->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
        if (e != hipSuccess) rc = set_error(VVLI_HIP_ERROR, "profile readback: %s", hipGetErrorString(e));
    }
    if (!rc) rc = check_persistent_error(m);
    (void)hipFree(d);
    if (rc) return rc;
    *n_blocks = m->mk_blocks;
    return VVLI_OK;
}

int vvli_gpu_last_launch_time(vvli_gpu_model* m, float* ms_out) {
    if (!m || !ms_out) return set_error(VVLI_NULL_ARG, "NULL argument to vvli_gpu_last_launch_time");
    if (!m->mk_timed) return set_error(VVLI_INVALID_CONFIG, "no timed persistent launch has run on this model");
    HIP_TRY(hipSetDevice(m->device));
    HIP_TRY(hipEventSynchronize(m->mk_ev1));
    HIP_TRY(hipEventElapsedTime(ms_out, m->mk_ev0, m->mk_ev1));
    return VVLI_OK;
}

int vvli_gpu_test_inject_step_error(vvli_gpu_model* m, uint32_t n) {
    if (!m) return set_error(VVLI_NULL_ARG, "model is NULL");
    HIP_TRY(hipSetDevice(m->device));
    RESIDENT_STOP(m);  // the flag is raised before the next launch
    m->mk_inject = n;
    return VVLI_OK;
}

int vvli_gpu_test_set_prefill_attention_form(int32_t form) {
    if (form < -1 || form > 2) return set_error(VVLI_INVALID_CONFIG, "attention form %d not in -1..2", form);
    prefill_fa_form.store(form, std::memory_order_relaxed);
    return VVLI_OK;
}

int vvli_gpu_kv_read(vvli_gpu_model* m, uint32_t layer, uint32_t pos, float* k_out, float* v_out) {
    if (!m) return set_error(VVLI_NULL_ARG, "model is NULL");
    if (layer >= m->cfg.layers || pos >= m->max_seq)
        return set_error(VVLI_INVALID_CONFIG, "layer %u / pos %u out of range", layer, pos);
    HIP_TRY(hipSetDevice(m->device));
    RESIDENT_STOP(m);
    const size_t kv = kv_dim(m->cfg);
    const size_t off = (static_cast<size_t>(layer) * m->max_seq + pos) * kv;
    if (k_out)
        HIP_TRY(hipMemcpyAsync(k_out, m->kcache + off, kv * sizeof(float), hipMemcpyDeviceToHost, m->stream));
    if (v_out)
        HIP_TRY(hipMemcpyAsync(v_out, m->vcache + off, kv * sizeof(float), hipMemcpyDeviceToHost, m->stream));
    HIP_TRY(hipStreamSynchronize(m->stream));
    return VVLI_OK;
}

int vvli_gpu_prefill(vvli_gpu_model* m, const uint32_t* tokens, uint32_t n, uint32_t start_pos, float* last_logits,
                     uint32_t* argmax_out) {
    if (!m || !tokens) return set_error(VVLI_NULL_ARG, "NULL argument to vvli_gpu_prefill");
    if (n == 0) return set_error(VVLI_EMPTY_PROMPT, "empty prompt");
    for (uint32_t i = 0; i < n; ++i)
        if (tokens[i] >= m->cfg.vocab) return set_error(VVLI_INVALID_TOKEN, "token %u >= vocab", tokens[i]);
    if (static_cast<uint64_t>(start_pos) + n > m->max_seq)
        return set_error(VVLI_CONTEXT_FULL, "prefill end %u > max_seq_len %u", start_pos + n, m->max_seq);
    HIP_TRY(hipSetDevice(m->device));
    RESIDENT_STOP(m);
    // Prompt tokens live at their absolute positions in `prompt`.
    HIP_TRY(hipMemcpyAsync(m->prompt + start_pos, tokens, n * sizeof(uint32_t), hipMemcpyHostToDevice, m->stream));
    if (use_batched_prefill(m)) {
        int rc = enqueue_prefill_batched(m, start_pos, n, tokens[n - 1], 0);
        if (rc) return rc;
        return read_outputs(m, last_logits, argmax_out);
    }
    HIP_TRY(launch_set_state(m->state, tokens[0], start_pos, start_pos + n, 0, m->stream));
    if (use_persistent(m)) {
        int rc = run_persistent(m, n, -1);
        if (rc) return rc;
        return read_outputs(m, last_logits, argmax_out);
    }
    int rc = ensure_graph(m);
    if (rc) return rc;
    for (uint32_t i = 0; i < n; ++i) HIP_TRY(hipGraphLaunch(m->graph, m->stream));
    return read_outputs(m, last_logits, argmax_out);
}

int vvli_gpu_generate_greedy(vvli_gpu_model* m, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                             int64_t eos, uint32_t flags, uint32_t* out_tokens, uint32_t* n_out,
                             vvli_gpu_stats* stats) {
    if (!m || !out_tokens || !n_out) return set_error(VVLI_NULL_ARG, "NULL argument to vvli_gpu_generate_greedy");
    if (n_prompt == 0 || !prompt) return set_error(VVLI_EMPTY_PROMPT, "empty prompt");  // generator.zig:230
    for (uint32_t i = 0; i < n_prompt; ++i)
        if (prompt[i] >= m->cfg.vocab) return set_error(VVLI_INVALID_TOKEN, "prompt token %u >= vocab", prompt[i]);
    if (n_prompt > m->max_seq)
        return set_error(VVLI_CONTEXT_FULL, "prompt of %u tokens > max_seq_len %u", n_prompt, m->max_seq);
    const bool batched = (flags & VVLI_GEN_BATCHED_PREFILL) && use_batched_prefill(m);
    HIP_TRY(hipSetDevice(m->device));
    RESIDENT_STOP(m);
    if (use_persistent(m))
        return generate_persistent(m, prompt, n_prompt, max_new, eos, batched, out_tokens, n_out, stats);
    int rc = ensure_graph(m);
    if (rc) return rc;
    const int64_t t0 = now_ns();
    // Prefill: batched, or one step per prompt token chained on the device.
    HIP_TRY(hipMemcpyAsync(m->prompt, prompt, n_prompt * sizeof(uint32_t), hipMemcpyHostToDevice, m->stream));
    if (batched) {
        if ((rc = enqueue_prefill_batched(m, 0, n_prompt, prompt[n_prompt - 1], 1))) return rc;
    } else {
        HIP_TRY(launch_set_state(m->state, prompt[0], 0, n_prompt, 1, m->stream));
        for (uint32_t i = 0; i < n_prompt; ++i) HIP_TRY(hipGraphLaunch(m->graph, m->stream));
    }
    HIP_TRY(hipStreamSynchronize(m->stream));
    const int64_t t1 = now_ns();
    // Decode: out[0] is the argmax of the last prompt step. Each step
    // forwards the last emitted token (the last one too, generator.zig:272).
    uint32_t produced = 0;
    if (max_new > 0) {
        if (eos < 0) {
            if (static_cast<uint64_t>(n_prompt) + max_new > m->max_seq)
                return set_error(VVLI_CONTEXT_FULL, "prompt %u + %u new tokens > max_seq_len %u", n_prompt, max_new,
                                 m->max_seq);
            for (uint32_t i = 0; i < max_new; ++i) HIP_TRY(hipGraphLaunch(m->graph, m->stream));
            produced = max_new;
        } else {
            uint32_t pos = n_prompt;
            while (produced < max_new) {
                HIP_TRY(hipMemcpyAsync(m->h_state, m->state, sizeof(StepState), hipMemcpyDeviceToHost, m->stream));
                HIP_TRY(hipStreamSynchronize(m->stream));
                const uint32_t next = m->h_state->argmax;
                ++produced;
                if (static_cast<int64_t>(next) == eos) break;
                if (pos >= m->max_seq) return set_error(VVLI_CONTEXT_FULL, "pos %u >= max_seq_len", pos);
                HIP_TRY(hipGraphLaunch(m->graph, m->stream));
                ++pos;
            }
        }
        HIP_TRY(hipMemcpyAsync(out_tokens, m->out_tokens, produced * sizeof(uint32_t), hipMemcpyDeviceToHost,
                               m->stream));
    }
    HIP_TRY(hipStreamSynchronize(m->stream));
    const int64_t t2 = now_ns();
    *n_out = produced;
    if (stats) {
        stats->prompt_tokens = n_prompt;
        stats->generated_tokens = produced;
        stats->prefill_ns = t1 - t0;
        stats->decode_ns = t2 - t1;
        stats->total_ns = t2 - t0;
    }
    return VVLI_OK;
}

int vvli_gpu_generate(vvli_gpu_model* m, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new, int64_t eos,
                      uint32_t flags, const vvli_gpu_sampling* opts, uint32_t* out_tokens, uint32_t* n_out,
                      vvli_gpu_stats* stats) {
    if (!m || !out_tokens || !n_out || !opts) return set_error(VVLI_NULL_ARG, "NULL argument to vvli_gpu_generate");
    if (n_prompt == 0 || !prompt) return set_error(VVLI_EMPTY_PROMPT, "empty prompt");
    int rc = validate_sampling(*opts, m->cfg.vocab);
    if (rc) return rc;
    // Greedy without a penalty is llm.argmax: the greedy path (persistent step where available).
    if (opts->temperature <= 0.0f && !(opts->repeat_penalty > 1.0f && opts->repeat_last_n > 0))
        return vvli_gpu_generate_greedy(m, prompt, n_prompt, max_new, eos, flags, out_tokens, n_out, stats);
    for (uint32_t i = 0; i < n_prompt; ++i)
        if (prompt[i] >= m->cfg.vocab) return set_error(VVLI_INVALID_TOKEN, "prompt token %u >= vocab", prompt[i]);
    if (n_prompt > m->max_seq)
        return set_error(VVLI_CONTEXT_FULL, "prompt of %u tokens > max_seq_len %u", n_prompt, m->max_seq);
    HIP_TRY(hipSetDevice(m->device));
    RESIDENT_STOP(m);
    const bool batched = (flags & VVLI_GEN_BATCHED_PREFILL) && use_batched_prefill(m);
    return generate_sampled(m, prompt, n_prompt, max_new, eos, batched, *opts, out_tokens, n_out, stats);
}

int vvli_gpu_test_sampler_trace(const float* logits, uint32_t n, const vvli_gpu_sampling* opts,
                                uint64_t prng_state[4], uint32_t* token_out, uint32_t* ids_out, float* probs_out,
                                float* sums_out, uint32_t* count_out) {
    if (!logits || !opts || !prng_state || !token_out || !ids_out || !probs_out || !sums_out || !count_out)
        return set_error(VVLI_NULL_ARG, "NULL argument to vvli_gpu_test_sampler_trace");
    if (n == 0) return set_error(VVLI_INVALID_CONFIG, "empty logits");
    clear_error();
    int rc = validate_sampling(*opts, n);
    if (rc) return rc;
    const uint32_t limit = (opts->top_k == 0 || opts->top_k > n) ? n : opts->top_k;
    if (!(opts->temperature > 0.0f) || limit <= static_cast<uint32_t>(kMaxSampleTopK))
        return set_error(VVLI_INVALID_CONFIG, "the trace covers the whole-vocabulary path (T > 0, over %d candidates)",
                         kMaxSampleTopK);
    const size_t full_bytes = sample_full_bytes(n);
    void* d_full = nullptr;
    float *d_logits = nullptr, *d_probs = nullptr, *d_sums = nullptr;
    uint32_t *d_ids = nullptr, *d_result = nullptr, *d_count = nullptr;
    unsigned long long* d_prng = nullptr;
    hipError_t e = hipMalloc(&d_full, full_bytes);
    if (e == hipSuccess) e = hipMalloc(&d_logits, n * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&d_probs, n * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&d_sums, n * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&d_ids, n * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&d_result, sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&d_count, sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&d_prng, 4 * sizeof(unsigned long long));
    if (e == hipSuccess) e = hipMemcpy(d_logits, logits, n * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(d_prng, prng_state, 4 * sizeof(uint64_t), hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        SampleArgs sa;
        sa.logits = d_logits;
        sa.vocab = n;
        sa.temperature = opts->temperature;
        sa.top_p = opts->top_p;
        sa.repeat_penalty = opts->repeat_penalty;
        sa.top_k = limit;
        sa.repeat_last_n = opts->repeat_last_n;
        sa.prng = d_prng;
        sa.result = d_result;
        sa.full = d_full;
        sa.trace_ids = d_ids;
        sa.trace_probs = d_probs;
        sa.trace_sums = d_sums;
        sa.trace_count = d_count;
        e = launch_sample(sa, nullptr);
    }
    uint32_t count = 0;
    if (e == hipSuccess) e = hipMemcpy(&count, d_count, sizeof(uint32_t), hipMemcpyDeviceToHost);
    if (e == hipSuccess && count > n) e = hipErrorUnknown;
    if (e == hipSuccess && count) e = hipMemcpy(ids_out, d_ids, count * sizeof(uint32_t), hipMemcpyDeviceToHost);
    if (e == hipSuccess && count) e = hipMemcpy(probs_out, d_probs, count * sizeof(float), hipMemcpyDeviceToHost);
    if (e == hipSuccess && count) e = hipMemcpy(sums_out, d_sums, count * sizeof(float), hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(token_out, d_result, sizeof(uint32_t), hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(prng_state, d_prng, 4 * sizeof(uint64_t), hipMemcpyDeviceToHost);
    *count_out = count;
    for (void* q : {static_cast<void*>(d_full), static_cast<void*>(d_logits), static_cast<void*>(d_probs),
                    static_cast<void*>(d_sums), static_cast<void*>(d_ids), static_cast<void*>(d_result),
                    static_cast<void*>(d_count), static_cast<void*>(d_prng)})
        if (q) (void)hipFree(q);
    if (e != hipSuccess)
        return set_error(e == hipErrorOutOfMemory ? VVLI_OUT_OF_MEMORY : VVLI_HIP_ERROR, "sampler trace: %s",
                         hipGetErrorString(e));
    return VVLI_OK;
}

void vvli_gpu_prng_seed(uint64_t seed, uint64_t state_out[4]) {
    if (state_out) prng_seed(seed, state_out);
}

int vvli_gpu_sampler_next(const float* logits, uint32_t n, const uint32_t* prompt, uint32_t n_prompt,
                          const uint32_t* generated, uint32_t n_generated, const vvli_gpu_sampling* opts,
                          uint64_t prng_state[4], uint32_t* token_out) {
    if (!logits || !opts || !prng_state || !token_out || (n_prompt && !prompt) || (n_generated && !generated))
        return set_error(VVLI_NULL_ARG, "NULL argument to vvli_gpu_sampler_next");
    if (n == 0) return set_error(VVLI_INVALID_CONFIG, "empty logits");
    clear_error();
    int rc = validate_sampling(*opts, n);
    if (rc) return rc;
    // buildRepeatCounts (src/generator.zig:335-351) on the host.
    std::vector<uint32_t> counts(n, 0);
    const bool penalty = opts->repeat_penalty > 1.0f && opts->repeat_last_n > 0;
    if (penalty) {
        const uint64_t total = static_cast<uint64_t>(n_prompt) + n_generated;
        const uint64_t start = total > opts->repeat_last_n ? total - opts->repeat_last_n : 0;
        for (uint64_t i = start; i < total; ++i) {
            const uint32_t t = i < n_prompt ? prompt[i] : generated[i - n_prompt];
            if (t < n && counts[t] < 0xffff) ++counts[t];
        }
    }
    float* d_logits = nullptr;
    uint32_t *d_counts = nullptr, *d_result = nullptr, *d_nf = nullptr;
    unsigned long long *d_prng = nullptr, *d_cand = nullptr;
    void* d_full = nullptr;
    const uint32_t limit = (opts->top_k == 0 || opts->top_k > n) ? n : opts->top_k;
    const bool full = opts->temperature > 0.0f && limit > static_cast<uint32_t>(kMaxSampleTopK);
    const size_t full_bytes = full ? sample_full_bytes(n) : 0;
    if (full && full_bytes == 0) return set_error(VVLI_HIP_ERROR, "sort storage size query failed");
    auto release = [&] {
        if (d_full) (void)hipFree(d_full);
        if (d_logits) (void)hipFree(d_logits);
        if (d_counts) (void)hipFree(d_counts);
        if (d_result) (void)hipFree(d_result);
        if (d_prng) (void)hipFree(d_prng);
        if (d_cand) (void)hipFree(d_cand);
        if (d_nf) (void)hipFree(d_nf);
    };
    hipError_t e = hipMalloc(&d_logits, n * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&d_cand, sample_cand_elems(n) * sizeof(unsigned long long));
    if (e == hipSuccess) e = hipMalloc(&d_nf, sample_nf_elems(n) * sizeof(uint32_t));
    if (e == hipSuccess && full) e = hipMalloc(&d_full, full_bytes);
    if (e == hipSuccess) e = hipMalloc(&d_counts, n * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&d_result, sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&d_prng, 4 * sizeof(unsigned long long));
    if (e == hipSuccess) e = hipMemcpy(d_logits, logits, n * sizeof(float), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(d_counts, counts.data(), n * sizeof(uint32_t), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(d_prng, prng_state, 4 * sizeof(uint64_t), hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        SampleArgs sa;
        sa.logits = d_logits;
        sa.vocab = n;
        sa.counts = penalty ? d_counts : nullptr;
        sa.temperature = opts->temperature;
        sa.top_p = opts->top_p;
        sa.repeat_penalty = opts->repeat_penalty;
        sa.top_k = (opts->top_k == 0 || opts->top_k > n) ? n : opts->top_k;
        sa.repeat_last_n = opts->repeat_last_n;
        sa.prng = d_prng;
        sa.result = d_result;
        sa.cand_buf = d_cand;
        sa.cand_nf = d_nf;
        sa.full = d_full;
        e = launch_sample(sa, nullptr);
    }
    if (e == hipSuccess) e = hipMemcpy(token_out, d_result, sizeof(uint32_t), hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(prng_state, d_prng, 4 * sizeof(uint64_t), hipMemcpyDeviceToHost);
    release();
    if (e != hipSuccess)
        return set_error(e == hipErrorOutOfMemory ? VVLI_OUT_OF_MEMORY : VVLI_HIP_ERROR, "sampler: %s",
                         hipGetErrorString(e));
    return VVLI_OK;
}

}  // extern "C"
