/*
 * vvli_oracle.h -- CPU restatement of VVLI's dense-decoder forward pass.
 *
 * TEST INFRASTRUCTURE ONLY. This library gives the reference results the
 * MI355X library (libvvli_gpu.so) is tested against, and the timed CPU
 * baseline in bench.py. Nothing in the product path links, loads or calls it.
 *
 * Every function restates a function of the reference (risingsunomi/vvli,
 * Zig) and cites the file:line it follows. Operation order is kept where it
 * changes rounding: x*w*s in RMSNorm, f32 pow -> angle -> cos/sin in RoPE,
 * two-pass softmax with a 1/sum multiply, sequential p*V accumulation over t,
 * simd-lane vector accumulators followed by an in-order lane reduction and a
 * fused-multiply-add scalar tail in the dot products.
 *
 * Pinning status (what checks each function; see tests/test_oracle_*.py):
 *   f32<->bf16, storage layout, param counts  : reference known answers + closed forms
 *   linear/dot                                : f64 brute force, reference matmul known answer
 *   rmsnorm                                   : reference known answer ([3,4] -> ...)
 *   rope                                      : reference known answer (pos 1, hd 4) + f64 closed form
 *   softmax / attention                       : reference softmax known answers + f64 brute force
 *   silu-mul, add, argmax                     : closed forms, tie/NaN special cases
 *   whole forward (split-half, interleaved)   : HF transformers f32 golden fixtures (tests/golden)
 *   greedy generator loop                     : token-by-token replay against orc_forward_token
 *   prompt pass (orc_prefill)                 : bit equality with the orc_forward_token loop
 * Bit-level agreement with Zig's std.math (pow/cos/sin/exp) and with the
 * host-dependent SIMD width is "parity unpinned"; tolerance-level parity is
 * pinned by the checks above.
 */
#ifndef VVLI_ORACLE_H
#define VVLI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes: same numbering as the GPU library's rc values. */
enum {
    ORC_OK = 0,
    ORC_INVALID_CONFIG = 1,
    ORC_INVALID_WEIGHT = 2,
    ORC_INVALID_TOKEN = 3,
    ORC_CONTEXT_FULL = 4,
    ORC_UNSUPPORTED_DTYPE = 5,
    ORC_UNSUPPORTED_ARCH = 6,
    ORC_OUT_OF_MEMORY = 7,
    ORC_THREAD_SPAWN_FAILED = 9,
    ORC_EMPTY_PROMPT = 10,
    ORC_INVALID_SAMPLING = 15,
    ORC_NULL_ARG = 100,
};

/* src/llm.zig:77-97 (Config) -- the fields the forward pass reads. */
typedef struct orc_config {
    uint32_t vocab, hidden, inter, layers, heads, kv_heads, max_pos;
    uint32_t rope_layout;   /* 0 interleaved, 1 split_half (src/llm.zig:50-53) */
    uint32_t weight_kind;   /* 0 f32, 1 bf16 (src/llm.zig:55-58) */
    uint32_t tie;           /* tie_word_embeddings */
    uint32_t qkv_bias;
    float rope_theta;
    float rms_eps;
} orc_config;

/* Blob slice offsets (in elements), src/llm.zig:488-522 assignSlices order. */
typedef struct orc_layer_offsets {
    size_t input_norm, q, q_bias, k, k_bias, v, v_bias, o, post_norm, gate, up, down;
} orc_layer_offsets;

/* ---- scalar helpers: src/llm.zig:791-803 ---- */
float orc_bf16_to_f32(uint16_t bits);
uint16_t orc_f32_to_bf16(float value);
float orc_f16_to_f32(uint16_t bits);

/* ---- config & layout: src/llm.zig:195-276, 488-537, 814-837 ---- */
int orc_config_validate(const orc_config* c);
size_t orc_parameter_count(const orc_config* c);
size_t orc_storage_element_count(const orc_config* c);
/* Fills per-layer offsets (array of c->layers) plus embed/final_norm/lm_head
 * offsets (lm_head = (size_t)-1 when tied). Returns storage element count. */
size_t orc_layout(const orc_config* c, orc_layer_offsets* layers, size_t* embed, size_t* final_norm,
                  size_t* lm_head);
/* src/llm.zig:466-477 fillDeterministicForTesting. */
void orc_fill_deterministic(void* blob, size_t n, uint32_t weight_kind);

/* ---- ops: src/llm.zig:1228-1466 ---- */
/* lanes = simd_lanes of the restated host (4 NEON, 8 AVX2, 16 AVX-512). */
void orc_linear(float* out, const void* w, uint32_t weight_kind, size_t rows, size_t cols, const float* x,
                const void* bias, int lanes);
/* Threaded variant: per-call thread spawn exactly as linearInto does. */
int orc_linear_threaded(float* out, const void* w, uint32_t weight_kind, size_t rows, size_t cols,
                        const float* x, const void* bias, int lanes, int threads, int min_rows);
void orc_rmsnorm(float* out, const float* x, const void* w, uint32_t weight_kind, size_t n, float eps, int lanes);
/* src/tensor.zig:683-733 matmulBlocked (f32): out[m][n] = a[m][k] . b[k][n],
 * columns in panels of 4 vectors of `lanes`, each accumulated over p in order
 * (unfused multiply, then add), then whole vectors, then a scalar @mulAdd tail. */
void orc_matmul_blocked(float* out, const float* a, size_t m, size_t k, const float* b, size_t n, int lanes);
/* inv_freq may be NULL: then the reference formula 1/pow(theta, d/hd) is used. */
void orc_rope(float* values, size_t heads, size_t head_dim, size_t pos, float theta, uint32_t layout,
              const float* inv_freq);
/* Llama-3 scaled frequency table (head_dim/2 values; no reference counterpart,
 * the published Llama-3 closed form applied to the reference's f32 table).
 * Returns ORC_INVALID_CONFIG for bad parameters. */
int orc_llama3_inv_freq(uint32_t head_dim, float theta, float factor, float low_freq_factor, float high_freq_factor,
                        uint32_t original_max_pos, float* out);
void orc_softmax(float* values, size_t n);
/* q: heads*hd; keys/values: [T][kv_heads*hd] rows for t = 0..pos. */
void orc_attention(float* out, const float* q, const float* keys, const float* values, size_t heads,
                   size_t kv_heads, size_t head_dim, size_t pos, float* scores, int lanes);
void orc_silu_mul(float* out, const float* gate, const float* up, size_t n);
void orc_add(float* out, const float* a, const float* b, size_t n);
size_t orc_argmax(const float* logits, size_t n);
float orc_dot_f32(const float* a, const float* b, size_t n, int lanes);
float orc_dot_bf16(const uint16_t* a, const float* b, size_t n, int lanes);

/* ---- runner: src/llm.zig:539-776 ---- */
typedef struct orc_runner orc_runner;
/* blob is borrowed (not copied); it must outlive the runner. threads == 0 uses
 * the host CPU count (src/llm.zig:1277-1285). */
int orc_runner_create(const orc_config* c, const void* blob, size_t blob_elems, uint32_t max_seq_len, int threads,
                      int lanes, orc_runner** out);
void orc_runner_destroy(orc_runner* r);
void orc_kv_clear(orc_runner* r);
/* Override the RoPE frequency table (n == head_dim/2); NULL restores the formula. */
int orc_set_rope_table(orc_runner* r, const float* inv_freq, uint32_t n);
/* logits_out: vocab floats (nullable). hidden_out: layers*hidden floats, the
 * residual stream after each layer (nullable). */
int orc_forward_token(orc_runner* r, uint32_t token, uint32_t pos, float* logits_out, float* hidden_out);
int orc_forward_embedding(orc_runner* r, const float* embedding, uint32_t pos, float* logits_out,
                          float* hidden_out);
/* The prompt loop (src/generator.zig:243-251): tokens at positions
 * start_pos.. through every layer with the loops interchanged (weight rows
 * shared by blocks of tokens, attention spread over threads by token). KV
 * rows and the last token's logits are bit-identical to n orc_forward_token
 * calls (checked by tests/test_oracle.py). */
int orc_prefill(orc_runner* r, const uint32_t* tokens, uint32_t n, uint32_t start_pos, float* logits_out);
int orc_kv_read(const orc_runner* r, uint32_t layer, uint32_t pos, float* k_out, float* v_out);
/* Overwrite n cache rows pos.. of one layer (tests continuing from another
 * implementation's cache; not part of the reference's API). */
int orc_kv_write(orc_runner* r, uint32_t layer, uint32_t pos, uint32_t n, const float* k, const float* v);

/* ---- generator: src/generator.zig:142-175, 221-293 ---- */
typedef struct orc_stats {
    uint64_t prompt_tokens, generated_tokens;
    int64_t prefill_ns, decode_ns, total_ns;
} orc_stats;
/* eos < 0 disables EOS. Greedy (temperature 0, penalty 1). */
int orc_generate_greedy(orc_runner* r, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new, int64_t eos,
                        uint32_t* out_tokens, uint32_t* n_out, orc_stats* stats);

/* ---- mixture-of-experts step (vvli_oracle_moe.c; no reference counterpart:
 * HF OLMoE semantics, see that file's header) ---- */
typedef struct orc_moe_config {
    orc_config base;  /* inter = per-expert intermediate size */
    uint32_t experts, top_k, qk_norm;
} orc_moe_config;
typedef struct orc_moe_layer_offsets {
    size_t input_norm, q, q_bias, k, k_bias, v, v_bias, q_norm, k_norm, o, post_norm, router, gate_up, down;
} orc_moe_layer_offsets;
/* Blob: embed; per layer input_norm, q, (q_bias), k, (k_bias), v, (v_bias),
 * (q_norm [hidden], k_norm [kv]), o, post_norm, router [E][H], gate_up
 * [E][2I][H] (gate rows then up rows), down [E][H][I]; final_norm; lm_head
 * unless tied. Each slice 64-byte aligned. Returns the element count. */
size_t orc_moe_layout(const orc_moe_config* c, orc_moe_layer_offsets* layers, size_t* embed, size_t* final_norm,
                      size_t* lm_head);
void orc_moe_rmsnorm(float* out, const float* x, const void* w, uint32_t kind, size_t n, float eps);
void orc_moe_route(const float* logits, size_t n, size_t top_k, uint32_t* idx, float* weights);
/* The routed experts of one layer: moe[h] = sum over the selected experts in
 * ascending expert index of weight * W_down,e . (silu(W_g,e . x) * (W_u,e . x)),
 * x = the post-attention norm (hidden floats). gate_up / down: element offsets
 * of the layer's expert matrices in the blob. matmul = 0: each product as
 * linearInto (the runner's path); 1: as src/tensor.zig's matmul of the row x
 * with the expert matrix transposed to f32 [K][N] (matmulBlocked). */
int orc_moe_experts(float* moe, const void* blob, uint32_t kind, size_t gate_up, size_t down, const float* x,
                    size_t hidden, size_t inter, size_t experts, size_t top_k, const uint32_t* idx,
                    const float* weights, int lanes, int threads, int matmul);
typedef struct orc_moe_runner orc_moe_runner;
int orc_moe_runner_create(const orc_moe_config* c, const void* blob, size_t blob_elems, uint32_t max_seq_len,
                          int threads, int lanes, orc_moe_runner** out);
void orc_moe_runner_destroy(orc_moe_runner* r);
/* experts_out: layers*top_k selected expert ids (nullable). */
int orc_moe_forward_token(orc_moe_runner* r, uint32_t token, uint32_t pos, float* logits_out, float* hidden_out,
                          uint32_t* experts_out);
int orc_moe_kv_read(const orc_moe_runner* r, uint32_t layer, uint32_t pos, float* k_out, float* v_out);

/* ---- sampler pieces: src/generator.zig:338-463 ---- */
float orc_adjusted_logit(float logit, uint16_t repeat_count, float repeat_penalty);
uint32_t orc_greedy_with_penalties(const float* logits, const uint16_t* counts, size_t n, float repeat_penalty);

/* ---- token sampler (vvli_oracle_sample.c): src/generator.zig:14-23, 65-127,
 * 329-463; PRNG = Zig's DefaultPrng (xoshiro256++ / SplitMix64) ---- */
typedef struct orc_sampling {
    float temperature, top_p;
    uint32_t top_k;
    float repeat_penalty;
    uint32_t repeat_last_n;
    uint64_t seed;
} orc_sampling;
uint64_t orc_splitmix64_next(uint64_t* state);
void orc_prng_seed(uint64_t state[4], uint64_t seed);
uint64_t orc_prng_next(uint64_t state[4]);
float orc_prng_float(uint64_t state[4]);
int orc_sampling_validate(const orc_sampling* o);
void orc_build_repeat_counts(uint16_t* counts, size_t n, const uint32_t* prompt, size_t n_prompt,
                             const uint32_t* generated, size_t n_generated, const orc_sampling* o);
size_t orc_build_candidates(uint32_t* ids, float* scores, const float* logits, const uint16_t* counts, size_t n,
                            const orc_sampling* o);
size_t orc_prepare_probabilities(float* probs, const float* scores, size_t count, const orc_sampling* o);
uint32_t orc_sample_candidate(const uint32_t* ids, const float* probs, size_t count, float random_unit);
int orc_sampler_next(const float* logits, size_t n, const uint32_t* prompt, size_t n_prompt,
                     const uint32_t* generated, size_t n_generated, const orc_sampling* o, uint64_t prng[4],
                     uint32_t* token_out);
int orc_generate_sampled(orc_runner* r, size_t vocab, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                         int64_t eos, const orc_sampling* o, uint32_t* out_tokens, uint32_t* n_out);

#ifdef __cplusplus
}
#endif
#endif
