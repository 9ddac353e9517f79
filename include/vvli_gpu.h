/*
 * vvli_gpu.h -- C ABI of the MI355X (gfx950) dense-decoder forward pass.
 *
 * This is the drop-in boundary for VVLI's CPU runner. A Zig host binds it with
 * @cImport and keeps its runner/generator API; the
 * library holds the weights, the KV cache and all activations in HBM and runs
 * hand-written HIP kernels.
 *
 * Conventions (after src/gpu/metal_smoke.zig:5-11 and src/gpu/metal_smoke.m:23-29):
 *   - every entry point returns int: 0 on success, a VVLI_* code otherwise;
 *   - outputs go through caller-owned pointers; NULL required args -> VVLI_NULL_ARG;
 *   - vvli_gpu_last_error() gives a thread-local message for the last failure.
 * Threading: one model handle owns one HIP stream and admits one call at a
 * time; separate handles may be used from separate threads. Every call is
 * synchronous on return unless it says otherwise. The library starts no
 * host threads.
 */
#ifndef VVLI_GPU_H
#define VVLI_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VVLI_GPU_ABI_VERSION 1u

/* Return codes. Each maps one member of the reference's error sets
 * (src/llm.zig:17-27, src/generator.zig:8-12, src/gguf.zig:7-12). */
enum {
    VVLI_OK = 0,
    VVLI_INVALID_CONFIG = 1,        /* llm.Error.InvalidConfig */
    VVLI_INVALID_WEIGHT = 2,        /* llm.Error.InvalidWeight */
    VVLI_INVALID_TOKEN = 3,         /* llm.Error.InvalidToken */
    VVLI_CONTEXT_FULL = 4,          /* llm.Error.ContextFull */
    VVLI_UNSUPPORTED_DTYPE = 5,     /* llm.Error.UnsupportedDType */
    VVLI_UNSUPPORTED_ARCH = 6,      /* llm.Error.UnsupportedModelArchitecture */
    VVLI_OUT_OF_MEMORY = 7,         /* error.OutOfMemory (hipMalloc / host alloc) */
    VVLI_HIP_ERROR = 8,             /* HIP runtime failure (no reference counterpart) */
    VVLI_MISSING_FIELD = 9,         /* llm.Error.MissingJsonField */
    VVLI_EMPTY_PROMPT = 10,         /* generator.Error.EmptyPrompt */
    VVLI_MISSING_TENSOR = 11,       /* llm.Error.MissingSafetensorsTensor */
    VVLI_INVALID_FILE = 12,         /* gguf.Error.InvalidGguf / bad safetensors header / IO */
    VVLI_UNSUPPORTED_VERSION = 13,  /* gguf.Error.UnsupportedGgufVersion */
    VVLI_OUTPUT_TOO_SMALL = 14,     /* generator.Error.OutputTooSmall */
    VVLI_INVALID_SAMPLING = 15,     /* generator.Error.InvalidSamplingOptions */
    VVLI_UNSUPPORTED_METADATA = 16, /* gguf.Error.UnsupportedMetadataType */
    VVLI_NULL_ARG = 100             /* NULL required argument (metal_smoke.m:24) */
};

/* Enumerations (src/llm.zig:29-58). */
enum { VVLI_ARCH_LLAMA = 0, VVLI_ARCH_MISTRAL = 1, VVLI_ARCH_OLMOE = 2, VVLI_ARCH_QWEN2 = 3 };
enum { VVLI_ROPE_INTERLEAVED = 0, VVLI_ROPE_SPLIT_HALF = 1 };
enum { VVLI_WEIGHT_F32 = 0, VVLI_WEIGHT_BF16 = 1 };

/* Model shape contract: the fields of llm.Config (src/llm.zig:77-97). */
typedef struct vvli_gpu_config {
    uint32_t abi_version;     /* must be VVLI_GPU_ABI_VERSION */
    uint32_t arch;            /* VVLI_ARCH_* */
    uint32_t vocab, hidden, inter, layers, heads, kv_heads, max_pos;
    uint32_t rope_layout;     /* VVLI_ROPE_* */
    uint32_t weight_kind;     /* VVLI_WEIGHT_*: dtype of the blob */
    uint32_t num_experts, experts_per_tok; /* 0 for dense models */
    float rope_theta, rms_eps;
    uint8_t tie, qkv_bias, qk_norm, _pad;
    uint32_t eos_token_id, pad_token_id;
} vvli_gpu_config;

typedef struct vvli_gpu_model vvli_gpu_model;

/* Generation statistics: generator.Stats (src/generator.zig:25-43). */
typedef struct vvli_gpu_stats {
    uint64_t prompt_tokens, generated_tokens;
    int64_t prefill_ns, decode_ns, total_ns;
} vvli_gpu_stats;

/* ---------------------------------------------------------------------- */
/* Library                                                                 */
/* ---------------------------------------------------------------------- */
uint32_t vvli_gpu_abi_version(void);
/* Thread-local text for the last non-zero return on this thread. */
const char* vvli_gpu_last_error(void);

/* ---------------------------------------------------------------------- */
/* Shape contract (host only; no GPU needed)                               */
/* ---------------------------------------------------------------------- */
/* Config.validate, src/llm.zig:195-216. */
int vvli_gpu_config_validate(const vvli_gpu_config* cfg);
/* Config.parameterCount, src/llm.zig:241-276. */
uint64_t vvli_gpu_parameter_count(const vvli_gpu_config* cfg);
/* storageElementCount, src/llm.zig:814-837: elements of the contiguous blob
 * (dtype = cfg->weight_kind), every slice starting on a 64-byte boundary. */
uint64_t vvli_gpu_storage_element_count(const vvli_gpu_config* cfg);

/* ---------------------------------------------------------------------- */
/* Model: weights + KV cache + scratch in HBM                              */
/* ---------------------------------------------------------------------- */
/* Replaces OwnedModel + KVCache.init + Scratch.init + Runner.init
 * (src/llm.zig:424-446, 545-563, 626-662, 694-700). host_blob is the
 * contiguous blob in the order of OwnedModel.assignSlices (src/llm.zig:488-522);
 * it is copied to the device before the call returns, so the caller may free
 * it afterwards. The KV cache is cleared (KVCache.clear). Dense llama /
 * mistral / qwen2 only: MoE configs return VVLI_UNSUPPORTED_ARCH like
 * OwnedModel.init (src/llm.zig:426). max_seq_len must be in 1..max_pos. */
int vvli_gpu_model_create(const vvli_gpu_config* cfg, uint32_t max_seq_len, const void* host_blob,
                          size_t blob_elems, vvli_gpu_model** out);
int vvli_gpu_model_destroy(vvli_gpu_model* model);

/* Progress callback: LoadProgress.report (called with (0, total, "start"),
 * then once per tensor with the tensor's name; src/llm.zig:68-75, 1067-1079). */
typedef void (*vvli_host_progress_fn)(void* user, size_t completed, size_t total, const char* name);

/* loadOwnedFromSafetensorsFile / loadOwnedFromGgufFile (src/llm.zig:849-921)
 * straight into HBM: the same parsing, names, checks and error codes as
 * vvli_host_load_safetensors / vvli_host_load_gguf, but no host blob. Tensors
 * whose dtype matches the blob are copied from `bytes` (e.g. a read-only file
 * mapping) to the device; F32 / F16 / BF16 tensors of another dtype are
 * converted by a device kernel with the same bit rules (f32 -> bf16 round to
 * nearest even, f16 widened exactly). The GGUF form derives the config
 * (Config.fromGguf) and returns it in cfg_out (nullable). */
int vvli_gpu_model_create_from_safetensors(const vvli_gpu_config* cfg, uint32_t max_seq_len, const void* bytes,
                                           size_t len, vvli_host_progress_fn progress, void* user,
                                           vvli_gpu_model** out);
int vvli_gpu_model_create_from_gguf(const void* bytes, size_t len, uint32_t weight_kind, uint32_t max_seq_len,
                                    vvli_host_progress_fn progress, void* user, vvli_gpu_config* cfg_out,
                                    vvli_gpu_model** out);
/* Copy n blob elements starting at elem_offset back to the host (the blob's
 * dtype; for checks of what a loader wrote). */
int vvli_gpu_read_weights(vvli_gpu_model* model, uint64_t elem_offset, uint64_t n, void* out);

/* Mixture-of-experts decoder (OLMoE form). No reference counterpart: the
 * reference's Config carries num_experts / num_experts_per_tok / qk_norm
 * (src/llm.zig:86-88) but its runner rejects them (src/llm.zig:218-223,426).
 * Semantics follow HF transformers' OLMoE: q and k RMS-normalised over their
 * full width after the projections (cfg->qk_norm), router softmax in f32,
 * top-k (ties to the lower expert id) without renormalisation, experts
 * silu(gate) * up then down, summed in ascending expert id with their
 * probabilities. Blob (dtype bf16 only): embed; per layer input_norm, q,
 * (q_bias), k, (k_bias), v, (v_bias), (q_norm [hidden], k_norm [kv]), o,
 * post_norm, router [E][hidden], gate_up [E][2*inter][hidden] (gate rows then
 * up rows, HF's fused layout), down [E][hidden][inter]; final_norm; lm_head
 * unless tied; every slice 64-byte aligned. The handle works with every token
 * entry point below: decode on the persistent step (head_dim 64 or 128) or
 * the per-kernel graph, prompts through the batched prefill (head_dim 32, 64
 * or 128; the (row, slot) pairs grouped by expert on the device) or the
 * token loop. Limits: <= 256 experts, experts_per_tok <= 16. */
uint64_t vvli_gpu_moe_storage_element_count(const vvli_gpu_config* cfg);
int vvli_gpu_moe_model_create(const vvli_gpu_config* cfg, uint32_t max_seq_len, const void* host_blob,
                              size_t blob_elems, vvli_gpu_model** out);
/* KVCache.clear, src/llm.zig:576-579. */
int vvli_gpu_kv_clear(vvli_gpu_model* model);
/* Replace the RoPE inverse-frequency table (n = head_dim/2). NULL restores
 * the reference formula inv_freq[i] = 1/pow(theta, 2i/head_dim)
 * (src/llm.zig:1360-1363). Used for llama3-scaled frequencies. */
int vvli_gpu_set_rope_table(vvli_gpu_model* model, const float* inv_freq, uint32_t n);

/* Runner.forwardToken, src/llm.zig:702-709. token >= vocab -> VVLI_INVALID_TOKEN,
 * pos >= max_seq_len -> VVLI_CONTEXT_FULL. logits_out (vocab floats) and
 * argmax_out (llm.argmax of the logits, src/llm.zig:778-789) are optional. */
int vvli_gpu_forward_token(vvli_gpu_model* model, uint32_t token, uint32_t pos, float* logits_out,
                           uint32_t* argmax_out);
/* Runner.forwardToken with the reference's return convention: it returns a
 * borrowed slice of scratch.logits, valid until the next call
 * (src/llm.zig:702-709,729). *logits_view points at the library's pinned host
 * copy of the vocab logits, overwritten by the next forward_token_view call
 * on this model (and, with resident steps, by the next forward_token call
 * that returns logits) and freed with it (set only on success); argmax_out is
 * optional. Same errors as vvli_gpu_forward_token. */
int vvli_gpu_forward_token_view(vvli_gpu_model* model, uint32_t token, uint32_t pos, const float** logits_view,
                                uint32_t* argmax_out);
/* Resident single steps for callers that drive the model one token at a time
 * (the forwardToken loop of src/generator.zig:243-293 run from the host). No
 * counterpart in the reference, which has no launches: with linger_us > 0, a
 * forward_token / forward_token_view call on the persistent decode path
 * leaves its launch running for up to linger_us of idle time, and the next
 * call hands it (token, pos) through pinned host memory instead of
 * launching again; the step writes the logits straight to pinned host memory
 * when the call returns them. Results are those of separate launches. While
 * such a launch waits it occupies every CU, so other work on the GPU waits up
 * to linger_us; every other entry point on the model ends it first. 0 (the
 * default) turns it off; linger_us over 100000 -> VVLI_INVALID_CONFIG. */
int vvli_gpu_set_resident(vvli_gpu_model* model, uint32_t linger_us);
/* Runner.forwardEmbedding, src/llm.zig:711-718: embedding = hidden floats (host). */
int vvli_gpu_forward_embedding(vvli_gpu_model* model, const float* embedding, uint32_t pos, float* logits_out,
                               uint32_t* argmax_out);
/* forwardToken that also returns the residual stream after every layer
 * (hidden_out: layers*hidden floats, layer-major) for per-layer parity. It
 * runs on the path forward_token takes (vvli_gpu_set_decode_path): the
 * persistent step, whose down-projection phases then also write the rows, or
 * the per-kernel step. */
int vvli_gpu_forward_token_debug(vvli_gpu_model* model, uint32_t token, uint32_t pos, float* logits_out,
                                 float* hidden_out);
/* Read back one KV-cache row (kv_heads*head_dim floats each; either output
 * may be NULL): KVCache.keySlice / valueSlice, src/llm.zig:581-589. */
int vvli_gpu_kv_read(vvli_gpu_model* model, uint32_t layer, uint32_t pos, float* k_out, float* v_out);

/* Prompt processing: the prompt loop of src/generator.zig:243-251. Writes K/V
 * for positions start_pos..start_pos+n-1 and returns the logits / argmax of
 * the last one, leaving the state the token loop leaves (the next forward is
 * at start_pos+n). Batched (every row of a chunk of up to 2048 tokens through
 * each layer at once: MFMA GEMMs with f32 activations split into two bf16
 * halves, causal GQA attention) for bf16 weights with head_dim 32/64/128,
 * else one token step per prompt token; see vvli_gpu_set_prefill_path. */
int vvli_gpu_prefill(vvli_gpu_model* model, const uint32_t* tokens, uint32_t n, uint32_t start_pos,
                     float* last_logits, uint32_t* argmax_out);

/* Greedy generation: generateGreedyMeasured* (src/generator.zig:221-293) with
 * temperature 0 and no repeat penalty. Prefill runs the prompt (flags bit 0:
 * batched vvli_gpu_prefill, else one forward per token), then decode takes the
 * on-device argmax, emits it, stops on EOS (eos < 0: never), else forwards it.
 * Without EOS the decode steps run back to back with no host round trip.
 * out_tokens must hold max_new entries; *n_out receives the count. */
#define VVLI_GEN_BATCHED_PREFILL 1u
int vvli_gpu_generate_greedy(vvli_gpu_model* model, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                             int64_t eos, uint32_t flags, uint32_t* out_tokens, uint32_t* n_out,
                             vvli_gpu_stats* stats);

/* Sampling options: generator.Options (src/generator.zig:14-23). */
typedef struct vvli_gpu_sampling {
    float temperature;       /* <= 0: greedy with the repeat penalty */
    float top_p;             /* (0, 1] */
    uint32_t top_k;          /* 0 = no limit (every finite candidate) */
    float repeat_penalty;    /* >= 1; 1 disables it */
    uint32_t repeat_last_n;  /* window of prompt + generated tokens, <= 65535 */
    uint64_t seed;           /* DefaultPrng seed; 0 -> 0x9e3779b97f4a7c15 as Sampler.init */
} vvli_gpu_sampling;

/* generateGreedyMeasured* with Options (src/generator.zig:221-293) and
 * Sampler.next (:93-120) on the device: repeat penalty over the last
 * repeat_last_n tokens, greedy when temperature <= 0, else the top_k finite
 * adjusted logits (ties to the lower id), p = exp((l - l_max) / T) summed in
 * candidate order, the top_p cut, one Random.float(f32) draw from Zig's
 * DefaultPrng (xoshiro256++, SplitMix64-seeded) and the cumulative pick. The
 * first token is sampled from the prompt's last logits; every sampled token is
 * forwarded (the last one too), so max_new tokens take max_new forwards, as
 * in the reference. Greedy without a penalty runs vvli_gpu_generate_greedy.
 * Candidate lists over 1024 (top_k 0 or > 1024 with a larger vocab) are
 * sorted whole on the device (a stable radix sort: ties to the lower id,
 * where the reference's unstable sort leaves their order open) and summed in
 * one sequential pass; scratch for them is allocated on first use. */
int vvli_gpu_generate(vvli_gpu_model* model, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                      int64_t eos, uint32_t flags, const vvli_gpu_sampling* opts, uint32_t* out_tokens,
                      uint32_t* n_out, vvli_gpu_stats* stats);
/* Sampler.next (src/generator.zig:93-120) on host logits with the device
 * kernel: the repeat counts come from prompt + generated (buildRepeatCounts),
 * prng_state is the DefaultPrng state (s[0..3]) advanced in place when a
 * random unit is drawn. For hosts that keep their own generation loop. */
int vvli_gpu_sampler_next(const float* logits, uint32_t n, const uint32_t* prompt, uint32_t n_prompt,
                          const uint32_t* generated, uint32_t n_generated, const vvli_gpu_sampling* opts,
                          uint64_t prng_state[4], uint32_t* token_out);
/* DefaultPrng.init(seed) as Sampler.init calls it (seed 0 mapped first). */
void vvli_gpu_prng_seed(uint64_t seed, uint64_t state_out[4]);

/* ---------------------------------------------------------------------- */
/* Measurement (no reference counterpart: the reference has no profiler)   */
/* ---------------------------------------------------------------------- */
/* Runs one token step of the per-kernel path (like forward_token) with every
 * kernel launched between its own start/stop HIP events on the model's
 * stream (hipExtLaunchKernel: the kernel's dispatch interval) and returns each
 * kernel's time in milliseconds, in launch order: embed, then per layer {qkv,
 * attention, o_proj, gate_up, down}, then logits, argmax. *n_out = kernels timed. */
int vvli_gpu_profile_step(vvli_gpu_model* model, uint32_t token, uint32_t pos, float* ms_out, uint32_t cap,
                          uint32_t* n_out);
/* Which implementation runs forward_token / prefill / generate:
 * 0 = auto (the persistent step where available, else the per-kernel graph),
 * 1 = per-kernel HIP graph, 2 = persistent one-launch step (bf16 weights
 * only; VVLI_INVALID_CONFIG if unavailable). For A/B measurement and for
 * checking both against the same reference. */
int vvli_gpu_set_decode_path(vvli_gpu_model* model, uint32_t path);
/* How vvli_gpu_prefill (and generate with VVLI_GEN_BATCHED_PREFILL) runs the
 * prompt: 0 = auto (batched where supported), 1 = token loop, 2 = batched
 * (VVLI_INVALID_CONFIG if the model does not support it). */
int vvli_gpu_set_prefill_path(vvli_gpu_model* model, uint32_t path);
/* One persistent step with phase timestamps (100 MHz ticks): ticks_out holds
 * (n_blocks + 1) * stride values. With stride >= 16 * (5 * layers + 2), phase
 * k of the step (per layer q/k/v, attention, o, gate/up, down; then logits)
 * fills ticks_out[b * stride + 16 k] with block b's staged input and
 * [b * stride + 16 k + 1 + w] with wave w's end of the phase, [.. + 9], [.. +
 * 10] with thread 0's entry into the input staging and the return of its
 * first attempt, [.. + 11] with its retry count, [.. + 12], [.. + 13] with
 * thread 0 past the phase's closing barrier and past the next phase's first
 * weight loads;
 * ticks_out[n_blocks * stride] is the kernel start. *n_blocks = blocks of the
 * persistent launch. */
int vvli_gpu_profile_persistent(vvli_gpu_model* model, uint32_t token, uint32_t pos, uint64_t* ticks_out,
                                uint32_t stride, uint32_t* n_blocks);
/* Device time of the last timed persistent launch on this model (HIP events
 * recorded on the model's stream right before and after the cooperative
 * launch), in milliseconds; for generate_greedy that is its decode launch,
 * for prefill its one launch. Single-step forward_token launches are not
 * timed. VVLI_INVALID_CONFIG if no timed persistent launch has run. Waits for
 * the launch to finish. */
int vvli_gpu_last_launch_time(vvli_gpu_model* model, float* ms_out);
/* Test hook for the persistent step's failure path (no reference
 * counterpart): the n-th persistent launch from now (n >= 1; 0 cancels)
 * starts with its device error flag raised, as if a poll of an earlier launch
 * had timed out. Its blocks leave before any phase, and the call that waits
 * for it returns VVLI_HIP_ERROR; the flag is cleared once the host has read
 * it. */
int vvli_gpu_test_inject_step_error(vvli_gpu_model* model, uint32_t n);
/* Test hook of the batched prefill (no reference counterpart): the launch
 * form of its flash attention for every later prefill in the process -- -1
 * chosen by the prompt's size (the default), 0 blocks of 128 query vectors,
 * 1 the same with two key groups per block, 2 blocks of 64 query vectors with
 * two key groups -- so that each form can be compared with the token loop.
 * Form 2 needs heads / kv_heads <= 64 (else the prefill returns
 * VVLI_HIP_ERROR). Values outside -1..2 -> VVLI_INVALID_CONFIG. */
int vvli_gpu_test_set_prefill_attention_form(int32_t form);
/* Test hook of the whole-vocabulary sampler (no reference counterpart):
 * Sampler.next as vvli_gpu_sampler_next with no repeat history, restricted to
 * candidate lists over 1024 (temperature > 0, top_k 0 or > 1024; else
 * VVLI_INVALID_CONFIG), that also returns, in candidate order, the
 * candidates' ids, their probabilities exp((s - s_max) / T) and the running
 * f32 sums of those probabilities (the sums prepareProbabilities and
 * sampleCandidate form, src/generator.zig:428-463); *count_out = candidates.
 * ids_out, probs_out and sums_out hold n entries. */
int vvli_gpu_test_sampler_trace(const float* logits, uint32_t n, const vvli_gpu_sampling* opts,
                                uint64_t prng_state[4], uint32_t* token_out, uint32_t* ids_out, float* probs_out,
                                float* sums_out, uint32_t* count_out);

/* ---------------------------------------------------------------------- */
/* Isolated matmul op (device pointers)                                    */
/* ---------------------------------------------------------------------- */
/* linearInto (src/llm.zig:1228-1275) generalised to M rows of activations:
 * Y[m,n] = sum_k bf16 W[n,k] * X[m,k] (+ bias[n]) with f32 accumulation.
 * dW: N*K bf16, dX: M*K f32, dBias: N bf16 or NULL, dY: M*N f32, all device
 * pointers; K must be a multiple of 8; dY must be device memory (hipMalloc:
 * the K-split paths publish partials with write-through stores). stream:
 * hipStream_t or NULL for the null stream. Asynchronous: returns after the
 * launch. M <= 3 (and M = 4 when W has few row tiles) runs the
 * GEMV kernel, one launch for all rows of X (one per row when they do not fit
 * its LDS); otherwise 4 <= M <= 64 one skinny MFMA kernel (W
 * read once, X split into two bf16 halves in registers so the products keep
 * about 16 bits of each f32 activation; few row tiles split K across blocks
 * and the last block of a tile sums the partials in a fixed order); M > 64 one
 * MFMA GEMM through planes of the split X. Results are deterministic except on
 * the GEMM path, whose split-K partial sums are added with atomics (the last
 * bits may vary run to run). Scratch (K-split partials and counters, or the
 * GEMM's planes: about 4*M*K bytes) is kept per stream, allocated
 * stream-ordered, grown when needed and kept until the process ends (calls on
 * one stream use it in turn). */
int vvli_gpu_linear(const uint16_t* dW, const float* dX, const uint16_t* dBias, float* dY, uint32_t M, uint32_t N,
                    uint32_t K, void* stream);

/* vvli_gpu_linear without any allocation. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops and harnesses that forbid hipMalloc). Same
 * arguments, kernels and results as vvli_gpu_linear. Where that call keeps a
 * stream-ordered scratch (M > 64: the activation planes, 4*M*ceil32(K)
 * bytes; 4 <= M <= 64 with few row tiles: K-split partials), this one uses a
 * static device array of VVLI_LINEAR_NOALLOC_SCRATCH_BYTES (plus 64 KiB of
 * counters) on each GPU it runs on, held until the process ends; a call
 * needing more returns VVLI_INVALID_CONFIG before any launch.
 * The array of the current device is used (stream must belong to it). Every
 * call on one GPU shares that array and nothing in it needs clearing, but
 * calls that overlap on one GPU (other streams, other threads) race on it:
 * serialise them. */
#define VVLI_LINEAR_NOALLOC_SCRATCH_BYTES (16u << 20)
int vvli_gpu_linear_noalloc(const uint16_t* dW, const float* dX, const uint16_t* dBias, float* dY, uint32_t M,
                            uint32_t N, uint32_t K, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* VVLI_GPU_H */
