/*
 * vvli_host.h -- host-side half of the library (no GPU needed): the parts of
 * VVLI's llm.zig / gguf.zig that produce the contiguous weight blob the
 * forward pass reads. A Zig host keeps its own loaders and calls only
 * vvli_gpu.h; C/C++/Python hosts use these to build or load the blob.
 */
#ifndef VVLI_HOST_H
#define VVLI_HOST_H

#include <stddef.h>
#include <stdint.h>

#include "vvli_gpu.h"

#ifdef __cplusplus
extern "C" {
#endif

/* OwnedModel.fillDeterministicForTesting, src/llm.zig:466-477: element i =
 * ((i % 251) - 125) * 0.001, rounded to bf16 (RNE) for bf16 blobs. */
void vvli_host_fill_deterministic(void* blob, size_t n, uint32_t weight_kind);

/* Seeded synthetic weights for a dense config laid out like
 * OwnedModel.assignSlices: RMSNorm weights = 1, every other tensor N(0, stddev)
 * (f32, then RNE to bf16 for bf16 blobs), alignment padding = 0. Element i of
 * tensor t is a pure function of (seed, t, i): splitmix64 of (seed, t, i/2)
 * -> two 24-bit uniforms -> Box-Muller in double precision, cosine branch for
 * even i and sine branch for odd i. Tensor ids: embed
 * 0; layer l slot j (input_norm, q, q_bias, k, k_bias, v, v_bias, o,
 * post_norm, gate, up, down) 1 + 12l + j; final norm 1 + 12L; lm_head 2 + 12L.
 * threads == 0 uses the host CPU count (worker threads exist only inside this
 * call). No reference counterpart: the reference only loads real checkpoints. */
int vvli_host_fill_synthetic(const vvli_gpu_config* cfg, uint64_t seed, float stddev, void* blob, size_t blob_elems,
                             uint32_t threads);

/* One synthetic value (the function used above), for checks and for filling
 * tensors that live outside the dense blob. */
double vvli_host_synthetic_normal(uint64_t seed, uint64_t tensor_id, uint64_t index);

/* Llama-3 RoPE frequency table for vvli_gpu_set_rope_table (head_dim / 2
 * values). No reference counterpart: the reference has no RoPE scaling (its
 * applyRoPE, src/llm.zig:1337-1371, always uses 1/pow(theta, 2i/head_dim)).
 * Starts from exactly that f32 table and applies the published Llama-3
 * scaling in f32: wavelen = 2*pi/inv_freq; wavelen > original_max_pos /
 * low_freq_factor -> inv_freq / factor; wavelen < original_max_pos /
 * high_freq_factor -> unchanged; otherwise (1 - s) * inv_freq / factor +
 * s * inv_freq with s = (original_max_pos / wavelen - low_freq_factor) /
 * (high_freq_factor - low_freq_factor). Returns VVLI_INVALID_CONFIG for an
 * odd or zero head_dim, factor <= 0 or high_freq_factor <= low_freq_factor. */
int vvli_host_llama3_inv_freq(uint32_t head_dim, float theta, float factor, float low_freq_factor,
                              float high_freq_factor, uint32_t original_max_pos, float* inv_freq_out);

/* ---------------------------------------------------------------------- */
/* Checkpoint loaders (src/llm.zig:839-1226, src/gguf.zig:234-354)          */
/* ---------------------------------------------------------------------- */
/* vvli_host_progress_fn (LoadProgress.report) is declared in vvli_gpu.h. */

/* Config.fromJson, src/llm.zig:98-145 (HF config.json text, len bytes):
 * model_type llama/mistral/olmoe/qwen2, required vocab_size, hidden_size,
 * intermediate_size, num_hidden_layers, num_attention_heads,
 * max_position_embeddings (absent -> VVLI_MISSING_FIELD, not a non-negative
 * integer -> VVLI_INVALID_CONFIG); defaults kv_heads = heads, rope_theta
 * 1e4, rms_norm_eps 1e-6, tie false, attention_bias = (qwen2), split-half
 * RoPE; eos/pad ids take the first element of an array. weight_kind is stored
 * in out. Malformed JSON -> VVLI_INVALID_FILE. Values above 2^32-1 ->
 * VVLI_INVALID_CONFIG (the C config holds 32-bit fields). */
int vvli_host_config_from_json(const char* json, size_t len, uint32_t weight_kind, vvli_gpu_config* out);

/* gguf.parse + Config.fromGguf, src/gguf.zig:234-284 and src/llm.zig:153-193:
 * magic "GGUF", version 2 or 3 (else VVLI_UNSUPPORTED_VERSION), metadata and
 * tensor tables (unknown metadata or tensor type ids ->
 * VVLI_UNSUPPORTED_METADATA, truncation or 0/ >8 dims -> VVLI_INVALID_FILE),
 * data start aligned to general.alignment (default 32). Config: prefix =
 * general.architecture, vocab = length of tokenizer.ggml.tokens, interleaved
 * RoPE, tie iff the file has no output.weight, no q/k/v bias. */
int vvli_host_config_from_gguf(const void* bytes, size_t len, uint32_t weight_kind, vvli_gpu_config* out);

/* loadSafetensorsIntoOwnedModel, src/llm.zig:923-1006 and 1149-1218: fills the
 * blob (cfg->weight_kind, OwnedModel.assignSlices layout, padding zeroed) from
 * a whole model.safetensors image. Tensors are looked up by their HF names;
 * F32 and BF16 only (else VVLI_UNSUPPORTED_DTYPE), converted to the blob's
 * type (f32->bf16 round-to-nearest-even, bf16->f32 exact). A missing tensor ->
 * VVLI_MISSING_TENSOR; a shape whose element count differs, offsets out of
 * range or a byte length that does not match -> VVLI_INVALID_WEIGHT. MoE and
 * olmoe configs -> VVLI_UNSUPPORTED_ARCH (OwnedModel.init, :424-446). */
int vvli_host_load_safetensors(const vvli_gpu_config* cfg, const void* bytes, size_t len, void* blob,
                               size_t blob_elems, vvli_host_progress_fn progress, void* user);

/* loadGgufIntoOwnedModel, src/llm.zig:1008-1147: the same for a GGUF image and
 * llama.cpp tensor names (token_embd, blk.N.attn_norm/attn_q/attn_k/attn_v/
 * attn_output/ffn_norm/ffn_gate/ffn_up/ffn_down, output_norm, output); F32,
 * F16 and BF16 tensors (f16 widened exactly, then RNE to bf16 for bf16 blobs);
 * quantised types -> VVLI_UNSUPPORTED_DTYPE; cfg->qkv_bias ->
 * VVLI_UNSUPPORTED_ARCH. cfg normally comes from vvli_host_config_from_gguf. */
int vvli_host_load_gguf(const vvli_gpu_config* cfg, const void* bytes, size_t len, void* blob, size_t blob_elems,
                        vvli_host_progress_fn progress, void* user);

/* Read-only memory map of a whole file (the reference maps checkpoints the
 * same way, src/llm.zig:870-880, 901-911). An empty or unreadable file ->
 * VVLI_INVALID_FILE. Release with vvli_host_unmap_file(data, len). */
int vvli_host_map_file(const char* path, const void** data, size_t* len);
int vvli_host_unmap_file(const void* data, size_t len);

/* f16ToF32, src/llm.zig:795-797: exact IEEE binary16 -> binary32 (NaN payloads
 * kept), exposed for tests. */
float vvli_host_f16_to_f32(uint16_t bits);

#ifdef __cplusplus
}
#endif
#endif /* VVLI_HOST_H */
