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

#ifdef __cplusplus
}
#endif
#endif /* VVLI_HOST_H */
