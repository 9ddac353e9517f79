// internal.hpp -- declarations shared by the host-side sources of libvvli_gpu.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "vvli_gpu.h"

namespace vvli {

// Thread-local error text; every failing entry point sets it and returns rc.
int set_error(int rc, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

constexpr size_t kNone = static_cast<size_t>(-1);
constexpr size_t kAlignBytes = 64;  // src/tensor.zig:8 data_alignment_bytes

inline uint32_t head_dim(const vvli_gpu_config& c) { return c.hidden / c.heads; }     // src/llm.zig:229-231
inline uint32_t kv_dim(const vvli_gpu_config& c) { return c.kv_heads * head_dim(c); }  // src/llm.zig:233-235
inline uint32_t kv_group(const vvli_gpu_config& c) { return c.heads / c.kv_heads; }    // src/llm.zig:237-239
inline size_t elem_bytes(const vvli_gpu_config& c) { return c.weight_kind == VVLI_WEIGHT_BF16 ? 2 : 4; }

// Offsets (elements) of every slice of the blob; OwnedModel.assignSlices
// order (src/llm.zig:488-522), each slice aligned to 64 bytes.
struct LayerSlices {
    size_t input_norm, q, q_bias, k, k_bias, v, v_bias, o, post_norm, gate, up, down;
};
struct BlobLayout {
    size_t embed = 0, final_norm = 0, lm_head = kNone, total = 0;
    std::vector<LayerSlices> layers;
};

// Mixture-of-experts blob (no reference counterpart: the reference rejects
// MoE configs). Per layer: input_norm, q, (q_bias), k, (k_bias), v, (v_bias),
// (q_norm [H], k_norm [kv]), o, post_norm, router [E][H], gate_up [E][2I][H]
// (gate rows, then up rows), down [E][H][I]; each slice 64-byte aligned.
struct MoeLayerSlices {
    size_t input_norm, q, q_bias, k, k_bias, v, v_bias, q_norm, k_norm, o, post_norm, router, gate_up, down;
};
struct MoeLayout {
    size_t embed = 0, final_norm = 0, lm_head = kNone, total = 0;
    std::vector<MoeLayerSlices> layers;
};

// Checkpoint loading (host_load.cpp): the parsers hand every tensor's raw
// bytes to a `put` callback that places them in the blob (host or device).
enum TensorSrc { kSrcF32 = 0, kSrcF16 = 1, kSrcBF16 = 2 };
using TensorPut = int (*)(void* ctx, size_t dst_elem, const uint8_t* raw, TensorSrc src, size_t n);
int load_safetensors_into(const vvli_gpu_config& cfg, const void* bytes, size_t len, TensorPut put, void* ctx,
                          void (*progress)(void*, size_t, size_t, const char*), void* user);
int load_gguf_into(const vvli_gpu_config& cfg, const void* bytes, size_t len, TensorPut put, void* ctx,
                   void (*progress)(void*, size_t, size_t, const char*), void* user);
int gguf_config(const void* bytes, size_t len, uint32_t weight_kind, vvli_gpu_config& out);

int validate_config(const vvli_gpu_config& c, bool require_dense);
uint64_t parameter_count(const vvli_gpu_config& c);
BlobLayout compute_layout(const vvli_gpu_config& c);
MoeLayout compute_moe_layout(const vvli_gpu_config& c);

// bf16 <-> f32 (src/llm.zig:791-803).
inline float bf16_to_f32(uint16_t b) {
    uint32_t u = static_cast<uint32_t>(b) << 16;
    float f;
    __builtin_memcpy(&f, &u, 4);
    return f;
}
inline uint16_t f32_to_bf16(float v) {
    uint32_t b;
    __builtin_memcpy(&b, &v, 4);
    return static_cast<uint16_t>((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

}  // namespace vvli
