// host_config.cpp -- the shape contract: Config.validate / parameterCount /
// storageElementCount / assignSlices, plus the library's error reporting.
#include <cstdarg>
#include <cstdio>

#include "internal.hpp"

namespace vvli {

static thread_local char g_last_error[512] = "";

int set_error(int rc, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return rc;
}

void clear_error() { g_last_error[0] = '\0'; }

int validate_config(const vvli_gpu_config& c, bool require_dense) {
    // Config.validate, src/llm.zig:195-216.
    if (c.abi_version != VVLI_GPU_ABI_VERSION)
        return set_error(VVLI_INVALID_CONFIG, "abi_version %u != %u", c.abi_version, VVLI_GPU_ABI_VERSION);
    if (c.vocab == 0 || c.hidden == 0 || c.inter == 0 || c.layers == 0 || c.heads == 0 || c.kv_heads == 0 ||
        c.max_pos == 0)
        return set_error(VVLI_INVALID_CONFIG, "zero-sized config field");
    if (c.hidden % c.heads != 0) return set_error(VVLI_INVALID_CONFIG, "hidden %% heads != 0");
    if (c.heads % c.kv_heads != 0) return set_error(VVLI_INVALID_CONFIG, "heads %% kv_heads != 0");
    if (head_dim(c) % 2 != 0) return set_error(VVLI_INVALID_CONFIG, "odd head_dim");
    if (c.arch > VVLI_ARCH_QWEN2) return set_error(VVLI_UNSUPPORTED_ARCH, "unknown architecture %u", c.arch);
    if (c.rope_layout > VVLI_ROPE_SPLIT_HALF) return set_error(VVLI_INVALID_CONFIG, "bad rope_layout");
    if (c.weight_kind > VVLI_WEIGHT_BF16) return set_error(VVLI_UNSUPPORTED_DTYPE, "bad weight_kind");
    const bool moe = c.num_experts != 0;
    if (!moe && c.experts_per_tok != 0) return set_error(VVLI_INVALID_CONFIG, "experts_per_tok without experts");
    if (moe && (c.experts_per_tok == 0 || c.experts_per_tok > c.num_experts))
        return set_error(VVLI_INVALID_CONFIG, "bad experts_per_tok");
    // supportsDenseRunner, src/llm.zig:218-223; OwnedModel.init rejects the rest (:426).
    if (require_dense && (moe || c.arch == VVLI_ARCH_OLMOE))
        return set_error(VVLI_UNSUPPORTED_ARCH, "MoE / olmoe is not a dense decoder");
    return VVLI_OK;
}

uint64_t parameter_count(const vvli_gpu_config& c) {
    // Config.layerParameterCount / parameterCount, src/llm.zig:241-276.
    const uint64_t h = c.hidden, kv = kv_dim(c), inter = c.inter;
    const uint64_t bias = c.qkv_bias ? h + kv + kv : 0;
    uint64_t layer = h + h * h + bias + kv * h + kv * h + h * h + h;
    if (c.qk_norm) layer += 2ull * head_dim(c);
    if (c.num_experts == 0)
        layer += 3 * inter * h;
    else
        layer += c.num_experts * h + c.num_experts * (inter * h * 2 + h * inter);
    uint64_t total = static_cast<uint64_t>(c.vocab) * h + c.layers * layer + h;
    if (!c.tie) total += static_cast<uint64_t>(c.vocab) * h;
    return total;
}

BlobLayout compute_layout(const vvli_gpu_config& c) {
    // assignSlices (src/llm.zig:488-522) with takeWeight's cursor alignment
    // (:524-532, :1495-1504): 64 bytes = 32 bf16 or 16 f32 elements.
    const size_t ea = kAlignBytes / elem_bytes(c);
    const size_t h = c.hidden, kv = kv_dim(c), inter = c.inter;
    size_t cur = 0;
    auto take = [&](size_t len) {
        cur = (cur + ea - 1) / ea * ea;
        size_t s = cur;
        cur += len;
        return s;
    };
    BlobLayout L;
    L.embed = take(static_cast<size_t>(c.vocab) * h);
    L.layers.resize(c.layers);
    for (auto& s : L.layers) {
        s.input_norm = take(h);
        s.q = take(h * h);
        s.q_bias = c.qkv_bias ? take(h) : kNone;
        s.k = take(kv * h);
        s.k_bias = c.qkv_bias ? take(kv) : kNone;
        s.v = take(kv * h);
        s.v_bias = c.qkv_bias ? take(kv) : kNone;
        s.o = take(h * h);
        s.post_norm = take(h);
        s.gate = take(inter * h);
        s.up = take(inter * h);
        s.down = take(h * inter);
    }
    L.final_norm = take(h);
    L.lm_head = c.tie ? kNone : take(static_cast<size_t>(c.vocab) * h);
    L.total = cur;
    return L;
}

MoeLayout compute_moe_layout(const vvli_gpu_config& c) {
    const size_t ea = kAlignBytes / elem_bytes(c);
    const size_t h = c.hidden, kv = kv_dim(c), inter = c.inter, e = c.num_experts;
    size_t cur = 0;
    auto take = [&](size_t len) {
        cur = (cur + ea - 1) / ea * ea;
        size_t s = cur;
        cur += len;
        return s;
    };
    MoeLayout L;
    L.embed = take(static_cast<size_t>(c.vocab) * h);
    L.layers.resize(c.layers);
    for (auto& s : L.layers) {
        s.input_norm = take(h);
        s.q = take(h * h);
        s.q_bias = c.qkv_bias ? take(h) : kNone;
        s.k = take(kv * h);
        s.k_bias = c.qkv_bias ? take(kv) : kNone;
        s.v = take(kv * h);
        s.v_bias = c.qkv_bias ? take(kv) : kNone;
        s.q_norm = c.qk_norm ? take(h) : kNone;
        s.k_norm = c.qk_norm ? take(kv) : kNone;
        s.o = take(h * h);
        s.post_norm = take(h);
        s.router = take(e * h);
        s.gate_up = take(e * 2 * inter * h);
        s.down = take(e * h * inter);
    }
    L.final_norm = take(h);
    L.lm_head = c.tie ? kNone : take(static_cast<size_t>(c.vocab) * h);
    L.total = cur;
    return L;
}

}  // namespace vvli

extern "C" {

uint32_t vvli_gpu_abi_version(void) { return VVLI_GPU_ABI_VERSION; }

const char* vvli_gpu_last_error(void) { return vvli::g_last_error; }

int vvli_gpu_config_validate(const vvli_gpu_config* cfg) {
    if (!cfg) return vvli::set_error(VVLI_NULL_ARG, "cfg is NULL");
    return vvli::validate_config(*cfg, false);
}

uint64_t vvli_gpu_parameter_count(const vvli_gpu_config* cfg) { return cfg ? vvli::parameter_count(*cfg) : 0; }

uint64_t vvli_gpu_storage_element_count(const vvli_gpu_config* cfg) {
    if (!cfg || cfg->num_experts != 0) return 0;
    return vvli::compute_layout(*cfg).total;
}

uint64_t vvli_gpu_moe_storage_element_count(const vvli_gpu_config* cfg) {
    if (!cfg || cfg->num_experts == 0) return 0;
    return vvli::compute_moe_layout(*cfg).total;
}

}  // extern "C"
