// host_synth.cpp -- deterministic blob fillers (host only).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "internal.hpp"
#include "vvli_host.h"

namespace vvli {
namespace {

inline uint64_t mix64(uint64_t z) {  // splitmix64 finaliser
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// Elements 2j and 2j+1 share one draw: Box-Muller cosine and sine branches.
inline void normal_pair(uint64_t seed, uint64_t tensor, uint64_t j, double& z0, double& z1) {
    const uint64_t h = mix64(mix64(seed ^ mix64(tensor)) + j);
    const double u1 = (static_cast<double>(h >> 40) + 0.5) * (1.0 / 16777216.0);
    const double u2 = (static_cast<double>(h & 0xffffffull) + 0.5) * (1.0 / 16777216.0);
    const double r = std::sqrt(-2.0 * std::log(u1)), a = 6.283185307179586 * u2;
    z0 = r * std::cos(a);
    z1 = r * std::sin(a);
}

inline double normal_at(uint64_t seed, uint64_t tensor, uint64_t i) {
    double z0, z1;
    normal_pair(seed, tensor, i >> 1, z0, z1);
    return (i & 1) ? z1 : z0;
}

struct Slice {
    size_t off, len;
    uint64_t id;
    bool norm;
};

}  // namespace
}  // namespace vvli

using namespace vvli;

extern "C" {

void vvli_host_fill_deterministic(void* blob, size_t n, uint32_t weight_kind) {
    for (size_t i = 0; i < n; ++i) {
        const float v = static_cast<float>(static_cast<int32_t>(i % 251) - 125) * 0.001f;
        if (weight_kind == VVLI_WEIGHT_BF16)
            static_cast<uint16_t*>(blob)[i] = f32_to_bf16(v);
        else
            static_cast<float*>(blob)[i] = v;
    }
}

double vvli_host_synthetic_normal(uint64_t seed, uint64_t tensor_id, uint64_t index) {
    return normal_at(seed, tensor_id, index);
}

int vvli_host_fill_synthetic(const vvli_gpu_config* cfg, uint64_t seed, float stddev, void* blob, size_t blob_elems,
                             uint32_t threads) {
    if (!cfg || !blob) return set_error(VVLI_NULL_ARG, "NULL argument to vvli_host_fill_synthetic");
    const bool moe = cfg->num_experts != 0;
    int rc = validate_config(*cfg, !moe);
    if (rc) return rc;
    const size_t h = cfg->hidden, kv = kv_dim(*cfg), inter = cfg->inter;
    std::vector<Slice> slices;
    size_t total = 0;
    if (moe) {
        const MoeLayout M = compute_moe_layout(*cfg);
        if (blob_elems < M.total) return set_error(VVLI_INVALID_WEIGHT, "blob too small for the layout");
        total = M.total;
        const size_t e = cfg->num_experts;
        slices.push_back({M.embed, static_cast<size_t>(cfg->vocab) * h, 0, false});
        for (uint32_t l = 0; l < cfg->layers; ++l) {
            const MoeLayerSlices& s = M.layers[l];
            const uint64_t b = 1 + 16ull * l;
            slices.push_back({s.input_norm, h, b + 0, true});
            slices.push_back({s.q, h * h, b + 1, false});
            if (s.q_bias != kNone) slices.push_back({s.q_bias, h, b + 2, false});
            slices.push_back({s.k, kv * h, b + 3, false});
            if (s.k_bias != kNone) slices.push_back({s.k_bias, kv, b + 4, false});
            slices.push_back({s.v, kv * h, b + 5, false});
            if (s.v_bias != kNone) slices.push_back({s.v_bias, kv, b + 6, false});
            if (s.q_norm != kNone) slices.push_back({s.q_norm, h, b + 7, true});
            if (s.k_norm != kNone) slices.push_back({s.k_norm, kv, b + 8, true});
            slices.push_back({s.o, h * h, b + 9, false});
            slices.push_back({s.post_norm, h, b + 10, true});
            slices.push_back({s.router, e * h, b + 11, false});
            slices.push_back({s.gate_up, e * 2 * inter * h, b + 12, false});
            slices.push_back({s.down, e * h * inter, b + 13, false});
        }
        slices.push_back({M.final_norm, h, 1 + 16ull * cfg->layers, true});
        if (M.lm_head != kNone)
            slices.push_back({M.lm_head, static_cast<size_t>(cfg->vocab) * h, 2 + 16ull * cfg->layers, false});
    }
    const BlobLayout L = moe ? BlobLayout{} : compute_layout(*cfg);
    if (!moe && blob_elems < L.total) return set_error(VVLI_INVALID_WEIGHT, "blob too small for the layout");
    if (!moe) {
        total = L.total;
        slices.push_back({L.embed, static_cast<size_t>(cfg->vocab) * h, 0, false});
    }
    for (uint32_t l = 0; !moe && l < cfg->layers; ++l) {
        const LayerSlices& s = L.layers[l];
        const uint64_t b = 1 + 12ull * l;
        slices.push_back({s.input_norm, h, b + 0, true});
        slices.push_back({s.q, h * h, b + 1, false});
        if (s.q_bias != kNone) slices.push_back({s.q_bias, h, b + 2, false});
        slices.push_back({s.k, kv * h, b + 3, false});
        if (s.k_bias != kNone) slices.push_back({s.k_bias, kv, b + 4, false});
        slices.push_back({s.v, kv * h, b + 5, false});
        if (s.v_bias != kNone) slices.push_back({s.v_bias, kv, b + 6, false});
        slices.push_back({s.o, h * h, b + 7, false});
        slices.push_back({s.post_norm, h, b + 8, true});
        slices.push_back({s.gate, inter * h, b + 9, false});
        slices.push_back({s.up, inter * h, b + 10, false});
        slices.push_back({s.down, h * inter, b + 11, false});
    }
    if (!moe) {
        slices.push_back({L.final_norm, h, 1 + 12ull * cfg->layers, true});
        if (L.lm_head != kNone)
            slices.push_back({L.lm_head, static_cast<size_t>(cfg->vocab) * h, 2 + 12ull * cfg->layers, false});
    }

    const bool bf16 = cfg->weight_kind == VVLI_WEIGHT_BF16;
    const size_t eb = bf16 ? 2 : 4;
    std::memset(blob, 0, total * eb);  // alignment padding
    unsigned nt = threads ? threads : std::thread::hardware_concurrency();
    if (nt == 0) nt = 1;
    // Work items: fixed-size chunks of every slice.
    constexpr size_t kChunk = 1 << 20;
    struct Item {
        const Slice* s;
        size_t begin, end;
    };
    std::vector<Item> items;
    for (const Slice& s : slices)
        for (size_t b = 0; b < s.len; b += kChunk) items.push_back({&s, b, std::min(s.len, b + kChunk)});
    auto work = [&](unsigned t) {
        for (size_t k = t; k < items.size(); k += nt) {
            const Item& it = items[k];
            double z0 = 0, z1 = 0;
            for (size_t i = it.begin; i < it.end; ++i) {
                float v = 1.0f;
                if (!it.s->norm) {
                    if (i == it.begin || (i & 1) == 0) normal_pair(seed, it.s->id, i >> 1, z0, z1);
                    v = static_cast<float>(((i & 1) ? z1 : z0) * stddev);
                }
                if (bf16)
                    static_cast<uint16_t*>(blob)[it.s->off + i] = f32_to_bf16(v);
                else
                    static_cast<float*>(blob)[it.s->off + i] = v;
            }
        }
    };
    std::vector<std::thread> pool;
    for (unsigned t = 1; t < nt; ++t) pool.emplace_back(work, t);
    work(0);
    for (auto& th : pool) th.join();
    return VVLI_OK;
}

}  // extern "C"
