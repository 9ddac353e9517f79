// host_rope.cpp -- RoPE frequency tables for vvli_gpu_set_rope_table (host only).
#include <cmath>

#include "internal.hpp"
#include "vvli_host.h"

extern "C" int vvli_host_llama3_inv_freq(uint32_t head_dim, float theta, float factor, float low_freq_factor,
                                         float high_freq_factor, uint32_t original_max_pos, float* inv_freq_out) {
    vvli::clear_error();
    if (!inv_freq_out) return vvli::set_error(VVLI_NULL_ARG, "inv_freq_out is NULL");
    if (head_dim == 0 || head_dim % 2 != 0)
        return vvli::set_error(VVLI_INVALID_CONFIG, "head_dim %u must be even and non-zero", head_dim);
    if (!(factor > 0.f) || !(high_freq_factor > low_freq_factor) || !(low_freq_factor > 0.f) || original_max_pos == 0)
        return vvli::set_error(VVLI_INVALID_CONFIG, "invalid llama3 RoPE scaling parameters");
    const float two_pi = static_cast<float>(2.0 * M_PI);
    const float old_ctx = static_cast<float>(original_max_pos);
    const float low_wavelen = old_ctx / low_freq_factor;
    const float high_wavelen = old_ctx / high_freq_factor;
    for (uint32_t i = 0; i < head_dim / 2; ++i) {
        // The reference's own frequency (rotatePair, src/llm.zig:1360-1366), f32.
        const float exponent = static_cast<float>(2 * i) / static_cast<float>(head_dim);
        const float inv = 1.0f / powf(theta, exponent);
        const float wavelen = two_pi / inv;
        float out = inv;
        if (wavelen > low_wavelen) {
            out = inv / factor;  // long wavelengths: fully interpolated
        } else if (!(wavelen < high_wavelen)) {
            const float s = (old_ctx / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor);
            out = (1.0f - s) * inv / factor + s * inv;  // smooth blend of the two
        }
        inv_freq_out[i] = out;
    }
    return VVLI_OK;
}
