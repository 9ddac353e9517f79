// convert.hip -- tensor dtype conversion on the device for the loaders that
// write the weight blob in HBM directly (vvli_gpu_model_create_from_*).
// Bit rules are the host loader's (src/llm.zig:791-803): f16 -> f32 exact
// (NaN payloads kept, no quieting), bf16 -> f32 by <<16, f32 -> bf16 round to
// nearest even with no NaN special case (the sum wraps in 32 bits).
#include <algorithm>

#include "device_common.hpp"
#include "kernels.hpp"

namespace vvli {

namespace {

__device__ inline uint32_t f16_bits_to_f32_bits(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    if (exp == 0x1f) return sign | 0x7f800000u | (man << 13);
    if (exp != 0) return sign | ((exp + 112u) << 23) | (man << 13);
    if (man == 0) return sign;
    const int shift = __clz(man) - 21;  // bring the leading one to bit 10
    man <<= shift;
    return sign | ((113u - static_cast<uint32_t>(shift)) << 23) | ((man & 0x3ffu) << 13);
}

__device__ inline uint16_t f32_bits_to_bf16(uint32_t b) {
    return static_cast<uint16_t>((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

// src: n elements of type `src` (0 f32, 1 f16, 2 bf16); dst: blob elements of
// type `kind` (0 f32, 1 bf16).
__global__ __launch_bounds__(256) void convert_kernel(const void* __restrict__ src, uint32_t src_type,
                                                      void* __restrict__ dst, uint32_t kind, size_t n) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256) {
        uint32_t f32bits;
        if (src_type == 0) f32bits = static_cast<const uint32_t*>(src)[i];
        else if (src_type == 1) f32bits = f16_bits_to_f32_bits(static_cast<const uint16_t*>(src)[i]);
        else f32bits = static_cast<uint32_t>(static_cast<const uint16_t*>(src)[i]) << 16;
        if (kind == 0) static_cast<uint32_t*>(dst)[i] = f32bits;
        else static_cast<uint16_t*>(dst)[i] = src_type == 2 ? static_cast<const uint16_t*>(src)[i]
                                                              : f32_bits_to_bf16(f32bits);
    }
}

}  // namespace

hipError_t launch_convert(const void* src, uint32_t src_type, void* dst, uint32_t kind, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>((n + 255) / 256, 8192);
    return vlaunch(convert_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s, src, src_type, dst, kind, n);
}

}  // namespace vvli
