// device_common.hpp -- gfx950 device helpers shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vvli {

constexpr int kWave = 64;  // CDNA wavefront width

// ---- bf16 / f32 weight access -------------------------------------------
// A 16-byte unit holds 8 bf16 or 4 f32 weights.
template <typename WT> struct WeightTraits;
template <> struct WeightTraits<uint16_t> {
    static constexpr int kPerUnit = 8;
    __device__ static inline float at(const uint16_t* p, size_t i) { return __uint_as_float((uint32_t)p[i] << 16); }
    // Expand one 16-byte unit into 8 floats.
    __device__ static inline void expand(const uint4& u, float* f) {
        f[0] = __uint_as_float(u.x << 16);
        f[1] = __uint_as_float(u.x & 0xffff0000u);
        f[2] = __uint_as_float(u.y << 16);
        f[3] = __uint_as_float(u.y & 0xffff0000u);
        f[4] = __uint_as_float(u.z << 16);
        f[5] = __uint_as_float(u.z & 0xffff0000u);
        f[6] = __uint_as_float(u.w << 16);
        f[7] = __uint_as_float(u.w & 0xffff0000u);
    }
};
template <> struct WeightTraits<float> {
    static constexpr int kPerUnit = 4;
    __device__ static inline float at(const float* p, size_t i) { return p[i]; }
    __device__ static inline void expand(const uint4& u, float* f) {
        f[0] = __uint_as_float(u.x);
        f[1] = __uint_as_float(u.y);
        f[2] = __uint_as_float(u.z);
        f[3] = __uint_as_float(u.w);
    }
};

// Device pointers handed around in structs (or read back from LDS) are
// generic; the casts to the global address space make the compiler emit
// global_* rather than flat_* memory instructions (flat ones also count
// against the LDS counter and cost more to issue).
#define VVLI_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ VVLI_GLOBAL T* as_global(T* p) {
    return (VVLI_GLOBAL T*)p;
}
typedef unsigned int vvli_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int vvli_u32x2 __attribute__((ext_vector_type(2)));
// Weights are streamed once per use: nontemporal loads (the nt cache policy)
// keep them from displacing what is reused in the caches -- the tagged
// activation words, the K/V rows, x (measured on the persistent decode step:
// 1340 -> 1354 tok/s at Llama-3.2-1B, 1298 -> 1308 at Qwen2.5-0.5B).
__device__ inline uint4 load_unit(const void* p) {
    const vvli_u32x4 v = __builtin_nontemporal_load(as_global(reinterpret_cast<const vvli_u32x4*>(p)));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ inline float4 load_f32x4(const float* p) {
    const vvli_u32x4 v = *as_global(reinterpret_cast<const vvli_u32x4*>(p));
    return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
__device__ inline uint2 load_u32x2(const void* p) {
    const vvli_u32x2 v = *as_global(reinterpret_cast<const vvli_u32x2*>(p));
    return make_uint2(v.x, v.y);
}

// ---- wave reductions with DPP --------------------------------------------
// quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E, row_half_mirror =
// 0x141, row_mirror = 0x140: after the four steps every lane of a 16-lane row
// holds the row total; the four row totals are combined through readlane.
#define VVLI_DPP(v, ctrl) __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, false))

__device__ inline float wave_sum(float v) {
    v += VVLI_DPP(v, 0xB1);
    v += VVLI_DPP(v, 0x4E);
    v += VVLI_DPP(v, 0x141);
    v += VVLI_DPP(v, 0x140);
    float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (a + b) + (c + d);
}

__device__ inline float wave_max(float v) {
    v = fmaxf(v, VVLI_DPP(v, 0xB1));
    v = fmaxf(v, VVLI_DPP(v, 0x4E));
    v = fmaxf(v, VVLI_DPP(v, 0x141));
    v = fmaxf(v, VVLI_DPP(v, 0x140));
    float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

__device__ inline unsigned long long wave_max_u64(unsigned long long v) {
    for (int off = 32; off > 0; off >>= 1) {
        unsigned long long o = __shfl_xor(v, off, kWave);
        v = o > v ? o : v;
    }
    return v;
}

// ---- argmax keys -----------------------------------------------------------
// llm.argmax (src/llm.zig:778-789) returns the first index of the strict
// maximum; NaN never wins (and index 0 wins if logits[0] is NaN, handled by
// the caller). Key = order-preserving bits of the value in the high word and
// ~index in the low word, so the max key is the max value at the lowest index.
// -0.0 is folded onto +0.0 because `>` treats them as equal.
__device__ inline unsigned long long argmax_key(float v, uint32_t index) {
    if (v != v) return 0ull;  // NaN
    if (v == 0.0f) v = 0.0f;
    uint32_t u = __float_as_uint(v);
    uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<unsigned long long>(ord) << 32) | static_cast<uint32_t>(~index);
}

__device__ inline uint32_t argmax_key_index(unsigned long long key) {
    return key == 0ull ? 0u : ~static_cast<uint32_t>(key & 0xffffffffu);
}

}  // namespace vvli
