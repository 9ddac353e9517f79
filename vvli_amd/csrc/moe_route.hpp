// moe_route.hpp -- softmax + top-k of router logits in one thread block,
// shared by the MoE token-step kernels (moe.hip) and the persistent step
// (decode_step.hip). Semantics: HF OLMoE's router (softmax in f32, top-k by
// probability, ties to the lower expert id, no renormalisation).
#pragma once

#include "device_common.hpp"

namespace vvli {

// logits[0, E) (E <= 256, LDS; overwritten with the probabilities) ->
// idx[0, top_k), weight[0, top_k). Called by every thread of the block
// (NT threads, NT >= 64 and a multiple of 64); keys / rank: LDS scratch of E
// entries each. Wave 0 takes the softmax; an expert's rank is then the number
// of larger keys, key = (probability bits + 1, ~expert id) -- a larger
// probability or, on a tie, the lower id; keys are distinct -- counted by all
// threads over slices of the keys (few registers, no cross-lane shuffles) and
// summed with LDS atomics. Ends with the outputs written (a barrier is up to
// the caller).
template <int NT>
__device__ inline void route_block(float* logits, uint32_t E, uint32_t top_k, uint32_t* idx, float* weight,
                                   unsigned long long* keys, uint32_t* rank) {
    // The thread index through an empty asm, so that the addresses derived
    // from it are formed here rather than hoisted to a caller's start.
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    if (tid < 64) {  // (experts walked per lane, not held in registers: the callers run near their limit)
        float mx = -INFINITY;
        for (uint32_t e = tid; e < E; e += 64) mx = fmaxf(mx, logits[e]);
        mx = wave_max(mx);
        float sum = 0.f;
        for (uint32_t e = tid; e < E; e += 64) sum += expf(logits[e] - mx);
        sum = wave_sum(sum);
        for (uint32_t e = tid; e < E; e += 64) {
            const float pr = expf(logits[e] - mx) / sum;
            logits[e] = pr;
            keys[e] = (static_cast<unsigned long long>(__float_as_uint(pr) + 1u) << 32) | (0xffffffffu - e);
            rank[e] = 0;
        }
    }
    __syncthreads();
    // Thread t: expert t % E against key slice t / E (slices of `per` keys).
    const uint32_t nslice = NT / E > 0 ? NT / E : 1;
    const uint32_t per = (E + nslice - 1) / nslice;
    for (uint32_t i = tid; i < E * nslice; i += NT) {
        const uint32_t e = i % E, k0 = (i / E) * per, k1 = min(E, k0 + per);
        const unsigned long long me = keys[e];
        uint32_t c = 0;
        for (uint32_t k = k0; k < k1; ++k) c += keys[k] > me;
        if (c) atomicAdd(rank + e, c);
    }
    __syncthreads();
    for (uint32_t e = tid; e < E; e += NT) {
        const uint32_t r = rank[e];
        if (r < top_k) {
            idx[r] = e;
            weight[r] = logits[e];
        }
    }
}

}  // namespace vvli
