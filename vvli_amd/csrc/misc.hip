// misc.hip -- embedding gather and the argmax / step-advance kernel.
#include "device_common.hpp"
#include "kernels.hpp"

namespace vvli {

thread_local std::vector<std::pair<hipEvent_t, hipEvent_t>>* g_launch_events = nullptr;

namespace {

template <typename WT>
__global__ void embed_kernel(const WT* __restrict__ embed, const StepState* __restrict__ st, float* __restrict__ x,
                             uint32_t hidden) {
    // copyEmbeddingToken, src/llm.zig:1373-1380 (bf16 widened by <<16).
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < hidden) x[i] = WeightTraits<WT>::at(embed, (size_t)st->token * hidden + i);
}

constexpr int kFinishThreads = 1024;

__global__ __launch_bounds__(kFinishThreads) void argmax_finish_kernel(const unsigned long long* __restrict__ keys,
                                                                      uint32_t nkeys, const float* __restrict__ logits,
                                                                      StepState* st,
                                                                      const uint32_t* __restrict__ prompt,
                                                                      uint32_t* out_tokens, uint32_t out_cap) {
    __shared__ unsigned long long red[kFinishThreads / kWave];
    const int tid = threadIdx.x;
    unsigned long long best = 0ull;
    for (uint32_t i = tid; i < nkeys; i += kFinishThreads) best = keys[i] > best ? keys[i] : best;
    best = wave_max_u64(best);
    if ((tid & 63) == 0) red[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kFinishThreads / kWave; ++w) best = red[w] > best ? red[w] : best;
        best = red[0] > best ? red[0] : best;
        // llm.argmax: logits[0] = NaN keeps index 0 (no value compares greater).
        const uint32_t tok = (logits[0] != logits[0]) ? 0u : argmax_key_index(best);
        const uint32_t next_pos = st->pos + 1;
        st->argmax = tok;
        st->pos = next_pos;
        if (next_pos < st->prompt_len) {
            st->token = prompt[next_pos];  // still inside the prompt (generator.zig:243-251)
        } else {
            st->token = tok;
            if (st->counting) {
                if (st->n_out < out_cap) out_tokens[st->n_out] = tok;
                st->n_out = st->n_out + 1;
            }
        }
    }
}

}  // namespace

hipError_t launch_embed(int weight_kind, const void* embed, const StepState* st, float* x, uint32_t hidden,
                        hipStream_t s) {
    const dim3 grid((hidden + 255) / 256);
    if (weight_kind == 1)
        return vlaunch(embed_kernel<uint16_t>, grid, dim3(256), 0, s, static_cast<const uint16_t*>(embed), st, x,
                       hidden);
    return vlaunch(embed_kernel<float>, grid, dim3(256), 0, s, static_cast<const float*>(embed), st, x, hidden);
}

hipError_t launch_argmax_finish(const unsigned long long* keys, uint32_t nkeys, const float* logits, StepState* st,
                                const uint32_t* prompt, uint32_t* out_tokens, uint32_t out_cap, hipStream_t s) {
    return vlaunch(argmax_finish_kernel, dim3(1), dim3(kFinishThreads), 0, s, keys, nkeys, logits, st, prompt,
                   out_tokens, out_cap);
}

namespace {
__global__ void set_state_kernel(StepState* st, uint32_t token, uint32_t pos, uint32_t prompt_len, uint32_t counting) {
    if (threadIdx.x == 0) {
        st->token = token;
        st->pos = pos;
        st->n_out = 0;
        st->counting = counting;
        st->argmax = 0;
        st->prompt_len = prompt_len;
        st->stop = 0;
    }
}
}  // namespace

hipError_t launch_set_state(StepState* st, uint32_t token, uint32_t pos, uint32_t prompt_len, uint32_t counting,
                            hipStream_t s) {
    return vlaunch(set_state_kernel, dim3(1), dim3(64), 0, s, st, token, pos, prompt_len, counting);
}

}  // namespace vvli
