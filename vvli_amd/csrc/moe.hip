// moe.hip -- mixture-of-experts pieces of the token step (OLMoE form).
//
// The reference has no MoE forward pass (its runner rejects such configs,
// src/llm.zig:218-223,426); the semantics follow HF transformers' OLMoE
// (models/olmoe/modeling_olmoe.py, transformers 5.15):
//   qk-norm   q = w_q * (q * 1/sqrt(mean(q^2) + eps)) over the full q, same for k
//   router    p = softmax(W_r . norm(x)) in f32, the top-k by p (ties: lower
//             expert id), weights p_k without renormalisation
//   experts   act_k = silu(gate_k) * up_k (fused [2I][H] gate|up matrix),
//             out_k = W_down,k . act_k
//   combine   x += sum over the selected experts in ascending expert id of
//             (out_k * p_k)
// Every step reads the selected experts from device memory, so the token
// step stays one replayable graph with no host round trip.
#include "device_common.hpp"
#include "gemv_tile.hpp"
#include "kernels.hpp"

namespace vvli {

namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;

__device__ inline float bf(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// One block per vector: block 0 normalises q (nq values), block 1 k (nk).
__global__ __launch_bounds__(kThreads) void qk_norm_kernel(float* __restrict__ q, const uint16_t* __restrict__ wq,
                                                          uint32_t nq, float* __restrict__ k,
                                                          const uint16_t* __restrict__ wk, uint32_t nk, float eps) {
    __shared__ float red[kWavesPerBlock];
    float* v = blockIdx.x == 0 ? q : k;
    const uint16_t* w = blockIdx.x == 0 ? wq : wk;
    const uint32_t n = blockIdx.x == 0 ? nq : nk;
    float ss = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += kThreads) ss = fmaf(v[i], v[i], ss);
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int i = 0; i < kWavesPerBlock; ++i) total += red[i];
    const float s = 1.0f / sqrtf(total / static_cast<float>(n) + eps);
    for (uint32_t i = threadIdx.x; i < n; i += kThreads) v[i] = bf(w[i]) * (v[i] * s);
}

// One wave: softmax over E <= 256 router logits, then top-k.
__global__ __launch_bounds__(64) void moe_route_kernel(const float* __restrict__ logits, uint32_t E, uint32_t top_k,
                                                      uint32_t* __restrict__ idx, float* __restrict__ weight) {
    const int lane = threadIdx.x;
    float p[4];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t e = lane + 64 * j;
        p[j] = e < E ? logits[e] : -INFINITY;
        mx = fmaxf(mx, p[j]);
    }
    mx = wave_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t e = lane + 64 * j;
        p[j] = e < E ? expf(p[j] - mx) : 0.f;
        sum += p[j];
    }
    sum = wave_sum(sum);
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] = p[j] / sum;
    // Key: probability bits + 1 (non-negative floats order as integers), then
    // the inverted id, so the maximum key is the highest probability, lowest id.
    uint32_t taken = 0;
    for (uint32_t r = 0; r < top_k; ++r) {
        unsigned long long best = 0ull;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t e = lane + 64 * j;
            if (e >= E || (taken >> j) & 1u) continue;
            const unsigned long long key =
                (static_cast<unsigned long long>(__float_as_uint(p[j]) + 1u) << 32) | (0xffffffffu - e);
            best = key > best ? key : best;
        }
        best = wave_max_u64(best);
        const uint32_t e = 0xffffffffu - static_cast<uint32_t>(best & 0xffffffffull);
        if (lane == 0) {
            idx[r] = e;
            weight[r] = __uint_as_float(static_cast<uint32_t>(best >> 32) - 1u);
        }
        if (static_cast<uint32_t>(lane) == e % 64) taken |= 1u << (e / 64);
    }
}

// Stages x (x_len floats) in LDS, optionally RMS-normalised (x * w) * s.
__device__ inline void moe_stage_x(float* xs, float* red, const float* __restrict__ x,
                                   const uint16_t* __restrict__ norm_w, float eps, uint32_t x_len) {
    const int tid = threadIdx.x;
    float ss = 0.f;
    for (uint32_t i = tid * 4; i < x_len; i += kThreads * 4) {
        const float4 v = *reinterpret_cast<const float4*>(x + i);
        *reinterpret_cast<float4*>(xs + i) = v;
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    if (norm_w != nullptr) {
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float total = 0.f;
#pragma unroll
        for (int w = 0; w < kWavesPerBlock; ++w) total += red[w];
        const float scale = 1.0f / sqrtf(total / static_cast<float>(x_len) + eps);
        for (uint32_t i = tid; i < x_len; i += kThreads) xs[i] = xs[i] * bf(norm_w[i]) * scale;
    }
    __syncthreads();
}

// Expert GEMVs. GateUp: rows g = slot * I + r of the selected experts' gate and
// up matrices (one gate + one up row per wave tile), x = norm(resid), output
// act[g] = silu(gate) * up. Down: rows g = slot * H + r of the selected
// experts' down matrices (two rows per tile, same slot since H is even), x =
// act (all slots staged), each tile reading its slot's I values; output
// partial[g]. Loads, double buffering and the dot products are the dense
// GEMV's (gemv_tile.hpp).
template <int MODE>
__global__ __launch_bounds__(kThreads) void moe_gemv_kernel(MoeGemvArgs a) {
    constexpr int R = MODE == kGemvGateUp ? 1 : 2;
    constexpr int NR = 2;  // GateUp: gate + up; Down: two rows
    constexpr int E = 8;   // bf16 per 16-byte unit
    extern __shared__ float smem[];
    float* xs = smem;
    float* red = smem + a.x_len;
    const int lane = threadIdx.x & 63;
    const uint32_t wid = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const uint32_t nwaves = gridDim.x * kWavesPerBlock;
    const uint32_t K = a.K;
    const uint32_t U = K / E;
    const uint32_t per_item = kNJC * kWave;
    const uint32_t nchunk = (U + per_item - 1) / per_item;
    const uint32_t total = a.top_k * a.rows_per_slot;
    const uint32_t ntiles = (total + R - 1) / R;
    const uint32_t my_tiles = wid < ntiles ? (ntiles - 1 - wid) / nwaves + 1 : 0;
    const uint32_t n_items = my_tiles * nchunk;

    struct MTile {
        const uint16_t* p[NR];
        uint32_t row0;
        uint32_t xoff;
    };
    auto make = [&](uint32_t tile, MTile& t) {
        const uint32_t g0 = tile * R;
        const uint32_t slot = g0 / a.rows_per_slot, r = g0 % a.rows_per_slot;
        const uint32_t e = a.experts[slot];
        t.row0 = g0;
        if (MODE == kGemvGateUp) {
            const uint16_t* base = a.w + static_cast<size_t>(e) * 2 * a.rows_per_slot * K;
            t.p[0] = base + static_cast<size_t>(r) * K;
            t.p[1] = base + static_cast<size_t>(a.rows_per_slot + r) * K;
            t.xoff = 0;
        } else {
            const uint16_t* base = a.w + static_cast<size_t>(e) * a.rows_per_slot * K;
            t.p[0] = base + static_cast<size_t>(r) * K;
            t.p[1] = t.p[0] + K;  // rows_per_slot is even: the pair stays in one slot
            t.xoff = slot * K;
        }
    };

    uint4 bufA[NR][kNJC], bufB[NR][kNJC];
    MTile tA, tB;
    if (n_items > 0) {
        make(wid, tA);
        issue<uint16_t, NR>(bufA, tA.p, 0, U, lane);
    }
    moe_stage_x(xs, red, a.x, a.norm_w, a.eps, a.x_len);

    float acc[NR] = {0.f, 0.f};
    auto step = [&](uint4(&cur)[NR][kNJC], MTile& tc, uint4(&nxt)[NR][kNJC], MTile& tn, uint32_t it) {
        const uint32_t chunk = it % nchunk;
        if (it + 1 < n_items) {
            const uint32_t nit = it + 1, nch = nit % nchunk;
            if (nch == 0) make(wid + (nit / nchunk) * nwaves, tn);
            else tn = tc;
            issue<uint16_t, NR>(nxt, tn.p, nch * per_item, U, lane);
        }
        consume<uint16_t, NR>(cur, xs + tc.xoff, chunk * per_item, U, lane, acc);
        if (chunk == nchunk - 1) {
            const float s0 = wave_sum(acc[0]), s1 = wave_sum(acc[1]);
            acc[0] = acc[1] = 0.f;
            if (lane == 0) {
                if (MODE == kGemvGateUp) {
                    a.out[tc.row0] = __fmul_rn(__fdiv_rn(s0, __fadd_rn(1.0f, expf(-s0))), s1);
                } else {
                    a.out[tc.row0] = s0;
                    a.out[tc.row0 + 1] = s1;
                }
            }
        }
    };
    uint32_t item = 0;
    while (item < n_items) {
        step(bufA, tA, bufB, tB, item);
        if (++item >= n_items) break;
        step(bufB, tB, bufA, tA, item);
        ++item;
    }
}

// x[r] += sum over slots in ascending expert id of partial[slot][r] * w[slot].
__global__ __launch_bounds__(kThreads) void moe_combine_kernel(float* __restrict__ x, const float* __restrict__ partial,
                                                              const uint32_t* __restrict__ idx,
                                                              const float* __restrict__ w, uint32_t top_k,
                                                              uint32_t H) {
    const uint32_t r = blockIdx.x * kThreads + threadIdx.x;
    if (r >= H) return;
    uint32_t order[kMaxTopK];
    for (uint32_t i = 0; i < top_k; ++i) order[i] = i;
    for (uint32_t i = 1; i < top_k; ++i)  // insertion sort by expert id (top_k <= 16)
        for (uint32_t j = i; j > 0 && idx[order[j - 1]] > idx[order[j]]; --j) {
            const uint32_t t = order[j];
            order[j] = order[j - 1];
            order[j - 1] = t;
        }
    float s = 0.f;
    for (uint32_t i = 0; i < top_k; ++i) {
        const uint32_t slot = order[i];
        s = __fadd_rn(s, __fmul_rn(partial[static_cast<size_t>(slot) * H + r], w[slot]));
    }
    x[r] = __fadd_rn(x[r], s);
}

}  // namespace

hipError_t launch_qk_norm(float* q, const uint16_t* wq, uint32_t nq, float* k, const uint16_t* wk, uint32_t nk,
                          float eps, hipStream_t s) {
    return vlaunch(qk_norm_kernel, dim3(2), dim3(kThreads), 0, s, q, wq, nq, k, wk, nk, eps);
}

hipError_t launch_moe_route(const float* logits, uint32_t E, uint32_t top_k, uint32_t* idx, float* weight,
                            hipStream_t s) {
    if (E == 0 || E > 256 || top_k == 0 || top_k > E || top_k > static_cast<uint32_t>(kMaxTopK))
        return hipErrorInvalidValue;
    return vlaunch(moe_route_kernel, dim3(1), dim3(64), 0, s, logits, E, top_k, idx, weight);
}

hipError_t moe_gemv_init_attributes() {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&moe_gemv_kernel<kGemvGateUp>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&moe_gemv_kernel<kGemvPlain>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
}

hipError_t launch_moe_gemv(int mode, const MoeGemvArgs& a, hipStream_t s) {
    if (a.K % 8 != 0 || a.x_len % 4 != 0 || (mode != kGemvGateUp && a.rows_per_slot % 2 != 0))
        return hipErrorInvalidValue;
    const uint32_t R = mode == kGemvGateUp ? 1 : 2;
    const uint32_t tiles = (a.top_k * a.rows_per_slot + R - 1) / R;
    uint32_t blocks = (tiles + kWavesPerBlock - 1) / kWavesPerBlock;
    if (blocks > 1024) blocks = 1024;
    const size_t lds = (static_cast<size_t>(a.x_len) + kWavesPerBlock) * sizeof(float);
    if (mode == kGemvGateUp) return vlaunch(moe_gemv_kernel<kGemvGateUp>, dim3(blocks), dim3(kThreads), lds, s, a);
    return vlaunch(moe_gemv_kernel<kGemvPlain>, dim3(blocks), dim3(kThreads), lds, s, a);
}

hipError_t launch_moe_combine(float* x, const float* partial, const uint32_t* idx, const float* w, uint32_t top_k,
                              uint32_t H, hipStream_t s) {
    if (top_k > static_cast<uint32_t>(kMaxTopK)) return hipErrorInvalidValue;
    return vlaunch(moe_combine_kernel, dim3((H + kThreads - 1) / kThreads), dim3(kThreads), 0, s, x, partial, idx, w,
                   top_k, H);
}

}  // namespace vvli
