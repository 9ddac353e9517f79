// gemv.hip -- batch-1 bf16/f32-weight GEMV for gfx950.
//
// Reference op: linearInto -> linearRange -> dotBf16 (src/llm.zig:1228-1275,
// 1445-1466): out[r] = sum_k W[r,k] * x[k] (+ bias[r]), bf16 widened exactly
// by <<16, f32 accumulation.
//
// Design: a 256-thread block owns R consecutive rows (R*K*2 contiguous bytes
// of HBM). The K dimension is cut into 16-byte units (8 bf16); thread t takes
// units t, t+256, ... of every row, so each wave load is 1 KiB contiguous and
// every thread reuses its x values across the R rows. Weight loads for the
// first batch are issued before x is staged (x and the RMSNorm scale come from
// LDS), so the x round trip hides under the weight latency. Per-thread partial
// sums are reduced with DPP inside the wave and through LDS across waves.
#include "device_common.hpp"
#include "kernels.hpp"

namespace vvli {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

template <int MODE> struct ModeCfg;
template <> struct ModeCfg<kGemvPlain> { static constexpr int R = 8, UB = 2; };
template <> struct ModeCfg<kGemvResid> { static constexpr int R = 4, UB = 2; };
template <> struct ModeCfg<kGemvGateUp> { static constexpr int R = 4, UB = 2; };
template <> struct ModeCfg<kGemvLogits> { static constexpr int R = 8, UB = 2; };

// Stage x (optionally RMS-normalised: out = x * w * s, s = 1/sqrt(mean(x^2)+eps),
// rmsNormInto src/llm.zig:1287-1300) into LDS.
template <typename WT>
__device__ inline void stage_x(float* xs, float* red, const float* __restrict__ x, const WT* __restrict__ norm_w,
                               float eps, uint32_t K) {
    const int tid = threadIdx.x;
    float ss = 0.f;
    for (uint32_t k = tid * 4; k < K; k += kThreads * 4) {
        float4 v = *reinterpret_cast<const float4*>(x + k);
        *reinterpret_cast<float4*>(xs + k) = v;
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    if (norm_w != nullptr) {
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float total = (red[0] + red[1]) + (red[2] + red[3]);
        float scale = 1.0f / sqrtf(total / (float)K + eps);
        for (uint32_t k = tid; k < K; k += kThreads) xs[k] = xs[k] * WeightTraits<WT>::at(norm_w, k) * scale;
    }
    __syncthreads();
}

template <typename WT, int MODE>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
    using T = WeightTraits<WT>;
    constexpr int E = T::kPerUnit;
    constexpr int R = ModeCfg<MODE>::R;
    constexpr int UB = ModeCfg<MODE>::UB;
    constexpr int NR = (MODE == kGemvGateUp) ? 2 * R : R;

    extern __shared__ float smem[];
    const uint32_t K = a.K;
    float* xs = smem;
    float* red = smem + K;  // kWaves * NR floats

    const int tid = threadIdx.x;
    const uint32_t row0 = blockIdx.x * R;
    int seg = 0;
    uint32_t base = 0;
    if (row0 >= a.rows[0]) {
        base = a.rows[0];
        seg = 1;
        if (row0 >= a.rows[0] + a.rows[1]) {
            base += a.rows[1];
            seg = 2;
        }
    }
    const uint32_t srow = row0 - base;
    const uint32_t seg_rows = a.rows[seg];

    const WT* rowp[NR];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        uint32_t rr = srow + r < seg_rows ? srow + r : seg_rows - 1;
        rowp[r] = static_cast<const WT*>(a.w[seg]) + (size_t)rr * K;
        if constexpr (MODE == kGemvGateUp) rowp[R + r] = static_cast<const WT*>(a.w_up) + (size_t)rr * K;
    }

    const uint32_t U = K / E;
    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = 0.f;

    // First batch of weight loads goes out before x is staged.
    uint4 wv[UB][NR];
    uint32_t u = tid;
#pragma unroll
    for (int b = 0; b < UB; ++b) {
        const uint32_t ub = u + b * kThreads;
#pragma unroll
        for (int r = 0; r < NR; ++r) wv[b][r] = ub < U ? load_unit(rowp[r] + (size_t)ub * E) : make_uint4(0, 0, 0, 0);
    }

    stage_x<WT>(xs, red, a.x, static_cast<const WT*>(a.norm_w), a.eps, K);

    while (true) {
#pragma unroll
        for (int b = 0; b < UB; ++b) {
            const uint32_t ub = u + b * kThreads;
            if (ub < U) {
                float xv[E];
#pragma unroll
                for (int e = 0; e < E; e += 4) {
                    float4 t = *reinterpret_cast<const float4*>(xs + (size_t)ub * E + e);
                    xv[e] = t.x;
                    xv[e + 1] = t.y;
                    xv[e + 2] = t.z;
                    xv[e + 3] = t.w;
                }
#pragma unroll
                for (int r = 0; r < NR; ++r) {
                    float wf[E];
                    T::expand(wv[b][r], wf);
#pragma unroll
                    for (int e = 0; e < E; ++e) acc[r] = fmaf(wf[e], xv[e], acc[r]);
                }
            }
        }
        u += UB * kThreads;
        if (u >= U) break;
#pragma unroll
        for (int b = 0; b < UB; ++b) {
            const uint32_t ub = u + b * kThreads;
#pragma unroll
            for (int r = 0; r < NR; ++r)
                wv[b][r] = ub < U ? load_unit(rowp[r] + (size_t)ub * E) : make_uint4(0, 0, 0, 0);
        }
    }

    // Block reduction: DPP within each wave, LDS across the 4 waves.
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        float s = wave_sum(acc[r]);
        if ((tid & 63) == 0) red[(tid >> 6) * NR + r] = s;
    }
    __syncthreads();
    if constexpr (MODE == kGemvLogits) {
        // Whole wave 0 takes part so the shuffle reduction has every lane.
        if (tid < kWave) {
            const uint32_t row = srow + tid;
            const bool valid = tid < R && row < seg_rows;
            unsigned long long key = 0ull;
            if (valid) {
                float s = (red[tid] + red[NR + tid]) + (red[2 * NR + tid] + red[3 * NR + tid]);
                a.out[0][row] = s;
                key = argmax_key(s, row);
            }
            key = wave_max_u64(key);
            if (tid == 0) a.block_keys[blockIdx.x] = key;
        }
    } else if (tid < R) {
        const int r = tid;
        const uint32_t row = srow + r;
        const bool valid = row < seg_rows;
        float s = (red[r] + red[NR + r]) + (red[2 * NR + r] + red[3 * NR + r]);
        if constexpr (MODE == kGemvPlain) {
            if (valid) {
                const WT* bias = static_cast<const WT*>(a.bias[seg]);
                a.out[seg][row] = s + (bias ? T::at(bias, row) : 0.0f);
            }
        } else if constexpr (MODE == kGemvResid) {
            if (valid) a.out[0][row] = a.out[0][row] + s;
        } else {  // gate/up: siluMulInto, src/llm.zig:1382-1387
            float u_ = (red[R + r] + red[NR + R + r]) + (red[2 * NR + R + r] + red[3 * NR + R + r]);
            if (valid) a.out[0][row] = (s / (1.0f + expf(-s))) * u_;
        }
    }
}

template <typename WT, int MODE>
hipError_t launch_t(const GemvArgs& a, hipStream_t s) {
    constexpr int R = ModeCfg<MODE>::R;
    constexpr int NR = (MODE == kGemvGateUp) ? 2 * R : R;
    const uint32_t total = a.rows[0] + a.rows[1] + a.rows[2];
    const uint32_t grid = (total + R - 1) / R;
    const size_t lds = (size_t)a.K * sizeof(float) + kWaves * NR * sizeof(float);
    hipLaunchKernelGGL((gemv_kernel<WT, MODE>), dim3(grid), dim3(kThreads), lds, s, a);
    return hipGetLastError();
}

template <typename WT, int MODE>
hipError_t set_attr() {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_kernel<WT, MODE>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
}

}  // namespace

uint32_t gemv_rows_per_block(int mode) {
    switch (mode) {
        case kGemvPlain: return ModeCfg<kGemvPlain>::R;
        case kGemvResid: return ModeCfg<kGemvResid>::R;
        case kGemvGateUp: return ModeCfg<kGemvGateUp>::R;
        default: return ModeCfg<kGemvLogits>::R;
    }
}

uint32_t gemv_grid(int mode, uint32_t total_rows) {
    uint32_t r = gemv_rows_per_block(mode);
    return (total_rows + r - 1) / r;
}

hipError_t gemv_init_attributes() {
    hipError_t e = hipSuccess;
#define VVLI_ATTR(WT)                                                  \
    if ((e = set_attr<WT, kGemvPlain>()) != hipSuccess) return e;      \
    if ((e = set_attr<WT, kGemvResid>()) != hipSuccess) return e;      \
    if ((e = set_attr<WT, kGemvGateUp>()) != hipSuccess) return e;     \
    if ((e = set_attr<WT, kGemvLogits>()) != hipSuccess) return e;
    VVLI_ATTR(uint16_t)
    VVLI_ATTR(float)
#undef VVLI_ATTR
    return e;
}

hipError_t launch_gemv(int weight_kind, int mode, const GemvArgs& a, hipStream_t s) {
    if (weight_kind == 1) {
        switch (mode) {
            case kGemvPlain: return launch_t<uint16_t, kGemvPlain>(a, s);
            case kGemvResid: return launch_t<uint16_t, kGemvResid>(a, s);
            case kGemvGateUp: return launch_t<uint16_t, kGemvGateUp>(a, s);
            default: return launch_t<uint16_t, kGemvLogits>(a, s);
        }
    }
    switch (mode) {
        case kGemvPlain: return launch_t<float, kGemvPlain>(a, s);
        case kGemvResid: return launch_t<float, kGemvResid>(a, s);
        case kGemvGateUp: return launch_t<float, kGemvGateUp>(a, s);
        default: return launch_t<float, kGemvLogits>(a, s);
    }
}

}  // namespace vvli
