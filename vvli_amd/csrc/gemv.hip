// gemv.hip -- batch-1 bf16/f32-weight GEMV for gfx950.
//
// Reference op: linearInto -> linearRange -> dotBf16 (src/llm.zig:1228-1275,
// 1445-1466): out[r] = sum_k W[r,k] * x[k] (+ bias[r]), bf16 widened exactly
// by <<16, f32 accumulation.
//
// Design (HBM-bound streaming):
//   * The block stages x in LDS once (optionally RMS-normalised:
//     x * w * (1/sqrt(mean(x^2) + eps)), rmsNormInto src/llm.zig:1287-1300).
//   * Work unit = a wave-tile of R rows (R gate rows + R up rows in the
//     SwiGLU mode). A row is cut into 16-byte units (8 bf16); lane l takes
//     units l, l+64, ... so every wave load is 1 KiB contiguous. A tile is
//     walked in "items" of NJC units per lane per row.
//   * Waves take tiles grid-stride. Items are double-buffered in registers:
//     the loads of item i+1 are in flight while item i is multiplied, and the
//     first item's loads are issued before x is staged.
//   * A row's partial sums are reduced inside the wave with DPP; lane 0
//     applies the fused epilogue (bias, residual add, SiLU*up, argmax key).
#include "device_common.hpp"
#include "gemv_tile.hpp"
#include "kernels.hpp"

namespace vvli {

namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;
constexpr uint32_t kMaxBlocks = 1024;

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
        float total = 0.f;
#pragma unroll
        for (int w = 0; w < kWavesPerBlock; ++w) total += red[w];
        const float scale = 1.0f / sqrtf(total / (float)K + eps);
        for (uint32_t k = tid; k < K; k += kThreads) xs[k] = xs[k] * WeightTraits<WT>::at(norm_w, k) * scale;
    }
    __syncthreads();
}

template <typename WT, int MODE>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
    constexpr int R = ModeCfg<MODE>::R;
    constexpr int NR = (MODE == kGemvGateUp ? 2 : 1) * R;
    constexpr int E = WeightTraits<WT>::kPerUnit;
    using TileT = Tile<WT, MODE, NR>;

    extern __shared__ float smem[];
    const uint32_t K = a.K;
    float* xs = smem;
    float* red = smem + K;
    const int lane = threadIdx.x & 63;
    const uint32_t wid = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const uint32_t nwaves = gridDim.x * kWavesPerBlock;
    const uint32_t U = K / E;
    const uint32_t per_item = kNJC * kWave;
    const uint32_t nchunk = (U + per_item - 1) / per_item;
    const uint32_t total = a.rows[0] + a.rows[1] + a.rows[2];
    const uint32_t ntiles = (total + R - 1) / R;
    // Items of this wave: (tile, chunk) for tile = wid, wid + nwaves, ...
    const uint32_t my_tiles = wid < ntiles ? (ntiles - 1 - wid) / nwaves + 1 : 0;
    const uint32_t n_items = my_tiles * nchunk;

    uint4 bufA[NR][kNJC], bufB[NR][kNJC];
    TileT tA, tB;
    uint32_t item = 0;
    if (n_items > 0) {
        make_tile<WT, MODE>(a, wid, K, tA);
        issue<WT, NR>(bufA, tA.p, 0, U, lane);
    }
    stage_x<WT>(xs, red, a.x, static_cast<const WT*>(a.norm_w), a.eps, K);

    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = 0.f;
    unsigned long long best = 0ull;

    // Process item `it` held in `cur`/`tc`; prefetch item it+1 into `nxt`/`tn`.
    auto step = [&](uint4(&cur)[NR][kNJC], TileT& tc, uint4(&nxt)[NR][kNJC], TileT& tn, uint32_t it) {
        const uint32_t chunk = it % nchunk;
        if (it + 1 < n_items) {
            const uint32_t nit = it + 1, nch = nit % nchunk;
            if (nch == 0) make_tile<WT, MODE>(a, wid + (nit / nchunk) * nwaves, K, tn);
            else tn = tc;
            issue<WT, NR>(nxt, tn.p, nch * per_item, U, lane);
        }
        consume<WT, NR>(cur, xs, chunk * per_item, U, lane, acc);
        if (chunk == nchunk - 1) {
            float s[NR];
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                s[r] = wave_sum(acc[r]);
                acc[r] = 0.f;
            }
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    if (!tc.valid[r]) continue;
                    const uint32_t row = tc.row[r];
                    if constexpr (MODE == kGemvPlain) {
                        const WT* bias = static_cast<const WT*>(a.bias[tc.seg[r]]);
                        a.out[tc.seg[r]][row] = s[r] + (bias ? WeightTraits<WT>::at(bias, row) : 0.0f);
                    } else if constexpr (MODE == kGemvResid) {
                        a.out[0][row] = a.out[0][row] + s[r];
                    } else if constexpr (MODE == kGemvGateUp) {
                        // siluMulInto, src/llm.zig:1382-1387
                        const float g = s[r], u = s[R + r];
                        a.out[0][row] = (g / (1.0f + expf(-g))) * u;
                    } else {
                        a.out[0][row] = s[r];
                        const unsigned long long key = argmax_key(s[r], row);
                        best = key > best ? key : best;
                    }
                }
            }
        }
    };

    while (item < n_items) {
        step(bufA, tA, bufB, tB, item);
        ++item;
        if (item >= n_items) break;
        step(bufB, tB, bufA, tA, item);
        ++item;
    }
    if constexpr (MODE == kGemvLogits) {
        if (lane == 0) a.block_keys[wid] = best;
    }
}

template <typename WT, int MODE>
hipError_t launch_t(const GemvArgs& a, hipStream_t s) {
    const uint32_t total = a.rows[0] + a.rows[1] + a.rows[2];
    const uint32_t grid = gemv_grid(MODE, total);
    const size_t lds = (size_t)a.K * sizeof(float) + kWavesPerBlock * sizeof(float);
    return vlaunch(gemv_kernel<WT, MODE>, dim3(grid), dim3(kThreads), lds, s, a);
}

template <typename WT, int MODE>
hipError_t set_attr() {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_kernel<WT, MODE>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
}

}  // namespace

uint32_t gemv_rows_per_block(int mode) {
    // Rows per wave-tile; stacked q|k|v segments must split on tile boundaries.
    return mode == kGemvGateUp ? ModeCfg<kGemvGateUp>::R : ModeCfg<kGemvPlain>::R;
}

uint32_t gemv_grid(int mode, uint32_t total_rows) {
    const uint32_t r = gemv_rows_per_block(mode);
    const uint32_t tiles = (total_rows + r - 1) / r;
    uint32_t blocks = (tiles + kWavesPerBlock - 1) / kWavesPerBlock;
    return blocks > kMaxBlocks ? kMaxBlocks : blocks;
}

uint32_t gemv_num_keys(uint32_t total_rows) { return gemv_grid(kGemvLogits, total_rows) * kWavesPerBlock; }

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
