// linear_gemv.hpp -- the isolated op at M <= 4 (one to four GEMVs over the
// same weights): linearInto / dotBf16 (src/llm.zig:1228-1275, 1445-1466),
// y[m][n] = sum_k bf16 W[n,k] * x[m][k] (+ bias[n]), f32 accumulation.
//
// HBM-bound streaming, sized so that every CU keeps enough bytes in flight
// to cover the memory latency:
//   * A wave owns tiles of RW whole rows, dealt grid-stride over all waves of
//     the grid (wave w: tiles w, w + waves, ...). A row is cut into 16-byte
//     units (8 bf16); lane l takes units l, l + 64, ... so a wave load is
//     1 KiB contiguous, and a tile is walked in items of UL units per lane per
//     row (RW * UL * 16 bytes per lane).
//   * x (MR rows) is copied into LDS with global_load_lds first, so it does
//     not queue behind the weights; then the first two items' loads are
//     issued. From there each item is multiplied while the next is in flight,
//     and its buffer is refilled with the item after that (prefetch distance
//     two, two register buffers). Every load is an unconditional instruction
//     on a clamped address, with out-of-range units masked by integer AND, so
//     the compiler's load-counter waits are exact (no waits behind branches).
//   * A row sum is reduced inside the wave with DPP. Results are parked in
//     lanes (lane j holds result j of a batch of 64) and written with one
//     vector store per batch: on gfx9 loads and stores share one completion
//     counter, so a store per tile would make the next item's load wait for
//     that store's acknowledgement.
// Four waves per block and as many blocks as fit (up to 4 per CU at <= 128
// VGPRs), so that a CU runs up to 16 waves, i.e. up to 32 items in flight.
#pragma once

#include "device_common.hpp"

namespace vvli {

constexpr int kLgThreads = 256;
constexpr int kLgWaves = kLgThreads / kWave;

template <int RW, int UL>
__device__ __forceinline__ void lg_issue(uint4 (&buf)[RW][UL], const uint16_t* __restrict__ W, uint32_t tile,
                                         uint32_t chunk, uint32_t N, uint32_t K, uint32_t U, int lane) {
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const uint32_t row = min(tile * RW + r, N - 1);
        const uint16_t* p = W + (size_t)row * K;
#pragma unroll
        for (int j = 0; j < UL; ++j) {
            const uint32_t u = chunk * (64 * UL) + j * 64 + lane;
            buf[r][j] = load_unit(p + (size_t)min(u, U - 1) * 8);
        }
    }
}

// acc[m][r] += W[r] . x[m] over this lane's units of the item; `live` false
// (a padding item) or a unit past the row end contributes nothing. The
// masking is integer AND on the weight bits, so no branch separates the
// loads in flight from the waits on them.
template <int MR, int RW, int UL>
__device__ __forceinline__ void lg_consume(const uint4 (&buf)[RW][UL], const float* xs, uint32_t chunk, uint32_t K,
                                           uint32_t U, int lane, bool live, float (&acc)[MR][RW]) {
#pragma unroll
    for (int j = 0; j < UL; ++j) {
        const uint32_t u = chunk * (64 * UL) + j * 64 + lane;
        const bool in = live && u < U;
        const uint32_t mask = in ? 0xffffffffu : 0u;
        const uint32_t uc = in ? u : 0;
        float wf[RW][8];
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const uint4 v = make_uint4(buf[r][j].x & mask, buf[r][j].y & mask, buf[r][j].z & mask, buf[r][j].w & mask);
            WeightTraits<uint16_t>::expand(v, wf[r]);
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const float4 a = *reinterpret_cast<const float4*>(xs + (size_t)m * K + (size_t)uc * 8);
            const float4 b = *reinterpret_cast<const float4*>(xs + (size_t)m * K + (size_t)uc * 8 + 4);
            const float xv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[m][r] = fmaf(wf[r][e], xv[e], acc[m][r]);
        }
    }
}

typedef __attribute__((address_space(3))) void lg_lds_void_t;

// s_waitcnt with only the vector-memory count set (n <= 63): expcnt and
// lgkmcnt fields at their maxima (no wait).
template <int N>
__device__ __forceinline__ void lg_wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// M rows of x (M <= MR), N rows of W, K % 8 == 0; LDS MR * K floats.
// x is copied into LDS by global_load_lds before any weight load is issued,
// so its arrival does not queue behind the weights.
template <int MR, int RW, int UL>
__global__ __launch_bounds__(kLgThreads) void linear_gemv_kernel(const uint16_t* __restrict__ W,
                                                                 const float* __restrict__ X,
                                                                 const uint16_t* __restrict__ bias,
                                                                 float* __restrict__ Y, uint32_t M, uint32_t N,
                                                                 uint32_t K) {
    extern __shared__ float xs[];  // [MR][K]
    const int lane = threadIdx.x & 63;
    const uint32_t wid = blockIdx.x * kLgWaves + (threadIdx.x >> 6);
    const uint32_t nw = gridDim.x * kLgWaves;
    const uint32_t U = K / 8;
    const uint32_t nchunk = (U + 64 * UL - 1) / (64 * UL);
    const uint32_t ntiles = (N + RW - 1) / RW;
    const uint32_t my_tiles = wid < ntiles ? (ntiles - 1 - wid) / nw + 1 : 0;
    const uint32_t n_items = my_tiles * nchunk;
    // Item i of this wave: tile wid + (i / nchunk) * nw, chunk i % nchunk.
    // Loads always name an item (clamped to the last one, or to tile wid for
    // a wave without items: rows are clamped to N - 1), so every issue is
    // unconditional; a clamped repeat reads lines just fetched (L2 hits).
    const uint32_t last = n_items > 0 ? n_items - 1 : 0;
    auto issue_item = [&](uint4(&buf)[RW][UL], uint32_t i) {
        i = min(i, last);
        lg_issue<RW, UL>(buf, W, wid + (i / nchunk) * nw, i % nchunk, N, K, U, lane);
    };

    // x (M rows; rows M..MR-1 of the LDS copy stay unused): wave-contiguous
    // 1 KiB copies, lane l of a wave's slot q0 landing at 16 * (q0 + l) bytes.
    const uint32_t nq = M * K / 4;
    for (uint32_t q0 = (threadIdx.x & ~63u); q0 < nq; q0 += kLgThreads) {
        const uint32_t q = q0 + lane;
        if (q < nq) __builtin_amdgcn_global_load_lds(X + (size_t)q * 4, (lg_lds_void_t*)(xs + (size_t)q0 * 4), 16, 0, 0);
    }
    uint4 bufA[RW][UL], bufB[RW][UL];
    issue_item(bufA, 0);
    issue_item(bufB, 1);
    // Wait for this wave's copies and the two items together: the compiler
    // treats an LDS copy as pending until a full wait, and a partial one here
    // would leave it waiting for everything before every LDS read of the
    // loop below (instead of the exact per-buffer counts it emits now).
    lg_wait_vm<0>();
    __builtin_amdgcn_s_barrier();  // every wave's copies are in LDS

    float acc[MR][RW];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int r = 0; r < RW; ++r) acc[m][r] = 0.f;
    float park[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) park[m] = 0.f;
    constexpr uint32_t kBatchTiles = 64 / RW;
    uint32_t batch_first = 0;  // tile ordinal of the batch's first tile

    // Tile ordinal `ord` is complete: reduce its rows, park them in lanes,
    // and store a full (or the final) batch with one store per x row.
    auto finish = [&](uint32_t ord) {
        const uint32_t slot = (ord - batch_first) * RW;
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                const float v = wave_sum(acc[m][r]);
                acc[m][r] = 0.f;
                if ((uint32_t)lane == slot + r) park[m] = v;
            }
        if (ord + 1 - batch_first == kBatchTiles || ord + 1 == my_tiles) {
            // Lane j: row RW * (tile of ordinal batch_first + j / RW) + j % RW.
            const uint32_t t = wid + (batch_first + lane / RW) * nw;
            const uint32_t row = t * RW + lane % RW;
            if ((uint32_t)lane < (ord + 1 - batch_first) * RW && row < N) {
                const float b = bias ? __uint_as_float((uint32_t)bias[row] << 16) : 0.f;
#pragma unroll
                for (int m = 0; m < MR; ++m)
                    if ((uint32_t)m < M) Y[(size_t)m * N + row] = park[m] + b;
            }
            batch_first = ord + 1;
        }
    };

    // Items in pairs (A: even, B: odd); an odd count ends with a padding B
    // item that is loaded (a clamped repeat) but masked out of the sums.
    for (uint32_t it = 0; it < n_items; it += 2) {
        lg_consume<MR, RW, UL>(bufA, xs, it % nchunk, K, U, lane, true, acc);
        issue_item(bufA, it + 2);
        if (it % nchunk == nchunk - 1) finish(it / nchunk);
        const bool live = it + 1 < n_items;
        lg_consume<MR, RW, UL>(bufB, xs, (it + 1) % nchunk, K, U, lane, live, acc);
        issue_item(bufB, it + 3);
        if (live && (it + 1) % nchunk == nchunk - 1) finish((it + 1) / nchunk);
    }
}

}  // namespace vvli
