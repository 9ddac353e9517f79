// linear.hip -- the isolated matmul op of include/vvli_gpu.h: linearInto
// (src/llm.zig:1228-1275) generalised to M activation rows,
// Y[m,n] = sum_k bf16 W[n,k] * X[m,k] (+ bias[n]), f32 accumulation.
//
// Two entry points share one enqueue routine and therefore the same kernels
// and results; they differ only in where the GEMM's activation split planes
// live: vvli_gpu_linear keeps a stream-ordered allocation per stream,
// vvli_gpu_linear_noalloc uses a static device array and allocates nothing.
#include <algorithm>
#include <mutex>
#include <utility>
#include <vector>

#include "internal.hpp"
#include "kernels.hpp"
#include "linear_gemv.hpp"

using namespace vvli;

namespace {

// Rows from which one MFMA kernel replaces the GEMV kernel (linear_gemv.hpp,
// up to 4 rows of x in one launch: 4 only where the skinny kernel would split
// K across blocks, linear_uses_gemv); up to kSkinnyMaxRows the skinny kernel
// below, beyond it the prefill GEMM.
constexpr uint32_t kLinearGemmMinRows = 4;
constexpr uint32_t kSkinnyMaxRows = 64;

// ---------------------------------------------------------------------------
// GEMV plan (M <= 4): one wave per row tile (RW = 1), UL units of 16 bytes per
// lane per item (4, i.e. 4 KiB rows in one item at K = 2048; fewer when rows
// are short), one block of four waves per CU. Measured on the Llama-3.2-1B
// shapes (per-dispatch time, cold weights): more waves per CU or two-row
// tiles are no faster on the 8-33 MB shapes and slower on the 525 MB lm_head
// (4 waves per CU 79.6 us, 8 waves 85.6 us, 16 waves 90.3 us) -- with two
// 4 KiB items per wave in flight, 32 KiB per CU cover the latency, and more
// outstanding requests only add contention.
// ---------------------------------------------------------------------------
constexpr uint32_t kGemvMaxLds = 160 * 1024;

uint32_t gemv_ul(uint32_t K) {
    const uint32_t U = K / 8;
    return U > 128 ? 4 : (U > 64 ? 2 : 1);
}

template <int MR, int UL>
hipError_t launch_gemv_t(const uint16_t* dW, const float* dX, const uint16_t* dBias, float* dY, uint32_t M, uint32_t N,
                         uint32_t K, hipStream_t s) {
    const uint32_t blocks = std::min<uint32_t>((N + kLgWaves - 1) / kLgWaves, 256);
    const size_t lds = (size_t)MR * K * sizeof(float);
    return vlaunch(linear_gemv_kernel<MR, 1, UL>, dim3(blocks), dim3(kLgThreads), lds, s, dW, dX, dBias, dY, M, N, K);
}

// One launch for up to 4 rows of x (x staged in LDS: MR * K * 4 bytes).
hipError_t launch_gemv_rows(const uint16_t* dW, const float* dX, const uint16_t* dBias, float* dY, uint32_t M,
                            uint32_t N, uint32_t K, hipStream_t s) {
    const uint32_t ul = gemv_ul(K);
#define VVLI_GEMV_MR(MR_)                                                                           \
    return ul == 4 ? launch_gemv_t<MR_, 4>(dW, dX, dBias, dY, M, N, K, s)                          \
           : ul == 2 ? launch_gemv_t<MR_, 2>(dW, dX, dBias, dY, M, N, K, s)                        \
                     : launch_gemv_t<MR_, 1>(dW, dX, dBias, dY, M, N, K, s);
    if (M == 1) VVLI_GEMV_MR(1)
    if (M == 2) VVLI_GEMV_MR(2)
    if (M == 3) VVLI_GEMV_MR(3)
    VVLI_GEMV_MR(4)
#undef VVLI_GEMV_MR
}

// ---------------------------------------------------------------------------
// Skinny GEMM (4 <= M <= 64): Y[m][n] = sum_k X[m][k] W[n][k] (+ bias[n]) on
// v_mfma_f32_16x16x32_bf16 in one launch, W streamed from HBM exactly once.
// A block owns NT * 16 rows of W and every row of X; its 8 waves split K into
// contiguous slices of 32-wide steps. Lane l holds the MFMA fragments of row
// l % 16 and k = 32 s + 8 (l / 16) .. + 7 (A = X rows, B = W rows, D[m][n] in
// rows 4 (l / 16) + j, column l % 16): W fragments are 16-byte loads straight
// into registers (a row's two consecutive steps fill one 128-byte line), X
// fragments are 2 x 16-byte f32 loads (X is small and L2-resident), split in
// registers into hi = bf16(x) and lo = bf16(x - hi) so that x . w = hi . w +
// lo . w keeps the f32 activation (bf16 weights are exact in both). Loads run
// one group of DEPTH steps ahead of the MFMAs. The 8 wave partials meet in LDS
// and are summed in wave order (deterministic), plus the bias.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kSkinnyThreads = 512;
constexpr int kSkinnyWaves = kSkinnyThreads / 64;

template <int MT, int NT, int DEPTH>
struct SkinnyGroup {
    uint4 w[DEPTH][NT];
    float4 x[DEPTH][MT][2];
};

template <int MT, int NT, int DEPTH>
__device__ __forceinline__ void skinny_issue(SkinnyGroup<MT, NT, DEPTH>& g, const uint16_t* const (&wrow)[NT],
                                             const float* const (&xrow)[MT], const bool (&xok)[MT], uint32_t s,
                                             uint32_t s_end, uint32_t koff, uint32_t K) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
        const uint32_t k = (s + d) * 32 + koff;
        const bool in = s + d < s_end && k < K;  // K % 8 == 0: a lane's 8 elements are all in or all out
#pragma unroll
        for (int j = 0; j < NT; ++j)
            g.w[d][j] = in ? *reinterpret_cast<const uint4*>(wrow[j] + k) : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            const bool ok = in && xok[i];
            g.x[d][i][0] = ok ? *reinterpret_cast<const float4*>(xrow[i] + k) : make_float4(0.f, 0.f, 0.f, 0.f);
            g.x[d][i][1] = ok ? *reinterpret_cast<const float4*>(xrow[i] + k + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
}

template <int MT, int NT, int DEPTH>
__device__ __forceinline__ void skinny_mfma(const SkinnyGroup<MT, NT, DEPTH>& g, f32x4 (&acc)[MT][NT]) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
        bf16x8 wf[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) wf[j] = __builtin_bit_cast(bf16x8, g.w[d][j]);
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            const float xs[8] = {g.x[d][i][0].x, g.x[d][i][0].y, g.x[d][i][0].z, g.x[d][i][0].w,
                                 g.x[d][i][1].x, g.x[d][i][1].y, g.x[d][i][1].z, g.x[d][i][1].w};
            bf16x8 hi, lo;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const __bf16 h = static_cast<__bf16>(xs[e]);  // round to nearest even
                hi[e] = h;
                lo[e] = static_cast<__bf16>(xs[e] - static_cast<float>(h));
            }
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, wf[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, wf[j], acc[i][j], 0, 0, 0);
            }
        }
    }
}

// K split across blocks (gridDim.y = KS > 1, few row tiles): block (t, ks)
// takes steps [ks * SB, (ks + 1) * SB) and writes its partial to
// ws[ks][m][n]; the last block of row tile t to arrive (counter cnt[t], zero
// between calls) sums the KS partials in ks order, adds the bias, writes Y and
// puts the counter back to zero -- one launch, deterministic results.
template <int MT, int NT, int DEPTH>
__global__ __launch_bounds__(kSkinnyThreads) void linear_skinny_kernel(const uint16_t* __restrict__ W,
                                                                       const float* __restrict__ X,
                                                                       const uint16_t* __restrict__ bias,
                                                                       float* __restrict__ Y, uint32_t M, uint32_t N,
                                                                       uint32_t K, float* ws, uint32_t* cnt) {
    extern __shared__ float red[];  // [wave][MT * 16][NT * 16]
    __shared__ uint32_t s_last;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t r16 = lane & 15, koff = 8 * (lane >> 4);
    const uint32_t n0 = blockIdx.x * (NT * 16);
    const uint32_t KS = gridDim.y, ks = blockIdx.y;
    const uint32_t S = (K + 31) / 32, SB = (S + KS - 1) / KS;
    const uint32_t b0 = min(ks * SB, S), b1 = min(b0 + SB, S);
    const uint32_t per = (b1 - b0 + kSkinnyWaves - 1) / kSkinnyWaves;
    const uint32_t s0 = min(b0 + wave * per, b1), s1 = min(s0 + per, b1);
    const uint16_t* wrow[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) wrow[j] = W + (size_t)min(n0 + 16 * j + r16, N - 1) * K;  // rows past N: masked at the store
    const float* xrow[MT];
    bool xok[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const uint32_t m = 16 * i + r16;
        xok[i] = m < M;
        xrow[i] = X + (size_t)(xok[i] ? m : 0) * K;
    }
    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    SkinnyGroup<MT, NT, DEPTH> ga, gb;
    uint32_t s = s0;
    if (s < s1) skinny_issue(ga, wrow, xrow, xok, s, s1, koff, K);
    while (s < s1) {
        const uint32_t sn = s + DEPTH;
        if (sn < s1) skinny_issue(gb, wrow, xrow, xok, sn, s1, koff, K);
        skinny_mfma(ga, acc);
        s = sn;
        if (s >= s1) break;
        const uint32_t sn2 = s + DEPTH;
        if (sn2 < s1) skinny_issue(ga, wrow, xrow, xok, sn2, s1, koff, K);
        skinny_mfma(gb, acc);
        s = sn2;
    }
    // Wave partials -> LDS, summed in wave order.
    constexpr int RM = MT * 16, RN = NT * 16;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                red[(wave * RM + 16 * i + (lane >> 4) * 4 + e) * RN + 16 * j + r16] = acc[i][j][e];
    __syncthreads();
    for (uint32_t idx = threadIdx.x; idx < (uint32_t)(RM * RN); idx += kSkinnyThreads) {
        const uint32_t m = idx / RN, n = n0 + idx % RN;
        if (m < M && n < N) {
            float v = 0.f;
#pragma unroll
            for (int w2 = 0; w2 < kSkinnyWaves; ++w2) v += red[(w2 * RM + m) * RN + (idx % RN)];
            if (KS > 1) {  // agent-scope (write-through) store: visible to the other XCDs once complete
                __hip_atomic_store(ws + ((size_t)ks * M + m) * N + n, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                if (bias) v += __uint_as_float((uint32_t)bias[n] << 16);
                Y[(size_t)m * N + n] = v;
            }
        }
    }
    if (KS == 1) return;
    // Release side, by hand: every thread waits for its partial stores to
    // complete (s_waitcnt vmcnt(0): the agent-scope stores are issued with
    // sc1, which on gfx950 writes them through the XCD's L2 to the memory
    // side, so a completed store is visible to every XCD) before the block
    // counts itself in. A release fence would add an L2 write-back
    // (buffer_wbl2) of the whole XCD's dirty lines, which nothing here needs:
    // measured, release/acquire fences made the op 5-7x slower.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(cnt + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == KS - 1;
    __syncthreads();
    if (!s_last) return;
    // Acquire side: the last block invalidates its L1 (buffer_inv sc1, no
    // write-back) before reading the partials, which it also reads with
    // agent-scope (sc1) loads.
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    for (uint32_t idx = threadIdx.x; idx < (uint32_t)(RM * RN); idx += kSkinnyThreads) {
        const uint32_t m = idx / RN, n = n0 + idx % RN;
        if (m < M && n < N) {
            float v = 0.f;
            for (uint32_t k2 = 0; k2 < KS; ++k2)
                v += __hip_atomic_load(ws + ((size_t)k2 * M + m) * N + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (bias) v += __uint_as_float((uint32_t)bias[n] << 16);
            Y[(size_t)m * N + n] = v;
        }
    }
    if (threadIdx.x == 0) cnt[blockIdx.x] = 0;  // zero for the next call (the kernel boundary orders it)
}

// Row tiles of the skinny kernel: 32 rows of W per block when that still
// gives a block per CU, 64 for very tall W (fewer re-reads of X), else 16.
uint32_t skinny_nt(uint32_t N) { return N >= 32768 ? 4 : (N >= 256 * 32 ? 2 : 1); }

// Row tiles of the skinny kernel at N rows of W.
uint32_t skinny_tiles(uint32_t N) { return (N + skinny_nt(N) * 16 - 1) / (skinny_nt(N) * 16); }

// K splits, only when the row tiles leave CUs idle (measured: at 256 tiles of
// 8192 x 2048 a split of 2 costs 4 us -- the partials' write-through and the
// last block's sum -- and gains nothing): enough blocks for two per CU, each
// wave keeping >= 8 K steps, at most 8 splits. The hand-off (write-through
// partials, counter, the last block's acquire and ordered sum) costs several
// microseconds, which only long K repays (one session: 2048 x 8192 at
// M = 16 / 32 23.5 / 30.5 us with 4 splits against 25.3 / 38.4 without; 2048 x
// 2048 at M = 16 / 32 8.4 / 12.4 us unsplit against 14.3 / 16.4 with 2 splits
// of 4 steps per wave).
uint32_t skinny_splits(uint32_t N, uint32_t K) {
    const uint32_t tiles = skinny_tiles(N);
    if (tiles >= 256) return 1;
    const uint32_t S = (K + 31) / 32;
    uint32_t ks = (512 + tiles - 1) / tiles;
    ks = std::min(ks, S / (8 * kSkinnyWaves));
    ks = std::min(ks, 8u);
    return ks < 1 ? 1 : ks;
}

template <int MT, int NT, int DEPTH>
hipError_t launch_skinny_t(const uint16_t* dW, const float* dX, const uint16_t* dBias, float* dY, uint32_t M,
                           uint32_t N, uint32_t K, uint32_t ks, float* ws, uint32_t* cnt, hipStream_t s) {
    const size_t lds = (size_t)kSkinnyWaves * MT * 16 * NT * 16 * sizeof(float);
    const dim3 grid((N + NT * 16 - 1) / (NT * 16), ks);
    return vlaunch(linear_skinny_kernel<MT, NT, DEPTH>, grid, dim3(kSkinnyThreads), lds, s, dW, dX, dBias, dY, M, N, K,
                   ws, cnt);
}

hipError_t launch_skinny(const uint16_t* dW, const float* dX, const uint16_t* dBias, float* dY, uint32_t M,
                         uint32_t N, uint32_t K, float* ws, uint32_t* cnt, hipStream_t s) {
    const uint32_t nt = skinny_nt(N), ks = skinny_splits(N, K), mt = (M + 15) / 16;
#define VVLI_SKINNY(MT_, DEPTH_)                                                                          \
    return nt == 4   ? launch_skinny_t<MT_, 4, (DEPTH_ + 1) / 2>(dW, dX, dBias, dY, M, N, K, ks, ws, cnt, s) \
           : nt == 2 ? launch_skinny_t<MT_, 2, DEPTH_>(dW, dX, dBias, dY, M, N, K, ks, ws, cnt, s)       \
                     : launch_skinny_t<MT_, 1, DEPTH_>(dW, dX, dBias, dY, M, N, K, ks, ws, cnt, s);
    if (mt <= 1) VVLI_SKINNY(1, 4)
    if (mt <= 2) VVLI_SKINNY(2, 2)
    VVLI_SKINNY(4, 1)
#undef VVLI_SKINNY
}

// Scratch of a call: [row-tile counters of the K-split skinny kernel,
// kCounterBytes, zero between calls][payload: the GEMM's activation split
// planes (M > 64) or the skinny kernel's K-split partials]. The payload is at
// most VVLI_LINEAR_NOALLOC_SCRATCH_BYTES for the allocation-free entry point,
// whose scratch is one static array on every GPU the library runs on, held
// until the process ends (zero-initialised, so its counters start at zero).
// Host code never passes `scratch` itself (its host-side name is a stand-in,
// not a device address): the address comes from hipGetSymbolAddress, once per
// device (scratch_on_device).
constexpr size_t kCounterBytes = 64 * 1024;
constexpr size_t kNoAllocScratchBytes = static_cast<size_t>(VVLI_LINEAR_NOALLOC_SCRATCH_BYTES);
static __device__ __align__(256) uint16_t scratch[(kCounterBytes + kNoAllocScratchBytes) / sizeof(uint16_t)];

constexpr int kMaxDevices = 64;

#define HIP_TRY(expr)                                                                                   \
    do {                                                                                                \
        hipError_t e_ = (expr);                                                                         \
        if (e_ != hipSuccess)                                                                           \
            return set_error(e_ == hipErrorOutOfMemory ? VVLI_OUT_OF_MEMORY : VVLI_HIP_ERROR, "%s: %s", \
                             #expr, hipGetErrorString(e_));                                             \
    } while (0)

int linear_setup() {
    static std::once_flag flag;
    static hipError_t err = hipSuccess;
    std::call_once(flag, [] {
        err = gemv_init_attributes();
        const void* gemv[] = {reinterpret_cast<const void*>(&linear_gemv_kernel<1, 1, 1>),
                              reinterpret_cast<const void*>(&linear_gemv_kernel<1, 1, 2>),
                              reinterpret_cast<const void*>(&linear_gemv_kernel<1, 1, 4>),
                              reinterpret_cast<const void*>(&linear_gemv_kernel<2, 1, 1>),
                              reinterpret_cast<const void*>(&linear_gemv_kernel<2, 1, 2>),
                              reinterpret_cast<const void*>(&linear_gemv_kernel<2, 1, 4>),
                              reinterpret_cast<const void*>(&linear_gemv_kernel<3, 1, 1>),
                              reinterpret_cast<const void*>(&linear_gemv_kernel<3, 1, 2>),
                              reinterpret_cast<const void*>(&linear_gemv_kernel<3, 1, 4>),
                              reinterpret_cast<const void*>(&linear_gemv_kernel<4, 1, 1>),
                              reinterpret_cast<const void*>(&linear_gemv_kernel<4, 1, 2>),
                              reinterpret_cast<const void*>(&linear_gemv_kernel<4, 1, 4>)};
        for (const void* k : gemv)
            if (err == hipSuccess) err = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, kGemvMaxLds);
        // Skinny variants keep up to 128 KiB of wave partials in LDS.
        const std::pair<const void*, int> skinny[] = {
            {reinterpret_cast<const void*>(&linear_skinny_kernel<1, 1, 4>), 8 * 16 * 16 * 4},
            {reinterpret_cast<const void*>(&linear_skinny_kernel<1, 2, 4>), 8 * 16 * 32 * 4},
            {reinterpret_cast<const void*>(&linear_skinny_kernel<1, 4, 2>), 8 * 16 * 64 * 4},
            {reinterpret_cast<const void*>(&linear_skinny_kernel<2, 1, 2>), 8 * 32 * 16 * 4},
            {reinterpret_cast<const void*>(&linear_skinny_kernel<2, 2, 2>), 8 * 32 * 32 * 4},
            {reinterpret_cast<const void*>(&linear_skinny_kernel<2, 4, 1>), 8 * 32 * 64 * 4},
            {reinterpret_cast<const void*>(&linear_skinny_kernel<4, 1, 1>), 8 * 64 * 16 * 4},
            {reinterpret_cast<const void*>(&linear_skinny_kernel<4, 2, 1>), 8 * 64 * 32 * 4},
            {reinterpret_cast<const void*>(&linear_skinny_kernel<4, 4, 1>), 8 * 64 * 64 * 4}};
        for (const auto& k : skinny)
            if (err == hipSuccess) err = hipFuncSetAttribute(k.first, hipFuncAttributeMaxDynamicSharedMemorySize, k.second);
    });
    HIP_TRY(err);
    return VVLI_OK;
}

int check_linear_args(const void* dW, const void* dX, const void* dY, uint32_t M, uint32_t N, uint32_t K,
                      const char* who) {
    if (!dW || !dX || !dY) return set_error(VVLI_NULL_ARG, "NULL device pointer to %s", who);
    if (M == 0 || N == 0 || K == 0 || K % 8 != 0)
        return set_error(VVLI_INVALID_CONFIG, "bad linear shape M=%u N=%u K=%u (K %% 8 == 0 required)", M, N, K);
    if (M < kLinearGemmMinRows && (size_t)K * sizeof(float) > kGemvMaxLds)
        return set_error(VVLI_INVALID_CONFIG, "linear K=%u too large for M=%u (x is staged in LDS: K <= %zu)", K, M,
                         kGemvMaxLds / sizeof(float));
    return linear_setup();
}

// Payload bytes a call needs beyond the counters (0 and no counters: none).
// M = 4 takes the GEMV kernel where the skinny kernel's row tiles leave CUs
// idle (fewer than 256: the GEMV spreads whole rows over every CU and reads
// the four x rows from LDS; one session: 2048 x 2048 5.7 against 6.4 us
// unsplit and 13.3 split, 512 x 2048 4.8 against 6.1 and 7.4, 2048 x 8192 13.3
// against 17.0 and 19.4). On tall W the skinny kernel stays: 8192 x 2048 11.7
// against 13.0 us, 128256 x 2048 117.9 against 148.9 (the x reads from LDS
// bound the GEMV there).
bool linear_uses_gemv(uint32_t M, uint32_t N, uint32_t K) {
    if (M < kLinearGemmMinRows) return true;
    return M == 4 && skinny_tiles(N) < 256 && (size_t)M * K * sizeof(float) <= kGemvMaxLds;
}

size_t linear_payload_bytes(uint32_t M, uint32_t N, uint32_t K) {
    if (M > kSkinnyMaxRows) return gemm_split_elems(M, K) * sizeof(uint16_t);
    if (linear_uses_gemv(M, N, K)) return 0;
    if (M >= kLinearGemmMinRows) {
        const uint32_t ks = skinny_splits(N, K);
        return ks > 1 ? (size_t)ks * M * N * sizeof(float) : 0;
    }
    return 0;
}

// Enqueue the op on s. scratch: kCounterBytes + linear_payload_bytes of
// device memory laid out as above, or null when the payload is 0.
int linear_enqueue(const uint16_t* dW, const float* dX, const uint16_t* dBias, float* dY, uint32_t M, uint32_t N,
                   uint32_t K, hipStream_t s, char* scratch_mem) {
    if (M >= kLinearGemmMinRows && M <= kSkinnyMaxRows && !linear_uses_gemv(M, N, K)) {
        float* ws = scratch_mem ? reinterpret_cast<float*>(scratch_mem + kCounterBytes) : nullptr;
        uint32_t* cnt = reinterpret_cast<uint32_t*>(scratch_mem);
        HIP_TRY(launch_skinny(dW, dX, dBias, dY, M, N, K, ws, cnt, s));
        return VVLI_OK;
    }
    if (M > kSkinnyMaxRows) {
        // One MFMA GEMM reads W once for all rows; the activations are split
        // hi/lo into a_hl first.
        GemmArgs g;
        g.a = dX, g.lda = K, g.w[0] = dW, g.bias[0] = dBias;
        g.seg_end[0] = g.seg_end[1] = g.seg_end[2] = N;
        g.out = dY, g.ldo = N, g.M = M, g.N = N, g.K = K;
        g.a_hl = reinterpret_cast<uint16_t*>(scratch_mem + kCounterBytes);
        HIP_TRY(launch_gemm_bf16(kGemmPlain, g, s));
        return VVLI_OK;
    }
    // M <= 4: one GEMV launch for all rows when their x fits LDS, else one per row.
    if ((size_t)M * K * sizeof(float) <= kGemvMaxLds) {
        HIP_TRY(launch_gemv_rows(dW, dX, dBias, dY, M, N, K, s));
        return VVLI_OK;
    }
    for (uint32_t mi = 0; mi < M; ++mi)
        HIP_TRY(launch_gemv_rows(dW, dX + static_cast<size_t>(mi) * K, dBias, dY + static_cast<size_t>(mi) * N, 1, N, K,
                                 s));
    return VVLI_OK;
}

// Device address of `scratch` on the current device, looked up on the
// device's first call (hipGetSymbolAddress with that device current) and
// kept per device: every GPU holds its own copy at its own address.
int scratch_on_device(char** out) {
    static std::mutex mu;
    static char* addr[kMaxDevices] = {};
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return set_error(VVLI_INVALID_CONFIG, "device %d out of range", dev);
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(VVLI_HIP_ERROR, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                             hipGetErrorString(e));
        addr[dev] = static_cast<char*>(p);
    }
    *out = addr[dev];
    return VVLI_OK;
}

}  // namespace

extern "C" {

int vvli_gpu_linear(const uint16_t* dW, const float* dX, const uint16_t* dBias, float* dY, uint32_t M, uint32_t N,
                    uint32_t K, void* stream) {
    int rc = check_linear_args(dW, dX, dY, M, N, K, "vvli_gpu_linear");
    if (rc) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t payload = linear_payload_bytes(M, N, K);
    if (payload == 0) return linear_enqueue(dW, dX, dBias, dY, M, N, K, s, nullptr);
    const size_t need = kCounterBytes + payload;
    // The scratch is kept per stream and grows stream-ordered (its counters
    // cleared once per allocation); the lock covers the enqueue, so calls on
    // one stream use it in turn.
    struct StreamScratch {
        hipStream_t stream;
        void* p;
        size_t bytes;
    };
    static std::mutex mu;
    static std::vector<StreamScratch> cache;
    std::lock_guard<std::mutex> lock(mu);
    StreamScratch* sc = nullptr;
    for (StreamScratch& c : cache)
        if (c.stream == s) sc = &c;
    if (!sc) {
        cache.push_back(StreamScratch{s, nullptr, 0});
        sc = &cache.back();
    }
    if (sc->bytes < need) {
        if (sc->p) HIP_TRY(hipFreeAsync(sc->p, s));
        sc->p = nullptr, sc->bytes = 0;
        HIP_TRY(hipMallocAsync(&sc->p, need, s));
        HIP_TRY(hipMemsetAsync(sc->p, 0, kCounterBytes, s));
        sc->bytes = need;
    }
    return linear_enqueue(dW, dX, dBias, dY, M, N, K, s, static_cast<char*>(sc->p));
}

int vvli_gpu_linear_noalloc(const uint16_t* dW, const float* dX, const uint16_t* dBias, float* dY, uint32_t M,
                            uint32_t N, uint32_t K, void* stream) {
    int rc = check_linear_args(dW, dX, dY, M, N, K, "vvli_gpu_linear_noalloc");
    if (rc) return rc;
    const size_t payload = linear_payload_bytes(M, N, K);
    if (payload > kNoAllocScratchBytes)
        return set_error(VVLI_INVALID_CONFIG,
                         "vvli_gpu_linear_noalloc: M=%u N=%u K=%u needs %zu bytes of scratch, more than its %zu", M, N,
                         K, payload, kNoAllocScratchBytes);
    char* mem = nullptr;
    if (payload && (rc = scratch_on_device(&mem))) return rc;
    return linear_enqueue(dW, dX, dBias, dY, M, N, K, static_cast<hipStream_t>(stream), mem);
}

}  // extern "C"
