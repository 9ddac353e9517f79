// linear.hip -- the isolated matmul op of include/vvli_gpu.h: linearInto
// (src/llm.zig:1228-1275) generalised to M activation rows,
// Y[m,n] = sum_k bf16 W[n,k] * X[m,k] (+ bias[n]), f32 accumulation.
//
// Two entry points share one enqueue routine and therefore the same kernels
// and results; they differ only in where the GEMM's activation split planes
// live: vvli_gpu_linear keeps a stream-ordered allocation per stream,
// vvli_gpu_linear_noalloc uses a static device array and allocates nothing.
#include <mutex>
#include <vector>

#include "internal.hpp"
#include "kernels.hpp"

using namespace vvli;

namespace {

// Rows from which one MFMA GEMM replaces a GEMV launch per row.
constexpr uint32_t kLinearGemmMinRows = 4;

// Split planes of vvli_gpu_linear_noalloc: one array on every GPU the library
// runs on, held until the process ends. Host code never passes `scratch`
// itself (its host-side name is a stand-in, not a device address): the
// address comes from hipGetSymbolAddress, once per device (scratch_on_device).
constexpr size_t kNoAllocScratchBytes = static_cast<size_t>(VVLI_LINEAR_NOALLOC_SCRATCH_BYTES);
static __device__ __align__(256) uint16_t scratch[kNoAllocScratchBytes / sizeof(uint16_t)];

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
    std::call_once(flag, [] { err = gemv_init_attributes(); });
    HIP_TRY(err);
    return VVLI_OK;
}

int check_linear_args(const void* dW, const void* dX, const void* dY, uint32_t M, uint32_t N, uint32_t K,
                      const char* who) {
    if (!dW || !dX || !dY) return set_error(VVLI_NULL_ARG, "NULL device pointer to %s", who);
    if (M == 0 || N == 0 || K == 0 || K % 8 != 0)
        return set_error(VVLI_INVALID_CONFIG, "bad linear shape M=%u N=%u K=%u (K %% 8 == 0 required)", M, N, K);
    return linear_setup();
}

// Bytes of split planes a call needs (0: the GEMV path, no scratch).
size_t linear_scratch_bytes(uint32_t M, uint32_t K) {
    return M >= kLinearGemmMinRows ? gemm_split_elems(M, K) * sizeof(uint16_t) : 0;
}

// Enqueue the op on s. a_hl: linear_scratch_bytes(M, K) of device memory
// (unused by the GEMV path).
int linear_enqueue(const uint16_t* dW, const float* dX, const uint16_t* dBias, float* dY, uint32_t M, uint32_t N,
                   uint32_t K, hipStream_t s, uint16_t* a_hl) {
    if (M >= kLinearGemmMinRows) {
        // One MFMA GEMM reads W once for all rows; the activations are split
        // hi/lo into a_hl first.
        GemmArgs g;
        g.a = dX, g.lda = K, g.w[0] = dW, g.bias[0] = dBias;
        g.seg_end[0] = g.seg_end[1] = g.seg_end[2] = N;
        g.out = dY, g.ldo = N, g.M = M, g.N = N, g.K = K;
        g.a_hl = a_hl;
        HIP_TRY(launch_gemm_bf16(kGemmPlain, g, s));
        return VVLI_OK;
    }
    for (uint32_t mi = 0; mi < M; ++mi) {
        GemvArgs g;
        g.w[0] = dW;
        g.bias[0] = dBias;
        g.out[0] = dY + static_cast<size_t>(mi) * N;
        g.rows[0] = N;
        g.x = dX + static_cast<size_t>(mi) * K;
        g.K = K;
        HIP_TRY(launch_gemv(VVLI_WEIGHT_BF16, kGemvPlain, g, s));
    }
    return VVLI_OK;
}

// Device address of `scratch` on the current device, looked up on the
// device's first call (hipGetSymbolAddress with that device current) and
// kept per device: every GPU holds its own copy at its own address.
int scratch_on_device(uint16_t** out) {
    static std::mutex mu;
    static uint16_t* addr[kMaxDevices] = {};
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
        addr[dev] = static_cast<uint16_t*>(p);
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
    const size_t need = linear_scratch_bytes(M, K);
    if (need == 0) return linear_enqueue(dW, dX, dBias, dY, M, N, K, s, nullptr);
    // The split scratch is kept per stream and grows stream-ordered; the lock
    // covers the enqueue, so calls on one stream use it in turn.
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
        sc->bytes = need;
    }
    return linear_enqueue(dW, dX, dBias, dY, M, N, K, s, static_cast<uint16_t*>(sc->p));
}

int vvli_gpu_linear_noalloc(const uint16_t* dW, const float* dX, const uint16_t* dBias, float* dY, uint32_t M,
                            uint32_t N, uint32_t K, void* stream) {
    int rc = check_linear_args(dW, dX, dY, M, N, K, "vvli_gpu_linear_noalloc");
    if (rc) return rc;
    const size_t need = linear_scratch_bytes(M, K);
    if (need > kNoAllocScratchBytes)
        return set_error(VVLI_INVALID_CONFIG,
                         "vvli_gpu_linear_noalloc: M=%u K=%u needs %zu bytes of split scratch, more than its %zu",
                         M, K, need, kNoAllocScratchBytes);
    uint16_t* a_hl = nullptr;
    if (need && (rc = scratch_on_device(&a_hl))) return rc;
    return linear_enqueue(dW, dX, dBias, dY, M, N, K, static_cast<hipStream_t>(stream), a_hl);
}

}  // extern "C"
