// sample.hip -- on-device token sampling: VVLI's Sampler.next
// (src/generator.zig:93-120) with its helpers (:335-463) and PRNG.
//
// One 1024-thread block per step, on the logits the step just wrote:
//   scores   s_i = adjustedLogit(l_i, count_i) (repeat penalty, :391-394)
//   T <= 0   greedyWithPenalties (:353-365): first index of the strict max
//   T > 0    candidates = the top_k largest finite scores, descending, ties
//            to the lower id (buildCandidates + insertTopCandidate), found by
//            a 4-pass radix select on order-preserving score keys, gathered
//            and bitonic-sorted in LDS (top_k <= 1024);
//            p_i = exp((s_i - s_0) / T) in parallel, then one thread sums
//            them in candidate order, applies the top_p cut (:428-449), draws
//            u = Random.float(f32) from Zig's DefaultPrng (xoshiro256++,
//            state in device memory) and walks the cumulative sum
//            (sampleCandidate, :451-463).
// Sequential f32 sums in candidate order keep the reference's rounding.
//
// Whole-vocabulary candidates (limit over 1024: top_k 0, which buildCandidates
// treats as "every finite score, sorted", :376-391, or top_k > 1024):
// sample_full_keys_kernel writes each id's order-preserving score key (0 for
// a non-finite score), rocPRIM's stable radix sort orders the (key, id) pairs
// descending -- ties keep ascending ids, the order insertTopCandidate gives
// and the oracle uses for the reference's unstable sort -- and
// sample_full_kernel takes the first min(limit, finite) of them: the
// probabilities in parallel, then one lane's single pass of sequential f32
// prefix sums in candidate order (the running sum of prepareProbabilities'
// total, of its top-p scan and of sampleCandidate's sums are the same
// sequence), then the top-p cut and the pick as searches over those sums.
//
// Two-stage top-k (top_k <= 128, at most 64 slices, scratch of
// sample_cand_elems keys given):
// sample_local_kernel cuts the vocab into slices of 4096 ids, one block each,
// and writes a slice's top_k keys (score key << 32 | ~id; 0 for a non-finite
// score), descending, with its finite count: each wave takes the top_k of its
// 256 ids (top_k rounds of a wave max over keys held in registers) and the
// first wave merges the 16 lists. The keys are distinct, so every member of
// the global top_k is in its slice's top_k; the sampling block's first wave then merges
// the slices' sorted lists (one list head per lane) instead of scanning the
// vocab (one block's scan is ~1 ms at a 128K vocab).
#include <rocprim/device/device_radix_sort.hpp>

#include "device_common.hpp"
#include "kernels.hpp"

namespace vvli {

namespace {

constexpr int kT = 1024;  // threads of the sampling block
constexpr int kMaxCand = kMaxSampleTopK;

__device__ inline float adjusted(float logit, uint32_t count, float penalty) {
    if (count == 0 || penalty <= 1.0f) return logit;
    return logit < 0.0f ? __fmul_rn(logit, penalty) : __fdiv_rn(logit, penalty);
}

// Order-preserving key of a finite float (larger float -> larger key), >= 1;
// -0 and +0 share a key, as they compare equal.
__device__ inline uint32_t order_key(float v) {
    const uint32_t b = v == 0.0f ? 0u : __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ inline float key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
__device__ inline uint64_t xoshiro_next(uint64_t* s) {
    const uint64_t result = rotl64(s[0] + s[3], 23) + s[0];
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return result;
}
// Random.float(f32) of Zig's std.Random on DefaultPrng.
__device__ inline float prng_float(uint64_t* s) {
    const uint64_t r = xoshiro_next(s);
    uint32_t lz = r ? static_cast<uint32_t>(__clzll(r)) : 64u;
    if (lz >= 41) {
        const uint64_t r2 = xoshiro_next(s);
        lz = 41 + (r2 ? static_cast<uint32_t>(__clzll(r2)) : 64u);
        if (lz == 41 + 64) lz += static_cast<uint32_t>(__clz(static_cast<uint32_t>(xoshiro_next(s)) | 0x7ffu));
    }
    return __uint_as_float(((126u - lz) << 23) | static_cast<uint32_t>(r & 0x7fffffull));
}

constexpr int kLocalIds = 4096;  // vocab slice of a local top-k block
constexpr int kFastTopK = 128;   // largest top_k of the two-stage path
constexpr int kSurvivors = 4096; // slice lists the sampling block stages in LDS (more: merged from scratch)

// Descending bitonic sort of n (a power of two) keys in LDS by the block.
__device__ inline void bitonic_desc(unsigned long long* k, uint32_t n) {
    for (uint32_t size = 2; size <= n; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t j = threadIdx.x; j < n; j += blockDim.x) {
                const uint32_t p = j ^ stride;
                if (p > j) {
                    const bool desc = (j & size) == 0;
                    const unsigned long long x = k[j], y = k[p];
                    if (desc ? (x < y) : (x > y)) {
                        k[j] = y;
                        k[p] = x;
                    }
                }
            }
            __syncthreads();
        }
    }
}

// Max over a fully active wave: DPP within each 16-lane row (quad swaps, then
// half-row and row mirrors; the moves fold into v_max_u32's DPP operand),
// then the four row maxima read out of lanes 0, 16, 32, 48. No LDS round
// trips, unlike a shuffle butterfly.
__device__ inline uint32_t wave_max_u32_dpp(uint32_t x) {
    x = max(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0xB1, 0xf, 0xf, true)));   // quad_perm [1,0,3,2]
    x = max(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x4E, 0xf, 0xf, true)));   // quad_perm [2,3,0,1]
    x = max(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x141, 0xf, 0xf, true)));  // row_half_mirror
    x = max(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x140, 0xf, 0xf, true)));  // row_mirror
    const uint32_t m0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), 0));
    const uint32_t m1 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), 16));
    const uint32_t m2 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), 32));
    const uint32_t m3 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), 48));
    return max(max(m0, m1), max(m2, m3));
}

// 64-bit max as two 32-bit ones: the high halves, then the low halves of the
// lanes holding the maximal high half.
__device__ inline unsigned long long wave_max_dpp(unsigned long long v) {
    const uint32_t hi = static_cast<uint32_t>(v >> 32);
    const uint32_t h = wave_max_u32_dpp(hi);
    const uint32_t l = wave_max_u32_dpp(hi == h ? static_cast<uint32_t>(v) : 0u);
    return (static_cast<unsigned long long>(h) << 32) | l;
}

// Merges up to 64 descending lists (list s at lists[s * len], zero padded;
// keys distinct) with one fully active wave, lane s holding list s's head:
// the k largest keys, descending, to out[0 .. k) (written by lane 0).
__device__ inline void wave_merge(const unsigned long long* lists, uint32_t n_lists, uint32_t len, uint32_t k,
                                  unsigned long long* out) {
    const uint32_t lane = threadIdx.x & 63;
    uint32_t pos = 0;
    unsigned long long head = lane < n_lists ? lists[lane * len] : 0ull;
    for (uint32_t i = 0; i < k; ++i) {
        const unsigned long long b = wave_max_dpp(head);
        if (lane == 0) out[i] = b;
        if (b != 0ull && head == b) {  // the one owner (lanes past n_lists hold 0)
            ++pos;
            head = pos < len ? lists[lane * len + pos] : 0ull;
        }
    }
}

struct SampleShared {
    uint32_t hist[256];
    unsigned long long cand[kMaxCand];  // (score key << 32) | ~id, sorted descending
    float prob[kMaxCand];
    uint32_t scan_gt[kT], scan_eq[kT];
    unsigned long long red[kT / 64];
    unsigned long long surv[kSurvivors];  // two-stage path: the slices' lists
    uint32_t prefix, remaining, n_finite, token;
};

__device__ inline uint32_t block_sum_u32(uint32_t v, unsigned long long* red) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    uint32_t total = 0;
    for (int w = 0; w < kT / 64; ++w) total += static_cast<uint32_t>(red[w]);
    __syncthreads();
    return total;
}

// Inclusive scan of one value per thread (thread order), via LDS.
__device__ inline uint32_t block_exclusive_scan(uint32_t v, uint32_t* buf) {
    buf[threadIdx.x] = v;
    __syncthreads();
    for (int off = 1; off < kT; off <<= 1) {
        const uint32_t add = threadIdx.x >= static_cast<uint32_t>(off) ? buf[threadIdx.x - off] : 0u;
        __syncthreads();
        buf[threadIdx.x] += add;
        __syncthreads();
    }
    const uint32_t incl = buf[threadIdx.x];
    __syncthreads();
    return incl - v;
}

// One slice of kLocalIds ids per block: its top_k keys and its finite count.
__global__ __launch_bounds__(kT) void sample_local_kernel(SampleArgs a) {
    constexpr int R = kLocalIds / kT;  // keys per lane
    constexpr int W = kT / 64;
    __shared__ unsigned long long lists[W * kFastTopK];
    __shared__ uint32_t nred[W];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t base = blockIdx.x * kLocalIds + wave * (64 * R), k = a.top_k;
    uint32_t nf = 0;
    unsigned long long v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t id = base + r * 64 + lane;  // the wave's 256 ids, coalesced
        v[r] = 0ull;
        if (id < a.vocab) {
            const float s = adjusted(a.logits[id], a.counts ? a.counts[id] : 0u, a.repeat_penalty);
            if (isfinite(s)) {
                v[r] = (static_cast<unsigned long long>(order_key(s)) << 32) | (0xffffffffu - id);
                ++nf;
            }
        }
    }
    // The wave's top k, descending: k rounds of a wave max, the owner zeroing its copy.
    for (uint32_t i = 0; i < k; ++i) {
        unsigned long long mx = v[0];
#pragma unroll
        for (int r = 1; r < R; ++r) mx = v[r] > mx ? v[r] : mx;
        const unsigned long long b = wave_max_dpp(mx);
        if (lane == 0) lists[wave * k + i] = b;
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (v[r] == b) v[r] = 0ull;
    }
    for (int off = 32; off > 0; off >>= 1) nf += __shfl_xor(nf, off, 64);
    if (lane == 0) nred[wave] = nf;
    __syncthreads();
    if (wave == 0) {
        wave_merge(lists, W, k, k, a.cand_buf + static_cast<size_t>(blockIdx.x) * k);
        if (lane == 0) {
            uint32_t total = 0;
            for (int w = 0; w < W; ++w) total += nred[w];
            a.cand_nf[blockIdx.x] = total;
        }
    }
}

__device__ __noinline__ void sample_finish(const SampleArgs& a, uint32_t tok);

__global__ __launch_bounds__(kT) void sample_kernel(SampleArgs a) {
    __shared__ SampleShared sh;
    const uint32_t tid = threadIdx.x;
    const uint32_t V = a.vocab;
    const uint32_t chunk = (V + kT - 1) / kT;
    const uint32_t i0 = tid * chunk, i1 = min(V, i0 + chunk);
    auto score = [&](uint32_t i) { return adjusted(a.logits[i], a.counts ? a.counts[i] : 0u, a.repeat_penalty); };

    uint32_t tok = 0;
    if (a.temperature <= 0.0f) {
        // greedyWithPenalties: best starts at index 0; NaN never replaces it.
        unsigned long long best = 0ull;
        for (uint32_t i = i0; i < i1; ++i) {
            const unsigned long long k = argmax_key(score(i), i);
            best = k > best ? k : best;
        }
        best = wave_max_u64(best);
        if ((tid & 63) == 0) sh.red[tid >> 6] = best;
        __syncthreads();
        if (tid == 0) {
            for (int w = 0; w < kT / 64; ++w) best = sh.red[w] > best ? sh.red[w] : best;
            const float s0 = score(0);
            sh.token = (s0 != s0) ? 0u : argmax_key_index(best);
        }
        __syncthreads();
        tok = sh.token;
    } else {
        // Finite candidates and the limit (buildCandidates, :367-372).
        const bool two_stage = a.cand_buf != nullptr;
        const uint32_t slices = (V + kLocalIds - 1) / kLocalIds;
        uint32_t nf = 0;
        if (two_stage)
            for (uint32_t b = tid; b < slices; b += kT) nf += a.cand_nf[b];
        else
            for (uint32_t i = i0; i < i1; ++i) nf += isfinite(score(i)) ? 1u : 0u;
        const uint32_t n_finite = block_sum_u32(nf, sh.red);
        const uint32_t limit = min(a.top_k, V);
        const uint32_t count = min(limit, n_finite);
        if (count == 0) {
            // llm.argmax of the raw logits (:111).
            unsigned long long best = 0ull;
            for (uint32_t i = i0; i < i1; ++i) {
                const unsigned long long k = argmax_key(a.logits[i], i);
                best = k > best ? k : best;
            }
            best = wave_max_u64(best);
            if ((tid & 63) == 0) sh.red[tid >> 6] = best;
            __syncthreads();
            if (tid == 0) {
                for (int w = 0; w < kT / 64; ++w) best = sh.red[w] > best ? sh.red[w] : best;
                sh.token = (a.logits[0] != a.logits[0]) ? 0u : argmax_key_index(best);
            }
            __syncthreads();
            tok = sh.token;
        } else {
          if (two_stage) {
            // The slices' lists (each top_k keys, descending, zero padded): the
            // first wave merges them, lane s holding list s's head; the top
            // count heads taken are the candidates, in order.
            // Lists staged in LDS when they fit, else merged from the scratch.
            const uint32_t total = slices * a.top_k;
            const bool staged = total <= static_cast<uint32_t>(kSurvivors);
            if (staged)
                for (uint32_t j = tid; j < total; j += kT) sh.surv[j] = a.cand_buf[j];
            for (uint32_t j = tid; j < static_cast<uint32_t>(kMaxCand); j += kT) sh.cand[j] = 0ull;
            __syncthreads();
            if (tid < 64) wave_merge(staged ? sh.surv : a.cand_buf, slices, a.top_k, count, sh.cand);
            __syncthreads();
          } else {
            // Radix select: the key of the count-th largest finite score.
            if (tid == 0) {
                sh.prefix = 0;
                sh.remaining = count;
            }
            for (int pass = 0; pass < 4; ++pass) {
                const int shift = 24 - 8 * pass;
                for (uint32_t b = tid; b < 256; b += kT) sh.hist[b] = 0;
                __syncthreads();
                const uint32_t prefix = sh.prefix;
                for (uint32_t i = i0; i < i1; ++i) {
                    const float s = score(i);
                    if (!isfinite(s)) continue;
                    const uint32_t k = order_key(s);
                    if (pass > 0 && (k >> (shift + 8)) != prefix) continue;
                    atomicAdd(&sh.hist[(k >> shift) & 255u], 1u);
                }
                __syncthreads();
                if (tid == 0) {
                    uint32_t rem = sh.remaining, b = 255;
                    for (;; --b) {
                        if (sh.hist[b] >= rem || b == 0) break;
                        rem -= sh.hist[b];
                    }
                    sh.prefix = (prefix << 8) | b;
                    sh.remaining = rem;
                }
                __syncthreads();
            }
            const uint32_t thr = sh.prefix;        // key of the count-th largest
            const uint32_t need_eq = sh.remaining;  // how many keys equal to thr are taken
            // Gather: every key > thr, and the need_eq lowest-id keys == thr.
            uint32_t ngt = 0, neq = 0;
            for (uint32_t i = i0; i < i1; ++i) {
                const float s = score(i);
                if (!isfinite(s)) continue;
                const uint32_t k = order_key(s);
                ngt += k > thr ? 1u : 0u;
                neq += k == thr ? 1u : 0u;
            }
            const uint32_t off_gt = block_exclusive_scan(ngt, sh.scan_gt);
            const uint32_t off_eq = block_exclusive_scan(neq, sh.scan_eq);
            const uint32_t n_gt = count - need_eq;
            for (uint32_t j = tid; j < static_cast<uint32_t>(kMaxCand); j += kT) sh.cand[j] = 0ull;
            __syncthreads();
            uint32_t wg = off_gt, we = off_eq;
            for (uint32_t i = i0; i < i1; ++i) {
                const float s = score(i);
                if (!isfinite(s)) continue;
                const uint32_t k = order_key(s);
                const unsigned long long key = (static_cast<unsigned long long>(k) << 32) | (0xffffffffu - i);
                if (k > thr) sh.cand[wg++] = key;
                else if (k == thr && we < need_eq) sh.cand[n_gt + we++] = key;
                else if (k == thr) ++we;
            }
            __syncthreads();
            // Bitonic sort of kMaxCand keys, descending.
            bitonic_desc(sh.cand, kMaxCand);
          }
            // Probabilities (prepareProbabilities): exp in parallel, sums in order.
            const float temperature = fmaxf(a.temperature, 1e-6f);
            const float s0 = key_value(static_cast<uint32_t>(sh.cand[0] >> 32));
            for (uint32_t j = tid; j < count; j += kT) {
                const float sj = key_value(static_cast<uint32_t>(sh.cand[j] >> 32));
                const float p = expf(__fdiv_rn(__fsub_rn(sj, s0), temperature));
                sh.prob[j] = isfinite(p) ? p : 0.0f;
            }
            __syncthreads();
            if (tid == 0) {
                float total = 0.0f;
                for (uint32_t j = 0; j < count; ++j) total = __fadd_rn(total, sh.prob[j]);
                uint32_t k = count;
                if (total <= 0.0f || !isfinite(total)) {
                    k = 1;
                } else if (a.top_p < 1.0f) {
                    float cum = 0.0f;
                    for (uint32_t j = 0; j < count; ++j) {
                        cum = __fadd_rn(cum, sh.prob[j]);
                        if (__fdiv_rn(cum, total) >= a.top_p) {
                            k = j + 1;
                            break;
                        }
                    }
                }
                // sampleCandidate with one draw of Random.float(f32).
                uint64_t s[4] = {a.prng[0], a.prng[1], a.prng[2], a.prng[3]};
                const float u = prng_float(s);
                for (int q = 0; q < 4; ++q) a.prng[q] = s[q];
                float t2 = 0.0f;
                for (uint32_t j = 0; j < k; ++j) t2 = __fadd_rn(t2, sh.prob[j]);
                uint32_t pick = 0;
                if (t2 > 0.0f && isfinite(t2)) {
                    const float target = __fmul_rn(fminf(u, 0.99999994f), t2);
                    float cum = 0.0f;
                    pick = k - 1;
                    for (uint32_t j = 0; j < k; ++j) {
                        cum = __fadd_rn(cum, sh.prob[j]);
                        if (target <= cum) {
                            pick = j;
                            break;
                        }
                    }
                }
                sh.token = 0xffffffffu - static_cast<uint32_t>(sh.cand[pick] & 0xffffffffull);
            }
            __syncthreads();
            tok = sh.token;
        }
    }
    if (tid != 0) return;
    sample_finish(a, tok);
}

// Whole-vocabulary path, pass 1: sort keys and ids (the ids in ascending
// order, so the stable sort keeps ties by ascending id).
__global__ __launch_bounds__(256) void sample_full_keys_kernel(SampleArgs a, uint32_t* keys, uint32_t* ids) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.vocab) return;
    const float s = adjusted(a.logits[i], a.counts ? a.counts[i] : 0u, a.repeat_penalty);
    keys[i] = isfinite(s) ? order_key(s) : 0u;
    ids[i] = i;
}

// Whole-vocabulary path, pass 3 (one block): the candidates are the first
// min(limit, finite) sorted pairs (finite keys are >= 1, so the finite ones
// come first).
__global__ __launch_bounds__(kT) void sample_full_kernel(SampleArgs a, const uint32_t* keys, const uint32_t* ids,
                                                         float* prob, float* prefix) {
    __shared__ unsigned long long red[kT / 64];
    __shared__ uint32_t s_n, s_cut, s_pick, s_tok;
    const uint32_t tid = threadIdx.x, V = a.vocab;
    // Finite count: the first zero key (binary search; keys are descending).
    if (tid == 0) {
        uint32_t lo = 0, hi = V;
        while (lo < hi) {
            const uint32_t mid = (lo + hi) / 2;
            if (keys[mid] != 0u) lo = mid + 1;
            else hi = mid;
        }
        s_n = lo;
    }
    __syncthreads();
    const uint32_t limit = min(a.top_k == 0 ? V : a.top_k, V);
    const uint32_t count = min(limit, s_n);
    uint32_t tok;
    if (count == 0) {
        // llm.argmax of the raw logits (:111).
        unsigned long long best = 0ull;
        for (uint32_t i = tid; i < V; i += kT) {
            const unsigned long long k = argmax_key(a.logits[i], i);
            best = k > best ? k : best;
        }
        best = wave_max_u64(best);
        if ((tid & 63) == 0) red[tid >> 6] = best;
        __syncthreads();
        if (tid == 0) {
            for (int w = 0; w < kT / 64; ++w) best = red[w] > best ? red[w] : best;
            s_tok = (a.logits[0] != a.logits[0]) ? 0u : argmax_key_index(best);
        }
        __syncthreads();
        tok = s_tok;
    } else {
        const float temperature = fmaxf(a.temperature, 1e-6f);
        const float s0 = key_value(keys[0]);
        for (uint32_t j = tid; j < count; j += kT) {
            const float p = expf(__fdiv_rn(__fsub_rn(key_value(keys[j]), s0), temperature));
            prob[j] = isfinite(p) ? p : 0.0f;
        }
        __syncthreads();
        if (tid == 0) {  // sequential sums in candidate order, 16 loads ahead of the adds
            float c = 0.0f;
            uint32_t j = 0;
            for (; j + 16 <= count; j += 16) {
                float v[16];
#pragma unroll
                for (int q = 0; q < 16; ++q) v[q] = prob[j + q];
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    c = __fadd_rn(c, v[q]);
                    prefix[j + q] = c;
                }
            }
            for (; j < count; ++j) {
                c = __fadd_rn(c, prob[j]);
                prefix[j] = c;
            }
            s_cut = count;
            s_pick = 0xffffffffu;
        }
        __syncthreads();
        const float total = prefix[count - 1];
        // prepareProbabilities' top-p cut: the first j with prefix[j] / total >= top_p.
        const bool bad_total = total <= 0.0f || !isfinite(total);
        if (!bad_total && a.top_p < 1.0f) {
            uint32_t first = count;
            for (uint32_t j = tid; j < count; j += kT)
                if (__fdiv_rn(prefix[j], total) >= a.top_p) {
                    first = j;
                    break;
                }
            atomicMin(&s_cut, first == count ? count : first + 1);
        }
        __syncthreads();
        const uint32_t k = bad_total ? 1u : s_cut;
        // sampleCandidate with one draw of Random.float(f32).
        __shared__ float s_target;
        __shared__ uint32_t s_ok;
        if (tid == 0) {
            uint64_t st4[4] = {a.prng[0], a.prng[1], a.prng[2], a.prng[3]};
            const float u = prng_float(st4);
            for (int q = 0; q < 4; ++q) a.prng[q] = st4[q];
            const float t2 = prefix[k - 1];
            s_ok = t2 > 0.0f && isfinite(t2);
            s_target = __fmul_rn(fminf(u, 0.99999994f), t2);
        }
        __syncthreads();
        if (s_ok) {
            const float target = s_target;
            uint32_t first = 0xffffffffu;
            for (uint32_t j = tid; j < k; j += kT)
                if (target <= prefix[j]) {
                    first = j;
                    break;
                }
            atomicMin(&s_pick, first);
        }
        __syncthreads();
        const uint32_t pick = !s_ok ? 0u : (s_pick == 0xffffffffu ? k - 1 : s_pick);
        tok = ids[pick];
    }
    if (tid != 0) return;
    sample_finish(a, tok);
}

// Advance the step state as the greedy finish does, then the repeat window
// (the sampling block's thread 0, with the sampled token).
__device__ __noinline__ void sample_finish(const SampleArgs& a, uint32_t tok) {
    if (a.result) *a.result = tok;
    StepState* st = a.state;
    if (!st) return;
    const uint32_t next_pos = st->pos + (a.advance_pos ? 1u : 0u);
    st->argmax = tok;
    st->pos = next_pos;
    st->token = tok;
    const uint32_t produced = st->n_out;
    if (produced < a.out_cap) a.out_tokens[produced] = tok;
    st->n_out = produced + 1;
    if (a.counts && a.repeat_penalty > 1.0f && a.repeat_last_n > 0) {
        a.counts[tok] += 1;
        const uint32_t total = a.n_prompt + produced + 1;  // history length after this token
        if (total > a.repeat_last_n) {
            const uint32_t h = total - 1 - a.repeat_last_n;  // leaves the window
            const uint32_t old = h < a.n_prompt ? a.prompt[h] : a.out_tokens[h - a.n_prompt];
            a.counts[old] -= 1;
        }
    }
}

// counts = occurrences of each token in the last repeat_last_n prompt tokens.
__global__ __launch_bounds__(kT) void sample_counts_kernel(uint32_t* counts, uint32_t V, const uint32_t* prompt,
                                                          uint32_t n_prompt, uint32_t last_n) {
    for (uint32_t i = threadIdx.x; i < V; i += kT) counts[i] = 0;
    __syncthreads();
    const uint32_t start = n_prompt > last_n ? n_prompt - last_n : 0;
    for (uint32_t i = start + threadIdx.x; i < n_prompt; i += kT) atomicAdd(&counts[prompt[i]], 1u);
}

}  // namespace

size_t sample_cand_elems(uint32_t vocab) {
    const size_t slices = (vocab + kLocalIds - 1) / kLocalIds;
    return (slices <= 64 ? slices : 1) * kFastTopK;
}
size_t sample_nf_elems(uint32_t vocab) { return (vocab + kLocalIds - 1) / kLocalIds; }

// Whole-vocabulary scratch: [keys in | keys out | ids in | ids out | prob |
// prefix] of vocab words each (256-byte aligned), then the sort's storage.
namespace {
size_t full_word_bytes(uint32_t vocab) { return ((size_t)vocab * 4 + 255) / 256 * 256; }
size_t full_sort_bytes(uint32_t vocab) {
    size_t bytes = 0;
    const hipError_t e = rocprim::radix_sort_pairs_desc(nullptr, bytes, static_cast<const uint32_t*>(nullptr),
                                                        static_cast<uint32_t*>(nullptr),
                                                        static_cast<const uint32_t*>(nullptr),
                                                        static_cast<uint32_t*>(nullptr), vocab, 0, 32);
    return e == hipSuccess ? bytes : 0;
}
}  // namespace

size_t sample_full_bytes(uint32_t vocab) {
    const size_t sort = full_sort_bytes(vocab);
    return sort ? 6 * full_word_bytes(vocab) + sort : 0;
}

hipError_t launch_sample(const SampleArgs& a, hipStream_t s) {
    if (a.temperature > 0.0f && (a.top_k == 0 ? a.vocab : a.top_k) > static_cast<uint32_t>(kMaxCand)) {
        if (!a.full) return hipErrorInvalidValue;
        const size_t wb = full_word_bytes(a.vocab);
        char* base = static_cast<char*>(a.full);
        uint32_t* k_in = reinterpret_cast<uint32_t*>(base);
        uint32_t* k_out = reinterpret_cast<uint32_t*>(base + wb);
        uint32_t* i_in = reinterpret_cast<uint32_t*>(base + 2 * wb);
        uint32_t* i_out = reinterpret_cast<uint32_t*>(base + 3 * wb);
        float* prob = reinterpret_cast<float*>(base + 4 * wb);
        float* prefix = reinterpret_cast<float*>(base + 5 * wb);
        size_t sort_bytes = full_sort_bytes(a.vocab);
        hipError_t e = vlaunch(sample_full_keys_kernel, dim3((a.vocab + 255) / 256), dim3(256), 0, s, a, k_in, i_in);
        if (e == hipSuccess)
            e = rocprim::radix_sort_pairs_desc(static_cast<void*>(base + 6 * wb), sort_bytes,
                                               static_cast<const uint32_t*>(k_in), k_out,
                                               static_cast<const uint32_t*>(i_in), i_out, a.vocab, 0, 32, s);
        if (e == hipSuccess) e = vlaunch(sample_full_kernel, dim3(1), dim3(kT), 0, s, a, k_out, i_out, prob, prefix);
        return e;
    }
    SampleArgs b = a;
    const uint32_t slices = (a.vocab + kLocalIds - 1) / kLocalIds;
    const bool two_stage = a.cand_buf && a.cand_nf && a.temperature > 0.0f && a.top_k <= kFastTopK &&
                           slices <= 64u;
    if (!two_stage) {
        b.cand_buf = nullptr;
        b.cand_nf = nullptr;
        return vlaunch(sample_kernel, dim3(1), dim3(kT), 0, s, b);
    }
    hipError_t e = vlaunch(sample_local_kernel, dim3(slices), dim3(kT), 0, s, b);
    return e != hipSuccess ? e : vlaunch(sample_kernel, dim3(1), dim3(kT), 0, s, b);
}

hipError_t launch_sample_counts(uint32_t* counts, uint32_t vocab, const uint32_t* prompt, uint32_t n_prompt,
                                uint32_t last_n, hipStream_t s) {
    return vlaunch(sample_counts_kernel, dim3(1), dim3(kT), 0, s, counts, vocab, prompt, n_prompt, last_n);
}

}  // namespace vvli
