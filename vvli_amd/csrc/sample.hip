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
//            p_i = exp((s_i - s_0) / T) in parallel, then the running sums
//            in candidate order (up to 128 candidates formed once by the
//            first wave, with the cut and the pick as ballots over them;
//            more by one thread), the top_p cut (:428-449), one draw of
//            u = Random.float(f32) from Zig's DefaultPrng (xoshiro256++,
//            state in device memory) and the walk of the cumulative sum
//            (sampleCandidate, :451-463).
// Sequential f32 sums in candidate order keep the reference's rounding.
//
// Whole-vocabulary candidates (limit over 1024: top_k 0, which buildCandidates
// treats as "every finite score, sorted", :376-391, or top_k > 1024):
// full_keys_kernel writes each id's sort key (descending score order, the
// non-finite ones last), four stable 8-bit radix passes (histogram + ballot-
// ranked scatter kernels) order the (key, id) pairs -- ties keep ascending
// ids, the order insertTopCandidate gives and the oracle uses for the
// reference's unstable sort -- and sample_full_kernel takes the first
// min(limit, finite) of them: the probabilities, then the sequential f32
// prefix sums in candidate order (the running sum of prepareProbabilities'
// total, of its top-p scan and of sampleCandidate's sums are the same
// sequence), computed bit-exactly as integer prefix sums per binade of the
// running sum, then the top-p cut and the pick as searches over those sums
// (both predicates are monotone along the nondecreasing sums).
//
// Two-stage top-k (top_k <= 128, at most 64 slices, scratch of
// sample_cand_elems keys given):
// sample_local_kernel cuts the vocab into slices of 4096 ids, one block each,
// and writes a slice's top_k keys (score key << 32 | ~id; 0 for a non-finite
// score), descending, with its finite count: each wave sorts its 256 ids'
// keys in registers (a bitonic network, lanes exchanged by DPP and shuffles)
// and the block tree-merges the 16 waves' first 128. The keys are distinct,
// so every member of the global top_k is in its slice's top_k; the sampling
// block then tree-merges the slices' lists (up to 32; more: its first wave
// merges them, one list head per lane) instead of scanning the vocab (one
// block's scan is ~1 ms at a 128K vocab), and its first wave forms the
// candidates' running sums, from which the top-p cut and the pick follow.
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

// ---- Wave-level bitonic networks over 64-bit keys held in registers ----
// Element e = lane * R + r of a wave's 64 R keys lives in v[r] of lane
// `lane`; a compare-exchange at distance d < R stays in the lane's
// registers, d >= R pairs lane with lane ^ (d / R): DPP moves within a row
// of 16 lanes (xor 1, 2 as quad permutes; xor 4, 8 as a row shift each way
// and a select), shuffles through the LDS crossbar for xor 16 and 32 (the
// crossbar's throughput, shared by the block's 16 waves, bounds the shuffle
// form: 25 us for the slice top-k with shuffles at every distance).
template <int LX>
__device__ inline uint32_t xor_lane32(uint32_t x, uint32_t lane) {
    const int xi = static_cast<int>(x);
    if constexpr (LX == 1) {
        return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(xi, 0xB1, 0xf, 0xf, true));  // quad_perm [1,0,3,2]
    } else if constexpr (LX == 2) {
        return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(xi, 0x4E, 0xf, 0xf, true));  // quad_perm [2,3,0,1]
    } else if constexpr (LX == 4 || LX == 8) {
        const int up = __builtin_amdgcn_mov_dpp(xi, 0x100 + LX, 0xf, 0xf, true);  // row_shl: lane + LX
        const int dn = __builtin_amdgcn_mov_dpp(xi, 0x110 + LX, 0xf, 0xf, true);  // row_shr: lane - LX
        return static_cast<uint32_t>((lane & LX) ? dn : up);
    } else {
        return static_cast<uint32_t>(__shfl_xor(xi, LX, 64));
    }
}
template <int LX>
__device__ inline unsigned long long xor_lane64(unsigned long long x, uint32_t lane) {
    const uint32_t lo = xor_lane32<LX>(static_cast<uint32_t>(x), lane);
    const uint32_t hi = xor_lane32<LX>(static_cast<uint32_t>(x >> 32), lane);
    return (static_cast<unsigned long long>(hi) << 32) | lo;
}
__device__ inline unsigned long long shfl_xor64(unsigned long long x, uint32_t lx, uint32_t lane) {
    switch (lx) {
        case 1: return xor_lane64<1>(x, lane);
        case 2: return xor_lane64<2>(x, lane);
        case 4: return xor_lane64<4>(x, lane);
        case 8: return xor_lane64<8>(x, lane);
        case 16: return xor_lane64<16>(x, lane);
        default: return xor_lane64<32>(x, lane);
    }
}
// One stage at distance d of a bitonic network; `size` picks each element's
// direction (descending where (e & size) == 0); size = 0: all descending.
template <int R>
__device__ inline void wave_cx(unsigned long long (&v)[R], uint32_t lane, uint32_t size, uint32_t d) {
    if (d < static_cast<uint32_t>(R)) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int q = r ^ static_cast<int>(d);
            if (q > r) {
                const bool desc = ((lane * R + r) & size) == 0;
                const unsigned long long a = v[r], b = v[q];
                const bool sw = desc ? a < b : a > b;
                v[r] = sw ? b : a;
                v[q] = sw ? a : b;
            }
        }
    } else {
        const uint32_t lx = d / R;
        const bool lower = (lane & lx) == 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const unsigned long long o = shfl_xor64(v[r], lx, lane);
            const bool desc = ((lane * R + r) & size) == 0;
            v[r] = (lower == desc) ? (v[r] > o ? v[r] : o) : (v[r] < o ? v[r] : o);
        }
    }
}
// The wave's 64 R keys sorted descending (element order e = lane * R + r).
// (Unrolled, so every stage's distance is a constant and its DPP form fixed.)
template <int R>
__device__ inline void wave_sort_desc(unsigned long long (&v)[R], uint32_t lane) {
#pragma unroll
    for (uint32_t size = 2; size <= 64u * R; size <<= 1)
#pragma unroll
        for (uint32_t d = size >> 1; d > 0; d >>= 1) wave_cx<R>(v, lane, size, d);
}
// A bitonic sequence of 64 R keys (descending, then ascending) sorted descending.
template <int R>
__device__ inline void wave_merge_desc(unsigned long long (&v)[R], uint32_t lane) {
#pragma unroll
    for (uint32_t d = 32u * R; d > 0; d >>= 1) wave_cx<R>(v, lane, 0u, d);
}
// Tree merge of n (a power of two, <= 2 * waves of the block) descending
// lists of kFastTopK keys, buf[0][i] (i < n), keeping the first kFastTopK:
// at each level wave w merges lists 2w and 2w + 1 (list 2w, then 2w + 1
// reversed: a bitonic sequence of 2 kFastTopK keys) into buf[other][w].
// Every thread of the block calls it; returns the buffer holding the result
// in its list 0.
__device__ inline int block_tree_merge(unsigned long long (*buf)[32][kFastTopK], uint32_t n) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int cur = 0;
    for (uint32_t nl = n; nl > 1; nl >>= 1) {
        if (wave < nl / 2) {
            const unsigned long long* A = buf[cur][2 * wave];
            const unsigned long long* B = buf[cur][2 * wave + 1];
            unsigned long long v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t e = lane * 4 + r;
                v[r] = e < static_cast<uint32_t>(kFastTopK) ? A[e] : B[2 * kFastTopK - 1 - e];
            }
            wave_merge_desc<4>(v, lane);
            if (lane < static_cast<uint32_t>(kFastTopK) / 4)
#pragma unroll
                for (int r = 0; r < 4; ++r) buf[cur ^ 1][wave][lane * 4 + r] = v[r];
        }
        __syncthreads();
        cur ^= 1;
    }
    return cur;
}
static_assert(kFastTopK == 128, "the tree merge holds 2 x 128 keys as 4 per lane");

struct SampleShared {
    uint32_t hist[256];
    unsigned long long cand[kMaxCand];  // (score key << 32) | ~id, sorted descending
    float prob[kMaxCand];
    uint32_t scan_gt[kT], scan_eq[kT];
    unsigned long long red[kT / 64];
    union {
        unsigned long long surv[kSurvivors];          // two-stage path: the slices' lists (more than 32)
        unsigned long long tree[2][32][kFastTopK];    // ... up to 32 lists: the tree merge's buffers
    } u;
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
// Each wave sorts its 256 keys (a register bitonic network) and the block
// tree-merges the 16 waves' first 128; the first top_k are the slice's list.
// (k rounds of a wave max per wave and a one-wave merge of the wave lists,
// the earlier form, took 5 + 0.53 k us: 26 us at top_k 40.)
__global__ __launch_bounds__(kT) void sample_local_kernel(SampleArgs a) {
    constexpr int R = kLocalIds / kT;  // keys per lane
    constexpr int W = kT / 64;
    static_assert(R == 4 && W == 16, "256 keys per wave, 16 waves");
    __shared__ unsigned long long lists[2][32][kFastTopK];
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
    wave_sort_desc<R>(v, lane);  // keys are distinct (ids in the low half); zeros last
    if (lane < static_cast<uint32_t>(kFastTopK) / R)
#pragma unroll
        for (int r = 0; r < R; ++r) lists[0][wave][lane * R + r] = v[r];
    for (int off = 32; off > 0; off >>= 1) nf += __shfl_xor(nf, off, 64);
    if (lane == 0) nred[wave] = nf;
    __syncthreads();
    const int cur = block_tree_merge(lists, W);
    unsigned long long* out = a.cand_buf + static_cast<size_t>(blockIdx.x) * k;
    for (uint32_t i = tid; i < k; i += kT) out[i] = lists[cur][0][i];
    if (tid == 0) {
        uint32_t total = 0;
        for (int w = 0; w < W; ++w) total += nred[w];
        a.cand_nf[blockIdx.x] = total;
    }
}

__device__ __forceinline__ void sample_finish(const SampleArgs& a, uint32_t tok);

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
            // The slices' lists (each top_k keys, descending, zero padded).
            // Up to 32 lists: a tree merge of the lists padded to 128 keys
            // (and to a power of two of lists with zero lists); more: the
            // first wave merges them, lane s holding list s's head, staged
            // in LDS when they fit, else from the scratch. The top count keys
            // are the candidates, in order.
            for (uint32_t j = tid; j < static_cast<uint32_t>(kMaxCand); j += kT) sh.cand[j] = 0ull;
            if (slices <= 32) {
                uint32_t n = 1;
                while (n < slices) n <<= 1;
                for (uint32_t j = tid; j < n * kFastTopK; j += kT) {
                    const uint32_t sl = j / kFastTopK, i = j % kFastTopK;
                    sh.u.tree[0][sl][i] = (sl < slices && i < a.top_k) ? a.cand_buf[sl * a.top_k + i] : 0ull;
                }
                __syncthreads();
                const int cur = block_tree_merge(sh.u.tree, n);
                for (uint32_t j = tid; j < count; j += kT) sh.cand[j] = sh.u.tree[cur][0][j];
            } else {
                const uint32_t total = slices * a.top_k;
                const bool staged = total <= static_cast<uint32_t>(kSurvivors);
                if (staged)
                    for (uint32_t j = tid; j < total; j += kT) sh.u.surv[j] = a.cand_buf[j];
                __syncthreads();
                if (tid < 64) wave_merge(staged ? sh.u.surv : a.cand_buf, slices, a.top_k, count, sh.cand);
            }
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
            if (count <= 128) {
                // prepareProbabilities' total, its top-p scan and sampleCandidate's
                // sums are one sequence of running sums P_j = P_{j-1} + p_j in
                // candidate order: the first wave forms it (lane l holds P_l and
                // P_{l+64}), then the cut and the pick are ballots over it.
                if (tid < 64) {
                    const uint32_t lane = tid;
                    const float q0 = lane < count ? sh.prob[lane] : 0.0f;
                    const float q1 = lane + 64 < count ? sh.prob[lane + 64] : 0.0f;
                    float run = 0.0f, P0 = 0.0f, P1 = 0.0f;
                    for (uint32_t j = 0; j < count; ++j) {
                        const float pj = __int_as_float(
                            __builtin_amdgcn_readlane(__float_as_int(j < 64 ? q0 : q1), static_cast<int>(j & 63)));
                        run = __fadd_rn(run, pj);
                        if (lane == (j & 63)) {
                            if (j < 64) P0 = run;
                            else P1 = run;
                        }
                    }
                    const float total = run;
                    uint32_t k = count;
                    if (total <= 0.0f || !isfinite(total)) {
                        k = 1;
                    } else if (a.top_p < 1.0f) {
                        const unsigned long long c0 = __ballot(lane < count && __fdiv_rn(P0, total) >= a.top_p);
                        const unsigned long long c1 = __ballot(lane + 64 < count && __fdiv_rn(P1, total) >= a.top_p);
                        if (c0) k = __ffsll(static_cast<long long>(c0));
                        else if (c1) k = 64 + __ffsll(static_cast<long long>(c1));
                    }
                    // sampleCandidate with one draw of Random.float(f32) (every lane
                    // draws the same value from the same state; lane 0 stores it).
                    uint64_t st[4] = {a.prng[0], a.prng[1], a.prng[2], a.prng[3]};
                    const float u = prng_float(st);
                    __builtin_amdgcn_wave_barrier();
                    if (lane == 0)
                        for (int q = 0; q < 4; ++q) a.prng[q] = st[q];
                    const uint32_t kl = k - 1;
                    const float t2 = __int_as_float(
                        __builtin_amdgcn_readlane(__float_as_int(kl < 64 ? P0 : P1), static_cast<int>(kl & 63)));
                    uint32_t pick = 0;
                    if (t2 > 0.0f && isfinite(t2)) {
                        const float target = __fmul_rn(fminf(u, 0.99999994f), t2);
                        const unsigned long long c0 = __ballot(lane < k && target <= P0);
                        const unsigned long long c1 = __ballot(lane + 64 < k && target <= P1);
                        pick = c0 ? __ffsll(static_cast<long long>(c0)) - 1
                                  : (c1 ? 64 + __ffsll(static_cast<long long>(c1)) - 1 : k - 1);
                    }
                    if (lane == 0) sh.token = 0xffffffffu - static_cast<uint32_t>(sh.cand[pick] & 0xffffffffull);
                }
            } else if (tid == 0) {
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

// ---- Whole-vocabulary candidates ---------------------------------------------
// Sort: LSD radix sort of (sort key, id) pairs, four passes of 8 bits over
// tiles of kSortTile ids. The sort key is ~order_key(score) (0xffffffff for a
// non-finite score), so ascending sort keys are descending scores with the
// non-finite ones last, and the stable passes keep ties in ascending id order
// (the ids start in ascending order), the order insertTopCandidate gives.
// A pass is a histogram kernel (per tile and digit) and a scatter kernel; the
// scatter ranks a tile's keys stably with wave ballots (lanes holding the
// same digit) and per-(slot, wave) digit counts in LDS, so no atomics decide
// an order.
constexpr uint32_t kSortThreads = 256;
constexpr uint32_t kSortSlots = 8;
constexpr uint32_t kSortTile = kSortThreads * kSortSlots;          // ids per tile
constexpr uint32_t kSortRows = kSortSlots * (kSortThreads / 64);   // (slot, wave) rows of a tile

__device__ inline uint32_t sort_key(float s) { return isfinite(s) ? ~order_key(s) : 0xffffffffu; }

// Pass-0 input: each id's sort key, the ids, and the tiles' low-byte histograms.
__global__ __launch_bounds__(kSortThreads) void full_keys_kernel(SampleArgs a, uint32_t* sk, uint32_t* ids,
                                                                 uint32_t* hist) {
    __shared__ uint32_t h[256];
    h[threadIdx.x] = 0;
    __syncthreads();
    const uint32_t base = blockIdx.x * kSortTile;
    for (uint32_t s = 0; s < kSortSlots; ++s) {
        const uint32_t i = base + s * kSortThreads + threadIdx.x;
        if (i < a.vocab) {
            const uint32_t k = sort_key(adjusted(a.logits[i], a.counts ? a.counts[i] : 0u, a.repeat_penalty));
            sk[i] = k;
            ids[i] = i;
            atomicAdd(&h[k & 255u], 1u);
        }
    }
    __syncthreads();
    hist[blockIdx.x * 256 + threadIdx.x] = h[threadIdx.x];
}

// Digit histogram of every tile for the pass at `shift`.
__global__ __launch_bounds__(kSortThreads) void full_hist_kernel(const uint32_t* sk, uint32_t n, uint32_t shift,
                                                                 uint32_t* hist) {
    __shared__ uint32_t h[256];
    h[threadIdx.x] = 0;
    __syncthreads();
    const uint32_t base = blockIdx.x * kSortTile;
    for (uint32_t s = 0; s < kSortSlots; ++s) {
        const uint32_t i = base + s * kSortThreads + threadIdx.x;
        if (i < n) atomicAdd(&h[(sk[i] >> shift) & 255u], 1u);
    }
    __syncthreads();
    hist[blockIdx.x * 256 + threadIdx.x] = h[threadIdx.x];
}

__device__ inline uint32_t wave_incl_scan_add(uint32_t v) {
    const uint32_t lane = threadIdx.x & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = static_cast<uint32_t>(__shfl_up(static_cast<int>(v), off, 64));
        if (lane >= static_cast<uint32_t>(off)) v += o;
    }
    return v;
}

// One stable pass at `shift`: tile t (input positions t * kSortTile + s * 256
// + thread, slot s) goes to base(digit) + (earlier tiles' count of the digit)
// + (its rank among the tile's keys of that digit in position order).
__global__ __launch_bounds__(kSortThreads) void full_scatter_kernel(const uint32_t* sk_in, const uint32_t* id_in,
                                                                    uint32_t* sk_out, uint32_t* id_out, uint32_t n,
                                                                    uint32_t shift, const uint32_t* hist,
                                                                    uint32_t tiles) {
    __shared__ uint32_t cnt[kSortRows][256];
    __shared__ uint32_t base[256];
    __shared__ uint32_t wsum[kSortThreads / 64];
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6, t = blockIdx.x;
    // Thread d: digit d's total and its count in tiles before t.
    uint32_t tot = 0, before = 0;
#pragma unroll 8
    for (uint32_t u = 0; u < tiles; ++u) {
        const uint32_t c = hist[u * 256 + tid];
        tot += c;
        before += u < t ? c : 0u;
    }
    const uint32_t incl = wave_incl_scan_add(tot);
    if (lane == 63) wsum[w] = incl;
#pragma unroll
    for (uint32_t r = 0; r < kSortRows; ++r) cnt[r][tid] = 0;
    __syncthreads();
    uint32_t excl = incl - tot;
    for (uint32_t u = 0; u < w; ++u) excl += wsum[u];
    base[tid] = excl + before;

    uint32_t key[kSortSlots], id[kSortSlots], rank[kSortSlots];
    const uint32_t t0 = t * kSortTile + tid;
#pragma unroll
    for (uint32_t s = 0; s < kSortSlots; ++s) {
        const uint32_t i = t0 + s * kSortThreads;
        key[s] = i < n ? sk_in[i] : 0u;
        id[s] = i < n ? id_in[i] : 0u;
    }
    const unsigned long long lt = (1ull << lane) - 1ull;
#pragma unroll
    for (uint32_t s = 0; s < kSortSlots; ++s) {
        const bool valid = t0 + s * kSortThreads < n;
        const uint32_t dg = (key[s] >> shift) & 255u;
        unsigned long long same = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const bool bit = (dg >> b) & 1u;
            const unsigned long long on = __ballot(bit);
            same &= bit ? on : ~on;
        }
        rank[s] = static_cast<uint32_t>(__popcll(same & lt));
        if (valid && rank[s] == 0) cnt[s * (kSortThreads / 64) + w][dg] = static_cast<uint32_t>(__popcll(same));
    }
    __syncthreads();
    // Thread d: exclusive prefix of digit d's counts over the rows in order.
    uint32_t run = 0;
#pragma unroll
    for (uint32_t r = 0; r < kSortRows; ++r) {
        const uint32_t c = cnt[r][tid];
        cnt[r][tid] = run;
        run += c;
    }
    __syncthreads();
#pragma unroll
    for (uint32_t s = 0; s < kSortSlots; ++s) {
        if (t0 + s * kSortThreads >= n) continue;
        const uint32_t dg = (key[s] >> shift) & 255u;
        const uint32_t pos = base[dg] + cnt[s * (kSortThreads / 64) + w][dg] + rank[s];
        sk_out[pos] = key[s];
        id_out[pos] = id[s];
    }
}

// p = exp((s - s_0) / T) of every sorted position (prepareProbabilities'
// exp, src/generator.zig:436-439), 0 where it is not finite or the score is;
// s_0 = the first sorted score.
__global__ __launch_bounds__(kSortThreads) void full_probs_kernel(const uint32_t* sk, uint32_t n, float temperature,
                                                                  float* prob) {
    const float s0 = key_value(~sk[0]);
    const float t = fmaxf(temperature, 1e-6f);
    const uint32_t base = blockIdx.x * kSortTile;
    for (uint32_t q = 0; q < kSortSlots; ++q) {
        const uint32_t j = base + q * kSortThreads + threadIdx.x;
        if (j >= n) break;
        const uint32_t k = sk[j];
        float v = 0.0f;
        if (k != 0xffffffffu) {
            v = expf(__fdiv_rn(__fsub_rn(key_value(~k), s0), t));
            v = isfinite(v) ? v : 0.0f;
        }
        prob[j] = v;
    }
}

// ---- exact sequential f32 prefix sums, computed in parallel --------------------
// prepareProbabilities and sampleCandidate (src/generator.zig:428-463) add the
// candidates' probabilities one after another in f32: c_j = fl(c_{j-1} + p_j).
// While the running sum stays in one binade [2^e, 2^(e+1)), every f32 there
// is a multiple of u = 2^(e-23), so with c = m * u (2^23 <= m < 2^24) and
// x = p / u (exact: a power-of-two scaling),
//   fl(c + p) = u * (m + round(x))   as long as m + x < 2^24,
// round-to-nearest with ties to the even result. Off ties, round(x) does not
// depend on m, and the chain is an integer prefix sum over the candidates. At
// a tie (x = f + 1/2) the result is the even one of m + f and m + f + 1:
// taking f tentatively (T_j = m + the tentative sums up to j) and correcting
// by +1 where m_{j-1} + f is odd, the correction at the k-th tie is
// parity(T at tie k) xor parity(T at tie k-1) (parity 0 before the first),
// because after every tie the corrected sum is even; so m_j = T_j + the number
// of parity changes along the ties up to j, also a prefix computation. The
// first candidate whose exact sum leaves the binade (m_{j-1} + floor(x_j) >=
// 2^24) is added as an ordinary f32 add (every thread computes it from the
// operands the block's min passes around), and the chunk resumes after it in
// the new binade (at most one restart per binade the sum enters, i.e. about
// log2(vocab) in all). Every stored prefix value is bit-identical to the
// one-after-another sum.
// One block, candidates in chunks of kChainChunk held in registers (thread t:
// kChainE consecutive ones); an iteration covers a window of the chunk from
// the next candidate on (waves holding none of it skip the arithmetic), with
// two barriers: after the (sum, ties) scan and after the min over the waves'
// first crossings.
constexpr int kChainE = 8;                       // candidates per thread and chunk (two float4 loads)
constexpr uint32_t kChainChunk = kT * kChainE;   // candidates per chunk
constexpr uint32_t kChainW0 = 1024;              // first window after a restart (grows x2 per full window)
constexpr uint32_t kSatCap = 1u << 30;           // saturation of the integer sums (> 2^24)
constexpr uint32_t kTieHas = 1u << 29;           // tie summary: count (bits 0-28), has, first, last parity

__device__ inline uint32_t sat_add(uint32_t a, uint32_t b) { return min(a + b, kSatCap); }  // a, b <= kSatCap

// Summary of a run of ties' parities: (has, first, last, changes inside);
// `a` precedes `b`; 0 is the identity.
__device__ inline uint32_t tie_comb(uint32_t a, uint32_t b) {
    if (!(a & kTieHas)) return b;
    if (!(b & kTieHas)) return a;
    const uint32_t cnt = (a & (kTieHas - 1)) + (b & (kTieHas - 1)) + ((a >> 31) != ((b >> 30) & 1u) ? 1u : 0u);
    return cnt | kTieHas | (a & (1u << 30)) | (b & (1u << 31));
}
__device__ inline uint32_t tie_leaf(uint32_t parity) { return kTieHas | (parity << 30) | (parity << 31); }

__device__ inline uint32_t tie_flip(uint32_t y, uint32_t par) {
    return (par && (y & kTieHas)) ? y ^ (3u << 30) : y;
}

// Saturating-sum scans and a min with DPP (no LDS round trips): row_shr:k
// shifts within 16-lane rows (lanes without a source read 0), row_bcast:15 /
// :31 add the last lane of the previous row(s) into rows 1, 3 / 2, 3,
// wave_shr:1 shifts the whole wave by one lane.
template <int kCtrl, int kRowMask>
__device__ inline uint32_t dpp_u32(uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), kCtrl, kRowMask, 0xf, false));
}
__device__ inline uint32_t row_scan_sat(uint32_t x) {  // inclusive, within each 16-lane row
    x = sat_add(x, dpp_u32<0x111, 0xf>(x));
    x = sat_add(x, dpp_u32<0x112, 0xf>(x));
    x = sat_add(x, dpp_u32<0x114, 0xf>(x));
    return sat_add(x, dpp_u32<0x118, 0xf>(x));
}
__device__ inline uint32_t wave_scan_sat(uint32_t x) {  // inclusive, over the wave
    x = row_scan_sat(x);
    x = sat_add(x, dpp_u32<0x142, 0xa>(x));
    return sat_add(x, dpp_u32<0x143, 0xc>(x));
}
__device__ inline uint32_t wave_shr1(uint32_t x) { return dpp_u32<0x138, 0xf>(x); }  // lane 0 reads 0
__device__ inline uint32_t row_min_u32(uint32_t x) {  // every lane: its row's min
    x = min(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0xB1, 0xf, 0xf, true)));
    x = min(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x4E, 0xf, 0xf, true)));
    x = min(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x141, 0xf, 0xf, true)));
    return min(x, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x140, 0xf, 0xf, true)));
}
__device__ inline uint32_t wave_min_u32(uint32_t x) {
    x = row_min_u32(x);
    const uint32_t a = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), 0));
    const uint32_t b = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), 16));
    const uint32_t c = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), 32));
    const uint32_t d = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), 48));
    return min(min(a, b), min(c, d));
}

// A run of candidates as (integer sum, tie summary with the parities taken as
// if the run started from an even sum); st_op(a, b) for a followed by b
// shifts b's parities by a's sum. Associative, (0, 0) the identity, so the
// sums and the tie corrections come out of one scan.
struct SumTies {
    uint32_t s, y;
};
__device__ inline SumTies st_op(SumTies a, SumTies b) {
    return {sat_add(a.s, b.s), tie_comb(a.y, tie_flip(b.y, a.s & 1u))};
}

__device__ inline uint32_t block_min_u32(uint32_t v, uint32_t* lds) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        v = min(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), off, 64)));
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    uint32_t r = lds[0];
    for (uint32_t u = 1; u < kT / 64; ++u) r = min(r, lds[u]);
    return r;
}

// First j in [0, n) with pred(j), for a predicate that is false then true
// along j; n if it is false everywhere. Each round probes the last element of
// kT equal segments (two rounds up to kT * kT elements).
template <typename Pred>
__device__ inline uint32_t block_first_true(uint32_t n, Pred pred, uint32_t* lds) {
    const uint32_t tid = threadIdx.x;
    uint32_t lo = 0, hi = n;
    bool first_round = true;
    while (hi - lo > 1 || (first_round && hi > lo)) {
        const uint32_t len = hi - lo, step = (len + kT - 1) / kT;
        const bool in = tid * step < len;
        const bool ok = in && pred(lo + min((tid + 1) * step, len) - 1);
        const uint32_t seg = block_min_u32(ok ? tid : kT, lds);
        __syncthreads();  // lds is rewritten by the next round
        if (seg == kT) return first_round ? n : hi - 1;  // (later rounds always hold a true element)
        const uint32_t nlo = lo + seg * step;
        hi = min(nlo + step, hi);
        lo = nlo;
        first_round = false;
    }
    return lo;
}

// Whole-vocabulary sampling (one block): the candidates are the first
// count = min(limit, finite) sorted pairs; their probabilities, the f32
// prefix sums above, the top-p cut and the draw.
__global__ __launch_bounds__(kT) void sample_full_kernel(SampleArgs a, const uint32_t* sk, const uint32_t* ids,
                                                         const float* prob, float* prefix) {
    __shared__ unsigned long long red[kT / 64];
    __shared__ uint32_t l_find[kT / 64];
    __shared__ uint2 l_scan[kT / 64];                            // waves' (sum, ties) totals
    __shared__ uint32_t l_first[kT / 64], l_prev[kT / 64];       // waves' first crossing, m before it
    __shared__ float l_pfirst[kT / 64];                          // and its probability
    __shared__ float s_last;                                     // the window's last running sum
    __shared__ uint32_t s_tok;
    const uint32_t tid = threadIdx.x, V = a.vocab;
    // Finite count: the first non-finite sort key (they sort last).
    const uint32_t finite = block_first_true(V, [&](uint32_t j) { return sk[j] == 0xffffffffu; }, l_find);
    const uint32_t limit = min(a.top_k == 0 ? V : a.top_k, V);
    const uint32_t count = min(limit, finite);
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
        const uint32_t lane = tid & 63, wv = tid >> 6;
        // Chain state, the same in every thread: the running sum, the next
        // candidate to add and the width of the next window of candidates.
        float c = 0.0f;
        uint32_t pos = 0, width = kChainW0;
        // The next chunk's probabilities, loaded a chunk ahead: two 16-byte
        // loads from a clamped offset (the buffer holds a multiple of 64
        // words, so the clamp stays inside it; positions at or past count are
        // not used).
        const uint32_t plim = (V + 63) / 64 * 64 - kChainE;
        float pn[kChainE];
        auto load_probs = [&](uint32_t base) {
            const uint32_t jj = min(base + tid * kChainE, plim);
            const float4 q0 = *reinterpret_cast<const float4*>(prob + jj);
            const float4 q1 = *reinterpret_cast<const float4*>(prob + jj + 4);
            pn[0] = q0.x, pn[1] = q0.y, pn[2] = q0.z, pn[3] = q0.w;
            pn[4] = q1.x, pn[5] = q1.y, pn[6] = q1.z, pn[7] = q1.w;
        };
        load_probs(0);
        for (uint32_t cbase = 0; cbase < count; cbase += kChainChunk) {
            const uint32_t cend = min(cbase + kChainChunk, count);
            const uint32_t j0 = cbase + tid * kChainE;
            float p[kChainE];
#pragma unroll
            for (int i = 0; i < kChainE; ++i) {
                const uint32_t j = j0 + i;
                p[i] = j < cend ? pn[i] : 0.0f;
                if (a.trace_probs && j < cend) a.trace_probs[j] = p[i];
            }
            if (cend < count) load_probs(cend);
            while (pos < cend) {
                // Candidates [pos, wend) in the binade of c; waves holding none
                // of them skip the arithmetic.
                const uint32_t wend = min(cend, pos + width);
                const uint32_t bits = __float_as_uint(c);
                // c >= 2^-100 keeps both power-of-two scalings below in range
                // (in practice c >= 1: the first candidate's probability is 1).
                const bool normal = c >= 7.88860905e-31f;
                const int e = static_cast<int>((bits >> 23) & 255u) - 127;
                const uint32_t m = (bits & 0x7fffffu) | 0x800000u;
                const float scale = normal ? __uint_as_float(static_cast<uint32_t>(150 - e) << 23) : 0.0f;  // 2^(23-e)
                const float ulp = normal ? __uint_as_float(static_cast<uint32_t>(104 + e) << 23) : 0.0f;    // 2^(e-23)
                const uint32_t wlo = cbase + wv * 64 * kChainE;
                const bool wact = normal && wlo < wend && wlo + 64 * kChainE > pos;  // uniform in the wave
                uint32_t tl[kChainE], ties = 0;
                SumTies mine = {0u, 0u};
                if (wact) {
                    uint32_t run = 0;
#pragma unroll
                    for (int i = 0; i < kChainE; ++i) {
                        const uint32_t j = j0 + i;
                        const bool act = j >= pos && j < wend;
                        // Clamped: a larger x leaves the binade anyway (a restart).
                        const float x = fminf(p[i] * scale, 33554432.0f);
                        const float fl = floorf(x);
                        const float fr = x - fl;  // exact
                        ties |= (act && fr == 0.5f) ? (1u << i) : 0u;
                        run = sat_add(run, act ? static_cast<uint32_t>(fl) + (fr > 0.5f ? 1u : 0u) : 0u);
                        tl[i] = run;
                    }
                    uint32_t y = 0;
                    if (__any(ties != 0u)) {
#pragma unroll
                        for (int i = 0; i < kChainE; ++i)
                            if ((ties >> i) & 1u) y = tie_comb(y, tie_leaf(tl[i] & 1u));
                    }
                    mine = {run, y};
                } else {
#pragma unroll
                    for (int i = 0; i < kChainE; ++i) tl[i] = 0u;
                }
                // Exclusive (sum, ties) scan over the block in candidate order:
                // within the wave, then over the waves' totals (lanes 0-15 of
                // every wave); sums alone where no tie is in play.
                SumTies up = {0u, 0u};
                if (wact) {
                    SumTies x = mine;
                    if (__any(mine.y != 0u)) {
#pragma unroll
                        for (int off = 1; off < 64; off <<= 1) {
                            const SumTies o = {static_cast<uint32_t>(__shfl_up(static_cast<int>(x.s), off, 64)),
                                               static_cast<uint32_t>(__shfl_up(static_cast<int>(x.y), off, 64))};
                            if (lane >= static_cast<uint32_t>(off)) x = st_op(o, x);
                        }
                        up = {static_cast<uint32_t>(__shfl_up(static_cast<int>(x.s), 1, 64)),
                              static_cast<uint32_t>(__shfl_up(static_cast<int>(x.y), 1, 64))};
                    } else {
                        x.s = wave_scan_sat(x.s);
                        up = {wave_shr1(x.s), 0u};
                    }
                    if (lane == 63) l_scan[wv] = make_uint2(x.s, x.y);
                } else if (lane == 63) {
                    l_scan[wv] = make_uint2(0u, 0u);
                }
                __syncthreads();
                SumTies wt = {0u, 0u};
                if (lane < kT / 64) wt = {l_scan[lane].x, l_scan[lane].y};
                if (__any(wt.y != 0u)) {
#pragma unroll
                    for (int off = 1; off < kT / 64; off <<= 1) {
                        const SumTies o = {static_cast<uint32_t>(__shfl_up(static_cast<int>(wt.s), off, 64)),
                                           static_cast<uint32_t>(__shfl_up(static_cast<int>(wt.y), off, 64))};
                        if (lane >= static_cast<uint32_t>(off)) wt = st_op(o, wt);
                    }
                } else {
                    wt.s = row_scan_sat(wt.s);  // lanes 0-15 are row 0
                }
                SumTies ex = {0u, 0u};
                const int wsrc = __builtin_amdgcn_readfirstlane(static_cast<int>(wv)) - 1;  // uniform
                if (wsrc >= 0)
                    ex = {static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(wt.s), wsrc)),
                          static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(wt.y), wsrc))};
                if (lane != 0) ex = st_op(ex, up);
                // m_j for this thread's candidates, and its first one leaving the binade.
                uint32_t mv[kChainE];
                uint32_t first = 0xffffffffu, prev_first = 0;
                float p_first = 0.0f;
                if (wact) {
                    const uint32_t yin = tie_comb(tie_leaf(0u), tie_flip(ex.y, m & 1u));
                    uint32_t corr = yin & (kTieHas - 1), lp = yin >> 31;
                    const uint32_t mb = sat_add(m, ex.s);
                    uint32_t prev = sat_add(mb, corr);
#pragma unroll
                    for (int i = 0; i < kChainE; ++i) {
                        const uint32_t j = j0 + i;
                        const uint32_t t = sat_add(mb, tl[i]);
                        if ((ties >> i) & 1u) {
                            const uint32_t par = t & 1u;
                            corr += par != lp ? 1u : 0u;
                            lp = par;
                        }
                        mv[i] = sat_add(t, corr);
                        const bool act = j >= pos && j < wend;
                        const uint32_t fl = static_cast<uint32_t>(floorf(fminf(p[i] * scale, 33554432.0f)));
                        if (act && first == 0xffffffffu && sat_add(prev, fl) >= (1u << 24)) {
                            first = j;
                            prev_first = prev;
                            p_first = p[i];
                        }
                        if (j == wend - 1) s_last = static_cast<float>(mv[i]) * ulp;
                        prev = mv[i];
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < kChainE; ++i) mv[i] = 0u;
                }
                if (!normal && j0 <= pos && pos < j0 + kChainE) {  // a plain f32 add
                    first = pos;
#pragma unroll
                    for (int i = 0; i < kChainE; ++i) p_first = j0 + i == pos ? p[i] : p_first;
                }
                // The block's first crossing with its operands, to every thread.
                const uint32_t wmin = wave_min_u32(first);
                if (lane == 0) l_first[wv] = wmin;
                if (first != 0xffffffffu && first == wmin) {
                    l_prev[wv] = prev_first;
                    l_pfirst[wv] = p_first;
                }
                __syncthreads();
                const uint32_t fw = lane < kT / 64 ? l_first[lane] : 0xffffffffu;
                const uint32_t stop =
                    static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(row_min_u32(fw)), 0));
                uint32_t prev_stop = 0;
                float p_stop = 0.0f;
                if (stop != 0xffffffffu) {
                    const int u = __ffsll(static_cast<unsigned long long>(__ballot(lane < kT / 64 && fw == stop))) - 1;
                    prev_stop = l_prev[u];
                    p_stop = l_pfirst[u];
                }
                const uint32_t done = min(stop, wend);
#pragma unroll
                for (int i = 0; i < kChainE; ++i) {
                    const uint32_t j = j0 + i;
                    if (j >= pos && j < done) prefix[j] = static_cast<float>(mv[i]) * ulp;  // exact
                }
                if (stop < wend) {
                    const float cp = stop == pos ? c : static_cast<float>(prev_stop) * ulp;
                    c = __fadd_rn(cp, p_stop);
                    if (j0 <= stop && stop < j0 + kChainE) prefix[stop] = c;
                    width = min(max(2 * (stop - pos + 1), kChainW0), kChainChunk);
                    pos = stop + 1;
                } else {
                    c = s_last;
                    width = min(2 * width, kChainChunk);
                    pos = wend;
                }
            }
        }
        __syncthreads();  // every thread's sums are stored
        const float total = c;  // prefix[count - 1]
        // prepareProbabilities' top-p cut: the first j with prefix[j] / total >= top_p.
        const bool bad_total = total <= 0.0f || !isfinite(total);
        uint32_t k = bad_total ? 1u : count;
        if (!bad_total && a.top_p < 1.0f) {
            const float top_p = a.top_p;
            const uint32_t first =
                block_first_true(count, [&](uint32_t j) { return __fdiv_rn(prefix[j], total) >= top_p; }, l_find);
            k = first == count ? count : first + 1;
        }
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
        uint32_t pick = 0;
        if (s_ok) {
            const float target = s_target;
            const uint32_t first = block_first_true(k, [&](uint32_t j) { return target <= prefix[j]; }, l_find);
            pick = first == k ? k - 1 : first;
        }
        tok = ids[pick];
        for (uint32_t j = tid; j < count; j += kT) {
            if (a.trace_ids) a.trace_ids[j] = ids[j];
            if (a.trace_sums) a.trace_sums[j] = prefix[j];
        }
    }
    if (tid != 0) return;
    if (a.trace_count) *a.trace_count = count;
    sample_finish(a, tok);
}

// Advance the step state as the greedy finish does, then the repeat window
// (the sampling block's thread 0, with the sampled token).
__device__ __forceinline__ void sample_finish(const SampleArgs& a, uint32_t tok) {
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

// Whole-vocabulary scratch: [sort keys A | sort keys B | ids A | ids B |
// probabilities | prefix sums] of vocab words each (256-byte aligned, so each
// holds a multiple of 64 words), then the tiles' digit histograms (256 words
// per tile).
namespace {
size_t full_word_bytes(uint32_t vocab) { return ((size_t)vocab * 4 + 255) / 256 * 256; }
uint32_t full_tiles(uint32_t vocab) { return (vocab + kSortTile - 1) / kSortTile; }
}  // namespace

size_t sample_full_bytes(uint32_t vocab) {
    return vocab ? 6 * full_word_bytes(vocab) + (size_t)full_tiles(vocab) * 256 * sizeof(uint32_t) : 0;
}

hipError_t launch_sample(const SampleArgs& a, hipStream_t s) {
    if (a.temperature > 0.0f && (a.top_k == 0 ? a.vocab : a.top_k) > static_cast<uint32_t>(kMaxCand)) {
        if (!a.full) return hipErrorInvalidValue;
        const size_t wb = full_word_bytes(a.vocab);
        char* base = static_cast<char*>(a.full);
        uint32_t* sk[2] = {reinterpret_cast<uint32_t*>(base), reinterpret_cast<uint32_t*>(base + wb)};
        uint32_t* id[2] = {reinterpret_cast<uint32_t*>(base + 2 * wb), reinterpret_cast<uint32_t*>(base + 3 * wb)};
        float* prob = reinterpret_cast<float*>(base + 4 * wb);
        float* prefix = reinterpret_cast<float*>(base + 5 * wb);
        uint32_t* hist = reinterpret_cast<uint32_t*>(base + 6 * wb);
        const uint32_t tiles = full_tiles(a.vocab);
        hipError_t e = vlaunch(full_keys_kernel, dim3(tiles), dim3(kSortThreads), 0, s, a, sk[0], id[0], hist);
        // Four stable 8-bit passes, A -> B -> A -> B -> A.
        for (uint32_t pass = 0; pass < 4 && e == hipSuccess; ++pass) {
            const uint32_t in = pass & 1u, shift = 8 * pass;
            if (pass > 0)
                e = vlaunch(full_hist_kernel, dim3(tiles), dim3(kSortThreads), 0, s,
                            static_cast<const uint32_t*>(sk[in]), a.vocab, shift, hist);
            if (e == hipSuccess)
                e = vlaunch(full_scatter_kernel, dim3(tiles), dim3(kSortThreads), 0, s,
                            static_cast<const uint32_t*>(sk[in]), static_cast<const uint32_t*>(id[in]), sk[in ^ 1u],
                            id[in ^ 1u], a.vocab, shift, static_cast<const uint32_t*>(hist), tiles);
        }
        if (e == hipSuccess)
            e = vlaunch(full_probs_kernel, dim3(tiles), dim3(kSortThreads), 0, s, static_cast<const uint32_t*>(sk[0]),
                        a.vocab, a.temperature, prob);
        if (e == hipSuccess)
            e = vlaunch(sample_full_kernel, dim3(1), dim3(kT), 0, s, a, static_cast<const uint32_t*>(sk[0]),
                        static_cast<const uint32_t*>(id[0]), static_cast<const float*>(prob), prefix);
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
