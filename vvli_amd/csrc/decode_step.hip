// decode_step.hip -- persistent decode step for gfx950: one cooperative launch
// runs whole token steps (Runner.forwardToken, src/llm.zig:702-766, plus
// llm.argmax, :778-789), optionally many in a row (the decode loop of
// generateGreedyMeasured, src/generator.zig:243-281).
//
// Why: at batch 1 every layer is 5 dependent, HBM-bound GEMV/attention
// phases. As separate kernels each pays ~4 us of launch/ramp/drain; here they
// are phases of one kernel separated by a software grid barrier (~1.6 us:
// each block publishes a generation flag, block 0 gathers and releases), and
// every wave issues the weight loads of its first tile of the next phase
// *before* it enters the barrier, so the barrier hides under the weight
// stream.
//
// Memory model: activations (x, q/k/v, ff, attention partials, argmax keys,
// step state) are exchanged across blocks on different XCDs through
// agent-scope atomic loads/stores, which gfx950 executes with sc1 (coherent
// across the per-XCD L2s), with no L2 writeback/invalidate fences. Each wave
// waits for its own stores (s_waitcnt 0) before the block reaches the barrier.
// New K/V rows are written the same way; older rows are read with plain loads
// (a row is never read before it is written within a launch, and the launch
// starts with clean caches).
//
// Deadlock safety: the launch is cooperative (all blocks co-resident or the
// launch fails), every spin is bounded, and a timeout raises a device error
// flag that makes every block leave at its next barrier; the host reports it.
#include "device_common.hpp"
#include "gemv_tile.hpp"
#include "kernels.hpp"

namespace vvli {

namespace {

constexpr int kMkThreads = 512;
constexpr int kMkWaves = kMkThreads / kWave;
constexpr int kMaxGroupMk = 16;
constexpr int kMaxSplitMk = 16;  // attention splits per kv head (merged by every block)
constexpr uint32_t kSpinLimit = 1u << 21;  // ~1 s of polling: phases take <= ~0.2 ms
constexpr uint32_t kFlagStride = 32;  // words between per-block flags (128 B)

__device__ __forceinline__ float ld_a(const float* p) {
    return __hip_atomic_load(as_global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_a(const uint32_t* p) {
    return __hip_atomic_load(as_global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_a(const unsigned long long* p) {
    return __hip_atomic_load(as_global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_a(float* p, float v) {
    __hip_atomic_store(as_global(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_a(uint32_t* p, uint32_t v) {
    __hip_atomic_store(as_global(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_a(unsigned long long* p, unsigned long long v) {
    __hip_atomic_store(as_global(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_all_mem() { __builtin_amdgcn_s_waitcnt(0); }

// 16-byte loads that see other XCDs' agent-scope stores: buffer loads with
// the sc1 cache policy (the bit the compiler uses for agent-scope atomic
// loads), through a raw buffer resource (out-of-range reads return 0).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
constexpr int kCpolSc1 = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coh_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float4 ld_coh4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCpolSc1);
    return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}

// ---------------------------------------------------------------------------
// Grid barrier: block b stores generation g in flags[b]; block 0 waits for all
// flags, then stores g in `release`; the others wait for `release`.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool mk_barrier(const DecodeStepParams& p, uint32_t* s_gen, int* s_ok) {
    __syncthreads();
    const uint32_t gen = *s_gen + 1;
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid == 0) *s_gen = gen;
    if (tid == 0) {
        *s_ok = 1;
        if (p.timing && (gen + 1) * p.timing_slots <= p.timing_stride)
            p.timing[blockIdx.x * p.timing_stride + gen * p.timing_slots + p.timing_slots - 1] =
                __builtin_amdgcn_s_memrealtime();
        st_a(p.flags + blockIdx.x * kFlagStride, gen);
    }
    if (blockIdx.x == 0) {
        __syncthreads();
        for (uint32_t b = tid; b < gridDim.x; b += kMkThreads) {
            uint32_t spins = 0;
            while (ld_a(p.flags + b * kFlagStride) < gen) {
                if (++spins > kSpinLimit || ((spins & 255u) == 0 && ld_a(p.error) != 0)) {
                    st_a(p.error, 1u);
                    *s_ok = 0;
                    break;
                }
            }
        }
        __syncthreads();
        if (tid == 0) {
            if (p.timing && (gen + 1) * p.timing_slots <= p.timing_stride)
                p.timing[(size_t)gridDim.x * p.timing_stride + gen * p.timing_slots + p.timing_slots - 1] =
                    __builtin_amdgcn_s_memrealtime();
            st_a(p.release, *s_ok ? gen : 0xffffffffu);
        }
    } else if (tid == 0) {
        uint32_t spins = 0;
        while (ld_a(p.release) < gen) {
            if (++spins > kSpinLimit || ((spins & 255u) == 0 && ld_a(p.error) != 0)) {
                st_a(p.error, 1u);
                *s_ok = 0;
                break;
            }
        }
        if (ld_a(p.error) != 0) *s_ok = 0;
    }
    __syncthreads();
    if (tid == 0 && p.timing && p.timing_slots > 1 && (gen + 1) * p.timing_slots <= p.timing_stride)
        p.timing[blockIdx.x * p.timing_stride + gen * p.timing_slots] = __builtin_amdgcn_s_memrealtime();
    return *s_ok != 0;
}

// Detail timing mark of the current phase (16-slot timing only).
__device__ __forceinline__ void mk_mark(const DecodeStepParams& p, uint32_t gen, int slot) {
    if (p.timing && p.timing_slots > 1 && (gen + 1) * p.timing_slots <= p.timing_stride)
        p.timing[blockIdx.x * p.timing_stride + gen * p.timing_slots + slot] = __builtin_amdgcn_s_memrealtime();
}

// ---------------------------------------------------------------------------
// GEMV phases (bf16 weights). A tile holds two row pointers: rows 2t, 2t+1
// (plain / residual / logits) or gate row t and up row t (SwiGLU).
// ---------------------------------------------------------------------------
using MkGemv = DecodeGemv;

__device__ __forceinline__ const uint16_t* seg_w(const MkGemv& g, int seg) {
    return seg == 0 ? g.w0 : (seg == 1 ? g.w1 : g.w2);
}
__device__ __forceinline__ const uint16_t* seg_bias(const MkGemv& g, int seg) {
    return seg == 0 ? g.b0 : (seg == 1 ? g.b1 : g.b2);
}
__device__ __forceinline__ float* seg_out(const MkGemv& g, int seg) { return seg == 0 ? g.o0 : (seg == 1 ? g.o1 : g.o2); }

struct MkTile {
    const uint16_t* p[2];  // weight rows streamed by this tile
    uint32_t row[2];       // output rows (row[1] unused in the SwiGLU mode)
    int seg;               // segment of both rows (q | k | v in the plain mode)
    bool valid[2];         // output row exists
};

__device__ __forceinline__ uint32_t mk_tiles(const MkGemv& g, int mode) {
    const uint32_t total = g.r0 + g.r1 + g.r2;
    return mode == kGemvGateUp ? total : (total + 1) / 2;
}

// Tile `tile`: gate row t and up row t (SwiGLU), else rows 2t, 2t+1 of the
// stacked segments (segments hold an even number of rows, so a tile never
// straddles two; an odd last row re-reads its own row as the second).
__device__ __forceinline__ void mk_make_tile(const MkGemv& g, int mode, uint32_t tile, MkTile& t) {
    const uint32_t K = g.K;
    if (mode == kGemvGateUp) {
        const bool v = tile < g.r0;
        const uint32_t r = v ? tile : 0;
        t.p[0] = g.w0 + (size_t)r * K;
        t.p[1] = g.w_up + (size_t)r * K;
        t.row[0] = t.row[1] = r;
        t.seg = 0;
        t.valid[0] = v;
        t.valid[1] = false;
    } else {
        const uint32_t total = g.r0 + g.r1 + g.r2;
        uint32_t first = tile * 2;
        int seg = 0;
        if (first >= g.r0) {
            first -= g.r0;
            seg = 1;
            if (first >= g.r1) {
                first -= g.r1;
                seg = 2;
            }
        }
        const uint16_t* wb = seg_w(g, seg);
        t.seg = seg;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            t.valid[r] = tile * 2 + r < total;
            const uint32_t gr = t.valid[r] ? first + r : first;
            t.p[r] = wb + (size_t)gr * K;
            t.row[r] = gr;
        }
    }
}

struct MkWave {
    uint32_t wid;    // wave (t mod blocks) ... : spreads a short phase over every CU
    uint32_t wid_c;  // block-contiguous wave index: long phases sweep memory together
    uint32_t nw;
    int lane;
};

// Wave index that owns tiles wid, wid + nw, ... of a phase with `ntiles` tiles.
__device__ __forceinline__ uint32_t mk_owner(const MkWave& w, uint32_t ntiles) {
    return ntiles > w.nw ? w.wid_c : w.wid;
}

// Issue the first item of this wave's first tile (weights only: may run
// before the phase input exists).
__device__ __forceinline__ bool mk_prefetch(const MkGemv& g, int mode, const MkWave& w, uint4 (&buf)[2][kNJC],
                                            MkTile& t) {
    const uint32_t ntiles = mk_tiles(g, mode);
    const uint32_t me = mk_owner(w, ntiles);
    if (me >= ntiles) return false;
    mk_make_tile(g, mode, me, t);
    issue<uint16_t, 2>(buf, t.p, 0, g.K / 8, w.lane);
    return true;
}

// Run this wave's tiles of a GEMV phase (`mode` is uniform over the grid);
// bufA/tA hold the prefetched first item when `have` is set.
//
// Tile results are parked in lanes -- lane k holds the k-th tile of the
// current batch of 64 -- and written with one vector store per batch: on gfx9
// loads and stores share one completion counter, so a store per tile would
// make every following weight wait for that store's acknowledgement. Each lane
// also loads its tile's addend (residual row or bias) when the batch opens.
__device__ __forceinline__ void mk_gemv(const MkGemv& g, int mode, const float* xs, const MkWave& w,
                                        uint4 (&bufA)[2][kNJC], MkTile& tA, bool have, unsigned long long& best) {
    const int lane = w.lane;
    const uint32_t U = g.K / 8;
    const uint32_t per_item = kNJC * kWave;
    const uint32_t nchunk = (U + per_item - 1) / per_item;
    const uint32_t ntiles = mk_tiles(g, mode);
    const uint32_t me = mk_owner(w, ntiles);
    const uint32_t my_tiles = me < ntiles ? (ntiles - 1 - me) / w.nw + 1 : 0;
    const uint32_t n_items = my_tiles * nchunk;
    if (n_items == 0) return;
    if (!have) {
        mk_make_tile(g, mode, me, tA);
        issue<uint16_t, 2>(bufA, tA.p, 0, U, lane);
    }
    // Lane state of the open batch: rows, segment, addends, parked results.
    uint32_t ra = 0, rb = 0;
    int sa = 0;
    bool va = false, vb = false;
    float ea = 0.f, eb = 0.f, oa = 0.f, ob = 0.f;
    uint32_t base = 0, pending = 0;
    auto open_batch = [&]() {
        const uint32_t k = base + (uint32_t)lane;
        const bool mine = k < my_tiles;
        MkTile t;
        mk_make_tile(g, mode, mine ? me + k * w.nw : me, t);
        ra = t.row[0];
        rb = t.row[1];
        sa = t.seg;
        va = mine && t.valid[0];
        vb = mine && t.valid[1];
        ea = eb = 0.f;
        if (mode == kGemvResid) {  // x = residual + proj (addInto, src/llm.zig:1389-1396)
            if (va) ea = ld_a(g.o0 + ra);
            if (vb) eb = ld_a(g.o0 + rb);
        } else if (mode == kGemvPlain) {  // linearRange: dot + bias (src/llm.zig:1273)
            const uint16_t* bias = seg_bias(g, sa);
            if (bias && va) ea = __uint_as_float((uint32_t)*as_global(bias + ra) << 16);
            if (bias && vb) eb = __uint_as_float((uint32_t)*as_global(bias + rb) << 16);
        }
    };
    auto flush = [&]() {
        if ((uint32_t)lane < pending) {
            if (mode == kGemvLogits) {
                if (va) {
                    if (ra == 0)
                        st_a(g.o0, oa);  // read back by the argmax block (NaN rule)
                    else
                        *as_global(g.o0 + ra) = oa;
                }
                if (vb) *as_global(g.o0 + rb) = ob;
            } else {
                float* o = mode == kGemvPlain ? seg_out(g, sa) : g.o0;
                if (va) st_a(o + ra, oa + ea);
                if (vb) st_a(o + rb, ob + eb);
            }
        }
        pending = 0;
    };
    open_batch();
    uint4 bufB[2][kNJC];
    MkTile tc = tA, tn = tA;  // tiles of the item being consumed / in flight
    float acc0 = 0.f, acc1 = 0.f;
    for (uint32_t it = 0; it < n_items; ++it) {
        const uint32_t chunk = it % nchunk;
        const bool more = it + 1 < n_items;
        if (more && chunk == nchunk - 1) mk_make_tile(g, mode, me + ((it + 1) / nchunk) * w.nw, tn);
        const uint32_t nbase = (chunk == nchunk - 1 ? 0 : chunk + 1) * per_item;
        float acc[2] = {acc0, acc1};
        if (it & 1) {
            if (more) issue<uint16_t, 2>(bufA, tn.p, nbase, U, lane);
            consume<uint16_t, 2>(bufB, xs, chunk * per_item, U, lane, acc);
        } else {
            if (more) issue<uint16_t, 2>(bufB, tn.p, nbase, U, lane);
            consume<uint16_t, 2>(bufA, xs, chunk * per_item, U, lane, acc);
        }
        acc0 = acc[0];
        acc1 = acc[1];
        if (chunk == nchunk - 1) {
            float v0 = wave_sum(acc0);
            const float v1 = wave_sum(acc1);
            acc0 = acc1 = 0.f;
            if (mode == kGemvGateUp) {
                v0 = (v0 / (1.0f + expf(-v0))) * v1;  // siluMulInto, src/llm.zig:1382-1387
            } else if (mode == kGemvLogits && lane == 0) {
                if (tc.valid[0]) {
                    const unsigned long long k0 = argmax_key(v0, tc.row[0]);
                    best = k0 > best ? k0 : best;
                }
                if (tc.valid[1]) {
                    const unsigned long long k1 = argmax_key(v1, tc.row[1]);
                    best = k1 > best ? k1 : best;
                }
            }
            if ((uint32_t)lane == pending) {
                oa = v0;
                ob = v1;
            }
            if (++pending == kWave) {
                flush();
                base += kWave;
                open_batch();
            }
            tc = tn;
        }
    }
    flush();
}

// ---------------------------------------------------------------------------
// Input staging into LDS.
// ---------------------------------------------------------------------------
// xs[k] = src[k] (* norm_w[k] * s) with s = 1/sqrt(mean(src^2) + eps)
// (rmsNormInto, src/llm.zig:1287-1300). src is an f32 activation read with
// agent-scope loads, or (src_bf16) a bf16 embedding row (copyEmbeddingToken,
// :1373-1380), which block 0 also publishes as the residual stream x_out.
// The norm weights are loaded in the same batch as the activation (into
// nws = xs + n), so the phase waits for one memory round trip, not two.
__device__ __forceinline__ void mk_stage(float* xs, float* red, const float* src, const uint16_t* src_bf16,
                                         float* x_out, const uint16_t* norm_w, float eps, uint32_t n) {
    const int tid = threadIdx.x;
    constexpr int B = 8;  // 16-byte loads issued before any is consumed
    float* nws = xs + n;
    float ss = 0.f;
    if (src_bf16) {
        for (uint32_t k = tid; k < n; k += kMkThreads) {
            const float v = WeightTraits<uint16_t>::at(src_bf16, k);
            xs[k] = v;
            if (norm_w) nws[k] = __uint_as_float((uint32_t)*as_global(norm_w + k) << 16);
            ss = fmaf(v, v, ss);
            if (x_out) st_a(x_out + k, v);
        }
    } else {
        const __amdgpu_buffer_rsrc_t r = coh_rsrc(src, n * 4);
        const uint32_t n4 = n / 4;
        for (uint32_t i0 = tid; i0 < n4; i0 += B * kMkThreads) {
            float4 v[B];
            uint2 nv[B];
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const uint32_t i = i0 + b * kMkThreads;
                v[b] = ld_coh4(r, i * 16);
                nv[b] = (norm_w && i < n4) ? load_u32x2(norm_w + 4 * i) : make_uint2(0, 0);
            }
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const uint32_t i = i0 + b * kMkThreads;
                if (i < n4) {
                    *reinterpret_cast<float4*>(xs + 4 * i) = v[b];
                    if (norm_w)
                        *reinterpret_cast<float4*>(nws + 4 * i) =
                            make_float4(__uint_as_float(nv[b].x << 16), __uint_as_float(nv[b].x & 0xffff0000u),
                                        __uint_as_float(nv[b].y << 16), __uint_as_float(nv[b].y & 0xffff0000u));
                    ss = fmaf(v[b].x, v[b].x, ss);
                    ss = fmaf(v[b].y, v[b].y, ss);
                    ss = fmaf(v[b].z, v[b].z, ss);
                    ss = fmaf(v[b].w, v[b].w, ss);
                }
            }
        }
    }
    if (norm_w) {
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float total = 0.f;
#pragma unroll
        for (int i = 0; i < kMkWaves; ++i) total += red[i];
        const float scale = 1.0f / sqrtf(total / (float)n + eps);
        for (uint32_t k = tid; k < n; k += kMkThreads) xs[k] = xs[k] * nws[k] * scale;
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// Attention phase: units (kv head h, split s) over blocks.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void rope_rot(const float* src, float* dst, int f, int sc, float c, float s) {
    const float x0 = src[f], x1 = src[sc];
    dst[f] = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, s));
    dst[sc] = __fadd_rn(__fmul_rn(x0, s), __fmul_rn(x1, c));
}

// LDS layout of the attention phase (floats): q [16][HDMAX], K tile
// [TILE][HDMAX+4] (16-byte aligned rows), V tile [TILE][HDMAX], probabilities
// [16][TILE], new k / v rows, running max / sum / correction per q head.
template <int HDMAX>
struct AttnLds {
    static constexpr int TILE = 4096 / HDMAX;  // 64 rows at hd 64, 32 at hd 128
    static constexpr int KS = HDMAX + 4;
    static constexpr int kQ = 0;
    static constexpr int kK = kQ + kMaxGroupMk * HDMAX;
    static constexpr int kV = kK + TILE * KS;
    static constexpr int kP = kV + TILE * HDMAX;
    static constexpr int kKnew = kP + kMaxGroupMk * TILE;
    static constexpr int kVnew = kKnew + HDMAX;
    static constexpr int kM = kVnew + HDMAX;
    static constexpr int kL = kM + kMaxGroupMk;
    static constexpr int kC = kL + kMaxGroupMk;
    static constexpr int kTotal = kC + kMaxGroupMk;
};

// One (kv head, split) unit per block iteration: RoPE of q and of the new k
// (applyRoPE, src/llm.zig:1337-1371), K/V append at pos (:744-745), and an
// online-softmax pass over the split's positions for the `group` q heads
// sharing the kv head (computeAttentionInto, :1302-1335). Partials (m, l,
// acc) are merged by the split that finishes last into p.attn. EXACT: hd == HDMAX (loops
// fully unrolled), else hd <= HDMAX at run time.
template <int HDMAX, bool EXACT>
__device__ __forceinline__ void mk_attention(const DecodeStepParams& p, uint32_t layer, uint32_t pos, uint32_t chunk,
                                          uint32_t ns, float* smem) {
    using LY = AttnLds<HDMAX>;
    constexpr int TILE = LY::TILE, KS = LY::KS;
    constexpr int NP = (kMaxGroupMk * HDMAX + kMkThreads - 1) / kMkThreads;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int hd = EXACT ? HDMAX : (int)p.hd;
    const int half = hd / 2;
    const int G = (int)(p.heads / p.kv_heads);
    const uint32_t kvw = p.kvdim;
    float* qs = smem + LY::kQ;
    float* ks = smem + LY::kK;
    float* vs = smem + LY::kV;
    float* ps = smem + LY::kP;
    float* knew = smem + LY::kKnew;
    float* vnew = smem + LY::kVnew;
    float* m_s = smem + LY::kM;
    float* l_s = smem + LY::kL;
    float* c_s = smem + LY::kC;
    const float* cs = p.rope_cs + (size_t)pos * hd;
    float* kc = p.kcache + (size_t)layer * p.max_seq * kvw;
    float* vc = p.vcache + (size_t)layer * p.max_seq * kvw;
    const float* q = p.qkv;
    const float* kn_all = p.qkv + p.heads * p.hd;
    const float* vn_all = kn_all + kvw;
    const bool inter = p.rope_layout == 0;

    for (uint32_t unit = blockIdx.x; unit < p.kv_heads * ns; unit += gridDim.x) {
        const uint32_t h = unit / ns, s = unit - h * ns;
        const uint32_t t0 = s * chunk, t1 = min(t0 + chunk, pos + 1);
        const bool owns = pos >= t0 && pos < t1;
        for (int idx = tid; idx < G * half; idx += kMkThreads) {
            const int g = idx / half, i = idx - g * half;
            const int f = inter ? 2 * i : i, sc = inter ? 2 * i + 1 : i + half;
            const float* src = q + (size_t)(h * G + g) * hd;
            const float x0 = ld_a(src + f), x1 = ld_a(src + sc);
            const float c = cs[2 * i], sn = cs[2 * i + 1];
            qs[g * HDMAX + f] = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, sn));
            qs[g * HDMAX + sc] = __fadd_rn(__fmul_rn(x0, sn), __fmul_rn(x1, c));
        }
        if (owns) {
            for (int i = tid; i < half; i += kMkThreads) {
                const int f = inter ? 2 * i : i, sc = inter ? 2 * i + 1 : i + half;
                const float x0 = ld_a(kn_all + (size_t)h * hd + f), x1 = ld_a(kn_all + (size_t)h * hd + sc);
                const float c = cs[2 * i], sn = cs[2 * i + 1];
                knew[f] = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, sn));
                knew[sc] = __fadd_rn(__fmul_rn(x0, sn), __fmul_rn(x1, c));
            }
            for (int d = tid; d < hd; d += kMkThreads) vnew[d] = ld_a(vn_all + (size_t)h * hd + d);
        }
        if (tid < kMaxGroupMk) {
            m_s[tid] = -INFINITY;
            l_s[tid] = 0.f;
        }
        __syncthreads();
        if (owns) {
            for (int d = tid; d < hd; d += kMkThreads) {
                st_a(kc + (size_t)pos * kvw + (size_t)h * hd + d, knew[d]);
                st_a(vc + (size_t)pos * kvw + (size_t)h * hd + d, vnew[d]);
            }
        }
        float acc[NP];
#pragma unroll
        for (int i = 0; i < NP; ++i) acc[i] = 0.f;
        for (uint32_t ta = t0; ta < t1; ta += TILE) {
            const int tlen = (int)min((uint32_t)TILE, t1 - ta);
            const int vpr = hd / 4;
            for (int idx = tid; idx < tlen * vpr; idx += kMkThreads) {
                const int j = idx / vpr, c4 = (idx - j * vpr) * 4;
                const uint32_t t = ta + j;
                float4 k4, v4;
                if (t == pos) {
                    k4 = *reinterpret_cast<const float4*>(knew + c4);
                    v4 = *reinterpret_cast<const float4*>(vnew + c4);
                } else {
                    const size_t off = (size_t)t * kvw + (size_t)h * hd + c4;
                    k4 = load_f32x4(kc + off);
                    v4 = load_f32x4(vc + off);
                }
                *reinterpret_cast<float4*>(ks + j * KS + c4) = k4;
                *reinterpret_cast<float4*>(vs + j * HDMAX + c4) = v4;
            }
            __syncthreads();
            // scores s[g][j] = (q_g . K_j) * scale, four independent chains
            for (int idx = tid; idx < G * TILE; idx += kMkThreads) {
                const int g = idx / TILE, j = idx - g * TILE;
                float d0 = -INFINITY;
                if (j < tlen) {
                    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
                    const float* qr = qs + g * HDMAX;
                    const float* kr = ks + j * KS;
                    if constexpr (EXACT) {
#pragma unroll
                        for (int d = 0; d < HDMAX; d += 4) {
                            const float4 q4 = *reinterpret_cast<const float4*>(qr + d);
                            const float4 k4 = *reinterpret_cast<const float4*>(kr + d);
                            a0 = fmaf(q4.x, k4.x, a0);
                            a1 = fmaf(q4.y, k4.y, a1);
                            a2 = fmaf(q4.z, k4.z, a2);
                            a3 = fmaf(q4.w, k4.w, a3);
                        }
                    } else {
                        for (int d = 0; d < hd; d += 4) {
                            const float4 q4 = *reinterpret_cast<const float4*>(qr + d);
                            const float4 k4 = *reinterpret_cast<const float4*>(kr + d);
                            a0 = fmaf(q4.x, k4.x, a0);
                            a1 = fmaf(q4.y, k4.y, a1);
                            a2 = fmaf(q4.z, k4.z, a2);
                            a3 = fmaf(q4.w, k4.w, a3);
                        }
                    }
                    d0 = ((a0 + a1) + (a2 + a3)) * p.scale;
                }
                ps[g * TILE + j] = d0;
            }
            __syncthreads();
            for (int g = wave; g < G; g += kMkWaves) {
                const float sc = lane < TILE ? ps[g * TILE + lane] : -INFINITY;
                const float m_old = m_s[g];
                const float m_new = fmaxf(m_old, wave_max(sc));
                const float corr = expf(m_old - m_new);
                const float e = lane < tlen ? expf(sc - m_new) : 0.f;
                if (lane < TILE) ps[g * TILE + lane] = e;
                const float lsum = wave_sum(e);
                if (lane == 0) {
                    l_s[g] = l_s[g] * corr + lsum;
                    m_s[g] = m_new;
                    c_s[g] = corr;
                }
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int idx = tid + i * kMkThreads;
                if (idx < G * hd) {
                    const int g = idx / hd, d = idx - g * hd;
                    const float* pr = ps + g * TILE;
                    float v0 = acc[i] * c_s[g], v1 = 0.f, v2 = 0.f, v3 = 0.f;
                    int j = 0;
                    for (; j + 4 <= tlen; j += 4) {
                        const float4 p4 = *reinterpret_cast<const float4*>(pr + j);
                        v0 = fmaf(p4.x, vs[(j + 0) * HDMAX + d], v0);
                        v1 = fmaf(p4.y, vs[(j + 1) * HDMAX + d], v1);
                        v2 = fmaf(p4.z, vs[(j + 2) * HDMAX + d], v2);
                        v3 = fmaf(p4.w, vs[(j + 3) * HDMAX + d], v3);
                    }
                    for (; j < tlen; ++j) v0 = fmaf(pr[j], vs[j * HDMAX + d], v0);
                    acc[i] = (v0 + v1) + (v2 + v3);
                }
            }
            __syncthreads();
        }
        // Partials of this split: (m, l) per q head and the unnormalised output.
        float* pml = p.part_ml + ((size_t)h * p.nsplit + s) * G * 2;
        float* pacc = p.part_acc + ((size_t)h * p.nsplit + s) * G * hd;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int idx = tid + i * kMkThreads;
            if (idx < G * hd) st_a(pacc + idx, acc[i]);  // idx = g * hd + d
        }
        if (tid < G) {
            st_a(pml + 2 * tid, m_s[tid]);
            st_a(pml + 2 * tid + 1, l_s[tid]);
        }
        // The last split of kv head h to finish merges all of them (flash-
        // decoding merge): out = sum_s exp(m_s - M) acc_s / sum_s exp(m_s - M) l_s.
        wait_all_mem();
        __syncthreads();
        if (tid == 0) {
            const uint32_t prev = __hip_atomic_fetch_add(p.counters + h, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *reinterpret_cast<uint32_t*>(m_s) = prev == ns - 1 ? 1u : 0u;  // m_s[0] is free now
        }
        __syncthreads();
        const bool last = *reinterpret_cast<uint32_t*>(m_s) != 0;
        __syncthreads();
        if (last) {
            float* wsp = ps;  // [split][group] merge weights
            for (int g = wave; g < G; g += kMkWaves) {
                float mv = -INFINITY, lv = 0.f;
                if ((uint32_t)lane < ns) {
                    const float* q2 = p.part_ml + (((size_t)h * p.nsplit + lane) * G + g) * 2;
                    mv = ld_a(q2);
                    lv = ld_a(q2 + 1);
                }
                const float M = wave_max(mv);
                const float e = (uint32_t)lane < ns ? expf(mv - M) : 0.f;
                const float L = wave_sum(lv * e);
                if ((uint32_t)lane < ns) wsp[lane * G + g] = e / L;
            }
            __syncthreads();
            const __amdgpu_buffer_rsrc_t r = coh_rsrc(p.part_acc + (size_t)h * p.nsplit * G * hd, ns * G * hd * 4);
            const int n4 = G * hd / 4;
            for (int i4 = tid; i4 < n4; i4 += kMkThreads) {
                const int g = (4 * i4) / hd;
                float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
                for (uint32_t s0 = 0; s0 < ns; s0 += 8) {
                    float4 v[8];
#pragma unroll
                    for (int b = 0; b < 8; ++b) v[b] = ld_coh4(r, ((s0 + b) * G * hd + 4 * i4) * 4);
#pragma unroll
                    for (int b = 0; b < 8; ++b) {
                        if (s0 + b < ns) {
                            const float w = wsp[(s0 + b) * G + g];
                            o.x = fmaf(v[b].x, w, o.x);
                            o.y = fmaf(v[b].y, w, o.y);
                            o.z = fmaf(v[b].z, w, o.z);
                            o.w = fmaf(v[b].w, w, o.w);
                        }
                    }
                }
                float* dst = p.attn + (size_t)h * G * hd + 4 * i4;
                st_a(dst, o.x);
                st_a(dst + 1, o.y);
                st_a(dst + 2, o.z);
                st_a(dst + 3, o.w);
            }
            if (tid == 0) st_a(p.counters + h, 0u);
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// The kernel.
// ---------------------------------------------------------------------------
// Phases of one token step: per layer Q (input RMSNorm + q/k/v), A (RoPE, KV
// append, attention), O (x += Wo.attn), G (post-attention RMSNorm, gate/up,
// SwiGLU), D (x += Wd.ff); then the logits phase (final RMSNorm + lm_head).
// All GEMV phases run through one code path with a grid-uniform mode, so the
// whole step loop stays small enough for the instruction cache.
enum : uint32_t { kPhQ = 0, kPhA = 1, kPhO = 2, kPhG = 3, kPhD = 4, kPhPerLayer = 5 };

struct MkPhase {
    uint32_t layer, kind;
    bool logits;
};

__device__ __forceinline__ MkPhase mk_phase(uint32_t ph, uint32_t layers) {
    MkPhase f;
    f.layer = ph / kPhPerLayer;
    f.kind = ph - f.layer * kPhPerLayer;
    f.logits = f.layer == layers;
    return f;
}

__device__ __forceinline__ int mk_mode(const MkPhase& f) {
    if (f.logits) return kGemvLogits;
    return f.kind == kPhQ ? kGemvPlain : (f.kind == kPhG ? kGemvGateUp : kGemvResid);
}

// The host-built tables (GEMV descriptors, norm weights per layer) are copied
// into LDS when the kernel starts: read from global memory they would miss the
// caches every phase (the weight stream evicts them) and put a memory round
// trip in front of every phase.
struct MkTables {
    const MkGemv* gemv;         // [layers * 4 + 1]
    const uint16_t* const* norm;  // [layers * 2]: input, post-attention
};

__device__ __forceinline__ MkTables mk_load_tables(const DecodeStepParams& p, char* lds) {
    MkGemv* g = reinterpret_cast<MkGemv*>(lds);
    const uint16_t** nrm = reinterpret_cast<const uint16_t**>(lds + (size_t)(p.layers * 4 + 1) * sizeof(MkGemv));
    const uint32_t gw = (p.layers * 4 + 1) * sizeof(MkGemv) / 4;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(p.gemv);
    for (uint32_t i = threadIdx.x; i < gw; i += kMkThreads) reinterpret_cast<uint32_t*>(g)[i] = src[i];
    for (uint32_t i = threadIdx.x; i < p.layers * 2; i += kMkThreads)
        nrm[i] = (i & 1) ? p.layer[i >> 1].post_norm : p.layer[i >> 1].input_norm;
    __syncthreads();
    return MkTables{g, nrm};
}

__device__ __forceinline__ const MkGemv& mk_gemv_of(const DecodeStepParams& p, const MkTables& t, const MkPhase& f) {
    return t.gemv[f.logits ? p.layers * 4 : f.layer * 4 + (f.kind == kPhQ ? 0 : f.kind - 1)];
}
__device__ __forceinline__ const uint16_t* mk_norm_of(const DecodeStepParams& p, const MkTables& t, const MkPhase& f) {
    if (f.logits) return p.final_norm;
    return f.kind == kPhQ ? t.norm[f.layer * 2] : (f.kind == kPhG ? t.norm[f.layer * 2 + 1] : nullptr);
}

template <int HDMAX, bool EXACT>
__global__ __launch_bounds__(kMkThreads) void decode_step_kernel(DecodeStepParams p) {
    extern __shared__ float smem[];
    __shared__ int s_ok;
    __shared__ uint32_t s_gen;
    __shared__ float red[kMkWaves];
    __shared__ uint32_t s_ctl[4];
    const int tid = threadIdx.x;
    MkWave w;
    w.lane = tid & 63;
    // Tile t goes to wave (t mod blocks) of ... so consecutive tiles land on
    // different CUs and a phase with fewer tiles than waves still uses them all.
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar registers)
    w.wid = wave * gridDim.x + blockIdx.x;
    w.wid_c = blockIdx.x * kMkWaves + wave;
    w.nw = gridDim.x * kMkWaves;
    if (tid == 0) s_gen = 0;
    uint4 buf[2][kNJC];
    MkTile tile;
    unsigned long long best = 0ull;
    const uint32_t H = p.hidden;
    if (p.timing && tid == 0 && blockIdx.x == 0)
        p.timing[(size_t)gridDim.x * p.timing_stride + p.timing_slots - 1] = __builtin_amdgcn_s_memrealtime();
    const uint32_t nph = kPhPerLayer * p.layers + 1;
    const MkTables tb = mk_load_tables(p, reinterpret_cast<char*>(smem) + p.table_lds_offset);

    for (uint32_t step = 0; step < p.n_steps; ++step) {
        // Step state (written by block 0 in the previous step's argmax phase).
        if (tid == 0) {
            s_ctl[0] = ld_a(&p.state->token);
            s_ctl[1] = ld_a(&p.state->pos);
        }
        __syncthreads();
        const uint32_t token = s_ctl[0], pos = s_ctl[1];
        __syncthreads();
        if (pos >= p.max_seq || token >= p.vocab) {  // host validated; defensive stop
            if (blockIdx.x == 0 && tid == 0) st_a(p.error, 2u);
            return;
        }
        const uint32_t T = pos + 1;
        uint32_t chunk = (T + p.nsplit - 1) / p.nsplit;
        if (chunk < p.min_chunk) chunk = p.min_chunk;
        const uint32_t ns = (T + chunk - 1) / chunk;
        bool have = mk_prefetch(tb.gemv[0], kGemvPlain, w, buf, tile);

        for (uint32_t ph = 0; ph < nph; ++ph) {
            const MkPhase f = mk_phase(ph, p.layers);
            if (f.kind == kPhA && !f.logits) {
                mk_attention<HDMAX, EXACT>(p, f.layer, pos, chunk, ns, smem);
            } else {
                const uint16_t* norm = mk_norm_of(p, tb, f);
                const float* src = f.kind == kPhO ? p.attn : (f.kind == kPhD ? p.ff : p.x);
                // Layer 0 reads the embedding row straight from the blob; block 0
                // publishes it as the residual stream, first read two barriers on.
                mk_stage(smem, red, src, ph == 0 ? p.embed + (size_t)token * H : nullptr,
                         (ph == 0 && blockIdx.x == 0) ? p.x : nullptr, norm, p.eps, f.kind == kPhD ? p.inter : H);
                if (tid == 0) mk_mark(p, s_gen, 1);
                if (f.logits) best = 0ull;
                mk_gemv(mk_gemv_of(p, tb, f), mk_mode(f), smem, w, buf, tile, have, best);
                if (f.logits && w.lane == 0) st_a(p.keys + w.wid, best);
            }
            if (w.lane == 0) mk_mark(p, s_gen, 2 + (tid >> 6));
            wait_all_mem();
            // Issue the first weights of the next GEMV phase before the barrier.
            if (ph + 1 < nph) {
                const MkPhase nf = mk_phase(ph + 1, p.layers);
                if (nf.kind != kPhA || nf.logits) have = mk_prefetch(mk_gemv_of(p, tb, nf), mk_mode(nf), w, buf, tile);
            }
            if (!mk_barrier(p, &s_gen, &s_ok)) return;
        }

        // ---- argmax + step advance (block 0) ----
        if (blockIdx.x == 0) {
            __shared__ unsigned long long kred[kMkWaves];
            unsigned long long b = 0ull;
            for (uint32_t i = tid; i < w.nw; i += kMkThreads) {
                const unsigned long long k = ld_a(p.keys + i);
                b = k > b ? k : b;
            }
            b = wave_max_u64(b);
            if (w.lane == 0) kred[tid >> 6] = b;
            __syncthreads();
            if (tid == 0) {
                for (int i = 0; i < kMkWaves; ++i) b = kred[i] > b ? kred[i] : b;
                const float l0 = ld_a(p.logits);
                const uint32_t tok = (l0 != l0) ? 0u : argmax_key_index(b);  // llm.argmax, src/llm.zig:778-789
                const uint32_t next_pos = pos + 1;
                const uint32_t prompt_len = ld_a(&p.state->prompt_len);
                uint32_t next_tok = tok, stop = 0;
                st_a(&p.state->argmax, tok);
                if (next_pos < prompt_len) {
                    next_tok = p.prompt[next_pos];  // still inside the prompt (generator.zig:243-251)
                } else if (ld_a(&p.state->counting)) {
                    const uint32_t n_out = ld_a(&p.state->n_out);
                    if (n_out < p.out_cap) st_a(p.out_tokens + n_out, tok);
                    st_a(&p.state->n_out, n_out + 1);
                    if (p.eos >= 0 && (int64_t)tok == p.eos) stop = 1;  // emit EOS, do not forward it
                }
                if (next_pos >= p.max_seq) stop = 1;
                st_a(&p.state->token, next_tok);
                st_a(&p.state->pos, next_pos);
                st_a(&p.state->stop, stop);
            }
        }
        if (step + 1 < p.n_steps) {
            wait_all_mem();
            if (!mk_barrier(p, &s_gen, &s_ok)) return;
            if (tid == 0) s_ctl[2] = ld_a(&p.state->stop);
            __syncthreads();
            if (s_ctl[2]) return;
        }
    }
}

}  // namespace

size_t decode_step_table_offset(uint32_t hidden, uint32_t inter, uint32_t hd) {
    const size_t attn = hd <= 64 ? (size_t)AttnLds<64>::kTotal : (size_t)AttnLds<128>::kTotal;
    // Staged input plus the norm weights of hidden-sized inputs.
    const size_t stage = (size_t)(2 * hidden > inter ? 2 * hidden : inter);
    const size_t need = attn > stage ? attn : stage;
    return (need * sizeof(float) + 15) / 16 * 16;
}

size_t decode_step_lds_bytes(uint32_t hidden, uint32_t inter, uint32_t layers, uint32_t hd) {
    return decode_step_table_offset(hidden, inter, hd) + (size_t)(layers * 4 + 1) * sizeof(DecodeGemv) +
           (size_t)layers * 2 * sizeof(const uint16_t*);
}

static const void* decode_step_fn(uint32_t hd) {
    if (hd == 64) return reinterpret_cast<const void*>(&decode_step_kernel<64, true>);
    if (hd == 128) return reinterpret_cast<const void*>(&decode_step_kernel<128, true>);
    if (hd <= 64) return reinterpret_cast<const void*>(&decode_step_kernel<64, false>);
    return reinterpret_cast<const void*>(&decode_step_kernel<128, false>);
}

hipError_t decode_step_max_blocks(uint32_t hd, size_t lds, int* blocks_per_cu) {
    const void* f = decode_step_fn(hd);
    hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, f, kMkThreads, lds);
}

hipError_t launch_decode_step(const DecodeStepParams& p, uint32_t blocks, size_t lds, hipStream_t s) {
    DecodeStepParams copy = p;
    void* args[] = {&copy};
    return hipLaunchCooperativeKernel(decode_step_fn(p.hd), dim3(blocks), dim3(kMkThreads), args, (unsigned)lds, s);
}

}  // namespace vvli
