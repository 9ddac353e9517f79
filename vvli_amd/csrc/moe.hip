// moe.hip -- mixture-of-experts pieces of the token step (OLMoE form).
//
// The reference has no MoE forward pass (its runner rejects such configs,
// src/llm.zig:218-223,426); the semantics follow HF transformers' OLMoE
// (models/olmoe/modeling_olmoe.py, transformers 5.15):
//   qk-norm   q = w_q * (q * 1/sqrt(mean(q^2) + eps)) over the full q, same for
//             k (folded into the decode attention kernel, attention.hip)
//   router    p = softmax(W_r . norm(x)) in f32, the top-k by p (ties: lower
//             expert id), weights p_k without renormalisation
//   experts   act_k = silu(gate_k) * up_k (fused [2I][H] gate|up matrix),
//             out_k = W_down,k . act_k
//   combine   x += sum over the selected experts of (out_k * p_k) (float
//             atomics: the order over experts varies at the ulp level)
// Every step reads the selected experts from device memory, so the token
// step stays one replayable graph with no host round trip.
#include "device_common.hpp"
#include "gemv_tile.hpp"
#include "kernels.hpp"
#include "moe_route.hpp"

namespace vvli {

namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;

__device__ inline float bf(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// Router: logits = W_r . norm(x), one row per wave over ceil(E / 4) blocks;
// the last block to finish (atomic ticket) runs the softmax and top-k on the
// logits (route_block) and resets the ticket.

__global__ __launch_bounds__(kThreads) void moe_router_kernel(MoeRouterArgs a) {
    extern __shared__ float smem[];
    float* xs = smem;                // [H] normalised input
    float* red = smem + a.H;         // [waves]
    __shared__ int last;
    __shared__ unsigned long long route_keys[256];
    __shared__ uint32_t route_rank[256];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Stage (x * w) * s.
    float ss = 0.f;
    for (uint32_t i = tid * 4; i < a.H; i += kThreads * 4) {
        const float4 v = *reinterpret_cast<const float4*>(a.x + i);
        *reinterpret_cast<float4*>(xs + i) = v;
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) total += red[w];
    const float scale = 1.0f / sqrtf(total / static_cast<float>(a.H) + a.eps);
    for (uint32_t i = tid; i < a.H; i += kThreads) xs[i] = xs[i] * bf(a.norm_w[i]) * scale;
    __syncthreads();
    // Rows e = global wave id, stride = all waves of all blocks; sums in LDS.
    __shared__ float row_logit[256];
    const uint32_t gw = blockIdx.x * kWavesPerBlock + wave, nw = gridDim.x * kWavesPerBlock;
    const uint32_t U = a.H / 8;
    for (uint32_t e = gw; e < a.E; e += nw) {
        const uint16_t* row = a.w + static_cast<size_t>(e) * a.H;
        float acc = 0.f;
        for (uint32_t u = lane; u < U; u += 64) {
            const uint4 q = load_unit(row + static_cast<size_t>(u) * 8);
            float wf[8];
            WeightTraits<uint16_t>::expand(q, wf);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc = fmaf(wf[j], xs[u * 8 + j], acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) row_logit[e] = acc;
    }
    __syncthreads();
    // Wave 0 publishes this block's rows, then takes a ticket (its release
    // orders the wave's own stores); the last block routes.
    if (wave == 0) {
        for (uint32_t e = lane; e < a.E; e += 64)
            if ((e % nw) / kWavesPerBlock == blockIdx.x)
                __hip_atomic_store(a.logits + e, row_logit[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0) {
            const uint32_t t = __hip_atomic_fetch_add(a.ticket, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            last = t == gridDim.x - 1;
        }
    }
    __syncthreads();
    if (!last) return;
    // The last block routes (route_block reads the logits from LDS).
    for (uint32_t e = tid; e < a.E; e += kThreads)
        xs[e] = __hip_atomic_load(a.logits + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    route_block<kThreads>(xs, a.E, a.top_k, a.idx, a.weight, route_keys, route_rank);
    if (tid == 0) __hip_atomic_store(a.ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// Down projection of the selected experts, combined into x: wave tiles of
// four rows r..r+3 of one slot's expert; K = I is short (1024 at OLMoE), so
// an item is two 16-byte units per lane per row (the whole row at once);
// lane 0 adds p_slot * (W_down,e . act_slot) for its rows into x with float
// atomics (the order over slots then varies at the ulp level).
constexpr int kDownRows = 4;
constexpr int kDownNJ = 2;

__global__ __launch_bounds__(kThreads) void moe_down_kernel(MoeGemvArgs a, float* __restrict__ x,
                                                           const float* __restrict__ slot_w) {
    extern __shared__ float smem[];
    float* xs = smem;
    const int lane = threadIdx.x & 63;
    const uint32_t wid = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const uint32_t nwaves = gridDim.x * kWavesPerBlock;
    const uint32_t K = a.K, U = K / 8;
    const uint32_t per_item = kDownNJ * kWave;
    const uint32_t nchunk = (U + per_item - 1) / per_item;
    const uint32_t ntiles = a.top_k * a.rows_per_slot / kDownRows;
    // Stage every slot's activations.
    for (uint32_t i = threadIdx.x * 4; i < a.x_len; i += kThreads * 4)
        *reinterpret_cast<float4*>(xs + i) = *reinterpret_cast<const float4*>(a.x + i);
    __syncthreads();
    for (uint32_t tile = wid; tile < ntiles; tile += nwaves) {
        const uint32_t g0 = tile * kDownRows;
        const uint32_t slot = g0 / a.rows_per_slot, r0 = g0 % a.rows_per_slot;
        const uint32_t e = a.experts[slot];
        const uint16_t* base = a.w + (static_cast<size_t>(e) * a.rows_per_slot + r0) * K;
        const float* xsl = xs + static_cast<size_t>(slot) * K;
        float acc[kDownRows] = {0.f, 0.f, 0.f, 0.f};
        for (uint32_t c = 0; c < nchunk; ++c) {
            uint4 buf[kDownRows][kDownNJ];
#pragma unroll
            for (int j = 0; j < kDownNJ; ++j) {
                const uint32_t u = c * per_item + j * kWave + lane;
#pragma unroll
                for (int r = 0; r < kDownRows; ++r)
                    buf[r][j] = u < U ? load_unit(base + static_cast<size_t>(r) * K + static_cast<size_t>(u) * 8)
                                      : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int j = 0; j < kDownNJ; ++j) {
                const uint32_t u = c * per_item + j * kWave + lane;
                if (u >= U) continue;
                float xv[8];
#pragma unroll
                for (int q = 0; q < 8; q += 4) {
                    const float4 t = *reinterpret_cast<const float4*>(xsl + static_cast<size_t>(u) * 8 + q);
                    xv[q] = t.x, xv[q + 1] = t.y, xv[q + 2] = t.z, xv[q + 3] = t.w;
                }
#pragma unroll
                for (int r = 0; r < kDownRows; ++r) {
                    float wf[8];
                    WeightTraits<uint16_t>::expand(buf[r][j], wf);
#pragma unroll
                    for (int q = 0; q < 8; ++q) acc[r] = fmaf(wf[q], xv[q], acc[r]);
                }
            }
        }
        const float pw = slot_w[slot];
#pragma unroll
        for (int r = 0; r < kDownRows; ++r) {
            const float s = wave_sum(acc[r]);
            if (lane == 0) unsafeAtomicAdd(x + r0 + r, __fmul_rn(s, pw));
        }
    }
}

// ---------------------------------------------------------------------------
// Batched (prefill) pieces: the P rows of a chunk are routed together, their
// P * top_k (row, slot) pairs grouped by expert, the experts run as grouped
// GEMMs over their rows (launch_gemm_grouped, prefill.hip) and the outputs
// combined per row in ascending expert id -- the oracle's order, so the
// combine adds exactly what the token step's combine adds.
// ---------------------------------------------------------------------------

// One 512-thread block per row: norm(x_r) staged in LDS, then each wave
// takes four router rows at a time (their loads in flight together: the
// router sits in L2, so a row costs a round trip, not bandwidth), then the
// block's softmax and top-k (route_block).
constexpr int kRouteThreads = 512;

__global__ __launch_bounds__(kRouteThreads) void moe_route_rows_kernel(MoeRouteRowsArgs a) {
    extern __shared__ float smem[];
    float* xs = smem;  // [H]
    __shared__ float row_logit[256];
    __shared__ unsigned long long route_keys[256];
    __shared__ uint32_t route_rank[256];
    constexpr int kWaves = kRouteThreads / 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t r = blockIdx.x;
    const float* x = a.x + static_cast<size_t>(r) * a.H;
    const float scale = a.row_scale[r];
    for (uint32_t i = tid; i < a.H; i += kRouteThreads) xs[i] = x[i] * bf(a.norm_w[i]) * scale;
    __syncthreads();
    const uint32_t U = a.H / 8;
    for (uint32_t e0 = wave * 4; e0 < a.E; e0 += kWaves * 4) {
        const uint16_t* rp[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) rp[q] = a.w + static_cast<size_t>(e0 + q < a.E ? e0 + q : a.E - 1) * a.H;
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        for (uint32_t ub = 0; ub < U; ub += kNJC * 64) {
            uint4 b[4][kNJC];
            issue<uint16_t, 4>(b, rp, ub, U, lane);
            consume<uint16_t, 4>(b, xs, ub, U, lane, acc);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float v = wave_sum(acc[q]);
            if (lane == 0 && e0 + q < a.E) row_logit[e0 + q] = v;
        }
    }
    __syncthreads();
    route_block<kRouteThreads>(row_logit, a.E, a.top_k, a.idx + static_cast<size_t>(r) * a.top_k,
                               a.weight + static_cast<size_t>(r) * a.top_k, route_keys, route_rank);
}

// Counting sort of the n = rows * top_k pairs by expert in one 1024-thread
// block. The expert ids are staged in LDS as bytes; thread (g, e) owns expert
// e in pair range g (G = 1024 / E ranges): it counts, the counts become
// offsets (per expert over ranges, then over experts in id order), and a
// second pass writes the pairs of its range at its offset, so the pairs of an
// expert keep their pair order. Every expert's rows are then cut into tiles
// of tile_rows for the grouped GEMM.
constexpr int kGroupThreads = 1024;
constexpr uint32_t kGroupMaxPairs = 32768;  // 2048 rows x top-16

__global__ __launch_bounds__(kGroupThreads) void moe_group_kernel(const uint32_t* __restrict__ idx, uint32_t n,
                                                                 uint32_t top_k, uint32_t E, uint32_t tile_rows,
                                                                 uint32_t* __restrict__ grouped_rows,
                                                                 uint32_t* __restrict__ pair_pos,
                                                                 uint4* __restrict__ tiles) {
    __shared__ uint8_t ids[kGroupMaxPairs];
    __shared__ uint32_t cnt[kGroupThreads];  // [g][e], then the pair offsets
    __shared__ uint32_t eoff[256], toff[257];
    const uint32_t tid = threadIdx.x;
    for (uint32_t p = tid; p < n; p += kGroupThreads) ids[p] = static_cast<uint8_t>(idx[p]);
    const uint32_t G = kGroupThreads / E;
    const uint32_t g = tid / E, e = tid % E;
    const uint32_t span = (n + G - 1) / G;
    const uint32_t p0 = g * span, p1 = min(n, p0 + span);
    __syncthreads();
    uint32_t c = 0;
    if (g < G)
        for (uint32_t p = p0; p < p1; ++p) c += ids[p] == e;
    cnt[tid] = c;
    __syncthreads();
    if (tid < E) {  // exclusive offsets over the ranges of expert tid
        uint32_t run = 0;
        for (uint32_t gg = 0; gg < G; ++gg) {
            const uint32_t v = cnt[gg * E + tid];
            cnt[gg * E + tid] = run;
            run += v;
        }
        eoff[tid] = run;  // the expert's total, for now
    }
    __syncthreads();
    // Totals -> offsets over experts, tile counts -> tile offsets: inclusive
    // scans over the E entries (Hillis-Steele in LDS), made exclusive below.
    __shared__ uint32_t scan_a[256], scan_b[256];
    if (tid < 256) {
        const uint32_t tot = tid < E ? eoff[tid] : 0u;
        scan_a[tid] = tot;
        scan_b[tid] = (tot + tile_rows - 1) / tile_rows;
    }
    __syncthreads();
    for (uint32_t d = 1; d < 256; d <<= 1) {
        uint32_t va = 0, vb = 0;
        if (tid < 256 && tid >= d) va = scan_a[tid - d], vb = scan_b[tid - d];
        __syncthreads();
        if (tid < 256) scan_a[tid] += va, scan_b[tid] += vb;
        __syncthreads();
    }
    if (tid < E) {
        const uint32_t tot = eoff[tid];
        eoff[tid] = scan_a[tid] - tot;
        toff[tid] = scan_b[tid] - (tot + tile_rows - 1) / tile_rows;
    }
    if (tid == 0) {
        toff[E] = scan_b[E - 1];
        tiles[0] = make_uint4(scan_b[E - 1], 0, 0, 0);
    }
    __syncthreads();
    if (g < G) {
        uint32_t at = eoff[e] + cnt[tid];
        for (uint32_t p = p0; p < p1; ++p)
            if (ids[p] == e) {
                grouped_rows[at] = p / top_k;
                pair_pos[p] = at;
                ++at;
            }
    }
    if (tid < E) {
        const uint32_t b = eoff[tid], end = tid + 1 < E ? eoff[tid + 1] : n;
        uint32_t t = toff[tid];
        for (uint32_t r0 = b; r0 < end; r0 += tile_rows) tiles[1 + t++] = make_uint4(tid, r0, min(end, r0 + tile_rows), 0);
    }
}

// One block per row: its (expert, weight, grouped position) triples sorted
// by expert id in LDS, then x[r][i] += sum_j eout[pos_j][i] * w_j in that
// order (products rounded, then added: the oracle's moe += out * w).
__global__ __launch_bounds__(kThreads) void moe_combine_kernel(const float* __restrict__ eout,
                                                              const uint32_t* __restrict__ pair_pos,
                                                              const uint32_t* __restrict__ idx,
                                                              const float* __restrict__ weight, uint32_t top_k,
                                                              uint32_t H, float* __restrict__ x) {
    __shared__ uint32_t se[kMaxTopK], sp[kMaxTopK];
    __shared__ float sw[kMaxTopK];
    const uint32_t r = blockIdx.x;
    if (threadIdx.x == 0) {
        for (uint32_t j = 0; j < top_k; ++j) {  // insertion sort by expert id (ids of a row are distinct)
            const size_t p = static_cast<size_t>(r) * top_k + j;
            const uint32_t ej = idx[p], pj = pair_pos[p];
            const float wj = weight[p];
            uint32_t k = j;
            while (k > 0 && se[k - 1] > ej) {
                se[k] = se[k - 1], sp[k] = sp[k - 1], sw[k] = sw[k - 1];
                --k;
            }
            se[k] = ej, sp[k] = pj, sw[k] = wj;
        }
    }
    __syncthreads();
    float* xr = x + static_cast<size_t>(r) * H;
    for (uint32_t i = threadIdx.x; i < H; i += kThreads) {
        float v[kMaxTopK];  // every slot's load in flight before the ordered sum
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j)
            v[j] = j < static_cast<int>(top_k) ? eout[static_cast<size_t>(sp[j]) * H + i] : 0.f;
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j)
            if (j < static_cast<int>(top_k)) acc = __fadd_rn(acc, __fmul_rn(v[j], sw[j]));
        xr[i] = __fadd_rn(xr[i], acc);
    }
}

}  // namespace

hipError_t launch_moe_route_rows(const MoeRouteRowsArgs& a, hipStream_t s) {
    if (a.rows == 0) return hipSuccess;
    if (a.E == 0 || a.E > 256 || a.top_k == 0 || a.top_k > a.E || a.top_k > static_cast<uint32_t>(kMaxTopK) ||
        a.H % 8 != 0 || a.H > 16384 || !a.row_scale)
        return hipErrorInvalidValue;
    return vlaunch(moe_route_rows_kernel, dim3(a.rows), dim3(kRouteThreads), static_cast<size_t>(a.H) * sizeof(float),
                   s, a);
}

hipError_t launch_moe_group(const uint32_t* idx, uint32_t rows, uint32_t top_k, uint32_t E, uint32_t tile_rows,
                            uint32_t* grouped_rows, uint32_t* pair_pos, uint4* tiles, hipStream_t s) {
    const size_t n = static_cast<size_t>(rows) * top_k;
    if (n == 0 || n > kGroupMaxPairs || E == 0 || E > 256 || tile_rows == 0) return hipErrorInvalidValue;
    return vlaunch(moe_group_kernel, dim3(1), dim3(kGroupThreads), 0, s, idx, static_cast<uint32_t>(n), top_k, E,
                   tile_rows, grouped_rows, pair_pos, tiles);
}

hipError_t launch_moe_combine(const float* eout, const uint32_t* pair_pos, const uint32_t* idx, const float* weight,
                              uint32_t rows, uint32_t top_k, uint32_t H, float* x, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    if (top_k == 0 || top_k > static_cast<uint32_t>(kMaxTopK)) return hipErrorInvalidValue;
    return vlaunch(moe_combine_kernel, dim3(rows), dim3(kThreads), 0, s, eout, pair_pos, idx, weight, top_k, H, x);
}

hipError_t moe_gemv_init_attributes() {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&moe_gemv_kernel<kGemvGateUp>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&moe_down_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    // The router kernel also has static LDS: its dynamic part (the hidden
    // vector) is capped at 64 KiB, hidden <= 16384.
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(&moe_router_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024);
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&moe_route_rows_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024);
}

hipError_t launch_moe_gemv(int mode, const MoeGemvArgs& a, hipStream_t s) {
    if (a.K % 8 != 0 || a.x_len % 4 != 0 || (mode != kGemvGateUp && a.rows_per_slot % 2 != 0))
        return hipErrorInvalidValue;
    const uint32_t R = mode == kGemvGateUp ? 1 : 2;
    const uint32_t tiles = (a.top_k * a.rows_per_slot + R - 1) / R;
    uint32_t blocks = (tiles + kWavesPerBlock - 1) / kWavesPerBlock;
    if (blocks > 1024) blocks = 1024;
    const size_t lds = (static_cast<size_t>(a.x_len) + kWavesPerBlock) * sizeof(float);
    if (mode != kGemvGateUp) return hipErrorInvalidValue;
    return vlaunch(moe_gemv_kernel<kGemvGateUp>, dim3(blocks), dim3(kThreads), lds, s, a);
}

hipError_t launch_moe_router(const MoeRouterArgs& a, hipStream_t s) {
    if (a.E == 0 || a.E > 256 || a.top_k == 0 || a.top_k > a.E || a.top_k > static_cast<uint32_t>(kMaxTopK) ||
        a.H % 8 != 0 || a.H > 16384 - kWavesPerBlock)
        return hipErrorInvalidValue;
    const size_t lds = (static_cast<size_t>(a.H) + kWavesPerBlock) * sizeof(float);
    return vlaunch(moe_router_kernel, dim3((a.E + kWavesPerBlock - 1) / kWavesPerBlock), dim3(kThreads), lds, s, a);
}

hipError_t launch_moe_down(const MoeGemvArgs& a, float* x, const float* slot_w, hipStream_t s) {
    if (a.K % 8 != 0 || a.x_len % 4 != 0 || a.rows_per_slot % kDownRows != 0) return hipErrorInvalidValue;
    const uint32_t tiles = a.top_k * a.rows_per_slot / kDownRows;
    uint32_t blocks = (tiles + kWavesPerBlock - 1) / kWavesPerBlock;
    if (blocks > 1024) blocks = 1024;
    const size_t lds = static_cast<size_t>(a.x_len) * sizeof(float);
    return vlaunch(moe_down_kernel, dim3(blocks), dim3(kThreads), lds, s, a, x, slot_w);
}

}  // namespace vvli
