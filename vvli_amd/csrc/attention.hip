// attention.hip -- batch-1 GQA decode attention over the f32 KV cache.
//
// Reference: Runner.forwardLayer (src/llm.zig:742-755) -> applyRoPE on q and
// k (:1337-1371), K/V append at `pos` (:744-745), computeAttentionInto
// (:1302-1335): per q head, s_t = (q.K_t)/sqrt(hd) for t <= pos, softmax,
// out = sum_t p_t V_t.
//
// Design: grid = (nsplit, kv_heads). Block (s, h) takes a contiguous range of
// positions of kv head h for all `group` q heads that share it (GQA), walks
// it in LDS tiles with an online softmax, and writes (m, l, acc) partials.
// The block whose range holds `pos` rotates the new k, appends k/v to the
// cache and uses them straight from LDS. The last block of each kv head
// (atomic ticket) merges the partials. The position is read from device
// memory, so the launch can be replayed from a graph.
#include "device_common.hpp"
#include "kernels.hpp"

namespace vvli {

namespace {

constexpr int kThreads = 256;
constexpr int kMaxGroup = 16;
constexpr int kMaxSplit = 64;

__device__ inline void rope_pair(const float* src, float* dst, int first, int second, float c, float s) {
    // rotatePair, src/llm.zig:1360-1371 (kept unfused: x0*c - x1*s, x0*s + x1*c)
    const float x0 = src[first], x1 = src[second];
    dst[first] = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, s));
    dst[second] = __fadd_rn(__fmul_rn(x0, s), __fmul_rn(x1, c));
}

__device__ inline float bf16_to_f32_dev(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

__device__ inline float ld_agent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline void pair_index(uint32_t layout, int i, int hd, int& first, int& second) {
    if (layout == 0) {  // interleaved: (2i, 2i+1)
        first = 2 * i;
        second = 2 * i + 1;
    } else {  // split_half: (i, i + hd/2)
        first = i;
        second = i + hd / 2;
    }
}

template <int HDMAX>
__global__ __launch_bounds__(kThreads) void attn_decode_kernel(AttnArgs a) {
    constexpr int TILE = 4096 / HDMAX;                      // 64 rows at hd 64, 32 at hd 128
    constexpr int NP = (kMaxGroup * HDMAX + kThreads - 1) / kThreads;  // (g,d) pairs per thread

    __shared__ float qs[kMaxGroup][HDMAX];
    __shared__ float ks[TILE][HDMAX + 1];
    __shared__ float vs[TILE][HDMAX];
    __shared__ float ps[kMaxGroup][TILE];
    __shared__ float knew[HDMAX], vnew[HDMAX];
    __shared__ float m_s[kMaxGroup], l_s[kMaxGroup], c_s[kMaxGroup];
    __shared__ float wsplit[kMaxSplit][kMaxGroup];  // combine weights exp(m_s - M) / L
    __shared__ int last_flag;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int hd = (int)a.hd;
    const int half = hd / 2;
    const uint32_t h = blockIdx.y;
    const uint32_t s = blockIdx.x;
    const int G = (int)(a.heads / a.kv_heads);
    const uint32_t kvw = a.kv_heads * a.hd;
    const uint32_t pos = *a.pos;
    const uint32_t T = pos + 1;
    uint32_t chunk = (T + a.nsplit - 1) / a.nsplit;
    if (chunk < static_cast<uint32_t>(TILE)) chunk = TILE;  // one LDS tile per split at least
    const uint32_t t0 = s * chunk;
    const uint32_t t1 = min(t0 + chunk, T);
    const float* cs = a.rope_cs + (size_t)pos * hd;  // [hd/2][2]

    if (t0 < t1) {
        const bool owns_pos = pos >= t0 && pos < t1;
        const float* qsrc = a.q + (size_t)h * G * hd;
        const float* ksrc = a.k_new + (size_t)h * hd;
        if (a.q_norm) {
            // QK-norm over the full q and the full k (HF OLMoE:
            // w * (x * 1/sqrt(mean(x^2) + eps))), then RoPE from LDS.
            float sq = 0.f, sk = 0.f;
            for (uint32_t i = tid; i < a.heads * a.hd; i += kThreads) sq = fmaf(a.q[i], a.q[i], sq);
            for (uint32_t i = tid; i < kvw; i += kThreads) sk = fmaf(a.k_new[i], a.k_new[i], sk);
            sq = wave_sum(sq);
            sk = wave_sum(sk);
            if (lane == 0) {
                wsplit[0][wave] = sq;
                wsplit[1][wave] = sk;
            }
            __syncthreads();
            float tq = 0.f, tk = 0.f;
            for (int w = 0; w < kThreads / kWave; ++w) tq += wsplit[0][w], tk += wsplit[1][w];
            const float scq = 1.0f / sqrtf(tq / (float)(a.heads * a.hd) + a.norm_eps);
            const float sck = 1.0f / sqrtf(tk / (float)kvw + a.norm_eps);
            for (int idx = tid; idx < G * hd; idx += kThreads) {
                const int g = idx / hd, d = idx - g * hd;
                const uint32_t qi = (h * G + g) * hd + d;
                qs[g][d] = bf16_to_f32_dev(a.q_norm[qi]) * (a.q[qi] * scq);
            }
            if (owns_pos)
                for (int d = tid; d < hd; d += kThreads)
                    knew[d] = bf16_to_f32_dev(a.k_norm[h * hd + d]) * (ksrc[d] * sck);
            __syncthreads();
            qsrc = nullptr;
        }
        // RoPE'd q for the group's heads.
        for (int idx = tid; idx < G * half; idx += kThreads) {
            const int g = idx / half, i = idx - g * half;
            int f, sc;
            pair_index(a.rope_layout, i, hd, f, sc);
            rope_pair(qsrc ? qsrc + (size_t)g * hd : qs[g], qs[g], f, sc, cs[2 * i], cs[2 * i + 1]);
        }
        if (owns_pos) {
            for (int i = tid; i < half; i += kThreads) {
                int f, sc;
                pair_index(a.rope_layout, i, hd, f, sc);
                rope_pair(a.q_norm ? knew : ksrc, knew, f, sc, cs[2 * i], cs[2 * i + 1]);
            }
            for (int d = tid; d < hd; d += kThreads) vnew[d] = a.v_new[(size_t)h * hd + d];
        }
        if (tid < kMaxGroup) {
            m_s[tid] = -INFINITY;
            l_s[tid] = 0.f;
        }
        __syncthreads();
        if (owns_pos) {
            float* kd = a.kcache + (size_t)pos * kvw + (size_t)h * hd;
            float* vd = a.vcache + (size_t)pos * kvw + (size_t)h * hd;
            for (int d = tid; d < hd; d += kThreads) {
                kd[d] = knew[d];
                vd[d] = vnew[d];
            }
        }

        float acc[NP];
#pragma unroll
        for (int i = 0; i < NP; ++i) acc[i] = 0.f;

        for (uint32_t ta = t0; ta < t1; ta += TILE) {
            const int tlen = (int)min((uint32_t)TILE, t1 - ta);
            // Stage K/V rows of this kv head (row `pos` comes from LDS).
            const int vec_per_row = hd / 4;
            for (int idx = tid; idx < tlen * vec_per_row; idx += kThreads) {
                const int j = idx / vec_per_row, c4 = (idx - j * vec_per_row) * 4;
                const uint32_t t = ta + j;
                float4 kv4, vv4;
                if (t == pos) {
                    kv4 = make_float4(knew[c4], knew[c4 + 1], knew[c4 + 2], knew[c4 + 3]);
                    vv4 = make_float4(vnew[c4], vnew[c4 + 1], vnew[c4 + 2], vnew[c4 + 3]);
                } else {
                    const size_t off = (size_t)t * kvw + (size_t)h * hd + c4;
                    kv4 = *reinterpret_cast<const float4*>(a.kcache + off);
                    vv4 = *reinterpret_cast<const float4*>(a.vcache + off);
                }
                ks[j][c4] = kv4.x;
                ks[j][c4 + 1] = kv4.y;
                ks[j][c4 + 2] = kv4.z;
                ks[j][c4 + 3] = kv4.w;
                *reinterpret_cast<float4*>(&vs[j][c4]) = vv4;
            }
            __syncthreads();
            // Scores s[g][j] = (q_g . K_j) * scale; QP threads per (g, j) pair
            // (adjacent lanes) each take hd / QP dimensions, summed by xor shuffles.
            {
                const int pairs = G * TILE;
                int QP = kThreads / pairs;
                QP = QP >= 16 ? 16 : QP >= 8 ? 8 : QP >= 4 ? 4 : QP >= 2 ? 2 : 1;
                while (QP > 1 && hd % QP != 0) QP >>= 1;
                const int dpart = hd / QP;
                for (int base = 0; base < pairs * QP; base += kThreads) {
                    const int idx = base + tid;
                    const int pr = idx / QP, qp = idx - pr * QP;
                    const int g = pr / TILE, j = pr - g * TILE;
                    float d0 = 0.f;
                    if (pr < pairs && j < tlen) {
                        const int d0i = qp * dpart;
                        for (int d = d0i; d < d0i + dpart; ++d) d0 = fmaf(qs[g][d], ks[j][d], d0);
                    }
                    for (int off = 1; off < QP; off <<= 1) d0 += __shfl_xor(d0, off, kWave);
                    if (pr < pairs && qp == 0) ps[g][j] = j < tlen ? d0 * a.scale : -INFINITY;
                }
            }
            __syncthreads();
            // Online softmax update, one wave per q head.
            for (int g = wave; g < G; g += kThreads / kWave) {
                const float sc = lane < TILE ? ps[g][lane] : -INFINITY;
                const float m_old = m_s[g];
                const float m_new = fmaxf(m_old, wave_max(sc));
                const float corr = expf(m_old - m_new);
                const float e = lane < tlen ? expf(sc - m_new) : 0.f;
                if (lane < TILE) ps[g][lane] = e;
                const float lsum = wave_sum(e);
                if (lane == 0) {
                    l_s[g] = l_s[g] * corr + lsum;
                    m_s[g] = m_new;
                    c_s[g] = corr;
                }
            }
            __syncthreads();
            // acc[g][d] = acc * corr + sum_j p[g][j] V[j][d]
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int idx = tid + i * kThreads;
                if (idx < G * hd) {
                    const int g = idx / hd, d = idx - g * hd;
                    float v = acc[i] * c_s[g];
                    for (int j = 0; j < tlen; ++j) v = fmaf(ps[g][j], vs[j][d], v);
                    acc[i] = v;
                }
            }
            __syncthreads();
        }
        // Partials: [h][s][g][2 + hd] = (m, l, acc[hd]). Agent-scope stores
        // write through to the coherence point, so the merging block (on any
        // XCD) reads them without an L2 writeback/invalidate.
        const size_t stride = (size_t)2 + hd;
        float* pbase = a.part + ((size_t)h * a.nsplit + s) * G * stride;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const int idx = tid + i * kThreads;
            if (idx < G * hd) {
                const int g = idx / hd, d = idx - g * hd;
                __hip_atomic_store(pbase + g * stride + 2 + d, acc[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        if (tid < G) {
            __hip_atomic_store(pbase + tid * stride, m_s[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pbase + tid * stride + 1, l_s[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // Ticket among the non-empty splits: the last one to finish merges. Every
    // thread waits for its partial stores to complete before the ticket.
    const uint32_t ns = min(a.nsplit, (T + chunk - 1) / chunk);
    if (t0 >= t1) return;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&a.counters[h], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_flag = prev == ns - 1;
    }
    __syncthreads();
    if (!last_flag) return;
    const size_t stride = (size_t)2 + hd;
    const float* hbase = a.part + (size_t)h * a.nsplit * G * stride;
    // Split weights: w[s][g] = exp(m_s - M) / sum_s' l_s' exp(m_s' - M).
    for (int g = wave; g < G; g += kThreads / kWave) {
        float mv = -INFINITY, lv = 0.f;
        if ((uint32_t)lane < ns) {
            mv = __hip_atomic_load(hbase + (lane * G + g) * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            lv = __hip_atomic_load(hbase + (lane * G + g) * stride + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const float M = wave_max(mv);
        const float e = (uint32_t)lane < ns ? expf(mv - M) : 0.f;
        const float L = wave_sum(lv * e);
        if ((uint32_t)lane < ns) wsplit[lane][g] = e / L;
    }
    __syncthreads();
    for (int idx = tid; idx < G * hd; idx += kThreads) {
        const int g = idx / hd, d = idx - g * hd;
        const float* p = hbase + (size_t)g * stride + 2 + d;
        float o = 0.f;
        uint32_t sp = 0;
        for (; sp + 4 <= ns; sp += 4) {
            const float a0 = ld_agent(p + (size_t)(sp + 0) * G * stride), a1 = ld_agent(p + (size_t)(sp + 1) * G * stride);
            const float a2 = ld_agent(p + (size_t)(sp + 2) * G * stride), a3 = ld_agent(p + (size_t)(sp + 3) * G * stride);
            o = fmaf(a0, wsplit[sp][g], o);
            o = fmaf(a1, wsplit[sp + 1][g], o);
            o = fmaf(a2, wsplit[sp + 2][g], o);
            o = fmaf(a3, wsplit[sp + 3][g], o);
        }
        for (; sp < ns; ++sp) o = fmaf(ld_agent(p + (size_t)sp * G * stride), wsplit[sp][g], o);
        a.out[(size_t)(h * G + g) * hd + d] = o;
    }
    if (tid == 0) __hip_atomic_store(&a.counters[h], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

uint32_t attn_nsplit(uint32_t max_seq, uint32_t hd) {
    const uint32_t tile = hd <= 64 ? 64u : 32u;  // TILE of the kernel instance
    const uint32_t n = (max_seq + tile - 1) / tile;
    return n < 1 ? 1 : (n > (uint32_t)kMaxSplit ? (uint32_t)kMaxSplit : n);
}

size_t attn_part_floats(uint32_t heads, uint32_t kv_heads, uint32_t hd, uint32_t nsplit) {
    return (size_t)kv_heads * nsplit * (heads / kv_heads) * (2 + hd);
}

hipError_t launch_attn_decode(const AttnArgs& a, hipStream_t s) {
    dim3 grid(a.nsplit, a.kv_heads);
    if (a.hd <= 64) return vlaunch(attn_decode_kernel<64>, grid, dim3(kThreads), 0, s, a);
    return vlaunch(attn_decode_kernel<128>, grid, dim3(kThreads), 0, s, a);
}

}  // namespace vvli
