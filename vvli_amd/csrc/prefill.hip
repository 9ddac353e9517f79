// prefill.hip -- batched prompt processing: the P prompt tokens of a chunk go
// through each layer together instead of one token step at a time.
//
// Reference semantics: the prefill loop of generator.zig (src/generator.zig:
// 243-251) forwards the prompt token by token (Runner.forwardToken,
// src/llm.zig:702-766); what it leaves behind is the KV cache rows of every
// prompt position and the logits of the last one. This file computes the same
// rows and logits with matrix products over all P tokens:
//
//   X = embed(tokens)                                    [P][H] f32
//   per layer:
//     s_r   = 1 / sqrt(mean(X_r^2) + eps)                row_rms_kernel
//     QKV   = ((X * w_in) * s) . [Wq|Wk|Wv]^T + bias     gemm (A-prologue norm)
//     rotate q, k (RoPE at each row's position); append k, v to the cache
//     A     = causal GQA attention over cache rows 0..pos  prefill_attn_kernel
//     X    += A . Wo^T                                   gemm (residual epilogue)
//     s_r   = RMS of X rows
//     F     = silu((X*w_post*s) . Wg^T) * ((X*w_post*s) . Wu^T)   gemm (gate/up)
//     X    += F . Wd^T                                   gemm (residual epilogue)
//   last row of X -> final norm, logits, argmax (the decode step's kernels)
//
// GEMM on MFMA (v_mfma_f32_16x16x32_bf16). Weights are bf16; activations are
// f32 and are split into hi = bf16(a) and lo = bf16(a - hi), so that
// a . w = hi . w + lo . w holds to about 2^-16 relative per product (bf16
// weights are exact in both): two MFMAs per product keep the f32 activation
// precision the reference computes with, where one bf16 rounding of the
// activations would cost about 2^-9.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "device_common.hpp"
#include "kernels.hpp"

namespace vvli {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// GEMM tile: 128 (rows of A) x 256 (rows of W) x 32 (K) per step, 512
// threads as 2 x 4 waves of 64 x 64, each wave 4 x 4 MFMA tiles of 16 x 16.
// v_mfma_f32_16x16x32_bf16 lane layout (lane l): A row l%16, k 8*(l/16)..+7;
// B column l%16, same k; D rows 4*(l/16)+j (j = 0..3), column l%16.
//
// Operands reach LDS by global_load_lds_dwordx4 (no registers in between):
// 4 stages of [A hi 8 KiB | A lo 8 KiB | W 16 KiB], three K steps in flight.
// An LDS row is 32 bf16 (64 bytes, four 16-byte chunks); chunk c of row r is
// stored at position c ^ swz(r). ds_read_b128 serves a wave in four passes of
// 16 lanes (lanes 0-7 with 24-31, 8-15 with 16-23, the same in the upper
// half) over 64 four-byte banks; with swz(r) = (r >> 1) & 3 the 16 fragment
// rows of each pass fall on 16 distinct 16-byte bank groups (no conflict
// cycles in SQ_LDS_BANK_CONFLICT). MFMA fragments
// are read with ds_read_b128 in inline asm and waited for explicitly, so the
// compiler does not tie them to the copies in flight.
// ---------------------------------------------------------------------------
constexpr int kGemmThreads = 512;
constexpr int kBM = 128, kBN = 256, kBK = 32, kStages = 4;
constexpr int kOpA = kBM * kBK * 2;                  // bytes of one A plane tile
constexpr int kStageBytes = 2 * kOpA + kBN * kBK * 2;
constexpr int kDmaPerWave = kStageBytes / 1024 / (kGemmThreads / 64);  // 1 KiB copies per wave per stage
constexpr int kGemmLds = kStages * kStageBytes;

__device__ inline uint16_t to_bf16_rne(float v) {
    uint32_t b = __float_as_uint(v);
    return static_cast<uint16_t>((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}
__device__ inline float from_bf16(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// Row stride of the split A planes (gemm_kp, kernels.hpp): K rounded up to
// whole K steps, the tail zero-filled by gemm_split_kernel.
static_assert(kBK == 32, "gemm_kp rounds to 32");

// Row of W feeding B-tile row r of block column n0 (GateUp interleaves gate and
// up rows in groups of 16 so one lane holds both halves of an output).
// eoff: element offset of the expert's matrix (grouped launches; else 0).
template <int MODE>
__device__ inline const uint16_t* gemm_w_row(const GemmArgs& g, uint32_t n0, int r, size_t eoff, bool& valid) {
    if (MODE == kGemmGateUp) {
        const uint32_t n = n0 / 2 + (r / 32) * 16 + (r % 16);
        valid = n < g.N;
        return ((r / 16) & 1 ? g.w_up : g.w[0]) + eoff + static_cast<size_t>(valid ? n : 0) * g.K;
    }
    const uint32_t n = n0 + r;
    valid = n < g.N;
    const uint32_t nn = valid ? n : 0;
    if (nn < g.seg_end[0]) return g.w[0] + eoff + static_cast<size_t>(nn) * g.K;
    if (nn < g.seg_end[1]) return g.w[1] + eoff + static_cast<size_t>(nn - g.seg_end[0]) * g.K;
    return g.w[2] + eoff + static_cast<size_t>(nn - g.seg_end[1]) * g.K;
}

typedef __attribute__((address_space(3))) void lds_void_t;

// Row `row` of this block's K split in the partial sums ([split][M][N] f32).
__device__ __forceinline__ float* part_row(const GemmArgs& g, uint32_t row) {
    return g.part + (static_cast<size_t>(blockIdx.z) * g.M + row) * g.N;
}

__device__ __forceinline__ uint32_t gemm_swz(uint32_t r) { return (r >> 1) & 3u; }

__device__ __forceinline__ void gemm_dma16(const void* src, char* dst) {
    __builtin_amdgcn_global_load_lds(src, (lds_void_t*)dst, 16, 0, 0);
}
__device__ __forceinline__ uint32_t gemm_lds_addr(char* p) { return (uint32_t)(uintptr_t)(lds_void_t*)p; }
__device__ __forceinline__ void gemm_barrier() { __builtin_amdgcn_s_barrier(); }

// Wait until at most n of this wave's memory loads are in flight (n = 0, 4
// or 8: whole stages of kDmaPerWave copies).
__device__ __forceinline__ void gemm_wait_vm(int n) {
    constexpr int kKeep = (7 << 4) | (15 << 8);  // expcnt, lgkmcnt: no wait
    if (n >= 12) __builtin_amdgcn_s_waitcnt(12 | kKeep);
    else if (n >= 8) __builtin_amdgcn_s_waitcnt(8 | kKeep);
    else if (n >= 4) __builtin_amdgcn_s_waitcnt(4 | kKeep);
    else __builtin_amdgcn_s_waitcnt(0 | kKeep);
}
static_assert(kDmaPerWave == 4, "gemm_wait_vm counts in stages of 4 copies");

__device__ __forceinline__ bf16x8 gemm_lds_read(uint32_t addr) {
    bf16x8 v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}
// Waits for the fragment reads; the fragments are operands, so nothing that
// uses them can be scheduled before the wait.
__device__ __forceinline__ void gemm_lds_wait(bf16x8 (&a)[4], bf16x8 (&l)[4], bf16x8 (&b)[4]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(l[0]), "+v"(l[1]), "+v"(l[2]), "+v"(l[3]),
                   "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]));
}

// A into hi | lo bf16 planes (a_hl[0][m][kp], a_hl[1][m][kp]) with the
// RMSNorm prologue when norm_w is set: v = (a * w) * scale in rmsNormInto's
// order (src/llm.zig:1297), hi = bf16(v), lo = bf16(v - hi); columns K .. kp
// are zeros. 8 columns per thread. With a_rows, row m is gathered from a
// row a_rows[m].
__global__ __launch_bounds__(256) void gemm_split_kernel(GemmArgs g) {
    const uint32_t kp = gemm_kp(g.K);
    const uint32_t groups = kp / 8;
    const size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= static_cast<size_t>(g.M) * groups) return;
    const uint32_t m = static_cast<uint32_t>(i / groups), k = static_cast<uint32_t>(i % groups) * 8;
    u16x8 hi = {0, 0, 0, 0, 0, 0, 0, 0}, lo = hi;
    if (k < g.K) {  // K % 8 == 0: the group is all in or all out
        const uint32_t src = g.a_rows ? g.a_rows[m] : m;
        const float* ap = g.a + static_cast<size_t>(src) * g.lda + k;
        const float4 v0 = *reinterpret_cast<const float4*>(ap);
        const float4 v1 = *reinterpret_cast<const float4*>(ap + 4);
        float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        if (g.norm_w) {
            const u16x8 w = *reinterpret_cast<const u16x8*>(g.norm_w + k);
            const float scale = g.row_scale[src];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = __fmul_rn(__fmul_rn(v[j], from_bf16(w[j])), scale);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint16_t h = to_bf16_rne(v[j]);
            hi[j] = h;
            lo[j] = to_bf16_rne(v[j] - from_bf16(h));
        }
    }
    uint16_t* out = g.a_hl + static_cast<size_t>(m) * kp + k;
    *reinterpret_cast<u16x8*>(out) = hi;
    *reinterpret_cast<u16x8*>(out + (g.a_plane ? g.a_plane : static_cast<size_t>(g.M) * kp)) = lo;
}

__device__ inline float silu_mul(float gv, float uv) {
    return __fmul_rn(__fdiv_rn(gv, __fadd_rn(1.0f, expf(-gv))), uv);  // siluMulInto, src/llm.zig:1382-1387
}

// GROUPED: the block's rows and expert come from the tile table (block b:
// tile b / tn, column tile b % tn); 16-row groups past the tile's end skip
// their MFMAs (their copies still run, reading the tile's first row, so
// every wave issues the same copies per stage).
template <int MODE, bool GROUPED = false>
__global__ __launch_bounds__(kGemmThreads) void gemm_bf16_kernel(GemmArgs g) {
    extern __shared__ __attribute__((aligned(1024))) char gemm_smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    const uint32_t cols = MODE == kGemmGateUp ? 2 * g.N : g.N;
    const uint32_t tn = (cols + kBN - 1) / kBN;
    uint32_t m0, n0, mlim;
    size_t eoff = 0;
    if (GROUPED) {
        const uint32_t t = blockIdx.x / tn;
        if (t >= g.tiles[0].x) return;  // uniform per block
        const uint4 td = g.tiles[1 + t];
        m0 = td.y, mlim = td.z;
        n0 = (blockIdx.x % tn) * kBN;
        eoff = static_cast<size_t>(td.x) * g.w_expert;
    } else {
        // Tile of this block. Consecutive blocks go to the 8 XCDs in turn and each
        // XCD has its own L2: block b is mapped to tile u = offset(xcd) + b / 8, so
        // every XCD walks a contiguous run of tiles, ordered in panels of 8 W
        // columns (M fastest inside a panel): the blocks an XCD runs together
        // cover about 8 x 8 tiles and share their A and W slabs through its L2.
        const uint32_t tm = (g.M + kBM - 1) / kBM;
        const uint32_t ntile = gridDim.x;
        const uint32_t xcd = blockIdx.x % 8, per = ntile / 8, rem = ntile % 8;
        const uint32_t u = xcd * per + min(xcd, rem) + blockIdx.x / 8;
        const uint32_t panel = u / (tm * 8), pw = min(8u, tn - 8 * panel), within = u - panel * tm * 8;
        m0 = (within / pw) * kBM;
        n0 = (8 * panel + within % pw) * kBN;
        mlim = g.M;
    }
    // Live 16-row groups of this wave (grouped tiles only).
    bool live[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        live[i] = !GROUPED || m0 + static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(wm)) * 64 + i * 16 < mlim;
    // Split K across gridDim.z blocks (partial sums added atomically).
    const uint32_t nk_all = (g.K + kBK - 1) / kBK;
    const uint32_t per_split = (nk_all + gridDim.z - 1) / gridDim.z;
    const uint32_t kt0 = blockIdx.z * per_split;
    const int nk = kt0 < nk_all ? static_cast<int>(min(per_split, nk_all - kt0)) : 0;
    const bool split = gridDim.z > 1;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (nk == 0) return;  // empty split (uniform per block)

    // Copies: wave w issues 1 KiB copies q = 4w .. 4w+3 of a stage: q < 8 A hi
    // rows 16q.., q < 16 A lo rows 16(q-8).., else W rows 16(q-16)..; lane l
    // fetches row 16 (q % 8 or q - 16) + l/4, chunk (l & 3) ^ swz(row), which
    // lands at position l & 3 of that row. A rows past M read row 0 and W rows
    // past N read row 0 (their outputs are never written); past K, A reads its
    // zero tail and W reads 8 zeros of that tail (only when K % 32 != 0).
    const uint32_t kp = gemm_kp(g.K);
    const uint16_t* zeros = g.a_hl + (kp - 8);
    const uint16_t* src[kDmaPerWave];
    uint32_t chunk[kDmaPerWave];
    bool is_w[kDmaPerWave];
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i) {
        const int q = wave * kDmaPerWave + i;
        const int grp = q < 16 ? q % 8 : q - 16;
        const uint32_t row = grp * 16 + lane / 4;
        chunk[i] = (static_cast<uint32_t>(lane & 3) ^ gemm_swz(row)) * 8;
        is_w[i] = q >= 16;
        if (q < 16) {
            const uint32_t gm = m0 + row < mlim ? m0 + row : (GROUPED ? m0 : 0);
            const size_t plane = g.a_plane ? g.a_plane : static_cast<size_t>(g.M) * kp;
            src[i] = g.a_hl + (q >= 8 ? plane : 0) + static_cast<size_t>(gm) * kp;
        } else {
            bool valid;
            src[i] = gemm_w_row<MODE>(g, n0, static_cast<int>(row), eoff, valid);
        }
    }
    auto issue_one = [&](int kt, int stage, int i) {
        const uint32_t k = (kt0 + kt) * kBK + chunk[i];
        const uint16_t* p = (is_w[i] && k >= g.K) ? zeros : src[i] + k;
        gemm_dma16(p, gemm_smem + stage * kStageBytes + (wave * kDmaPerWave + i) * 1024);
    };
    auto issue = [&](int kt, int stage) {
#pragma unroll
        for (int i = 0; i < kDmaPerWave; ++i) issue_one(kt, stage, i);
    };
    // Fragment addresses within a stage.
    const uint32_t lds0 = gemm_lds_addr(gemm_smem);
    uint32_t fa[4], fb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t ra = wm * 64 + i * 16 + (lane & 15), rb = wn * 64 + i * 16 + (lane & 15);
        const uint32_t qk = static_cast<uint32_t>(lane) >> 4;
        fa[i] = lds0 + ra * 64 + ((qk ^ gemm_swz(ra)) << 4);
        fb[i] = lds0 + 2 * kOpA + rb * 64 + ((qk ^ gemm_swz(rb)) << 4);
    }
    bf16x8 fh[2][4], fl[2][4], fw[2][4];
    auto read_frags = [&](int kt, bf16x8 (&a)[4], bf16x8 (&l)[4], bf16x8 (&w)[4]) {
        const uint32_t so = static_cast<uint32_t>(kt % kStages) * kStageBytes;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[i] = gemm_lds_read(fa[i] + so);
            l[i] = gemm_lds_read(fa[i] + so + kOpA);
            w[i] = gemm_lds_read(fb[i] + so);
        }
    };
    // Prologue: stages 0 .. kStages-2 in flight, step 0's fragments read.
    for (int s0 = 0; s0 < kStages - 1; ++s0)
        if (s0 < nk) issue(s0, s0);
    gemm_wait_vm(min(kStages - 2, nk - 1) * kDmaPerWave);
    gemm_barrier();
    read_frags(0, fh[0], fl[0], fw[0]);
    gemm_lds_wait(fh[0], fl[0], fw[0]);
    // Step kt: once stage kt+1 is in LDS for every wave (and every wave has
    // read stage kt-1's fragments), refill stage kt-1 with step kt+3, read
    // step kt+1's fragments and multiply step kt's.
    // The copies and fragment reads are spread between four groups of 8 MFMAs
    // (hi products of A rows 0-31, 32-63, then the lo products) so that every
    // wave keeps the MFMA pipe fed while it issues them; sched_barrier keeps
    // the compiler from regrouping them.
    auto step = [&](int kt, int cur) {
        if (kt + 1 < nk) gemm_wait_vm(min(kStages - 3, nk - 2 - kt) * kDmaPerWave);
        gemm_barrier();
        const bool more = kt + kStages - 1 < nk, next = kt + 1 < nk;
        const int kn = kt + kStages - 1;
        const uint32_t so = static_cast<uint32_t>((kt + 1) % kStages) * kStageBytes;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma unroll
            for (int i = (q & 1) * 2; i < (q & 1) * 2 + 2; ++i) {
                if (!live[i]) continue;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(q < 2 ? fh[cur][i] : fl[cur][i], fw[cur][j],
                                                                        acc[i][j], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (more) issue_one(kn, kn % kStages, q);
            if (next) {
                fh[cur ^ 1][q] = gemm_lds_read(fa[q] + so);
                fl[cur ^ 1][q] = gemm_lds_read(fa[q] + so + kOpA);
                fw[cur ^ 1][q] = gemm_lds_read(fb[q] + so);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (next) gemm_lds_wait(fh[cur ^ 1], fl[cur ^ 1], fw[cur ^ 1]);
    };
    for (int kt = 0; kt < nk; kt += 2) {
        step(kt, 0);
        if (kt + 1 < nk) step(kt + 1, 1);
    }

    // Epilogue.
    const int fr = lane & 15;
    const int rq = 4 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int jr = 0; jr < 4; ++jr) {
            const uint32_t row = m0 + wm * 64 + i * 16 + rq + jr;
            if (row >= mlim) continue;
            float* orow = g.out + static_cast<size_t>(row) * g.ldo;
            if (MODE == kGemmGateUp) {
#pragma unroll
                for (int j = 0; j < 4; j += 2) {
                    const uint32_t n = n0 / 2 + (wn * 2 + j / 2) * 16 + fr;
                    if (split) {  // partial gate and up sums; gemm_swiglu_kernel finishes
                        if (n < g.N) {
                            float* gu = g.gu_acc + static_cast<size_t>(row) * (2 * g.N) + n;
                            unsafeAtomicAdd(gu, acc[i][j][jr]);
                            unsafeAtomicAdd(gu + g.N, acc[i][j + 1][jr]);
                        }
                    } else if (g.out_hl) {  // split planes of the next GEMM's A, zeros in the tail
                        const uint32_t kpo = gemm_kp(g.N);
                        if (n < kpo) {
                            const float v = n < g.N ? silu_mul(acc[i][j][jr], acc[i][j + 1][jr]) : 0.f;
                            const uint16_t h = to_bf16_rne(v);
                            uint16_t* o = g.out_hl + static_cast<size_t>(row) * kpo + n;
                            o[0] = h;
                            o[g.out_plane] = to_bf16_rne(v - from_bf16(h));
                        }
                    } else if (n < g.N) {
                        orow[n] = silu_mul(acc[i][j][jr], acc[i][j + 1][jr]);
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t n = n0 + wn * 64 + j * 16 + fr;
                    if (n >= g.N) continue;
                    float v = acc[i][j][jr];
                    if (MODE == kGemmResid) {
                        if (split && g.part) part_row(g, row)[n] = v;  // the consumer adds the splits in order
                        else if (split) unsafeAtomicAdd(&orow[n], v);
                        else orow[n] = __fadd_rn(orow[n], v);  // addInto (src/llm.zig:1389-1396)
                    } else {
                        const uint16_t* b = n < g.seg_end[0] ? g.bias[0] : n < g.seg_end[1] ? g.bias[1] : g.bias[2];
                        if (b && blockIdx.z == 0) {
                            const uint32_t bi = n < g.seg_end[0] ? n : n < g.seg_end[1] ? n - g.seg_end[0]
                                                                                        : n - g.seg_end[1];
                            v = __fadd_rn(v, from_bf16(b[bi]));
                        }
                        if (split && g.part) part_row(g, row)[n] = v;
                        else if (split) unsafeAtomicAdd(&orow[n], v);  // output zeroed before the launch
                        else orow[n] = v;
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Row statistics, embedding, RoPE + cache append.
// ---------------------------------------------------------------------------
constexpr int kRowThreads = 256;

// s_r = 1 / sqrt(sum(x^2) / n + eps) for each row (rmsNormInto's scale, src/llm.zig:1292-1293).
// With K-split partial sums of the residual GEMM that produced x (part:
// [splits][rows][n]), x_r is first completed as x_r + p_0 + p_1 + ... in split
// order (addInto per split, src/llm.zig:1389-1396) and written back.
__global__ __launch_bounds__(kRowThreads) void row_rms_kernel(float* __restrict__ x, uint32_t n, uint32_t rows,
                                                             float eps, float* __restrict__ scale,
                                                             const float* __restrict__ part, uint32_t splits) {
    const uint32_t wave = (blockIdx.x * kRowThreads + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (wave >= rows) return;
    float* r = x + static_cast<size_t>(wave) * n;
    float acc = 0.f;
    for (uint32_t i = lane * 4; i < n; i += 256) {
        float4 v = *reinterpret_cast<const float4*>(r + i);
        if (part) {
            for (uint32_t z = 0; z < splits; ++z) {
                const float4 p = *reinterpret_cast<const float4*>(part + (static_cast<size_t>(z) * rows + wave) * n + i);
                v.x = __fadd_rn(v.x, p.x), v.y = __fadd_rn(v.y, p.y), v.z = __fadd_rn(v.z, p.z), v.w = __fadd_rn(v.w, p.w);
            }
            *reinterpret_cast<float4*>(r + i) = v;
        }
        acc = fmaf(v.x, v.x, acc);
        acc = fmaf(v.y, v.y, acc);
        acc = fmaf(v.z, v.z, acc);
        acc = fmaf(v.w, v.w, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) scale[wave] = 1.0f / sqrtf(acc / static_cast<float>(n) + eps);
}

// Up to 8 K-split partial sums of one float4 (stride elements apart), loaded
// together, added onto v in split order.
constexpr uint32_t kMaxPartSplits = 8;
__device__ __forceinline__ float4 add_parts(float4 v, const float* __restrict__ p, size_t stride, uint32_t splits) {
    float4 q[kMaxPartSplits];
#pragma unroll
    for (uint32_t z = 0; z < kMaxPartSplits; ++z)
        q[z] = z < splits ? *reinterpret_cast<const float4*>(p + z * stride) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (uint32_t z = 0; z < kMaxPartSplits; ++z)
        if (z < splits)
            v.x = __fadd_rn(v.x, q[z].x), v.y = __fadd_rn(v.y, q[z].y), v.z = __fadd_rn(v.z, q[z].z),
            v.w = __fadd_rn(v.w, q[z].w);
    return v;
}

// As row_rms_kernel with partial sums (at most kMaxPartSplits), a block per
// row: x_r = x_r + p_0 + p_1 + ... (split order), written back, then the
// row's scale.
__global__ __launch_bounds__(kRowThreads) void row_rms_part_kernel(float* __restrict__ x, uint32_t n, uint32_t rows,
                                                                  float eps, float* __restrict__ scale,
                                                                  const float* __restrict__ part, uint32_t splits) {
    __shared__ float red[kRowThreads / 64];
    const uint32_t row = blockIdx.x;
    float* r = x + static_cast<size_t>(row) * n;
    float acc = 0.f;
    for (uint32_t i = threadIdx.x * 4; i < n; i += kRowThreads * 4) {
        float4 v = add_parts(*reinterpret_cast<const float4*>(r + i), part + static_cast<size_t>(row) * n + i,
                             static_cast<size_t>(rows) * n, splits);
        *reinterpret_cast<float4*>(r + i) = v;
        acc = fmaf(v.x, v.x, acc);
        acc = fmaf(v.y, v.y, acc);
        acc = fmaf(v.z, v.z, acc);
        acc = fmaf(v.w, v.w, acc);
    }
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < kRowThreads / 64; ++w) t += red[w];
        scale[row] = 1.0f / sqrtf(t / static_cast<float>(n) + eps);
    }
}

// Row pass in front of a normalising GEMM, a block per row: complete x_r with
// the K-split partial sums of the GEMM that produced it (split order, written
// back), s_r = 1 / sqrt(mean(x_r^2) + eps), then the GEMM's A planes of
// (x_r * w) * s_r: hi = bf16(a), lo = bf16(a - hi), rows of gemm_kp(n) with a
// zero tail (what launch_row_rms + gemm_split_kernel write, in one pass: the
// row stays in registers). n <= kNormSplitMaxGroups * 8 * kRowThreads.
constexpr int kNormSplitMaxGroups = 4;
__global__ __launch_bounds__(kRowThreads) void row_norm_split_kernel(float* __restrict__ x, uint32_t n, uint32_t rows,
                                                                    float eps, const uint16_t* __restrict__ norm_w,
                                                                    const float* __restrict__ part, uint32_t splits,
                                                                    uint16_t* __restrict__ a_hl, size_t a_plane) {
    __shared__ float red[kRowThreads / 64];
    const uint32_t row = blockIdx.x;
    float* r = x + static_cast<size_t>(row) * n;
    const uint32_t kp = gemm_kp(n), groups = kp / 8;
    float v[kNormSplitMaxGroups][8];
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < kNormSplitMaxGroups; ++q) {
        const uint32_t k = (threadIdx.x + q * kRowThreads) * 8;
        if (k < n) {  // n % 8 == 0: a group is all in or all out
            float4 a = *reinterpret_cast<const float4*>(r + k), b = *reinterpret_cast<const float4*>(r + k + 4);
            if (part && splits > 1) {
                const size_t stride = static_cast<size_t>(rows) * n;
                a = add_parts(a, part + static_cast<size_t>(row) * n + k, stride, splits);
                b = add_parts(b, part + static_cast<size_t>(row) * n + k + 4, stride, splits);
                *reinterpret_cast<float4*>(r + k) = a;
                *reinterpret_cast<float4*>(r + k + 4) = b;
            }
            v[q][0] = a.x, v[q][1] = a.y, v[q][2] = a.z, v[q][3] = a.w;
            v[q][4] = b.x, v[q][5] = b.y, v[q][6] = b.z, v[q][7] = b.w;
#pragma unroll
            for (int j = 0; j < 8; ++j) ss = fmaf(v[q][j], v[q][j], ss);
        }
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kRowThreads / 64; ++w) t += red[w];
    const float scale = 1.0f / sqrtf(t / static_cast<float>(n) + eps);  // rmsNormInto, src/llm.zig:1292-1293
    uint16_t* out = a_hl + static_cast<size_t>(row) * kp;
#pragma unroll
    for (int q = 0; q < kNormSplitMaxGroups; ++q) {
        const uint32_t gi = threadIdx.x + q * kRowThreads, k = gi * 8;
        if (gi >= groups) continue;
        u16x8 hi = {0, 0, 0, 0, 0, 0, 0, 0}, lo = hi;
        if (k < n) {
            const u16x8 w = *reinterpret_cast<const u16x8*>(norm_w + k);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float a = __fmul_rn(__fmul_rn(v[q][j], from_bf16(w[j])), scale);  // x * w * s (:1297)
                const uint16_t h = to_bf16_rne(a);
                hi[j] = h;
                lo[j] = to_bf16_rne(a - from_bf16(h));
            }
        }
        *reinterpret_cast<u16x8*>(out + k) = hi;
        *reinterpret_cast<u16x8*>(out + a_plane + k) = lo;
    }
}

// X[t] = embed[tokens[t]] (copyEmbeddingToken, src/llm.zig:1373-1380).
__global__ __launch_bounds__(kRowThreads) void prefill_embed_kernel(const uint16_t* __restrict__ embed,
                                                                   const uint32_t* __restrict__ tokens, uint32_t n,
                                                                   float* __restrict__ x) {
    const uint32_t t = blockIdx.y;
    const uint32_t i = blockIdx.x * kRowThreads + threadIdx.x;
    if (i >= n) return;
    x[static_cast<size_t>(t) * n + i] = from_bf16(embed[static_cast<size_t>(tokens[t]) * n + i]);
}

// ---------------------------------------------------------------------------
// Packed K/V tile images of the MFMA attention (prefill_kv_pack_kernel writes
// them from the cache rows; the RoPE / KV pass writes a prompt's new rows
// directly): per (kv head, tile of TK keys) [K hi | K lo | V^T hi | V^T lo],
// K planes TK rows of head_dim bf16, V^T planes head_dim rows of TK bf16,
// 16-byte chunks swizzled by the row (fa_swz), V^T positions permuted within
// each 32-key group (fa_pos_key).
// ---------------------------------------------------------------------------
template <int HD>
struct FaShape {
    static constexpr int TK = HD == 128 ? 32 : 64;  // keys per tile
    static constexpr int Plane = TK * HD * 2;       // bytes of one bf16 plane
    static constexpr int Stage = 4 * Plane;         // K hi | K lo | V^T hi | V^T lo
    static_assert(Stage % (1024 * 4) == 0, "whole 1 KiB copies per wave for 2 or 4 waves");
};

// Chunk position of 16-byte chunk c of row r in a plane of `chunks` chunks per row.
__device__ __forceinline__ uint32_t fa_swz(uint32_t r, uint32_t c, uint32_t chunks) {
    return chunks >= 16 ? c ^ (r & 15u) : chunks == 8 ? c ^ (r & 7u) : c ^ ((r >> 1) & (chunks - 1u));
}
// Key (within the tile) held at V^T position p.
__device__ __forceinline__ uint32_t fa_pos_key(uint32_t p) {
    return (p & ~31u) | (((p >> 2) & 1u) << 4) | (((p >> 3) & 3u) << 2) | (p & 3u);
}
// V^T position of key k (within the tile): the inverse of fa_pos_key.
__device__ __forceinline__ uint32_t fa_key_pos(uint32_t k) {
    return (k & ~31u) | (((k >> 2) & 3u) << 3) | (((k >> 4) & 1u) << 2) | (k & 3u);
}

__device__ inline void split_bf16(float v, uint16_t& hi, uint16_t& lo) {
    hi = to_bf16_rne(v);
    lo = to_bf16_rne(v - from_bf16(hi));
}

// Byte offsets of element d of key row r in a tile image (head_dim hd).
struct FaImage {
    uint32_t hd, tk, plane, stage, tiles;
    __device__ FaImage(uint32_t head_dim, uint32_t n_keys)
        : hd(head_dim), tk(head_dim == 128 ? 32u : 64u), plane(tk * head_dim * 2), stage(4 * plane),
          tiles((n_keys + tk - 1) / tk) {}
    __device__ size_t tile(uint32_t h, uint32_t key) const { return (static_cast<size_t>(h) * tiles + key / tk) * stage; }
    __device__ uint32_t k_off(uint32_t r, uint32_t d) const {
        return r * (2 * hd) + fa_swz(r, d / 8, hd / 8) * 16 + (d % 8) * 2;
    }
    __device__ uint32_t v_off(uint32_t r, uint32_t d) const {
        const uint32_t p = fa_key_pos(r);
        return 2 * plane + d * (2 * tk) + fa_swz(d, p / 8, tk / 8) * 16 + (p % 8) * 2;
    }
};
// Key row `key` of head h: k and v values of dimension d, split hi / lo.
__device__ __forceinline__ void fa_image_put(char* img, const FaImage& f, uint32_t h, uint32_t key, uint32_t d,
                                             const float* k, const float* v) {
    char* t = img + f.tile(h, key);
    const uint32_t r = key % f.tk;
    uint16_t hi, lo;
    if (k) {
        split_bf16(*k, hi, lo);
        *reinterpret_cast<uint16_t*>(t + f.k_off(r, d)) = hi;
        *reinterpret_cast<uint16_t*>(t + f.plane + f.k_off(r, d)) = lo;
    }
    if (v) {
        split_bf16(*v, hi, lo);
        *reinterpret_cast<uint16_t*>(t + f.v_off(r, d)) = hi;
        *reinterpret_cast<uint16_t*>(t + f.plane + f.v_off(r, d)) = lo;
    }
}

// One block per token row t (position start + t): rotate its q heads in place
// and its k head vectors (after the QK-norm when the model has one), then
// write k and v to the cache rows of that position.
__global__ __launch_bounds__(kRowThreads) void prefill_rope_kv_kernel(PrefillRopeArgs a) {
    const uint32_t t = blockIdx.x;
    const uint32_t pos = a.start + t;
    float* row = a.qkv + static_cast<size_t>(t) * a.ld;
    if (a.part) {  // the q|k|v GEMM's K-split partial sums, added in split order (the bias is in split 0's)
        const float* pr = a.part + static_cast<size_t>(t) * a.ld;
        const size_t stride = static_cast<size_t>(a.rows) * a.ld;
        for (uint32_t i = threadIdx.x * 4; i < a.ld; i += kRowThreads * 4) {
            const float4 p0 = *reinterpret_cast<const float4*>(pr + i);
            *reinterpret_cast<float4*>(row + i) = add_parts(p0, pr + stride + i, stride, a.splits - 1);
        }
        __syncthreads();
    }
    const float* cs = a.rope_cs + static_cast<size_t>(pos) * a.hd;
    const uint32_t half = a.hd / 2;
    const uint32_t qpairs = a.heads * half, kpairs = a.kv_heads * half;
    float* kc = a.kcache + static_cast<size_t>(pos) * a.kvdim;
    float* vc = a.vcache + static_cast<size_t>(pos) * a.kvdim;
    // With kv_pack: the new rows' tile images too (the attention's pack pass
    // then covers only the tiles of earlier rows).
    char* const img = static_cast<char*>(a.kv_pack);
    const uint32_t n_keys = a.start + a.rows;
    const FaImage fi(a.hd, n_keys);
    float scq = 1.f, sck = 1.f;
    if (a.q_norm) {
        __shared__ float red[2][kRowThreads / 64];
        const uint32_t qw = a.heads * a.hd;
        float sq = 0.f, sk = 0.f;
        for (uint32_t i = threadIdx.x; i < qw; i += kRowThreads) sq = fmaf(row[i], row[i], sq);
        for (uint32_t i = threadIdx.x; i < a.kvdim; i += kRowThreads) sk = fmaf(row[qw + i], row[qw + i], sk);
        sq = wave_sum(sq), sk = wave_sum(sk);
        if ((threadIdx.x & 63) == 0) red[0][threadIdx.x >> 6] = sq, red[1][threadIdx.x >> 6] = sk;
        __syncthreads();
        float tq = 0.f, tk = 0.f;
#pragma unroll
        for (int w = 0; w < kRowThreads / 64; ++w) tq += red[0][w], tk += red[1][w];
        scq = 1.0f / sqrtf(tq / static_cast<float>(qw) + a.norm_eps);
        sck = 1.0f / sqrtf(tk / static_cast<float>(a.kvdim) + a.norm_eps);
    }
    // Four pairs per thread per pass, their loads issued before any store (the
    // stores go to the same row, so one pair at a time would serialise the
    // round trips).
    constexpr int kPairs = 4;
    const uint32_t total = qpairs + kpairs;
    for (uint32_t p0 = threadIdx.x; p0 < total; p0 += kPairs * kRowThreads) {
        float x0[kPairs], x1[kPairs], c[kPairs], sn[kPairs], w0[kPairs], w1[kPairs];
#pragma unroll
        for (int u = 0; u < kPairs; ++u) {
            const uint32_t p = p0 + u * kRowThreads;
            const uint32_t pc = p < total ? p : 0;
            const bool is_q = pc < qpairs;
            const uint32_t pp = is_q ? pc : pc - qpairs;
            const uint32_t h = pp / half, i = pp % half;
            const float* v = row + (is_q ? 0 : a.heads * a.hd) + h * a.hd;
            const int f = a.rope_layout == 0 ? 2 * i : i;
            const int sidx = a.rope_layout == 0 ? 2 * i + 1 : i + half;
            x0[u] = v[f], x1[u] = v[sidx];
            c[u] = cs[2 * i], sn[u] = cs[2 * i + 1];
            w0[u] = w1[u] = 1.f;
            if (a.q_norm) {
                const uint16_t* nw = (is_q ? a.q_norm : a.k_norm) + h * a.hd;
                w0[u] = from_bf16(nw[f]), w1[u] = from_bf16(nw[sidx]);
            }
        }
#pragma unroll
        for (int u = 0; u < kPairs; ++u) {
            const uint32_t p = p0 + u * kRowThreads;
            if (p >= total) break;
            const bool is_q = p < qpairs;
            const uint32_t pp = is_q ? p : p - qpairs;
            const uint32_t h = pp / half, i = pp % half;
            float* v = row + (is_q ? 0 : a.heads * a.hd) + h * a.hd;
            const int f = a.rope_layout == 0 ? 2 * i : i;
            const int sidx = a.rope_layout == 0 ? 2 * i + 1 : i + half;
            float a0 = x0[u], a1 = x1[u];
            if (a.q_norm) {  // weight * (x * s), OlmoeRMSNorm's order
                const float sc = is_q ? scq : sck;
                a0 = w0[u] * (a0 * sc);
                a1 = w1[u] * (a1 * sc);
            }
            // rotatePair, src/llm.zig:1360-1371: x0*c - x1*s, x0*s + x1*c (unfused)
            const float r0 = __fsub_rn(__fmul_rn(a0, c[u]), __fmul_rn(a1, sn[u]));
            const float r1 = __fadd_rn(__fmul_rn(a0, sn[u]), __fmul_rn(a1, c[u]));
            v[f] = r0;
            v[sidx] = r1;
            if (!is_q) {
                kc[h * a.hd + f] = r0;
                kc[h * a.hd + sidx] = r1;
                if (img) {
                    fa_image_put(img, fi, h, pos, f, &r0, nullptr);
                    fa_image_put(img, fi, h, pos, sidx, &r1, nullptr);
                }
            }
        }
    }
    const float* vsrc = row + (a.heads + a.kv_heads) * a.hd;
    for (uint32_t i = threadIdx.x; i < a.kvdim; i += kRowThreads) {
        vc[i] = vsrc[i];
        if (img) fa_image_put(img, fi, i / a.hd, pos, i % a.hd, nullptr, vsrc + i);
    }
    if (img) {  // the last tile's rows past the prompt's keys: zeros (the pack kernel's padding)
        const float zero = 0.f;
        for (uint32_t key = n_keys + t; key < fi.tiles * fi.tk; key += a.rows)
            for (uint32_t i = threadIdx.x; i < a.kvdim; i += kRowThreads)
                fa_image_put(img, fi, i / a.hd, key, i % a.hd, &zero, &zero);
    }
}

// ---------------------------------------------------------------------------
// Causal GQA attention for a chunk of prompt rows (computeAttentionInto,
// src/llm.zig:1302-1335, for every row at once). One wave per (kv head,
// group of consecutive rows); four lanes per (row, q head) pair, each holding
// a quarter of head_dim of q and of the output accumulator, so one wave
// covers 16 pairs (16 / G rows of the G heads sharing the kv head). The wave
// walks cache rows 0 .. its last row's position in chunks of 16 keys: a dot
// product is a quarter per lane plus two xor shuffles, then an online softmax
// (chunk max, one rescale per chunk). Keys past a pair's own position are
// masked. Waves take the row groups from the last (longest) to the first.
// ---------------------------------------------------------------------------
constexpr int kAttnThreads = 256;
constexpr int kKeyChunk = 16;
constexpr int kLanesPerPair = 4;
constexpr int kPairsPerWave = 64 / kLanesPerPair;

template <int HD>
__global__ __launch_bounds__(kAttnThreads) void prefill_attn_kernel(PrefillAttnArgs a) {
    constexpr int DS = HD / kLanesPerPair;  // dims per lane
    const int lane = threadIdx.x & 63;
    const uint32_t item = blockIdx.x * (kAttnThreads / 64) + (threadIdx.x >> 6);
    const uint32_t G = a.heads / a.kv_heads;
    const uint32_t rows_per_wave = kPairsPerWave / G;
    const uint32_t row_groups = (a.rows + rows_per_wave - 1) / rows_per_wave;
    if (item >= row_groups * a.kv_heads) return;
    const uint32_t kvh = item % a.kv_heads;
    const uint32_t r0 = (row_groups - 1 - item / a.kv_heads) * rows_per_wave;
    const uint32_t pair = lane / kLanesPerPair, part = lane % kLanesPerPair;
    const uint32_t lr = pair / G, gq = pair % G;
    const bool active = lr < rows_per_wave && r0 + lr < a.rows;
    const uint32_t row = active ? r0 + lr : r0;
    const uint32_t my_pos = a.start + row;
    const uint32_t last_row = min(r0 + rows_per_wave, a.rows) - 1;
    const uint32_t n_keys = a.start + last_row + 1;  // wave-uniform
    const uint32_t qh = kvh * G + (active ? gq : 0);
    const uint32_t d0 = part * DS;

    float q[DS], acc[DS];
    const float* qp = a.q + static_cast<size_t>(row) * a.ldq + qh * HD + d0;
#pragma unroll
    for (int d = 0; d < DS; d += 4) {
        const float4 v = *reinterpret_cast<const float4*>(qp + d);
        q[d] = v.x, q[d + 1] = v.y, q[d + 2] = v.z, q[d + 3] = v.w;
        acc[d] = acc[d + 1] = acc[d + 2] = acc[d + 3] = 0.f;
    }
    float m = -INFINITY, l = 0.f;
    const float* kb = a.kcache + kvh * HD + d0;
    const float* vb = a.vcache + kvh * HD + d0;
    for (uint32_t j0 = 0; j0 < n_keys; j0 += kKeyChunk) {
        float s[kKeyChunk];
        float cmax = -INFINITY;
#pragma unroll
        for (int c = 0; c < kKeyChunk; ++c) {
            const uint32_t j = j0 + c;
            float dot = 0.f;
            if (j < n_keys) {
                const float* kr = kb + static_cast<size_t>(j) * a.kvdim;
#pragma unroll
                for (int d = 0; d < DS; d += 4) {
                    const float4 kv4 = *reinterpret_cast<const float4*>(kr + d);
                    dot = fmaf(q[d], kv4.x, dot);
                    dot = fmaf(q[d + 1], kv4.y, dot);
                    dot = fmaf(q[d + 2], kv4.z, dot);
                    dot = fmaf(q[d + 3], kv4.w, dot);
                }
            }
            dot += __shfl_xor(dot, 1, 64);
            dot += __shfl_xor(dot, 2, 64);
            s[c] = j <= my_pos ? __fmul_rn(dot, a.scale) : -INFINITY;
            cmax = fmaxf(cmax, s[c]);
        }
        const float m_new = fmaxf(m, cmax);
        const float corr = expf(m - m_new);
        l *= corr;
#pragma unroll
        for (int d = 0; d < DS; ++d) acc[d] *= corr;
#pragma unroll
        for (int c = 0; c < kKeyChunk; ++c) {
            const uint32_t j = j0 + c;
            if (j < n_keys) {
                const float e = expf(s[c] - m_new);
                l += e;
                const float* vr = vb + static_cast<size_t>(j) * a.kvdim;
#pragma unroll
                for (int d = 0; d < DS; d += 4) {
                    const float4 vv = *reinterpret_cast<const float4*>(vr + d);
                    acc[d] = fmaf(e, vv.x, acc[d]);
                    acc[d + 1] = fmaf(e, vv.y, acc[d + 1]);
                    acc[d + 2] = fmaf(e, vv.z, acc[d + 2]);
                    acc[d + 3] = fmaf(e, vv.w, acc[d + 3]);
                }
            }
        }
        m = m_new;
    }
    if (!active) return;
    const float inv = 1.0f / l;
    float* op = a.out + static_cast<size_t>(row) * a.ldo + qh * HD + d0;
#pragma unroll
    for (int d = 0; d < DS; d += 4)
        *reinterpret_cast<float4*>(op + d) =
            make_float4(acc[d] * inv, acc[d + 1] * inv, acc[d + 2] * inv, acc[d + 3] * inv);
}

// ---------------------------------------------------------------------------
// Causal GQA attention on MFMA (flash-attention form) for a chunk of prompt
// rows.
//
// Packing (prefill_kv_pack_kernel): first, cache rows 0 .. start + rows - 1
// of each kv head are split once into bf16 hi/lo halves and written as
// per-tile images of the attention kernel's LDS stage,
//   [K hi: TK keys x HD] [K lo] [V^T hi: HD dims x TK positions] [V^T lo],
// TK = 64 keys (32 for head_dim 128). In every plane the 16-byte chunk c of
// row r sits at chunk fa_swz(r, c), which keeps the fragment reads free of
// bank conflicts under ds_read_b128's passes (see the GEMM tile notes): the
// 16 lanes of a pass read 16 rows, two chunk columns, and land on 16 distinct
// 16-byte bank groups for rows of 64, 128 and 256 bytes. V^T positions are permuted within
// each 32-key group: position 8q + 4u + j holds key 16u + 4q + j (below).
// Keys past the last cache row are zeros.
//
// Attention (prefill_fa_kernel): block = (kv head, 128 query vectors); a
// query vector is one (row, q head) pair of the G heads sharing the kv head,
// rows_per_block = 128 / G rows (vectors past rows_per_block * G are idle).
// Wave w owns vectors 32w .. 32w + 31 as two groups of 16. Tile images are
// copied whole into LDS by global_load_lds_dwordx4, two stages, tile i + 1
// landing while tile i is used. Products are taken transposed so that the
// softmax state of a vector stays in the lanes of one column:
//   S^T  = K . Q^T   A = K rows (LDS), B = Q (registers); lane l gets
//                    keys 16u + 4(l/16) + j of vector l%16
//   O^T += V^T . P^T A = V^T rows (LDS), B = P: a lane's 8 values of a
//                    32-key step, in (u, j) order, are its B fragment under
//                    the permuted V^T positions, so P never leaves registers
// Each product is hi.hi + lo.hi + hi.lo with f32 accumulation (about 2^-16
// relative, like the f32 path it replaces). Online softmax per 32-key step in
// f32: the row max over the lane's 8 values and two xor shuffles; the row sum
// stays per lane until the end. v_mfma_f32_16x16x32_bf16 layout as the GEMM's.
// ---------------------------------------------------------------------------
constexpr int kFaVecs = 128;  // query vectors (4 waves of 32) per block of the first two forms


// One block per (key tile, kv head): K chunks straight to the K planes, the V
// tile through LDS to the transposed planes.
template <int HD>
__global__ __launch_bounds__(256) void prefill_kv_pack_kernel(PrefillAttnArgs a) {
    using S = FaShape<HD>;
    constexpr int TK = S::TK, KCH = HD / 8, VCH = TK / 8;
    __shared__ float vs[TK][HD + 1];
    const uint32_t tile = blockIdx.x, h = blockIdx.y;
    const uint32_t n_keys = a.start + a.rows;
    char* img = static_cast<char*>(a.kv_pack) + (static_cast<size_t>(h) * a.kv_tiles + tile) * S::Stage;
    for (int i = threadIdx.x; i < TK * KCH; i += 256) {
        const uint32_t r = i / KCH, c = i % KCH, key = tile * TK + r;
        float k[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (key < n_keys) {
            const size_t off = static_cast<size_t>(key) * a.kvdim + h * HD + 8 * c;
            const float4 k0 = *reinterpret_cast<const float4*>(a.kcache + off);
            const float4 k1 = *reinterpret_cast<const float4*>(a.kcache + off + 4);
            const float4 v0 = *reinterpret_cast<const float4*>(a.vcache + off);
            const float4 v1 = *reinterpret_cast<const float4*>(a.vcache + off + 4);
            k[0] = k0.x, k[1] = k0.y, k[2] = k0.z, k[3] = k0.w, k[4] = k1.x, k[5] = k1.y, k[6] = k1.z, k[7] = k1.w;
            v[0] = v0.x, v[1] = v0.y, v[2] = v0.z, v[3] = v0.w, v[4] = v1.x, v[5] = v1.y, v[6] = v1.z, v[7] = v1.w;
        }
        u16x8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            uint16_t hh, ll;
            split_bf16(k[e], hh, ll);
            hi[e] = hh, lo[e] = ll;
            vs[r][8 * c + e] = v[e];
        }
        const uint32_t o = r * (2 * HD) + fa_swz(r, c, KCH) * 16;
        *reinterpret_cast<u16x8*>(img + o) = hi;
        *reinterpret_cast<u16x8*>(img + S::Plane + o) = lo;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < HD * VCH; i += 256) {
        const uint32_t d = i / VCH, c = i % VCH;
        u16x8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            uint16_t hh, ll;
            split_bf16(vs[fa_pos_key(8 * c + e)][d], hh, ll);
            hi[e] = hh, lo[e] = ll;
        }
        const uint32_t o = d * (2 * TK) + fa_swz(d, c, VCH) * 16;
        *reinterpret_cast<u16x8*>(img + 2 * S::Plane + o) = hi;
        *reinterpret_cast<u16x8*>(img + 3 * S::Plane + o) = lo;
    }
}

// Waits for a group of fragment reads (the fragments are operands, so their
// uses cannot move above the wait).
__device__ __forceinline__ void fa_lds_wait(bf16x8 (&f)[4]) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]));
}

// A block holds QW * 32 query vectors (QW query waves). KS = 2 (prompts
// whose blocks would leave CUs idle or alone on them): two groups of QW waves
// take the block's key tiles in turn (group 1 the odd tiles), each through
// its own two stages, and group 0 merges group 1's running max, sum and
// outputs at the end (flash-decoding's merge of two splits): half the tiles
// on the longest block.
// (Two waves per SIMD where the LDS lets two blocks or two groups share a CU.)
template <int HD, int QW, int KS>
__global__ __launch_bounds__(64 * QW * KS) __attribute__((amdgpu_waves_per_eu(QW * KS == 4 && KS == 2 ? 1 : 2)))
void prefill_fa_kernel(
    PrefillAttnArgs a) {
    using S = FaShape<HD>;
    constexpr int TK = S::TK, DS = HD / 32, NT = HD / 16, SUB = TK / 32;
    constexpr int KCH = HD / 8, VCH = TK / 8;
    constexpr int DMA = S::Stage / 1024 / QW;  // 1 KiB copies per wave per tile
    static_assert(HD % 32 == 0 && (DS + NT / 2) % 2 == 0, "head_dim 32, 64 or 128");
    static_assert((KS == 1 || KS == 2) && (QW == 2 || QW == 4), "one or two key groups of 2 or 4 waves");
    __shared__ __attribute__((aligned(1024))) char lds[KS * 2 * S::Stage];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = (tid >> 6) % QW;  // query wave within the key group
    const int kg = (tid >> 6) / QW;    // key group: tiles kg, kg + KS, ...
    const int fr = lane & 15, fq = lane >> 4;
    const uint32_t G = a.heads / a.kv_heads;
    const uint32_t rows_per_block = (32 * QW) / G;
    const uint32_t row_groups = (a.rows + rows_per_block - 1) / rows_per_block;
    const uint32_t kvh = blockIdx.x % a.kv_heads;
    const uint32_t r0 = (row_groups - 1 - blockIdx.x / a.kv_heads) * rows_per_block;  // longest first
    const uint32_t last_row = min(r0 + rows_per_block, a.rows) - 1;
    const uint32_t n_tiles = (a.start + last_row + TK) / TK;  // keys 0 .. start + last_row

    // Q as the B operand: group gi, lane l holds vector 32 wave + 16 gi + l%16,
    // dims 32 s + 8 (l/16) .. +7, scaled by scale * log2(e) (scores come out in
    // base-2 units for v_exp_f32) and split hi/lo.
    const float qscale = a.scale * 1.44269504088896341f;
    bf16x8 qh[2][DS], ql[2][DS];
    uint32_t pos[2];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
        const uint32_t v = wave * 32 + gi * 16 + fr;
        const uint32_t t = v / G, g = v % G;
        const bool valid = t < rows_per_block && r0 + t < a.rows;
        pos[gi] = a.start + min(r0 + min(t, rows_per_block - 1), a.rows - 1);
        const float* qp = a.q + static_cast<size_t>(valid ? r0 + t : 0) * a.ldq + (kvh * G + (valid ? g : 0)) * HD;
#pragma unroll
        for (int s = 0; s < DS; ++s) {
            float x[8];
            const float4 x0 = valid ? *reinterpret_cast<const float4*>(qp + 32 * s + 8 * fq) : make_float4(0, 0, 0, 0);
            const float4 x1 = valid ? *reinterpret_cast<const float4*>(qp + 32 * s + 8 * fq + 4) : make_float4(0, 0, 0, 0);
            x[0] = x0.x, x[1] = x0.y, x[2] = x0.z, x[3] = x0.w, x[4] = x1.x, x[5] = x1.y, x[6] = x1.z, x[7] = x1.w;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float xs = __fmul_rn(x[e], qscale);
                const __bf16 hb = static_cast<__bf16>(xs);  // v_cvt_pk_bf16_f32: round to nearest even
                qh[gi][s][e] = hb;
                ql[gi][s][e] = static_cast<__bf16>(xs - static_cast<float>(hb));
            }
        }
    }
    // First and last positions among the wave's vectors: tiles that start past
    // the last are skipped, tiles that end at or before the first need no mask.
    const uint32_t t_first = min((static_cast<uint32_t>(wave) * 32u) / G, rows_per_block - 1);
    const uint32_t t_last = min((static_cast<uint32_t>(wave) * 32u + 31u) / G, rows_per_block - 1);
    const uint32_t pos_first = a.start + min(r0 + t_first, a.rows - 1);
    const uint32_t pos_last = a.start + min(r0 + t_last, a.rows - 1);

    f32x4 o[2][NT];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi)
#pragma unroll
        for (int n = 0; n < NT; ++n) o[gi][n] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};

    // Copies: wave w moves bytes [w, w + 1) * DMA KiB of each tile image of
    // its key group, into the group's two stages.
    const char* src0 = static_cast<const char*>(a.kv_pack) + static_cast<size_t>(kvh) * a.kv_tiles * S::Stage +
                       wave * DMA * 1024 + lane * 16;
    char* dst0 = lds + kg * 2 * S::Stage + wave * DMA * 1024;
    auto issue = [&](uint32_t t, int st) {
        const char* src = src0 + static_cast<size_t>(t) * S::Stage;
#pragma unroll
        for (int i = 0; i < DMA; ++i) gemm_dma16(src + i * 1024, dst0 + st * S::Stage + i * 1024);
    };
    // Fragment offsets: K row 16u + l%16 of a 32-key step, chunk 4s + l/16;
    // V^T row 16n + l%16, chunk 4ks + l/16 (both swizzled by the row).
    const uint32_t lds0 = gemm_lds_addr(lds);
    static_assert(KCH <= 16 && VCH <= 16, "rows of at most 256 bytes");
    const uint32_t fk = KCH == 16 ? fr : KCH == 8 ? (fr & 7) : ((fr >> 1) & 3);  // fa_swz of rows 16u + fr
    const uint32_t fv = VCH == 16 ? fr : VCH == 8 ? (fr & 7) : ((fr >> 1) & 3);
    uint32_t koff[DS], voff[SUB];
#pragma unroll
    for (int s = 0; s < DS; ++s) koff[s] = fr * (2 * HD) + (((4 * s + fq) ^ fk) << 4);
#pragma unroll
    for (int ks = 0; ks < SUB; ++ks) voff[ks] = 2 * S::Plane + fr * (2 * TK) + (((4 * ks + fq) ^ fv) << 4);
    // Fragment groups: K of step ks, dims 32s.. = {hi, lo} x keys {0..15, 16..31};
    // V^T of step ks, dims 32vg.. = {hi, lo} x dims {16(2vg).., 16(2vg+1)..}.
    auto read_k = [&](bf16x8 (&f)[4], uint32_t sb, int ks, int s) {
        const uint32_t b = sb + ks * 32 * (2 * HD) + koff[s];
        f[0] = gemm_lds_read(b);
        f[1] = gemm_lds_read(b + S::Plane);
        f[2] = gemm_lds_read(b + 16 * (2 * HD));
        f[3] = gemm_lds_read(b + 16 * (2 * HD) + S::Plane);
    };
    auto read_v = [&](bf16x8 (&f)[4], uint32_t sb, int ks, int vg) {
        const uint32_t b = sb + voff[ks] + 2 * vg * 16 * (2 * TK);
        f[0] = gemm_lds_read(b);
        f[1] = gemm_lds_read(b + S::Plane);
        f[2] = gemm_lds_read(b + 16 * (2 * TK));
        f[3] = gemm_lds_read(b + 16 * (2 * TK) + S::Plane);
    };

    // One tile from LDS stage sb (keys j0 ..): MASKED compares every key with
    // its vector's position, else the whole tile is visible to the wave.
    auto tile = [&](uint32_t sb, uint32_t j0, auto masked_tag) {
        constexpr bool MASKED = decltype(masked_tag)::value;
        bf16x8 f[2][4];
        read_k(f[0], sb, 0, 0);
        fa_lds_wait(f[0]);
#pragma unroll
        for (int ks = 0; ks < SUB; ++ks) {
            // S^T for 32 keys: group s holds dims 32s .. 32s + 31.
            f32x4 sacc[2][2];
#pragma unroll
            for (int gi = 0; gi < 2; ++gi) sacc[gi][0] = sacc[gi][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < DS; ++s) {
                bf16x8(&cur)[4] = f[s & 1];
                bf16x8(&nx)[4] = f[(s + 1) & 1];
                if (s + 1 < DS) read_k(nx, sb, ks, s + 1);
                else read_v(nx, sb, ks, 0);
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int gi = 0; gi < 2; ++gi)
                        sacc[gi][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur[2 * u], qh[gi][s], sacc[gi][u], 0, 0, 0);
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int gi = 0; gi < 2; ++gi)
                        sacc[gi][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur[2 * u + 1], qh[gi][s], sacc[gi][u], 0, 0, 0);
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int gi = 0; gi < 2; ++gi)
                        sacc[gi][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur[2 * u], ql[gi][s], sacc[gi][u], 0, 0, 0);
                fa_lds_wait(nx);
            }
            // Mask, online softmax in base 2 (v_exp_f32); P as hi/lo B fragments.
            bf16x8 ph[2], pl[2];
            float corr[2];
            bool grew = false;
#pragma unroll
            for (int gi = 0; gi < 2; ++gi) {
                float mx = -INFINITY;
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (MASKED && j0 + 32 * ks + 16 * u + 4 * fq + j > pos[gi]) sacc[gi][u][j] = -INFINITY;
                        mx = fmaxf(mx, sacc[gi][u][j]);
                    }
                mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                // Finite with one key group: key 0 is in its first step. The
                // second group's first tiles can hide every key from a
                // vector: the max then stays -inf and p = 0, corr = 0.
                const float m_new = fmaxf(m_run[gi], mx);
                const float m_sub = KS == 1 || m_new != -INFINITY ? m_new : 0.f;
                grew |= m_new != m_run[gi];
                corr[gi] = __builtin_amdgcn_exp2f(m_run[gi] - m_sub);
                float sum = 0.f;
#pragma unroll
                for (int u = 0; u < 2; ++u)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float p = __builtin_amdgcn_exp2f(sacc[gi][u][j] - m_sub);
                        sum += p;
                        const __bf16 hb = static_cast<__bf16>(p);
                        ph[gi][4 * u + j] = hb;
                        pl[gi][4 * u + j] = static_cast<__bf16>(p - static_cast<float>(hb));
                    }
                l_run[gi] = l_run[gi] * corr[gi] + sum;
                m_run[gi] = m_new;
            }
            if (__any(grew)) {  // corr is 1 wherever no row max grew
#pragma unroll
                for (int gi = 0; gi < 2; ++gi)
#pragma unroll
                    for (int n = 0; n < NT; ++n) o[gi][n] *= corr[gi];
            }
            // O^T += V^T . P^T, two 16-dim tiles per group.
#pragma unroll
            for (int vg = 0; vg < NT / 2; ++vg) {
                bf16x8(&cur)[4] = f[(DS + vg) & 1];
                bf16x8(&nx)[4] = f[(DS + vg + 1) & 1];
                const bool more = vg + 1 < NT / 2 || ks + 1 < SUB;
                if (vg + 1 < NT / 2) read_v(nx, sb, ks, vg + 1);
                else if (ks + 1 < SUB) read_k(nx, sb, ks + 1, 0);
#pragma unroll
                for (int nn = 0; nn < 2; ++nn)
#pragma unroll
                    for (int gi = 0; gi < 2; ++gi)
                        o[gi][2 * vg + nn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur[2 * nn], ph[gi], o[gi][2 * vg + nn], 0, 0, 0);
#pragma unroll
                for (int nn = 0; nn < 2; ++nn)
#pragma unroll
                    for (int gi = 0; gi < 2; ++gi)
                        o[gi][2 * vg + nn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur[2 * nn + 1], ph[gi], o[gi][2 * vg + nn], 0, 0, 0);
#pragma unroll
                for (int nn = 0; nn < 2; ++nn)
#pragma unroll
                    for (int gi = 0; gi < 2; ++gi)
                        o[gi][2 * vg + nn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur[2 * nn], pl[gi], o[gi][2 * vg + nn], 0, 0, 0);
                if (more) fa_lds_wait(nx);
            }
        }
    };

    if (static_cast<uint32_t>(kg) < n_tiles) issue(kg, 0);
    const uint32_t n_it = (n_tiles + KS - 1) / KS;
    for (uint32_t it = 0; it < n_it; ++it) {
        const int st = it & 1;
        const uint32_t t = it * KS + kg;
        gemm_wait_vm(0);  // this wave's copies of tile t
        gemm_barrier();   // every wave's copies landed; stage st ^ 1 is no longer read
        if (t + KS < n_tiles) issue(t + KS, st ^ 1);
        if (t >= n_tiles) continue;
        const uint32_t j0 = t * TK;
        if (j0 > pos_last) continue;  // every key of the tile is masked for this wave
        const uint32_t sb = lds0 + (kg * 2 + st) * S::Stage;
        if (j0 + TK - 1 <= pos_first) tile(sb, j0, std::false_type{});
        else tile(sb, j0, std::true_type{});
    }
    if constexpr (KS == 2) {
        // Group 1's state through LDS (field f of lane l of query wave w at
        // [w][f][l]); group 0 combines in group order: M = max(m0, m1),
        // O = O0 2^(m0 - M) + O1 2^(m1 - M), the same for the sums.
        constexpr int F = 4 + 8 * NT;
        static_assert(QW * F * 64 * 4 <= KS * 2 * S::Stage, "the merge fits the stages");
        float* xs = reinterpret_cast<float*>(lds) + static_cast<size_t>(wave) * F * 64 + lane;
        __syncthreads();  // both groups are done with their stages
        if (kg == 1) {
#pragma unroll
            for (int gi = 0; gi < 2; ++gi) {
                xs[(2 * gi) * 64] = m_run[gi];
                xs[(2 * gi + 1) * 64] = l_run[gi];
#pragma unroll
                for (int n = 0; n < NT; ++n)
#pragma unroll
                    for (int e = 0; e < 4; ++e) xs[(4 + (gi * NT + n) * 4 + e) * 64] = o[gi][n][e];
            }
        }
        __syncthreads();
        if (kg == 1) return;
#pragma unroll
        for (int gi = 0; gi < 2; ++gi) {
            const float m1 = xs[(2 * gi) * 64], l1 = xs[(2 * gi + 1) * 64];
            const float m = fmaxf(m_run[gi], m1);  // finite: group 0 saw key 0
            const float c0 = __builtin_amdgcn_exp2f(m_run[gi] - m), c1 = __builtin_amdgcn_exp2f(m1 - m);
            l_run[gi] = l_run[gi] * c0 + l1 * c1;
#pragma unroll
            for (int n = 0; n < NT; ++n)
#pragma unroll
                for (int e = 0; e < 4; ++e) o[gi][n][e] = o[gi][n][e] * c0 + xs[(4 + (gi * NT + n) * 4 + e) * 64] * c1;
        }
    }
    // out[row][(kvh G + g) HD + d] = O / l: lane l holds dims 16n + 4(l/16) .. +3 of vector l%16.
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
        float l = l_run[gi];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        const uint32_t v = wave * 32 + gi * 16 + fr;
        const uint32_t t = v / G, g = v % G;
        if (t >= rows_per_block || r0 + t >= a.rows) continue;
        const float inv = 1.0f / l;
        if (a.out_hl) {  // split planes of the o_proj GEMM's A (heads * HD is a multiple of 32: no tail)
            uint16_t* hp = a.out_hl + static_cast<size_t>(r0 + t) * (a.heads * HD) + (kvh * G + g) * HD + 4 * fq;
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                u16x4 h, lo;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    uint16_t hh, ll;
                    split_bf16(o[gi][n][e] * inv, hh, ll);
                    h[e] = hh, lo[e] = ll;
                }
                *reinterpret_cast<u16x4*>(hp + 16 * n) = h;
                *reinterpret_cast<u16x4*>(hp + a.out_plane + 16 * n) = lo;
            }
            continue;
        }
        float* op = a.out + static_cast<size_t>(r0 + t) * a.ldo + (kvh * G + g) * HD + 4 * fq;
#pragma unroll
        for (int n = 0; n < NT; ++n)
            *reinterpret_cast<float4*>(op + 16 * n) =
                make_float4(o[gi][n][0] * inv, o[gi][n][1] * inv, o[gi][n][2] * inv, o[gi][n][3] * inv);
    }
}

}  // namespace

std::atomic<int> prefill_fa_form{-1};

// VVLI_PREFILL_ATTN=vector selects the f32 vector kernel (A/B measurement).
bool prefill_attn_vector = [] {
    const char* e = getenv("VVLI_PREFILL_ATTN");
    return e != nullptr && strcmp(e, "vector") == 0;
}();

// silu(gate) * up from the split-K sums of a GateUp GEMM, written as out's
// f32 rows or as out_hl's split planes (zero tail), like the unsplit epilogue.
__global__ __launch_bounds__(256) void gemm_swiglu_kernel(GemmArgs g) {
    const uint32_t kpo = gemm_kp(g.N);
    const uint32_t n = blockIdx.x * 256 + threadIdx.x, row = blockIdx.y;
    if (n >= kpo) return;
    const float* gu = g.gu_acc + static_cast<size_t>(row) * (2 * g.N);
    const float v = n < g.N ? silu_mul(gu[n], gu[g.N + n]) : 0.f;
    if (g.out_hl) {
        const uint16_t h = to_bf16_rne(v);
        uint16_t* o = g.out_hl + static_cast<size_t>(row) * kpo + n;
        o[0] = h;
        o[g.out_plane] = to_bf16_rne(v - from_bf16(h));
    } else if (n < g.N) {
        g.out[static_cast<size_t>(row) * g.ldo + n] = v;
    }
}

__global__ __launch_bounds__(256) void zero_rows_kernel(float* __restrict__ out, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) out[i] = 0.f;
}

// K splits for a launch. One block runs per CU. Splitting costs atomics, a
// zeroing pass and shorter K loops (the copy pipeline fills and drains per
// split), so it is used only when the tiles leave more than half of the CUs
// idle: then as many splits as keep the launch within one round (each split
// at least 8 or 16 K steps, at most 32). Plain tiles split only when the
// output rows are dense (they are zeroed first); SwiGLU tiles only with a
// gate/up scratch (the epilogue is nonlinear: the sums go there and a
// separate pass applies it).
static uint32_t gemm_cus() {
    static const uint32_t cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                     hipSuccess || n <= 0)
            n = 256;
        return static_cast<uint32_t>(n);
    }();
    return cus;
}

uint32_t gemm_k_splits(int mode, const GemmArgs& g, uint32_t tiles) {
    if ((mode == kGemmGateUp && !g.gu_acc) || (mode == kGemmPlain && g.ldo != g.N)) return 1;
    const uint32_t cus = gemm_cus();
    const uint32_t nk = (g.K + kBK - 1) / kBK;
    // Each split keeps at least 8 K steps (16 once there are 32 tiles: then
    // half the CUs with twice the steps beat a full round of short loops,
    // whose copy pipeline fills and drains per split).
    const uint32_t min_steps = tiles >= 32 ? 16 : 8;
    const uint32_t max_splits = std::min<uint32_t>(32, nk / min_steps > 0 ? nk / min_steps : 1);
    if (2 * tiles > cus) return 1;
    uint32_t splits = std::max<uint32_t>(1, std::min<uint32_t>(max_splits, cus / tiles));
    // Every split gets K steps: the kernel gives split z steps from z * ceil(nk / splits).
    while (splits > 1 && (splits - 1) * ((nk + splits - 1) / splits) >= nk) --splits;
    return splits;
}

uint32_t gemm_splits(int mode, const GemmArgs& g) {
    const uint32_t cols = mode == kGemmGateUp ? 2 * g.N : g.N;
    return gemm_k_splits(mode, g, ((cols + kBN - 1) / kBN) * ((g.M + kBM - 1) / kBM));
}

size_t gemm_part_elems() { return static_cast<size_t>(gemm_cus()) * kBM * kBN; }

static uint32_t fa_tile_keys(uint32_t hd) { return hd == 128 ? FaShape<128>::TK : FaShape<64>::TK; }
static_assert(FaShape<32>::Stage == 8 * 64 * 32 && FaShape<64>::Stage == 8 * 64 * 64 &&
                  FaShape<128>::Stage == 8 * 32 * 128,
              "prefill_kv_pack_bytes sizes tiles as 8 * keys * head_dim bytes");

size_t prefill_kv_pack_bytes(uint32_t keys, uint32_t kv_heads, uint32_t hd) {
    if (hd != 32 && hd != 64 && hd != 128) return 0;
    const size_t tk = fa_tile_keys(hd);
    return static_cast<size_t>(kv_heads) * ((keys + tk - 1) / tk) * (8 * tk * hd);
}

uint32_t gemm_gateup_split_rows(uint32_t N) {
    const uint32_t tn = (2 * N + kBN - 1) / kBN;
    return gemm_cus() / (2 * tn) * kBM;  // row count whose tiles leave half of the CUs idle
}

size_t gemm_split_elems(uint32_t M, uint32_t K) { return static_cast<size_t>(2) * M * gemm_kp(K); }

hipError_t launch_gemm_bf16(int mode, const GemmArgs& g, hipStream_t s) {
    if (g.M == 0 || g.N == 0) return hipSuccess;
    if (!g.a_hl || g.K % 8 != 0 || (g.norm_w && !g.row_scale)) return hipErrorInvalidValue;
    if ((g.out_hl && mode != kGemmGateUp) || (!g.out_hl && !g.out) ||
        (g.a_plane && g.a_plane < static_cast<size_t>(g.M) * gemm_kp(g.K)) ||
        (g.out_hl && g.out_plane < static_cast<size_t>(g.M) * gemm_kp(g.N)))
        return hipErrorInvalidValue;
    if (!g.a_ready) {
        const size_t n = static_cast<size_t>(g.M) * (gemm_kp(g.K) / 8);
        hipError_t e = vlaunch(gemm_split_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, s, g);
        if (e != hipSuccess) return e;
    }
    static const hipError_t attr = [] {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_bf16_kernel<kGemmPlain>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kGemmLds);
        if (e == hipSuccess)
            e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_bf16_kernel<kGemmResid>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, kGemmLds);
        if (e == hipSuccess)
            e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_bf16_kernel<kGemmGateUp>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, kGemmLds);
        return e;
    }();
    if (attr != hipSuccess) return attr;
    const uint32_t cols = mode == kGemmGateUp ? 2 * g.N : g.N;
    const uint32_t gx = (cols + kBN - 1) / kBN, gy = (g.M + kBM - 1) / kBM;
    const uint32_t splits = gemm_k_splits(mode, g, gx * gy);
    if (splits > 1 && g.part && static_cast<size_t>(splits) * g.M * g.N > gemm_part_elems())
        return hipErrorInvalidValue;  // (splits * tiles <= CUs keeps every launch within it)
    if (splits > 1 && mode != kGemmResid && !(mode == kGemmPlain && g.part)) {
        const bool gu = mode == kGemmGateUp;
        const size_t n = static_cast<size_t>(g.M) * (gu ? 2 * g.N : g.ldo);
        const uint32_t blocks = static_cast<uint32_t>(std::min<size_t>((n + 255) / 256, 4096));
        hipError_t e = vlaunch(zero_rows_kernel, dim3(blocks), dim3(256), 0, s, gu ? g.gu_acc : g.out, n);
        if (e != hipSuccess) return e;
    }
    if (splits > 1 && mode == kGemmGateUp) {
        const dim3 grid(gx * gy, 1, splits);
        hipError_t e = vlaunch(gemm_bf16_kernel<kGemmGateUp>, grid, dim3(kGemmThreads), kGemmLds, s, g);
        if (e != hipSuccess) return e;
        return vlaunch(gemm_swiglu_kernel, dim3((gemm_kp(g.N) + 255) / 256, g.M), dim3(256), 0, s, g);
    }
    const dim3 grid(gx * gy, 1, splits);  // tiles in the XCD-aware order of the kernel
    switch (mode) {
        case kGemmPlain: return vlaunch(gemm_bf16_kernel<kGemmPlain>, grid, dim3(kGemmThreads), kGemmLds, s, g);
        case kGemmResid: return vlaunch(gemm_bf16_kernel<kGemmResid>, grid, dim3(kGemmThreads), kGemmLds, s, g);
        case kGemmGateUp: return vlaunch(gemm_bf16_kernel<kGemmGateUp>, grid, dim3(kGemmThreads), kGemmLds, s, g);
        default: return hipErrorInvalidValue;
    }
}

uint32_t grouped_gemm_tile_rows() { return kBM; }
uint32_t grouped_gemm_max_tiles(uint32_t M, uint32_t E) { return M / kBM + E; }

hipError_t launch_gemm_grouped(int mode, const GemmArgs& g, hipStream_t s) {
    if (g.M == 0 || g.N == 0) return hipSuccess;
    if (!g.a_hl || !g.tiles || g.max_tiles == 0 || g.K % 8 != 0 || (g.norm_w && !g.row_scale) ||
        (mode != kGemmGateUp && mode != kGemmPlain) || (mode == kGemmGateUp && !g.out_hl) ||
        (mode == kGemmPlain && (g.out_hl || !g.out || g.bias[0] || g.seg_end[0] != g.N)) ||
        (g.a_plane && g.a_plane < static_cast<size_t>(g.M) * gemm_kp(g.K)) ||
        (g.out_hl && g.out_plane < static_cast<size_t>(g.M) * gemm_kp(g.N)))
        return hipErrorInvalidValue;
    if (!g.a_ready) {
        const size_t n = static_cast<size_t>(g.M) * (gemm_kp(g.K) / 8);
        hipError_t e = vlaunch(gemm_split_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, s, g);
        if (e != hipSuccess) return e;
    }
    static const hipError_t attr = [] {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_bf16_kernel<kGemmPlain, true>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kGemmLds);
        if (e == hipSuccess)
            e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_bf16_kernel<kGemmGateUp, true>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, kGemmLds);
        return e;
    }();
    if (attr != hipSuccess) return attr;
    const uint32_t cols = mode == kGemmGateUp ? 2 * g.N : g.N;
    const dim3 grid((cols + kBN - 1) / kBN * g.max_tiles);
    if (mode == kGemmGateUp) return vlaunch(gemm_bf16_kernel<kGemmGateUp, true>, grid, dim3(kGemmThreads), kGemmLds, s, g);
    return vlaunch(gemm_bf16_kernel<kGemmPlain, true>, grid, dim3(kGemmThreads), kGemmLds, s, g);
}

hipError_t launch_row_rms(float* x, uint32_t n, uint32_t rows, float eps, float* scale, hipStream_t s,
                          const float* part, uint32_t splits) {
    if (n % 4 != 0) return hipErrorInvalidValue;
    if (part && splits > kMaxPartSplits) return hipErrorInvalidValue;
    if (part && splits > 1)  // a block per row: the partial sums are splits x the row's bytes
        return vlaunch(row_rms_part_kernel, dim3(rows), dim3(kRowThreads), 0, s, x, n, rows, eps, scale, part,
                       splits);
    const uint32_t waves_per_block = kRowThreads / 64;
    return vlaunch(row_rms_kernel, dim3((rows + waves_per_block - 1) / waves_per_block), dim3(kRowThreads), 0, s, x,
                   n, rows, eps, scale, nullptr, 0u);
}

bool row_norm_split_fits(uint32_t n) {
    return n % 8 == 0 && gemm_kp(n) / 8 <= static_cast<uint32_t>(kNormSplitMaxGroups * kRowThreads);
}

hipError_t launch_row_norm_split(float* x, uint32_t n, uint32_t rows, float eps, const uint16_t* norm_w,
                                 const float* part, uint32_t splits, uint16_t* a_hl, size_t a_plane, hipStream_t s) {
    if (!row_norm_split_fits(n) || !norm_w || !a_hl || a_plane < static_cast<size_t>(rows) * gemm_kp(n) ||
        (part && splits > kMaxPartSplits))
        return hipErrorInvalidValue;
    return vlaunch(row_norm_split_kernel, dim3(rows), dim3(kRowThreads), 0, s, x, n, rows, eps, norm_w,
                   splits > 1 ? part : nullptr, splits, a_hl, a_plane);
}

hipError_t launch_prefill_embed(const uint16_t* embed, const uint32_t* tokens, uint32_t rows, uint32_t hidden,
                                float* x, hipStream_t s) {
    return vlaunch(prefill_embed_kernel, dim3((hidden + kRowThreads - 1) / kRowThreads, rows), dim3(kRowThreads), 0,
                   s, embed, tokens, hidden, x);
}

hipError_t launch_prefill_rope_kv(const PrefillRopeArgs& a, hipStream_t s) {
    if ((a.q_norm == nullptr) != (a.k_norm == nullptr)) return hipErrorInvalidValue;
    if (a.kv_pack && (a.kv_pack_bytes < prefill_kv_pack_bytes(a.start + a.rows, a.kv_heads, a.hd) ||
                      prefill_kv_pack_bytes(a.start + a.rows, a.kv_heads, a.hd) == 0 || a.kvdim != a.kv_heads * a.hd))
        return hipErrorInvalidValue;
    if (a.part && (a.splits < 2 || a.splits > kMaxPartSplits || a.ld % 4 != 0)) return hipErrorInvalidValue;
    return vlaunch(prefill_rope_kv_kernel, dim3(a.rows), dim3(kRowThreads), 0, s, a);
}

hipError_t launch_prefill_attn(const PrefillAttnArgs& a, uint32_t hd, hipStream_t s) {
    if (a.rows == 0) return hipSuccess;
    if (!prefill_attn_vector) {
        const uint32_t G = a.heads / a.kv_heads;
        if (G == 0 || G > static_cast<uint32_t>(kFaVecs)) return hipErrorInvalidValue;
        const uint32_t keys = a.start + a.rows;
        const size_t need = prefill_kv_pack_bytes(keys, a.kv_heads, hd);
        if (need == 0 || !a.kv_pack || a.kv_pack_bytes < need) return hipErrorInvalidValue;
        if (a.out_hl && a.out_plane < static_cast<size_t>(a.rows) * a.heads * hd) return hipErrorInvalidValue;
        PrefillAttnArgs b = a;
        b.kv_tiles = (keys + fa_tile_keys(hd) - 1) / fa_tile_keys(hd);
        // Blocks of 64 query vectors with two key groups while they fit one
        // round of the CUs (one block of 4 waves per CU), else blocks of 128
        // with two key groups up to two rounds, else one key group (two
        // blocks per CU). Measured at Llama-3.2-1B / Qwen2.5-7B, whole
        // prefill against one key group throughout: 512 rows -2.0 / -1.3 %,
        // 1024 rows -2.0 %, 2048 rows -1.4 / -1.4 %.
        const uint32_t cus = gemm_cus();
        const uint32_t blocks4 = (a.rows + kFaVecs / G - 1) / (kFaVecs / G) * a.kv_heads;
        const uint32_t rows2 = 64 / G;
        const uint32_t blocks2 = rows2 ? (a.rows + rows2 - 1) / rows2 * a.kv_heads : 0;
        const int forced = prefill_fa_form.load(std::memory_order_relaxed);
        const int f = forced >= 0 ? forced : (rows2 && blocks2 <= cus ? 2 : (blocks4 <= 2 * cus ? 1 : 0));
        if (f == 2 && !rows2) return hipErrorInvalidValue;
        // Tiles holding rows before `start` (all tiles unless the RoPE / KV
        // pass wrote the new rows' images).
        const uint32_t tk = fa_tile_keys(hd);
        const dim3 pack(a.new_rows_packed ? (a.start + tk - 1) / tk : b.kv_tiles, a.kv_heads);
        const dim3 grid(f == 2 ? blocks2 : blocks4), blk(f == 0 ? 256 : 512);
        hipError_t e;
        switch (hd) {
            case 32:
                e = pack.x ? vlaunch(prefill_kv_pack_kernel<32>, pack, dim3(256), 0, s, b) : hipSuccess;
                if (e != hipSuccess) return e;
                if (f == 0) return vlaunch(prefill_fa_kernel<32, 4, 1>, grid, blk, 0, s, b);
                if (f == 1) return vlaunch(prefill_fa_kernel<32, 4, 2>, grid, dim3(512), 0, s, b);
                return vlaunch(prefill_fa_kernel<32, 2, 2>, grid, dim3(256), 0, s, b);
            case 64:
                e = pack.x ? vlaunch(prefill_kv_pack_kernel<64>, pack, dim3(256), 0, s, b) : hipSuccess;
                if (e != hipSuccess) return e;
                if (f == 0) return vlaunch(prefill_fa_kernel<64, 4, 1>, grid, blk, 0, s, b);
                if (f == 1) return vlaunch(prefill_fa_kernel<64, 4, 2>, grid, dim3(512), 0, s, b);
                return vlaunch(prefill_fa_kernel<64, 2, 2>, grid, dim3(256), 0, s, b);
            case 128:
                e = pack.x ? vlaunch(prefill_kv_pack_kernel<128>, pack, dim3(256), 0, s, b) : hipSuccess;
                if (e != hipSuccess) return e;
                if (f == 0) return vlaunch(prefill_fa_kernel<128, 4, 1>, grid, blk, 0, s, b);
                if (f == 1) return vlaunch(prefill_fa_kernel<128, 4, 2>, grid, dim3(512), 0, s, b);
                return vlaunch(prefill_fa_kernel<128, 2, 2>, grid, dim3(256), 0, s, b);
            default: return hipErrorInvalidValue;
        }
    }
    const uint32_t G = a.heads / a.kv_heads;
    if (G == 0 || G > static_cast<uint32_t>(kPairsPerWave) || a.out_hl) return hipErrorInvalidValue;  // f32 out only
    const uint32_t rows_per_wave = kPairsPerWave / G;
    const uint32_t items = (a.rows + rows_per_wave - 1) / rows_per_wave * a.kv_heads;
    const dim3 grid((items + kAttnThreads / 64 - 1) / (kAttnThreads / 64));
    switch (hd) {
        case 32: return vlaunch(prefill_attn_kernel<32>, grid, dim3(kAttnThreads), 0, s, a);
        case 64: return vlaunch(prefill_attn_kernel<64>, grid, dim3(kAttnThreads), 0, s, a);
        case 128: return vlaunch(prefill_attn_kernel<128>, grid, dim3(kAttnThreads), 0, s, a);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace vvli
