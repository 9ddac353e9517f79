// decode_step.hip -- persistent decode step for gfx950: one cooperative launch
// runs whole token steps (Runner.forwardToken, src/llm.zig:702-766, plus
// llm.argmax, :778-789), optionally many in a row (the decode loop of
// generateGreedyMeasured, src/generator.zig:243-281).
//
// Why: at batch 1 every layer is five dependent, HBM-bound phases (q/k/v
// GEMV, attention, o GEMV, gate/up GEMV, down GEMV). As separate kernels each
// pays launch, ramp and drain; here they are phases of one kernel, and every
// wave issues the weight loads of its first tile of the next phase before it
// waits for that phase's input.
//
// Dataflow instead of grid barriers: every activation that crosses blocks is
// an array of 64-bit tagged words, value bits in the low half and the epoch of
// the phase that wrote it in the high half, stored and loaded with single
// agent-scope 64-bit accesses (gfx950: sc1, coherent across the per-XCD L2s).
// A consumer polls exactly the words it needs until each carries the epoch it
// expects, so a phase boundary costs one store->load hop instead of a flag
// barrier plus a separate load of the data, and nobody waits for a store
// acknowledgement. Epochs grow monotonically over launches (the host passes
// the first one), so buffers never need clearing between steps.
//
// Why a word is never overwritten before every reader has it: a phase only
// reads inputs if it produces outputs, and the next write of any buffer lies
// downstream (through the dependency chain of later phases) of every output of
// the phases that read it. A block with no work in a phase skips its input.
//
// KV rows: the attention unit that owns position pos appends its K/V row with
// agent-scope stores and waits for their acknowledgement before it publishes
// the attention output; later steps read rows with plain loads (a row is never
// read before it is written within a launch, and a launch starts with clean
// caches).
//
// Deadlock safety: the launch is cooperative (all blocks co-resident or the
// launch fails), every poll is bounded, and a timeout raises a device error
// flag that makes every block leave at its next poll; the host reports it.
#include <algorithm>
#include <cstdlib>

#include "device_common.hpp"
#include "gemv_tile.hpp"
#include "kernels.hpp"
#include "moe_route.hpp"

namespace vvli {

namespace {

constexpr int kMkThreads = 512;
constexpr int kMkWaves = kMkThreads / kWave;
constexpr int kMaxGroupMk = 16;
constexpr int kMaxSplitMk = 64;  // attention splits per kv head
// Delay of the gate/up LDS copies after the q/k/v words appear: two
// s_sleep of 64 x kGldsSleep cycles, ~1.5 us at the 2.2 GHz shader clock
// of a decode step. Measured best near 1.5 us (Llama-3.2-1B 1315 -> 1331
// tok/s, Qwen2.5-0.5B 1259 -> 1278; delays of 0.5, 1, 2 and 3 us gave
// 1322, 1329, 1328, 1320 at Llama-3.2-1B).
constexpr int kGldsSleep = 26;
constexpr int kOwnerMergeMax = 16;  // splits merged by one block (the one that appends the K/V row)
static_assert(kMaxSplitMk <= 64, "the split merge weights are one wave's lanes");
constexpr uint32_t kSpinLimit = 1u << 22;  // polls of one word (each after a short sleep): seconds

typedef unsigned long long tword;

__device__ __forceinline__ float ld_a(const float* p) {
    return __hip_atomic_load(as_global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_a(const uint32_t* p) {
    return __hip_atomic_load(as_global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ tword ld_a(const tword* p) {
    return __hip_atomic_load(as_global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_a(float* p, float v) {
    __hip_atomic_store(as_global(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_a(uint32_t* p, uint32_t v) {
    __hip_atomic_store(as_global(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_a(tword* p, tword v) {
    __hip_atomic_store(as_global(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Pinned host memory (vector store at system scope).
__device__ __forceinline__ void st_sys(uint32_t* p, uint32_t v) {
    __hip_atomic_store(as_global(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void st_sys(float* p, float v) {
    __hip_atomic_store(as_global(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint32_t ld_sys(const uint32_t* p) {
    return __hip_atomic_load(as_global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void wait_all_mem() { __builtin_amdgcn_s_waitcnt(0); }

__device__ __forceinline__ tword tw_make(float v, uint32_t tag) {
    return ((tword)tag << 32) | (tword)__float_as_uint(v);
}
__device__ __forceinline__ tword tw_make_u(uint32_t v, uint32_t tag) { return ((tword)tag << 32) | (tword)v; }
__device__ __forceinline__ float tw_val(tword w) { return __uint_as_float((uint32_t)w); }
__device__ __forceinline__ uint32_t tw_tag(tword w) { return (uint32_t)(w >> 32); }

// 16-byte loads (two tagged words) that see other XCDs' agent-scope stores:
// buffer loads with the sc1 cache policy, through a raw buffer resource
// (out-of-range reads return 0).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef float mk_f32x4 __attribute__((ext_vector_type(4)));
constexpr int kCpolSc1 = 16;
constexpr int kCpolNt = 2;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coh_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float4 ld_coh4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCpolSc1);
    return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
__device__ __forceinline__ void ld_coh_tw2(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, tword& a, tword& b) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCpolSc1);
    a = ((tword)v.y << 32) | v.x;
    b = ((tword)v.w << 32) | v.z;
}

// Wait until *p carries `tag` (w holds a first load). False: the spin limit
// passed (the error flag is raised) or another block raised it.
__device__ __forceinline__ bool poll_tw(const tword* p, uint32_t tag, tword& w, uint32_t* err) {
    uint32_t spins = 0;
    while (tw_tag(w) != tag) {
        if (++spins > kSpinLimit) {
            st_a(err, kDecodeErrTimeout);
            return false;
        }
        if ((spins & 63u) == 0 && ld_a(err) != 0) return false;
        __builtin_amdgcn_s_sleep(1);
        w = ld_a(p);
    }
    return true;
}

// Wait until both words carry `tag`: a retry reloads both (a word that is
// there stays there until its reader is done), so the pair costs one memory
// round trip after its later word lands.
__device__ __forceinline__ bool poll_tw2(const tword* p0, const tword* p1, uint32_t tag, tword& w0, tword& w1,
                                         uint32_t* err) {
    uint32_t spins = 0;
    while (tw_tag(w0) != tag || tw_tag(w1) != tag) {
        if (++spins > kSpinLimit) {
            st_a(err, kDecodeErrTimeout);
            return false;
        }
        if ((spins & 63u) == 0 && ld_a(err) != 0) return false;
        __builtin_amdgcn_s_sleep(1);
        w0 = ld_a(p0);
        w1 = ld_a(p1);
    }
    return true;
}

// Detail timing mark (16-slot timing only): slot 0 the block's staged input,
// 1 + w wave w's end of the phase; slots 9-11 (thread 0 in the input staging):
// its entry, the return of its first attempt, its retry count; 12, 13 (thread
// 0): past the phase's closing barrier, past the next phase's weight issue;
// 14, 15 (thread 0, MoE gate/up): routed, its router row published (producers).
// Attention units: 9 q (and the new k / v) in LDS, 10 the split's pass done,
// 11 its partials stored, 14 the partials it merges polled, 15 merge weights
// computed (and the K/V row stores acknowledged), 0 its merged outputs
// published (a split that stores partials for another to merge: 9-11 only).
__device__ __forceinline__ void mk_mark(const DecodeStepParams& p, uint32_t ph, int slot) {
    if (p.timing && p.timing_slots == 16 && (ph + 1) * 16 <= p.timing_stride)
        p.timing[blockIdx.x * p.timing_stride + ph * p.timing_slots + slot] = __builtin_amdgcn_s_memrealtime();
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
__device__ __forceinline__ tword* seg_out(const MkGemv& g, int seg) { return seg == 0 ? g.o0 : (seg == 1 ? g.o1 : g.o2); }

struct MkTile {
    const uint16_t* p[2];  // weight rows streamed by this tile
    uint32_t row[2];       // output rows (row[1] unused in the SwiGLU mode)
    int seg;               // segment of both rows (q | k | v in the plain mode)
    bool valid[2];         // output row exists
};

template <bool MOE = false>
__device__ __forceinline__ uint32_t mk_tiles(const MkGemv& g, int mode) {
    const uint32_t total = g.r0 + g.r1 + g.r2;
    if constexpr (MOE) {
        if (g.moe == 2) return total;  // MoE down: one output row per tile
    }
    return (mode == kGemvGateUp || g.split) ? total : (total + 1) / 2;
}

// Units (8 weights) streamed per tile row: a split tile streams half rows.
__device__ __forceinline__ uint32_t mk_units(const MkGemv& g) { return g.split ? g.K / 16 : g.K / 8; }

// Tile `tile`: gate row t and up row t (SwiGLU), else rows 2t, 2t+1 of the
// stacked segments (segments hold an even number of rows, so a tile never
// straddles two; an odd last row re-reads its own row as the second).
// MOE phases take the expert of a slot from ex (LDS): gate/up tile t is row
// t % r_slot of slot t / r_slot's expert; down tile t is output row t, its
// item `slot` streams that row of the experts of slots 2 slot and 2 slot + 1
// (p[0], p[1]; an odd last pair repeats its first slot).
template <bool MOE = false>
__device__ __forceinline__ void mk_make_tile(const MkGemv& g, int mode, uint32_t tile, MkTile& t, uint32_t slot = 0,
                                             const uint32_t* ex = nullptr) {
    const uint32_t K = g.K;
    if constexpr (MOE) {
        if (g.moe == 1) {
            const bool v = tile < g.r0;
            const uint32_t tt = v ? tile : 0;
            const uint32_t sl = tt / g.r_slot, r = tt - sl * g.r_slot;
            const size_t off = (size_t)ex[sl] * g.w_expert + (size_t)r * K;
            t.p[0] = g.w0 + off;
            t.p[1] = g.w_up + off;
            t.row[0] = t.row[1] = tt;
            t.seg = 0;
            t.valid[0] = v;
            t.valid[1] = false;
            return;
        }
        if (g.moe == 2) {
            const uint32_t s0 = 2 * slot, s1 = s0 + 1 < g.r_slot ? s0 + 1 : s0;
            const bool v = tile < g.r0;
            const size_t r = v ? tile : 0;
            t.p[0] = g.w0 + (size_t)ex[s0] * g.w_expert + r * K;
            t.p[1] = g.w0 + (size_t)ex[s1] * g.w_expert + r * K;
            t.row[0] = t.row[1] = (uint32_t)r;
            t.seg = 0;
            t.valid[0] = v;
            t.valid[1] = false;
            return;
        }
    }
    if (g.split) {  // row t: first half in p[0], second half in p[1]
        const bool v = tile < g.r0;
        const uint32_t r = v ? tile : 0;
        t.p[0] = g.w0 + (size_t)r * K;
        t.p[1] = t.p[0] + K / 2;
        t.row[0] = t.row[1] = r;
        t.seg = 0;
        t.valid[0] = v;
        t.valid[1] = false;
    } else if (mode == kGemvGateUp) {
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
    uint32_t wid;    // wave (t mod blocks) ... : tile t goes to block t mod blocks
    uint32_t nw;
    uint32_t wave;   // wave of the block
    int lane;
};

// Wave index that owns tiles wid, wid + nw, ... of a phase with `ntiles` tiles:
// consecutive tiles go to consecutive blocks, so a phase with fewer tiles than
// waves still uses every CU and the tiles of a partial last round spread over
// all blocks (one more tile for some waves, never a whole block's waves more).
// Block b owns a tile of the phase iff b < ntiles (b - fb < ntiles for a wave
// from mk_wave_from(w, fb)).
__device__ __forceinline__ uint32_t mk_owner(const MkWave& w, uint32_t ntiles) {
    (void)ntiles;
    return w.wid;
}

// The wave as a phase sees it whose tiles run on blocks [fb, grid) only
// (blocks below fb own none).
__device__ __forceinline__ MkWave mk_wave_from(const MkWave& w, uint32_t fb) {
    if (fb == 0) return w;
    MkWave v = w;
    const uint32_t nb = gridDim.x - fb;
    v.nw = nb * kMkWaves;
    if (blockIdx.x < fb) {
        v.wid = 0xffffffffu;
    } else {
        v.wid = w.wave * nb + (blockIdx.x - fb);
    }
    return v;
}

// Issue the first item of this wave's first tile (weights only: may run
// before the phase input exists). Defines buf and t on every path, so they are
// dead between a phase's last item and the next prefetch.
template <bool MOE = false>
__device__ __forceinline__ bool mk_prefetch(const MkGemv& g, int mode, const MkWave& w, uint4 (&buf)[2][kNJC],
                                            MkTile& t, uint32_t t0 = 0, const uint32_t* ex = nullptr) {
    const uint32_t ntiles = mk_tiles<MOE>(g, mode) - t0;
    const uint32_t me = mk_owner(w, ntiles);
    mk_make_tile<MOE>(g, mode, t0 + (me < ntiles ? me : 0), t, 0, ex);
    if (me >= ntiles) {
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int j = 0; j < kNJC; ++j) buf[r][j] = make_uint4(0, 0, 0, 0);
        return false;
    }
    issue<uint16_t, 2>(buf, t.p, 0, mk_units(g), w.lane);
    return true;
}


// Where a residual-mode phase takes its residual rows: tagged words of an
// earlier phase, or (layer 0) the bf16 embedding row of the token.
struct MkResid {
    const tword* src;
    uint32_t tag;
    const uint16_t* bf16;
};

// acc[r] += W_r . x_r over one item's units: row 0 against xs0, row 1
// against xs1 (the same vector unless the tile holds a split row).
__device__ __forceinline__ void consume_rows(const uint4 (&buf)[2][kNJC], const float* xs0, const float* xs1,
                                             uint32_t ubase, uint32_t U, int lane, float (&acc)[2]) {
    if (xs1 == xs0) {  // two rows against one x: load x once
        consume<uint16_t, 2>(buf, xs0, ubase, U, lane, acc);
        return;
    }
#pragma unroll
    for (int j = 0; j < kNJC; ++j) {
        const uint32_t u = ubase + j * kWave + lane;
        if (u < U) {
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const float* xr = (r == 0 ? xs0 : xs1) + (size_t)u * 8;
                const float4 x0 = *reinterpret_cast<const float4*>(xr);
                const float4 x1 = *reinterpret_cast<const float4*>(xr + 4);
                const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                float wf[8];
                WeightTraits<uint16_t>::expand(buf[r][j], wf);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[r] = fmaf(wf[e], xv[e], acc[r]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Gate/up tiles in LDS. The attention phase leaves most blocks idle (only
// kv_heads * splits units run) and HBM nearly so; those blocks copy the first
// gate/up tiles of the layer into LDS (global_load_lds, 1 KiB per wave load)
// and the gate/up phase takes them from there, so it streams fewer bytes
// after its input arrives. Tiles [0, n) of the phase are LDS tiles: block
// first_block + i holds tiles i*per_block .. +per_block-1, tile i*per_block+j
// belongs to wave j mod 8 of the block (it loads and consumes it, so only its
// own completion counter orders the copy and the reads). The remaining tiles
// are streamed by every wave as usual.
// LDS tile layout: [row (gate, up)][chunk][j < kNJC][lane] 16-byte units,
// i.e. exactly the registers an item would hold.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;

struct GLds {
    uint32_t first_block;  // blocks >= first_block hold LDS tiles
    uint32_t per_block;
    uint32_t n;            // LDS tiles of the phase
    uint32_t nchunk;       // items per row
    uint32_t tile_bytes;
    uint32_t per1;         // tiles of the first LDS range
    uint32_t off1, off2;   // byte offsets of the two ranges in the dynamic LDS
};

// Byte offset (dynamic LDS) of the block's j-th tile.
__device__ __forceinline__ uint32_t mk_glds_tile(const GLds& q, uint32_t j) {
    return j < q.per1 ? q.off1 + j * q.tile_bytes : q.off2 + (j - q.per1) * q.tile_bytes;
}

__device__ __forceinline__ GLds mk_glds(const DecodeStepParams& p, uint32_t units, const MkGemv& g, bool on = true) {
    GLds q;
    q.first_block = units < gridDim.x ? units : gridDim.x;
    q.per_block = on ? p.g_lds_tiles : 0;
    const uint32_t cap = (gridDim.x - q.first_block) * q.per_block;
    q.n = cap < g.r0 ? cap : g.r0;
    q.nchunk = (g.K / 8 + kNJC * kWave - 1) / (kNJC * kWave);
    q.tile_bytes = 2 * q.nchunk * kNJC * kWave * 16;
    q.per1 = p.g_lds_tiles1;
    q.off1 = p.g_lds_offset1;
    q.off2 = p.g_lds_offset2;
    return q;
}

// LDS tiles of this wave: j = wave, wave + 8, ... while j < per_block and the
// tile index is < n.
__device__ __forceinline__ uint32_t mk_glds_count(const GLds& q, uint32_t wave) {
    if (q.n == 0 || blockIdx.x < q.first_block) return 0;
    const uint32_t t0 = (blockIdx.x - q.first_block) * q.per_block;
    if (t0 >= q.n) return 0;
    const uint32_t lim = q.n - t0 < q.per_block ? q.n - t0 : q.per_block;
    if (wave >= lim) return 0;
    return (lim - 1 - wave) / kMkWaves + 1;
}

__device__ __forceinline__ void mk_glds_issue(const GLds& q, const MkGemv& g, char* lds, uint32_t wave, int lane) {
    const uint32_t cnt = mk_glds_count(q, wave);
    const uint32_t U = g.K / 8;
    for (uint32_t k = 0; k < cnt; ++k) {
        const uint32_t j = wave + k * kMkWaves;
        const uint32_t t = (blockIdx.x - q.first_block) * q.per_block + j;
        char* dst = lds + mk_glds_tile(q, j);
        const uint16_t* gate = g.w0 + (size_t)t * g.K;
        const uint16_t* up = g.w_up + (size_t)t * g.K;
        for (uint32_t rc = 0; rc < 2 * q.nchunk; ++rc) {
            const uint16_t* row = rc < q.nchunk ? gate : up;
            const uint32_t c = rc < q.nchunk ? rc : rc - q.nchunk;
#pragma unroll
            for (int jj = 0; jj < kNJC; ++jj) {
                const uint32_t u = c * (kNJC * kWave) + jj * kWave + lane;
                // (nontemporal, like every weight stream: 1356 -> 1369 tok/s at
                // Llama-3.2-1B, 1305 -> 1331 at Qwen2.5-0.5B)
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(row + (size_t)(u < U ? u : 0) * 8),
                                                 (lds_void_t*)(dst + (rc * kNJC + jj) * kWave * 16), 16, 0, kCpolNt);
            }
        }
    }
}

// The wave's LDS gate/up tiles: silu(gate . x) * (up . x) of its k-th tile
// parked at park[k] in LDS (written out by mk_gemv once the streamed tiles
// are done, so no store sits in front of the streamed loads).
__device__ __forceinline__ void mk_glds_compute(const GLds& gl, const MkGemv& g, const float* xs, char* lds,
                                                uint32_t park_off, const MkWave& w) {
    const uint32_t n = mk_glds_count(gl, w.wave);
    const uint32_t U = g.K / 8;
    for (uint32_t k = 0; k < n; ++k) {
        const char* src = lds + mk_glds_tile(gl, w.wave + k * kMkWaves) + w.lane * 16;
        float acc[2] = {0.f, 0.f};
        for (uint32_t c = 0; c < gl.nchunk; ++c) {
            uint4 lb[2][kNJC];
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int jj = 0; jj < kNJC; ++jj)
                    lb[r][jj] = *reinterpret_cast<const uint4*>(src + (((size_t)r * gl.nchunk + c) * kNJC + jj) *
                                                                          kWave * 16);
            consume<uint16_t, 2>(lb, xs, c * kNJC * kWave, U, w.lane, acc);
        }
        const float v0 = wave_sum(acc[0]), v1 = wave_sum(acc[1]);
        if (w.lane == 0)  // siluMulInto, src/llm.zig:1382-1387
            reinterpret_cast<float*>(lds + park_off)[w.wave * kWave + k] = (v0 / (1.0f + expf(-v0))) * v1;
    }
}


// Run this wave's tiles of a GEMV phase (`mode` is uniform over the grid),
// among the phase's tiles t0 .. end (t0 > 0: the first ones were taken from
// LDS); bufA/tA hold the prefetched first item when `have` is set. Outputs are
// tagged with `tag` (logits: plain floats plus the argmax key in `best`).
//
// Tile results are parked in lanes -- lane k holds the k-th tile of the
// current batch of 64 -- and written with one vector store per batch: on gfx9
// loads and stores share one completion counter, so a store per tile would
// make every following weight wait for that store's acknowledgement. Each lane
// also loads its tile's addend (residual row or bias) when the batch opens and
// checks the residual's tag only when it writes. dbg (nullable): a second
// destination of the outputs -- the residual rows after the layer (parity
// dumps) -- or, in the logits phase with WT, a flag: the logits are written
// through (every block then copies a slice of them to host memory).
// MOE down phase (g.moe == 2): a tile (one output row) has an item per pair
// of slots (and chunk of the row); slots s, s + 1 multiply their experts'
// rows with xs + s * K and xs + (s + 1) * K and add wsl[s], wsl[s + 1] times
// the dot products, per lane, before the wave sum.
template <bool MOE = false, bool WT = false>
__device__ __forceinline__ bool mk_gemv(const MkGemv& g, int mode, const float* xs, const MkWave& w,
                                        uint4 (&bufA)[2][kNJC], MkTile& tA, bool have, unsigned long long& best,
                                        uint32_t tag, const MkResid& rs, uint32_t t0, const float* park,
                                        uint32_t lds_first, uint32_t n_lds, uint32_t* err, float* dbg,
                                        const uint32_t* ex = nullptr, const float* wsl = nullptr) {
    const int lane = w.lane;
    const uint32_t U = mk_units(g);
    const uint32_t per_item = kNJC * kWave;
    const float* xs1 = g.split ? xs + g.K / 2 : xs;  // x of the second streamed row
    const uint32_t cps = (U + per_item - 1) / per_item;  // items per row
    bool md = false;
    if constexpr (MOE) md = g.moe == 2;
    const uint32_t npair = md ? (g.r_slot + 1) / 2 : 1;
    const uint32_t nchunk = cps * npair;
    const uint32_t ntiles = mk_tiles<MOE>(g, mode) - t0;
    const uint32_t me = mk_owner(w, ntiles);
    const uint32_t my_tiles = me < ntiles ? (ntiles - 1 - me) / w.nw + 1 : 0;
    const uint32_t n_items = my_tiles * nchunk;
    bool ok = true;
    if (n_items) {
        if (!have) {
            mk_make_tile<MOE>(g, mode, t0 + me, tA, 0, ex);
            issue<uint16_t, 2>(bufA, tA.p, 0, U, lane);
        }
        // Lane state of the open batch: rows, segment, addends, parked results.
        uint32_t ra = 0, rb = 0;
        int sa = 0;
        bool va = false, vb = false;
        tword wa = 0, wb = 0;  // residual words (tag checked at write time)
        float ea = 0.f, eb = 0.f, oa = 0.f, ob = 0.f;
        uint32_t base = 0, pending = 0;
        auto open_batch = [&]() {
            const uint32_t k = base + (uint32_t)lane;
            const bool mine = k < my_tiles;
            MkTile t;
            mk_make_tile<MOE>(g, mode, t0 + (mine ? me + k * w.nw : me), t, 0, ex);
            ra = t.row[0];
            rb = t.row[1];
            sa = t.seg;
            va = mine && t.valid[0];
            vb = mine && t.valid[1];
            ea = eb = 0.f;
            if (mode == kGemvResid) {  // x = residual + proj (addInto, src/llm.zig:1389-1396)
                if (rs.bf16) {
                    if (va) ea = __uint_as_float((uint32_t)*as_global(rs.bf16 + ra) << 16);
                    if (vb) eb = __uint_as_float((uint32_t)*as_global(rs.bf16 + rb) << 16);
                } else {
                    wa = va ? ld_a(rs.src + ra) : tw_make_u(0, rs.tag);
                    wb = vb ? ld_a(rs.src + rb) : tw_make_u(0, rs.tag);
                }
            } else if (mode == kGemvPlain) {  // linearRange: dot + bias (src/llm.zig:1273)
                const uint16_t* bias = seg_bias(g, sa);
                if (bias && va) ea = __uint_as_float((uint32_t)*as_global(bias + ra) << 16);
                if (bias && vb) eb = __uint_as_float((uint32_t)*as_global(bias + rb) << 16);
            }
        };
        auto flush = [&]() {
            if ((uint32_t)lane < pending) {
                if (mode == kGemvLogits) {
                    if (WT && dbg) {  // written through, for the copy to host memory (resident single steps)
                        if (va) st_a(g.plain + ra, oa);
                        if (vb) st_a(g.plain + rb, ob);
                    } else {
                        if (va) *as_global(g.plain + ra) = oa;
                        if (vb) *as_global(g.plain + rb) = ob;
                    }
                } else {
                    if (mode == kGemvResid && !rs.bf16) {
                        ok = ok && poll_tw(rs.src + ra, rs.tag, wa, err) && poll_tw(rs.src + rb, rs.tag, wb, err);
                        ea = tw_val(wa);
                        eb = tw_val(wb);
                    }
                    tword* o = mode == kGemvPlain ? seg_out(g, sa) : g.o0;
                    if (va) st_a(o + ra, tw_make(oa + ea, tag));
                    if (vb) st_a(o + rb, tw_make(ob + eb, tag));
                    if (dbg) {  // residual stream after the layer (parity dumps only)
                        if (va) dbg[ra] = oa + ea;
                        if (vb) dbg[rb] = ob + eb;
                    }
                }
            }
            pending = 0;
        };
        open_batch();
        uint4 bufB[2][kNJC];
        MkTile tc = tA, tn = tA;  // tiles of the item being consumed / in flight
        float acc0 = 0.f, acc1 = 0.f;
        float tot0 = 0.f;  // MOE down: router-weighted sum over the slots
        // The tile of the consumed item (tc) is complete: reduce, epilogue,
        // park the result in its lane, write a full batch.
        auto end_tile = [&]() {
            float v0, v1 = 0.f;
            if (g.split) {
                v0 = wave_sum(acc0 + acc1);  // the row's two halves
            } else {
                v0 = wave_sum(acc0);
                v1 = wave_sum(acc1);
            }
            acc0 = acc1 = 0.f;
            if (mode == kGemvGateUp) {
                v0 = (v0 / (1.0f + expf(-v0))) * v1;  // siluMulInto, src/llm.zig:1382-1387
            } else if (mode == kGemvLogits && lane == 0) {
                // llm.argmax (src/llm.zig:778-789): a NaN logit 0 makes the
                // result 0 (every comparison with it fails): top key, index 0.
                if (tc.valid[0]) {
                    const unsigned long long k0 =
                        (tc.row[0] == 0 && v0 != v0) ? ~0ull : argmax_key(v0, tc.row[0]);
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
        };
        for (uint32_t it = 0; it < n_items; ++it) {
            const uint32_t chunk = it % nchunk;
            const bool more = it + 1 < n_items;
            const uint32_t nchunk_next = chunk == nchunk - 1 ? 0 : chunk + 1;
            if (more && chunk == nchunk - 1)
                mk_make_tile<MOE>(g, mode, t0 + me + ((it + 1) / nchunk) * w.nw, tn, 0, ex);
            uint32_t nbase = nchunk_next * per_item, ubase = chunk * per_item;
            const float* xa = xs;
            const float* xb = xs1;
            if constexpr (MOE) {
                if (md) {
                    if (more && nchunk_next != 0 && nchunk_next % cps == 0)  // next slot pair of the same tile
                        mk_make_tile<MOE>(g, mode, t0 + me + (it / nchunk) * w.nw, tn, nchunk_next / cps, ex);
                    nbase = (nchunk_next % cps) * per_item;
                    ubase = (chunk % cps) * per_item;
                    const uint32_t s0 = 2 * (chunk / cps), s1 = s0 + 1 < g.r_slot ? s0 + 1 : s0;
                    xa = xs + (size_t)s0 * g.K;
                    xb = xs + (size_t)s1 * g.K;
                }
            }
            float acc[2] = {acc0, acc1};
            if (it & 1) {
                if (more) issue<uint16_t, 2>(bufA, tn.p, nbase, U, lane);
                consume_rows(bufB, xa, xb, ubase, U, lane, acc);
            } else {
                if (more) issue<uint16_t, 2>(bufB, tn.p, nbase, U, lane);
                consume_rows(bufA, xa, xb, ubase, U, lane, acc);
            }
            acc0 = acc[0];
            acc1 = acc[1];
            if constexpr (MOE) {
                if (md && chunk % cps == cps - 1) {  // end of a slot pair's rows
                    const uint32_t s0 = 2 * (chunk / cps);
                    tot0 = fmaf(wsl[s0], acc0, tot0);
                    if (s0 + 1 < g.r_slot) tot0 = fmaf(wsl[s0 + 1], acc1, tot0);
                    acc0 = acc1 = 0.f;
                    if (chunk == nchunk - 1) {
                        acc0 = tot0;
                        tot0 = 0.f;
                    }
                }
            }
            if (chunk == nchunk - 1) {
                end_tile();
                tc = tn;
            }
        }
        flush();
    }
    // Results of the wave's LDS tiles (gate/up phase), parked in LDS: written
    // after the streamed tiles, so no store sits in front of their loads.
    if ((uint32_t)lane < n_lds)
        st_a(g.o0 + lds_first + (uint32_t)lane * kMkWaves, tw_make(park[w.wave * kWave + lane], tag));
    return ok;
}

// ---------------------------------------------------------------------------
// Input staging into LDS.
// ---------------------------------------------------------------------------
// xs[k] = src[k] (* norm_w[k] * s) with s = 1/sqrt(mean(src^2) + eps)
// (rmsNormInto, src/llm.zig:1287-1300). src is a tagged activation of phase
// `tag` (polled until every word carries it) or (src_bf16) a bf16 embedding
// row (copyEmbeddingToken, :1373-1380). The norm weights are loaded in the
// same batch as the activation (into nws = xs + n). arrived() runs on every
// thread once its share of the input is in registers, before the block-wide
// normalisation. False: a poll failed.
// The thread index, optionally through an empty asm: the lane-dependent
// addresses derived from it are then formed where the phase runs instead of
// being hoisted to the kernel's start and held (or spilled) across every
// phase. Pinned in the variants that would otherwise spill; the hd-64 exact
// step keeps them hoisted (no spills there, and a shorter staging path).
template <bool kPin>
__device__ __forceinline__ int mk_tid() {
    int tid = threadIdx.x;
    if constexpr (kPin) asm volatile("" : "+v"(tid));
    return tid;
}

template <bool kPin = false, typename F>
__device__ __forceinline__ bool mk_stage(float* xs, float* red, const tword* src, uint32_t tag,
                                         const uint16_t* src_bf16, const uint16_t* norm_w, float eps, uint32_t n,
                                         uint32_t* err, unsigned long long* tmark, F&& arrived) {
    const int tid = mk_tid<kPin>();
    // Detail timing (profiling runs only): thread 0 records its entry, the
    // return of its first attempt, and its retry count.
    if (tmark && tid == 0) tmark[0] = __builtin_amdgcn_s_memrealtime();
    constexpr int B = 8;  // word pairs issued before any is consumed
    float* nws = xs + n;
    float ss = 0.f;
    bool ok = true;
    if (src_bf16) {
        for (uint32_t k = tid; k < n; k += kMkThreads) {
            const float v = __uint_as_float((uint32_t)*as_global(src_bf16 + k) << 16);
            xs[k] = v;
            if (norm_w) nws[k] = __uint_as_float((uint32_t)*as_global(norm_w + k) << 16);
            ss = fmaf(v, v, ss);
        }
    } else {
        const __amdgpu_buffer_rsrc_t r = coh_rsrc(src, n * 8);
        const uint32_t n2 = n / 2;
        // A batch: B word pairs per thread issued together (pairs past n read
        // as zeros), with the norm weights of the same elements.
        auto load_batch = [&](uint32_t i0, tword (&a)[B], tword (&b)[B], uint32_t (&nv)[B]) {
#pragma unroll
            for (int k = 0; k < B; ++k) {
                const uint32_t i = i0 + k * kMkThreads;
                ld_coh_tw2(r, i * 16, a[k], b[k]);
                nv[k] = (norm_w && i < n2) ? *as_global(reinterpret_cast<const uint32_t*>(norm_w + 2 * i)) : 0u;
            }
        };
        auto complete = [&](uint32_t i0, const tword (&a)[B], const tword (&b)[B]) {
            bool done = true;
#pragma unroll
            for (int k = 0; k < B; ++k)
                if (i0 + k * kMkThreads < n2 && (tw_tag(a[k]) != tag || tw_tag(b[k]) != tag)) done = false;
            return done;
        };
        // The batch is polled as a whole: a retry reloads every pair that is
        // not complete, so it ends one round trip after its last word lands
        // (word-by-word polls would add a round trip per late word). The
        // first attempt is straight-line code (no retry loop's back edge
        // merges into its waits). Then the values go to LDS.
        auto finish_batch = [&](uint32_t i0, tword (&a)[B], tword (&b)[B], const uint32_t (&nv)[B]) {
            bool done = complete(i0, a, b);
            if (tmark && tid == 0) tmark[1] = __builtin_amdgcn_s_memrealtime();
            for (uint32_t spins = 0; !done;) {
                if (++spins > kSpinLimit) {
                    st_a(err, kDecodeErrTimeout);
                    ok = false;
                    break;
                }
                if ((spins & 63u) == 0 && ld_a(err) != 0) {
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
                // Every pair is reloaded (a complete word stays as it is until
                // its reader is done).
#pragma unroll
                for (int k = 0; k < B; ++k) ld_coh_tw2(r, (i0 + k * kMkThreads) * 16, a[k], b[k]);
                done = complete(i0, a, b);
                if (tmark && tid == 0) tmark[2] = spins;
            }
#pragma unroll
            for (int k = 0; k < B; ++k) {
                const uint32_t i = i0 + k * kMkThreads;
                if (i < n2) {
                    const float v0 = tw_val(a[k]), v1 = tw_val(b[k]);
                    *reinterpret_cast<float2*>(xs + 2 * i) = make_float2(v0, v1);
                    if (norm_w)
                        *reinterpret_cast<float2*>(nws + 2 * i) =
                            make_float2(__uint_as_float(nv[k] << 16), __uint_as_float(nv[k] & 0xffff0000u));
                    ss = fmaf(v0, v0, ss);
                    ss = fmaf(v1, v1, ss);
                }
            }
        };
        for (uint32_t i0 = tid; i0 < n2; i0 += B * kMkThreads) {
            tword a[B], b[B];
            uint32_t nv[B];
            load_batch(i0, a, b, nv);
            finish_batch(i0, a, b, nv);
        }
    }
    arrived();
    if (__syncthreads_or(!ok)) return false;
    if (norm_w) {
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        float total = 0.f;
#pragma unroll
        for (int i = 0; i < kMkWaves; ++i) total += red[i];
        const float scale = 1.0f / sqrtf(total / (float)n + eps);
        for (uint32_t k = tid; k < n; k += kMkThreads) xs[k] = xs[k] * nws[k] * scale;
        __syncthreads();
    }
    return true;
}

// ---------------------------------------------------------------------------
// Attention phase: units (kv head h, split s) over blocks.
// ---------------------------------------------------------------------------
// LDS layout of the attention phase (floats): q [16][HDMAX], K tile
// [TILE][HDMAX+4] (16-byte aligned rows), V tile [TILE][HDMAX], probabilities
// [16][TILE], new k / v rows, running max / sum / correction per q head, and
// at head_dim 128 the matrix-core tile's partials.
// The merge of the splits reuses the K tile (every split's (m, l) and merge
// weights) and the V tile with the probabilities (the slice's partial values).
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
    // head_dim 128 (matrix-core tile): score partials [kq][jb][16][16],
    // then the P.V slices [js][16][HDMAX]
    static constexpr int kRed = kC + kMaxGroupMk;
    static constexpr int kTotal = kRed + (HDMAX == 128 ? 2048 : 0);
};

// One (kv head, split) unit per block: RoPE of q and of the new k (applyRoPE,
// src/llm.zig:1337-1371), K/V append at pos (:744-745), and an online-softmax
// pass over the split's positions for the `group` q heads sharing the kv head
// (computeAttentionInto, :1302-1335). The splits of a head then merge their
// partials (m, l, acc) into the attention output, each split one slice of it
// (flash-decoding: out = sum_s exp(m_s - M) acc_s / sum_s exp(m_s - M) l_s).
// Every split waits for the others, so the kv_heads * ns units must all hold
// a block at once (the host caps the splits at blocks / kv_heads).
// The K/V rows of the first tile are loaded before q is waited for. EXACT:
// hd == HDMAX (loops fully unrolled), else hd <= HDMAX at run time.
// QK-norm scales (MOE models that carry it): s_q = 1/sqrt(mean(q^2) + eps)
// over the full q, s_k the same over the full k, from the q | k words of
// phase `tag` (polled as one batch per thread, like the input staging).
// Block-uniform; false: a poll failed.
__device__ __forceinline__ bool mk_qk_scales(const DecodeStepParams& p, uint32_t tag, float& scq, float& sck,
                                             float* qk_lds) {
    __shared__ float red2[2][kMkWaves];
    const int tid = mk_tid<true>();  // MoE variants only
    const uint32_t nq = p.heads * p.hd, n2 = (nq + p.kvdim) / 2;  // word pairs of q | k (nq is even)
    const __amdgpu_buffer_rsrc_t r = coh_rsrc(p.tqkv, n2 * 16);
    constexpr int B = 4;
    float sq = 0.f, sk = 0.f;
    bool ok = true;
    for (uint32_t i0 = tid; i0 < n2 && ok; i0 += B * kMkThreads) {
        tword a[B], b[B];
#pragma unroll
        for (int k = 0; k < B; ++k) ld_coh_tw2(r, (i0 + k * kMkThreads) * 16, a[k], b[k]);
        for (uint32_t spins = 0;;) {
            bool done = true;
#pragma unroll
            for (int k = 0; k < B; ++k)
                if (i0 + k * kMkThreads < n2 && (tw_tag(a[k]) != tag || tw_tag(b[k]) != tag)) done = false;
            if (done) break;
            if (++spins > kSpinLimit) {
                st_a(p.error, kDecodeErrTimeout);
                ok = false;
                break;
            }
            if ((spins & 63u) == 0 && ld_a(p.error) != 0) {
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int k = 0; k < B; ++k) ld_coh_tw2(r, (i0 + k * kMkThreads) * 16, a[k], b[k]);
        }
#pragma unroll
        for (int k = 0; k < B; ++k) {
            const uint32_t i = i0 + k * kMkThreads;
            if (i < n2) {
                const float v0 = tw_val(a[k]), v1 = tw_val(b[k]);
                if (qk_lds) *reinterpret_cast<float2*>(qk_lds + 2 * i) = make_float2(v0, v1);
                const float s2 = fmaf(v1, v1, v0 * v0);
                if (2 * i < nq) sq += s2;
                else sk += s2;
            }
        }
    }
    sq = wave_sum(sq);
    sk = wave_sum(sk);
    if ((tid & 63) == 0) red2[0][tid >> 6] = sq, red2[1][tid >> 6] = sk;
    if (__syncthreads_or(!ok)) return false;
    float tq = 0.f, tk = 0.f;
#pragma unroll
    for (int i = 0; i < kMkWaves; ++i) tq += red2[0][i], tk += red2[1][i];
    scq = 1.0f / sqrtf(tq / (float)nq + p.eps);
    sck = 1.0f / sqrtf(tk / (float)p.kvdim + p.eps);
    return true;
}

__device__ __forceinline__ float bf_val(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

template <int HDMAX, bool EXACT, bool MOE = false>
__device__ __forceinline__ bool mk_attention(const DecodeStepParams& p, uint32_t layer, uint32_t pos, uint32_t chunk,
                                             uint32_t ns, float* smem, uint32_t tag_in, uint32_t tag_out,
                                             uint32_t ph) {
    using LY = AttnLds<HDMAX>;
    constexpr int TILE = LY::TILE, KS = LY::KS;
    constexpr int NP = (kMaxGroupMk * HDMAX + kMkThreads - 1) / kMkThreads;
    constexpr int NT = (TILE * HDMAX / 4 + kMkThreads - 1) / kMkThreads;  // float4 of a K (V) tile per thread
    const int tid = mk_tid<!(HDMAX == 64 && EXACT && !MOE)>();
    const int lane = tid & 63, wave = tid >> 6;
    const int hd = EXACT ? HDMAX : (int)p.hd;
    const int half = hd / 2;
    const int vpr = hd / 4;
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
    const __amdgpu_buffer_rsrc_t kr = coh_rsrc(kc, pos * kvw * 4u);  // rows [0, pos)
    const __amdgpu_buffer_rsrc_t vr = coh_rsrc(vc, pos * kvw * 4u);
    const tword* q = p.tqkv;
    const tword* kn_all = p.tqkv + p.heads * p.hd;
    const tword* vn_all = kn_all + kvw;
    const bool inter = p.rope_layout == 0;
    bool ok = true;

    for (uint32_t unit = blockIdx.x; unit < p.kv_heads * ns; unit += gridDim.x) {
        // Units [0, kv_heads) are the splits that append the new K/V row
        // (each head's last), the others follow head by head.
        uint32_t h, s;
        if (unit < p.kv_heads) {
            h = unit;
            s = ns - 1;
        } else {
            const uint32_t u = unit - p.kv_heads;
            h = u / (ns - 1);
            s = u - h * (ns - 1);
        }
        const uint32_t t0 = s * chunk, t1 = min(t0 + chunk, pos + 1);
        const bool owns = s == ns - 1;  // the last split ends at pos
        // K/V rows of a tile travel through registers (rk, rv) so the next
        // tile's loads are in flight while the current one is computed. They
        // are loaded coherently: a row written in this launch may share a
        // cache line with one read earlier by another XCD. (Rows outside the
        // tile and the new row, taken from LDS, load as zeros: out of range.)
        float4 rk[NT], rv[NT];
#define VVLI_TILE_LOAD(ta_, tlen_)                                                    \
    _Pragma("unroll") for (int i = 0; i < NT; ++i) {                                  \
        const int idx = tid + i * kMkThreads;                                         \
        const int j = idx / vpr, c4 = (idx - j * vpr) * 4;                            \
        const uint32_t t = (ta_) + j;                                                 \
        const bool in = idx < (tlen_) * vpr && t != pos;                              \
        const uint32_t off = in ? (t * kvw + (uint32_t)h * hd + c4) * 4u : 0xffffffffu; \
        rk[i] = ld_coh4(kr, off);                                                     \
        rv[i] = ld_coh4(vr, off);                                                     \
    }
#define VVLI_TILE_STORE(ta_, tlen_)                                                   \
    _Pragma("unroll") for (int i = 0; i < NT; ++i) {                                  \
        const int idx = tid + i * kMkThreads;                                         \
        if (idx < (tlen_) * vpr) {                                                    \
            const int j = idx / vpr, c4 = (idx - j * vpr) * 4;                        \
            float4* kd = reinterpret_cast<float4*>(ks + j * KS + c4);                 \
            float4* vd = reinterpret_cast<float4*>(vs + j * HDMAX + c4);              \
            *kd = rk[i];                                                              \
            *vd = rv[i];                                                              \
            if ((ta_) + j == pos) { /* the new row comes from LDS, not the cache */  \
                *kd = *reinterpret_cast<const float4*>(knew + c4);                    \
                *vd = *reinterpret_cast<const float4*>(vnew + c4);                    \
            }                                                                         \
        }                                                                             \
    }
        VVLI_TILE_LOAD(t0, (int)min((uint32_t)TILE, t1 - t0));
        // QK-norm (weight * (x * s), OlmoeRMSNorm's order) before the rotation.
        const uint16_t* qn = nullptr;
        const uint16_t* kn = nullptr;
        float scq = 1.f, sck = 1.f;
        // With QK-norm the whole q | k is polled for the scales; its values
        // land in the K and V tile space (free until the first tile), so the
        // head's q and the new k come from LDS, and the appending split's v
        // word goes out with that batch: one memory round trip, not two.
        float* qkl = nullptr;
        tword wv_pre = 0;
        if constexpr (MOE) {
            qn = p.layer[layer].q_norm;
            kn = p.layer[layer].k_norm;
            if (qn) {
                if (p.heads * p.hd + kvw <= (uint32_t)(TILE * KS + TILE * HDMAX)) qkl = ks;
                if (qkl && owns && tid < hd) wv_pre = ld_a(vn_all + (size_t)h * hd + tid);
                if (!mk_qk_scales(p, tag_in, scq, sck, qkl)) return false;
            }
        }
        // q (and the owner's new k / v) of this kv head, RoPE'd into LDS.
        for (int idx = tid; idx < G * half; idx += kMkThreads) {
            const int g = idx / half, i = idx - g * half;
            const int f = inter ? 2 * i : i, sc = inter ? 2 * i + 1 : i + half;
            float x0, x1;
            if (qkl) {
                x0 = qkl[(h * G + g) * hd + f];
                x1 = qkl[(h * G + g) * hd + sc];
            } else {
                const tword* src = q + (size_t)(h * G + g) * hd;
                tword w0 = ld_a(src + f), w1 = ld_a(src + sc);
                ok = ok && poll_tw2(src + f, src + sc, tag_in, w0, w1, p.error);
                x0 = tw_val(w0);
                x1 = tw_val(w1);
            }
            if constexpr (MOE) {
                if (qn) {
                    const uint16_t* nw = qn + (size_t)(h * G + g) * hd;
                    x0 = bf_val(nw[f]) * (x0 * scq);
                    x1 = bf_val(nw[sc]) * (x1 * scq);
                }
            }
            const float c = cs[2 * i], sn = cs[2 * i + 1];
            qs[g * HDMAX + f] = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, sn));
            qs[g * HDMAX + sc] = __fadd_rn(__fmul_rn(x0, sn), __fmul_rn(x1, c));
        }
        if (owns) {  // the new k pair and v word of thread tid (hd <= kMkThreads), loaded together
            static_assert(HDMAX <= kMkThreads, "one k pair and one v word per thread");
            const tword* ksrc = kn_all + (size_t)h * hd;
            const tword* vsrc = vn_all + (size_t)h * hd + tid;
            const bool hk = tid < half, hv = tid < hd;
            const int f = inter ? 2 * tid : tid, sc = inter ? 2 * tid + 1 : tid + half;
            tword w0 = 0, w1 = 0, wv = wv_pre;
            if (hk && !qkl) {
                w0 = ld_a(ksrc + f);
                w1 = ld_a(ksrc + sc);
            }
            if (hv && !qkl) wv = ld_a(vsrc);
            if (hk && !qkl) ok = ok && poll_tw2(ksrc + f, ksrc + sc, tag_in, w0, w1, p.error);
            if (hv) ok = ok && poll_tw(vsrc, tag_in, wv, p.error);
            if (hk) {
                const uint32_t kq = p.heads * p.hd + (uint32_t)h * hd;  // the new k in the q | k staging
                float x0 = qkl ? qkl[kq + f] : tw_val(w0), x1 = qkl ? qkl[kq + sc] : tw_val(w1);
                if constexpr (MOE) {
                    if (kn) {
                        x0 = bf_val(kn[(size_t)h * hd + f]) * (x0 * sck);
                        x1 = bf_val(kn[(size_t)h * hd + sc]) * (x1 * sck);
                    }
                }
                const float c = cs[2 * tid], sn = cs[2 * tid + 1];
                knew[f] = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, sn));
                knew[sc] = __fadd_rn(__fmul_rn(x0, sn), __fmul_rn(x1, c));
            }
            if (hv) vnew[tid] = tw_val(wv);
        }
        if (tid < kMaxGroupMk) {
            m_s[tid] = -INFINITY;
            l_s[tid] = 0.f;
        }
        if (__syncthreads_or(!ok)) return false;
        if (tid == 0) mk_mark(p, ph, 9);
        if (owns) {
            for (int d = tid; d < hd; d += kMkThreads) {
                st_a(kc + (size_t)pos * kvw + (size_t)h * hd + d, knew[d]);
                st_a(vc + (size_t)pos * kvw + (size_t)h * hd + d, vnew[d]);
            }
        }
        // Work split of a tile (TILE * HDMAX = 4096 floats):
        // scores: thread (row qj, chunk qc) -- HDMAX / 8 chunks of 8 floats
        // per row, one pair per thread -- holds its 8 floats of K_j and forms
        // q_g . K_j over the chunk for every q head g, summed across the
        // row's chunk lanes by DPP: the K tile is read from LDS once per tile
        // (the q reads are broadcasts).
        // P.V: thread (slice psl, dim pd) -- slices of 8 rows -- keeps the
        // running outputs of all G heads for its slice (pa), rescaled with the
        // running max like the whole; the V tile is read once per tile and the
        // slices are summed after the last tile.
        const int god = G * hd;
        float acc[NP];  // the split's unnormalised outputs, idx = g * hd + d at thread idx % kMkThreads
        // head_dim 128: the scores and P.V on the matrix cores (the tile's
        // dependent LDS round trips halve: 5.3k -> 2.7k cycles per 32-row tile
        // at group 7); head_dim <= 64: the vector units (one 64-row tile per
        // split at the timed lengths, where the matrix-core tile measured no
        // faster).
        if constexpr (HDMAX == 128) {
            // The tile's products on the matrix cores (v_mfma_f32_16x16x4f32; a
            // wave's 64 lanes: A[m][k] from lane m + 16 k, B[k][n] from lane
            // n + 16 k, lane l gets D[4 (l / 16) + i][l % 16], i < 4; q heads past
            // the group give rows that are not used, rows past the tile are
            // masked (scores) or zeroed (V)).
            // Scores: wave (row block jb of 16 K rows, quarter kq of 32 dims)
            // forms S_kq[g][j] over its dims -- 8 MFMAs, the K dims of a lane
            // contiguous -- into red; the softmax wave of head g sums the kKq
            // partials. P.V: wave (16-dim block db, 32-row slice js) keeps the
            // running outputs O[g][d] of its slice in o4, rescaled by the running
            // max's correction each tile; the slices are summed after the last
            // tile.
            constexpr int kJb = TILE / 16, kKq = 8 / kJb;  // 2 x 4 at hd 128, 4 x 2 at hd 64
            constexpr int kDb = HDMAX / 16, kJs = 8 / kDb;
            static_assert(kKq * 32 == HDMAX && kJs * 32 == TILE && kJb * kKq == kMkWaves, "MFMA wave split of a tile");
            const int ml = lane & 15, mg = lane >> 4;
            float* red = smem + LY::kRed;
            mk_f32x4 o4 = {0.f, 0.f, 0.f, 0.f};
            for (uint32_t ta = t0; ta < t1; ta += TILE) {
                const int tlen = (int)min((uint32_t)TILE, t1 - ta);
                VVLI_TILE_STORE(ta, tlen);
                if (ta + TILE < t1) {
                    VVLI_TILE_LOAD(ta + TILE, (int)min((uint32_t)TILE, t1 - ta - TILE));
                }
                __syncthreads();
                {
                    const int jb = wave % kJb, kq = wave / kJb;
                    const int d0 = kq * 32 + mg * 8;
                    const bool in0 = EXACT || d0 < hd, in1 = EXACT || d0 + 4 < hd;  // (hd % 4 == 0)
                    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
                    const float* qr = qs + ml * HDMAX + d0;
                    const float* kr = ks + (jb * 16 + ml) * KS + d0;
                    const float4 qa0 = in0 ? *reinterpret_cast<const float4*>(qr) : z4;
                    const float4 qa1 = in1 ? *reinterpret_cast<const float4*>(qr + 4) : z4;
                    const float4 kb0 = in0 ? *reinterpret_cast<const float4*>(kr) : z4;
                    const float4 kb1 = in1 ? *reinterpret_cast<const float4*>(kr + 4) : z4;
                    mk_f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
                    sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa0.x, kb0.x, sacc, 0, 0, 0);
                    sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa0.y, kb0.y, sacc, 0, 0, 0);
                    sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa0.z, kb0.z, sacc, 0, 0, 0);
                    sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa0.w, kb0.w, sacc, 0, 0, 0);
                    sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa1.x, kb1.x, sacc, 0, 0, 0);
                    sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa1.y, kb1.y, sacc, 0, 0, 0);
                    sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa1.z, kb1.z, sacc, 0, 0, 0);
                    sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa1.w, kb1.w, sacc, 0, 0, 0);
                    float* rp = red + (kq * kJb + jb) * 256 + (4 * mg) * 16 + ml;  // [kq][jb][g][j % 16]
                    rp[0] = sacc[0];
                    rp[16] = sacc[1];
                    rp[32] = sacc[2];
                    rp[48] = sacc[3];
                }
                __syncthreads();
                for (int g = wave; g < G; g += kMkWaves) {
                    // s[g][j] = (q_g . K_j) * scale, j = lane: the kKq partial products summed
                    float sc = -INFINITY;
                    if (lane < tlen) {
                        const int jb = lane >> 4, jj = lane & 15;
                        float x = 0.f;
    #pragma unroll
                        for (int kq = 0; kq < kKq; ++kq) x += red[(kq * kJb + jb) * 256 + g * 16 + jj];
                        sc = x * p.scale;
                    }
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
                {
                    const int db = wave % kDb, js = wave / kDb;
                    const int d = db * 16 + ml, j0 = js * 32 + mg * 8;
                    const float4 pa0 = *reinterpret_cast<const float4*>(ps + ml * TILE + j0);
                    const float4 pa1 = *reinterpret_cast<const float4*>(ps + ml * TILE + j0 + 4);
                    float vb[8];
    #pragma unroll
                    for (int r = 0; r < 8; ++r) vb[r] = j0 + r < tlen ? vs[(j0 + r) * HDMAX + d] : 0.f;
                    o4[0] *= c_s[4 * mg + 0];
                    o4[1] *= c_s[4 * mg + 1];
                    o4[2] *= c_s[4 * mg + 2];
                    o4[3] *= c_s[4 * mg + 3];
                    o4 = __builtin_amdgcn_mfma_f32_16x16x4f32(pa0.x, vb[0], o4, 0, 0, 0);
                    o4 = __builtin_amdgcn_mfma_f32_16x16x4f32(pa0.y, vb[1], o4, 0, 0, 0);
                    o4 = __builtin_amdgcn_mfma_f32_16x16x4f32(pa0.z, vb[2], o4, 0, 0, 0);
                    o4 = __builtin_amdgcn_mfma_f32_16x16x4f32(pa0.w, vb[3], o4, 0, 0, 0);
                    o4 = __builtin_amdgcn_mfma_f32_16x16x4f32(pa1.x, vb[4], o4, 0, 0, 0);
                    o4 = __builtin_amdgcn_mfma_f32_16x16x4f32(pa1.y, vb[5], o4, 0, 0, 0);
                    o4 = __builtin_amdgcn_mfma_f32_16x16x4f32(pa1.z, vb[6], o4, 0, 0, 0);
                    o4 = __builtin_amdgcn_mfma_f32_16x16x4f32(pa1.w, vb[7], o4, 0, 0, 0);
                }
                __syncthreads();
            }
            // The slices' outputs, summed in slice order into the layout of the
            // merge (output idx = g * hd + d at thread idx % kMkThreads).
            {
                const int db = wave % kDb, js = wave / kDb;
                const int d = db * 16 + ml;
    #pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (4 * mg + i < G) red[(js * 16 + 4 * mg + i) * HDMAX + d] = o4[i];  // [js][g][d]
                __syncthreads();
    #pragma unroll
                for (int i = 0; i < NP; ++i) {
                    const int idx = tid + i * kMkThreads;
                    acc[i] = 0.f;
                    if (idx < god) {
                        const int g = idx / hd, dd = idx - g * hd;
                        float o = 0.f;
    #pragma unroll
                        for (int sl = 0; sl < kJs; ++sl) o += red[(sl * 16 + g) * HDMAX + dd];
                        acc[i] = o;
                    }
                }
            }
        } else {
            // P.V work items: (slice sl, q head g, dim d); with G * hd <= 256 the
            // tile's rows are cut into nsl slices of span rows each (nsl * G * hd
            // <= kMkThreads, span a multiple of 16) so every thread works, and the
            // slices are summed after the last tile.
            constexpr int kPvBatch = 8;
            // (Slices only where registers allow: not in the dense hd-128 kernel,
            // whose groups are wide enough for every thread anyway.)
            constexpr bool kPvSlices = HDMAX <= 64 || MOE;
            int nsl = 1;
            if constexpr (kPvSlices)
                while (nsl < TILE / 16 && 2 * nsl * god <= kMkThreads) nsl *= 2;
            const int span = TILE / nsl;
    #pragma unroll
            for (int i = 0; i < NP; ++i) acc[i] = 0.f;
            for (uint32_t ta = t0; ta < t1; ta += TILE) {
                const int tlen = (int)min((uint32_t)TILE, t1 - ta);
                VVLI_TILE_STORE(ta, tlen);
                if (ta + TILE < t1) {
                    VVLI_TILE_LOAD(ta + TILE, (int)min((uint32_t)TILE, t1 - ta - TILE));
                }
                __syncthreads();
                // scores s[g][j] = (q_g . K_j) * scale: thread pairs, each over half
                // of the dimensions (two independent chains), summed across the pair.
                for (int idx2 = tid; idx2 < 2 * G * TILE; idx2 += kMkThreads) {
                    const int idx = idx2 >> 1, half_d = idx2 & 1;
                    const int g = idx / TILE, j = idx - g * TILE;
                    float a0 = 0.f, a1 = 0.f;
                    if (j < tlen) {
                        const float* qr = qs + g * HDMAX;
                        const float* kr = ks + j * KS;
                        if constexpr (EXACT) {
    #pragma unroll
                            for (int d = half_d * 4; d < HDMAX; d += 8) {  // float4 chunks alternate in the pair
                                const float4 q4 = *reinterpret_cast<const float4*>(qr + d);
                                const float4 k4 = *reinterpret_cast<const float4*>(kr + d);
                                a0 = fmaf(q4.x, k4.x, a0);
                                a1 = fmaf(q4.y, k4.y, a1);
                                a0 = fmaf(q4.z, k4.z, a0);
                                a1 = fmaf(q4.w, k4.w, a1);
                            }
                        } else {
                            for (int d = half_d * 4; d < hd; d += 8) {
                                const float4 q4 = *reinterpret_cast<const float4*>(qr + d);
                                const float4 k4 = *reinterpret_cast<const float4*>(kr + d);
                                a0 = fmaf(q4.x, k4.x, a0);
                                a1 = fmaf(q4.y, k4.y, a1);
                                a0 = fmaf(q4.z, k4.z, a0);
                                a1 = fmaf(q4.w, k4.w, a1);
                            }
                        }
                    }
                    const float part = a0 + a1;
                    const float dot = part + __shfl_xor(part, 1, kWave);
                    if (half_d == 0) ps[g * TILE + j] = j < tlen ? dot * p.scale : -INFINITY;
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
                // Rows in batches of kPvBatch (every LDS read of a batch issued
                // before its FMAs, one wait per batch).
    #pragma unroll
                for (int i = 0; i < NP; ++i) {
                    const int idx = tid + i * kMkThreads;
                    if (idx < god * nsl) {
                        // (Recomputed per tile: registers are scarce here.)
                        const int sl = nsl > 1 ? idx / god : 0;  // i > 0 only when nsl == 1
                        const int o = idx - sl * god;
                        const int g = o / hd, d = o - g * hd;
                        const float* pr = ps + g * TILE;
                        const int j0 = sl * span, j1 = min(j0 + span, tlen);
                        float v0 = acc[i] * c_s[g], v1 = 0.f, v2 = 0.f, v3 = 0.f;
                        int j = j0;
                        for (; j + kPvBatch <= j1; j += kPvBatch) {
                            float4 p4[kPvBatch / 4];
                            float vv[kPvBatch];
    #pragma unroll
                            for (int k = 0; k < kPvBatch / 4; ++k) p4[k] = *reinterpret_cast<const float4*>(pr + j + 4 * k);
    #pragma unroll
                            for (int k = 0; k < kPvBatch; ++k) vv[k] = vs[(j + k) * HDMAX + d];
    #pragma unroll
                            for (int k = 0; k < kPvBatch / 4; ++k) {
                                v0 = fmaf(p4[k].x, vv[4 * k + 0], v0);
                                v1 = fmaf(p4[k].y, vv[4 * k + 1], v1);
                                v2 = fmaf(p4[k].z, vv[4 * k + 2], v2);
                                v3 = fmaf(p4[k].w, vv[4 * k + 3], v3);
                            }
                        }
                        for (; j < j1; ++j) v0 = fmaf(pr[j], vs[j * HDMAX + d], v0);
                        acc[i] = (v0 + v1) + (v2 + v3);
                    }
                }
                __syncthreads();
            }
            if (nsl > 1) {  // slices 1.. through the (now free) K tile, added in slice order
                float* sred = ks;
                if (tid >= god && tid < god * nsl) sred[tid - god] = acc[0];
                __syncthreads();
                if (tid < god)
                    for (int k = 1; k < nsl; ++k) acc[0] += sred[(k - 1) * god + tid];
                __syncthreads();  // the merge reuses the K tile
            }
        }
        if (tid == 0) mk_mark(p, ph, 10);
        if (ns == 1) {  // one split: normalise its own outputs
            if (owns) wait_all_mem();  // the K/V row stores land before the output is published
            __syncthreads();
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int idx = tid + i * kMkThreads;
                if (idx < G * hd) {
                    const int g = idx / hd;
                    int idx_o = idx;  // (an opaque copy: hoisted, the 64-bit store address would hold registers)
                    asm volatile("" : "+v"(idx_o));
                    st_a(p.tattn + (size_t)h * G * hd + idx_o, tw_make(fmaf(acc[i], 1.0f / l_s[g], 0.f), tag_out));
                }
            }
            if (__syncthreads_or(!ok)) return false;
            if (tid == 0) mk_mark(p, ph, 0);
            continue;
        }
        // Flash-decoding merge: out = sum_s e^{m_s - M} acc_s / sum_s e^{m_s - M} l_s
        // (splits in ascending order). With 3..kOwnerMergeMax splits the
        // split that appended the K/V row merges them all and the others store
        // their partials and leave (their blocks start the next phase early);
        // with 2 or more than kOwnerMergeMax splits every split stores its
        // partials and merges a slice of the outputs from all of them, so no
        // block reads more than its slice of the partials. (Measured: the
        // former at Llama-3.2-1B heads with 9-10 splits, the latter at 2 and
        // at 43-46 splits.) The merge tables live in the K tile, free after
        // the last tile.
        const bool owner_merge = ns > 2 && ns <= kOwnerMergeMax;  // (the kernel's o-phase rule follows it)
        const size_t pbase = (size_t)h * p.nsplit;
        float* pm = ks;                              // [split][group]
        float* pl = pm + kMaxSplitMk * kMaxGroupMk;  // [split][group]
        float* wsp = pl + kMaxSplitMk * kMaxGroupMk; // merge weights [split][group]
        static_assert(3 * kMaxSplitMk * kMaxGroupMk <= TILE * KS, "merge tables fit in the K tile");
        if (!owner_merge || !owns) {  // partials: (m, l) per q head and the unnormalised outputs
            tword* pml = p.tpart_ml + (pbase + s) * G * 2;
            tword* pacc = p.tpart_acc + (pbase + s) * G * hd;
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int idx = tid + i * kMkThreads;
                if (idx < G * hd) st_a(pacc + idx, tw_make(acc[i], tag_out));  // idx = g * hd + d
            }
            if (tid < G) {
                st_a(pml + 2 * tid, tw_make(m_s[tid], tag_out));
                st_a(pml + 2 * tid + 1, tw_make(l_s[tid], tag_out));
            }
            if (tid == 0) mk_mark(p, ph, 11);
        }
        if (owner_merge) {
            if (!owns) continue;
            // Owner: fetch the other splits' partials -- (m, l) together with the
            // first batch of outputs, re-polled as a whole until every word
            // carries the tag (one memory round trip when they are there) -- then
            // merge, own split last.
            const int nml = (int)(ns - 1) * G;
            const int npe = (G * hd + kMkThreads - 1) / kMkThreads;  // output batches in use
            const tword* mls = p.tpart_ml + (pbase * G + (size_t)tid) * 2;  // split tid / G, head tid % G
            const tword* accs = p.tpart_acc + pbase * G * hd;
            tword wv[kOwnerMergeMax - 1] = {};
#define VVLI_POLL_PARTIALS(i_, with_ml_)                                                                    \
    {                                                                                                       \
        const int idx_ = tid + (i_) * kMkThreads;                                                           \
        const bool mine_ = idx_ < G * hd;                                                                   \
        const bool ml_ = (with_ml_) && tid < nml;                                                           \
        tword wm_ = 0, wl_ = 0;                                                                             \
        for (uint32_t spins = 0;; ++spins) {                                                                \
            bool good = true;                                                                               \
            if (ml_) {                                                                                      \
                wm_ = ld_a(mls);                                                                            \
                wl_ = ld_a(mls + 1);                                                                        \
            }                                                                                               \
            _Pragma("unroll") for (int s2 = 0; s2 < kOwnerMergeMax - 1; ++s2) if (mine_ && s2 < (int)ns - 1)\
                wv[s2] = ld_a(accs + (size_t)s2 * G * hd + idx_);                                           \
            if (ml_) good = tw_tag(wm_) == tag_out && tw_tag(wl_) == tag_out;                               \
            _Pragma("unroll") for (int s2 = 0; s2 < kOwnerMergeMax - 1; ++s2) if (mine_ && s2 < (int)ns - 1)\
                good = good && tw_tag(wv[s2]) == tag_out;                                                   \
            if (good) break;                                                                                \
            if (spins > kSpinLimit) {                                                                       \
                st_a(p.error, kDecodeErrTimeout);                                                           \
                ok = false;                                                                                 \
                break;                                                                                      \
            }                                                                                               \
            if ((spins & 63u) == 63u && ld_a(p.error) != 0) {                                               \
                ok = false;                                                                                 \
                break;                                                                                      \
            }                                                                                               \
            __builtin_amdgcn_s_sleep(1);                                                                    \
        }                                                                                                   \
        if (ml_) {                                                                                          \
            pm[tid] = tw_val(wm_);                                                                          \
            pl[tid] = tw_val(wl_);                                                                          \
        }                                                                                                   \
    }
            VVLI_POLL_PARTIALS(0, true)
            if (tid < G) {
                pm[(ns - 1) * G + tid] = m_s[tid];
                pl[(ns - 1) * G + tid] = l_s[tid];
            }
            if (__syncthreads_or(!ok)) return false;
            if (tid == 0) mk_mark(p, ph, 14);
            for (int g = wave; g < G; g += kMkWaves) {
                const bool in = (uint32_t)lane < ns;
                const float mv = in ? pm[lane * G + g] : -INFINITY;
                const float lv = in ? pl[lane * G + g] : 0.f;
                const float M = wave_max(mv);
                const float e = in ? expf(mv - M) : 0.f;
                const float L = wave_sum(lv * e);
                if (in) wsp[lane * G + g] = e / L;
            }
            wait_all_mem();  // the K/V row stores (wave 0) land before any wave publishes the output
            __syncthreads();
            if (tid == 0) mk_mark(p, ph, 15);
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                if (i >= npe) break;
                if (i > 0) VVLI_POLL_PARTIALS(i, false)
                const int idx = tid + i * kMkThreads;
                if (idx < G * hd) {
                    const int g = idx / hd;
                    // Every weight is read (in bounds: the weight table holds
                    // kMaxSplitMk * kMaxGroupMk floats), so the reads go out
                    // together; splits past ns are dropped by a select.
                    float wt[kOwnerMergeMax - 1];
#pragma unroll
                    for (int s2 = 0; s2 < kOwnerMergeMax - 1; ++s2) wt[s2] = wsp[s2 * G + g];
                    float o = 0.f;
#pragma unroll
                    for (int s2 = 0; s2 < kOwnerMergeMax - 1; ++s2) {
                        const float t = fmaf(tw_val(wv[s2]), wt[s2], o);
                        o = s2 < (int)ns - 1 ? t : o;
                    }
                    o = fmaf(acc[i], wsp[(ns - 1) * G + g], o);
                    // (An opaque copy of idx: hoisted out of every loop, the
                    // 64-bit store addresses would hold registers all kernel long.)
                    int idx_o = idx;
                    asm volatile("" : "+v"(idx_o));
                    st_a(p.tattn + (size_t)h * G * hd + idx_o, tw_make(o, tag_out));
                }
            }
#undef VVLI_POLL_PARTIALS
            if (__syncthreads_or(!ok)) return false;
            if (tid == 0) mk_mark(p, ph, 0);
            continue;
        }
        // Slices in reverse split order: the split that appended the K/V row
        // (the last) takes slice 0, never empty, so its publication also
        // orders the row stores before any reader of the output.
        const int per = (god + (int)ns - 1) / (int)ns;
        const int o0 = min(god, ((int)ns - 1 - (int)s) * per), nout = min(god, o0 + per) - o0;
        float* pv = vs;                              // slice values [output][split] (V tile, probabilities)
        static_assert(LY::kP + kMaxGroupMk * TILE - LY::kV >= kMaxGroupMk * HDMAX + kMaxSplitMk,
                      "slice values fit in the V tile and the probabilities");
        // Every split's (m, l) per q head and the slice's values of every
        // split (pair q = output * ns + split, in batches of two per thread),
        // each polled (its split may still be storing); the first batch of
        // values is issued with the (m, l) loads, so one memory round trip
        // fetches the lot when it is there.
        const tword* mlb = p.tpart_ml + pbase * G * 2;     // [split][group][2]
        const tword* accb = p.tpart_acc + pbase * G * hd;  // [split][G * hd]
        const int nq = nout * (int)ns;
        tword wv[2] = {};
#define VVLI_VALUES_LOAD(qb_)                                              \
    _Pragma("unroll") for (int k = 0; k < 2; ++k) {                        \
        const int q = (qb_) + tid + k * kMkThreads;                        \
        if (q < nq) {                                                      \
            const int ol = q / (int)ns, s2 = q - ol * (int)ns;             \
            wv[k] = ld_a(accb + (size_t)s2 * god + o0 + ol);               \
        }                                                                  \
    }
        VVLI_VALUES_LOAD(0)
        for (int i = tid; i < (int)ns * G; i += kMkThreads) {
            tword wm = ld_a(mlb + (size_t)i * 2), wl = ld_a(mlb + (size_t)i * 2 + 1);
            ok = ok && poll_tw2(mlb + (size_t)i * 2, mlb + (size_t)i * 2 + 1, tag_out, wm, wl, p.error);
            pm[i] = tw_val(wm);
            pl[i] = tw_val(wl);
        }
        for (int qb = 0; qb < nq; qb += 2 * kMkThreads) {
            if (qb > 0) VVLI_VALUES_LOAD(qb)
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int q = qb + tid + k * kMkThreads;
                if (q < nq) {
                    const int ol = q / (int)ns, s2 = q - ol * (int)ns;
                    ok = ok && poll_tw(accb + (size_t)s2 * god + o0 + ol, tag_out, wv[k], p.error);
                    pv[q] = tw_val(wv[k]);
                }
            }
        }
#undef VVLI_VALUES_LOAD
        if (__syncthreads_or(!ok)) return false;
        if (tid == 0) mk_mark(p, ph, 14);
        for (int g = wave; g < G; g += kMkWaves) {
            const bool in = lane < (int)ns;
            const float mv = in ? pm[lane * G + g] : -INFINITY;
            const float lv = in ? pl[lane * G + g] : 0.f;
            const float M = wave_max(mv);
            const float e = in ? expf(mv - M) : 0.f;
            const float L = wave_sum(lv * e);
            if (in) wsp[lane * G + g] = e / L;
        }
        if (owns) wait_all_mem();  // the K/V row stores land before the output is published
        __syncthreads();
        if (tid == 0) mk_mark(p, ph, 15);
        // Output o0 + ol sums its ns weighted values over a segment of wdt
        // lanes (ns rounded up to a power of two; a fixed butterfly order).
        int wdt = 1;
        while (wdt < (int)ns) wdt <<= 1;
        const int sl = tid & (wdt - 1);
        for (int ob = 0; ob < nout; ob += kMkThreads / wdt) {  // uniform over the block
            const int ol = ob + tid / wdt;
            float x = 0.f;
            if (ol < nout && sl < (int)ns) x = pv[ol * (int)ns + sl] * wsp[sl * G + (o0 + ol) / hd];
            for (int off = wdt >> 1; off > 0; off >>= 1) x += __shfl_xor(x, off, kWave);
            if (sl == 0 && ol < nout) {
                // (An opaque copy of the index: hoisted out of every loop, the
                // 64-bit store addresses would hold registers all kernel long.)
                int o_st = o0 + ol;
                asm volatile("" : "+v"(o_st));
                st_a(p.tattn + (size_t)h * G * hd + o_st, tw_make(x, tag_out));
            }
        }
        if (__syncthreads_or(!ok)) return false;
        if (tid == 0) mk_mark(p, ph, 0);
    }
    return true;
#undef VVLI_TILE_LOAD
#undef VVLI_TILE_STORE
}

// ---------------------------------------------------------------------------
// The kernel.
// ---------------------------------------------------------------------------
// Phases of one token step: per layer Q (input RMSNorm + q/k/v), A (RoPE, KV
// append, attention), O (x += Wo.attn), G (post-attention RMSNorm, gate/up,
// SwiGLU), D (x += Wd.ff); then the logits phase (final RMSNorm + lm_head) and
// the argmax (block 0), which publishes the next token. All GEMV phases run
// through one code path with a grid-uniform mode, so the whole step loop
// stays small enough for the instruction cache.
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
    const MkGemv* gemv;           // [layers * 4 + 1]
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

// MOE routing in the gate/up phase. Router row e is computed by wave
// e / grid of block grid - 1 - e % grid (the last blocks: the first ones run
// the attention units and reach the phase later) on its block's staged
// norm(x) and published as a tagged word; every block that runs
// gate/up or down tiles then polls the E logits (one hop: the router stays
// one 8 KiB row per producing wave instead of the whole matrix per block)
// and the block takes the softmax + top-k into ex / wsl (`need`: the block
// has tiles in this layer's gate/up or down).
// Why the next layer's write of trl cannot overtake a reader: a block that
// polls trl here has gate/up or down tiles, so its gate/up outputs (staged
// by every down block) or its down outputs (staged by the next q/k/v phase)
// lie upstream of the next layer's gate/up staging, which precedes any write
// of trl for that layer. Blocks without tiles do not poll, so a late one
// never waits for words that have moved on to a later epoch. The gate/up and down
// phases of the layer take their experts from there. Block-uniform; false:
// a poll failed.
// The producing wave's first router row, loaded at the end of the previous
// phase into `pre` (the gate/up phase has no weight prefetch of its own).
__device__ __forceinline__ uint32_t mk_router_row(const MkWave& w) {
    return w.wave * gridDim.x + (gridDim.x - 1 - blockIdx.x);
}

__device__ __forceinline__ void mk_router_prefetch(const DecodeStepParams& p, uint32_t layer, const MkWave& w,
                                                   uint4 (&pre)[kNJC]) {
    const uint32_t e = mk_router_row(w);
    if (e >= p.experts) return;
    const uint16_t* rp[1] = {p.layer[layer].router + (size_t)e * p.hidden};
    uint4 b[1][kNJC];
    issue<uint16_t, 1>(b, rp, 0, p.hidden / 8, w.lane);
#pragma unroll
    for (int j = 0; j < kNJC; ++j) pre[j] = b[0][j];
}

__device__ __forceinline__ bool mk_route(const DecodeStepParams& p, uint32_t layer, const float* xs, uint32_t tag,
                                         bool need, float* s_rl, unsigned long long* s_key, uint32_t* s_rank,
                                         uint32_t* ex, float* wsl, const MkWave& w, const uint4 (&pre)[kNJC],
                                         uint32_t ph) {
    const uint16_t* rw = p.layer[layer].router;
    const uint32_t E = p.experts, H = p.hidden, U = H / 8;
    const uint32_t e0 = mk_router_row(w);
    for (uint32_t e = e0; e < E; e += w.nw) {
        const uint16_t* rp[1] = {rw + (size_t)e * H};
        float acc[1] = {0.f};
        for (uint32_t ub = 0; ub < U; ub += kNJC * kWave) {
            uint4 b[1][kNJC];
            if (e == e0 && ub == 0) {
#pragma unroll
                for (int j = 0; j < kNJC; ++j) b[0][j] = pre[j];
            } else {
                issue<uint16_t, 1>(b, rp, ub, U, w.lane);
            }
            consume<uint16_t, 1>(b, xs, ub, U, w.lane, acc);
        }
        const float v = wave_sum(acc[0]);
        if (w.lane == 0) st_a(p.trl + e, tw_make(v, tag));
        if (threadIdx.x == 0) mk_mark(p, ph, 15);
    }
    if (!need) return true;
    bool ok = true;
    const int tid = mk_tid<true>();  // MoE variants only
    if ((uint32_t)tid < E) {
        tword wv = ld_a(p.trl + tid);
        ok = poll_tw(p.trl + tid, tag, wv, p.error);
        s_rl[tid] = tw_val(wv);
    }
    if (__syncthreads_or(!ok)) return false;
    route_block<kMkThreads>(s_rl, E, p.top_k, ex, wsl, s_key, s_rank);
    __syncthreads();
    return true;
}

// RES: the resident single-step form (p.mbox set); its code is compiled only
// into those instances, so the other launches run exactly the plain step.
template <int HDMAX, bool EXACT, bool MOE = false, bool RES = false>
__global__ __launch_bounds__(kMkThreads) void decode_step_kernel(DecodeStepParams p) {
    extern __shared__ float smem[];
    __shared__ float red[kMkWaves];
    __shared__ unsigned long long kred[kMkWaves];
    __shared__ uint32_t s_ctl[4];
    // MOE: the layer's routed experts and their weights, router logits.
    __shared__ uint32_t s_ex[MOE ? kMaxTopK : 1];
    __shared__ float s_w[MOE ? kMaxTopK : 1];
    __shared__ float s_rl[MOE ? 256 : 1];
    __shared__ unsigned long long s_key[MOE ? 256 : 1];
    __shared__ uint32_t s_rank[MOE ? 256 : 1];
    const int tid = threadIdx.x;
    MkWave w;
    w.lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar registers)
    // Tile t goes to block t mod blocks, wave (t / blocks) mod 8: consecutive
    // tiles land on different CUs and a phase with fewer tiles than waves
    // still uses them all.
    w.wid = wave * gridDim.x + blockIdx.x;
    w.nw = gridDim.x * kMkWaves;
    w.wave = wave;
    uint4 buf[2][kNJC];
    MkTile tile;
    unsigned long long best = 0ull;
    const uint32_t H = p.hidden;
    const uint32_t nps = kPhPerLayer * p.layers + 2;  // phases per step: layers, logits, argmax
    const uint32_t logits_ph = kPhPerLayer * p.layers;
    if (p.timing && tid == 0 && blockIdx.x == 0)
        p.timing[(size_t)gridDim.x * p.timing_stride] = __builtin_amdgcn_s_memrealtime();
    const MkTables tb = mk_load_tables(p, reinterpret_cast<char*>(smem) + p.table_lds_offset);
    if (tid == 0) {
        if (p.init_step) {
            s_ctl[0] = p.init_token;
            // (bit 31, resident steps: this step writes its logits to host memory)
            s_ctl[1] = p.init_pos | ((RES && p.host_logits && p.init_logits) ? 0x80000000u : 0u);
            if (blockIdx.x == 0) {  // the same thread finishes the step and reads these back
                st_a(&p.state->token, p.init_token);
                st_a(&p.state->pos, p.init_pos);
                st_a(&p.state->n_out, 0u);
                st_a(&p.state->counting, 0u);
                st_a(&p.state->argmax, 0u);
                st_a(&p.state->prompt_len, 0u);
                st_a(&p.state->stop, 0u);
            }
        } else {
            s_ctl[0] = ld_a(&p.state->token);
            s_ctl[1] = ld_a(&p.state->pos);
        }
        s_ctl[3] = ld_a(p.error);
    }
    __syncthreads();
    // A flag still raised (an earlier launch of an unchecked sequence failed,
    // or the host raised it): leave before any phase.
    if (s_ctl[3] != 0) return;
    uint32_t token = s_ctl[0];
    const uint32_t pos0 = s_ctl[1] & 0x7fffffffu;
    // Resident single steps carry their own position (and whether to write
    // the logits to host memory, bit 31) in a second step word, kept in
    // s_ctl[1] for the step (read where needed, not held in registers).
    auto host_lg = [&]() { return RES && p.host_logits && (s_ctl[1] >> 31); };
    bool have = mk_prefetch(tb.gemv[0], kGemvPlain, w, buf, tile);
    // The o phases leave out blocks [0, kv_heads) -- they run the attention
    // units that append the K/V row and merge, the last to finish the
    // attention phase -- when the other blocks' waves cover the tiles; with
    // a spread merge (every split merging) all the unit blocks, when they are
    // few (measured: OLMoE's 32 units at 2 splits, +1.1 %).
    const uint32_t o_tiles = mk_tiles<MOE>(tb.gemv[1], kGemvResid);
    const uint32_t o_fb_heads =
        (p.kv_heads < gridDim.x && o_tiles <= (gridDim.x - p.kv_heads) * kMkWaves) ? p.kv_heads : 0;

    for (uint32_t step = 0; step < p.n_steps; ++step) {
        const uint32_t e0 = p.epoch0 + step * nps;  // epoch of this step's phase 0
        if (step > 0) {  // next token from the previous step's argmax (or the host's request)
            __syncthreads();
            if (tid == 0) {
                tword wv = ld_a(p.step_word);
                s_ctl[2] = poll_tw(p.step_word, e0 - 1, wv, p.error) ? (uint32_t)wv : 0xfffffffeu;
                if (RES && s_ctl[2] < 0xfffffffeu) {
                    tword wp = ld_a(p.step_word + 1);
                    if (poll_tw(p.step_word + 1, e0 - 1, wp, p.error)) s_ctl[1] = (uint32_t)wp;
                    else s_ctl[2] = 0xfffffffeu;
                }
            }
            __syncthreads();
            token = s_ctl[2];
            if (token >= 0xfffffffeu) break;  // stop (EOS / context full / no request) or error
        }
        // (Block-uniform: read into a scalar register.)
        const uint32_t pos =
            RES ? (uint32_t)__builtin_amdgcn_readfirstlane((int)(s_ctl[1] & 0x7fffffffu)) : pos0 + step;
        if (pos >= p.max_seq || token >= p.vocab) {  // host validated; defensive stop
            if (blockIdx.x == 0 && tid == 0) st_a(p.error, kDecodeErrState);
            return;
        }
        const uint32_t T = pos + 1;
        // Positions per attention split: a whole number of K/V tiles (a split
        // pays one tile's load latency per tile, so 65 rows cost as much as
        // 96 -- fewer splits then merge, and more blocks stay free).
        constexpr uint32_t kTile = AttnLds<HDMAX>::TILE;
        uint32_t chunk = (T + p.nsplit - 1) / p.nsplit;
        if (chunk < p.min_chunk) chunk = p.min_chunk;
        chunk = (chunk + kTile - 1) / kTile * kTile;
        const uint32_t ns = (T + chunk - 1) / chunk;
        const uint16_t* emb = p.embed + (size_t)token * H;
        const uint32_t units = p.kv_heads * ns;  // attention units run by blocks [0, units)
        const bool spread_merge = ns <= 2 || ns > kOwnerMergeMax;  // (mk_attention's merge rule)
        const uint32_t o_fb =
            (spread_merge && units <= 32 && units < gridDim.x && o_tiles <= (gridDim.x - units) * kMkWaves)
                ? units
                : o_fb_heads;

        for (uint32_t ph = 0; ph <= logits_ph; ++ph) {
            const MkPhase f = mk_phase(ph, p.layers);
            const uint32_t tag = e0 + ph;
            bool ok = true;
            if (f.kind == kPhA && !f.logits) {
                ok = mk_attention<HDMAX, EXACT, MOE>(p, f.layer, pos, chunk, ns, smem, tag - 1, tag, ph);
                if (!MOE && p.g_lds_tiles) {  // blocks without a unit: this layer's first gate/up tiles into LDS
                    const MkGemv& gg = tb.gemv[f.layer * 4 + 2];
                    const GLds q = mk_glds(p, units, gg);
                    if (mk_glds_count(q, w.wave)) {
                        // Start the copy kGldsDelay after the q/k/v words
                        // show up, so it does not queue in front of them, of
                        // the units' K/V loads and of their q polls (which
                        // return ~1.5 us after the words appear; the copies
                        // still end well before the gate/up phase).
                        tword qw = ld_a(p.tqkv);
                        ok = ok && poll_tw(p.tqkv, tag - 1, qw, p.error);
                        if (ok) {
                            __builtin_amdgcn_s_sleep(kGldsSleep);  // 64 x kGldsSleep cycles, twice
                            __builtin_amdgcn_s_sleep(kGldsSleep);
                            mk_glds_issue(q, gg, reinterpret_cast<char*>(smem), w.wave, w.lane);
                        }
                    }
                }
            } else {
                const MkGemv& g = mk_gemv_of(p, tb, f);
                const int mode = mk_mode(f);
                if (f.logits) best = 0ull;
                // LDS tiles: gate/up phases only (gl.n = 0 otherwise).
                const GLds gl = mk_glds(p, units, g, !MOE && f.kind == kPhG && !f.logits && p.g_lds_tiles);
                // The block has tiles (streamed: block < their count; or LDS
                // tiles): stage the input.
                const uint32_t n_streamed = mk_tiles<MOE>(g, mode) - gl.n;
                const bool has_lds =
                    gl.n && blockIdx.x >= gl.first_block && (blockIdx.x - gl.first_block) * gl.per_block < gl.n;
                // MOE gate/up: every block stages (the router rows are spread over
                // the grid's waves); blocks with gate/up or down tiles route.
                const bool routes = MOE && f.kind == kPhG && !f.logits;
                const uint32_t fb = (f.kind == kPhO && !f.logits) ? o_fb : 0;
                const MkWave wp = mk_wave_from(w, fb);
                if ((blockIdx.x >= fb && blockIdx.x - fb < n_streamed) || has_lds || routes) {
                    const tword* src = f.kind == kPhO ? p.tattn
                                                      : (f.kind == kPhD ? p.tff : (f.kind == kPhG ? p.tx + H : p.tx));
                    // The phase's first weights, once the wave's share of the
                    // input is in (not with LDS tiles, which cover that
                    // latency, nor before the MoE routing picks the experts).
                    auto first_weights = [&]() {
                        if (!have && !gl.n && !routes) have = mk_prefetch<MOE>(g, mode, wp, buf, tile, 0, s_ex);
                    };
                    ok = mk_stage<HDMAX == 128 && (MOE || !EXACT)>(smem, red, src, tag - 1, ph == 0 ? emb : nullptr, mk_norm_of(p, tb, f), p.eps,
                                  f.kind == kPhD ? p.inter : H, p.error,
                                  (p.timing && p.timing_slots == 16 && (ph + 1) * 16 <= p.timing_stride)
                                      ? p.timing + blockIdx.x * p.timing_stride + ph * 16 + 9
                                      : nullptr,
                                  first_weights);
                    if (tid == 0) mk_mark(p, ph, 0);
                    if constexpr (MOE) {
                        if (routes && ok) {
                            const uint32_t nd = mk_tiles<MOE>(tb.gemv[f.layer * 4 + 3], kGemvResid);
                            const bool need = blockIdx.x < n_streamed || has_lds || blockIdx.x < nd;
                            ok = mk_route(p, f.layer, smem, tag, need, s_rl, s_key, s_rank, s_ex, s_w, w, buf[0], ph);
                            if (tid == 0) mk_mark(p, ph, 14);
                        }
                    }
                    // Residual rows: O reads x of the previous layer's D (or the
                    // embedding), D reads x of this layer's O.
                    MkResid rs;
                    rs.src = f.kind == kPhO ? p.tx : p.tx + H;
                    rs.tag = f.kind == kPhO ? tag - 3 : tag - 2;
                    rs.bf16 = (f.kind == kPhO && f.layer == 0) ? emb : nullptr;
                    const uint32_t n_lds = mk_glds_count(gl, w.wave);
                    if (gl.n) {  // grid-uniform: LDS tiles while the first streamed item loads
                        have = mk_prefetch(g, mode, w, buf, tile, gl.n);
                        mk_glds_compute(gl, g, smem, reinterpret_cast<char*>(smem), p.g_lds_park, w);
                    }
                    ok = ok && mk_gemv<MOE, RES>(g, mode, smem, wp, buf, tile, have, best, tag, rs, gl.n,
                                            reinterpret_cast<const float*>(reinterpret_cast<const char*>(smem) +
                                                                           p.g_lds_park),
                                            n_lds ? (blockIdx.x - gl.first_block) * gl.per_block + w.wave : 0,
                                            n_lds, p.error,
                                            (f.kind == kPhD && p.hidden_dbg) ? p.hidden_dbg + (size_t)f.layer * H
                                            : (f.logits && host_lg())         ? p.host_logits
                                                                             : nullptr,
                                            s_ex, s_w);
                }
                // The wave's written-through logits are complete before its
                // key is published (the blocks copy them to host memory once
                // every key is there).
                if (f.logits && host_lg()) wait_all_mem();
                if (f.logits && w.lane == 0) {
                    st_a(p.tkeys + 2 * w.wid, tw_make_u((uint32_t)(best >> 32), tag));
                    st_a(p.tkeys + 2 * w.wid + 1, tw_make_u((uint32_t)best, tag));
                }
            }
            if (w.lane == 0) mk_mark(p, ph, 1 + (int)wave);
            if (__syncthreads_or(!ok)) return;
            if (tid == 0) mk_mark(p, ph, 12);
            // Issue the first weights of the next GEMV phase (the next step's
            // first phase after the logits) before waiting for its input.
            // (Not when the next phase starts with LDS tiles: those cover the
            // first streamed item's latency, and the input poll is not queued
            // behind it.)
            if (ph < logits_ph) {
                const MkPhase nf = mk_phase(ph + 1, p.layers);
                const MkGemv& ng = mk_gemv_of(p, tb, nf);
                if (MOE && nf.kind == kPhG && !nf.logits) {  // experts not routed yet: the router row instead
                    have = false;
                    mk_router_prefetch(p, nf.layer, w, buf[0]);
                }
                else if (nf.kind == kPhG && !nf.logits && p.g_lds_tiles &&
                    mk_glds(p, units, ng).n > 0)
                    have = false;
                else have = false;
            } else if (!RES && step + 1 < p.n_steps) {
                have = mk_prefetch(tb.gemv[0], kGemvPlain, w, buf, tile);
            }
            if (tid == 0) mk_mark(p, ph, 13);
        }

        // ---- resident step that returns its logits: every block copies a
        // slice of them to host memory once every wave's key shows that its
        // (written-through) logits are complete, then marks its slice copied.
        if (host_lg()) {
            constexpr bool kPin = HDMAX == 128 && (MOE || !EXACT);  // (as the staging: no hoisted addresses)
            const uint32_t ktag = e0 + logits_ph;
            bool ok = true;
            for (uint32_t i = mk_tid<kPin>(); i < w.nw; i += kMkThreads) {
                tword hi = ld_a(p.tkeys + 2 * i), lo = ld_a(p.tkeys + 2 * i + 1);
                ok = ok && poll_tw2(p.tkeys + 2 * i, p.tkeys + 2 * i + 1, ktag, hi, lo, p.error);
            }
            if (__syncthreads_or(!ok)) return;
            const uint32_t per = (p.vocab + gridDim.x - 1) / gridDim.x;
            const uint32_t end = min(p.vocab, (blockIdx.x + 1) * per);
            for (uint32_t i = blockIdx.x * per + mk_tid<kPin>(); i < end; i += kMkThreads)
                st_sys(p.host_logits + i, ld_a(p.logits + i));
            wait_all_mem();
            __syncthreads();
            if (tid == 0) st_a(p.tcopied + blockIdx.x, tw_make_u(0u, ktag));
        }

        // ---- argmax + step advance (block 0) ----
        if (blockIdx.x == 0) {
            const uint32_t ktag = e0 + logits_ph;
            unsigned long long b = 0ull;
            bool ok = true;
            for (uint32_t i = tid; i < w.nw; i += kMkThreads) {
                tword hi = ld_a(p.tkeys + 2 * i), lo = ld_a(p.tkeys + 2 * i + 1);
                ok = ok && poll_tw2(p.tkeys + 2 * i, p.tkeys + 2 * i + 1, ktag, hi, lo, p.error);
                const unsigned long long k = ((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo;
                b = k > b ? k : b;
            }
            b = wave_max_u64(b);
            if (w.lane == 0) kred[wave] = b;
            if (__syncthreads_or(!ok)) return;
            if (host_lg()) {  // every block's slice of the logits is in host memory
                const uint32_t ktag = e0 + logits_ph;
                for (uint32_t bl = mk_tid<HDMAX == 128 && (MOE || !EXACT)>(); bl < gridDim.x; bl += kMkThreads) {
                    tword cw = ld_a(p.tcopied + bl);
                    ok = ok && poll_tw(p.tcopied + bl, ktag, cw, p.error);
                }
                if (__syncthreads_or(!ok)) return;
            }
            if constexpr (RES) {
                if (tid == 0) {
                    for (int i = 0; i < kMkWaves; ++i) b = kred[i] > b ? kred[i] : b;
                    const uint32_t tok = argmax_key_index(b);  // llm.argmax, src/llm.zig:778-789
                    st_a(&p.state->argmax, tok);
                    // Resident single steps: report this one, then wait for the
                    // host's next request (bounded by the linger time).
                    // (The report goes to coherent host memory: each store is
                    // complete before the sequence number is issued, and every
                    // block's logits stores were complete before its mark.)
                    HostStepOut* h = p.host_out;
                    st_sys(&h->argmax, tok);
                    st_sys(&h->stop, 0u);
                    st_sys(&h->error, 0u);
                    wait_all_mem();
                    st_sys(&h->seq, p.host_seq + step);
                    if (step + 1 < p.n_steps) {
                        const uint32_t want = p.host_seq + step + 1;
                        uint32_t next_tok = 0xffffffffu, next_pos = 0;
                        const unsigned long long deadline = __builtin_amdgcn_s_memrealtime() + p.linger_ticks;
                        for (uint32_t spins = 0;; ++spins) {
                            if (ld_sys(&p.mbox->seq) == want) {
                                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");  // the request's fields after its number
                                if (ld_sys(&p.mbox->cmd) == 0) {
                                    next_tok = ld_sys(&p.mbox->token);
                                    next_pos = ld_sys(&p.mbox->pos);
                                }
                                break;
                            }
                            if ((spins & 15u) == 15u && __builtin_amdgcn_s_memrealtime() > deadline) break;
                            __builtin_amdgcn_s_sleep(2);
                        }
                        if (next_tok != 0xffffffffu) {
                            st_a(&p.state->token, next_tok);
                            st_a(&p.state->pos, next_pos & 0x7fffffffu);
                            st_a(p.step_word + 1, tw_make_u(next_pos, e0 + nps - 1));
                        }
                        st_a(p.step_word, tw_make_u(next_tok, e0 + nps - 1));
                    }
                }
            } else if (tid == 0) {
                for (int i = 0; i < kMkWaves; ++i) b = kred[i] > b ? kred[i] : b;
                const uint32_t tok = argmax_key_index(b);  // llm.argmax, src/llm.zig:778-789
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
                if (step + 1 < p.n_steps) st_a(p.step_word, tw_make_u(stop ? 0xffffffffu : next_tok, e0 + nps - 1));
            }
        }
        // (Resident steps: the next step's first weights after block 0's
        // argmax, report and copy, so that none is held in registers across
        // that code.)
        if (RES && step + 1 < p.n_steps) have = mk_prefetch(tb.gemv[0], kGemvPlain, w, buf, tile);
    }
    // The thread that finished every step (or saw the stop or the error flag)
    // reports to the host; the step state holds its own last writes.
    if (!RES && p.host_out && blockIdx.x == 0 && tid == 0) {
        HostStepOut* h = p.host_out;
        st_sys(&h->argmax, ld_a(&p.state->argmax));
        st_sys(&h->stop, ld_a(&p.state->stop));
        st_sys(&h->error, ld_a(p.error));
        st_sys(&h->seq, p.host_seq);
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

uint32_t decode_step_phases_per_step(uint32_t layers) { return kPhPerLayer * layers + 2; }

uint32_t decode_step_glds_tile_bytes(uint32_t K) {
    const uint32_t nchunk = (K / 8 + kNJC * kWave - 1) / (kNJC * kWave);
    return 2 * nchunk * kNJC * kWave * 16;
}

// Range 1: from the end of the hidden-sized staging (x and norm weights of the
// q/k/v, o and gate/up phases, live while tiles are held) to the tables.
// Range 2: after the tables and the result parking area, up to the LDS of a
// CU (160 KiB) minus the kernel's static LDS and a margin.
uint32_t decode_step_glds_plan(uint32_t hidden, uint32_t inter, uint32_t hd, size_t* lds, uint32_t* off1,
                               uint32_t* tiles1, uint32_t* off2, uint32_t* park) {
    constexpr size_t kLdsPerCu = 160 * 1024, kReserve = 1024, kMaxTiles = 64;
    const size_t tb = decode_step_glds_tile_bytes(hidden);
    const size_t a1 = ((size_t)2 * hidden * sizeof(float) + 1023) / 1024 * 1024;
    const size_t e1 = decode_step_table_offset(hidden, inter, hd);
    const size_t n1 = e1 > a1 ? std::min((e1 - a1) / tb, kMaxTiles) : 0;
    const size_t ap = (*lds + 1023) / 1024 * 1024;  // result parking, then range 2
    const size_t a2 = ap + kMkWaves * kWave * sizeof(float);
    const size_t n2 = a2 + kReserve < kLdsPerCu ? std::min((kLdsPerCu - kReserve - a2) / tb, kMaxTiles - n1) : 0;
    *off1 = static_cast<uint32_t>(a1);
    *tiles1 = static_cast<uint32_t>(n1);
    *off2 = static_cast<uint32_t>(a2);
    *park = static_cast<uint32_t>(ap);
    if (n2 > 0) *lds = a2 + n2 * tb;
    return static_cast<uint32_t>(n1 + n2);
}

bool decode_step_moe_supported(uint32_t hd) { return hd == 64 || hd == 128; }

template <bool RES>
static const void* decode_step_fn_t(uint32_t hd, bool moe) {
    if (moe) {
        if (hd == 64) return reinterpret_cast<const void*>(&decode_step_kernel<64, true, true, RES>);
        return reinterpret_cast<const void*>(&decode_step_kernel<128, true, true, RES>);
    }
    if (hd == 64) return reinterpret_cast<const void*>(&decode_step_kernel<64, true, false, RES>);
    if (hd == 128) return reinterpret_cast<const void*>(&decode_step_kernel<128, true, false, RES>);
    if (hd <= 64) return reinterpret_cast<const void*>(&decode_step_kernel<64, false, false, RES>);
    return reinterpret_cast<const void*>(&decode_step_kernel<128, false, false, RES>);
}
static const void* decode_step_fn(uint32_t hd, bool moe, bool resident = false) {
    return resident ? decode_step_fn_t<true>(hd, moe) : decode_step_fn_t<false>(hd, moe);
}

hipError_t decode_step_max_blocks(uint32_t hd, size_t lds, int* blocks_per_cu, bool moe) {
    if (moe && !decode_step_moe_supported(hd)) return hipErrorInvalidValue;
    const void* f = decode_step_fn(hd, moe);
    hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e == hipSuccess)
        e = hipFuncSetAttribute(decode_step_fn(hd, moe, true), hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    int res_blocks = 0;  // the resident form fits as many blocks
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&res_blocks, decode_step_fn(hd, moe, true), kMkThreads, lds);
    if (e != hipSuccess) return e;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, f, kMkThreads, lds);
    if (e == hipSuccess && res_blocks < *blocks_per_cu) *blocks_per_cu = res_blocks;
    return e;
}

// The launch is cooperative (the runtime guarantees that all blocks are
// resident at once, which the inter-block polls rely on). With
// VVLI_PLAIN_LAUNCH=1 it is an ordinary launch of the same grid -- one block
// per CU, which the occupancy check at model creation showed fits -- for
// tools that do not follow cooperative dispatches (rocprofv3 kernel traces).
// Were a block not resident, the bounded polls would report a device error.
hipError_t launch_decode_step(const DecodeStepParams& p, uint32_t blocks, size_t lds, hipStream_t s) {
    DecodeStepParams copy = p;
    void* args[] = {&copy};
    static const bool plain = [] {
        const char* e = getenv("VVLI_PLAIN_LAUNCH");
        return e && e[0] == '1';
    }();
    const bool moe = p.experts > 0;
    if (moe && (!decode_step_moe_supported(p.hd) || p.experts > 256 || p.top_k == 0 || p.top_k > kMaxTopK ||
                p.top_k > p.experts || p.hidden % 8 != 0))
        return hipErrorInvalidValue;
    if (p.mbox && (!p.host_out || !p.init_step)) return hipErrorInvalidValue;
    const void* f = decode_step_fn(p.hd, moe, p.mbox != nullptr);
    if (plain) return hipLaunchKernel(f, dim3(blocks), dim3(kMkThreads), args, lds, s);
    return hipLaunchCooperativeKernel(f, dim3(blocks), dim3(kMkThreads), args, (unsigned)lds,
                                      s);
}

}  // namespace vvli
