// kernels.hpp -- host-side launch interface of the HIP kernels.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <utility>
#include <vector>

namespace vvli {

// While non-null (vvli_gpu_profile_step), every kernel launch records a
// start/stop event pair at its own dispatch boundaries (hipExtLaunchKernel),
// which times the kernel alone, as a kernel trace does.
extern thread_local std::vector<std::pair<hipEvent_t, hipEvent_t>>* g_launch_events;

template <typename... Args, typename F>
inline hipError_t vlaunch(F kernel, dim3 grid, dim3 block, size_t shmem, hipStream_t s, Args... args) {
    if (g_launch_events) {
        hipEvent_t a = nullptr, b = nullptr;
        hipError_t e = hipEventCreate(&a);
        if (e == hipSuccess) e = hipEventCreate(&b);
        if (e != hipSuccess) return e;
        g_launch_events->push_back({a, b});
        hipExtLaunchKernelGGL(kernel, grid, block, static_cast<std::uint32_t>(shmem), s, a, b, 0u, args...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, shmem, s, args...);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// GEMV (batch-1 linearInto, src/llm.zig:1228-1275) with fused prologue /
// epilogues. Weights are row-major [rows][K] in the blob dtype.
// ---------------------------------------------------------------------------
enum GemvMode {
    kGemvPlain = 0,   // out[r] = W.x (+ bias[r]); up to 3 stacked segments (q|k|v)
    kGemvResid = 1,   // out[r] += W.x            (o_proj / down_proj + residual add)
    kGemvGateUp = 2,  // out[r] = silu(Wg.x) * (Wu.x)   (gate/up + siluMulInto)
    kGemvLogits = 3,  // out[r] = W.x; per-block argmax key -> block_keys[block]
};

struct GemvArgs {
    const void* w[3] = {nullptr, nullptr, nullptr};
    const void* bias[3] = {nullptr, nullptr, nullptr};
    float* out[3] = {nullptr, nullptr, nullptr};
    uint32_t rows[3] = {0, 0, 0};
    const void* w_up = nullptr;      // gate/up mode: the up matrix (rows of w[0])
    const float* x = nullptr;        // input vector, K floats
    const void* norm_w = nullptr;    // RMSNorm weight applied to x first (nullable)
    float eps = 0.f;
    uint32_t K = 0;
    unsigned long long* block_keys = nullptr;  // logits mode
};

// Rows per block for a mode (host uses it to size block_keys and to check
// that stacked segments split on block boundaries).
uint32_t gemv_rows_per_block(int mode);
uint32_t gemv_grid(int mode, uint32_t total_rows);
// Argmax keys written by a logits-mode launch over total_rows rows (one per wave).
uint32_t gemv_num_keys(uint32_t total_rows);
hipError_t launch_gemv(int weight_kind, int mode, const GemvArgs& a, hipStream_t s);
hipError_t gemv_init_attributes();

// ---------------------------------------------------------------------------
// Decode attention (computeAttentionInto, src/llm.zig:1302-1335) with RoPE of
// q / new k (applyRoPE, :1337-1371) and the KV append (:744-745) fused in.
// ---------------------------------------------------------------------------
struct AttnArgs {
    const float* q = nullptr;      // raw q (after bias), heads*hd
    const float* k_new = nullptr;  // raw k of this position, kv floats
    const float* v_new = nullptr;
    float* kcache = nullptr;       // this layer's [max_seq][kv] keys
    float* vcache = nullptr;
    const uint32_t* pos = nullptr;  // device: current position
    const float* rope_cs = nullptr;  // [max_seq][hd/2][2] (cos, sin)
    float* part = nullptr;           // [kv_heads][nsplit][group][hd+2]
    uint32_t* counters = nullptr;    // [kv_heads], zero between launches
    float* out = nullptr;            // heads*hd
    uint32_t heads = 0, kv_heads = 0, hd = 0, nsplit = 0, rope_layout = 0;
    float scale = 0.f;               // 1/sqrt(hd)
    // QK-norm (MoE models): RMSNorm weights of the full q / k, applied before RoPE.
    const uint16_t* q_norm = nullptr;
    const uint16_t* k_norm = nullptr;
    float norm_eps = 0.f;
};
hipError_t launch_attn_decode(const AttnArgs& a, hipStream_t s);
size_t attn_part_floats(uint32_t heads, uint32_t kv_heads, uint32_t hd, uint32_t nsplit);
// Split count for a cache of max_seq positions (grid = nsplit x kv_heads; a
// step at position pos uses ceil((pos+1)/chunk) of them, chunk >= one LDS
// tile: 64 positions at head_dim <= 64, 32 above).
uint32_t attn_nsplit(uint32_t max_seq, uint32_t hd);

// ---------------------------------------------------------------------------
// Small kernels.
// ---------------------------------------------------------------------------
// Device step state read and advanced by the graph-replayable token step.
// A step embeds `token` at `pos`; the finish kernel then sets pos + 1 and
// picks the next token: prompt[pos + 1] while inside the prompt, else the
// argmax, which it appends to out_tokens when `counting` is set.
struct StepState {
    uint32_t token;       // token to embed
    uint32_t pos;         // position of this step
    uint32_t n_out;       // tokens appended to out_tokens so far
    uint32_t counting;    // 1: append post-prompt argmaxes to out_tokens
    uint32_t argmax;      // argmax of the last logits
    uint32_t prompt_len;  // tokens of `prompt` still to be fed, counted from pos 0
    uint32_t stop;        // set by the persistent step: EOS emitted or cache full
    uint32_t pad;
};

// copyEmbeddingToken (src/llm.zig:1373-1380): x = embed[token] as f32.
hipError_t launch_embed(int weight_kind, const void* embed, const StepState* st, float* x, uint32_t hidden,
                        hipStream_t s);
// Reduce block argmax keys, then advance the step state (see StepState).
hipError_t launch_argmax_finish(const unsigned long long* keys, uint32_t nkeys, const float* logits,
                                StepState* st, const uint32_t* prompt, uint32_t* out_tokens, uint32_t out_cap,
                                hipStream_t s);
// Host-free state reset (a kernel, so it is safe to capture and to enqueue
// back to back without a pinned staging buffer).
hipError_t launch_set_state(StepState* st, uint32_t token, uint32_t pos, uint32_t prompt_len, uint32_t counting,
                            hipStream_t s);

// ---------------------------------------------------------------------------
// Persistent decode step (decode_step.hip): bf16 weights only.
// ---------------------------------------------------------------------------
struct DecodeLayer {
    const uint16_t *input_norm, *q, *q_bias, *k, *k_bias, *v, *v_bias, *o, *post_norm, *gate, *up, *down;
    // Mixture-of-experts layers: router [E][H], QK-norm weights (null: none).
    const uint16_t *router, *q_norm, *k_norm;
};

// One GEMV phase of the persistent step: up to three stacked row segments
// (q | k | v; each of an even row count) or a gate and an up matrix. Built by
// the host in device memory; the kernel copies the table into LDS.
struct DecodeGemv {
    const uint16_t *w0, *w1, *w2;
    const uint16_t *b0, *b1, *b2;
    unsigned long long *o0, *o1, *o2;  // tagged outputs per segment (value bits | epoch << 32)
    float* plain;                      // logits phase: plain f32 outputs
    uint32_t r0, r1, r2;
    const uint16_t* w_up;
    uint32_t K;
    uint32_t split;  // one row per tile, its two halves streamed side by side (long rows, few of them)
    // Mixture-of-experts phases: 1 = gate/up of the routed experts (tile t:
    // slot t / r_slot, row t % r_slot of that slot's expert), 2 = down (a tile
    // of rows 2t, 2t+1 streams them from every slot's expert and adds the
    // router-weighted sum); w_expert elements lie between experts' matrices.
    uint32_t moe, r_slot;
    size_t w_expert;
};

// Values of DecodeStepParams::error: a poll passed its spin limit, the step
// state was out of range, or the host raised it before the launch (test hook).
// The word is zero at a launch's start unless an earlier launch of an
// unchecked sequence failed; the host clears it once it has reported it.
enum : uint32_t { kDecodeErrTimeout = 1, kDecodeErrState = 2, kDecodeErrInjected = 3 };

// What the persistent step's finishing thread leaves in pinned host memory at
// the end of its last step: the argmax, the stop flag, the device error word
// as it read it, then the launch's sequence number (the host compares it with
// the one it passed: a launch whose blocks left early never writes it).
struct HostStepOut {
    uint32_t seq;
    uint32_t argmax;
    uint32_t stop;
    uint32_t error;
};

// Pinned host memory through which the host hands a resident launch its next
// single step: the host writes token, pos (bit 31: write the step's logits to
// host memory) and cmd (0 step, 1 leave), then seq; the launch takes request
// seq == (its first step's sequence number) + (steps done).
struct HostMailbox {
    uint32_t seq;
    uint32_t token;
    uint32_t pos;
    uint32_t cmd;
};

// Activations of the persistent step are arrays of tagged 64-bit words: the
// f32 value (or u32) in the low half, the epoch of the phase that wrote it in
// the high half.
struct DecodeStepParams {
    uint32_t vocab, hidden, inter, layers, heads, kv_heads, hd, kvdim, rope_layout, max_seq;
    float eps, scale;
    const uint16_t* embed;
    const uint16_t* final_norm;
    const uint16_t* lm_head;  // the embedding when tied
    const DecodeLayer* layer;  // device array [layers]
    const DecodeGemv* gemv;    // device array [layers * 4 + 1]: per layer qkv, o, gate_up, down; then logits
    float* kcache;
    float* vcache;
    const float* rope_cs;
    unsigned long long* tx;         // residual stream: [2][hidden] (layer input | after attention)
    unsigned long long* tqkv;       // q | k | v
    unsigned long long* tattn;      // merged attention output [heads * hd]
    unsigned long long* tff;        // [inter]
    unsigned long long* tpart_ml;   // attention partials: (max, sum) [kv_heads][nsplit][group][2]
    unsigned long long* tpart_acc;  // attention partials: unnormalised out [kv_heads][nsplit][group][hd]
    unsigned long long* tkeys;      // argmax key of every wave: [waves][2] (high, low half)
    unsigned long long* tcopied;    // resident steps with logits: block b's slice copied to the host [blocks]
    unsigned long long* step_word;  // next token (0xffffffff: stop) published by the argmax
    float* logits;                  // [vocab]
    StepState* state;
    const uint32_t* prompt;
    uint32_t* out_tokens;
    uint32_t out_cap;
    uint32_t* error;  // non-zero: a poll timed out (all blocks leave)
    uint32_t epoch0;  // epoch of the first phase of this launch (>= 1)
    uint32_t nsplit, min_chunk;
    uint32_t n_steps;
    int64_t eos;  // < 0: none
    // Optional phase timing (100 MHz s_memrealtime ticks): kernel start in
    // timing[gridDim * timing_stride]; with timing_slots = 16, phase k of the
    // first step writes block b's staged input at timing[b * timing_stride +
    // k * 16] and wave w's end of the phase at [... + 1 + w].
    unsigned long long* timing;
    uint32_t timing_stride;
    uint32_t timing_slots;
    uint32_t table_lds_offset;  // bytes: where the kernel copies gemv[] / norms into LDS
    // Gate/up tiles prefetched into LDS during the attention phase by the
    // blocks that run no attention unit: g_lds_tiles tiles per block (0: off),
    // tiles [0, g_lds_tiles1) from byte g_lds_offset1 of the dynamic LDS (the
    // attention / down-projection staging space, which those blocks do not use
    // while the tiles are held), the rest from byte g_lds_offset2.
    uint32_t g_lds_offset1, g_lds_tiles1;
    uint32_t g_lds_offset2;
    uint32_t g_lds_tiles;
    uint32_t g_lds_park;  // byte offset of [8 waves][64] f32: LDS tile results until they are written
    // Nullable: the down-projection phase of layer l also writes the residual
    // stream after the layer to hidden_dbg[l * hidden ..] (plain f32 stores;
    // with n_steps > 1 the last step's values remain).
    float* hidden_dbg;
    // Mixture-of-experts step (experts > 0): the gate/up phase routes (router
    // logits as tagged words trl[experts], one row per producing wave; every
    // block with tiles takes the softmax + top-k) and runs the top_k experts;
    // `inter` is then top_k * the expert width (the down phase's staged input).
    uint32_t experts, top_k;
    unsigned long long* trl;
    // Single-step calls (init_step != 0): the token and position come from
    // here instead of the step state, which block 0's first thread then
    // initialises (no prompt, no counting) before any phase.
    uint32_t init_step, init_token, init_pos;
    // Nullable pinned host memory, written at the end of the last step.
    HostStepOut* host_out;
    uint32_t host_seq;
    // Resident single steps (mbox != nullptr, with init_step and host_out):
    // after each step the finishing thread reports it in host_out (sequence
    // number host_seq + step) and waits up to linger_ticks (100 MHz clock)
    // for the next request in mbox, which the other blocks take from the step
    // words; no request in time, a leave command or n_steps reached: the
    // launch ends. host_logits: where a step that asks for them writes its
    // logits (pinned host memory); init_logits: whether the first step does.
    HostMailbox* mbox;
    uint32_t linger_ticks;
    float* host_logits;
    uint32_t init_logits;
};

// LDS bytes of one gate/up tile (gate row + up row of K bf16 weights, in
// 1 KiB wave loads).
uint32_t decode_step_glds_tile_bytes(uint32_t K);
// Where the gate/up tiles fit (fills the offsets and first-range count) and
// the new dynamic LDS size in *lds; returns the tile count per block.
uint32_t decode_step_glds_plan(uint32_t hidden, uint32_t inter, uint32_t hd, size_t* lds, uint32_t* off1,
                               uint32_t* tiles1, uint32_t* off2, uint32_t* park);

size_t decode_step_table_offset(uint32_t hidden, uint32_t inter, uint32_t hd);
size_t decode_step_lds_bytes(uint32_t hidden, uint32_t inter, uint32_t layers, uint32_t hd);
uint32_t decode_step_phases_per_step(uint32_t layers);
// moe: the mixture-of-experts instantiation (head_dim 64 or 128 only).
bool decode_step_moe_supported(uint32_t hd);
hipError_t decode_step_max_blocks(uint32_t hd, size_t lds, int* blocks_per_cu, bool moe = false);
hipError_t launch_decode_step(const DecodeStepParams& p, uint32_t blocks, size_t lds, hipStream_t s);

// ---------------------------------------------------------------------------
// Batched prefill (prefill.hip): bf16-weight GEMM on MFMA with f32 activations
// split hi/lo, and the per-row kernels around it.
// ---------------------------------------------------------------------------
enum GemmMode {
    kGemmPlain = 0,   // out[m][n] = A_m . W_n (+ bias[n]); W stacked from up to 3 segments
    kGemmResid = 1,   // out[m][n] += A_m . W_n
    kGemmGateUp = 2,  // out[m][n] = silu(A_m . Wg_n) * (A_m . Wu_n)
};

struct GemmArgs {
    const float* a = nullptr;          // [M][lda] f32
    uint32_t lda = 0;
    const float* row_scale = nullptr;  // with norm_w: A_m = (a_m * norm_w) * row_scale[m]
    const uint16_t* norm_w = nullptr;  // [K] bf16
    const uint16_t* w[3] = {nullptr, nullptr, nullptr};  // bf16 [rows][K] segments (GateUp: w[0] = gate)
    const uint16_t* bias[3] = {nullptr, nullptr, nullptr};
    uint32_t seg_end[3] = {0, 0, 0};   // cumulative rows of the segments (seg_end[2] = N for Plain)
    const uint16_t* w_up = nullptr;    // GateUp: up rows
    float* out = nullptr;
    uint32_t ldo = 0;
    uint32_t M = 0, N = 0, K = 0;      // K % 8 == 0
    // Device scratch of gemm_split_elems(M, K) bf16: the launcher splits A
    // (normalised when norm_w is set) into hi | lo planes there before the
    // GEMM reads it -- unless a_ready: a producer already wrote the planes.
    // Rows are gemm_kp(K) elements with a zero tail; a_plane elements lie
    // between the hi and the lo plane (0: M * gemm_kp(K)).
    uint16_t* a_hl = nullptr;
    bool a_ready = false;
    size_t a_plane = 0;
    // GateUp only: write silu(gate) * up as split planes for the next GEMM
    // (rows of gemm_kp(N) with a zero tail, out_plane elements apart) instead
    // of f32 rows in out.
    uint16_t* out_hl = nullptr;
    size_t out_plane = 0;
    // GateUp: f32 scratch of M * 2N. When set, few row tiles may split K: the
    // gate and up sums are added there atomically (the launcher zeroes it) and
    // a SwiGLU pass writes out / out_hl.
    float* gu_acc = nullptr;
    // Gather: A row m of the split planes is a[a_rows[m]], normalised with
    // row_scale[a_rows[m]] (launch_gemm_grouped's gate/up input).
    const uint32_t* a_rows = nullptr;
    // launch_gemm_grouped: row tiles from a device table, tiles[0].x = count,
    // tiles[1 + t] = {expert, first row, end row, 0} (rows of the A planes and
    // of the output); the expert's W is w[0] (and w_up) + expert * w_expert.
    const uint4* tiles = nullptr;
    uint32_t max_tiles = 0;
    size_t w_expert = 0;
    // Plain / Resid: when set and the launch splits K (gemm_splits > 1), each
    // split stores its partial sums to part[split][M][N] (f32, at most
    // gemm_part_elems(); split 0 includes the bias) instead of adding them
    // atomically into out, which is then left for the consumer: Resid adds
    // nothing to out, Plain does not zero it. The consumer sums the splits in
    // order (deterministic).
    float* part = nullptr;
};
// K splits a launch of launch_gemm_bf16 will use (1: no split), and the
// capacity of the partial sums buffer any launch needs (elements).
uint32_t gemm_splits(int mode, const GemmArgs& g);
size_t gemm_part_elems();
__host__ __device__ inline uint32_t gemm_kp(uint32_t K) { return (K + 31) / 32 * 32; }
size_t gemm_split_elems(uint32_t M, uint32_t K);
// Most rows for which a GateUp GEMM of N outputs may split K (gu_acc of
// rows * 2N floats is then needed).
uint32_t gemm_gateup_split_rows(uint32_t N);
hipError_t launch_gemm_bf16(int mode, const GemmArgs& g, hipStream_t s);
// Rows of one grouped GEMM tile; a table for M grouped rows over E experts
// holds at most grouped_gemm_max_tiles(M, E) tiles.
uint32_t grouped_gemm_tile_rows();
uint32_t grouped_gemm_max_tiles(uint32_t M, uint32_t E);
// Per-expert GEMMs over grouped rows (kGemmGateUp or kGemmPlain; no K split,
// no bias): each tile of g.tiles multiplies its rows by its expert's W.
hipError_t launch_gemm_grouped(int mode, const GemmArgs& g, hipStream_t s);

// part / splits: the K-split partial sums of the Resid GEMM that produced x
// ([splits][rows][n]; nullptr or splits <= 1: x is complete), added into x first.
hipError_t launch_row_rms(float* x, uint32_t n, uint32_t rows, float eps, float* scale, hipStream_t s,
                          const float* part = nullptr, uint32_t splits = 0);
// launch_row_rms (with the partial sums) and the split pass of a normalising
// GEMM in one launch: writes the GEMM's A planes of rmsnorm(x) with weight
// norm_w (hi at a_hl, lo a_plane elements later); the GEMM then runs with
// a_ready. For rows of n floats with row_norm_split_fits(n) (n <= 8192).
bool row_norm_split_fits(uint32_t n);
hipError_t launch_row_norm_split(float* x, uint32_t n, uint32_t rows, float eps, const uint16_t* norm_w,
                                 const float* part, uint32_t splits, uint16_t* a_hl, size_t a_plane, hipStream_t s);
hipError_t launch_prefill_embed(const uint16_t* embed, const uint32_t* tokens, uint32_t rows, uint32_t hidden,
                                float* x, hipStream_t s);

struct PrefillRopeArgs {
    float* qkv;              // [rows][ld]: q | k | v of each row
    uint32_t ld, rows, start;
    uint32_t heads, kv_heads, hd, kvdim, rope_layout;
    const float* rope_cs;    // [max_seq][hd/2][2]
    float* kcache;           // this layer's [max_seq][kvdim]
    float* vcache;
    // QK-norm (models that carry it): q = q_norm * (q * 1/sqrt(mean(q^2) + eps))
    // over the row's full q, the same for k, before the rotation.
    const uint16_t* q_norm = nullptr;
    const uint16_t* k_norm = nullptr;
    float norm_eps = 0.f;
    // The q|k|v GEMM's K-split partial sums ([splits][rows][ld]) when it split
    // K into a partial-sum buffer: summed into qkv first.
    const float* part = nullptr;
    uint32_t splits = 0;
    // The MFMA attention's packed K/V tiles (prefill_kv_pack_bytes(start +
    // rows, ..)): the new rows' images are written here too, and the last
    // tile's rows past them zeroed; the attention launch then packs only the
    // tiles of rows before start (PrefillAttnArgs::new_rows_packed).
    void* kv_pack = nullptr;
    size_t kv_pack_bytes = 0;
};
hipError_t launch_prefill_rope_kv(const PrefillRopeArgs& a, hipStream_t s);

struct PrefillAttnArgs {
    const float* q;          // [rows][ldq], rotated
    uint32_t ldq;
    const float* kcache;     // this layer's [max_seq][kvdim]
    const float* vcache;
    float* out;              // [rows][ldo]
    uint32_t ldo;
    uint32_t rows, start;    // row t sits at position start + t
    uint32_t heads, kv_heads, kvdim;
    float scale;
    void* kv_pack = nullptr;       // MFMA kernel: packed K/V tiles, prefill_kv_pack_bytes(start + rows, ..)
    size_t kv_pack_bytes = 0;
    uint32_t kv_tiles = 0;         // set by launch_prefill_attn
    // MFMA kernel: write the output as GEMM split planes (rows of
    // gemm_kp(heads * head_dim), out_plane elements apart) instead of out.
    uint16_t* out_hl = nullptr;
    size_t out_plane = 0;
    // The RoPE / KV pass already wrote the images of rows start .. start +
    // rows - 1 (and the last tile's padding) into kv_pack.
    bool new_rows_packed = false;
};
// Bytes of the packed K/V tiles the MFMA attention kernel reads for `keys`
// cache rows (0 for an unsupported head_dim).
size_t prefill_kv_pack_bytes(uint32_t keys, uint32_t kv_heads, uint32_t hd);
hipError_t launch_prefill_attn(const PrefillAttnArgs& a, uint32_t hd, hipStream_t s);
// false (default): the MFMA flash-attention kernel; true: the f32 vector kernel.
extern bool prefill_attn_vector;
// Form of the MFMA flash-attention launch: -1 chosen by the prompt (default),
// 0 blocks of 128 query vectors, 1 the same with two key groups, 2 blocks of
// 64 query vectors with two key groups (group size up to 64).
extern std::atomic<int> prefill_fa_form;

// ---------------------------------------------------------------------------
// Mixture-of-experts step pieces (moe.hip).
// ---------------------------------------------------------------------------
constexpr int kMaxTopK = 16;

struct MoeGemvArgs {
    const uint16_t* w = nullptr;         // GateUp: [E][2 rows_per_slot][K]; Down: [E][rows_per_slot][K]
    const uint32_t* experts = nullptr;   // [top_k] expert ids (device)
    uint32_t top_k = 0, rows_per_slot = 0, K = 0;
    const float* x = nullptr;            // GateUp: residual stream (K); Down: activations (top_k * K)
    uint32_t x_len = 0;
    const uint16_t* norm_w = nullptr;    // GateUp: post-attention RMSNorm weight
    float eps = 0.f;
    float* out = nullptr;                // [top_k * rows_per_slot]
};
hipError_t moe_gemv_init_attributes();
hipError_t launch_moe_gemv(int mode, const MoeGemvArgs& a, hipStream_t s);  // kGemvGateUp
// Down projection of the selected experts added into x (float atomics).
hipError_t launch_moe_down(const MoeGemvArgs& a, float* x, const float* slot_w, hipStream_t s);
struct MoeRouterArgs {
    const uint16_t* w = nullptr;       // [E][H] router
    const float* x = nullptr;          // residual stream [H]
    const uint16_t* norm_w = nullptr;  // post-attention RMSNorm weight
    float eps = 0.f;
    uint32_t H = 0, E = 0, top_k = 0;
    float* logits = nullptr;           // [E] scratch
    uint32_t* ticket = nullptr;        // zero between launches (the routing block resets it)
    uint32_t* idx = nullptr;           // [top_k] selected experts
    float* weight = nullptr;           // [top_k] their probabilities
};
// Router GEMV + softmax + top-k in one launch.
hipError_t launch_moe_router(const MoeRouterArgs& a, hipStream_t s);

// Batched (prefill) routing of `rows` residual rows: per row the router
// logits of norm(x_r) (row_scale from launch_row_rms), softmax, top-k into
// idx[r * top_k ..] and weight[r * top_k ..].
struct MoeRouteRowsArgs {
    const uint16_t* w = nullptr;       // [E][H] router
    const float* x = nullptr;          // [rows][H]
    const float* row_scale = nullptr;  // [rows]
    const uint16_t* norm_w = nullptr;  // post-attention RMSNorm weight
    uint32_t rows = 0, H = 0, E = 0, top_k = 0;
    uint32_t* idx = nullptr;
    float* weight = nullptr;
};
hipError_t launch_moe_route_rows(const MoeRouteRowsArgs& a, hipStream_t s);
// Groups the rows * top_k (row, slot) pairs by expert, pairs of one expert
// in pair order: grouped_rows[g] = the row of grouped pair g, pair_pos[p] =
// where pair p went, tiles = the grouped GEMM's tile table (tile_rows rows per
// tile, at most grouped_gemm_max_tiles entries).
hipError_t launch_moe_group(const uint32_t* idx, uint32_t rows, uint32_t top_k, uint32_t E, uint32_t tile_rows,
                            uint32_t* grouped_rows, uint32_t* pair_pos, uint4* tiles, hipStream_t s);
// x[r] += sum over row r's experts in ascending expert id of
// eout[pair_pos[p]] * weight[p] (eout rows of H floats).
hipError_t launch_moe_combine(const float* eout, const uint32_t* pair_pos, const uint32_t* idx, const float* weight,
                              uint32_t rows, uint32_t top_k, uint32_t H, float* x, hipStream_t s);

// ---------------------------------------------------------------------------
// Token sampling (sample.hip): Sampler.next on device logits.
// ---------------------------------------------------------------------------
constexpr int kMaxSampleTopK = 1024;
struct SampleArgs {
    const float* logits = nullptr;
    uint32_t vocab = 0;
    uint32_t* counts = nullptr;       // [vocab] repeat counts of the window (nullable: no penalty)
    float temperature = 0.f, top_p = 1.f, repeat_penalty = 1.f;
    uint32_t top_k = 0, repeat_last_n = 0;
    unsigned long long* prng = nullptr;  // device xoshiro256++ state [4]
    uint32_t* result = nullptr;       // nullable: the token
    StepState* state = nullptr;       // nullable: advanced like the greedy finish
    uint32_t advance_pos = 1;         // 0 for a sample taken before any forward
    const uint32_t* prompt = nullptr;
    uint32_t n_prompt = 0;
    uint32_t* out_tokens = nullptr;
    uint32_t out_cap = 0;
    // Scratch of the two-stage top-k (nullable: one block scans the vocab):
    // sample_cand_elems(vocab) keys and sample_nf_elems(vocab) counts.
    unsigned long long* cand_buf = nullptr;
    uint32_t* cand_nf = nullptr;
    // Scratch of the whole-vocabulary path (candidate limits over 1024: top_k
    // 0 or > 1024), sample_full_bytes(vocab) bytes (nullable: such limits are
    // an error).
    void* full = nullptr;
    // Test hook of the whole-vocabulary path (each nullable): the candidates'
    // ids, probabilities and running sums in candidate order, and their count.
    uint32_t* trace_ids = nullptr;
    float* trace_probs = nullptr;
    float* trace_sums = nullptr;
    uint32_t* trace_count = nullptr;
};
size_t sample_cand_elems(uint32_t vocab);
size_t sample_nf_elems(uint32_t vocab);
// Scratch bytes of the whole-vocabulary path (sort keys and ids twice,
// probabilities, prefix sums, the sort's temporary storage); 0 on failure.
size_t sample_full_bytes(uint32_t vocab);
hipError_t launch_sample(const SampleArgs& a, hipStream_t s);
hipError_t launch_sample_counts(uint32_t* counts, uint32_t vocab, const uint32_t* prompt, uint32_t n_prompt,
                                uint32_t last_n, hipStream_t s);

// Dtype conversion for device-side loading (convert.hip): n elements of type
// src_type (0 f32, 1 f16, 2 bf16) into dst elements of type kind (0 f32, 1 bf16).
hipError_t launch_convert(const void* src, uint32_t src_type, void* dst, uint32_t kind, size_t n, hipStream_t s);

}  // namespace vvli
