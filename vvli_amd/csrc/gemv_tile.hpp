// gemv_tile.hpp -- wave-level GEMV tiles shared by the standalone GEMV
// kernels and the persistent decode-step kernel.
//
// A tile is R rows (R gate + R up rows in the SwiGLU mode) of a row-major
// [rows][K] weight matrix. Rows are cut into 16-byte units; lane l takes
// units l, l+64, ..., so each wave load is 1 KiB contiguous. A tile is walked
// in items of kNJC units per lane per row: issue() puts one item's loads in
// flight, consume() multiplies it with x staged in LDS.
#pragma once

#include "device_common.hpp"
#include "kernels.hpp"

namespace vvli {

constexpr int kNJC = 4;  // units per lane per row per item

template <int MODE> struct ModeCfg { static constexpr int R = 2; };
template <> struct ModeCfg<kGemvGateUp> { static constexpr int R = 1; };  // 1 gate + 1 up row per tile

template <int MODE> constexpr int mode_nr() { return (MODE == kGemvGateUp ? 2 : 1) * ModeCfg<MODE>::R; }

// Row pointers of one tile.
template <typename WT, int MODE, int NR>
struct Tile {
    const WT* p[NR];
    uint32_t row[NR / (MODE == kGemvGateUp ? 2 : 1)];
    int seg[NR];
    bool valid[NR];
};

template <typename WT, int MODE>
__device__ __forceinline__ void make_tile(const GemvArgs& a, uint32_t tile, uint32_t K,
                                 Tile<WT, MODE, (MODE == kGemvGateUp ? 2 : 1) * ModeCfg<MODE>::R>& t) {
    constexpr int R = ModeCfg<MODE>::R;
    const uint32_t total = a.rows[0] + a.rows[1] + a.rows[2];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        uint32_t g = tile * R + r;
        const bool v = g < total;
        if (!v) g = total - 1;
        int seg = 0;
        uint32_t srow = g;
        if (srow >= a.rows[0]) {
            srow -= a.rows[0];
            seg = 1;
            if (srow >= a.rows[1]) {
                srow -= a.rows[1];
                seg = 2;
            }
        }
        t.p[r] = static_cast<const WT*>(a.w[seg]) + (size_t)srow * K;
        t.row[r] = srow;
        t.seg[r] = seg;
        t.valid[r] = v;
        if constexpr (MODE == kGemvGateUp) {
            t.p[R + r] = static_cast<const WT*>(a.w_up) + (size_t)srow * K;
            t.seg[R + r] = 0;
            t.valid[R + r] = v;
        }
    }
}

template <typename WT, int NR>
__device__ __forceinline__ void issue(uint4 (&buf)[NR][kNJC], const WT* const (&p)[NR], uint32_t ubase, uint32_t U, int lane) {
    constexpr int E = WeightTraits<WT>::kPerUnit;
#pragma unroll
    for (int j = 0; j < kNJC; ++j) {
        const uint32_t u = ubase + j * kWave + lane;
#pragma unroll
        for (int r = 0; r < NR; ++r) buf[r][j] = u < U ? load_unit(p[r] + (size_t)u * E) : make_uint4(0, 0, 0, 0);
    }
}

template <typename WT, int NR>
__device__ __forceinline__ void consume(const uint4 (&buf)[NR][kNJC], const float* xs, uint32_t ubase, uint32_t U, int lane,
                               float (&acc)[NR]) {
    constexpr int E = WeightTraits<WT>::kPerUnit;
#pragma unroll
    for (int j = 0; j < kNJC; ++j) {
        const uint32_t u = ubase + j * kWave + lane;
        if (u < U) {
            float xv[E];
#pragma unroll
            for (int e = 0; e < E; e += 4) {
                const float4 t = *reinterpret_cast<const float4*>(xs + (size_t)u * E + e);
                xv[e] = t.x;
                xv[e + 1] = t.y;
                xv[e + 2] = t.z;
                xv[e + 3] = t.w;
            }
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                float wf[E];
                WeightTraits<WT>::expand(buf[r][j], wf);
#pragma unroll
                for (int e = 0; e < E; ++e) acc[r] = fmaf(wf[e], xv[e], acc[r]);
            }
        }
    }
}


}  // namespace vvli
