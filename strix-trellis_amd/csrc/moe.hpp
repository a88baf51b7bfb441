// Routed-expert (MoE) block: host-side launch interface.
//
// Operator (reference docs/TP_RANK.md:64-76, include/strix_trellis.h:207-233):
//   hidden[r,s] = SwiGLU(gate_e(X[r]), up_e(X[r]))        e = ids[r,s]
//   Y[r]        = alpha * sum_s(score[r,s] * down_e(hidden[r,s])) + beta * Y[r]
// Every projection is a complete EXL3 linear (input stage, core, output
// stage with svh and bias).  The slot sum runs s = 0..k-1 from +0, each term
// RN32(score * value) added with one FP32 rounding; an exactly zero score
// skips its term and reads neither hidden values nor down weights.  A token
// whose routes are invalid (id outside the bank, repeated id, non-finite or
// negative score) gets an all-NaN output row; no invalid id reaches the bank.
//
// Both launches take the routes as device buffers [rows][k] of bank indices;
// the plans built from host routes upload them once.  The union of experts is
// resolved inside the kernels: the first valid occurrence of an expert in
// row-major route order leads its group, every other occurrence's workgroups
// exit, so each expert's weights are streamed once for all its tokens.
#pragma once
#include "backend.hpp"

namespace stx {

struct MoeExpert {
    GroupWeights gate, up, down;
};

constexpr uint32_t MOE_MAX_ROUTES = 64;   // rows * k: one wave resolves all of them
constexpr uint32_t MOE_MAX_TOPK = 8;
constexpr uint32_t MOE_MAX_BANK = 256;       // experts a bank may hold

struct MoeArgs {
    const MoeExpert* bank;
    const uint32_t* ids;      // [rows][k] bank indices
    const float* scores;      // [rows][k]
    const float* x;           // [rows][x_stride], width I
    float* y;                 // [rows][y_stride], width I
    float* hidden;            // [rows][k][H] F32
    float* p_gu;              // [rows*k][s_gu][2][H] partial planes of gate (0) and up (1)
    float* p_d;               // [rows*k][s_d][I] partial planes of down
    uint16_t* a_gu;           // [rows*k][2][I] FP16 core inputs of gate (0) and up (1), per route
    uint32_t* c_gu;           // [rows*k][H/128] arrival counters, zero between launches
    uint32_t* c_d;            // [rows][I/128]
    uint64_t x_stride, y_stride;
    uint32_t bank_count, rows, topk, I, H;
    uint32_t s_gu, bps_gu, s_d, bps_d;
    uint32_t gate_bits, up_bits, down_bits;
    float alpha, beta;
    uint32_t down_mode;       // MoeDownMode of a down launch
};

// What a down launch does.  The staged modes write the per-split partial
// planes p_d of every computed route (valid token, non-zero score) and
// nothing else: no arrivals, no output, no NaN rows.
enum MoeDownMode : uint32_t {
    kMoeDownFused = 0,       // planes, arrivals, ordered finish by the last arrival
    kMoeDownCore = 1,        // planes only; each expert group streams its weights once
    kMoeDownRouteCore = 2,   // planes only; one route per workgroup (no expert grouping)
};

// Split-K decomposition of one MoE projection with `blocks` 16-channel input
// blocks: the largest whole-H128 split of at most max_bps blocks.  Long splits
// amortise each workgroup's route resolution and input stage over more decode
// work; the maxima size the kernels' LDS activation buffers.
struct MoeSplit {
    uint32_t bps, splits;
};
constexpr int MOE_GU_MAX_BPS = 64;   // gate/up: input I
constexpr int MOE_D_MAX_BPS = 96;    // down: input H
MoeSplit moe_split(uint32_t input, uint32_t max_bps);
// 128-channel groups that down split s touches: its blocks are
// [s bps, (s + 1) bps), which need not start or end on a group boundary.
constexpr uint32_t moe_down_groups(uint32_t bps, uint32_t s) { return (s * bps + bps + 7) / 8 - (s * bps) / 8; }
// Down split of a split plan, whose planes P [rows][k][S][I] are the staged
// checkpoint: the reference's four equal parts of the T = H / 16 input blocks,
// split s over blocks [s T / 4, (s + 1) T / 4) (reference
// src/tp_fused_layout.hpp:19-24, P indexed as src/tp_moe_split_layout.hpp:119-122),
// when every part's groups fit the down kernel's LDS; otherwise moe_split.
MoeSplit moe_split_staged(uint32_t H);
uint64_t moe_partial_floats(uint32_t routes, uint32_t I, uint32_t H);
uint64_t moe_counter_words(uint32_t rows, uint32_t routes, uint32_t I, uint32_t H);

// Gate/up: the routes' core inputs (one launch), then the expert cores and
// SwiGLU (a second launch that reads them).
hipError_t launch_moe_gate_up(const MoeArgs& a, hipStream_t stream);
hipError_t launch_moe_down(const MoeArgs& a, hipStream_t stream);
// Bytes of a_gu for `routes` routes of input width I.
constexpr uint64_t moe_core_input_bytes(uint32_t routes, uint32_t I) { return uint64_t(routes) * 2 * I * 2; }
// Staged down: the core alone in `mode` (kMoeDownCore or kMoeDownRouteCore),
// and the finish alone, which folds the planes p_d as they are in memory
// (ascending split from +0, output stage, ordered score-weighted slot sum,
// alpha/beta; NaN rows for invalid tokens), with the fused finish's code.
hipError_t launch_moe_down_core(const MoeArgs& a, MoeDownMode mode, hipStream_t stream);
hipError_t launch_moe_down_finish(const MoeArgs& a, hipStream_t stream);
uint64_t moe_gate_up_partial_floats(uint32_t routes, uint32_t I, uint32_t H);
uint64_t moe_down_partial_floats(uint32_t routes, uint32_t I, uint32_t H);   // plain plans' planes
// Diagnostic: h[i] = SwiGLU(g[i], u[i]) with the block's activation arithmetic.
hipError_t launch_moe_swiglu(const float* g, const float* u, float* h, uint64_t n, hipStream_t stream);

}  // namespace stx
