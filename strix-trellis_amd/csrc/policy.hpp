// Host-side decomposition policy shared by the launch code and the C ABI
// layer (implemented in policy.cpp, which holds no device code).
#pragma once
#include "backend.hpp"
#include "moe.hpp"

namespace stx {

inline uint64_t align256(uint64_t v) { return (v + 255) & ~uint64_t(255); }

// Prefill GEMM (gemm.hip): rows per pass, fragment-order input bytes, column
// and K decomposition of a wide (M >= 256) pass, split-tile handoff.
struct WideSplit {
    uint32_t full, half;   // 256-column blocks of each width
};
struct Handoff {
    uint32_t q = 0, x = 0;
};
constexpr uint32_t kWideSplitMinStages = 8;   // 64-channel stages per K split, at least
uint64_t gemm_pass_rows(const DeviceWeights& w);
uint64_t afrag_bytes(const DeviceWeights& w, uint64_t m);
bool wide_can_split(const DeviceWeights& w);
WideSplit wide_split(uint64_t m, const DeviceWeights& w);
bool gemm_wide(uint64_t m, const DeviceWeights& w);
uint32_t wide_splits(uint64_t m, const DeviceWeights& w);
uint32_t narrow_splits(const DeviceWeights& w);
Handoff gemm_handoff(uint64_t m, const DeviceWeights& w);
uint64_t handoff_bytes(uint32_t x);
uint64_t pass_workspace(const DeviceWeights& w, uint64_t m);

}  // namespace stx
