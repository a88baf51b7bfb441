// H128 input and output stages for gfx950 wave64.
//
// Arithmetic (reference docs/NUMERICS.md:30-65, python/strix_trellis/linear.py:82-163):
//   input : a = RN16( H32( f32( RN16( RN32(x * f32(suh)) ) ) ) )
//   output: y = RN32(H32(core) * f32(svh)) [+ bias] ; y = RN32(y * alpha) ; y = RN32(y + RN32(beta * old)) iff beta != 0
//   H32   : butterflies of strides 1, 2, ..., 64 in that order, each add/sub
//           rounded to FP32, then one multiply by RN32(1/sqrt(128)).
// Every step is a single IEEE FP32 operation (the library is compiled with
// -ffp-contract=off), so any schedule that performs the same operations on the
// same pairs gives the same bits.  Here one wave owns one 128-block: lane l
// holds elements l and l+64; strides 1..32 pair lanes through shuffles, stride
// 64 pairs the two registers of a lane.
#pragma once
#include <type_traits>

#include "trellis.hpp"

namespace stx {

// Partial sums that cross workgroups (and XCDs, each with its own L2) are
// written and read with agent-scope coherent accesses (sc1): completed
// stores are visible device-wide without the full-L2 writeback an agent-scope
// release fence costs.
__device__ __forceinline__ void store_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr float INV_SQRT128 = 0x1.6a09e6p-4f;   // RN32(1/sqrt(128))

__device__ __forceinline__ float half_bits_to_float(uint16_t bits) {
    return (float)__builtin_bit_cast(_Float16, bits);
}

// v of lane l ^ S, without the LDS crossbar: DPP quad permutes for strides 1
// and 2, two bank-masked row shifts for 4, a row rotate for 8, and the gfx950
// permlane swaps (odd/even 16-lane rows, upper/lower 32-lane halves) for 16
// and 32.
template <int S>
__device__ __forceinline__ float xor_lane(float v) {
    const int lane = threadIdx.x & 63;
    const int iv = __builtin_bit_cast(int, v);
    if constexpr (S == 1) {
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0xB1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
    } else if constexpr (S == 2) {
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x4E, 0xf, 0xf, false));   // quad_perm 2,3,0,1
    } else if constexpr (S == 4) {
        // Banks 0 and 2 of each row (lanes 0-3, 8-11) take lane + 4 (row_shl:4),
        // banks 1 and 3 take lane - 4 (row_shr:4) over that result.
        const int up = __builtin_amdgcn_update_dpp(iv, iv, 0x104, 0xf, 0x5, false);
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(up, iv, 0x114, 0xf, 0xA, false));
    } else if constexpr (S == 8) {
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x128, 0xf, 0xf, false));  // row_ror:8
    } else if constexpr (S == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(uint32_t(iv), uint32_t(iv), false, false);
        return __builtin_bit_cast(float, (lane & 16) ? r[0] : r[1]);
    } else {
        static_assert(S == 32, "lane exchange stride");
        const auto r = __builtin_amdgcn_permlane32_swap(uint32_t(iv), uint32_t(iv), false, false);
        return __builtin_bit_cast(float, (lane & 32) ? r[0] : r[1]);
    }
}

// +1 on lanes with bit S clear, -1 where it is set.
template <int S>
__device__ __forceinline__ float lane_sign() {
    return (threadIdx.x & S) ? -1.0f : 1.0f;
}

// One butterfly level at DPP stride S (1, 2, 4, 8) on a lane's value: the
// lower lane keeps own + partner, the upper one partner - own.  Both are
// fma(sign, own, partner): sign * own is exact (a sign flip), so the fma
// rounds once, to the same bits as the add or subtract, signed zeros
// included (a NaN operand gives a NaN either way).
template <int S>
__device__ __forceinline__ float bfly_lane(float v, float sign) {
    return __builtin_fmaf(sign, v, xor_lane<S>(v));
}

// The level at stride 16 or 32 on the lane's two values at once: one swap
// puts each lane's value beside its partner's (own and partner of v0 on the
// lower lanes, of v1 on the upper ones), one add and one subtract form both
// results in the operand order above, and a second swap returns them to
// their lanes.
template <int S>
__device__ __forceinline__ void bfly_pair(float& v0, float& v1) {
    static_assert(S == 16 || S == 32, "swap stride");
    const uint32_t a = __builtin_bit_cast(uint32_t, v0), b = __builtin_bit_cast(uint32_t, v1);
    const auto s1 = S == 16 ? __builtin_amdgcn_permlane16_swap(a, b, false, false)
                            : __builtin_amdgcn_permlane32_swap(a, b, false, false);
    const float x = __builtin_bit_cast(float, uint32_t(s1[0])), y = __builtin_bit_cast(float, uint32_t(s1[1]));
    const uint32_t lo = __builtin_bit_cast(uint32_t, x + y), hi = __builtin_bit_cast(uint32_t, x - y);
    const auto s2 = S == 16 ? __builtin_amdgcn_permlane16_swap(lo, hi, false, false)
                            : __builtin_amdgcn_permlane32_swap(lo, hi, false, false);
    v0 = __builtin_bit_cast(float, uint32_t(s2[0]));
    v1 = __builtin_bit_cast(float, uint32_t(s2[1]));
}

template <int S>
__device__ __forceinline__ void butterfly(float& v0, float& v1) {
    if constexpr (S >= 16) {
        bfly_pair<S>(v0, v1);
    } else {
        const float sign = lane_sign<S>();
        v0 = bfly_lane<S>(v0, sign);
        v1 = bfly_lane<S>(v1, sign);
    }
}

__device__ __forceinline__ void h32_wave(float& v0, float& v1) {
    butterfly<1>(v0, v1);
    butterfly<2>(v0, v1);
    butterfly<4>(v0, v1);
    butterfly<8>(v0, v1);
    butterfly<16>(v0, v1);
    butterfly<32>(v0, v1);
    const float a = v0, b = v1;
    v0 = rn32(a + b);
    v1 = rn32(a - b);
    v0 = rn32(v0 * INV_SQRT128);
    v1 = rn32(v1 * INV_SQRT128);
}

// H32 of P independent (v0, v1) pairs, stage by stage across the pairs so
// their dependency chains interleave (same operations, same bits as h32_wave).
template <int P>
__device__ __forceinline__ void h32_wave_multi(float (&v0)[P], float (&v1)[P]) {
    auto stage = [&](auto s) {
        constexpr int S = decltype(s)::value;
#pragma unroll
        for (int i = 0; i < P; ++i) butterfly<S>(v0[i], v1[i]);
    };
    stage(std::integral_constant<int, 1>{});
    stage(std::integral_constant<int, 2>{});
    stage(std::integral_constant<int, 4>{});
    stage(std::integral_constant<int, 8>{});
    stage(std::integral_constant<int, 16>{});
    stage(std::integral_constant<int, 32>{});
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const float a = v0[i], b = v1[i];
        v0[i] = rn32(rn32(a + b) * INV_SQRT128);
        v1[i] = rn32(rn32(a - b) * INV_SQRT128);
    }
}

// Input stage of one 128-block, split into the loads and the arithmetic so a
// kernel can issue the loads ahead of other memory traffic.  x and suh point
// at the block's first channel; a dead row (live = false) reads nothing and
// produces zeros.
struct InputLoad {
    float x0, x1;
    uint16_t u0, u1;
};

__device__ __forceinline__ InputLoad input_load(const float* x, const uint16_t* suh, bool live) {
    // Branch-free: a dead row still loads (from a valid address) and is zeroed
    // afterwards, so the loads stay in one basic block with their issuers.
    const int lane = threadIdx.x & 63;
    InputLoad l;
    const float a = ld_global(x + lane), b = ld_global(x + lane + 64);
    l.x0 = live ? a : 0.0f;
    l.x1 = live ? b : 0.0f;
    l.u0 = ld_global(suh + lane);
    l.u1 = ld_global(suh + lane + 64);
    return l;
}

// The wave writes the 128 FP16 core inputs to `out` (LDS or global).
// Core inputs of elements lane and lane+64 of the block.
__device__ __forceinline__ void input_values(const InputLoad& l, _Float16& o0, _Float16& o1) {
    float v0 = (float)(_Float16)rn32(l.x0 * half_bits_to_float(l.u0));
    float v1 = (float)(_Float16)rn32(l.x1 * half_bits_to_float(l.u1));
    h32_wave(v0, v1);
    o0 = (_Float16)v0;
    o1 = (_Float16)v1;
}

__device__ __forceinline__ void input_compute(const InputLoad& l, _Float16* out) {
    const int lane = threadIdx.x & 63;
    _Float16 o0, o1;
    input_values(l, o0, o1);
    out[lane] = o0;
    out[lane + 64] = o1;
}

__device__ __forceinline__ void input_block(const float* x, const uint16_t* suh, _Float16* out, bool live) {
    input_compute(input_load(x, suh, live), out);
}

// Output epilogue for one element after the H32 of its 128-block.
__device__ __forceinline__ float output_element(float h, uint16_t svh, const float* bias, int n,
                                                float alpha, float beta, const float* old) {
    float y = rn32(h * half_bits_to_float(svh));
    if (bias) y = rn32(y + ld_global(bias + n));
    y = rn32(y * alpha);
    if (beta != 0.0f) y = rn32(y + rn32(beta * ld_global(old)));
    return y;
}

// The same epilogue with svh bits and the bias value already loaded.
__device__ __forceinline__ float output_value(float h, uint16_t svh, bool has_bias, float bias, float alpha,
                                              float beta, const float* old) {
    float y = rn32(h * half_bits_to_float(svh));
    if (has_bias) y = rn32(y + bias);
    y = rn32(y * alpha);
    if (beta != 0.0f) y = rn32(y + rn32(beta * ld_global(old)));
    return y;
}

}  // namespace stx
