// Host side of the routed-expert block: argument checks and launches (its
// split policy and workspace sizes are in policy.cpp).
#include "moe_kernel.hpp"

namespace stx {

using MoeDispatch = hipError_t (*)(const MoeArgs&, hipStream_t);
static const MoeDispatch gate_up_table[2] = {moe_gate_up_dispatch<2>, moe_gate_up_dispatch<3>};
static const MoeDispatch down_table[2] = {moe_down_dispatch<2>, moe_down_dispatch<3>};

static bool moe_args_ok(const MoeArgs& a) {
    const uint32_t routes = a.rows * a.topk;
    // Down splits may start and end inside a 128-channel group; the groups a
    // split touches must fit the down kernel's activation buffer.
    bool down_fits = a.bps_d >= 1 && a.s_d >= 1 && a.s_d <= a.H / 16;
    for (uint32_t s = 0; down_fits && s < a.s_d; ++s) down_fits = moe_down_groups(a.bps_d, s) <= uint32_t(MOE_D_MAX_BPS) / 8;
    return a.rows >= 1 && a.rows <= 8 && a.topk >= 1 && a.topk <= MOE_MAX_TOPK && routes <= MOE_MAX_ROUTES &&
           a.bank_count >= 1 && a.bank_count <= MOE_MAX_BANK &&
           a.I % 128 == 0 && a.H % 128 == 0 && a.gate_bits >= 2 && a.gate_bits <= 3 && a.up_bits >= 2 &&
           a.up_bits <= 3 && a.down_bits >= 2 && a.down_bits <= 3 && a.bps_gu <= uint32_t(MOE_GU_MAX_BPS) &&
           a.bps_gu % 8 == 0 && down_fits && a.bps_gu * a.s_gu * 16 == a.I && a.bps_d * a.s_d * 16 == a.H;
}

// Core inputs of the gate and up projections, once per route j:
// a_gu[j][p] = RN16(H32(RN16(RN32(x[j / k] * suh_p)))) with the suh of the
// route's expert, p = gate (0) or up (1); the values and bits of the gate/up
// core's own input stage (input_values).  Wave w of workgroup (bx, j) takes
// 128-block 4 bx + w.  A route whose id is outside the bank writes nothing:
// its token is invalid, and the gate/up launch reads only valid tokens' routes.
__global__ __launch_bounds__(GEMV_THREADS) void moe_input_kernel(const float* x, const uint32_t* ids,
                                                                 const MoeExpert* bank, uint32_t topk,
                                                                 uint32_t bank_count, uint32_t x_stride, MoeArgs args) {
    // Everything its first loads need is preloaded (scalar arguments).
    MoeArgs a = args;
    a.x = x;
    a.ids = ids;
    a.bank = bank;
    a.topk = topk;
    a.bank_count = bank_count;
    a.x_stride = x_stride;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const uint32_t j = blockIdx.y, b = blockIdx.x * GEMV_WAVES + uint32_t(w);
    if (b >= a.I / 128) return;
    const float* xr = a.x + uint64_t(j / a.topk) * a.x_stride + 128 * b;
    const float x0 = ld_global(xr + lane), x1 = ld_global(xr + lane + 64);   // issued ahead of the id's round trip
    const uint32_t e = moe_first(ld_global(a.ids + j));
    if (e >= a.bank_count) return;
    const MoeExpert& ex = a.bank[e];
    const uint32_t n0 = 128 * b + lane;
    const InputLoad lg{x0, x1, ld_global(ex.gate.suh + n0), ld_global(ex.gate.suh + n0 + 64)};
    const InputLoad lu{x0, x1, ld_global(ex.up.suh + n0), ld_global(ex.up.suh + n0 + 64)};
    _Float16 g0, g1, u0, u1;
    input_values(lg, g0, g1);
    input_values(lu, u0, u1);
    uint16_t* out = a.a_gu + uint64_t(j) * 2 * a.I;
    out[n0] = __builtin_bit_cast(uint16_t, g0);
    out[n0 + 64] = __builtin_bit_cast(uint16_t, g1);
    out[a.I + n0] = __builtin_bit_cast(uint16_t, u0);
    out[a.I + n0 + 64] = __builtin_bit_cast(uint16_t, u1);
}

hipError_t launch_moe_gate_up(const MoeArgs& a, hipStream_t stream) {
    if (!moe_args_ok(a) || !a.a_gu) return hipErrorInvalidValue;
    if (a.x_stride > 0xFFFFFFFFull) return hipErrorInvalidValue;
    hipLaunchKernelGGL(moe_input_kernel, dim3((a.I / 128 + GEMV_WAVES - 1) / GEMV_WAVES, a.rows * a.topk),
                       dim3(GEMV_THREADS), 0, stream, a.x, a.ids, a.bank, a.topk, a.bank_count,
                       uint32_t(a.x_stride), a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return gate_up_table[a.gate_bits - 2](a, stream);
}

hipError_t launch_moe_down(const MoeArgs& a, hipStream_t stream) {
    if (!moe_args_ok(a)) return hipErrorInvalidValue;
    MoeArgs b = a;
    b.down_mode = kMoeDownFused;
    return down_table[a.down_bits - 2](b, stream);
}

hipError_t launch_moe_down_core(const MoeArgs& a, MoeDownMode mode, hipStream_t stream) {
    if (!moe_args_ok(a) || (mode != kMoeDownCore && mode != kMoeDownRouteCore)) return hipErrorInvalidValue;
    MoeArgs b = a;
    b.down_mode = mode;
    return down_table[a.down_bits - 2](b, stream);
}

// Staged finish: one wave per (column group, token).  Token validity comes
// from the same route resolution as the fused launch's; an invalid token gets
// its NaN row block, a valid one the fused last arrival's ordered finish over
// the planes as they are in memory.
__global__ __launch_bounds__(64) void moe_down_finish_kernel(MoeArgs a) {
    const uint32_t c = blockIdx.x, r = blockIdx.y;
    const int lane = threadIdx.x;
    __shared__ uint32_t route_words[2 * MOE_MAX_ROUTES];
    const MoeRoutes rt = moe_routes(a);
    moe_keep_routes(rt, route_words);
    __builtin_amdgcn_wave_barrier();
    if ((rt.valid >> (r * a.topk)) & 1) {
        moe_finish_token(a, r, c, lane, route_words);
    } else {
        float* yr = a.y + uint64_t(r) * a.y_stride + 128 * c;
        yr[lane] = yr[lane + 64] = __builtin_bit_cast(float, 0x7fc00000u);
    }
}

hipError_t launch_moe_down_finish(const MoeArgs& a, hipStream_t stream) {
    if (!moe_args_ok(a)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(moe_down_finish_kernel, dim3(a.I / 128, a.rows), dim3(64), 0, stream, a);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void moe_swiglu_kernel(const float* g, const float* u, float* h, uint64_t n) {
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) h[i] = moe_swiglu(g[i], u[i]);
}

hipError_t launch_moe_swiglu(const float* g, const float* u, float* h, uint64_t n, hipStream_t stream) {
    if (!n) return hipSuccess;
    const uint64_t blocks = (n + 255) / 256;
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    hipLaunchKernelGGL(moe_swiglu_kernel, dim3(uint32_t(blocks)), dim3(256), 0, stream, g, u, h, n);
    return hipGetLastError();
}

}  // namespace stx
