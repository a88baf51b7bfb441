// Decode GEMV (rows 1..8) for gfx950: input stage, trellis decode + FP16 dot
// with FP32 accumulation, split-K fold and output stage.
//
// Replaces the reference's generic GEMV family (src/gemv_lds.hip:14-168,
// src/gemv_fused.hip:17-128, src/transforms.hpp:8-52) with one wave64 design:
//
//   1-D grid of 256-thread workgroups (4 waves).  Workgroup (c, s, z) owns
//   output columns [128c, 128c+128) of group z and input blocks
//   [s*bps, (s+1)*bps) (16 channels each, bps a multiple of 8 so the split
//   holds whole H128 input blocks).  The grid runs split-major: every column
//   group's split s is dispatched before any split s + 1, so the last split,
//   which finishes a single launch, comes after all the work it waits for.
//   * prologue: the workgroup computes the FP16 core input of its channels
//     into LDS (one wave per 128-block); the weight loads of the prefetch
//     ring are issued before it so their latency overlaps it;
//   * main loop: wave w takes input blocks w, w+4, ...; per block every lane
//     loads its K-word chunk (K*256 contiguous bytes per wave), decodes 32
//     weights in VGPRs and multiplies them, as the B operand of 8 or 16
//     v_mfma_f32_4x4x4_16b_f16 (row counts up to four or eight), with the
//     block's activations read from LDS;
//   * the four waves' partial sums meet in LDS and are added in wave order;
//   * S == 1: the workgroup applies the output stage itself.  Otherwise it
//     writes its [rows][128] partial plane; the finishing step (a second
//     kernel, or in a single-launch plan the workgroup of split S-1, which
//     waits for the other splits' planes) folds the S planes in
//     ascending split order from +0 and applies the output stage.
//
// Per-output accumulation order (defines the core's bits; depends on I, N,
// K only, never on the row count):
//   lane chain  : +0, then blocks in ascending order; within a block the four
//                 K steps of four input rows (one MFMA product sum each);
//   wave fold   : chain(w0) + chain(w1) + chain(w2) + chain(w3);
//   split fold  : ((+0 + P0) + P1) + ... + P(S-1).
#pragma once
#include "backend.hpp"
#include "stages.hpp"

namespace stx {

constexpr int GEMV_WAVES = 4;
constexpr int GEMV_THREADS = 64 * GEMV_WAVES;
constexpr uint32_t kGemvCus = 256;   // compute units of an MI355X (8 XCDs x 32)

struct GemvArgs {
    GroupWeights w;               // weights of a single-group launch
    const GroupWeights* table;    // per-group weights (grouped launch) or null
    const float* x;
    float* y;
    float* partials;              // two-launch path: F32 planes [groups][S][rows][N]
    FusedState state;             // single-launch path (mode 1)
    uint64_t x_row_stride, y_row_stride;
    uint64_t x_group_stride, y_group_stride;
    uint32_t I, N, rows, splits, bps;
    uint32_t ncg, groups;         // N / 128 column groups per group; groups
    float alpha, beta;
    uint32_t mode;                // 0: partial planes only, 1: the last split finishes
    uint32_t poll_limit;          // mode 1: finisher poll rounds before giving up (0: at once)
};

__device__ __forceinline__ GroupWeights group_weights(const GemvArgs& a, int z) {
    return a.table ? a.table[z] : a.w;
}

// Workgroup L -> column group cz = L % (groups * ncg) (cz = z * ncg + c) and
// split s = L / (groups * ncg).  The grid holds exactly groups * ncg * S
// workgroups.  (A layout that also kept a column group's splits on one XCD --
// workgroup L runs on XCD L % 8 -- measured slower: the device-scope partials
// are written through to memory either way.)
struct GemvSlot {
    uint32_t c, s, z, cz;
};
__device__ __forceinline__ GemvSlot gemv_slot(const GemvArgs& a) {
    const uint32_t cgs = a.ncg * a.groups, L = blockIdx.x;
    GemvSlot r;
    r.s = L / cgs;
    r.cz = L - r.s * cgs;
    r.z = r.cz / a.ncg;
    r.c = r.cz - r.z * a.ncg;
    return r;
}

// Output-stage operands of one lane's two columns (128c + lane, +64), loaded
// ahead of the fold so their latency overlaps the completion round trip.
constexpr int kFoldBatch = 16;

struct ColumnOperands {
    uint16_t sv0, sv1;
    float b0, b1;
};

// A missing bias is read through an empty buffer range (zeros, no memory
// access) rather than behind a branch: with every load unconditional the
// compiler counts outstanding loads exactly, and the plane polls issued next
// do not wait for these operands to arrive first.
__device__ __forceinline__ ColumnOperands column_operands(const GroupWeights& gw, int c, uint32_t N) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t n0 = 128u * c + lane, n1 = n0 + 64;
    ColumnOperands o;
    o.sv0 = ld_global(gw.svh + n0);
    o.sv1 = ld_global(gw.svh + n1);
    const auto rb = make_rsrc(gw.bias, gw.bias ? N * 4u : 0u);
    o.b0 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, n0 * 4u, 0, 0));
    o.b1 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, n1 * 4u, 0, 0));
    return o;
}

// Output stage of column group c for every row: fold, H32, epilogue.  Rows
// are spread over the waves of the grid's y dimension (one row per wave and
// step; a grid with gridDim.y == 1 walks all rows in its four waves).
// `plane(s, r)` returns the pointer to the 128 values of split s, row r.
// The splits are folded in ascending order from +0; all their loads are
// issued before the first add (one memory round trip per kFoldBatch splits).
template <typename Plane>
__device__ __forceinline__ void finish_columns(const GemvArgs& a, const GroupWeights& gw, const ColumnOperands& op,
                                               float* y, int c, int splits, Plane plane) {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (uint32_t r = blockIdx.y * GEMV_WAVES + w; r < a.rows; r += gridDim.y * GEMV_WAVES) {
        float z0 = 0.0f, z1 = 0.0f;
        for (int s = 0; s < splits; s += kFoldBatch) {
            float v0[kFoldBatch], v1[kFoldBatch];
#pragma unroll
            for (int u = 0; u < kFoldBatch; ++u) {
                if (s + u < splits) {
                    const float* p = plane(s + u, r);
                    v0[u] = p[lane];
                    v1[u] = p[lane + 64];
                }
            }
#pragma unroll
            for (int u = 0; u < kFoldBatch; ++u) {
                if (s + u < splits) {
                    z0 = z0 + v0[u];
                    z1 = z1 + v1[u];
                }
            }
        }
        h32_wave(z0, z1);
        const int n0 = 128 * c + lane, n1 = n0 + 64;
        float* yr = y + r * a.y_row_stride;
        const float o0 = output_value(z0, op.sv0, gw.bias != nullptr, op.b0, a.alpha, a.beta, yr + n0);
        const float o1 = output_value(z1, op.sv1, gw.bias != nullptr, op.b1, a.alpha, a.beta, yr + n1);
        *(__attribute__((address_space(1))) float*)(yr + n0) = o0;
        *(__attribute__((address_space(1))) float*)(yr + n1) = o1;
    }
}

// ---------------------------------------------------------------------------
// Single-launch completion (state layout in backend.hpp).
//
// Every workgroup of column group cz reads epochs[cz] when it starts; the
// launch uses plane set epochs[cz] & 1.  Splits 0..S-2 publish their partial
// sums into it, re-arm their own plane of the other set (the previous
// launch's, which has ended: nothing of this launch reads it) and exit.  The
// workgroup of split S-1 (dispatched after them) loads its set's words until
// none is EMPTY, folds them in ascending split order with its own sums (in
// LDS, split S-1) last, finishes the output and advances epochs[cz].
//   * An aligned 32-bit store is seen whole or not at all.  No partial sum can
//     be the EMPTY pattern: FP16 operands make every NaN the core produces
//     carry 13 zero low bits, and EMPTY has none.
//   * Publication and polls are device-scope accesses (sc1): a store is
//     written through to memory, a poll reads past the L1.
//   * The poll is bounded.  A finisher that gives up writes NaN outputs, sets
//     GEMV_STATUS_GAVE_UP in the sticky status word and poisons epochs[cz]
//     (GEMV_EPOCH_POISON).  Workgroups are dispatched in grid order only
//     within one XCD, so a split of the same launch may still start after the
//     give-up: it reads the epoch as the next launch's splits will, and no
//     word of the state tells the two apart.  Instead a finisher that reads a
//     poisoned epoch trusts no plane: it writes NaN without polling, and the
//     column group stays poisoned until the host re-initialises the whole
//     state in stream order (after every earlier launch, late splits
//     included, has ended).
//   * Its dependencies were dispatched before it on their XCDs and at most
//     ncg * groups finishers exist, so the wait ends unless another stream's
//     work holds CUs for longer than the poll limit.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t load_epoch(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A wave-uniform value loaded earlier into a vector register, read into a
// scalar one here.  The empty asm keeps the value in its vector register up to
// this point, so the load's wait lands here instead of right after the load.
__device__ __forceinline__ uint32_t uniform_late(uint32_t v) {
    asm volatile("" : "+v"(v));
    return uint32_t(__builtin_amdgcn_readfirstlane(int(v)));
}

// Plane words of column group cz in set k: [S-1][rows][128].
__device__ __forceinline__ float* fused_planes(const GemvArgs& a, uint32_t cz, uint32_t k) {
    const uint64_t per_cg = uint64_t(a.splits - 1) * a.rows * 128u;
    return a.state.planes + (uint64_t(k) * a.ncg * a.groups + cz) * per_cg;
}

// Workgroup barrier that waits only for LDS traffic: global loads issued
// before it (the finisher's output-stage operands) stay in flight, where
// __syncthreads would wait for them too.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Plane poll: the F32 words of columns 2l and 2l + 1 at voffset + soffset of
// the planes, one 64-bit device-coherent load (sc1, the cache policy of an
// agent-scope atomic load).  Each 32-bit word is seen whole or not at all;
// the two words are checked separately.
constexpr int kCoherentAux = 16;   // sc1
typedef float gemv_f2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ gemv_f2_t poll_pair(__amdgpu_buffer_rsrc_t planes, uint32_t voffset, uint32_t soffset) {
    return __builtin_bit_cast(gemv_f2_t,
                              __builtin_amdgcn_raw_buffer_load_b64(planes, voffset, soffset, kCoherentAux));
}
__device__ __forceinline__ bool filled(gemv_f2_t v) {
    return __builtin_bit_cast(uint32_t, v.x) != GEMV_PLANE_EMPTY && __builtin_bit_cast(uint32_t, v.y) != GEMV_PLANE_EMPTY;
}

// The plane stride, opaque to the compiler: the poll offsets derived from it
// are recomputed (one scalar add each) in every poll round instead of being
// hoisted out of the loop, where every live offset would hold a scalar
// register.
__device__ __forceinline__ uint32_t step_offset(uint32_t bytes) {
    asm volatile("" : "+s"(bytes));
    return bytes;
}

// 64-bit plane loads one lane holds in flight in one poll round (a wave's
// vector-load counter tracks at most 63).
constexpr int kPollLoads = 32;
constexpr uint32_t kPollOutOfRange = 0x80000000u;   // answered with zeros (filled), never folded

// One poll round of P x NB pair loads per lane: load (p, u) at soffset
// (first + u) * stride + p * row_step, for p < rows_live and u < count (both
// wave-uniform; the rest out of range, so every load is issued before the
// first wait and none sits behind a branch).  Polls until every word has
// arrived or the limit runs out (false); then adds load u to z[p] for
// u < count in ascending u.
template <int P, int NB>
__device__ __forceinline__ bool poll_fold_round(gemv_f2_t (&z)[P], __amdgpu_buffer_rsrc_t planes, uint32_t voff,
                                                uint32_t first, uint32_t stride, uint32_t row_step, int rows_live,
                                                int count, uint32_t limit) {
    gemv_f2_t v[P][NB];
    for (uint32_t spin = 0;; ++spin) {
        asm volatile("" ::: "memory");
        const int cnt = int(step_offset(uint32_t(count)));
#pragma unroll
        for (int p = 0; p < P; ++p) {
            uint32_t so = step_offset(stride) * first + uint32_t(p) * row_step;
            const int c = p < rows_live ? cnt : 0;
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                v[p][u] = poll_pair(planes, u < c ? voff : kPollOutOfRange, so);
                so += stride;
            }
        }
        bool ready = true;
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
            for (int u = 0; u < NB; ++u) ready &= filled(v[p][u]);
        if (__all(ready)) break;
        if (spin + 1 >= limit) return false;
        __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const float t0 = z[p].x + v[p][u].x, t1 = z[p].y + v[p][u].y;
            z[p].x = u < count ? t0 : z[p].x;
            z[p].y = u < count ? t1 : z[p].y;
        }
    return true;
}

// H32 of P rows held as element pairs (2l, 2l + 1) per lane: the stride-1
// level inside the lane, strides 2..64 across lanes 1..32 apart.  Each level
// combines the same element pairs with the same operations (lower + upper,
// lower - upper, one FP32 rounding each) as h32_wave, so the bits are those
// of h32_wave on the (l, l + 64) layout.
template <int P>
__device__ __forceinline__ void h32_pairs(gemv_f2_t (&v)[P]) {
    float v0[P], v1[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const float a = v[i].x, b = v[i].y;
        v0[i] = a + b;
        v1[i] = a - b;
    }
    auto stage = [&](auto st) {
        constexpr int S = decltype(st)::value;
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
        v[i].x = rn32(v0[i] * INV_SQRT128);
        v[i].y = rn32(v1[i] * INV_SQRT128);
    }
}

// Finisher of a single launch.  `red` holds this workgroup's [rows][128] sums
// (split S-1); `flag` is an LDS word cleared before the barrier that precedes
// this call; `cur` the column group's planes of this launch's set.  Wave w
// finishes rows w and w + 4, lane l columns 2l and 2l + 1 of them: it loads
// each other split's word pair with one 64-bit load, kPollLoads per round
// over its rows (one round for up to 32 other splits at rows <= 4, 16 at
// five to eight), folds ((+0 + P0) + P1) + ... + P(S-2) + own -- the split
// fold of the two-launch path, bit for bit -- and applies H32 and the output
// stage.  Each wave polls with its own bound; a wave that gives up writes
// NaN rows, and after a barrier the workgroup poisons the epoch if any did.
template <int RT>
__device__ __forceinline__ void finish_polled(const GemvArgs& a, const GroupWeights& gw, float* y, int c,
                                              const float* red, uint32_t* flag, const float* cur, uint32_t epoch,
                                              uint32_t cz) {
    const int w = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6)), lane = threadIdx.x & 63;
    constexpr int RPW = (RT + GEMV_WAVES - 1) / GEMV_WAVES, B = kPollLoads / RPW;
    if (uint32_t(w) < a.rows) {
        const int others = int(a.splits) - 1;
        const uint32_t stride = a.rows * 512u;   // one split's [rows][128] F32
        const auto planes = make_rsrc(cur, uint32_t(others) * stride);
        const uint32_t limit = a.poll_limit, voff = uint32_t(w) * 512u + uint32_t(lane) * 8u;
        const int rows_live = uint32_t(w + GEMV_WAVES) < a.rows && RPW > 1 ? 2 : 1;
        // Output-stage operands of columns 128c + 2l, +1 (in flight during the polls).
        const uint32_t n0 = 128u * uint32_t(c) + 2u * uint32_t(lane);
        const uint32_t svp = ld_global(reinterpret_cast<const uint32_t*>(gw.svh + n0));
        const auto rb = make_rsrc(gw.bias, gw.bias ? a.N * 4u : 0u);
        const gemv_f2_t bias = __builtin_bit_cast(gemv_f2_t, __builtin_amdgcn_raw_buffer_load_b64(rb, n0 * 4u, 0, 0));
        gemv_f2_t z[RPW];
#pragma unroll
        for (int i = 0; i < RPW; ++i) z[i] = gemv_f2_t{0.0f, 0.0f};
        bool complete = limit != 0 && !(epoch & GEMV_EPOCH_POISON);
        for (int s0 = 0; s0 < others && complete;) {
            const int count = others - s0 < B ? others - s0 : B;
            constexpr uint32_t step = GEMV_WAVES * 512u;
            if (count <= 8)
                complete = poll_fold_round<RPW, 8>(z, planes, voff, uint32_t(s0), stride, step, rows_live, count, limit);
            else if (count <= 16 || B <= 16)
                complete = poll_fold_round<RPW, (B < 16 ? B : 16)>(z, planes, voff, uint32_t(s0), stride, step,
                                                                   rows_live, count, limit);
            else if (count <= 24)
                complete = poll_fold_round<RPW, 24>(z, planes, voff, uint32_t(s0), stride, step, rows_live, count,
                                                    limit);
            else
                complete = poll_fold_round<RPW, B>(z, planes, voff, uint32_t(s0), stride, step, rows_live, count, limit);
            s0 += count;
        }
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const uint32_t r = uint32_t(w + GEMV_WAVES * i) < a.rows ? uint32_t(w + GEMV_WAVES * i) : uint32_t(w);
            const gemv_f2_t own = *reinterpret_cast<const gemv_f2_t*>(red + r * 128 + 2 * lane);
            z[i].x = complete ? z[i].x + own.x : __builtin_nanf("");
            z[i].y = complete ? z[i].y + own.y : __builtin_nanf("");
        }
        if (!complete) *flag = 1u;
        h32_pairs<RPW>(z);
        const uint16_t sv0 = uint16_t(svp), sv1 = uint16_t(svp >> 16);
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            if (i >= rows_live) continue;
            float* yr = y + uint32_t(w + GEMV_WAVES * i) * a.y_row_stride + n0;
            gemv_f2_t o;
            o.x = output_value(z[i].x, sv0, gw.bias != nullptr, bias.x, a.alpha, a.beta, yr);
            o.y = output_value(z[i].y, sv1, gw.bias != nullptr, bias.y, a.alpha, a.beta, yr + 1);
            *(__attribute__((address_space(1))) gemv_f2_t*)(yr) = o;
        }
    }
    // Every wave's verdict is in `flag`: advance the epoch (the splits have
    // re-armed the other set), or poison it.  Off the outputs' critical path.
    lds_barrier();
    if (threadIdx.x == 0) {
        const bool gave_up = *flag != 0u;
        if (gave_up)
            __hip_atomic_fetch_or(a.state.status, GEMV_STATUS_GAVE_UP, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t next = gave_up ? (epoch | GEMV_EPOCH_POISON) : ((epoch + 1u) & ~GEMV_EPOCH_POISON);
        __hip_atomic_store(a.state.epochs + cz, next, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Five to eight rows: plane words in quads.  Each 32-lane half of a wave
// holds one row, lane l = lane & 31 its columns 4l .. 4l + 3, so one 16-byte
// access carries what two 8-byte ones do in the pair layout: a finisher wave
// then polls each other split's words of its two rows with one load per lane,
// where the pair layout takes two (at two rows per wave the poll round is
// bound by the loads in flight, not by their bytes).
typedef float gemv_q_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ gemv_q_t poll_quad(__amdgpu_buffer_rsrc_t planes, uint32_t voffset, uint32_t soffset) {
    return __builtin_bit_cast(gemv_q_t, __builtin_amdgcn_raw_buffer_load_b128(planes, voffset, soffset, kCoherentAux));
}
__device__ __forceinline__ bool filled(gemv_q_t v) {
    return __builtin_bit_cast(uint32_t, v.x) != GEMV_PLANE_EMPTY && __builtin_bit_cast(uint32_t, v.y) != GEMV_PLANE_EMPTY &&
           __builtin_bit_cast(uint32_t, v.z) != GEMV_PLANE_EMPTY && __builtin_bit_cast(uint32_t, v.w) != GEMV_PLANE_EMPTY;
}

// One poll round of NB quad loads per lane at soffset (first + u) * stride
// (u < count, the rest out of range): polls until every word has arrived or
// the limit runs out (false); then adds load u to z for u < count in
// ascending u.
template <int NB>
__device__ __forceinline__ bool poll_fold_quads(gemv_q_t& z, __amdgpu_buffer_rsrc_t planes, uint32_t voff,
                                                uint32_t first, uint32_t stride, int count, uint32_t limit) {
    gemv_q_t v[NB];
    for (uint32_t spin = 0;; ++spin) {
        asm volatile("" ::: "memory");
        const int cnt = int(step_offset(uint32_t(count)));
        uint32_t so = step_offset(stride) * first;
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            v[u] = poll_quad(planes, u < cnt ? voff : kPollOutOfRange, so);
            so += stride;
        }
        bool ready = true;
#pragma unroll
        for (int u = 0; u < NB; ++u) ready &= filled(v[u]);
        if (__all(ready)) break;
        if (spin + 1 >= limit) return false;
        __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
        const gemv_q_t t = z + v[u];
        z = u < count ? t : z;
    }
    return true;
}

// H32 of one row held as quads over a 32-lane half: element strides 1 and 2
// inside the lane, 4 .. 64 across lanes 1 .. 16 apart.  Each level combines
// the same element pairs with the same operations (lower + upper,
// lower - upper, one FP32 rounding each) as h32_wave, so the same bits.
__device__ __forceinline__ void h32_quads(gemv_q_t& z) {
    const float a0 = z.x + z.y, a1 = z.x - z.y, a2 = z.z + z.w, a3 = z.z - z.w;
    float v0 = a0 + a2, v2 = a0 - a2, v1 = a1 + a3, v3 = a1 - a3;
    auto stage = [&](auto st) {
        constexpr int S = decltype(st)::value;
        butterfly<S>(v0, v1);
        butterfly<S>(v2, v3);
    };
    stage(std::integral_constant<int, 1>{});
    stage(std::integral_constant<int, 2>{});
    stage(std::integral_constant<int, 4>{});
    stage(std::integral_constant<int, 8>{});
    stage(std::integral_constant<int, 16>{});
    z.x = rn32(v0 * INV_SQRT128);
    z.y = rn32(v1 * INV_SQRT128);
    z.z = rn32(v2 * INV_SQRT128);
    z.w = rn32(v3 * INV_SQRT128);
}

// Input stage of one 128-channel unit per 32-lane half: lane l = lane & 31
// loads x and suh of channels 4l .. 4l + 3 with one 16-byte and one 8-byte
// load (a quarter of the load instructions of the (l, l + 64) layout), then
// the same per-element arithmetic, H32 pairs and FP16 rounding.  x need only
// be 4-byte aligned: ROCm runs compute queues in the unaligned memory-access
// mode, where a multi-dword global load takes any dword-aligned address.
struct InputQuad {
    gemv_q_t x;
    u32x2 u;
};
__device__ __forceinline__ InputQuad input_load_quad(const float* x, const uint16_t* suh, bool live) {
    const int l = threadIdx.x & 31;
    InputQuad q;
    const gemv_q_t v = ld_global(reinterpret_cast<const gemv_q_t*>(x + 4 * l));
    q.x = live ? v : gemv_q_t{0.0f, 0.0f, 0.0f, 0.0f};
    q.u = ld_global(reinterpret_cast<const u32x2*>(suh + 4 * l));
    return q;
}
__device__ __forceinline__ void input_compute_quad(const InputQuad& q, _Float16* out) {
    const int l = threadIdx.x & 31;
    gemv_q_t v;
    v.x = (float)(_Float16)rn32(q.x.x * half_bits_to_float(uint16_t(q.u.x)));
    v.y = (float)(_Float16)rn32(q.x.y * half_bits_to_float(uint16_t(q.u.x >> 16)));
    v.z = (float)(_Float16)rn32(q.x.z * half_bits_to_float(uint16_t(q.u.y)));
    v.w = (float)(_Float16)rn32(q.x.w * half_bits_to_float(uint16_t(q.u.y >> 16)));
    h32_quads(v);
    typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
    *reinterpret_cast<h4_t*>(out + 4 * l) = h4_t{(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
}

// Finisher of a single launch at five to eight rows (finish_polled's
// protocol and fold order, quads instead of pairs): wave w finishes rows w
// and w + 4 (lanes 0-31 and 32-63), up to kQuadPolls other splits per round
// (16-byte loads: the registers of a pair round's 8-byte ones).
constexpr int kQuadPolls = kPollLoads / 2;
template <int RT>
__device__ __forceinline__ void finish_polled_wide(const GemvArgs& a, const GroupWeights& gw, float* y, int c,
                                                   const float* red, uint32_t* flag, const float* cur, uint32_t epoch,
                                                   uint32_t cz) {
    static_assert(RT > GEMV_WAVES && RT <= 2 * GEMV_WAVES, "two rows per wave");
    const int w = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6)), lane = threadIdx.x & 63, l = lane & 31;
    const uint32_t r = uint32_t(w + GEMV_WAVES * (lane >> 5));   // rows >= 5: every wave has row w
    const bool live = r < a.rows;
    const int others = int(a.splits) - 1;
    const uint32_t stride = a.rows * 512u;   // one split's [rows][128] F32
    const auto planes = make_rsrc(cur, uint32_t(others) * stride);
    const uint32_t limit = a.poll_limit, voff = live ? r * 512u + uint32_t(l) * 16u : kPollOutOfRange;
    // Output-stage operands of columns 128c + 4l .. +3 (in flight during the polls).
    const uint32_t n0 = 128u * uint32_t(c) + 4u * uint32_t(l);
    const u32x2 svq = ld_global(reinterpret_cast<const u32x2*>(gw.svh + n0));
    const auto rb = make_rsrc(gw.bias, gw.bias ? a.N * 4u : 0u);
    const gemv_q_t bias = __builtin_bit_cast(gemv_q_t, __builtin_amdgcn_raw_buffer_load_b128(rb, n0 * 4u, 0, 0));
    gemv_q_t z = {0.0f, 0.0f, 0.0f, 0.0f};
    bool complete = limit != 0 && !(epoch & GEMV_EPOCH_POISON);
    for (int s0 = 0; s0 < others && complete;) {
        const int count = others - s0 < kQuadPolls ? others - s0 : kQuadPolls;
        if (count <= 8)
            complete = poll_fold_quads<8>(z, planes, voff, uint32_t(s0), stride, count, limit);
        else
            complete = poll_fold_quads<kQuadPolls>(z, planes, voff, uint32_t(s0), stride, count, limit);
        s0 += count;
    }
    const uint32_t rr = live ? r : uint32_t(w);
    const gemv_q_t own = *reinterpret_cast<const gemv_q_t*>(red + rr * 128 + 4 * l);
    const float nan = __builtin_nanf("");
    z = complete ? z + own : gemv_q_t{nan, nan, nan, nan};
    if (!complete) *flag = 1u;
    h32_quads(z);
    if (live) {
        const uint16_t sv[4] = {uint16_t(svq.x), uint16_t(svq.x >> 16), uint16_t(svq.y), uint16_t(svq.y >> 16)};
        float* yr = y + r * a.y_row_stride + n0;
        const bool hb = gw.bias != nullptr;
        gemv_f2_t o0, o1;
        o0.x = output_value(z.x, sv[0], hb, bias.x, a.alpha, a.beta, yr);
        o0.y = output_value(z.y, sv[1], hb, bias.y, a.alpha, a.beta, yr + 1);
        o1.x = output_value(z.z, sv[2], hb, bias.z, a.alpha, a.beta, yr + 2);
        o1.y = output_value(z.w, sv[3], hb, bias.w, a.alpha, a.beta, yr + 3);
        *(__attribute__((address_space(1))) gemv_f2_t*)(yr) = o0;
        *(__attribute__((address_space(1))) gemv_f2_t*)(yr + 2) = o1;
    }
    // Every wave's verdict is in `flag`: advance the epoch, or poison it.
    lds_barrier();
    if (threadIdx.x == 0) {
        const bool gave_up = *flag != 0u;
        if (gave_up)
            __hip_atomic_fetch_or(a.state.status, GEMV_STATUS_GAVE_UP, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t next = gave_up ? (epoch | GEMV_EPOCH_POISON) : ((epoch + 1u) & ~GEMV_EPOCH_POISON);
        __hip_atomic_store(a.state.epochs + cz, next, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ---------------------------------------------------------------------------
// Matrix-core dot: v_mfma_f32_4x4x4_16b_f16, sixteen 4x4x4 products per
// instruction.  Operand layout, checked on the device: block b uses lanes
// 4b..4b+3; A[b][i][k] sits in lane 4b+i, B[b][k][j] in lane 4b+j (halves
// k = 0..3), D[b][i][j] in lane 4b+j, element i.  Here A holds the
// activations of four rows and B the decoded weights, so every lane feeds
// its own decoded columns as B with no data movement across lanes:
//   * lane 8t+g holds columns g and g+8 (half h = 0, 1) of tile t, input
//     rows 0..15 of the block (wq[V][khalf + 2h]); K step q (block rows
//     4q..4q+3) of half h is wq[2 (q & 1)][q / 2 + 2 h] followed by
//     wq[2 (q & 1) + 1][q / 2 + 2 h];
//   * A (step q, row quad rh): lane l reads activation row 4 rh + l % 4,
//     clamped to RT - 1 (rows past RT are never read back), block rows
//     4q..4q+3, the same for every block b;
//   * D[h][rh] of lane l, element i, is row 4 rh + i of output column
//     16 (l >> 3) + (l & 7) + 8 h of the 128-column group.
// Per output: +0, then blocks in ascending order, within a block K steps
// q = 0..3 (four products each, in the hardware's order).  A row's products
// are the D elements of its own A row, so its bits do not depend on the
// other rows.
// ---------------------------------------------------------------------------
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float gemv_f4_t __attribute__((ext_vector_type(4)));

template <int RT>
struct MfmaAcc {
    static constexpr int RH = (RT + 3) / 4;   // row quads
    gemv_f4_t d[2][RH];                        // [half h][row quad]
};

template <int RT>
__device__ __forceinline__ void mfma_acc_zero(MfmaAcc<RT>& acc) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int rh = 0; rh < MfmaAcc<RT>::RH; ++rh) acc.d[h][rh] = gemv_f4_t{0.0f, 0.0f, 0.0f, 0.0f};
}

__device__ __forceinline__ half4_t join_h4(half2_t lo, half2_t hi) { return half4_t{lo.x, lo.y, hi.x, hi.y}; }

// One decoded block (wq) against the activations `act` of its 16 input rows
// (act + r * act_row: activation row r).
template <int RT>
__device__ __forceinline__ void mfma_dot_block(const half2_t (&wq)[4][4], const _Float16* act, uint32_t act_row,
                                               MfmaAcc<RT>& acc) {
    constexpr int RH = MfmaAcc<RT>::RH;
    const int lane = threadIdx.x & 63;
    half4_t xa[4][RH];
#pragma unroll
    for (int rh = 0; rh < RH; ++rh) {
        const int row = 4 * rh + (lane & 3) < RT ? 4 * rh + (lane & 3) : RT - 1;
#pragma unroll
        for (int q = 0; q < 4; ++q) xa[q][rh] = *reinterpret_cast<const half4_t*>(act + row * act_row + 4 * q);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const half4_t wb = join_h4(wq[2 * (q & 1)][q / 2 + 2 * h], wq[2 * (q & 1) + 1][q / 2 + 2 * h]);
#pragma unroll
            for (int rh = 0; rh < RH; ++rh)
                acc.d[h][rh] = __builtin_amdgcn_mfma_f32_4x4x4f16(xa[q][rh], wb, acc.d[h][rh], 0, 0, 0);
        }
}

// The wave's sums to `red` ([RT][128] F32, row-major): lane l holds rows
// 4 rh + i (element i) of columns 16 (l >> 3) + (l & 7) + 8 h.
template <int RT>
__device__ __forceinline__ void mfma_partials(const MfmaAcc<RT>& acc, float* red) {
    const int lane = threadIdx.x & 63;
    const int col = 16 * (lane >> 3) + (lane & 7);
#pragma unroll
    for (int rh = 0; rh < MfmaAcc<RT>::RH; ++rh)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (4 * rh + i < RT) {
#pragma unroll
                for (int h = 0; h < 2; ++h) red[(4 * rh + i) * 128 + col + 8 * h] = acc.d[h][rh][i];
            }
}

// Register budget: five waves per SIMD (<= 96 VGPRs), measured faster than
// four (C1 8.9 -> 8.3 us; 16 x 4096 -> 1024 R4 32.5 -> 30.4 us) even where the
// grid is smaller than one resident round.  The 8-row K >= 6 instances would
// spill at that budget and keep four.
template <int K, int RT>
constexpr int gemv_waves_per_eu() { return RT == 8 && K >= 6 ? 4 : 5; }

// The fields every workgroup needs before its first memory access come as
// scalar arguments ahead of GemvArgs (16-bit pairs where the values fit), so
// that the dispatcher preloads them into SGPRs (kernel-argument preloading,
// built with -amdgpu-kernarg-preload-count); a by-value struct is never
// preloaded, and each workgroup would otherwise wait for a scalar load of its
// arguments before issuing any load of its own.  The rest of GemvArgs is
// needed later.  Same bits; with nothing else read from memory ahead of the
// first loads (below) measured 3.8 % faster on C1 (7.20 -> 6.93 us) and 1-4 %
// on 4096 -> 12288 and 5120^2 at R1-R8.
// Weight blocks in flight per wave.  Fewer than four left the later
// workgroups of a CU less to wait behind (their input loads queue after the
// earlier workgroups' rings): interleaved A/B, same bits, 4 -> 3 measured
// 2-5 % faster on 4096 -> 12288 at K4-K6 R1-R8, up to 4 % on 5120^2, C1 and
// grouped o_a unchanged; 6 and 8 were slower everywhere, 2 mixed.
constexpr int kGemvRing = 3;

template <int K, int CB, int RT>
__global__ __launch_bounds__(GEMV_THREADS) __attribute__((amdgpu_waves_per_eu(gemv_waves_per_eu<K, RT>())))
void gemv_kernel(const uint32_t* trellis, const uint16_t* suh, const float* x0, uint32_t* epochs,
                 const GroupWeights* table, uint32_t ncg_groups, uint32_t bps_splits, uint32_t rows_mode, uint32_t n,
                 uint32_t x_row_stride, GemvArgs args) {
    GemvArgs a = args;
    a.w.trellis = trellis;
    a.w.suh = suh;
    a.x = x0;
    a.state.epochs = epochs;
    a.table = table;
    a.ncg = ncg_groups & 0xFFFFu;
    a.groups = ncg_groups >> 16;
    a.bps = bps_splits & 0xFFFFu;
    a.splits = bps_splits >> 16;
    a.rows = rows_mode & 0xFFu;
    a.mode = (rows_mode >> 8) & 0xFFu;
    // Workgroups below this index wait for their input before most of their
    // weight ring (the two-round ordering below); computed on the host, so
    // no workgroup reads the grid size from memory first.
    const uint32_t first_round_end = rows_mode >> 16;
    a.N = n;
    a.x_row_stride = x_row_stride;
    extern __shared__ __align__(16) unsigned char smem[];
    const GemvSlot place = gemv_slot(a);
    const int c = int(place.c), s = int(place.s), z = int(place.z);
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int jt = lane >> 3, g = lane & 7;
    // Up to its first loads a single-group launch uses preloaded arguments
    // only (trellis, suh, x); a grouped launch reads its group's weights from
    // the table.  svh, bias and y, needed at the finish only, are taken there
    // (gw_finish, y_of), so that no wait for the rest of GemvArgs sits ahead
    // of the first loads.
    GroupWeights gw{trellis, suh, nullptr, nullptr};
    const float* x = x0;
    if (table) {
        gw.trellis = table[z].trellis;
        gw.suh = table[z].suh;
        x = x0 + uint64_t(z) * a.x_group_stride;
    }
    auto gw_finish = [&]() {
        GroupWeights f = gw;
        f.svh = table ? table[z].svh : args.w.svh;
        f.bias = table ? table[z].bias : args.w.bias;
        return f;
    };
    auto y_of = [&]() { return a.y + uint64_t(z) * a.y_group_stride; };

    constexpr uint32_t tile_bytes = 32u * K;
    const uint32_t row_bytes = (a.N >> 4) * tile_bytes;
    const uint32_t a0 = s * a.bps;
    const auto rsrc = make_rsrc(reinterpret_cast<const char*>(gw.trellis) + uint64_t(a0) * row_bytes,
                                a.bps * row_bytes);
    const uint32_t lane_off = (8u * c + jt) * tile_bytes + g * 4u * K;
    const int nb = a.bps / GEMV_WAVES;   // even: bps is a multiple of 8
    const uint32_t act_row = a.bps * 16;

    _Float16* act = reinterpret_cast<_Float16*>(smem);                  // [RT][bps*16]
    float* red = reinterpret_cast<float*>(smem + RT * act_row * 2);       // [4][RT][128]

    // Prefetch ring of kGemvRing blocks per wave.  Loads are issued
    // unconditionally so the compiler can count them exactly; past the last
    // block the offset is out of the buffer's range, which the hardware
    // answers with zeros and no memory access.
    constexpr uint32_t kOutOfRange = 0x80000000u;
    auto block_off = [&](int t) -> uint32_t {
        return t < nb ? (w + GEMV_WAVES * t) * row_bytes + lane_off : kOutOfRange;
    };
    // The launch's epoch (single launch with splits): issued first, so its
    // round trip overlaps the prologue.  The finisher (S == 1, or in a single
    // launch the workgroup of the last split) keeps its own sums in LDS;
    // every other split publishes a plane.
    const bool fused = a.mode == 1 && a.splits > 1;
    const bool finisher = a.splits == 1 || (fused && uint32_t(s) == a.splits - 1);
    // The loaded word stays in a vector register until the planes are chosen
    // (uniform_late below): read into a scalar register at once, the load's
    // wait would sit here, ahead of every input and weight load.
    const uint32_t epoch_v = fused ? load_epoch(a.state.epochs + place.cz) : 0u;

    // Prologue: FP16 core input of this split's channels, one 128-block unit
    // per wave at a time, the loads of kUnits units per wave in flight
    // together (each batch is one memory round trip; one unit at a time made
    // the 8-row input stage six round trips long).  The first batch is issued
    // before the weight prefetch, so waiting for it does not wait for the
    // weights.  (Four units in flight make the 4-row mcg / 3inst kernels
    // spill, so those keep two.)
    // The 2- and 8-row templates' work item is a pair of units, one per
    // 32-lane half (input_load_quad): the same units per wave and batch from a
    // quarter of the load instructions.  (Measured: 3-5 % faster at 7-8 rows
    // and up to 5.6 % at 2 rows; mixed at 4 rows, where single units stay.)
    constexpr bool kQuadIn = RT == 2 * GEMV_WAVES || RT == 2;
    using Unit = std::conditional_t<kQuadIn, InputQuad, InputLoad>;
    constexpr int kUnits = (RT <= 2 ? 2 : RT <= 4 ? (CB == CB_MUL1 ? 4 : 2) : 8) / (kQuadIn ? 2 : 1);
    const int hblocks = a.bps / 8, units = kQuadIn ? RT * hblocks / 2 : RT * hblocks;
    // Unit u is row u % RT of 128-block u / RT (constant divisors); a quad
    // item v holds units 2v (lanes 0-31) and 2v + 1 (lanes 32-63).
    auto unit_load = [&](int u) {
        if constexpr (kQuadIn) {
            const int uu = 2 * u + int(threadIdx.x >> 5 & 1), r = uu % RT, hb = uu / RT;
            const uint32_t ch = a0 * 16 + hb * 128;
            const bool live = uint32_t(r) < a.rows;
            return input_load_quad(x + (live ? r * a.x_row_stride : 0) + ch, gw.suh + ch, live);
        } else {
            const int r = u % RT, hb = u / RT;
            const uint32_t ch = a0 * 16 + hb * 128;
            const bool live = uint32_t(r) < a.rows;
            return input_load(x + (live ? r * a.x_row_stride : 0) + ch, gw.suh + ch, live);
        }
    };
    auto unit_out = [&](int u) -> _Float16* {
        const int uu = kQuadIn ? 2 * u + int(threadIdx.x >> 5 & 1) : u;
        return act + (uu % RT) * act_row + (uu / RT) * 128;
    };
    // Units past the end load unit 0 again (valid addresses, result unused).
    auto batch_load = [&](int u0, Unit (&l)[kUnits]) {
#pragma unroll
        for (int i = 0; i < kUnits; ++i) {
            const int u = u0 + GEMV_WAVES * i;
            l[i] = unit_load(u < units ? u : 0);
        }
    };
    auto batch_compute = [&](int u0, const Unit (&l)[kUnits]) {
#pragma unroll
        for (int i = 0; i < kUnits; ++i) {
            const int u = u0 + GEMV_WAVES * i;
            if (u < units) {
                if constexpr (kQuadIn) input_compute_quad(l[i], unit_out(u));
                else input_compute(l[i], unit_out(u));
            }
        }
    };
    Unit pre[kUnits];
    batch_load(w, pre);
    __builtin_amdgcn_sched_barrier(0);   // keep these loads ahead of the weight prefetch
    // A grid of two dispatch rounds (257..512 workgroups on 256 CUs, the
    // 4096^2 decode shape): each CU's vector loads return in issue order, so
    // the second workgroup's input would wait behind the first one's weight
    // ring.  The first round's workgroups therefore issue one block of the
    // ring, then the rest only once their own input has arrived (4096^2 K4 R1:
    // 7.53 -> 7.32 us; the whole ring after the input: 7.46 us).  With three or
    // more rounds the wait measured 1-3 % slower, so it is not taken.
    Chunk<K> ring[kGemvRing];
    load_chunk(ring[0], rsrc, block_off(0));
    __builtin_amdgcn_sched_barrier(0);
    if (blockIdx.x < first_round_end) {
        // every load but block 0's (one instruction for K <= 4, two above)
        if constexpr (K <= 4) asm volatile("s_waitcnt vmcnt(1)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 1; u < kGemvRing; ++u) load_chunk(ring[u], rsrc, block_off(u));

    // The chunks stay in their registers across the input stage: decoding
    // blocks ahead of the barrier (to overlap the input loads) was measured
    // slower, the decoded weights holding 32 more VGPRs per lane.
    batch_compute(w, pre);
    for (int u0 = w + kUnits * GEMV_WAVES; u0 < units; u0 += kUnits * GEMV_WAVES) {
        Unit l[kUnits];
        batch_load(u0, l);
        batch_compute(u0, l);
    }
    __syncthreads();

    const bool first = g == 0;
    MfmaAcc<RT> acc;
    mfma_acc_zero(acc);
    // Slot t % kGemvRing holds block t; it is refilled with block t + kGemvRing.
    for (int t = 0; t < nb; t += kGemvRing) {
#pragma unroll
        for (int u = 0; u < kGemvRing; ++u) {
            Chunk<K>& slot = ring[u];
            if (t + u < nb) {
                half2_t wq[4][4];
                link_chunk(slot, first);
                decode_chunk<K, CB>(slot, wq);
                mfma_dot_block<RT>(wq, act + (w + GEMV_WAVES * (t + u)) * 16, act_row, acc);
            }
            load_chunk(slot, rsrc, block_off(t + u + kGemvRing));
        }
    }

    // Wave partials -> LDS, added in wave order.
    mfma_partials<RT>(acc, red + w * RT * 128);
    lds_barrier();
    const uint32_t epoch = uniform_late(epoch_v);
    float* cur = fused ? fused_planes(a, place.cz, epoch & 1u) : nullptr;
    float* prev = fused ? fused_planes(a, place.cz, (epoch & 1u) ^ 1u) : nullptr;
    float* plane_base = a.partials + (uint64_t(z) * a.splits) * a.rows * a.N;
    if constexpr (RT > GEMV_WAVES) {
        // Five to eight rows: a quad of columns per thread, 16-byte LDS reads
        // and plane stores (the same element-wise adds in wave order); the
        // single-launch words go out with the sc1 policy, as store_coherent's.
        const uint32_t set_bytes = (a.splits - 1) * a.rows * 512u;
        const auto cur_rs = make_rsrc(cur, fused ? set_bytes : 0u);
        const auto prev_rs = make_rsrc(prev, fused ? set_bytes : 0u);
        for (int q = tid; q < RT * 32; q += GEMV_THREADS) {
            const int r = q >> 5, n = (q & 31) * 4;
            gemv_q_t v = *reinterpret_cast<const gemv_q_t*>(red + (0 * RT + r) * 128 + n);
#pragma unroll
            for (int ww = 1; ww < GEMV_WAVES; ++ww) v = v + *reinterpret_cast<const gemv_q_t*>(red + (ww * RT + r) * 128 + n);
            if (finisher) {
                *reinterpret_cast<gemv_q_t*>(red + r * 128 + n) = v;
            } else if (uint32_t(r) < a.rows) {
                if (fused) {
                    const uint32_t off = ((uint32_t(s) * a.rows + uint32_t(r)) * 128u + uint32_t(n)) * 4u;
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), cur_rs, off, 0, kCoherentAux);
                    __builtin_amdgcn_raw_buffer_store_b128(u32x4{GEMV_PLANE_EMPTY, GEMV_PLANE_EMPTY, GEMV_PLANE_EMPTY,
                                                                 GEMV_PLANE_EMPTY},
                                                           prev_rs, off, 0, kCoherentAux);
                } else {
                    *(__attribute__((address_space(1))) gemv_q_t*)(plane_base + (uint64_t(s) * a.rows + r) * a.N +
                                                                  128 * c + n) = v;
                }
            }
        }
    } else {
        for (int idx = tid; idx < RT * 128; idx += GEMV_THREADS) {
            const int r = idx >> 7, n = idx & 127;
            float v = red[(0 * RT + r) * 128 + n];
#pragma unroll
            for (int ww = 1; ww < GEMV_WAVES; ++ww) v = v + red[(ww * RT + r) * 128 + n];
            if (finisher) {
                red[r * 128 + n] = v;
            } else if (uint32_t(r) < a.rows) {
                if (fused) {
                    const uint64_t word = (uint64_t(s) * a.rows + r) * 128u + n;
                    store_coherent(cur + word, v);
                    store_coherent(prev + word, __builtin_bit_cast(float, GEMV_PLANE_EMPTY));
                }
                else
                    *(__attribute__((address_space(1))) float*)(plane_base + (uint64_t(s) * a.rows + r) * a.N + 128 * c + n) = v;
            }
        }
    }
    if (!finisher) return;
    // The core inputs are dead (every wave has passed the barrier after its
    // loop): their first word is the finisher's give-up flag.
    uint32_t* flag = reinterpret_cast<uint32_t*>(smem);
    if (tid == 0) *flag = 0u;
    if (a.splits == 1) {
        // Loading the output-stage operands in the prologue instead keeps them
        // live across the main loop and made the 1-row kernel spill (slower).
        const GroupWeights gf = gw_finish();
        const ColumnOperands op = column_operands(gf, c, a.N);
        lds_barrier();
        finish_columns(a, gf, op, y_of(), c, 1, [&](int, int r) -> const float* { return red + r * 128; });
        return;
    }
    lds_barrier();
    if constexpr (RT > GEMV_WAVES)
        finish_polled_wide<RT>(a, gw_finish(), y_of(), c, red, flag, cur, epoch, place.cz);
    else
        finish_polled<RT>(a, gw_finish(), y_of(), c, red, flag, cur, epoch, place.cz);
}

// ---------------------------------------------------------------------------
// Owner-fold GEMV: one 16-wave workgroup per 128-column group folds every
// split itself, so nothing crosses workgroups (reference
// src/dense_r1_group_owner.hip:1-10 describes the same plan for wave32).
//
// The workgroup is four groups of the split kernel's four waves.  Pass p runs
// splits 4p .. 4p+3 side by side, group j taking split 4p + j exactly as a
// split workgroup would: its input stage, its blocks (wave w of the group
// takes blocks w, w+4, ...), its lane chains and its wave-order fold.  Thread
// t < RT*128 owns output (row t/128, column t%128) and adds each split's
// partial to its running sum in ascending split order from +0.  So every
// output has the bits of the split plan (gemv_kernel), whose finisher adds
// the same partials in the same order.
// LDS: the groups' core inputs [4][RT][bps*16] FP16, aliased (after a barrier)
// with the wave partials [4][4][RT][128] F32; after the last pass the row
// sums [RT][128] F32 reuse the same space.
// ---------------------------------------------------------------------------
constexpr int OWNER_GROUPS = 4;
constexpr int OWNER_THREADS = GEMV_THREADS * OWNER_GROUPS;

inline size_t owner_lds_bytes(uint32_t rows_template, uint32_t bps) {
    const size_t act = size_t(OWNER_GROUPS) * rows_template * bps * 16 * 2;
    const size_t red = size_t(OWNER_GROUPS) * GEMV_WAVES * rows_template * 128 * 4;
    return act > red ? act : red;
}

template <int K, int CB, int RT>
__global__ __launch_bounds__(OWNER_THREADS) void gemv_owner_kernel(GemvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const uint32_t cz = blockIdx.x, z = cz / a.ncg, c = cz - z * a.ncg;
    const int tid = threadIdx.x, grp = __builtin_amdgcn_readfirstlane(tid >> 8),
              w = __builtin_amdgcn_readfirstlane((tid >> 6) & 3), lane = tid & 63;
    const int jt = lane >> 3, g = lane & 7;
    const GroupWeights gw = group_weights(a, int(z));
    const float* x = a.x + z * a.x_group_stride;
    float* y = a.y + z * a.y_group_stride;

    constexpr uint32_t tile_bytes = 32u * K;
    const uint32_t row_bytes = (a.N >> 4) * tile_bytes;
    const uint32_t lane_off = (8u * c + jt) * tile_bytes + g * 4u * K;
    const int nb = a.bps / GEMV_WAVES;
    const uint32_t act_row = a.bps * 16;
    _Float16* act = reinterpret_cast<_Float16*>(smem) + size_t(grp) * RT * act_row;   // [RT][bps*16]
    float* red = reinterpret_cast<float*>(smem);                                       // [4][4][RT][128]
    constexpr uint32_t kOutOfRange = 0x80000000u;
    const int hblocks = a.bps / 8, units = RT * hblocks;
    const bool first = g == 0;

    float sum = 0.0f;   // thread tid < RT*128: output (tid / 128, tid % 128)
    for (uint32_t s0 = 0; s0 < a.splits; s0 += OWNER_GROUPS) {
        const uint32_t s = s0 + uint32_t(grp);
        const bool active = s < a.splits;
        MfmaAcc<RT> acc;
        mfma_acc_zero(acc);
        Chunk<K> ring[4];
        const uint32_t a0 = (active ? s : s0) * a.bps;
        const auto rsrc = make_rsrc(reinterpret_cast<const char*>(gw.trellis) + uint64_t(a0) * row_bytes,
                                    active ? a.bps * row_bytes : 0u);
        auto block_off = [&](int t) -> uint32_t {
            return t < nb ? (w + GEMV_WAVES * t) * row_bytes + lane_off : kOutOfRange;
        };
        if (active) {
            auto unit_load = [&](int u) -> InputLoad {
                const int r = u / hblocks, hb = u % hblocks;
                const uint32_t ch = a0 * 16 + hb * 128;
                const bool live = uint32_t(r) < a.rows;
                return input_load(x + (live ? r * a.x_row_stride : 0) + ch, gw.suh + ch, live);
            };
            auto unit_out = [&](int u) -> _Float16* { return act + (u / hblocks) * act_row + (u % hblocks) * 128; };
            const InputLoad pre0 = unit_load(w < units ? w : 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < 4; ++u) load_chunk(ring[u], rsrc, block_off(u));
            if (w < units) input_compute(pre0, unit_out(w));
            for (int u = w + GEMV_WAVES; u < units; u += GEMV_WAVES) input_compute(unit_load(u), unit_out(u));
        }
        __syncthreads();
        if (active) {
            for (int t = 0; t < nb; t += 4) {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    Chunk<K>& slot = ring[u];
                    if (t + u < nb) {
                        half2_t wq[4][4];
                        link_chunk(slot, first);
                        decode_chunk<K, CB>(slot, wq);
                        mfma_dot_block<RT>(wq, act + (w + GEMV_WAVES * (t + u)) * 16, act_row, acc);
                    }
                    load_chunk(slot, rsrc, block_off(t + u + 4));
                }
            }
        }
        __syncthreads();   // every group's dots are done: the partials may overwrite the inputs
        if (active) mfma_partials<RT>(acc, red + (grp * GEMV_WAVES + w) * RT * 128);
        __syncthreads();
        if (tid < RT * 128) {
            const int r = tid >> 7, n = tid & 127;
#pragma unroll
            for (int j = 0; j < OWNER_GROUPS; ++j) {
                if (s0 + uint32_t(j) >= a.splits) break;
                const float* pj = red + (j * GEMV_WAVES * RT + r) * 128 + n;
                float v = pj[0];
#pragma unroll
                for (int ww = 1; ww < GEMV_WAVES; ++ww) v = v + pj[ww * RT * 128];
                sum = sum + v;
            }
        }
        __syncthreads();   // the partials are read before the next pass's inputs overwrite them
    }
    float* rows = reinterpret_cast<float*>(smem);   // [RT][128]
    if (tid < RT * 128) rows[tid] = sum;
    __syncthreads();
    const int wv = tid >> 6;
    if (wv < RT && uint32_t(wv) < a.rows) {
        const ColumnOperands op = column_operands(gw, int(c), a.N);
        float z0 = rows[wv * 128 + lane], z1 = rows[wv * 128 + lane + 64];
        h32_wave(z0, z1);
        const int n0 = 128 * int(c) + lane, n1 = n0 + 64;
        float* yr = y + wv * a.y_row_stride;
        const float o0 = output_value(z0, op.sv0, gw.bias != nullptr, op.b0, a.alpha, a.beta, yr + n0);
        const float o1 = output_value(z1, op.sv1, gw.bias != nullptr, op.b1, a.alpha, a.beta, yr + n1);
        *(__attribute__((address_space(1))) float*)(yr + n0) = o0;
        *(__attribute__((address_space(1))) float*)(yr + n1) = o1;
    }
}

// Second launch of the two-kernel path: fold + output stage per column group.
__global__ __launch_bounds__(GEMV_THREADS) void gemv_finish_kernel(GemvArgs a);

// Decode to FP16 Q[I][N] (diagnostic): grid (N/128, I/16), one wave per 8 tiles.
template <int K, int CB>
__global__ __launch_bounds__(64) void decode_kernel(const uint32_t* trellis, uint32_t N, uint64_t bytes,
                                                    _Float16* q) {
    const int c = blockIdx.x, blk = blockIdx.y, lane = threadIdx.x;
    const int jt = lane >> 3, g = lane & 7;
    constexpr uint32_t tile_bytes = 32u * K;
    const uint32_t row_bytes = (N >> 4) * tile_bytes;
    const auto rsrc = make_rsrc(reinterpret_cast<const char*>(trellis) + uint64_t(blk) * row_bytes, row_bytes);
    Chunk<K> ch;
    load_chunk(ch, rsrc, (8u * c + jt) * tile_bytes + g * 4u * K);
    link_chunk(ch, g == 0);
    half2_t wq[4][4];
    decode_chunk<K, CB>(ch, wq);
    const uint64_t col0 = 16u * (8u * c + jt) + g, col1 = col0 + 8;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const uint64_t r0 = 16u * blk + 2 * v, r8 = r0 + 8;
        q[r0 * N + col0] = wq[v][0].x;
        q[(r0 + 1) * N + col0] = wq[v][0].y;
        q[r8 * N + col0] = wq[v][1].x;
        q[(r8 + 1) * N + col0] = wq[v][1].y;
        q[r0 * N + col1] = wq[v][2].x;
        q[(r0 + 1) * N + col1] = wq[v][2].y;
        q[r8 * N + col1] = wq[v][3].x;
        q[(r8 + 1) * N + col1] = wq[v][3].y;
    }
}

struct GemvLaunch {
    GemvArgs args;
    dim3 grid;
    uint32_t rows_template;   // 1, 2, 4 or 8 (the owner-fold kernel also 3 and 6)
    uint32_t codebook;
    size_t lds;
    hipStream_t stream;
};

template <int K>
hipError_t gemv_dispatch(const GemvLaunch& l);
// Owner-fold launch: grid = groups * ncg workgroups of OWNER_THREADS.
template <int K>
hipError_t gemv_owner_dispatch(const GemvLaunch& l);
template <int K>
hipError_t decode_dispatch(uint32_t codebook, const uint32_t* trellis, uint32_t I, uint32_t N, uint64_t bytes,
                           _Float16* q, hipStream_t stream);

#define STX_INSTANTIATE_GEMV(K)                                                                           \
    template <>                                                                                           \
    hipError_t gemv_dispatch<K>(const GemvLaunch& l) {                                                    \
        using Fn = void (*)(const uint32_t*, const uint16_t*, const float*, uint32_t*, const GroupWeights*,  \
                            uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, GemvArgs);                   \
        static const Fn table[3][4] = {                                                                   \
            {gemv_kernel<K, 0, 1>, gemv_kernel<K, 0, 2>, gemv_kernel<K, 0, 4>, gemv_kernel<K, 0, 8>},     \
            {gemv_kernel<K, 1, 1>, gemv_kernel<K, 1, 2>, gemv_kernel<K, 1, 4>, gemv_kernel<K, 1, 8>},     \
            {gemv_kernel<K, 2, 1>, gemv_kernel<K, 2, 2>, gemv_kernel<K, 2, 4>, gemv_kernel<K, 2, 8>}};    \
        const int rt = int(l.rows_template);                                                              \
        if (rt != 1 && rt != 2 && rt != 4 && rt != 8) return hipErrorInvalidValue;                       \
        const int ri = rt <= 2 ? rt - 1 : rt == 4 ? 2 : 3;                                                \
        const GemvArgs& a = l.args;                                                                       \
        if (a.ncg > 0xFFFFu || a.groups > 0xFFFFu || a.bps > 0xFFFFu || a.splits > 0xFFFFu ||             \
            a.rows > 0xFFu || a.mode > 0xFFu || a.x_row_stride > 0xFFFFFFFFull)                           \
            return hipErrorInvalidValue;                                                                  \
        /* two dispatch rounds (257..512 workgroups): the first round ends at grid - 256 */               \
        const uint32_t gx = l.grid.x;                                                                     \
        const uint32_t fre = gx > kGemvCus && gx <= 2 * kGemvCus ? gx - kGemvCus : 0u;                    \
        hipLaunchKernelGGL(table[l.codebook][ri], l.grid, dim3(GEMV_THREADS), l.lds, l.stream, a.w.trellis, \
                           a.w.suh, a.x, a.state.epochs, a.table, a.ncg | (a.groups << 16),                \
                           a.bps | (a.splits << 16), a.rows | (a.mode << 8) | (fre << 16), a.N,           \
                           uint32_t(a.x_row_stride), a);                                                  \
        return hipGetLastError();                                                                         \
    }                                                                                                     \
    template <>                                                                                           \
    hipError_t gemv_owner_dispatch<K>(const GemvLaunch& l) {                                              \
        using Fn = void (*)(GemvArgs);                                                                    \
        static const Fn table[3][6] = {                                                                   \
            {gemv_owner_kernel<K, 0, 1>, gemv_owner_kernel<K, 0, 2>, gemv_owner_kernel<K, 0, 3>,          \
             gemv_owner_kernel<K, 0, 4>, gemv_owner_kernel<K, 0, 6>, gemv_owner_kernel<K, 0, 8>},         \
            {gemv_owner_kernel<K, 1, 1>, gemv_owner_kernel<K, 1, 2>, gemv_owner_kernel<K, 1, 3>,          \
             gemv_owner_kernel<K, 1, 4>, gemv_owner_kernel<K, 1, 6>, gemv_owner_kernel<K, 1, 8>},         \
            {gemv_owner_kernel<K, 2, 1>, gemv_owner_kernel<K, 2, 2>, gemv_owner_kernel<K, 2, 3>,          \
             gemv_owner_kernel<K, 2, 4>, gemv_owner_kernel<K, 2, 6>, gemv_owner_kernel<K, 2, 8>}};        \
        const int rt = int(l.rows_template);                                                              \
        const int ri = rt <= 4 ? rt - 1 : rt == 6 ? 4 : 5;                                                \
        hipLaunchKernelGGL(table[l.codebook][ri], l.grid, dim3(OWNER_THREADS), l.lds, l.stream, l.args);  \
        return hipGetLastError();                                                                         \
    }                                                                                                     \
    template <>                                                                                           \
    hipError_t decode_dispatch<K>(uint32_t codebook, const uint32_t* trellis, uint32_t I, uint32_t N,     \
                                  uint64_t bytes, _Float16* q, hipStream_t stream) {                      \
        using Fn = void (*)(const uint32_t*, uint32_t, uint64_t, _Float16*);                               \
        static const Fn table[3] = {decode_kernel<K, 0>, decode_kernel<K, 1>, decode_kernel<K, 2>};       \
        hipLaunchKernelGGL(table[codebook], dim3(N / 128, I / 16), dim3(64), 0, stream, trellis, N, bytes, q); \
        return hipGetLastError();                                                                         \
    }

}  // namespace stx
