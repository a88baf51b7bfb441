// Prefill GEMM, wide variant for M >= 256: workgroup tile 256 x 256, eight
// waves (two per SIMD) of 128 x 64, K stages of 64 channels, built on
// v_mfma_f32_32x32x16_f16.
//
// Measured on MI355X (independent accumulators, no memory traffic): the
// 32x32x16 MFMA sustains ~2.1 PFLOP/s (85 % of the fp16 peak) with one or two
// waves per SIMD, the 16x16x32 form only ~1.3-1.5 PFLOP/s; LDS reads run at
// ~150 B/clk/CU.  So both operands are staged once per workgroup in LDS and
// each wave computes a 128 x 64 block as 4 x 2 tiles of 32 x 32.  Per stage:
//   * A (256 rows x 64 channels, 32 KiB) is DMA'd (buffer_load ... lds) from
//     the 32x16 fragment-ordered core input straight into LDS, two stages
//     ahead (three buffers);
//   * B (64 x 256 = 4 input blocks x 16 tiles) is decoded from the trellis:
//     wave w decodes block w / 2, tiles 8 (w % 2) .. +7, one chunk per lane,
//     straight into 16x32 B-fragment order in LDS (double-buffered); the
//     decode of stage st + 1 is interleaved with the MFMAs of stage st;
//   * each wave runs 4 K16 steps x 4 x 2 v_mfma_f32_32x32x16_f16.
// LDS: 3 A + 2 B buffers of 32 KiB; the epilogue reuses it as a [128][256]
// FP32 tile (one half of the rows at a time) so each wave can run H128 over
// whole 128-column groups.
//
// MFMA 32x32x16 f16 operand layout (lane l, e = 0..7, r = 0..15), checked on
// the device:  A: A[l % 32][8 (l / 32) + e]   B: B[8 (l / 32) + e][l % 32]
//              D: D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32]
// Per output the K order is the MFMA K16 steps in ascending K from +0, as in
// every other GEMM path here (the order inside one MFMA is the hardware's),
// so rows have the same bits whichever tile computes them.
#pragma once
#include <type_traits>

#include "gemm_kernel.hpp"

namespace stx {

typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int WIDE_TILE_BYTES = 32 * 64 * 16;        // 32 fragments (8 x 4 K16) x 64 lanes x 16 B
constexpr int WIDE_EPI_STRIDE = 260;                 // floats per staged row (256 + pad)
constexpr size_t WIDE_LDS_BYTES =
    5 * size_t(WIDE_TILE_BYTES) > 128 * WIDE_EPI_STRIDE * 4 ? 5 * size_t(WIDE_TILE_BYTES) : 128 * WIDE_EPI_STRIDE * 4;

// Byte offset of the 32 x 16 A fragment (32-row block rb, 16-channel block kb) of lane l.
__host__ __device__ __forceinline__ uint64_t afrag32_offset(uint32_t rb, uint32_t kb, uint32_t I, uint32_t lane) {
    return ((uint64_t(rb) * (I / 16) + kb) * 64 + lane) * 16;
}

// Work items.  Without a handoff every workgroup computes one whole tile.
// With one (M = 2048 on 4096 -> 12288: 384 tiles for 256 CUs, one workgroup
// per CU at a time) x tiles are split at half of K: the grid is [x heads]
// [256 q whole tiles][x tails], dispatched in that order.  A head computes K
// stages [0, S/2) of its tile and publishes the FP32 accumulators; its CU then
// takes the next whole tile; a tail, dispatched last, continues the same tile
// over [S/2, S).  The accumulators carry over exactly, so every output keeps
// the bits of an unsplit tile, and each CU runs about q + 1/2 tile-times
// instead of q + 1.
enum : int { kItemFull = 0, kItemHead = 1, kItemTail = 2 };

// K split (no handoff; a pass whose tiles fill at most half the CUs): grid y is
// the split s, which computes K stages [s * stages / S, (s + 1) * stages / S)
// of its tile from +0 and writes the raw accumulators to planes[s][M][N]; a
// second launch folds the planes in ascending s and runs the output stage.

// Handoff flags: 0 idle, 1 head published, 2 head abandoned.  The tail polls
// (bounded; its head was dispatched before it, so the wait ends); when the
// head is late it takes the tile over from K = 0 instead, and whichever of the
// two comes second puts the flag back to 0, so it is 0 at the end of every
// launch.
constexpr uint32_t kHandoffForceRecompute = 0xFFFFFFFFu;   // poll_limit: always take over

// BN = 256: 8 waves as 2 (M) x 4 (N), each 128 x 64 (4 x 2 MFMA tiles), all
// eight decode.  BN = 128: 4 (M) x 2 (N), each 64 x 64 (2 x 2 tiles); the
// stage's B is 8 tiles x 4 blocks, decoded by waves 0..3 (one per SIMD) while
// waves 4..7 issue empty chunk loads so every wave counts the same vmcnt.
template <int K, int CB, int BN, bool HANDOFF>
__global__ __launch_bounds__(512) void gemm_wide_kernel(GemmArgs a) {
    static_assert(!HANDOFF || BN == 256, "the handoff runs on 256 x 256 tiles");
    constexpr int WNW = BN / 64;                         // waves along N
    constexpr int TI = 256 / (8 / WNW) / 32;             // 32-row MFMA tiles per wave
    constexpr int TJ = 2;                                // 32-column MFMA tiles per wave
    constexpr int NT = BN / 16;                          // trellis tiles per stage row
    extern __shared__ __align__(16) unsigned char smem[];   // all 160 KiB: no static LDS besides
    unsigned char* abuf = smem;                          // 3 x [8 rb32][4 kb16][64][16 B]
    unsigned char* bbuf = smem + 3 * WIDE_TILE_BYTES;    // 2 x [BN/32 n32][4 kb16][64][16 B]
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int wm = w / WNW, wn = w % WNW;
    const int jt8 = lane >> 3, g = lane & 7;
    const uint32_t I = a.I, N = a.N, stages = I / 64, half = stages / 2;

    constexpr uint32_t tile_bytes = 32u * K;
    const uint32_t row_bytes = (N >> 4) * tile_bytes;
    const auto wrsrc = make_rsrc(a.trellis, uint32_t(uint64_t(I / 16) * row_bytes));
    const auto arsrc = make_rsrc(a.afrag, uint32_t(a.afrag_bytes));
    constexpr int kDecoders = NT * 4 / 8;                // wave units of 8 tiles x 1 block
    const bool decoder = BN == 256 || w < kDecoders;
    const int dblk = BN == 256 ? w >> 1 : w & 3;         // decode role
    const int dtile = BN == 256 ? 8 * (w & 1) + jt8 : jt8;

    // XCD-aware tile order: workgroup i runs on XCD i % 8 (round-robin
    // dispatch), and each XCD takes a contiguous run of tiles in row-block-major
    // order, so the workgroups of one XCD share A row blocks in its own L2.
    // With the handoff, XCD x owns tiles [x * per_xcd, +per_xcd): 32 q whole
    // tiles, then x / 8 split ones; every role keeps a tile on its XCD.
    const uint32_t per_xcd = a.tiles / 8;
    int kind = kItemFull;
    uint32_t t, hslot = 0;
    if constexpr (!HANDOFF) {
        t = blockIdx.x;
        if (a.tiles % 8 == 0) t = (t % 8) * per_xcd + t / 8;
    } else {
        const uint32_t i = blockIdx.x, whole = 256 * a.q;
        if (i < a.x || i >= a.x + whole) {
            kind = i < a.x ? kItemHead : kItemTail;
            hslot = i < a.x ? i : i - a.x - whole;
            t = (hslot % 8) * per_xcd + 32 * a.q + hslot / 8;
        } else {
            const uint32_t j = i - a.x;
            t = (j % 8) * per_xcd + j / 8;
        }
    }
    const int c = t % a.col_blocks + a.col_block0, mb = t / a.col_blocks;   // c: BN-column block
    const uint32_t lane_off = (uint32_t(NT) * c + dtile) * tile_bytes + g * 4u * K;

    // Partial accumulators of split tile hslot: element e of wave w's lane l
    // at [hslot][w][e][l] (coalesced per element).
    auto hpart = [&]() -> float* { return a.handoff + ((uint64_t(hslot) * 8 + w) * (TI * TJ * 16)) * 64 + lane; };

    // K stages [s0, s_end) of this item.
    const uint32_t split = HANDOFF ? 0 : blockIdx.y;
    uint32_t s0 = HANDOFF ? 0 : uint32_t(uint64_t(split) * stages / a.splits);
    uint32_t s_end = HANDOFF ? (kind == kItemHead ? half : stages) : uint32_t(uint64_t(split + 1) * stages / a.splits);
    if (HANDOFF && kind == kItemTail) {
        if (tid == 0) {
            uint32_t* flag = a.flags + hslot;
            int take = 0;
            if (a.poll_limit != kHandoffForceRecompute) {
                for (uint32_t spin = 0;; ++spin) {
                    if (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 1u) {
                        take = 1;
                        break;
                    }
                    if (spin >= a.poll_limit) break;
                    __builtin_amdgcn_s_sleep(8);
                }
            }
            if (take) {
                __hip_atomic_store(flag, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                // Abandon: from here on the head's publish fails.  If it was
                // published in the meantime, this side clears the flag.
                const uint32_t old = __hip_atomic_exchange(flag, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (old == 1u) __hip_atomic_store(flag, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            *reinterpret_cast<volatile int*>(smem) = take;
        }
        __syncthreads();
        if (*reinterpret_cast<volatile int*>(smem)) s0 = half;
        __syncthreads();   // every wave has read it before the prologue's DMAs reuse the word
    }

    // ---- B: chunk ring (stage st in slot st % D), one chunk per lane ----
    constexpr int D = 1;   // chunk ring depth; 2 would spill at 256 VGPRs
    Chunk<K> ring[D];
    auto load_stage = [&](Chunk<K>& dst, uint32_t st) {
        load_chunk(dst, wrsrc, (decoder && st < s_end) ? (st * 4 + dblk) * row_bytes + lane_off : 0x80000000u);
    };
    // Lane (tile dtile, chunk g) holds rows 0..15 of tile columns g and g+8 of
    // input block dblk: column n = 16 (dtile % 2) + g (+8) of 32-column block
    // dtile / 2; rows 0..7 go to fragment lane n, rows 8..15 to lane 32 + n.
    auto store_bfrag = [&](const half2_t (&wq)[4][4], int buf) {
        unsigned char* base = bbuf + buf * WIDE_TILE_BYTES + ((dtile >> 1) * 4 + dblk) * 1024;
        const int n = 16 * (dtile & 1) + g;
        auto frag = [&](int l) -> u32x4* { return reinterpret_cast<u32x4*>(base + l * 16); };
        *frag(n) = u32x4{as_u32(wq[0][0]), as_u32(wq[1][0]), as_u32(wq[2][0]), as_u32(wq[3][0])};
        *frag(32 + n) = u32x4{as_u32(wq[0][1]), as_u32(wq[1][1]), as_u32(wq[2][1]), as_u32(wq[3][1])};
        *frag(n + 8) = u32x4{as_u32(wq[0][2]), as_u32(wq[1][2]), as_u32(wq[2][2]), as_u32(wq[3][2])};
        *frag(40 + n) = u32x4{as_u32(wq[0][3]), as_u32(wq[1][3]), as_u32(wq[2][3]), as_u32(wq[3][3])};
    };
    auto decode_stage = [&](Chunk<K>& src, int buf) {
        if (!decoder) return;
        link_chunk(src, g == 0);
        half2_t wq[4][4];
        decode_chunk<K, CB>(src, wq);
        store_bfrag(wq, buf);
    };

    // ---- A: wave w DMAs fragments 4w..4w+3 (fragment f = 32-row block f/4,
    // K16 step f%4) of a stage straight into LDS (buffer_load ... lds).  Three
    // A buffers: stage st is issued two stages ahead, into buffer st % 3.
    auto dma_a = [&](uint32_t st) {
        const uint32_t kb = st < s_end ? 4 * st : 0;
        unsigned char* base = abuf + (st % 3) * WIDE_TILE_BYTES;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int f = 4 * w + q;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                arsrc, (__attribute__((address_space(3))) void*)(base + f * 1024), 16,
                uint32_t(afrag32_offset(uint32_t(mb) * 8 + (f >> 2), kb + (f & 3), I, lane)), 0, 0, 0);
        }
    };
    // The compiler does not see the LDS side of these loads, so their
    // completion is awaited by hand: vmcnt(n) with n the vector-memory
    // operations issued after the awaited ones.  Per stage the issue order is
    // [4 A DMAs][decode][kChunkOps chunk loads].
    constexpr int kChunkOps = K <= 4 ? 1 : 2;
    // Stage barrier: this wave's LDS writes done (lgkmcnt(0)), its A DMAs of
    // the next stage done (vmcnt(n)), then s_barrier.  The memory clobber keeps
    // the compiler from moving LDS accesses across it; __syncthreads() would
    // instead drain every LDS DMA in flight (its release fence covers them),
    // losing the two-stage A prefetch.
    auto stage_barrier = [](auto n) {
        constexpr int v = decltype(n)::value;
        static_assert(v < 16, "vmcnt immediate");
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(v) : "memory");
    };

    float16_t acc[TI][TJ];
    if (!HANDOFF || s0 == 0) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) acc[i][j] = float16_t{};
    } else {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = load_coherent(hpart() + ((i * TJ + j) * 16 + r) * 64);
    }

    // Prologue: A stages s0 and s0 + 1 in flight, B stage s0 decoded, chunk ring full.
#pragma unroll
    for (int d = 0; d < D; ++d) load_stage(ring[d], s0 + d);
    __builtin_amdgcn_sched_barrier(0);
    dma_a(s0);
    dma_a(s0 + 1);
    __builtin_amdgcn_sched_barrier(0);
    decode_stage(ring[0], s0 & 1);
    load_stage(ring[0], s0 + D);
    __builtin_amdgcn_sched_barrier(0);
    stage_barrier(std::integral_constant<int, 4 + kChunkOps>{});   // A stage s0 landed

    for (uint32_t st0 = s0; st0 < s_end; st0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const uint32_t st = st0 + d;
            __builtin_amdgcn_sched_barrier(0);
            dma_a(st + 2);
            __builtin_amdgcn_sched_barrier(0);
            // One instruction stream per stage: the MFMAs of stage st and the
            // VALU decode of stage st + 1 are independent and interleaved in
            // source order (one weight pair after every two MFMAs), so the
            // matrix core and the VALU work at the same time.  The decoder's
            // inline v_mad_u32_u16 pins the order for the machine scheduler.
            const unsigned char* ab = abuf + (st % 3) * WIDE_TILE_BYTES;
            const unsigned char* bb = bbuf + (st & 1) * WIDE_TILE_BYTES;
            const int slot = (d + 1) % D;   // compile-time after unrolling
            Chunk<K>& dc = ring[slot];
            if (decoder) link_chunk(dc, g == 0);
            half2_t wq[4][4];
            // Fragments of K16 step kb + 1 are read while step kb multiplies.
            half8_t bf[2][TJ], af[2][TI];
            auto read_frags = [&](int kb) {
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    bf[kb & 1][j] = *reinterpret_cast<const half8_t*>(bb + (((TJ * wn + j) * 4 + kb) * 64 + lane) * 16);
#pragma unroll
                for (int i = 0; i < TI; ++i)
                    af[kb & 1][i] = *reinterpret_cast<const half8_t*>(ab + (((TI * wm + i) * 4 + kb) * 64 + lane) * 16);
            };
            read_frags(0);
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                if (kb < 3) read_frags(kb + 1);
#pragma unroll
                for (int i = 0; i < TI; ++i) {
#pragma unroll
                    for (int j = 0; j < TJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[kb & 1][i], bf[kb & 1][j], acc[i][j], 0, 0, 0);
                    // 16 weight pairs per stage, spread over the TI x 4 MFMA groups
                    if (decoder) {
#pragma unroll
                        for (int q = 0; q < 4 / TI; ++q) decode_pair_at<K, CB>(dc, wq, 4 * kb + (4 / TI) * i + q);
                    }
                }
            }
            // Decoded stage st + 1 -> the other B buffer (past the end: zeros
            // of out-of-range loads into an unused buffer).
            if (decoder) store_bfrag(wq, (st + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
            load_stage(ring[slot], st + 1 + D);
            __builtin_amdgcn_sched_barrier(0);
            // A stage st + 1 (issued one stage ago) has landed once at most the
            // last stage's chunk loads, this stage's 4 DMAs and chunk loads remain.
            stage_barrier(std::integral_constant<int, 4 + 2 * kChunkOps>{});
        }
    }
    // The last stages issued A DMAs past the end (dummy rows into A buffers):
    // they land before LDS is reused as the epilogue tile or by the next item.
    stage_barrier(std::integral_constant<int, 0>{});

    if (!HANDOFF && a.splits > 1) {
        float* const plane = a.planes + uint64_t(split) * a.M * N;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t row = uint32_t(mb) * 256 + 32 * TI * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    const uint32_t col = uint32_t(BN) * c + 64 * wn + 32 * j + (lane & 31);
                    if (row < a.M) plane[uint64_t(row) * N + col] = acc[i][j][r];
                }
        return;
    }

    if (HANDOFF && kind == kItemHead) {
        float* const hp = hpart();
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) store_coherent(hp + ((i * TJ + j) * 16 + r) * 64, acc[i][j][r]);
        __builtin_amdgcn_s_waitcnt(0);   // every partial store complete
        __syncthreads();
        if (tid == 0) {
            uint32_t expected = 0;
            if (!__hip_atomic_compare_exchange_strong(a.flags + hslot, &expected, 1u, __ATOMIC_RELAXED,
                                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
                __hip_atomic_store(a.flags + hslot, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // abandoned
        }
        return;
    }

    // ---- Epilogue: rows [128 p, +128) through an LDS [128][BN] FP32 tile ----
    // A wave always finishes column group w % (BN/128) of its rows, so its svh
    // and bias operands are loaded once, ahead of the first pass.
    constexpr int GROUPS = BN / 128;
    const int grp = w % GROUPS;
    const uint32_t n0 = uint32_t(BN) * c + 128u * grp + lane, n1 = n0 + 64;
    const uint16_t sv0 = ld_global(a.svh + n0), sv1 = ld_global(a.svh + n1);
    const bool has_bias = a.bias != nullptr;
    const float b0 = has_bias ? ld_global(a.bias + n0) : 0.0f, b1 = has_bias ? ld_global(a.bias + n1) : 0.0f;
    float* tile = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        if ((32 * TI * wm) / 128 == p) {
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row = (32 * TI * wm) % 128 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                        const int col = 64 * wn + 32 * j + (lane & 31);
                        tile[row * WIDE_EPI_STRIDE + col] = acc[i][j][r];
                    }
        }
        __syncthreads();
        // 128 rows x GROUPS column groups; wave w takes rows w/GROUPS + RS q of
        // group w % GROUPS, four rows per step with their butterflies interleaved.
        constexpr int RS = 8 / GROUPS;
        for (int r0 = w / GROUPS; r0 < 128; r0 += 4 * RS) {
            float z0[4], z1[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                z0[q] = tile[(r0 + RS * q) * WIDE_EPI_STRIDE + 128 * grp + lane];
                z1[q] = tile[(r0 + RS * q) * WIDE_EPI_STRIDE + 128 * grp + lane + 64];
            }
            h32_wave_multi<4>(z0, z1);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t row = uint32_t(mb) * 256 + 128 * p + r0 + RS * q;
                if (row < a.M) {
                    float* yr = a.y + uint64_t(row) * N;
                    const float o0 = output_value(z0[q], sv0, has_bias, b0, a.alpha, a.beta, yr + n0);
                    const float o1 = output_value(z1[q], sv1, has_bias, b1, a.alpha, a.beta, yr + n1);
                    *(__attribute__((address_space(1))) float*)(yr + n0) = o0;
                    *(__attribute__((address_space(1))) float*)(yr + n1) = o1;
                }
            }
        }
        __syncthreads();
    }
}

template <int K>
hipError_t gemm_wide_dispatch(const GemmLaunch& l);

#define STX_INSTANTIATE_GEMM_WIDE(K)                                                                   \
    template <>                                                                                        \
    hipError_t gemm_wide_dispatch<K>(const GemmLaunch& l) {                                            \
        using Fn = void (*)(GemmArgs);                                                                 \
        static const Fn table[3][3] = {                                                                \
            {gemm_wide_kernel<K, 0, 256, false>, gemm_wide_kernel<K, 1, 256, false>,                   \
             gemm_wide_kernel<K, 2, 256, false>},                                                      \
            {gemm_wide_kernel<K, 0, 128, false>, gemm_wide_kernel<K, 1, 128, false>,                   \
             gemm_wide_kernel<K, 2, 128, false>},                                                      \
            {gemm_wide_kernel<K, 0, 256, true>, gemm_wide_kernel<K, 1, 256, true>,                     \
             gemm_wide_kernel<K, 2, 256, true>}};                                                      \
        static const hipError_t attr = [] {                                                            \
            for (const auto& row : table)                                                              \
                for (Fn f : row) {                                                                     \
                    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(f),         \
                        hipFuncAttributeMaxDynamicSharedMemorySize, int(WIDE_LDS_BYTES));               \
                    if (e != hipSuccess) return e;                                                     \
                }                                                                                      \
            return hipSuccess;                                                                         \
        }();                                                                                           \
        if (attr != hipSuccess) return attr;                                                           \
        if (l.bn != 256 && l.bn != 128) return hipErrorInvalidValue;                                   \
        GemmArgs args = l.args;                                                                        \
        args.col_blocks = l.col_blocks;                                                                \
        args.tiles = l.col_blocks * ((l.args.M + 255) / 256);                                          \
        const uint32_t wgs = args.x ? args.tiles + args.x : args.tiles;   /* handoff: + x tails */      \
        const int variant = args.x ? 2 : l.bn == 128 ? 1 : 0;                                          \
        if (args.splits < 1 || (args.x && args.splits != 1)) return hipErrorInvalidValue;              \
        hipLaunchKernelGGL(table[variant][l.codebook], dim3(wgs, args.splits), dim3(512), WIDE_LDS_BYTES, \
                           l.stream, args);                                                            \
        return hipGetLastError();                                                                      \
    }

}  // namespace stx
