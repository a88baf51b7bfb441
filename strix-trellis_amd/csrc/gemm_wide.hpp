// Prefill GEMM, wide variant for M >= 256: workgroup tile 256 x 256, eight
// waves (two per SIMD) of 128 x 64, K stages of 64 channels.
//
// Measured on MI355X: v_mfma_f32_16x16x32_f16 reaches ~77% of peak with two
// waves per SIMD but only ~51% with one; LDS reads run at ~150 B/clk/CU and
// the vector-memory path at ~64 B/clk/CU.  So both operands are staged once
// per workgroup in LDS (never re-read per wave from L2) and waves are 128 x 64
// (operand bytes per flop 1/64 + 1/128 instead of 1/32 for 64 x 64).  Per stage:
//   * A (256 rows x 64 channels, 32 KiB) is copied from the fragment-ordered
//     core input in global memory into LDS through VGPRs, one stage ahead;
//   * B (64 x 256 = 4 input blocks x 16 tiles) is decoded from the trellis:
//     wave w decodes block w / 2, tiles 8 (w % 2) .. +7, one chunk per lane,
//     straight into MFMA B-fragment order in LDS; the raw chunks stream
//     through a register ring 2 stages deep;
//   * each wave runs 2 K32 steps x 8 x 4 v_mfma_f32_16x16x32_f16.
// LDS: A and B double-buffered, 4 x 32 KiB; the epilogue reuses it as a
// [128][256] FP32 tile (one half of the rows at a time) so each wave can run
// H128 over whole 128-column groups.
#pragma once
#include <type_traits>

#include "gemm_kernel.hpp"

namespace stx {

constexpr int WIDE_TILE_BYTES = 16 * 2 * 64 * 16;   // 16 fragment rows/tiles x 2 K32 x 64 lanes x 16 B
constexpr int WIDE_EPI_STRIDE = 260;                 // floats per staged row (256 + pad)
constexpr size_t WIDE_LDS_BYTES =
    5 * size_t(WIDE_TILE_BYTES) > 128 * WIDE_EPI_STRIDE * 4 ? 5 * size_t(WIDE_TILE_BYTES) : 128 * WIDE_EPI_STRIDE * 4;

template <int K, int CB>
__global__ __launch_bounds__(512) void gemm_wide_kernel(GemmArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned char* abuf = smem;                          // 3 x [16 rb][2 k32][64][16 B]
    unsigned char* bbuf = smem + 3 * WIDE_TILE_BYTES;    // 2 x [16 tiles][2 k32][64][16 B]
    const int c = blockIdx.x, mb = blockIdx.y;           // c: 256-column block
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int wm = w >> 2, wn = w & 3;
    const int jt8 = lane >> 3, g = lane & 7;
    const uint32_t I = a.I, N = a.N, stages = I / 64;

    constexpr uint32_t tile_bytes = 32u * K;
    const uint32_t row_bytes = (N >> 4) * tile_bytes;
    const auto wrsrc = make_rsrc(a.trellis, uint32_t(uint64_t(I / 16) * row_bytes));
    const auto arsrc = make_rsrc(a.afrag, uint32_t(a.afrag_bytes));
    const int dblk = w >> 1, dtile = 8 * (w & 1) + jt8;  // decode role
    const uint32_t lane_off = (16u * c + dtile) * tile_bytes + g * 4u * K;

    // ---- B: chunk ring (stage st in slot st % D), one chunk per lane ----
    constexpr int D = 1;   // chunk ring depth; 2 would spill at 256 VGPRs
    Chunk<K> ring[D];
    auto load_stage = [&](Chunk<K>& dst, uint32_t st) {
        load_chunk(dst, wrsrc, st < stages ? (st * 4 + dblk) * row_bytes + lane_off : 0x80000000u);
    };
    auto store_bfrag = [&](const half2_t (&wq)[4][4], int buf) {
        unsigned char* base = bbuf + buf * WIDE_TILE_BYTES;
        const int k32 = dblk >> 1, kg = (dblk & 1) * 2;
        auto frag = [&](int n, int kgroup) -> u32x4* {
            return reinterpret_cast<u32x4*>(base + ((dtile * 2 + k32) * 64 + kgroup * 16 + n) * 16);
        };
        *frag(g, kg) = u32x4{as_u32(wq[0][0]), as_u32(wq[1][0]), as_u32(wq[2][0]), as_u32(wq[3][0])};
        *frag(g, kg + 1) = u32x4{as_u32(wq[0][1]), as_u32(wq[1][1]), as_u32(wq[2][1]), as_u32(wq[3][1])};
        *frag(g + 8, kg) = u32x4{as_u32(wq[0][2]), as_u32(wq[1][2]), as_u32(wq[2][2]), as_u32(wq[3][2])};
        *frag(g + 8, kg + 1) = u32x4{as_u32(wq[0][3]), as_u32(wq[1][3]), as_u32(wq[2][3]), as_u32(wq[3][3])};
    };
    auto decode_stage = [&](Chunk<K>& src, int buf) {
        link_chunk(src, g == 0);
        half2_t wq[4][4];
        decode_chunk<K, CB>(src, wq);
        store_bfrag(wq, buf);
    };

    // ---- A: wave w DMAs fragments 4w..4w+3 (fragment f = row block f/2, K32 step f%2)
    // of a stage straight into LDS (buffer_load ... lds).  Three A buffers:
    // stage st is issued two stages ahead, into buffer st % 3.
    auto dma_a = [&](uint32_t st) {
        const uint32_t kb = st < stages ? 2 * st : 0;
        unsigned char* base = abuf + (st % 3) * WIDE_TILE_BYTES;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int f = 4 * w + q;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                arsrc, (__attribute__((address_space(3))) void*)(base + f * 1024), 16,
                uint32_t(afrag_offset(uint32_t(mb) * 16 + (f >> 1), kb + (f & 1), I, lane)), 0, 0, 0);
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

    float4_t acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // Prologue: A stages 0 and 1 in flight, B stage 0 decoded, chunk ring full.
    load_stage(ring[0], 0);
    load_stage(ring[1], 1);
    __builtin_amdgcn_sched_barrier(0);
    dma_a(0);
    dma_a(1);
    __builtin_amdgcn_sched_barrier(0);
    decode_stage(ring[0], 0);
    load_stage(ring[0], D);
    __builtin_amdgcn_sched_barrier(0);
    stage_barrier(std::integral_constant<int, 4 + kChunkOps>{});   // A stage 0 landed

    for (uint32_t st0 = 0; st0 < stages; st0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const uint32_t st = st0 + d;
            __builtin_amdgcn_sched_barrier(0);
            dma_a(st + 2);
            __builtin_amdgcn_sched_barrier(0);
            // One instruction stream per stage: the MFMAs of stage st and the
            // VALU decode of stage st + 1 are independent, and they are
            // interleaved in source order -- one weight pair decoded after
            // every 4 MFMAs -- so the matrix core and the VALU work at the
            // same time (issued as two phases they take turns: both waves of
            // a SIMD move in lockstep between barriers).  The decoder's inline
            // v_mad_u32_u16 pins the order for the machine scheduler.
            // stages = I / 64 is even, so every unrolled stage is live.
            const unsigned char* ab = abuf + (st % 3) * WIDE_TILE_BYTES;
            const unsigned char* bb = bbuf + (st & 1) * WIDE_TILE_BYTES;
            const int slot = (d + 1) % D;   // compile-time after unrolling
            Chunk<K>& dc = ring[slot];
            link_chunk(dc, g == 0);
            half2_t wq[4][4];
#pragma unroll
            for (int k32 = 0; k32 < 2; ++k32) {
                half8_t bf[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    bf[j] = *reinterpret_cast<const half8_t*>(bb + (((4 * wn + j) * 2 + k32) * 64 + lane) * 16);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const half8_t af =
                        *reinterpret_cast<const half8_t*>(ab + (((8 * wm + i) * 2 + k32) * 64 + lane) * 16);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[i][j], 0, 0, 0);
                    decode_pair_at<K, CB>(dc, wq, 8 * k32 + i);
                }
            }
            // Decoded stage st + 1 -> the other B buffer (past the end: zeros
            // of out-of-range loads into an unused buffer).
            store_bfrag(wq, (st + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
            load_stage(ring[slot], st + 1 + D);
            __builtin_amdgcn_sched_barrier(0);
            // A stage st + 1 (issued one stage ago) has landed once at most the
            // last stage's chunk loads, this stage's 4 DMAs and chunk loads remain.
            stage_barrier(std::integral_constant<int, 4 + 2 * kChunkOps>{});
        }
    }

    // ---- Epilogue: rows [128 p, +128) through an LDS [128][256] FP32 tile ----
    float* tile = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        if (wm == p) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int row = 16 * i + 4 * (lane >> 4) + e;
                        const int col = 64 * wn + 16 * j + (lane & 15);
                        tile[row * WIDE_EPI_STRIDE + col] = acc[i][j][e];
                    }
        }
        __syncthreads();
        // 128 rows x 2 column groups; a wave takes one (row, group) at a time.
        for (int u = w; u < 256; u += 8) {
            const int rr = u >> 1, grp = u & 1;
            const uint32_t row = uint32_t(mb) * 256 + 128 * p + rr;
            float z0 = tile[rr * WIDE_EPI_STRIDE + 128 * grp + lane];
            float z1 = tile[rr * WIDE_EPI_STRIDE + 128 * grp + lane + 64];
            h32_wave(z0, z1);
            if (row < a.M) {
                const uint32_t n0 = 256u * c + 128u * grp + lane, n1 = n0 + 64;
                float* yr = a.y + uint64_t(row) * N;
                const float o0 = output_element(z0, ld_global(a.svh + n0), a.bias, n0, a.alpha, a.beta, yr + n0);
                const float o1 = output_element(z1, ld_global(a.svh + n1), a.bias, n1, a.alpha, a.beta, yr + n1);
                yr[n0] = o0;
                yr[n1] = o1;
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
        static const Fn table[3] = {gemm_wide_kernel<K, 0>, gemm_wide_kernel<K, 1>, gemm_wide_kernel<K, 2>}; \
        static const hipError_t attr = [] {                                                            \
            for (Fn f : table) {                                                                       \
                const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(f),             \
                    hipFuncAttributeMaxDynamicSharedMemorySize, int(WIDE_LDS_BYTES));                   \
                if (e != hipSuccess) return e;                                                         \
            }                                                                                          \
            return hipSuccess;                                                                         \
        }();                                                                                           \
        if (attr != hipSuccess) return attr;                                                           \
        const dim3 grid(l.args.N / 256, (l.args.M + 255) / 256);                                       \
        hipLaunchKernelGGL(table[l.codebook], grid, dim3(512), WIDE_LDS_BYTES, l.stream, l.args);  \
        return hipGetLastError();                                                                      \
    }

}  // namespace stx
