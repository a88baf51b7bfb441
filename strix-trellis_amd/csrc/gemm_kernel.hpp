// Prefill GEMM on MFMA for gfx950: C[M][N] = A[M][I] . Q[I][N] with Q decoded
// from the trellis on the fly, FP16 operands, FP32 accumulation, and the
// output stage (H128 over N, svh, bias, alpha/beta) fused into the epilogue.
//
// Replaces the reference's WMMA prefill cores (src/wmma_tiled.hip:87-269,
// src/gemm.hip:15-76) with a CDNA4 design built around v_mfma_f32_16x16x32_f16:
//
//   * workgroup tile BM x 128: 128 columns are one H128 output group, so the
//     workgroup owns complete output rows of its group and applies the output
//     stage itself; BM = 256 (8 waves as 4 x 2) or 128 (4 waves as 2 x 2);
//     each wave computes a 64 x 64 block (4 x 4 MFMA tiles of 16 x 16);
//   * K advances in stages of 128 channels (8 input blocks of 16).  In every
//     stage the workgroup decodes 8 x 8 trellis tiles: a wave decodes 8/NW
//     input blocks with the GEMV chunk decoder (lane = chunk g of tile jt) and
//     stores each lane's four 8-deep column fragments straight into the MFMA
//     B-operand order in LDS (double-buffered, 32 KiB per stage);
//   * A is read from global memory (L2-resident: every column group re-reads
//     it) in MFMA A-operand order, which the input-stage kernel already wrote:
//     one fully coalesced 16-byte load per lane per 16 x 32 fragment;
//   * per-output accumulation: MFMA K32 steps in ascending K from +0 (the
//     order inside one MFMA step is the hardware's).
//
// MFMA 16x16x32 f16 operand layout (lane l, e = 0..7 / 0..3):
//   A: A[l % 16][8 (l / 16) + e]      B: B[8 (l / 16) + e][l % 16]
//   D: D[4 (l / 16) + e][l % 16]
#pragma once
#include "backend.hpp"
#include "stages.hpp"

namespace stx {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

struct GemmArgs {
    const uint32_t* trellis;
    const uint16_t* svh;
    const float* bias;
    const _Float16* afrag;    // core input in fragment order: [ceil(M/16)][I/32][64 lanes][8]
    uint64_t afrag_bytes;
    float* y;                 // [M][N]
    uint32_t M, I, N;
    float alpha, beta;
    uint32_t col_block0;      // wide kernel: first column block of the launch,
    uint32_t col_blocks;      // column blocks launched,
    uint32_t tiles;           // and tiles (column blocks x row blocks)
    // Wide kernel K-split handoff (x > 0): x tiles of the launch split at half
    // of K between a head and a tail workgroup, 256 q whole tiles.
    uint32_t q, x;
    float* handoff;           // [x][8 waves][128 accumulators][64 lanes]
    uint32_t* flags;          // [x], 0 at launch
    uint32_t poll_limit;      // tail's polls before it takes a tile over
    // K split: `splits` workgroups per tile (narrow kernel: grid z, I/splits
    // channels each; wide kernel: grid y, stage ranges) write their raw core
    // rows to planes[s][M][N], which a second launch folds in ascending s from
    // +0 before the output stage.
    uint32_t splits;
    float* planes;
#if STX_STAGE_CLOCK
    // Instrumented build only: per-wave phase cycle records of the wide
    // kernel, [workgroup][8 waves][16] (null: none written).
    unsigned long long* clock;
#endif
};

// Byte offset of the A fragment (row block rb, 32-channel block kb) of lane l.
__host__ __device__ __forceinline__ uint64_t afrag_offset(uint32_t rb, uint32_t kb, uint32_t I, uint32_t lane) {
    return ((uint64_t(rb) * (I / 32) + kb) * 64 + lane) * 16;
}

constexpr int GEMM_STAGE_BLOCKS = 8;                              // input blocks per K stage
constexpr int GEMM_BSTAGE_BYTES = 8 * 4 * 64 * 16;                // 8 tiles x 4 K32 x 64 lanes x 16 B

template <int K, int CB, int BM>
__global__ __launch_bounds__(2 * BM) void gemm_kernel(GemmArgs a) {
    constexpr int WM = BM / 64, NW = 2 * WM, BPW = GEMM_STAGE_BLOCKS / NW;
    extern __shared__ __align__(16) unsigned char smem[];   // 2 B stages; reused by the epilogue
    const int c = blockIdx.x, mb = blockIdx.y, split = blockIdx.z;
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wm = w >> 1, wn = w & 1;
    const int jt = lane >> 3, g = lane & 7;
    // This workgroup's K range: stages (128 channels each) [split * stages, +stages).
    const uint32_t I = a.I, N = a.N, stages = I / 128 / a.splits, kb0 = uint32_t(split) * stages * 4;

    constexpr uint32_t tile_bytes = 32u * K;
    const uint32_t row_bytes = (N >> 4) * tile_bytes;
    const auto wrsrc = make_rsrc(reinterpret_cast<const char*>(a.trellis) +
                                     uint64_t(split) * stages * GEMM_STAGE_BLOCKS * row_bytes,
                                 uint32_t(uint64_t(stages) * GEMM_STAGE_BLOCKS * row_bytes));
    const auto arsrc = make_rsrc(a.afrag, uint32_t(a.afrag_bytes));
    const uint32_t lane_off = (8u * c + jt) * tile_bytes + g * 4u * K;

    // Decode role: wave w decodes input blocks w*BPW .. w*BPW+BPW-1 of each
    // stage.  Their chunks stream through a register ring D stages deep, so a
    // chunk load has D stages of MFMA work to arrive from HBM.
    constexpr int D = BPW == 1 ? 4 : 2;
    Chunk<K> ring[D][BPW];
    auto load_stage = [&](Chunk<K> (&dst)[BPW], uint32_t st) {
#pragma unroll
        for (int i = 0; i < BPW; ++i) {
            const uint32_t blk = st * GEMM_STAGE_BLOCKS + w * BPW + i;
            load_chunk(dst[i], wrsrc, st < stages ? blk * row_bytes + lane_off : 0x80000000u);
        }
    };
    auto decode_stage = [&](Chunk<K> (&src)[BPW], int buf) {
        unsigned char* base = smem + buf * GEMM_BSTAGE_BYTES;
#pragma unroll
        for (int i = 0; i < BPW; ++i) {
            link_chunk(src[i], g == 0);
            half2_t wq[4][4];
            decode_chunk<K, CB>(src[i], wq);
            const int kb = w * BPW + i;            // block within the stage
            const int k32 = kb >> 1, kg = (kb & 1) * 2;
            // fragment (column n, k-group) -> [tile][k32][lane = 16 * kgroup + n]
            auto frag = [&](int n, int kgroup) -> uint32_t* {
                return reinterpret_cast<uint32_t*>(base + ((jt * 4 + k32) * 64 + kgroup * 16 + n) * 16);
            };
            u32x4 f;
            f = {as_u32(wq[0][0]), as_u32(wq[1][0]), as_u32(wq[2][0]), as_u32(wq[3][0])};
            *reinterpret_cast<u32x4*>(frag(g, kg)) = f;
            f = {as_u32(wq[0][1]), as_u32(wq[1][1]), as_u32(wq[2][1]), as_u32(wq[3][1])};
            *reinterpret_cast<u32x4*>(frag(g, kg + 1)) = f;
            f = {as_u32(wq[0][2]), as_u32(wq[1][2]), as_u32(wq[2][2]), as_u32(wq[3][2])};
            *reinterpret_cast<u32x4*>(frag(g + 8, kg)) = f;
            f = {as_u32(wq[0][3]), as_u32(wq[1][3]), as_u32(wq[2][3]), as_u32(wq[3][3])};
            *reinterpret_cast<u32x4*>(frag(g + 8, kg + 1)) = f;
        }
    };

    // MFMA role: rows [mb*BM + 64 wm, +64), columns [64 wn, +64) of the group.
    const uint32_t rb0 = (uint32_t(mb) * BM + 64 * wm) / 16;
    auto load_a = [&](half8_t (&af)[4], uint32_t kb32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
                arsrc, uint32_t(afrag_offset(rb0 + i, kb0 + kb32, I, lane)), 0, 0);
            af[i] = __builtin_bit_cast(half8_t, v);
        }
    };
    float4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

#pragma unroll
    for (int d = 0; d < D; ++d) load_stage(ring[d], d);
    decode_stage(ring[0], 0);
    load_stage(ring[0], D);
    __syncthreads();

    // A ring: slot k32 holds the wave's four 16 x 32 fragments of K32 step
    // k32 of the current stage and is refilled with the same step of the next
    // stage as soon as it is consumed, so every A load has a full stage
    // (16 MFMAs x 4 steps) to arrive from L2 / MALL.
    half8_t af[4][4];
#pragma unroll
    for (int k32 = 0; k32 < 4; ++k32) load_a(af[k32], k32);
    // Stage st's chunks sit in ring slot st % D; the loop is unrolled by D so
    // slots are compile-time.  Loads stay unconditional (past the end they are
    // out of range or repeat a valid A step); only the MFMAs are guarded.
    for (uint32_t st0 = 0; st0 < stages; st0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const uint32_t st = st0 + d;
            const bool live = st < stages;
            const unsigned char* bbase = smem + (st & 1) * GEMM_BSTAGE_BYTES;
#pragma unroll
            for (int k32 = 0; k32 < 4; ++k32) {
                if (live) {
                    half8_t bf[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        bf[j] = *reinterpret_cast<const half8_t*>(bbase + (((4 * wn + j) * 4 + k32) * 64 + lane) * 16);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[k32][i], bf[j], acc[i][j], 0, 0, 0);
                }
                const uint32_t next = (st + 1) * 4 + k32;
                load_a(af[k32], next < stages * 4 ? next : k32);
            }
            // Decode stage st + 1 into the other buffer while MFMAs drain, and
            // refill its ring slot with stage st + 1 + D.  Past the end this
            // decodes the zeros of out-of-range loads into an unused buffer.
            const int slot = (d + 1) % D;   // compile-time after unrolling
            decode_stage(ring[slot], (st + 1) & 1);
            load_stage(ring[slot], st + 1 + D);
            __syncthreads();
        }
    }

    if (a.splits > 1) {
        // Raw core rows of this split -> its plane (folded by a second launch).
        float* plane = a.planes + uint64_t(split) * a.M * N;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t row = uint32_t(mb) * BM + 64 * wm + 16 * i + 4 * (lane >> 4) + e;
                if (row < a.M) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) plane[uint64_t(row) * N + 128 * c + 64 * wn + 16 * j + (lane & 15)] = acc[i][j][e];
                }
            }
        return;
    }

    // Epilogue, 64 rows (one wm) at a time through a [64][128] FP32 LDS tile.
    float* tile = reinterpret_cast<float*>(smem);
    for (int p = 0; p < WM; ++p) {
        if (wm == p) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int row = 16 * i + 4 * (lane >> 4) + e;
                        const int col = 64 * wn + 16 * j + (lane & 15);
                        tile[row * 129 + col] = acc[i][j][e];
                    }
        }
        __syncthreads();
        for (int rr = w; rr < 64; rr += NW) {
            const uint32_t row = uint32_t(mb) * BM + 64 * p + rr;
            float z0 = tile[rr * 129 + lane], z1 = tile[rr * 129 + lane + 64];
            h32_wave(z0, z1);
            if (row < a.M) {
                const uint32_t n0 = 128 * c + lane, n1 = n0 + 64;
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

struct GemmLaunch {
    GemmArgs args;
    uint32_t codebook;
    uint32_t bm;
    uint32_t bn, col_blocks;  // wide kernel: tile width and column blocks launched
    hipStream_t stream;
};

template <int K>
hipError_t gemm_dispatch(const GemmLaunch& l);

inline size_t gemm_lds_bytes(int bm) {
    const size_t stages = 2 * size_t(GEMM_BSTAGE_BYTES);
    const size_t epilogue = size_t(64) * 129 * 4;
    (void)bm;
    return stages > epilogue ? stages : epilogue;
}

#define STX_INSTANTIATE_GEMM(K)                                                                         \
    template <>                                                                                         \
    hipError_t gemm_dispatch<K>(const GemmLaunch& l) {                                                  \
        using Fn = void (*)(GemmArgs);                                                                  \
        static const Fn t256[3] = {gemm_kernel<K, 0, 256>, gemm_kernel<K, 1, 256>, gemm_kernel<K, 2, 256>}; \
        static const Fn t128[3] = {gemm_kernel<K, 0, 128>, gemm_kernel<K, 1, 128>, gemm_kernel<K, 2, 128>}; \
        const Fn fn = l.bm == 256 ? t256[l.codebook] : t128[l.codebook];                               \
        const dim3 grid(l.args.N / 128, (l.args.M + l.bm - 1) / l.bm, l.args.splits);                   \
        hipLaunchKernelGGL(fn, grid, dim3(2 * l.bm), gemm_lds_bytes(l.bm), l.stream, l.args);          \
        return hipGetLastError();                                                                       \
    }

}  // namespace stx
