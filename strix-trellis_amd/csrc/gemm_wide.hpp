// Prefill GEMM, wide variant for M >= 256: workgroup tile 256 x BN, eight
// waves (two per SIMD), K stages of 64 channels, built on
// v_mfma_f32_32x32x16_f16.
//
// Measured on MI355X (independent accumulators, no memory traffic): the
// 32x32x16 MFMA sustains ~2.1 PFLOP/s (85 % of the fp16 peak) with one or two
// waves per SIMD, the 16x16x32 form only ~1.3-1.5 PFLOP/s.  So both operands
// are staged once per workgroup in LDS.  Per stage:
//   * the core input (256 rows x 64 channels, 32 KiB) is DMA'd
//     (buffer_load ... lds) from the 32x16 fragment-ordered workspace straight
//     into LDS, two stages ahead (three buffers);
//   * the weights (64 x BN = 4 input blocks x BN/16 tiles) are decoded from the
//     trellis: wave w decodes one block's eight tiles, one chunk per lane,
//     straight into 32x16 fragment order in LDS (double-buffered); the decode of
//     stage st + 1 is interleaved with the MFMAs of stage st;
//   * each wave multiplies its 128 output channels by its 64 (BN = 256) or 32
//     (BN = 128) rows: 4 K16 steps x 4 x TM MFMAs.
//
// Operand roles: the decoded weights are the MFMA's A operand and the core
// input its B operand, so the accumulators hold the transposed tile
// D[channel][row].  A lane then holds 64 of the 128 channels of an output
// H128 group for each of its rows (the other 64 in lane l ^ 32), and the
// epilogue's Hadamard runs in registers: six butterfly levels between
// registers and one through v_permlane32_swap, no LDS tile.
//
// MFMA 32x32x16 f16 operand layout (lane l, e = 0..7, r = 0..15), checked on
// the device:  A: A[l % 32][8 (l / 32) + e]   B: B[8 (l / 32) + e][l % 32]
//              D: D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32]
// A weight fragment (k = 8 (l / 32) + e, column n = l % 32) and a core-input
// fragment (row m = l % 32, k = 8 (l / 32) + e) therefore enter as A[n][k] and
// B[k][m], and D[n][m] is output (row m, channel n): channel
// 8 (r / 4) + 4 (l / 32) + r % 4 of the 32-channel tile, row l % 32.
// Per output the K order is the MFMA K16 steps in ascending K from +0, as in
// every other GEMM path here (the order inside one MFMA is the hardware's),
// so rows have the same bits whichever tile computes them.
#pragma once
#include <type_traits>

#include "gemm_kernel.hpp"

namespace stx {

typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int WIDE_TILE_BYTES = 32 * 64 * 16;        // 32 fragments (8 x 4 K16) x 64 lanes x 16 B
constexpr size_t WIDE_LDS_BYTES = 5 * size_t(WIDE_TILE_BYTES);

// Bit casts through by-value parameters.  hipcc (ROCm 7.2) miscompiles
// __builtin_bit_cast applied directly to an element of an ext_vector_type
// value (it reads element 0), so vector elements pass through these.
__device__ __forceinline__ uint32_t bits_of(float v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ float float_of(uint32_t v) { return __builtin_bit_cast(float, v); }

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
// launch.  The head publishes with an agent-scope release CAS after its
// partial stores (and a workgroup barrier), the tail polls with agent-scope
// acquire loads before a barrier that orders its waves' partial loads: the
// partials are ordered before the flag in the language's memory model, not
// only by the hardware's write-through stores and wait counts.  (Measured:
// the release's L2 write-back and the acquire's invalidate cost 0.8 % at
// M = 2048 on 4096 -> 12288 K4 against relaxed flags over the same
// device-coherent partials, 221.2 vs 219.5 us; nothing at K6 or M = 1536.)
constexpr uint32_t kHandoffForceRecompute = 0xFFFFFFFFu;   // poll_limit: always take over

// Phase clock of one wave (s_memtime, shader clock cycles), compiled in only
// by the instrumented build (STX_STAGE_CLOCK=1, build.py --stage-clock); in
// the product build every member is empty.  Per K stage the loop is cut into
//   0: MFMAs of stage st with the interleaved decode of stage st + 1,
//   1: the decoded B fragments to LDS and the next chunk loads issued,
//   2: the wait for A stage st + 1 (vmcnt),
//   3: the stage barrier;
// scheduling barriers pin each mark, so the instrumented loop keeps these
// phases in this order.  A record is 16 words per wave:
//   [phase 0..3 sums][prologue][epilogue][t0][realtime0][t1][realtime1]
//   [stages][kind][tile][first stage][split][0]
// (s_memrealtime counts at 100 MHz).
struct StageClock {
#if STX_STAGE_CLOCK
    uint64_t phase[4] = {0, 0, 0, 0};
    uint64_t t0 = 0, rt0 = 0, loop0 = 0, loop1 = 0, mark = 0;
    uint32_t stages = 0;
    __device__ __forceinline__ static uint64_t now() {
        __builtin_amdgcn_sched_barrier(0);
        const uint64_t t = __builtin_amdgcn_s_memtime();
        __builtin_amdgcn_sched_barrier(0);
        return t;
    }
    __device__ __forceinline__ void begin() {
        t0 = __builtin_amdgcn_s_memtime();
        rt0 = __builtin_amdgcn_s_memrealtime();
    }
    __device__ __forceinline__ void loop_begin() { loop0 = now(); }
    __device__ __forceinline__ void stage_begin() { mark = now(); }
    template <int I>
    __device__ __forceinline__ void phase_end() {
        const uint64_t t = now();
        phase[I] += t - mark;
        mark = t;
    }
    __device__ __forceinline__ void stage_end() { ++stages; }
    __device__ __forceinline__ void loop_end() { loop1 = now(); }
    __device__ __forceinline__ void record(const GemmArgs& a, int kind, uint32_t tile, uint32_t s0) const {
        const uint64_t t1 = now(), rt1 = __builtin_amdgcn_s_memrealtime();
        if (!a.clock || (threadIdx.x & 63) != 0) return;
        const uint64_t wg = uint64_t(blockIdx.y) * gridDim.x + blockIdx.x;
        auto* r = (__attribute__((address_space(1))) unsigned long long*)(a.clock + (wg * 8 + (threadIdx.x >> 6)) * 16);
        const uint64_t v[16] = {phase[0], phase[1], phase[2], phase[3], loop0 - t0, t1 - loop1, t0, rt0,
                                t1, rt1, stages, uint64_t(kind), tile, s0, blockIdx.y, 0};
#pragma unroll
        for (int i = 0; i < 16; ++i) r[i] = v[i];
    }
#else
    __device__ __forceinline__ void begin() {}
    __device__ __forceinline__ void loop_begin() {}
    __device__ __forceinline__ void stage_begin() {}
    template <int I>
    __device__ __forceinline__ void phase_end() {}
    __device__ __forceinline__ void stage_end() {}
    __device__ __forceinline__ void loop_end() {}
    __device__ __forceinline__ void record(const GemmArgs&, int, uint32_t, uint32_t) const {}
#endif
};

// Each wave owns the 128 channels of one output H128 group and TM 32-row
// blocks: BN = 256 as 4 (M) x 2 (N) waves of 64 rows, all eight decode;
// BN = 128 as 8 (M) x 1 (N) waves of 32 rows, the stage's 8 tiles x 4 blocks
// decoded by waves 0..3 (one per SIMD) while waves 4..7 issue empty chunk
// loads so every wave counts the same vmcnt.
template <int K, int CB, int BN, bool HANDOFF>
__global__ __launch_bounds__(512) void gemm_wide_kernel(GemmArgs a) {
    static_assert(!HANDOFF || BN == 256, "the handoff runs on 256 x 256 tiles");
    static_assert(BN == 256 || BN == 128, "tile width");
    constexpr int WN = BN / 128;                         // waves along N, one H128 group each
    constexpr int TM = 256 / (8 / WN) / 32;              // 32-row MFMA tiles per wave
    constexpr int TN = 4;                                // 32-channel MFMA tiles per wave
    constexpr int NT = BN / 16;                          // trellis tiles per stage row
    extern __shared__ __align__(16) unsigned char smem[];   // all 160 KiB: no static LDS besides
    unsigned char* abuf = smem;                          // 3 x [8 rb32][4 kb16][64][16 B] core input
    unsigned char* bbuf = smem + 3 * WIDE_TILE_BYTES;    // 2 x [BN/32 n32][4 kb16][64][16 B] weights
    // The wave index is uniform: readfirstlane keeps everything derived from it in SGPRs.
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wm = w / WN, wn = w % WN;
    const int jt8 = lane >> 3, g = lane & 7;
    const uint32_t I = a.I, N = a.N, stages = I / 64, half = stages / 2;
    StageClock clk;
    clk.begin();

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

    // Partial accumulators of split tile hslot, 256 KiB per tile: elements
    // 4q .. 4q+3 of wave w's lane l at [hslot][w][q][l][4], one 16-byte
    // device-coherent (sc1) access per lane and quad, 1 KiB contiguous per
    // wave; quad q = (jn TM + im) 4 + r / 4.  (One 4-byte access per element
    // made the handoff's partial traffic the slower part of a split tile.)
    constexpr int kCoherent = 16;   // buffer cache policy bits: sc1
    const auto hrsrc = make_rsrc(a.handoff + uint64_t(hslot) * (8u * TN * TM * 16 * 64), 8u * TN * TM * 16 * 64 * 4);
    auto quad_off = [&](int q) { return uint32_t(((w * (TN * TM * 4) + q) * 64 + lane) * 16); };

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
                    if (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) == 1u) {
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
        // Uniform (readfirstlane): the K loop's counter then stays scalar.
        if (__builtin_amdgcn_readfirstlane(*reinterpret_cast<volatile int*>(smem))) s0 = half;
        __syncthreads();   // every wave has read it before the prologue's DMAs reuse the word
    }

    // ---- B: chunk ring (stage st in slot st % D), one chunk per lane ----
    constexpr int D = 1;   // chunk ring depth; 2 would spill at 256 VGPRs
    Chunk<K> ring[D];
    // The stage's part of the offset is a scalar operand.  Past the end, or for
    // a wave that does not decode, the lane offset itself goes out of range:
    // the buffer range check covers the vector and immediate offsets, not the
    // scalar one.
    auto load_stage = [&](Chunk<K>& dst, uint32_t st) {
        const bool live = decoder && st < s_end;
        load_chunk(dst, wrsrc, lane_off + (live ? 0u : 0x80000000u), live ? (st * 4 + dblk) * row_bytes : 0u);
    };
    // Lane (tile dtile, chunk g) holds rows 0..15 of tile columns g and g+8 of
    // input block dblk: column n = 16 (dtile % 2) + g (+8) of 32-column block
    // dtile / 2; rows 0..7 go to fragment lane n, rows 8..15 to lane 32 + n
    // (the A-operand order A[n][k]).
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
    // Lane part of the fragment offsets (row block 8 mb + w); the stage's K
    // part is a scalar operand (always in range), and K16 step q the
    // immediate offset q * 1 KiB, which the load adds to both the memory and
    // the LDS address.
    const uint32_t a_voff = uint32_t(afrag32_offset(uint32_t(mb) * 8 + w, 0, I, lane));
    auto dma_a = [&](uint32_t st) {
        const uint32_t a_soff = (st < s_end ? 4 * st : 0) * 1024u;
        unsigned char* base = abuf + (st % 3) * WIDE_TILE_BYTES + 4 * w * 1024;
        auto frag = [&](auto qc) {
            constexpr int q = decltype(qc)::value;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (__attribute__((address_space(3))) void*)base, 16, a_voff,
                                                     a_soff, q * 1024, 0);
        };
        frag(std::integral_constant<int, 0>{});
        frag(std::integral_constant<int, 1>{});
        frag(std::integral_constant<int, 2>{});
        frag(std::integral_constant<int, 3>{});
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

    // acc[jn][im]: channels 32 jn.. of the wave's group x rows 32 im.. of its block.
    float16_t acc[TN][TM];
    if (!HANDOFF || s0 == 0) {
#pragma unroll
        for (int jn = 0; jn < TN; ++jn)
#pragma unroll
            for (int im = 0; im < TM; ++im) acc[jn][im] = float16_t{};
    } else {
#pragma unroll
        for (int jn = 0; jn < TN; ++jn)
#pragma unroll
            for (int im = 0; im < TM; ++im)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(hrsrc, quad_off((jn * TM + im) * 4 + r4), 0,
                                                                          kCoherent);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[jn][im][4 * r4 + e] = float_of(v[e]);
                }
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
    clk.loop_begin();

    for (uint32_t st0 = s0; st0 < s_end; st0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const uint32_t st = st0 + d;
            clk.stage_begin();
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
            half8_t wf[2][TN], xf[2][TM];
            auto read_frags = [&](int kb) {
#pragma unroll
                for (int jn = 0; jn < TN; ++jn)
                    wf[kb & 1][jn] = *reinterpret_cast<const half8_t*>(bb + (((TN * wn + jn) * 4 + kb) * 64 + lane) * 16);
#pragma unroll
                for (int im = 0; im < TM; ++im)
                    xf[kb & 1][im] = *reinterpret_cast<const half8_t*>(ab + (((TM * wm + im) * 4 + kb) * 64 + lane) * 16);
            };
            read_frags(0);
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                if (kb < 3) read_frags(kb + 1);
#pragma unroll
                for (int jn = 0; jn < TN; ++jn) {
#pragma unroll
                    for (int im = 0; im < TM; ++im)
                        acc[jn][im] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[kb & 1][jn], xf[kb & 1][im], acc[jn][im], 0, 0, 0);
                    // 16 weight pairs per stage, one after each of the 4 x 4 channel groups
                    if (decoder) decode_pair_at<K, CB>(dc, wq, 4 * kb + jn);
                }
            }
            // Decoded stage st + 1 -> the other B buffer (past the end: zeros
            // of out-of-range loads into an unused buffer).
            clk.phase_end<0>();
            if (decoder) store_bfrag(wq, (st + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
            load_stage(ring[slot], st + 1 + D);
            __builtin_amdgcn_sched_barrier(0);
            clk.phase_end<1>();
            // A stage st + 1 (issued one stage ago) has landed once at most the
            // last stage's chunk loads, this stage's 4 DMAs and chunk loads remain.
#if STX_STAGE_CLOCK
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(4 + 2 * kChunkOps) : "memory");
            clk.phase_end<2>();
            asm volatile("s_barrier" ::: "memory");
            clk.phase_end<3>();
            clk.stage_end();
#else
            stage_barrier(std::integral_constant<int, 4 + 2 * kChunkOps>{});
#endif
        }
    }
    // The last stages issued A DMAs past the end (dummy rows into A buffers):
    // they land before LDS is reused as the epilogue tile or by the next item.
    stage_barrier(std::integral_constant<int, 0>{});
    clk.loop_end();

    // Lane l holds rows 32 (TM wm + im) + l % 32 of the tile and, per MFMA
    // tile jn and accumulator r, channel 32 jn + 8 (r / 4) + 4 (l / 32) + r % 4
    // of the wave's group: four consecutive channels per (jn, r / 4), stored
    // as one 16-byte access.  Row-major [rows][N] F32 outputs of the tile's 256
    // rows go through a buffer resource sized to the rows below M, so accesses
    // to rows >= M are dropped (stores) or read zeros (loads).
    const uint32_t row0 = uint32_t(mb) * 256;
    const uint32_t slab_bytes = (a.M - row0 < 256u ? a.M - row0 : 256u) * N * 4u;
    const uint32_t out_off = ((32u * TM * wm + (lane & 31)) * N + uint32_t(BN) * c + 128u * wn + 4u * (lane >> 5)) * 4u;
    auto acc4 = [&](int jn, int im, int r4) {
        return u32x4{bits_of(acc[jn][im][4 * r4]), bits_of(acc[jn][im][4 * r4 + 1]), bits_of(acc[jn][im][4 * r4 + 2]),
                     bits_of(acc[jn][im][4 * r4 + 3])};
    };

    if (!HANDOFF && a.splits > 1) {
        const auto prsrc = make_rsrc(a.planes + (uint64_t(split) * a.M + row0) * N, slab_bytes);
#pragma unroll
        for (int im = 0; im < TM; ++im)
#pragma unroll
            for (int jn = 0; jn < TN; ++jn)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    __builtin_amdgcn_raw_buffer_store_b128(acc4(jn, im, r4), prsrc, out_off + (32 * jn + 8 * r4) * 4,
                                                           32 * im * N * 4, 0);
        clk.record(a, kind, t, s0);
        return;
    }

    if (HANDOFF && kind == kItemHead) {
#pragma unroll
        for (int jn = 0; jn < TN; ++jn)
#pragma unroll
            for (int im = 0; im < TM; ++im)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    __builtin_amdgcn_raw_buffer_store_b128(acc4(jn, im, r4), hrsrc, quad_off((jn * TM + im) * 4 + r4), 0,
                                                           kCoherent);
        __builtin_amdgcn_s_waitcnt(0);   // every partial store complete
        __syncthreads();
        if (tid == 0) {
            uint32_t expected = 0;
            if (!__hip_atomic_compare_exchange_strong(a.flags + hslot, &expected, 1u, __ATOMIC_RELEASE,
                                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
                __hip_atomic_store(a.flags + hslot, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // abandoned
        }
        clk.record(a, kind, t, s0);
        return;
    }

    // ---- Epilogue: H128 per row in registers, then the output stage ----
    // The tile's svh (and bias) go to LDS by DMA while the butterflies run:
    // wave 0 brings BN x 2 B of svh to bytes [0, 1024), wave 1 BN x 4 B of
    // bias to [1024, 2048) (lanes past the end read zeros).
    const bool has_bias = a.bias != nullptr;
    if (w < (has_bias ? 2 : 1)) {
        const void* src = w == 0 ? static_cast<const void*>(a.svh + uint64_t(BN) * c)
                                 : static_cast<const void*>(a.bias + uint64_t(BN) * c);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(src, w == 0 ? BN * 2 : BN * 4),
                                                 (__attribute__((address_space(3))) void*)(smem + 1024 * w), 16,
                                                 uint32_t(lane) * 16u, 0, 0, 0);
    }
    // Butterfly levels in the reference's order, channel bit 0 first; lower
    // element a + b, upper element a - b.  Channel bits 0, 1, 3, 4 are bits of
    // r, bits 5, 6 of jn, bit 2 is lane bit 5.  The values of one row block
    // leave the accumulator tuples first (plain registers, no tuple copies).
    auto bfly = [](float& lo, float& hi) {
        const float x = lo, y = hi;
        lo = x + y;
        hi = x - y;
    };
    auto h128 = [&](auto imc, float (&v)[TN][16]) {
        constexpr int im = decltype(imc)::value;
#pragma unroll
        for (int jn = 0; jn < TN; ++jn)
#pragma unroll
            for (int r = 0; r < 16; ++r) v[jn][r] = acc[jn][im][r];
#pragma unroll
        for (int jn = 0; jn < TN; ++jn) {
            float* t = v[jn];
#pragma unroll
            for (int r = 0; r < 16; r += 2) bfly(t[r], t[r + 1]);                           // bit 0
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (!(r & 2)) bfly(t[r], t[r + 2]);                                            // bit 1
#pragma unroll
            for (int r = 0; r < 16; r += 2) {                                                  // bit 2
                // Swap the upper half of t[r] with the lower half of t[r + 1]:
                // each lane then holds both bit-2 halves of one channel pair
                // (lanes < 32: channel of t[r], lanes >= 32: of t[r + 1]);
                // the same swap afterwards restores the layout.
                const auto s1 = __builtin_amdgcn_permlane32_swap(bits_of(t[r]), bits_of(t[r + 1]), false, false);
                const float x = float_of(s1[0]), y = float_of(s1[1]);
                const auto s2 = __builtin_amdgcn_permlane32_swap(bits_of(x + y), bits_of(x - y), false, false);
                t[r] = float_of(s2[0]);
                t[r + 1] = float_of(s2[1]);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (!(r & 4)) bfly(t[r], t[r + 4]);                                            // bit 3
#pragma unroll
            for (int r = 0; r < 8; ++r) bfly(t[r], t[r + 8]);                                  // bit 4
            // One tile at a time: the scheduler's interleaving across tiles spills.
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            bfly(v[0][r], v[1][r]);                                                            // bit 5
            bfly(v[2][r], v[3][r]);
#pragma unroll
            for (int jn = 0; jn < 2; ++jn) {                                                   // bit 6, scaled
                const float x = v[jn][r], y = v[jn + 2][r];
                v[jn][r] = (x + y) * INV_SQRT128;   // (a + b) * c: nothing to contract
                v[jn + 2][r] = (x - y) * INV_SQRT128;
            }
        }
    };

    // Output stage per element, as output_value() with the operands in
    // registers: RN32(h * svh), + bias, * alpha, + RN32(beta * y).  A missing
    // bias adds -0.0, which leaves every value (signed zeros included)
    // unchanged; y is read only when beta != 0.
    const uint16_t* sv_lds = reinterpret_cast<const uint16_t*>(smem);
    const float* bias_lds = reinterpret_cast<const float*>(smem + 1024);
    const uint32_t lc0 = 128u * wn + 4u * (lane >> 5);   // first channel of the lane within the tile
    const auto yrsrc = make_rsrc(a.y + uint64_t(row0) * N, slab_bytes);
    auto emit = [&](auto imc, const float (&v)[TN][16], auto with_beta) {
        constexpr int im = decltype(imc)::value;
        constexpr bool BETA = decltype(with_beta)::value;
#pragma unroll
        for (int jn = 0; jn < TN; ++jn)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const uint32_t lc = lc0 + 32 * jn + 8 * r4;
                const uint2 sv = *reinterpret_cast<const uint2*>(sv_lds + lc);
                const float4_t bv = has_bias ? *reinterpret_cast<const float4_t*>(bias_lds + lc)
                                             : float4_t{-0.0f, -0.0f, -0.0f, -0.0f};
                const uint32_t sw[4] = {sv.x & 0xFFFFu, sv.x >> 16, sv.y & 0xFFFFu, sv.y >> 16};
                const uint32_t off = out_off + (32 * jn + 8 * r4) * 4;
                u32x4 old{};
                if constexpr (BETA) old = __builtin_amdgcn_raw_buffer_load_b128(yrsrc, off, 32 * im * N * 4, 0);
                u32x4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float y = rn32(v[jn][4 * r4 + e] * half_bits_to_float(uint16_t(sw[e])));
                    y = rn32(y + bv[e]);
                    y = rn32(y * a.alpha);
                    if constexpr (BETA) y = rn32(y + rn32(a.beta * float_of(old[e])));
                    o[e] = bits_of(y);
                }
                __builtin_amdgcn_raw_buffer_store_b128(o, yrsrc, off, 32 * im * N * 4, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
    };
    // Row block by row block: each one's results are stored before the next
    // one's butterflies, which bounds the live values.
    const bool use_beta = a.beta != 0.0f;
    auto emit_any = [&](auto imc, const float (&v)[TN][16]) {
        if (use_beta) emit(imc, v, std::true_type{});
        else emit(imc, v, std::false_type{});
    };
    float v[TN][16];
    constexpr std::integral_constant<int, 0> first{};
    h128(first, v);
    __builtin_amdgcn_s_waitcnt(0);   // this wave's svh / bias DMA landed
    __syncthreads();
    emit_any(first, v);
    if constexpr (TM == 2) {
        constexpr std::integral_constant<int, 1> second{};
        h128(second, v);
        emit_any(second, v);
    }
    clk.record(a, kind, t, s0);
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
