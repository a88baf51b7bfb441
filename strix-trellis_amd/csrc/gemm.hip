// Host side of the prefill GEMM and the fragment-order input stage.
#include "gemm_wide.hpp"

namespace stx {

// Input stage of RB rows x 128 channels into MFMA A-fragment order: RB = 16
// for the 16x32 fragments of gemm_kernel, RB = 32 for the 32x16 fragments of
// gemm_wide_kernel.  Each wave stages RB / 4 rows (one 128-block each) into an
// LDS tile; then every thread writes whole fragment lanes -- 8 consecutive
// channels of one row, 16 contiguous bytes -- so each fragment (64 lanes x
// 16 B) is one coalesced 1 KiB store.  Rows past M are zero.
// Workgroup (0, 0) also clears the wide GEMM's `nflags` handoff flags.
template <int RB>
__global__ __launch_bounds__(256) void input_stage_frag_kernel(const float* x, const uint16_t* suh, uint32_t M,
                                                               uint32_t I, _Float16* afrag, uint32_t* flags,
                                                               uint32_t nflags) {
    __shared__ __align__(16) _Float16 tile[RB][128 + 8];
    const uint32_t blk = blockIdx.x, rb = blockIdx.y;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    if (blk == 0 && rb == 0)
        for (uint32_t i = tid; i < nflags; i += 256) flags[i] = 0;
    const uint32_t ch = blk * 128;
    // All of the wave's row loads are issued before the first row's arithmetic
    // (one memory round trip per wave instead of one per row).
    InputLoad l[RB / 4];
#pragma unroll
    for (int q = 0; q < RB / 4; ++q) {
        const uint32_t row = rb * RB + (RB / 4) * w + q;
        const bool live = row < M;
        l[q] = input_load(x + (live ? uint64_t(row) * I : 0) + ch, suh + ch, live);
    }
#pragma unroll
    for (int q = 0; q < RB / 4; ++q) {
        const int r = (RB / 4) * w + q;
        input_values(l[q], tile[r][lane], tile[r][lane + 64]);
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < RB / 16; ++q) {
        const int fl = tid + 256 * q;
        const int f = fl >> 6, l = fl & 63;        // fragment within the 128 block, its lane
        uint64_t off;
        u32x4 v;
        if constexpr (RB == 16) {
            v = *reinterpret_cast<const u32x4*>(&tile[l & 15][f * 32 + (l >> 4) * 8]);
            off = afrag_offset(rb, blk * 4 + f, I, l);
        } else {
            v = *reinterpret_cast<const u32x4*>(&tile[l & 31][f * 16 + (l >> 5) * 8]);
            off = afrag32_offset(rb, blk * 8 + f, I, l);
        }
        u32x4* dst = reinterpret_cast<u32x4*>(reinterpret_cast<char*>(afrag) + off);
        *(__attribute__((address_space(1))) u32x4*)(dst) = v;
    }
}

// Rows per GEMM pass: the fragment buffer of one pass stays below 1 GiB so
// its buffer resource (32-bit range) and the workspace stay bounded.
static uint64_t gemm_pass_rows(const DeviceWeights& w) {
    const uint64_t per_row = uint64_t(w.input) * 2;
    uint64_t rows = (uint64_t(1) << 30) / per_row;
    rows -= rows % 256;
    return rows < 256 ? 256 : rows;
}

static uint64_t align256(uint64_t v) { return (v + 255) & ~uint64_t(255); }

static uint64_t afrag_bytes(const DeviceWeights& w, uint64_t m) {
    return align256(((m + 31) / 32) * 32 * w.input * 2);   // rows padded for either fragment order
}

// Column split and K split of a wide pass over the 256 CUs (one 512-thread
// workgroup per CU).  `full` 256-column blocks run as 256 x 256 tiles, `half`
// as 256 x 128 tiles, twice the workgroups at half the work each; a 256 x 128
// tile takes ~0.8 of a 256 x 256 tile's time (the stage barrier and the A
// stream do not shrink with it).  A pass whose tiles fill at most half the CUs
// splits K (below), and there the full tiles win once eight splits or fewer
// fill the CUs (tiles >= 32; measured on M = 256..768 of 5120^2 and 4096 ->
// 12288, e.g. M = 512 on 4096 -> 12288: 110 -> 108 us, M = 256: 72 -> 64 us):
// the plane traffic grows with S, so 20 tiles (M = 256 on 5120^2) stay half
// tiles at half the split count.  A layer too short to split takes the half
// tiles whenever all of them fit one wave of workgroups.
struct WideSplit {
    uint32_t full, half;   // 256-column blocks of each width
};
constexpr uint32_t kWideSplitMinStages = 8;   // 64-channel stages per K split, at least
static bool wide_can_split(const DeviceWeights& w) { return (w.input / 64) / kWideSplitMinStages >= 2; }
static WideSplit wide_split(uint64_t m, const DeviceWeights& w) {
    constexpr uint64_t kCus = 256;
    const uint64_t mb = (m + 255) / 256, nc = w.output / 256, tiles = mb * nc;
    if (2 * tiles <= kCus && (!wide_can_split(w) || 8 * tiles < kCus)) return {0, uint32_t(nc)};
    return {uint32_t(nc), 0};
}

static bool gemm_wide(uint64_t m, const DeviceWeights& w) { return m >= 256 && w.output % 256 == 0; }

// K split of a wide pass (no handoff) whose workgroups fill at most half of
// the 256 CUs, e.g. M = 256..768 on 5120^2 (20 to 60 tiles): S workgroups per
// tile, as many as one round holds, each over at least eight 64-channel
// stages.  The planes add 2 S M N floats of traffic (written, then folded).
// S depends on the layer and on the number of 256-row blocks, so rows of calls
// in the same class share bits.
static uint32_t wide_splits(uint64_t m, const DeviceWeights& w) {
    if (!gemm_wide(m, w)) return 1;
    const WideSplit sp = wide_split(m, w);
    const uint64_t wgs = ((m + 255) / 256) * (uint64_t(sp.full) + 2 * uint64_t(sp.half));
    if (2 * wgs > 256) return 1;
    uint64_t s = 256 / wgs;
    const uint64_t cap = (w.input / 64) / kWideSplitMinStages;
    if (s > cap) s = cap;
    return s > 1 ? uint32_t(s) : 1;
}

// K-split of the narrow (M < 256) kernel: N/128 column groups alone leave
// most CUs idle (96 workgroups on 4096 -> 12288, 40 on 5120^2), so the input
// splits in S power-of-two parts until the column groups x S reach the 256
// CUs (S <= 16, whole 128-channel stages per split).  S depends on the layer
// only, so every row of every M < 256 call has the same bits; it is part of
// the core's accumulation order (planes folded in ascending split order from
// +0, as the split GEMV does).
static uint32_t narrow_splits(const DeviceWeights& w) {
    const uint32_t groups = w.output / 128, stages = w.input / 128;
    uint32_t s = 1;
    while (groups * s < 256 && s < 16 && stages % (2 * s) == 0) s *= 2;
    return s;
}

// K-split handoff of a wide pass with only 256 x 256 tiles: T = 256 q + x
// tiles with 0 < x <= 128 (and T a multiple of the 8 XCDs) launch as x
// heads, 256 q whole tiles and x tails (one workgroup per CU at a time), so
// each CU runs about q + 1/2 tile-times instead of q + 1.
struct Handoff {
    uint32_t q = 0, x = 0;
};
static Handoff gemm_handoff(uint64_t m, const DeviceWeights& w) {
    Handoff h;
    if (!gemm_wide(m, w) || w.input / 64 < 2) return h;
    const WideSplit sp = wide_split(m, w);
    if (sp.half) return h;
    const uint64_t tiles = ((m + 255) / 256) * (w.output / 256), rem = tiles % 256;
    if (tiles < 256 || rem == 0 || rem > 128 || tiles % 8) return h;
    h.q = uint32_t(tiles / 256);
    h.x = uint32_t(rem);
    return h;
}
static uint64_t handoff_bytes(uint32_t x) { return uint64_t(x) * 8 * 128 * 64 * sizeof(float); }

// Workspace of one pass of m rows: fragment-order input, then the handoff's
// partial accumulators and flags (wide) or the split planes (narrow).
static uint64_t pass_workspace(const DeviceWeights& w, uint64_t m) {
    if (!gemm_wide(m, w)) {
        const uint32_t s = narrow_splits(w);
        return afrag_bytes(w, m) + (s > 1 ? align256(uint64_t(s) * m * w.output * sizeof(float)) : 0);
    }
    const Handoff h = gemm_handoff(m, w);
    const uint32_t s = wide_splits(m, w);
    return afrag_bytes(w, m) + (h.x ? align256(handoff_bytes(h.x)) + align256(uint64_t(h.x) * 4) : 0) +
           (s > 1 ? align256(uint64_t(s) * m * w.output * sizeof(float)) : 0);
}

uint64_t gemm_workspace_bytes(const DeviceWeights& w, uint64_t rows) {
    const uint64_t pass = gemm_pass_rows(w);
    if (rows <= pass) return pass_workspace(w, rows);
    const uint64_t a = pass_workspace(w, pass), b = rows % pass ? pass_workspace(w, rows % pass) : 0;
    return a > b ? a : b;
}

uint32_t gemm_launch_count(const DeviceWeights& w, uint64_t rows) {
    const uint64_t pass = gemm_pass_rows(w);
    uint32_t n = 0;
    for (uint64_t r0 = 0; r0 < rows; r0 += pass) {
        const uint64_t m = rows - r0 < pass ? rows - r0 : pass;
        n += 2;
        if (!gemm_wide(m, w) && narrow_splits(w) > 1) ++n;   // plane fold
        if (gemm_wide(m, w)) {
            const WideSplit sp = wide_split(m, w);
            n += sp.full && sp.half;
            if (wide_splits(m, w) > 1) ++n;   // plane fold
        }
    }
    return n;
}

uint32_t gemm_split_count(const DeviceWeights& w, uint64_t rows) {
    const uint64_t pass = gemm_pass_rows(w), m = rows < pass ? rows : pass;
    return gemm_wide(m, w) ? wide_splits(m, w) : narrow_splits(w);
}

using GemmDispatch = hipError_t (*)(const GemmLaunch&);
static const GemmDispatch gemm_table[8] = {gemm_dispatch<1>, gemm_dispatch<2>, gemm_dispatch<3>, gemm_dispatch<4>,
                                           gemm_dispatch<5>, gemm_dispatch<6>, gemm_dispatch<7>, gemm_dispatch<8>};
static const GemmDispatch gemm_wide_table[8] = {gemm_wide_dispatch<1>, gemm_wide_dispatch<2>, gemm_wide_dispatch<3>,
                                                gemm_wide_dispatch<4>, gemm_wide_dispatch<5>, gemm_wide_dispatch<6>,
                                                gemm_wide_dispatch<7>, gemm_wide_dispatch<8>};

// Row-block height: 256 halves the decode work per flop; 128 when the rows
// would not fill a 256 block or when 256-row blocks leave most CUs idle.
static uint32_t gemm_bm(uint64_t rows, uint32_t groups) {
    if (rows <= 128) return 128;
    const uint64_t wg256 = uint64_t(groups) * ((rows + 255) / 256);
    return wg256 >= 256 ? 256 : 128;
}

hipError_t launch_gemm(const DeviceWeights& w, const LinearCall& call, hipStream_t stream) {
    if (uint64_t(w.input / 16) * (w.output / 16) * 32u * w.bits >= (uint64_t(1) << 31)) return hipErrorInvalidValue;
    const uint64_t pass = gemm_pass_rows(w);
    _Float16* afrag = static_cast<_Float16*>(call.workspace);
    for (uint64_t r0 = 0; r0 < call.rows; r0 += pass) {
        const uint64_t m = call.rows - r0 < pass ? call.rows - r0 : pass;
        // 256 x 256 tiles (32x16 fragments) once the rows fill them and N
        // splits into 256-column blocks; 128-row tiles (16x32 fragments) otherwise.
        const bool wide = gemm_wide(m, w);
        const uint32_t rb = wide ? 32 : 16;
        const uint64_t mpad = (m + rb - 1) / rb * rb;
        const float* x = call.x + r0 * call.x_row_stride;
        const Handoff h = gemm_handoff(m, w);
        char* hbase = reinterpret_cast<char*>(call.workspace) + afrag_bytes(w, m);
        float* handoff = reinterpret_cast<float*>(hbase);
        uint32_t* flags = reinterpret_cast<uint32_t*>(hbase + align256(handoff_bytes(h.x)));
        if (wide)
            hipLaunchKernelGGL(input_stage_frag_kernel<32>, dim3(w.input / 128, uint32_t(mpad / 32)), dim3(256), 0,
                               stream, x, w.suh, uint32_t(m), w.input, afrag, flags, h.x);
        else
            hipLaunchKernelGGL(input_stage_frag_kernel<16>, dim3(w.input / 128, uint32_t(mpad / 16)), dim3(256), 0,
                               stream, x, w.suh, uint32_t(m), w.input, afrag, flags, 0u);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        GemmLaunch l{};
        l.args.trellis = w.trellis;
        l.args.svh = w.svh;
        l.args.bias = w.bias;
        l.args.afrag = afrag;
        l.args.afrag_bytes = mpad * w.input * 2;
        l.args.y = call.y + r0 * call.y_row_stride;
        l.args.M = uint32_t(m);
        l.args.I = w.input;
        l.args.N = w.output;
        l.args.alpha = call.alpha;
        l.args.beta = call.beta;
        l.args.q = h.q;
        l.args.x = h.x;
        l.args.handoff = h.x ? handoff : nullptr;
        l.args.flags = h.x ? flags : nullptr;
        l.args.poll_limit = call.handoff_poll_limit;
        l.args.splits = wide ? wide_splits(m, w) : narrow_splits(w);
        l.args.planes = reinterpret_cast<float*>(hbase);   // a split pass has no handoff
        l.codebook = w.codebook;
        l.bm = gemm_bm(m, w.output / 128);
        l.stream = stream;
        auto fold_planes = [&]() -> hipError_t {
            if (l.args.splits == 1) return hipSuccess;
            LinearCall pc = call;
            pc.rows = m;
            pc.y = l.args.y;
            pc.y_row_stride = w.output;
            return launch_plane_finish(w, pc, l.args.planes, l.args.splits, stream);
        };
        if (!wide) {
            e = gemm_table[w.bits - 1](l);
            if (e != hipSuccess) return e;
            e = fold_planes();
            if (e != hipSuccess) return e;
            continue;
        }
        const WideSplit sp = wide_split(m, w);
        if (sp.full) {
            l.bn = 256;
            l.col_blocks = sp.full;
            l.args.col_block0 = 0;
            e = gemm_wide_table[w.bits - 1](l);
            if (e != hipSuccess) return e;
        }
        if (sp.half) {
            l.bn = 128;
            l.col_blocks = 2 * sp.half;
            l.args.col_block0 = 2 * sp.full;
            e = gemm_wide_table[w.bits - 1](l);
            if (e != hipSuccess) return e;
        }
        e = fold_planes();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace stx
