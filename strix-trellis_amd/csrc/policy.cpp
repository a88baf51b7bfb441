// Host-side decomposition policy of every core: GEMV splits and workspace,
// prefill GEMM passes, tile widths, K splits and split-tile handoff, MoE
// splits.  Plain host code (no device code), so the C ABI layer can be built
// and tested against a fake HIP runtime with these same policies.
#include "policy.hpp"

namespace stx {

// Split decomposition.  The whole matrix must be in flight at once for the
// small decode shapes (8 MiB at K4 4096^2 is about one HBM latency-bandwidth
// product), so aim for >= 512 workgroups of 4 waves (measured on MI355X:
// 1024 adds more cross-workgroup fold traffic than it hides, 256 leaves SIMDs
// idle); among candidate splits (bps = 8m with m dividing (I/16)/8, m <= 16)
// take the largest bps that keeps the grid at or above that target, else the
// smallest bps.
GemvShape gemv_shape(uint32_t input, uint32_t output, uint32_t /*bits*/) {
    const uint32_t nb = input / 16, nc = output / 128, units = nb / 8;
    constexpr uint32_t target = 512;
    // When no split count reaches the target (few column groups), 16-block
    // splits are kept while they leave at least 128 workgroups: 8-block ones
    // are dominated by each workgroup's fixed costs (4096 -> 1024 alone: 7.8
    // -> 7.0 us; sixteen of them as the grouped o_a plan: 23.0 -> 20.4 us),
    // while smaller layers (2048 -> 512) need the workgroups more.
    GemvShape best = units % 2 == 0 && uint64_t(nc) * (nb / 16) >= 128 ? GemvShape{16, nb / 16}
                                                                        : GemvShape{8, nb / 8};
    for (uint32_t m = 1; m <= 16; ++m) {
        if (units % m) continue;
        const uint32_t bps = 8 * m, splits = nb / bps;
        if (uint64_t(nc) * splits >= target) best = {bps, splits};
    }
    // A finisher wave polls two rows' other splits per round at five to eight
    // rows, 32 loads at most, so more than 17 splits take a second coherent
    // round trip there, and their planes a longer fold at every row count.
    // Such a pick gives way to the most workgroups among splits of at most 17
    // parts, if they still fill 1.5 per CU, keep at least half the splits and
    // load the busiest CU no more (ceil(W / 256) / W, every workgroup being
    // resident at once and sharing its CU's VALU): 5120^2 (S = 20 -> 10, 800
    // -> 400 workgroups, 4 -> 2 on the busiest CU) measured 1 / 4 / 9 % faster
    // at R1 / R4 / R8 (K4) and 2 / 6 / 10 % (K5).  3072 -> 4096 (768 -> 384,
    // 3 -> 2) would load it more, and measured 4 % slower at R1 (10 % faster
    // at R8): it keeps S = 24.
    if (best.splits > kOneRoundSplits) {
        constexpr uint64_t kCus = 256;
        const uint32_t picked = best.splits;
        const uint64_t w0 = uint64_t(nc) * picked;
        for (uint32_t m = 1; m <= 16; ++m) {
            if (units % m) continue;
            const uint32_t splits = nb / (8 * m);
            const uint64_t w1 = uint64_t(nc) * splits;
            if (splits <= kOneRoundSplits && 2 * splits >= picked && w1 >= kOneRoundMinWorkgroups &&
                (w1 + kCus - 1) / kCus * w0 <= (w0 + kCus - 1) / kCus * w1) {
                best = {8 * m, splits};
                break;
            }
        }
    }
    return best;
}

uint64_t gemv_workspace_bytes(const DeviceWeights& w, uint32_t rows) {
    const GemvShape sh = gemv_shape(w.input, w.output, w.bits);
    if (sh.splits <= 1) return 0;
    return align256(uint64_t(sh.splits) * rows * w.output * sizeof(float));
}

// Single-launch state: [status][epochs: groups * N/128 u32][2 plane sets].
static uint64_t fused_epochs_offset() { return 256; }
uint64_t fused_planes_offset(const DeviceWeights& w, uint32_t groups) {
    return align256(fused_epochs_offset() + uint64_t(groups) * (w.output / 128) * 4);
}

uint64_t fused_state_bytes(const DeviceWeights& w, uint64_t rows, uint32_t groups) {
    const GemvShape sh = gemv_shape(w.input, w.output, w.bits);
    if (sh.splits <= 1 || !rows || !groups) return 0;
    const uint64_t words = 2 * uint64_t(groups) * (sh.splits - 1) * rows * w.output;
    return fused_planes_offset(w, groups) + align256(words * 4);
}

FusedState fused_state_at(void* base, const DeviceWeights& w, uint64_t /*rows*/, uint32_t groups) {
    char* b = static_cast<char*>(base);
    FusedState st;
    st.status = reinterpret_cast<uint32_t*>(b);
    st.epochs = reinterpret_cast<uint32_t*>(b + fused_epochs_offset());
    st.planes = reinterpret_cast<float*>(b + fused_planes_offset(w, groups));
    return st;
}

// Grouped plans: the owner-fold plan runs one 16-wave workgroup per column
// group of every group, so it needs at least one per CU (256) to fill the
// GPU, and then only beats the split plan when each owner's work is short and
// the rows are many (measured on MI355X, both folds, R1/R4/R8):
//   16 x 4096 -> 1024 K5 (128 owners): split  20.1 / 26.4 / 38.4 us, owner 36.7 / 47.7 / 62.7
//   32 x 4096 -> 1024 K5 (256 owners): split  33.9 / 43.9 / 60.5 us, owner 40.5 / 52.7 / 68.6
//   64 x 2048 ->  512 K4 (256 owners): split  21.2 / 28.0 / 37.1 us, owner 22.2 / 28.0 / 37.0
//    8 x 2048 -> 4096 K4 (256 owners): split  21.3 / 27.7 / 37.0 us, owner 21.7 / 27.3 / 35.3
bool grouped_owner_preferred(const DeviceWeights& geometry, uint32_t groups, uint64_t rows) {
    return uint64_t(groups) * (geometry.output / 128) >= 256 && geometry.input <= 2048 && rows >= 4;
}

// Rows per GEMM pass: the fragment buffer of one pass stays below 1 GiB so
// its buffer resource (32-bit range) and the workspace stay bounded.
uint64_t gemm_pass_rows(const DeviceWeights& w) {
    const uint64_t per_row = uint64_t(w.input) * 2;
    uint64_t rows = (uint64_t(1) << 30) / per_row;
    rows -= rows % 256;
    return rows < 256 ? 256 : rows;
}

uint64_t afrag_bytes(const DeviceWeights& w, uint64_t m) {
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
bool wide_can_split(const DeviceWeights& w) { return (w.input / 64) / kWideSplitMinStages >= 2; }
WideSplit wide_split(uint64_t m, const DeviceWeights& w) {
    constexpr uint64_t kCus = 256;
    const uint64_t mb = (m + 255) / 256, nc = w.output / 256, tiles = mb * nc;
    if (2 * tiles <= kCus && (!wide_can_split(w) || 8 * tiles < kCus)) return {0, uint32_t(nc)};
    return {uint32_t(nc), 0};
}

// The wide kernel addresses each 256-row slab of its output (256 x N x 4
// bytes) through one buffer resource, so N stays below 2^22.
bool gemm_wide(uint64_t m, const DeviceWeights& w) {
    return m >= 256 && w.output % 256 == 0 && w.output < (1u << 22);
}

// K split of a wide pass (no handoff) whose workgroups fill at most half of
// the 256 CUs, e.g. M = 256..768 on 5120^2 (20 to 60 tiles): S workgroups per
// tile, as many as one round holds, each over at least eight 64-channel
// stages.  The planes add 2 S M N floats of traffic (written, then folded).
// S depends on the layer and on the number of 256-row blocks, so rows of calls
// in the same class share bits.
uint32_t wide_splits(uint64_t m, const DeviceWeights& w) {
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
uint32_t narrow_splits(const DeviceWeights& w) {
    const uint32_t groups = w.output / 128, stages = w.input / 128;
    uint32_t s = 1;
    while (groups * s < 256 && s < 16 && stages % (2 * s) == 0) s *= 2;
    return s;
}

// K-split handoff of a wide pass with only 256 x 256 tiles: T = 256 q + x
// tiles with 0 < x <= 128 (and T a multiple of the 8 XCDs) launch as x
// heads, 256 q whole tiles and x tails (one workgroup per CU at a time), so
// each CU runs about q + 1/2 tile-times instead of q + 1.
Handoff gemm_handoff(uint64_t m, const DeviceWeights& w) {
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
uint64_t handoff_bytes(uint32_t x) { return uint64_t(x) * 8 * 128 * 64 * sizeof(float); }

// Workspace of one pass of m rows: fragment-order input, then the handoff's
// partial accumulators and flags (wide) or the split planes (narrow).
uint64_t pass_workspace(const DeviceWeights& w, uint64_t m) {
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

MoeSplit moe_split(uint32_t input, uint32_t max_bps) {
    const uint32_t blocks = input / 16;
    uint32_t bps = 8;
    for (uint32_t b = 16; b <= max_bps; b += 8)
        if (blocks % b == 0) bps = b;
    return {bps, blocks / bps};
}

MoeSplit moe_split_staged(uint32_t H) {
    const uint32_t blocks = H / 16;
    if (blocks % 4 == 0) {
        const uint32_t bps = blocks / 4;
        bool fits = bps >= 1;
        for (uint32_t s = 0; s < 4; ++s) fits = fits && moe_down_groups(bps, s) <= uint32_t(MOE_D_MAX_BPS) / 8;
        if (fits) return {bps, 4};
    }
    return moe_split(H, MOE_D_MAX_BPS);
}

uint64_t moe_gate_up_partial_floats(uint32_t routes, uint32_t I, uint32_t H) {
    return uint64_t(routes) * moe_split(I, MOE_GU_MAX_BPS).splits * 2 * H;
}

uint64_t moe_down_partial_floats(uint32_t routes, uint32_t I, uint32_t H) {
    return uint64_t(routes) * moe_split(H, MOE_D_MAX_BPS).splits * I;
}

uint64_t moe_partial_floats(uint32_t routes, uint32_t I, uint32_t H) {
    return moe_gate_up_partial_floats(routes, I, H) + moe_down_partial_floats(routes, I, H);
}

uint64_t moe_counter_words(uint32_t rows, uint32_t routes, uint32_t I, uint32_t H) {
    return uint64_t(routes) * (H / 128) + uint64_t(rows) * (I / 128);
}

// Shapes of the streaming-read kernel (launch_stream_read): the kernel is
// instantiated for these thread counts and loads in flight per lane.
bool stream_read_shape_ok(uint32_t threads, uint32_t depth) {
    const bool t = threads == 64 || threads == 128 || threads == 256 || threads == 512 || threads == 1024;
    const bool d = depth == 1 || depth == 2 || depth == 4 || depth == 8 || depth == 16;
    return t && d;
}

}  // namespace stx
