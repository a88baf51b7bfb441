// Routed-expert (MoE) kernels for gfx950: grouped gate/up + SwiGLU, and down
// with the ordered score-weighted top-k fold.
//
// Both launches reuse the GEMV building blocks (in-register trellis decode,
// the matrix-core dot, LDS wave fold, coherent partial planes, last-arrival
// finish) with routed rows instead of a fixed row range:
//
//   gate/up : grid (H/128, s_gu, rows*k), 256 threads.  Workgroup (c, s, r)
//             takes the r-th expert group (its leader is the first valid
//             occurrence of the expert in route order).  It gathers the group's
//             non-zero-score token rows of X, streams gate AND up tiles of
//             column group c over input split s and writes both partial
//             planes; the last split to arrive folds them, applies both output
//             stages and SwiGLU and writes hidden[r, slot, 128c .. 128c+127].
//   down    : grid (I/128, s_d, rows*k).  The group leader streams the down
//             tiles once for all its rows (input = hidden of each row) and
//             writes one plane per row; every workgroup of a group then
//             arrives at the counter of each member token.  The last arrival
//             for token r folds each slot's planes in ascending slot order,
//             applies that slot's output stage, weights it by its score and
//             finishes alpha/beta.  Invalid tokens get NaN rows.
//
// Accumulation order per projection (fixes the bits; independent of which
// other tokens are routed to the same expert): over the wave's blocks w,
// w+4, ... in ascending order, four MFMA K steps per block; wave fold 0..3;
// split fold ascending from +0 — the GEMV order of the same split
// decomposition.
#pragma once
#include "moe.hpp"
#include "gemv_kernel.hpp"

namespace stx {

// ---------------------------------------------------------------------------
// Activation.  exp(x) for x <= 0, which is all the stable sigmoid needs:
// Cody–Waite reduction x = n*ln2 + r with |r| <= ln2/2, ln2 split into a head
// with 16 significant bits (n*head is exact for |n| <= 256) and a tail; exp(r)
// by its degree-7 Taylor polynomial in Horner form (truncation below 6e-9
// relative); 2^n applied as two power-of-two factors so that a subnormal
// result is rounded once.  Every step is a single FP32 operation, so a host
// restatement with the same operations gives the same bits.
// ---------------------------------------------------------------------------
constexpr float MOE_LOG2E = 1.44269504088896341f;
constexpr float MOE_LN2_HEAD = 0x1.62e4p-1f;             // 0.693145751953125
constexpr float MOE_LN2_TAIL = 1.42860682030941723e-6f;  // RN32(ln2 - head)
constexpr float MOE_INV_FACT[8] = {1.0f, 1.0f, 1.0f / 2, 1.0f / 6, 1.0f / 24, 1.0f / 120, 1.0f / 720, 1.0f / 5040};

__device__ __forceinline__ float moe_pow2(int k) { return __builtin_bit_cast(float, uint32_t(k + 127) << 23); }

__device__ __forceinline__ float moe_exp_nonpos(float x) {
    if (!(x == x)) return x;
    if (x < -104.0f) return 0.0f;
    const float n = __builtin_rintf(x * MOE_LOG2E);
    const float r = (x - n * MOE_LN2_HEAD) - n * MOE_LN2_TAIL;
    float p = MOE_INV_FACT[7];
#pragma unroll
    for (int k = 6; k >= 0; --k) p = p * r + MOE_INV_FACT[k];
    const int ni = int(n), n1 = ni / 2, n2 = ni - n1;
    return (p * moe_pow2(n1)) * moe_pow2(n2);
}

// SwiGLU of one hidden element: g * sigmoid(g) * u, sigmoid in the stable
// form 1/(1+e^-g) for g >= 0 and e^g/(1+e^g) for g < 0 (reference
// src/tp_moe_activation.hpp:46-60), divisions correctly rounded.
__device__ __forceinline__ float moe_swiglu(float g, float u) {
    const bool neg = g < 0.0f;
    const float ex = moe_exp_nonpos(neg ? g : -g);
    const float den = 1.0f + ex;
    const float sig = neg ? __fdiv_rn(ex, den) : __fdiv_rn(1.0f, den);
    const float act = rn32(g * sig);
    return rn32(act * u);
}

// ---------------------------------------------------------------------------
// Route resolution (wave 0; one lane per route j = r*k + slot, rows*k <= 64).
// ---------------------------------------------------------------------------
// Route index of the i-th set bit of m (i < popcount(m)).
__device__ __forceinline__ uint32_t moe_nth_route(uint64_t m, int i) {
    for (int q = 0; q < i; ++q) m &= m - 1;
    return uint32_t(__builtin_ctzll(m));
}

// Every field is wave-uniform.
struct MoeGroup {
    uint64_t members;   // valid routes selecting this group's expert
    uint64_t active;    // members with a non-zero score
    uint32_t expert;
    uint32_t route;     // the group's leader route
    bool leader;        // this workgroup has a group (rank < number of groups)
    int nan_row;        // else: the invalid token whose NaN rows it writes, or -1
};

// The routes of all tokens, one lane per route j = r*k + slot (one wave): the
// lane's bank index, and as wave-wide masks the routes of valid tokens and the
// routes with a non-zero score.  A token is valid when each of its ids is in
// the bank and distinct from its other ids, and each score is finite and >= 0.
struct MoeRoutes {
    uint32_t id;
    float score;
    uint64_t valid, nonzero;
};
__device__ __forceinline__ MoeRoutes moe_routes(const MoeArgs& a) {
    const int lane = threadIdx.x & 63;
    const uint32_t k = a.topk, n = a.rows * k;
    const bool live = uint32_t(lane) < n;
    const uint32_t id = ld_global(a.ids + (live ? lane : 0));
    const float sc = ld_global(a.scores + (live ? lane : 0));
    const uint32_t row = uint32_t(lane) / k, slot = uint32_t(lane) - row * k;
    bool ok = live && id < a.bank_count && __builtin_isfinite(sc) && sc >= 0.0f;
#pragma unroll
    for (uint32_t q = 0; q < MOE_MAX_TOPK; ++q) {
        const uint32_t src = q < k ? row * k + q : uint32_t(lane);
        const uint32_t other = __shfl(id, int(src & 63), 64);
        if (q < k && q != slot && other == id) ok = false;
    }
    const uint64_t bad = __ballot(live && !ok);
    const uint64_t row_bits = live ? ((1ull << k) - 1) << (row * k) : 0;   // k <= 8, row*k + k <= 64
    const bool tv = live && (bad & row_bits) == 0;
    return {id, sc, __ballot(tv), __ballot(live && sc != 0.0f)};
}

// Every route's bank index and score (word j and MOE_MAX_ROUTES + j of
// `words`, LDS), written by the wave that resolved them, so that a later
// token finish in the same workgroup reads them without a memory round trip.
__device__ __forceinline__ void moe_keep_routes(const MoeRoutes& rt, uint32_t* words) {
    const int lane = threadIdx.x & 63;
    words[lane] = rt.id;
    words[MOE_MAX_ROUTES + lane] = __builtin_bit_cast(uint32_t, rt.score);
}

// Workgroup rank r (grid z, the slowest dimension) takes the r-th expert group
// in route order: the group led by the r-th leader, a leader being the first
// route of a valid token to select its expert.  So the workgroups with work
// form one prefix of the grid over all column groups and splits, dispatched
// first and spread evenly over the CUs, instead of sitting wherever their
// routes happen to lead.  Ranks past the groups take the
// invalid tokens in order (there are at least as many: an invalid token's k
// routes lead nothing).  One lane per route, in one wave (moe_group_shared).
//
// A route leads its group when no lower valid route selects the same expert.
// The leaders come from a table of each expert's first valid route (an LDS
// minimum over the valid lanes), so the resolution costs the same for every
// rank; the r-th leader in route order is the r-th set bit of their ballot.
// `table` is MOE_MAX_BANK words of LDS that nothing else uses meanwhile.
__device__ __forceinline__ MoeGroup moe_resolve(const MoeArgs& a, uint32_t rank, uint32_t* table,
                                                uint32_t* keep = nullptr) {
    const int lane = threadIdx.x & 63;
    const uint32_t k = a.topk, n = a.rows * k;
    const bool live = uint32_t(lane) < n;
    const uint32_t slot = uint32_t(lane) % k;
    const MoeRoutes rt = moe_routes(a);
    if (keep) moe_keep_routes(rt, keep);
    const uint32_t id = rt.id;
    const bool tv = (rt.valid >> lane) & 1;   // valid implies id < bank_count <= MOE_MAX_BANK
    for (uint32_t i = uint32_t(lane); i < a.bank_count; i += 64) table[i] = ~0u;
    __builtin_amdgcn_wave_barrier();   // lanes exchange through the table: keep the three steps in order
    if (tv) __hip_atomic_fetch_min(table + id, uint32_t(lane), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __builtin_amdgcn_wave_barrier();
    const bool leads = tv && __hip_atomic_load(table + id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) ==
                                 uint32_t(lane);
    const uint64_t leaders = __ballot(leads);
    const uint32_t groups = uint32_t(__builtin_popcountll(leaders));
    if (rank < groups) {
        const uint32_t lead = moe_nth_route(leaders, int(rank));
        const uint32_t e = uint32_t(__builtin_amdgcn_readlane(int(id), int(lead)));
        const uint64_t members = __ballot(id == e) & rt.valid;
        return {members, members & rt.nonzero, e, lead, true, -1};
    }
    // Invalid tokens: slot 0 of each row whose routes are not valid.
    const uint64_t firsts = __ballot(live && slot == 0 && !tv);
    int nan_row = -1;
    if (rank - groups < uint32_t(__builtin_popcountll(firsts)))
        nan_row = int(moe_nth_route(firsts, int(rank - groups)) / k);
    return {0, 0, 0, 0, false, nan_row};
}

// Route-alone resolution (the reference-core down): workgroup rank j takes
// route j by itself when its token is valid and its score non-zero, else
// nothing.  Each route then streams its expert's weights on its own, with the
// one-row core a grouped route also runs, so its planes must come out the same.
__device__ __forceinline__ MoeGroup moe_resolve_route(const MoeArgs& a, uint32_t j) {
    const MoeRoutes rt = moe_routes(a);
    const uint64_t bit = 1ull << (j & 63);   // j < rows * k <= 64
    const bool live = j < a.rows * a.topk && (rt.valid & rt.nonzero & bit) != 0;
    const uint32_t e = uint32_t(__builtin_amdgcn_readlane(int(rt.id), int(j & 63)));
    return {live ? bit : 0, live ? bit : 0, e, j, live, -1};
}

// The group with every field read from the first lane: the values are uniform
// already, but the compiler cannot prove it through the resolution loop, and
// without this the expert's buffer descriptors would sit in VGPRs and every
// weight load would run a per-lane descriptor loop.
__device__ __forceinline__ uint32_t moe_first(uint32_t v) { return uint32_t(__builtin_amdgcn_readfirstlane(int(v))); }
__device__ __forceinline__ uint64_t moe_first(uint64_t v) {
    return uint64_t(moe_first(uint32_t(v))) | (uint64_t(moe_first(uint32_t(v >> 32))) << 32);
}
// A weight base pointer read from the bank (a vector load) as a uniform value.
__device__ __forceinline__ const char* moe_first_ptr(const uint32_t* p) {
    return reinterpret_cast<const char*>(moe_first(uint64_t(reinterpret_cast<uintptr_t>(p))));
}
__device__ __forceinline__ MoeGroup moe_uniform(const MoeGroup& g) {
    return {moe_first(g.members), moe_first(g.active), moe_first(g.expert), moe_first(g.route),
            moe_first(uint32_t(g.leader)) != 0, int(moe_first(uint32_t(g.nan_row)))};
}

// The group of the workgroup (rank = grid z): wave 0 resolves it and shares
// it through LDS (`slot`, 8 words), one barrier instead of four resolutions,
// each a few hundred issue slots of a CU that the decode keeps busy.  With
// `alone` (uniform) rank j is route j by itself (moe_resolve_route).  `table`
// (MOE_MAX_BANK words) is LDS that the workgroup uses only after the barrier;
// `keep` (2 x MOE_MAX_ROUTES words of LDS, or null) receives every route's bank
// index and score (moe_keep_routes).
__device__ __forceinline__ MoeGroup moe_group_shared(const MoeArgs& a, uint32_t rank, uint32_t* slot,
                                                     uint32_t* table, bool alone = false, uint32_t* keep = nullptr) {
    if (threadIdx.x < 64) {
        const MoeGroup g = moe_uniform(alone ? moe_resolve_route(a, rank) : moe_resolve(a, rank, table, keep));
        if (threadIdx.x == 0) {
            slot[0] = uint32_t(g.members);
            slot[1] = uint32_t(g.members >> 32);
            slot[2] = uint32_t(g.active);
            slot[3] = uint32_t(g.active >> 32);
            slot[4] = g.expert;
            slot[5] = g.route;
            slot[6] = uint32_t(g.leader);
            slot[7] = uint32_t(g.nan_row);
        }
    }
    __syncthreads();
    const volatile uint32_t* v = slot;
    const MoeGroup g = {uint64_t(v[0]) | (uint64_t(v[1]) << 32), uint64_t(v[2]) | (uint64_t(v[3]) << 32), v[4], v[5],
                        v[6] != 0, int(v[7])};
    return moe_uniform(g);
}

// Fold `splits` planes of two sets p and q (stride between splits `step`
// floats) at +0 and +64, each from +0 in ascending split order; the loads of
// both sets are issued together, eight splits at a time.
__device__ __forceinline__ void moe_fold2(const float* p, const float* q, uint32_t splits, uint64_t step, float& p0,
                                          float& p1, float& q0, float& q1) {
    const int lane = threadIdx.x & 63;
    p0 = p1 = q0 = q1 = 0.0f;
    uint32_t s = 0;
    for (; s + 8 <= splits; s += 8) {
        float v[4][8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            v[0][u] = load_coherent(p + (s + u) * step + lane);
            v[1][u] = load_coherent(p + (s + u) * step + lane + 64);
            v[2][u] = load_coherent(q + (s + u) * step + lane);
            v[3][u] = load_coherent(q + (s + u) * step + lane + 64);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            p0 = p0 + v[0][u];
            p1 = p1 + v[1][u];
            q0 = q0 + v[2][u];
            q1 = q1 + v[3][u];
        }
    }
    for (; s < splits; ++s) {
        const float a0 = load_coherent(p + s * step + lane), a1 = load_coherent(p + s * step + lane + 64);
        const float b0 = load_coherent(q + s * step + lane), b1 = load_coherent(q + s * step + lane + 64);
        p0 = p0 + a0;
        p1 = p1 + a1;
        q0 = q0 + b0;
        q1 = q1 + b1;
    }
}

// A 64-bit value of lane l (uniform l) as a uniform value.
__device__ __forceinline__ uint64_t moe_lane64(uint64_t v, int l) {
    return uint64_t(uint32_t(__builtin_amdgcn_readlane(int(uint32_t(v)), l))) |
           (uint64_t(uint32_t(__builtin_amdgcn_readlane(int(uint32_t(v >> 32)), l))) << 32);
}

// Every store of this workgroup is complete before any of its threads goes on
// to arrive at a counter.
__device__ __forceinline__ void moe_release() {
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
}

constexpr int MOE_MAX_RT = 8;
// Chunk loads in flight per wave and projection.  With five to seven
// workgroups per CU the CU has enough bytes in flight without deep rings, and
// the later workgroups' first loads queue behind fewer of the earlier ones':
// interleaved A/B on C5, same bits, gate/up 4 -> 3 with down 8 -> 4 measured
// 1.3-1.6 % faster over two rounds (down 6 and gate/up 3 alone less or none).
constexpr int MOE_RING_GU = 3;
constexpr int MOE_RING_D = 4;
// LDS: the FP16 activations live until the main loop ends, the wave partials
// only after it, so both share one buffer.
constexpr int MOE_GU_ACT_BYTES = 2 * MOE_MAX_RT * MOE_GU_MAX_BPS * 16 * 2;
constexpr int MOE_GU_RED_BYTES = GEMV_WAVES * 2 * MOE_MAX_RT * 128 * 4;
constexpr int MOE_D_ACT_BYTES = MOE_MAX_RT * MOE_D_MAX_BPS * 16 * 2;
constexpr int MOE_D_RED_BYTES = GEMV_WAVES * MOE_MAX_RT * 128 * 4;
static_assert(MOE_GU_ACT_BYTES >= int(MOE_MAX_BANK * 4) && MOE_D_ACT_BYTES >= int(MOE_MAX_BANK * 4),
              "the route resolution's expert table lives in the activation buffer");
constexpr int moe_max(int a, int b) { return a > b ? a : b; }

// Input-stage units of a wave (u = w, w + 4, ...) in batches of MOE_UNITS
// whose loads are in flight together, one memory round trip per batch.
// Units past the end load unit 0 again (valid addresses, result unused).
constexpr int MOE_UNITS = 4;
template <class Load>
__device__ __forceinline__ void moe_batch_load(int u0, int units, InputLoad (&l)[MOE_UNITS], Load load) {
#pragma unroll
    for (int i = 0; i < MOE_UNITS; ++i) {
        const int u = u0 + GEMV_WAVES * i;
        l[i] = load(u < units ? u : 0);
    }
}
// Computes the batch loaded in `pre` (units from w), then the wave's other units.
template <class Load, class Out>
__device__ __forceinline__ void moe_input_stage(int w, int units, const InputLoad (&pre)[MOE_UNITS], Load load,
                                                Out out) {
    auto compute = [&](int u0, const InputLoad (&l)[MOE_UNITS]) {
#pragma unroll
        for (int i = 0; i < MOE_UNITS; ++i) {
            const int u = u0 + GEMV_WAVES * i;
            if (u < units) input_compute(l[i], out(u));
        }
    };
    compute(w, pre);
    for (int u0 = w + MOE_UNITS * GEMV_WAVES; u0 < units; u0 += MOE_UNITS * GEMV_WAVES) {
        InputLoad l[MOE_UNITS];
        moe_batch_load(u0, units, l, load);
        compute(u0, l);
    }
}

// ---------------------------------------------------------------------------
// Gate/up core of one workgroup: NP = 2 projections sharing the routed rows.
// ---------------------------------------------------------------------------
template <int KG, int KU, int RT>
__device__ __forceinline__ void moe_gate_up_core(const MoeArgs& a, const MoeExpert& ex, uint32_t c, uint32_t split,
                                                 uint64_t active, int nrows, _Float16* act, float* red) {
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int jt = lane >> 3, g = lane & 7;
    const uint32_t bps = a.bps_gu, a0 = split * bps;
    const uint32_t act_row = bps * 16;
    constexpr uint32_t tg = 32u * KG, tu = 32u * KU;
    const uint32_t rbg = (a.H >> 4) * tg, rbu = (a.H >> 4) * tu;
    const auto rg = make_rsrc(moe_first_ptr(ex.gate.trellis) + uint64_t(a0) * rbg, bps * rbg);
    const auto ru = make_rsrc(moe_first_ptr(ex.up.trellis) + uint64_t(a0) * rbu, bps * rbu);
    const uint32_t og = (8u * c + jt) * tg + g * 4u * KG, ou = (8u * c + jt) * tu + g * 4u * KU;
    const int nb = int(bps) / GEMV_WAVES;
    constexpr uint32_t kOut = 0x80000000u;
    auto offg = [&](int t) -> uint32_t { return t < nb ? (w + GEMV_WAVES * t) * rbg + og : kOut; };
    auto offu = [&](int t) -> uint32_t { return t < nb ? (w + GEMV_WAVES * t) * rbu + ou : kOut; };

    // Core inputs of the split's channels, computed once per route by
    // moe_input_kernel (every column group of an expert used to recompute
    // them): one 256-byte unit per (projection, row, 128-block), 4 bytes per
    // lane, straight into LDS by DMA, no registers in flight.  Issued before
    // the weight prefetch: vector loads complete in issue order, so loads
    // issued after the chunks would wait for the chunks' HBM round trip.
    // Wave w takes 128-blocks w, w + 4, ... of every row and projection
    // (scalar loops, no divisions).
    const int hblocks = int(bps) / 8;
    const auto ars = make_rsrc(a.a_gu, uint32_t(moe_core_input_bytes(a.rows * a.topk, a.I)));
    uint64_t left = active;
    for (int i = 0; i < nrows; ++i) {   // wave-uniform
        const uint32_t j = uint32_t(__builtin_ctzll(left));
        left &= left - 1;
        for (int p = 0; p < 2; ++p)
            for (int hb = w; hb < hblocks; hb += GEMV_WAVES) {
                const uint32_t src = ((j * 2 + uint32_t(p)) * a.I + a0 * 16 + uint32_t(hb) * 128) * 2;
                _Float16* dst = act + (p * MOE_MAX_RT + i) * act_row + hb * 128;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ars, (__attribute__((address_space(3))) void*)dst, 4,
                                                         uint32_t(lane) * 4u, src, 0, 0);
            }
    }
    __builtin_amdgcn_sched_barrier(0);

    Chunk<KG> cg[MOE_RING_GU];
    Chunk<KU> cu[MOE_RING_GU];
#pragma unroll
    for (int u = 0; u < MOE_RING_GU; ++u) {
        load_chunk(cg[u], rg, offg(u));
        load_chunk(cu[u], ru, offu(u));
    }
    __builtin_amdgcn_sched_barrier(0);
    // The compiler does not see the DMAs' LDS side: wait for them by count
    // (the 2 x MOE_RING_GU chunk loads, one instruction each at K <= 3, were
    // issued after them), then the barrier makes every wave's units visible.
    static_assert(KG <= 3 && KU <= 3, "one load instruction per chunk");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * MOE_RING_GU) : "memory");
    // Rows past nrows stay unused: rows nrows..RT-1 hold stale LDS, their
    // columns of the products are independent of the others, and the fold
    // below reads only rows < nrows.
    __syncthreads();

    MfmaAcc<RT> accg, accu;
    mfma_acc_zero(accg);
    mfma_acc_zero(accu);
    const bool first = g == 0;
    for (int t = 0; t < nb; t += MOE_RING_GU) {
#pragma unroll
        for (int u = 0; u < MOE_RING_GU; ++u) {
            if (t + u < nb) {
                const int blk = w + GEMV_WAVES * (t + u);
                half2_t wq[4][4];
                link_chunk(cg[u], first);
                decode_chunk<KG, CB_MUL1>(cg[u], wq);
                mfma_dot_block<RT>(wq, act + blk * 16, act_row, accg);
                link_chunk(cu[u], first);
                decode_chunk<KU, CB_MUL1>(cu[u], wq);
                mfma_dot_block<RT>(wq, act + MOE_MAX_RT * act_row + blk * 16, act_row, accu);
            }
            load_chunk(cg[u], rg, offg(t + u + MOE_RING_GU));
            load_chunk(cu[u], ru, offu(t + u + MOE_RING_GU));
        }
    }
    __syncthreads();   // every wave is done with act before red overwrites it
    mfma_partials<RT>(accg, red + (w * 2 + 0) * MOE_MAX_RT * 128);
    mfma_partials<RT>(accu, red + (w * 2 + 1) * MOE_MAX_RT * 128);
    __syncthreads();
}

// Waves per SIMD the MoE kernels ask the register allocator for: five
// workgroups per CU where the 2-bit cores fit 96 VGPRs, else four (a 3-bit
// projection would spill at five).
constexpr int moe_waves_per_eu(int bits_sum, int projections) { return bits_sum <= 2 * projections ? 5 : 4; }

// LDS is the one activation / partial buffer and nothing else (32 KiB at the
// largest split), so that five workgroups fit a CU.
template <int KG, int KU>
__global__ __launch_bounds__(GEMV_THREADS) __attribute__((amdgpu_waves_per_eu(moe_waves_per_eu(KG + KU, 2))))
void moe_gate_up_kernel(const uint32_t* ids, const float* scores, const MoeExpert* bank, uint32_t rows_topk,
                        uint32_t bank_count, MoeArgs args) {
    // The route resolution's inputs and the bank come as scalar arguments, so
    // the dispatcher preloads them into SGPRs and the first loads (the routes)
    // wait for no argument load (the rest of MoeArgs is needed after them).
    MoeArgs a = args;
    a.ids = ids;
    a.scores = scores;
    a.bank = bank;
    a.rows = rows_topk & 0xFFFFu;
    a.topk = rows_topk >> 16;
    a.bank_count = bank_count;
    __shared__ __align__(16) unsigned char lds[moe_max(MOE_GU_ACT_BYTES, MOE_GU_RED_BYTES)];
    _Float16* act = reinterpret_cast<_Float16*>(lds);
    float* red = reinterpret_cast<float*>(lds);
    __shared__ uint32_t group_slot[8];
    const uint32_t c = blockIdx.x, split = blockIdx.y;
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const MoeGroup grp = moe_group_shared(a, blockIdx.z, group_slot, reinterpret_cast<uint32_t*>(lds));
    if (!grp.leader || !grp.active) return;
    const uint32_t route = grp.route;
    const uint64_t active = grp.active;
    const int nrows = __builtin_popcountll(active);
    const MoeExpert& ex = a.bank[grp.expert];
    if (nrows <= 1) moe_gate_up_core<KG, KU, 1>(a, ex, c, split, active, nrows, act, red);
    else if (nrows <= 2) moe_gate_up_core<KG, KU, 2>(a, ex, c, split, active, nrows, act, red);
    else if (nrows <= 4) moe_gate_up_core<KG, KU, 4>(a, ex, c, split, active, nrows, act, red);
    else moe_gate_up_core<KG, KU, 8>(a, ex, c, split, active, nrows, act, red);

    // Wave fold in wave order -> planes [route][split][proj][H].
    const uint32_t S = a.s_gu, H = a.H;
    for (int idx = tid; idx < 2 * nrows * 128; idx += GEMV_THREADS) {
        const int n = idx & 127, pr = idx >> 7, p = pr & 1, i = pr >> 1;
        float v = red[((0 * 2 + p) * MOE_MAX_RT + i) * 128 + n];
#pragma unroll
        for (int ww = 1; ww < GEMV_WAVES; ++ww) v = v + red[((ww * 2 + p) * MOE_MAX_RT + i) * 128 + n];
        const uint32_t j = moe_nth_route(active, i);
        store_coherent(a.p_gu + ((uint64_t(j) * S + split) * 2 + p) * H + 128 * c + n, v);
    }
    moe_release();
    // The partials in LDS are consumed: word 0 carries the arrival result.
    uint32_t* counter = a.c_gu + uint64_t(route) * (H >> 7) + c;
    int* last = reinterpret_cast<int*>(lds);
    if (tid == 0) *last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1;
    __syncthreads();
    if (!*last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");

    // Last split: both output stages, SwiGLU, hidden.  The output-stage
    // operands are loaded first, then gate and up planes together, so the
    // finish waits for about one memory round trip.
    const int lane = tid & 63;
    const int n0 = 128 * int(c) + lane, n1 = n0 + 64;
    const uint16_t gv0 = ld_global(ex.gate.svh + n0), gv1 = ld_global(ex.gate.svh + n1);
    const uint16_t uv0 = ld_global(ex.up.svh + n0), uv1 = ld_global(ex.up.svh + n1);
    const bool gb = ex.gate.bias != nullptr, ub = ex.up.bias != nullptr;
    const float gb0 = gb ? ld_global(ex.gate.bias + n0) : 0.0f, gb1 = gb ? ld_global(ex.gate.bias + n1) : 0.0f;
    const float ub0 = ub ? ld_global(ex.up.bias + n0) : 0.0f, ub1 = ub ? ld_global(ex.up.bias + n1) : 0.0f;
    for (int i = w; i < nrows; i += GEMV_WAVES) {
        const uint32_t j = moe_nth_route(active, i);
        const float* pg = a.p_gu + uint64_t(j) * S * 2 * H + 128 * c;
        float g0, g1, u0, u1;
        moe_fold2(pg, pg + H, S, 2ull * H, g0, g1, u0, u1);
        h32_wave(g0, g1);
        h32_wave(u0, u1);
        g0 = output_value(g0, gv0, gb, gb0, 1.0f, 0.0f, nullptr);
        g1 = output_value(g1, gv1, gb, gb1, 1.0f, 0.0f, nullptr);
        u0 = output_value(u0, uv0, ub, ub0, 1.0f, 0.0f, nullptr);
        u1 = output_value(u1, uv1, ub, ub1, 1.0f, 0.0f, nullptr);
        float* hrow = a.hidden + uint64_t(j) * H;
        *(__attribute__((address_space(1))) float*)(hrow + n0) = moe_swiglu(g0, u0);
        *(__attribute__((address_space(1))) float*)(hrow + n1) = moe_swiglu(g1, u1);
    }
    if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Down core of one workgroup (one projection, rows = the group's active routes).
// ---------------------------------------------------------------------------
template <int K, int RT>
__device__ __forceinline__ void moe_down_core(const MoeArgs& a, const MoeExpert& ex, uint32_t c, uint32_t split,
                                              uint64_t active, int nrows, _Float16* act, float* red) {
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int jt = lane >> 3, g = lane & 7;
    // Blocks [a0, a0 + bps) of the input, inside 128-channel groups
    // [g0, g0 + hblocks): the input stage covers whole groups (its Hadamard
    // spans 128 channels) and the dot reads the split's blocks from `lead` on.
    const uint32_t bps = a.bps_d, a0 = split * bps, g0 = a0 / 8, lead = a0 - 8 * g0;
    const int hblocks = int(moe_down_groups(bps, split));
    const uint32_t act_row = uint32_t(hblocks) * 128;
    constexpr uint32_t tb = 32u * K;
    const uint32_t rb = (a.I >> 4) * tb;
    const auto rs = make_rsrc(moe_first_ptr(ex.down.trellis) + uint64_t(a0) * rb, bps * rb);
    const uint32_t lo = (8u * c + jt) * tb + g * 4u * K;
    const int nb = (int(bps) - w + GEMV_WAVES - 1) / GEMV_WAVES;   // blocks w, w + 4, ... of the split
    constexpr uint32_t kOut = 0x80000000u;
    auto off = [&](int t) -> uint32_t { return t < nb ? (w + GEMV_WAVES * t) * rb + lo : kOut; };

    // Input stage of the hidden rows; the first batch of units is loaded
    // ahead of the weight prefetch (see the gate/up core).
    const int units = nrows * hblocks;
    auto unit_load = [&](int u) -> InputLoad {
        const int i = u / hblocks, hb = u - i * hblocks;
        const uint32_t j = moe_nth_route(active, i);
        const uint32_t ch = (g0 + uint32_t(hb)) * 128;
        return input_load(a.hidden + uint64_t(j) * a.H + ch, ex.down.suh + ch, true);
    };
    auto unit_out = [&](int u) -> _Float16* { return act + (u / hblocks) * act_row + (u % hblocks) * 128; };
    InputLoad pre[MOE_UNITS];
    moe_batch_load(w, units, pre, unit_load);
    __builtin_amdgcn_sched_barrier(0);

    Chunk<K> ring[MOE_RING_D];
#pragma unroll
    for (int u = 0; u < MOE_RING_D; ++u) load_chunk(ring[u], rs, off(u));

    moe_input_stage(w, units, pre, unit_load, unit_out);
    __syncthreads();

    MfmaAcc<RT> acc;
    mfma_acc_zero(acc);
    const bool first = g == 0;
    for (int t = 0; t < nb; t += MOE_RING_D) {
#pragma unroll
        for (int u = 0; u < MOE_RING_D; ++u) {
            if (t + u < nb) {
                half2_t wq[4][4];
                link_chunk(ring[u], first);
                decode_chunk<K, CB_MUL1>(ring[u], wq);
                mfma_dot_block<RT>(wq, act + (lead + w + GEMV_WAVES * (t + u)) * 16, act_row, acc);
            }
            load_chunk(ring[u], rs, off(t + u + MOE_RING_D));
        }
    }
    __syncthreads();   // every wave is done with act before red overwrites it
    mfma_partials<RT>(acc, red + w * MOE_MAX_RT * 128);
    __syncthreads();
}

// Ordered finish of token r over column group c, by one wave (lane 0..63
// holds columns 128c + lane and +64): each slot's planes p_d summed from +0 in
// ascending split order, its output stage, RN32(score * value) added in
// ascending slot order from +0, then alpha/beta.  Lane s fetches slot s's
// score and expert; then the output-stage operands of every slot and the
// planes of every slot are loaded together, so a token waits for about three
// memory round trips however many slots it has.  A zero-score slot loads
// nothing of its expert and adds no term.  Used by the fused down's last
// arrival and by the staged finish, so both give the same bits.  `routes` is
// every route's bank index and score in LDS (moe_keep_routes).
__device__ __forceinline__ void moe_finish_token(const MoeArgs& a, uint32_t r, uint32_t c, int lane,
                                                 const uint32_t* routes) {
    const uint32_t k = a.topk, I = a.I, S = a.s_d;
    const int n0 = 128 * int(c) + lane, n1 = n0 + 64;
    const uint32_t jl = r * k + (uint32_t(lane) < k ? uint32_t(lane) : 0u);
    const float sc_l = __builtin_bit_cast(float, routes[MOE_MAX_ROUTES + jl]);
    const MoeExpert& el = a.bank[routes[jl]];
    const uint64_t svh_l = reinterpret_cast<uintptr_t>(el.down.svh);
    const uint64_t bias_l = reinterpret_cast<uintptr_t>(el.down.bias);
    float sc[MOE_MAX_TOPK], z0[MOE_MAX_TOPK], z1[MOE_MAX_TOPK], b0[MOE_MAX_TOPK], b1[MOE_MAX_TOPK];
    uint16_t v0[MOE_MAX_TOPK], v1[MOE_MAX_TOPK];
    bool hb[MOE_MAX_TOPK];
#pragma unroll
    for (int s = 0; s < int(MOE_MAX_TOPK); ++s) {
        const int sl = uint32_t(s) < k ? s : 0;
        sc[s] = uint32_t(s) < k ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc_l), sl))
                                : 0.0f;
        v0[s] = v1[s] = 0;
        b0[s] = b1[s] = 0.0f;
        hb[s] = false;
        z0[s] = z1[s] = 0.0f;
        if (sc[s] != 0.0f) {
            const auto* svh = reinterpret_cast<const uint16_t*>(moe_lane64(svh_l, sl));
            const auto* bias = reinterpret_cast<const float*>(moe_lane64(bias_l, sl));
            v0[s] = ld_global(svh + n0);
            v1[s] = ld_global(svh + n1);
            hb[s] = bias != nullptr;
            if (hb[s]) {
                b0[s] = ld_global(bias + n0);
                b1[s] = ld_global(bias + n1);
            }
        }
    }
    // Each slot's planes from +0 in ascending split order, all slots per split.
    for (uint32_t u = 0; u < S; ++u) {
        float p0[MOE_MAX_TOPK], p1[MOE_MAX_TOPK];
#pragma unroll
        for (int s = 0; s < int(MOE_MAX_TOPK); ++s) {
            const uint32_t j = r * k + (uint32_t(s) < k ? uint32_t(s) : 0u);
            const float* p = a.p_d + (uint64_t(j) * S + u) * I + 128 * c;
            p0[s] = load_coherent(p + lane);
            p1[s] = load_coherent(p + lane + 64);
        }
#pragma unroll
        for (int s = 0; s < int(MOE_MAX_TOPK); ++s) {
            z0[s] = z0[s] + p0[s];
            z1[s] = z1[s] + p1[s];
        }
    }
    float comb0 = 0.0f, comb1 = 0.0f;
#pragma unroll
    for (int s = 0; s < int(MOE_MAX_TOPK); ++s) {
        if (sc[s] == 0.0f) continue;   // also every s >= k
        h32_wave(z0[s], z1[s]);
        const float y0 = output_value(z0[s], v0[s], hb[s], b0[s], 1.0f, 0.0f, nullptr);
        const float y1 = output_value(z1[s], v1[s], hb[s], b1[s], 1.0f, 0.0f, nullptr);
        comb0 = rn32(comb0 + rn32(sc[s] * y0));
        comb1 = rn32(comb1 + rn32(sc[s] * y1));
    }
    float* yr = a.y + uint64_t(r) * a.y_stride;
    float o0 = rn32(a.alpha * comb0), o1 = rn32(a.alpha * comb1);
    if (a.beta != 0.0f) {
        o0 = rn32(o0 + rn32(a.beta * ld_global(yr + n0)));
        o1 = rn32(o1 + rn32(a.beta * ld_global(yr + n1)));
    }
    *(__attribute__((address_space(1))) float*)(yr + n0) = o0;
    *(__attribute__((address_space(1))) float*)(yr + n1) = o1;
}

template <int K>
__global__ __launch_bounds__(GEMV_THREADS) __attribute__((amdgpu_waves_per_eu(moe_waves_per_eu(K, 1))))
void moe_down_kernel(const uint32_t* ids, const float* scores, const MoeExpert* bank, uint32_t rows_topk,
                     uint32_t bank_count, MoeArgs args) {
    // Preloaded resolution inputs, as in the gate/up kernel.
    MoeArgs a = args;
    a.ids = ids;
    a.scores = scores;
    a.bank = bank;
    a.rows = rows_topk & 0xFFFFu;
    a.topk = rows_topk >> 16;
    a.bank_count = bank_count;
    __shared__ __align__(16) unsigned char lds[moe_max(MOE_D_ACT_BYTES, MOE_D_RED_BYTES)];
    _Float16* act = reinterpret_cast<_Float16*>(lds);
    float* red = reinterpret_cast<float*>(lds);
    __shared__ uint32_t finish_mask;
    const uint32_t c = blockIdx.x, split = blockIdx.y;
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const uint32_t k = a.topk, I = a.I, S = a.s_d;
    __shared__ uint32_t group_slot[8];
    const bool staged = a.down_mode != kMoeDownFused;   // a kernel argument: uniform
    __shared__ uint32_t route_words[2 * MOE_MAX_ROUTES];
    const MoeGroup grp = moe_group_shared(a, blockIdx.z, group_slot, reinterpret_cast<uint32_t*>(lds),
                                          a.down_mode == kMoeDownRouteCore, route_words);
    if (!grp.leader) {
        // One workgroup per (invalid token, column group) writes its NaN row block.
        if (!staged && grp.nan_row >= 0 && split == 0 && tid < 128)
            a.y[uint64_t(grp.nan_row) * a.y_stride + 128 * c + tid] = __builtin_bit_cast(float, 0x7fc00000u);
        return;
    }
    const uint64_t active = grp.active, members = grp.members;
    const int nrows = __builtin_popcountll(active);
    const MoeExpert& ex = a.bank[grp.expert];
    if (nrows) {
        if (nrows <= 1) moe_down_core<K, 1>(a, ex, c, split, active, nrows, act, red);
        else if (nrows <= 2) moe_down_core<K, 2>(a, ex, c, split, active, nrows, act, red);
        else if (nrows <= 4) moe_down_core<K, 4>(a, ex, c, split, active, nrows, act, red);
        else moe_down_core<K, 8>(a, ex, c, split, active, nrows, act, red);
        for (int idx = tid; idx < nrows * 128; idx += GEMV_THREADS) {
            const int n = idx & 127, i = idx >> 7;
            float v = red[(0 * MOE_MAX_RT + i) * 128 + n];
#pragma unroll
            for (int ww = 1; ww < GEMV_WAVES; ++ww) v = v + red[(ww * MOE_MAX_RT + i) * 128 + n];
            const uint32_t j = moe_nth_route(active, i);
            store_coherent(a.p_d + (uint64_t(j) * S + split) * I + 128 * c + n, v);
        }
    }
    if (staged) return;   // the planes are the staged core's result
    moe_release();
    // One arrival per member route (one route per token), lanes in parallel.
    const uint32_t expected = k * S;
    if (w == 0) {
        const int nm = __builtin_popcountll(members);
        bool fin = false;
        uint32_t r = 0;
        if (lane < nm) {
            r = moe_nth_route(members, lane) / k;
            uint32_t* counter = a.c_d + uint64_t(r) * (I >> 7) + c;
            fin = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == expected - 1;
        }
        const uint64_t fins = __ballot(fin);
        uint32_t mask = 0;
        for (uint64_t m = fins; m; m &= m - 1) mask |= 1u << __shfl(int(r), __builtin_ctzll(m), 64);
        if (lane == 0) finish_mask = mask;
    }
    __syncthreads();
    const uint32_t fm = finish_mask;
    if (!fm) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");

    // Tokens whose last arrival this was, one per wave (moe_finish_token).
    int q = 0;
    for (uint32_t m = fm; m; m &= m - 1, ++q) {
        if (q % GEMV_WAVES != w) continue;
        const uint32_t r = uint32_t(__builtin_ctz(m));
        moe_finish_token(a, r, c, lane, route_words);
        if (lane == 0) __hip_atomic_store(a.c_d + uint64_t(r) * (I >> 7) + c, 0u, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
    }
}

#define STX_INSTANTIATE_MOE(KG)                                                                                   \
    template <>                                                                                                   \
    hipError_t moe_gate_up_dispatch<KG>(const MoeArgs& a, hipStream_t s) {                                        \
        const dim3 grid(a.H / 128, a.s_gu, a.rows * a.topk);                                                      \
        const uint32_t rk = a.rows | (a.topk << 16);                                                              \
        if (a.up_bits == 2)                                                                                       \
            hipLaunchKernelGGL((moe_gate_up_kernel<KG, 2>), grid, dim3(GEMV_THREADS), 0, s, a.ids, a.scores,       \
                               a.bank, rk, a.bank_count, a);                                                      \
        else                                                                                                      \
            hipLaunchKernelGGL((moe_gate_up_kernel<KG, 3>), grid, dim3(GEMV_THREADS), 0, s, a.ids, a.scores,       \
                               a.bank, rk, a.bank_count, a);                                                      \
        return hipGetLastError();                                                                                 \
    }                                                                                                             \
    template <>                                                                                                   \
    hipError_t moe_down_dispatch<KG>(const MoeArgs& a, hipStream_t s) {                                           \
        hipLaunchKernelGGL(moe_down_kernel<KG>, dim3(a.I / 128, a.s_d, a.rows * a.topk), dim3(GEMV_THREADS), 0, s, \
                           a.ids, a.scores, a.bank, a.rows | (a.topk << 16), a.bank_count, a);                    \
        return hipGetLastError();                                                                                 \
    }

template <int KG>
hipError_t moe_gate_up_dispatch(const MoeArgs& a, hipStream_t s);
template <int K>
hipError_t moe_down_dispatch(const MoeArgs& a, hipStream_t s);

}  // namespace stx
