// Host side of the prefill GEMM (launches; the pass, tile-width, K-split and
// handoff policy is in policy.cpp) and the fragment-order input stage.
#include "gemm_wide.hpp"
#include "policy.hpp"

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
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
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

#if STX_STAGE_CLOCK
// Instrumented build only (build.py --stage-clock): where the wide kernel
// writes its per-wave phase cycle records; null writes none.
static unsigned long long* g_stage_clock = nullptr;
extern "C" int strix_amd_debug_stage_clock(void* records) {
    g_stage_clock = static_cast<unsigned long long*>(records);
    return 0;
}
#endif

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
#if STX_STAGE_CLOCK
        l.args.clock = g_stage_clock;
#endif
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
