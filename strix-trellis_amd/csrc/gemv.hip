// Host side of the decode GEMV: launches (the split decomposition and
// workspace sizes are in policy.cpp); plus the finishing kernels and the
// diagnostic stage kernels.
#include "gemv_kernel.hpp"

namespace stx {

// Row template of a call: rows are computed in groups of 1, 2, 4 or 8 (the
// rows past the call's are zero inputs whose results are never stored).  A
// row's arithmetic does not depend on the template.  Measured against
// templates of their own: three rows run 2.6-7 % faster on the 4-row one
// (C1 neutral), five and six rows 0.4-2.9 % faster on the 8-row one (one cell
// +0.1 %).  The owner-fold kernel keeps 3- and 6-row templates (its 8-row
// instance: 42.2-42.5 us at 7-8 rows of 16 x 4096 -> 1024 K5 against 40.1 us
// for the 6-row one at 5-6).
static uint32_t rows_template(uint64_t rows) { return rows <= 2 ? uint32_t(rows ? rows : 1) : rows <= 4 ? 4 : 8; }
static uint32_t owner_rows_template(uint64_t rows) {
    return rows == 3 ? 3 : rows == 5 || rows == 6 ? 6 : rows_template(rows);
}

using GemvDispatch = hipError_t (*)(const GemvLaunch&);
static const GemvDispatch gemv_table[8] = {gemv_dispatch<1>, gemv_dispatch<2>, gemv_dispatch<3>,
                                           gemv_dispatch<4>, gemv_dispatch<5>, gemv_dispatch<6>,
                                           gemv_dispatch<7>, gemv_dispatch<8>};

__global__ __launch_bounds__(GEMV_THREADS) void gemv_finish_kernel(GemvArgs a) {
    const int c = blockIdx.x, z = blockIdx.z;
    const GroupWeights gw = group_weights(a, z);
    float* y = a.y + z * a.y_group_stride;
    const float* plane_base = a.partials + (uint64_t(z) * a.splits) * a.rows * a.N;
    finish_columns(a, gw, column_operands(gw, c, a.N), y, c, a.splits, [&](int s, int r) -> const float* {
        return plane_base + (uint64_t(s) * a.rows + r) * a.N + 128 * c;
    });
}

// Fold of the prefill GEMM's K-split planes [S][rows][N] (written by the
// previous launch) and the output stage: grid (N/128, ceil(rows/16)), each
// wave four rows.  Per batch of four splits the wave issues all 32 plane loads
// before the first add, and the four rows' H32 butterflies are interleaved;
// every row is still folded from +0 in ascending split order, so its bits are
// those of the one-row-per-wave fold.
constexpr uint32_t kPlaneRowsPerWave = 4;
__global__ __launch_bounds__(GEMV_THREADS) void plane_finish_kernel(GemvArgs a) {
    const int c = blockIdx.x, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const uint32_t r0 = (blockIdx.y * GEMV_WAVES + w) * kPlaneRowsPerWave;
    if (r0 >= a.rows) return;
    const ColumnOperands op = column_operands(a.w, c, a.N);
    constexpr int P = int(kPlaneRowsPerWave);
    float z0[P], z1[P];
#pragma unroll
    for (int i = 0; i < P; ++i) z0[i] = z1[i] = 0.0f;
    const float* base = a.partials + 128 * c + lane;
    for (uint32_t s = 0; s < a.splits; s += 4) {
        float v0[4][P], v1[4][P];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int i = 0; i < P; ++i) {
                // Past the last split or row: a valid address again, unused.
                const uint32_t ss = s + u < a.splits ? s + u : s;
                const uint32_t r = r0 + i < a.rows ? r0 + i : r0;
                const float* p = base + (uint64_t(ss) * a.rows + r) * a.N;
                v0[u][i] = p[0];
                v1[u][i] = p[64];
            }
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (s + u < a.splits)
#pragma unroll
                for (int i = 0; i < P; ++i) {
                    z0[i] = z0[i] + v0[u][i];
                    z1[i] = z1[i] + v1[u][i];
                }
    }
    h32_wave_multi<P>(z0, z1);
    const int n0 = 128 * c + lane, n1 = n0 + 64;
    const bool has_bias = a.w.bias != nullptr;
#pragma unroll
    for (int i = 0; i < P; ++i) {
        if (r0 + i >= a.rows) break;
        float* yr = a.y + (r0 + i) * a.y_row_stride;
        const float o0 = output_value(z0[i], op.sv0, has_bias, op.b0, a.alpha, a.beta, yr + n0);
        const float o1 = output_value(z1[i], op.sv1, has_bias, op.b1, a.alpha, a.beta, yr + n1);
        *(__attribute__((address_space(1))) float*)(yr + n0) = o0;
        *(__attribute__((address_space(1))) float*)(yr + n1) = o1;
    }
}

static GemvLaunch make_launch(const DeviceWeights& w, const GroupWeights* table, uint32_t groups,
                              const LinearCall& call, uint64_t xg, uint64_t yg, float* planes,
                              const FusedState* state, hipStream_t stream) {
    const GemvShape sh = gemv_shape(w.input, w.output, w.bits);
    GemvLaunch l{};
    GemvArgs& a = l.args;
    a.w = {w.trellis, w.suh, w.svh, w.bias};
    a.table = table;
    a.x = call.x;
    a.y = call.y;
    a.partials = planes;
    if (state) a.state = *state;
    a.x_row_stride = call.x_row_stride;
    a.y_row_stride = call.y_row_stride;
    a.x_group_stride = xg;
    a.y_group_stride = yg;
    a.I = w.input;
    a.N = w.output;
    a.rows = uint32_t(call.rows);
    a.splits = sh.splits;
    a.bps = sh.bps;
    a.alpha = call.alpha;
    a.beta = call.beta;
    a.mode = state ? 1 : 0;
    a.poll_limit = call.gemv_poll_limit;
    a.ncg = w.output / 128;
    a.groups = groups;
    l.rows_template = rows_template(call.rows);
    // Split-major 1-D grid (gemv_slot).
    l.grid = dim3(a.ncg * groups * sh.splits, 1, 1);
    l.codebook = w.codebook;
    l.lds = size_t(l.rows_template) * (32u * sh.bps + 2048u);
    l.stream = stream;
    return l;
}

// The per-split buffer resource spans bps rows of tiles and must stay below
// 2^31 bytes (its out-of-range sentinel); the 1-D grid holds every column
// group x split; the planes of one column group fit a buffer resource.
static bool gemv_fits(const DeviceWeights& w, uint32_t groups, uint64_t rows) {
    const GemvShape sh = gemv_shape(w.input, w.output, w.bits);
    const uint64_t cgs = uint64_t(w.output / 128) * groups;
    return uint64_t(sh.bps) * (w.output / 16) * 32u * w.bits < (uint64_t(1) << 31) &&
           cgs * sh.splits < (uint64_t(1) << 31) &&
           uint64_t(sh.splits) * rows * 128 * 8 < (uint64_t(1) << 31);
}

hipError_t launch_gemv(const DeviceWeights& w, const LinearCall& call, hipStream_t stream) {
    if (!gemv_fits(w, 1, call.rows)) return hipErrorInvalidValue;
    GemvLaunch l = make_launch(w, nullptr, 1, call, 0, 0, static_cast<float*>(call.workspace), nullptr, stream);
    hipError_t e = gemv_table[w.bits - 1](l);
    if (e != hipSuccess || l.args.splits == 1) return e;
    hipLaunchKernelGGL(gemv_finish_kernel, dim3(w.output / 128, 1, 1), dim3(GEMV_THREADS), 0, stream, l.args);
    return hipGetLastError();
}

hipError_t launch_plane_finish(const DeviceWeights& w, const LinearCall& call, const float* planes, uint32_t splits,
                               hipStream_t stream) {
    if (!call.rows) return hipSuccess;
    GemvArgs a{};
    a.w = {w.trellis, w.suh, w.svh, w.bias};
    a.y = call.y;
    a.partials = const_cast<float*>(planes);
    a.y_row_stride = call.y_row_stride;
    a.I = w.input;
    a.N = w.output;
    a.rows = uint32_t(call.rows);
    a.splits = splits;
    a.alpha = call.alpha;
    a.beta = call.beta;
    constexpr uint64_t rows_per_wg = GEMV_WAVES * kPlaneRowsPerWave;
    const uint32_t row_groups = uint32_t((call.rows + rows_per_wg - 1) / rows_per_wg);
    hipLaunchKernelGGL(plane_finish_kernel, dim3(w.output / 128, row_groups, 1), dim3(GEMV_THREADS), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_gemv_fused(const DeviceWeights& w, const LinearCall& call, const FusedState& state,
                             hipStream_t stream) {
    if (!gemv_fits(w, 1, call.rows)) return hipErrorInvalidValue;
    GemvLaunch l = make_launch(w, nullptr, 1, call, 0, 0, nullptr, &state, stream);
    return gemv_table[w.bits - 1](l);
}

hipError_t launch_gemv_grouped(const DeviceWeights& geometry, const GroupWeights* table, uint32_t groups,
                               const LinearCall& call, uint64_t x_group_stride, uint64_t y_group_stride,
                               const FusedState* state, hipStream_t stream) {
    if (!gemv_fits(geometry, groups, call.rows)) return hipErrorInvalidValue;
    GemvLaunch l = make_launch(geometry, table, groups, call, x_group_stride, y_group_stride,
                               static_cast<float*>(call.workspace), state, stream);
    hipError_t e = gemv_table[geometry.bits - 1](l);
    if (e != hipSuccess || state || l.args.splits == 1) return e;
    hipLaunchKernelGGL(gemv_finish_kernel, dim3(geometry.output / 128, 1, groups), dim3(GEMV_THREADS), 0,
                       stream, l.args);
    return hipGetLastError();
}

using GemvOwnerDispatch = hipError_t (*)(const GemvLaunch&);
static const GemvOwnerDispatch owner_table[8] = {gemv_owner_dispatch<1>, gemv_owner_dispatch<2>,
                                                 gemv_owner_dispatch<3>, gemv_owner_dispatch<4>,
                                                 gemv_owner_dispatch<5>, gemv_owner_dispatch<6>,
                                                 gemv_owner_dispatch<7>, gemv_owner_dispatch<8>};

// The owner kernel keeps its inputs and wave partials in at most 64 KiB of LDS.
bool gemv_owner_fits(const DeviceWeights& w, uint64_t rows) {
    const GemvShape sh = gemv_shape(w.input, w.output, w.bits);
    return rows >= 1 && rows <= 8 && sh.splits > 1 && owner_lds_bytes(owner_rows_template(rows), sh.bps) <= 65536;
}

hipError_t launch_gemv_owner(const DeviceWeights& geometry, const GroupWeights* table, uint32_t groups,
                             const LinearCall& call, uint64_t x_group_stride, uint64_t y_group_stride,
                             hipStream_t stream) {
    if (!gemv_fits(geometry, groups, call.rows) || !gemv_owner_fits(geometry, call.rows)) return hipErrorInvalidValue;
    GemvLaunch l = make_launch(geometry, table, groups, call, x_group_stride, y_group_stride, nullptr, nullptr,
                               stream);
    l.grid = dim3(l.args.ncg * groups, 1, 1);
    l.rows_template = owner_rows_template(call.rows);
    l.lds = owner_lds_bytes(l.rows_template, l.args.bps);
    return owner_table[geometry.bits - 1](l);
}

// ---------------------------------------------------------------------------
// Diagnostics and utilities.
// ---------------------------------------------------------------------------
using DecodeDispatch = hipError_t (*)(uint32_t, const uint32_t*, uint32_t, uint32_t, uint64_t, _Float16*,
                                      hipStream_t);
static const DecodeDispatch decode_table[8] = {decode_dispatch<1>, decode_dispatch<2>, decode_dispatch<3>,
                                               decode_dispatch<4>, decode_dispatch<5>, decode_dispatch<6>,
                                               decode_dispatch<7>, decode_dispatch<8>};

hipError_t launch_decode(const DeviceWeights& w, _Float16* q, hipStream_t stream) {
    return decode_table[w.bits - 1](w.codebook, w.trellis, w.input, w.output, w.trellis_bytes, q, stream);
}

__global__ __launch_bounds__(64) void input_stage_kernel(const float* x, const uint16_t* suh, uint32_t I,
                                                         _Float16* out) {
    const uint64_t r = blockIdx.y;
    const uint32_t ch = blockIdx.x * 128;
    input_block(x + r * I + ch, suh + ch, out + r * I + ch, true);
}

hipError_t launch_input_stage(const DeviceWeights& w, const float* x, uint64_t rows, _Float16* a,
                              hipStream_t stream) {
    if (!rows) return hipSuccess;
    hipLaunchKernelGGL(input_stage_kernel, dim3(w.input / 128, rows), dim3(64), 0, stream, x, w.suh, w.input, a);
    return hipGetLastError();
}

__global__ __launch_bounds__(64) void output_stage_kernel(const float* core, const uint16_t* svh,
                                                          const float* bias, uint32_t N, float alpha,
                                                          float beta, float* y) {
    const uint64_t r = blockIdx.y;
    const int lane = threadIdx.x;
    const uint32_t n0 = blockIdx.x * 128 + lane, n1 = n0 + 64;
    float z0 = core[r * N + n0], z1 = core[r * N + n1];
    h32_wave(z0, z1);
    float* yr = y + r * N;
    const float o0 = output_element(z0, svh[n0], bias, n0, alpha, beta, yr + n0);
    const float o1 = output_element(z1, svh[n1], bias, n1, alpha, beta, yr + n1);
    yr[n0] = o0;
    yr[n1] = o1;
}

hipError_t launch_output_stage(const DeviceWeights& w, const float* core, uint64_t rows, float* y, float alpha,
                               float beta, hipStream_t stream) {
    if (!rows) return hipSuccess;
    hipLaunchKernelGGL(output_stage_kernel, dim3(w.output / 128, rows), dim3(64), 0, stream, core, w.svh, w.bias,
                       w.output, alpha, beta, y);
    return hipGetLastError();
}

// Streaming read: workgroup b reads its contiguous 1/workgroups of the bytes
// with 16-byte buffer loads and folds them with XOR; one word per workgroup is
// stored.  Each lane keeps DEPTH loads in flight as a rolling ring (a load is
// refilled as soon as its slot is consumed), so the read never drains between
// batches; loads past the slice are out of range (zeros, no memory access).
// The call floor of a kernel that reads a given number of bytes once is the
// fastest of these shapes (threads x depth x workgroups).
template <int DEPTH, int THREADS>
__global__ __launch_bounds__(THREADS) void stream_read_kernel(const unsigned char* src, uint64_t bytes,
                                                              uint32_t* sink) {
    const uint64_t per = bytes / gridDim.x;   // a multiple of 16 (checked by the launcher)
    const auto rsrc = make_rsrc(src + uint64_t(blockIdx.x) * per, uint32_t(per));
    const uint32_t n = uint32_t(per / 16), loads = (n + THREADS - 1) / THREADS;
    auto off = [&](uint32_t t) -> uint32_t {
        const uint32_t j = threadIdx.x + t * THREADS;
        return j < n ? j * 16u : 0x80000000u;
    };
    u32x4 ring[DEPTH];
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) ring[u] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off(u), 0, 0);
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (uint32_t t = 0; t < loads; t += DEPTH) {
#pragma unroll
        for (int u = 0; u < DEPTH; ++u) {
            acc ^= ring[u];
            ring[u] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off(t + u + DEPTH), 0, 0);
        }
    }
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) acc ^= ring[u];   // out of range: zeros
    uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
    for (int off2 = 32; off2 > 0; off2 >>= 1) r ^= __shfl_xor(r, off2);
    __shared__ uint32_t part[THREADS / 64];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = r;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t v = 0;
        for (int k = 0; k < THREADS / 64; ++k) v ^= part[k];
        sink[blockIdx.x] = v;
    }
}

hipError_t launch_stream_read(const void* src, uint64_t bytes, uint32_t workgroups, uint32_t threads, uint32_t depth,
                              uint32_t* sink, hipStream_t stream) {
    if (!workgroups || bytes % (16ull * workgroups) || bytes / workgroups >= (uint64_t(1) << 31) ||
        !stream_read_shape_ok(threads, depth))
        return hipErrorInvalidValue;
    using Fn = void (*)(const unsigned char*, uint64_t, uint32_t*);
    static const Fn table[5][5] = {
        {stream_read_kernel<1, 64>, stream_read_kernel<2, 64>, stream_read_kernel<4, 64>, stream_read_kernel<8, 64>,
         stream_read_kernel<16, 64>},
        {stream_read_kernel<1, 128>, stream_read_kernel<2, 128>, stream_read_kernel<4, 128>,
         stream_read_kernel<8, 128>, stream_read_kernel<16, 128>},
        {stream_read_kernel<1, 256>, stream_read_kernel<2, 256>, stream_read_kernel<4, 256>,
         stream_read_kernel<8, 256>, stream_read_kernel<16, 256>},
        {stream_read_kernel<1, 512>, stream_read_kernel<2, 512>, stream_read_kernel<4, 512>,
         stream_read_kernel<8, 512>, stream_read_kernel<16, 512>},
        {stream_read_kernel<1, 1024>, stream_read_kernel<2, 1024>, stream_read_kernel<4, 1024>,
         stream_read_kernel<8, 1024>, stream_read_kernel<16, 1024>}};
    const int ti = __builtin_ctz(threads) - 6, di = __builtin_ctz(depth);
    hipLaunchKernelGGL(table[ti][di], dim3(workgroups), dim3(threads), 0, stream,
                       static_cast<const unsigned char*>(src), bytes, sink);
    return hipGetLastError();
}

__global__ void fill_u32_kernel(uint32_t* p, uint32_t value, uint64_t count) {
    const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < count) p[i] = value;
}

hipError_t launch_fill_u32(uint32_t* p, uint32_t value, uint64_t count, hipStream_t stream) {
    if (!count) return hipSuccess;
    hipLaunchKernelGGL(fill_u32_kernel, dim3(uint32_t((count + 255) / 256)), dim3(256), 0, stream, p, value, count);
    return hipGetLastError();
}

}  // namespace stx
