// Fake kernel launchers.  Each records its call, checks that every device
// buffer the real kernels would touch lies inside a live fake allocation of
// sufficient size (and, for the single-launch GEMV, that its state arrives
// zero-filled), and returns the injected launch result.  A failed
// check aborts: it is a contract violation of the API layer.
#include "fake.hpp"
#include "backend.hpp"
#include "moe.hpp"

#include <cstdio>
#include <cstdlib>
#include <map>
#include <vector>

namespace {

void require(bool ok, const char* what, const char* launcher) {
    if (ok) return;
    std::fprintf(stderr, "contract violation in %s: %s\n", launcher, what);
    std::abort();
}

fake::Launch record(const char* name, uint64_t rows, const void* ws, const void* planes, hipStream_t s, float alpha,
                    float beta) {
    fake::Launch l;
    l.name = name;
    l.rows = rows;
    l.workspace = ws;
    l.planes = planes;
    l.stream = s;
    l.alpha = alpha;
    l.beta = beta;
    fake::launches.push_back(l);
    return l;
}

// The input and output rows of a linear call lie in device memory.
void check_call(const stx::DeviceWeights& w, const stx::LinearCall& c, const char* who) {
    require(c.rows > 0, "zero rows reach a launcher", who);
    const uint64_t xb = ((c.rows - 1) * c.x_row_stride + w.input) * 4;
    const uint64_t yb = ((c.rows - 1) * c.y_row_stride + w.output) * 4;
    require(fake::in_live_block(c.x, xb), "input outside device memory", who);
    require(fake::in_live_block(c.y, yb), "output outside device memory", who);
    require(fake::in_live_block(w.trellis, w.trellis_bytes), "trellis outside device memory", who);
}

}  // namespace

namespace stx {

hipError_t launch_gemv(const DeviceWeights& w, const LinearCall& c, hipStream_t s) {
    check_call(w, c, "launch_gemv");
    const uint64_t need = gemv_workspace_bytes(w, uint32_t(c.rows));
    require(!need || fake::in_live_block(c.workspace, need), "GEMV workspace too small", "launch_gemv");
    record("gemv", c.rows, c.workspace, nullptr, s, c.alpha, c.beta);
    return fake::launch_result();
}

// The single-launch state of `groups` groups starts at st.status, lies in
// device memory and holds what a fresh plan holds (no launch ran): status and
// epochs 0, every plane word EMPTY.
void check_state(const DeviceWeights& w, uint64_t rows, uint32_t groups, const FusedState& st, const char* who) {
    const uint64_t bytes = fused_state_bytes(w, rows, groups);
    require(bytes > 0, "single launch without split partials", who);
    require(fake::in_live_block(st.status, bytes), "single-launch state outside device memory", who);
    const FusedState at = fused_state_at(st.status, w, rows, groups);
    require(at.epochs == st.epochs && at.planes == st.planes, "single-launch state layout", who);
    const uint64_t planes = fused_planes_offset(w, groups) / 4;
    const uint32_t* p = st.status;
    for (uint64_t i = 0; i < bytes / 4; ++i)
        require(p[i] == (i < planes ? 0u : GEMV_PLANE_EMPTY), "single-launch state not initialised", who);
}

hipError_t launch_gemv_fused(const DeviceWeights& w, const LinearCall& c, const FusedState& st, hipStream_t s) {
    check_call(w, c, "launch_gemv_fused");
    check_state(w, c.rows, 1, st, "launch_gemv_fused");
    record("gemv_fused", c.rows, c.workspace, st.planes, s, c.alpha, c.beta);
    return fake::launch_result();
}

hipError_t launch_plane_finish(const DeviceWeights& w, const LinearCall& c, const float* planes, uint32_t splits,
                               hipStream_t s) {
    check_call(w, c, "launch_plane_finish");
    require(fake::in_live_block(planes, uint64_t(splits) * c.rows * w.output * 4), "planes outside device memory",
            "launch_plane_finish");
    record("plane_finish", c.rows, c.workspace, planes, s, c.alpha, c.beta);
    return fake::launch_result();
}

hipError_t launch_gemv_grouped(const DeviceWeights& g, const GroupWeights* table, uint32_t groups,
                               const LinearCall& c, uint64_t x_group_stride, uint64_t y_group_stride,
                               const FusedState* st, hipStream_t s) {
    const bool single_launch = st != nullptr;
    require(groups > 0, "no groups", "launch_gemv_grouped");
    require(fake::in_live_block(table, groups * sizeof(GroupWeights)), "group table outside device memory",
            "launch_gemv_grouped");
    const uint64_t xb = ((groups - 1) * x_group_stride + (c.rows - 1) * c.x_row_stride + g.input) * 4;
    const uint64_t yb = ((groups - 1) * y_group_stride + (c.rows - 1) * c.y_row_stride + g.output) * 4;
    require(fake::in_live_block(c.x, xb), "grouped input outside device memory", "launch_gemv_grouped");
    require(fake::in_live_block(c.y, yb), "grouped output outside device memory", "launch_gemv_grouped");
    if (single_launch) check_state(g, c.rows, groups, *st, "launch_gemv_grouped");
    record(single_launch ? "gemv_grouped_fused" : "gemv_grouped", c.rows, c.workspace, nullptr, s, c.alpha, c.beta);
    return fake::launch_result();
}

hipError_t launch_gemv_owner(const DeviceWeights& g, const GroupWeights* table, uint32_t groups,
                             const LinearCall& c, uint64_t x_group_stride, uint64_t y_group_stride, hipStream_t s) {
    require(groups > 0 && gemv_owner_fits(g, c.rows), "owner fold shape", "launch_gemv_owner");
    require(fake::in_live_block(table, groups * sizeof(GroupWeights)), "group table outside device memory",
            "launch_gemv_owner");
    const uint64_t xb = ((groups - 1) * x_group_stride + (c.rows - 1) * c.x_row_stride + g.input) * 4;
    const uint64_t yb = ((groups - 1) * y_group_stride + (c.rows - 1) * c.y_row_stride + g.output) * 4;
    require(fake::in_live_block(c.x, xb), "grouped input outside device memory", "launch_gemv_owner");
    require(fake::in_live_block(c.y, yb), "grouped output outside device memory", "launch_gemv_owner");
    record("gemv_owner", c.rows, c.workspace, nullptr, s, c.alpha, c.beta);
    return fake::launch_result();
}

bool gemv_owner_fits(const DeviceWeights& w, uint64_t rows) {
    const GemvShape sh = gemv_shape(w.input, w.output, w.bits);
    return rows >= 1 && rows <= 8 && sh.splits > 1;
}

hipError_t launch_gemm(const DeviceWeights& w, const LinearCall& c, hipStream_t s) {
    check_call(w, c, "launch_gemm");
    require(fake::in_live_block(c.workspace, gemm_workspace_bytes(w, c.rows)), "GEMM workspace too small",
            "launch_gemm");
    record("gemm", c.rows, c.workspace, nullptr, s, c.alpha, c.beta);
    return fake::launch_result();
}

hipError_t launch_decode(const DeviceWeights& w, _Float16* q, hipStream_t s) {
    require(fake::in_live_block(q, uint64_t(w.input) * w.output * 2), "decode output outside device memory",
            "launch_decode");
    record("decode", 0, nullptr, nullptr, s, 0, 0);
    return fake::launch_result();
}

hipError_t launch_input_stage(const DeviceWeights& w, const float* x, uint64_t rows, _Float16* a, hipStream_t s) {
    require(fake::in_live_block(x, rows * w.input * 4), "stage input outside device memory", "launch_input_stage");
    require(fake::in_live_block(a, rows * w.input * 2), "stage output outside device memory", "launch_input_stage");
    record("input_stage", rows, nullptr, nullptr, s, 0, 0);
    return fake::launch_result();
}

hipError_t launch_output_stage(const DeviceWeights& w, const float* core, uint64_t rows, float* y, float alpha,
                               float beta, hipStream_t s) {
    require(fake::in_live_block(core, rows * w.output * 4), "core outside device memory", "launch_output_stage");
    require(fake::in_live_block(y, rows * w.output * 4), "output outside device memory", "launch_output_stage");
    record("output_stage", rows, nullptr, nullptr, s, alpha, beta);
    return fake::launch_result();
}

hipError_t launch_fill_u32(uint32_t* p, uint32_t value, uint64_t count, hipStream_t s) {
    require(fake::in_live_block(p, count * 4), "fill outside device memory", "launch_fill_u32");
    record("fill", count, nullptr, p, s, 0, 0);
    const hipError_t e = fake::launch_result();
    if (e == hipSuccess)
        for (uint64_t i = 0; i < count; ++i) p[i] = value;
    return e;
}

// The static scratch of the allocation-free GEMV: one host block per fake
// device, registered as a live device block once (not a hipMalloc).
hipError_t gemv_scratch_address(int device, void** out) {
    static std::map<int, std::vector<unsigned char>> blocks;
    auto it = blocks.find(device);
    if (it == blocks.end()) {
        it = blocks.emplace(device, std::vector<unsigned char>(kGemvScratchBytes)).first;
        fake::live[reinterpret_cast<uintptr_t>(it->second.data())] = fake::Block{kGemvScratchBytes, device};
    }
    *out = it->second.data();
    return hipSuccess;
}

hipError_t launch_stream_read(const void* src, uint64_t bytes, uint32_t workgroups, uint32_t threads, uint32_t depth,
                              uint32_t* sink, hipStream_t s) {
    require(workgroups > 0 && bytes % (16ull * workgroups) == 0 && stream_read_shape_ok(threads, depth),
            "stream read shape", "launch_stream_read");
    require(fake::in_live_block(src, bytes), "stream read source outside device memory", "launch_stream_read");
    require(fake::in_live_block(sink, uint64_t(workgroups) * 4), "stream read sink outside device memory",
            "launch_stream_read");
    record("stream_read", 0, nullptr, nullptr, s, 0, 0);
    return fake::launch_result();
}

static void check_moe(const MoeArgs& a, bool gate_up, const char* who) {
    const uint64_t routes = uint64_t(a.rows) * a.topk;
    require(fake::in_live_block(a.bank, a.bank_count * sizeof(MoeExpert)), "expert table outside device memory", who);
    require(fake::in_live_block(a.ids, routes * 4), "route ids outside device memory", who);
    require(fake::in_live_block(a.scores, routes * 4), "route scores outside device memory", who);
    require(fake::in_live_block(a.hidden, routes * a.H * 4), "hidden outside device memory", who);
    if (gate_up) {
        require(fake::in_live_block(a.x, ((a.rows - 1) * a.x_stride + a.I) * 4), "input outside device memory", who);
        const uint64_t words = routes * (a.H / 128);
        require(fake::in_live_block(a.c_gu, words * 4), "gate/up counters outside device memory", who);
        for (uint64_t i = 0; i < words; ++i) require(a.c_gu[i] == 0, "gate/up counters not zero on entry", who);
        require(fake::in_live_block(a.p_gu, routes * a.s_gu * 2 * a.H * 4), "gate/up planes outside device memory",
                who);
        require(fake::in_live_block(a.a_gu, moe_core_input_bytes(uint32_t(routes), a.I)),
                "gate/up core inputs outside device memory", who);
    } else {
        require(fake::in_live_block(a.y, ((a.rows - 1) * a.y_stride + a.I) * 4), "output outside device memory", who);
        const uint64_t words = uint64_t(a.rows) * (a.I / 128);
        require(fake::in_live_block(a.c_d, words * 4), "down counters outside device memory", who);
        for (uint64_t i = 0; i < words; ++i) require(a.c_d[i] == 0, "down counters not zero on entry", who);
        require(fake::in_live_block(a.p_d, routes * a.s_d * a.I * 4), "down planes outside device memory", who);
    }
}

hipError_t launch_moe_gate_up(const MoeArgs& a, hipStream_t s) {
    check_moe(a, true, "launch_moe_gate_up");
    record("moe_gate_up", a.rows, nullptr, nullptr, s, a.alpha, a.beta);
    return fake::launch_result();
}

hipError_t launch_moe_down(const MoeArgs& a, hipStream_t s) {
    check_moe(a, false, "launch_moe_down");
    record("moe_down", a.rows, nullptr, nullptr, s, a.alpha, a.beta);
    return fake::launch_result();
}

hipError_t launch_moe_down_core(const MoeArgs& a, MoeDownMode mode, hipStream_t s) {
    check_moe(a, false, "launch_moe_down_core");
    require(mode == kMoeDownCore || mode == kMoeDownRouteCore, "staged down mode", "launch_moe_down_core");
    record(mode == kMoeDownCore ? "moe_down_core" : "moe_down_route_core", a.rows, nullptr, nullptr, s, a.alpha,
           a.beta);
    return fake::launch_result();
}

hipError_t launch_moe_down_finish(const MoeArgs& a, hipStream_t s) {
    check_moe(a, false, "launch_moe_down_finish");
    record("moe_down_finish", a.rows, nullptr, nullptr, s, a.alpha, a.beta);
    return fake::launch_result();
}

hipError_t launch_moe_swiglu(const float* g, const float* u, float* h, uint64_t count, hipStream_t s) {
    require(fake::in_live_block(g, count * 4) && fake::in_live_block(u, count * 4) &&
                fake::in_live_block(h, count * 4),
            "SwiGLU operands outside device memory", "launch_moe_swiglu");
    record("moe_swiglu", count, nullptr, nullptr, s, 0, 0);
    return fake::launch_result();
}

}  // namespace stx
