// CPU contract test of the C ABI layer (api*.cpp, dispatch.cpp, policy.cpp
// compiled unchanged against a fake HIP runtime).  It checks the status each
// HIP failure maps to, that failed calls leave no device allocation behind,
// that plan submission allocates, copies, synchronises and queries nothing,
// and that every launcher receives device buffers large enough for its
// policy.  The reference's own contract test follows the same idea with its
// own fake (reference tests/test_api_contract.cpp:1-115, docs/API.md:349-374).
#include "fake.hpp"
#include "policy.hpp"
#include "strix_trellis.h"
#include "strix_trellis_amd.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

static int checks = 0;
#define CHECK(cond)                                                                    \
    do {                                                                               \
        ++checks;                                                                      \
        if (!(cond)) {                                                                 \
            std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #cond); \
            std::exit(1);                                                              \
        }                                                                              \
    } while (0)
#define STATUS(expr, want)                                                                           \
    do {                                                                                             \
        ++checks;                                                                                    \
        const strix_status got_ = (expr);                                                            \
        if (got_ != (want)) {                                                                        \
            std::fprintf(stderr, "%s:%d: %s returned %d (%s), want %d\n", __FILE__, __LINE__, #expr, \
                         int(got_), strix_status_string(got_), int(want));                          \
            std::exit(1);                                                                            \
        }                                                                                            \
    } while (0)

template <class T>
static T header() {
    T d;
    std::memset(&d, 0, sizeof(d));
    d.struct_size = sizeof(T);
    d.abi_version = STRIX_TRELLIS_ABI_VERSION;
    return d;
}

static strix_stream stream_of(hipStream_t s) {
    strix_stream st = header<strix_stream>();
    st.hip_stream = s;
    return st;
}

// Host regions of one EXL3 linear (mul1 codebook), deterministic bytes.
struct HostLinear {
    uint64_t rows, columns;
    uint32_t bits;
    bool bias;
    std::vector<uint8_t> trellis, suh, svh, b;
    HostLinear(uint64_t n, uint64_t i, uint32_t k, bool with_bias) : rows(n), columns(i), bits(k), bias(with_bias) {
        trellis.resize(n * i / 8 * k);
        suh.resize(i * 2);
        svh.resize(n * 2);
        if (bias) b.resize(n * 4);
        uint32_t x = 12345;
        for (auto* v : {&trellis, &suh, &svh, &b})
            for (auto& c : *v) c = uint8_t((x = x * 1103515245u + 12345u) >> 16);
    }
    strix_exl3_parts_desc parts() const {
        strix_exl3_parts_desc d = header<strix_exl3_parts_desc>();
        d.transport_version = STRIX_TRELLIS_TRANSPORT_VERSION;
        d.bits_x2 = bits * 2;
        d.rows = rows;
        d.columns = columns;
        d.codebook = STRIX_CODEBOOK_MUL1;
        d.marker = STRIX_EXL3_MARKER_MUL1;
        d.trellis = {trellis.data(), trellis.size()};
        d.suh = {suh.data(), suh.size()};
        d.svh = {svh.data(), svh.size()};
        if (bias) d.bias = {b.data(), b.size()};
        return d;
    }
};

static void* device_alloc(size_t bytes) {
    void* p = nullptr;
    CHECK(hipMalloc(&p, bytes) == hipSuccess);
    return p;
}

static strix_tensor_desc tensor(void* data, uint64_t bytes, uint64_t rows, uint64_t width, uint32_t rank) {
    strix_tensor_desc t = header<strix_tensor_desc>();
    t.data = data;
    t.buffer_bytes = bytes;
    t.dtype = STRIX_DTYPE_F32;
    t.rank = rank;
    if (rank == 1) {
        t.shape[0] = width;
        t.strides[0] = 1;
    } else {
        t.shape[0] = rows;
        t.shape[1] = width;
        t.strides[0] = width;
        t.strides[1] = 1;
    }
    return t;
}

// No HIP call beyond the device query that validates the calling thread.
static void check_quiet_since(const fake::Counters& before) {
    CHECK(fake::n.mallocs == before.mallocs);
    CHECK(fake::n.frees == before.frees);
    CHECK(fake::n.copies == before.copies);
    CHECK(fake::n.syncs == before.syncs);
    CHECK(fake::n.pointer_queries == before.pointer_queries);
    CHECK(fake::n.range_queries == before.range_queries);
    CHECK(fake::n.stream_queries == before.stream_queries);
}

static void context_rules() {
    strix_context_desc cd = header<strix_context_desc>();
    strix_context c = reinterpret_cast<strix_context>(0x1);
    STATUS(strix_context_create(&cd, &c), STRIX_SUCCESS);
    CHECK(c != nullptr);
    STATUS(strix_context_destroy(c), STRIX_SUCCESS);

    // Only gfx950 with 64-lane waves is accepted.
    const char* wrong[] = {"gfx1151", "gfx942:sramecc+:xnack-", "gfx9500", "gfx95"};
    for (const char* a : wrong) {
        fake::arch = a;
        c = reinterpret_cast<strix_context>(0x1);
        STATUS(strix_context_create(&cd, &c), STRIX_ERROR_UNSUPPORTED_DEVICE);
        CHECK(c == nullptr);
    }
    fake::arch = "gfx950";
    STATUS(strix_context_create(&cd, &c), STRIX_SUCCESS);
    STATUS(strix_context_destroy(c), STRIX_SUCCESS);
    fake::arch = "gfx950:sramecc+:xnack-";
    fake::wave = 32;
    STATUS(strix_context_create(&cd, &c), STRIX_ERROR_UNSUPPORTED_DEVICE);
    fake::wave = 64;

    // Device property failures.
    const struct {
        hipError_t e;
        strix_status s;
    } props[] = {{hipErrorNoDevice, STRIX_ERROR_UNSUPPORTED_DEVICE},
                 {hipErrorInvalidDevice, STRIX_ERROR_UNSUPPORTED_DEVICE},
                 {hipErrorOutOfMemory, STRIX_ERROR_OUT_OF_MEMORY},
                 {hipErrorUnknown, STRIX_ERROR_BACKEND}};
    for (const auto& p : props) {
        fake::props_error = p.e;
        c = reinterpret_cast<strix_context>(0x1);
        STATUS(strix_context_create(&cd, &c), p.s);
        CHECK(c == nullptr);
    }
    fake::props_error = hipSuccess;
    cd.device_ordinal = 9;
    STATUS(strix_context_create(&cd, &c), STRIX_ERROR_UNSUPPORTED_DEVICE);
    cd.device_ordinal = -1;
    STATUS(strix_context_create(&cd, &c), STRIX_ERROR_INVALID_ARGUMENT);
    cd.device_ordinal = 0;

    // Descriptor header rules.
    cd.struct_size = sizeof(cd) - 8;
    STATUS(strix_context_create(&cd, &c), STRIX_ERROR_ABI_MISMATCH);
    cd.struct_size = sizeof(cd);
    cd.abi_version = 2;
    STATUS(strix_context_create(&cd, &c), STRIX_ERROR_ABI_MISMATCH);
    cd.abi_version = STRIX_TRELLIS_ABI_VERSION;
    cd.reserved[3] = 1;
    STATUS(strix_context_create(&cd, &c), STRIX_ERROR_INVALID_ARGUMENT);
    cd.reserved[3] = 0;
    cd.flags = 1;
    STATUS(strix_context_create(&cd, &c), STRIX_ERROR_INVALID_ARGUMENT);
    STATUS(strix_context_create(nullptr, &c), STRIX_ERROR_INVALID_ARGUMENT);
    STATUS(strix_context_create(&cd, nullptr), STRIX_ERROR_INVALID_ARGUMENT);
    STATUS(strix_context_destroy(nullptr), STRIX_ERROR_INVALID_ARGUMENT);
}

// Every prepare failure drains the stream, frees its allocation and returns
// the mapped status.
static void prepare_failures(strix_context c, hipStream_t hs) {
    const HostLinear L(256, 512, 4, true);
    const strix_exl3_parts_desc parts = L.parts();
    strix_stream st = stream_of(hs);
    const size_t live0 = fake::live.size();
    strix_weights w = reinterpret_cast<strix_weights>(0x1);

    fake::malloc_fail_at = 0;
    STATUS(strix_weights_prepare_parts(c, &parts, &st, &w), STRIX_ERROR_OUT_OF_MEMORY);
    CHECK(w == nullptr && fake::live.size() == live0);
    fake::malloc_fail_at = 0;
    fake::malloc_error = hipErrorUnknown;
    STATUS(strix_weights_prepare_parts(c, &parts, &st, &w), STRIX_ERROR_BACKEND);
    fake::reset_failures();

    for (int at = 0; at < 4; ++at) {   // trellis, suh, svh, bias copies
        const fake::Counters before = fake::n;
        fake::copy_fail_at = at;
        STATUS(strix_weights_prepare_parts(c, &parts, &st, &w), STRIX_ERROR_BACKEND);
        CHECK(w == nullptr && fake::live.size() == live0);
        CHECK(fake::n.copies == before.copies + at + 1);   // nothing enqueued after the failure
        CHECK(fake::n.syncs == before.syncs + 1);          // the stream is drained before the free
        fake::reset_failures();
    }
    fake::copy_fail_at = 1;
    fake::copy_error = hipErrorOutOfMemory;
    STATUS(strix_weights_prepare_parts(c, &parts, &st, &w), STRIX_ERROR_OUT_OF_MEMORY);
    fake::reset_failures();
    fake::sync_fail_at = 0;
    STATUS(strix_weights_prepare_parts(c, &parts, &st, &w), STRIX_ERROR_BACKEND);
    CHECK(w == nullptr && fake::live.size() == live0);
    fake::reset_failures();

    // Thread and stream validation happens before any allocation.
    fake::get_device_error = hipErrorUnknown;
    STATUS(strix_weights_prepare_parts(c, &parts, &st, &w), STRIX_ERROR_BACKEND);
    fake::get_device_error = hipSuccess;
    fake::current_device = 1;
    STATUS(strix_weights_prepare_parts(c, &parts, &st, &w), STRIX_ERROR_INVALID_ARGUMENT);
    fake::current_device = 0;
    strix_stream other = stream_of(fake::make_stream(1));
    STATUS(strix_weights_prepare_parts(c, &parts, &other, &w), STRIX_ERROR_INVALID_ARGUMENT);
    strix_stream bogus = stream_of(reinterpret_cast<hipStream_t>(&other));
    STATUS(strix_weights_prepare_parts(c, &parts, &bogus, &w), STRIX_ERROR_INVALID_ARGUMENT);
    STATUS(strix_weights_prepare_parts(c, &parts, nullptr, &w), STRIX_ERROR_INVALID_ARGUMENT);
    CHECK(fake::live.size() == live0);

    // Format rules reject before allocating.
    strix_exl3_parts_desc bad = parts;
    bad.marker = STRIX_EXL3_MARKER_MCG;
    STATUS(strix_weights_prepare_parts(c, &bad, &st, &w), STRIX_ERROR_UNSUPPORTED_FORMAT);
    bad = parts;
    bad.columns = 500;
    STATUS(strix_weights_prepare_parts(c, &bad, &st, &w), STRIX_ERROR_UNSUPPORTED_FORMAT);
    bad = parts;
    bad.trellis.bytes -= 4;
    STATUS(strix_weights_prepare_parts(c, &bad, &st, &w), STRIX_ERROR_UNSUPPORTED_FORMAT);
    bad = parts;
    bad.svh.data = bad.suh.data;   // overlapping host regions
    STATUS(strix_weights_prepare_parts(c, &bad, &st, &w), STRIX_ERROR_INVALID_ARGUMENT);
    bad = parts;
    bad.bits_x2 = 7;
    STATUS(strix_weights_prepare_parts(c, &bad, &st, &w), STRIX_ERROR_UNSUPPORTED_FORMAT);
    CHECK(fake::live.size() == live0);

    // Success: one allocation, one copy per region, one synchronisation, and
    // the regions land in 256-byte aligned slices in order.
    const fake::Counters before = fake::n;
    STATUS(strix_weights_prepare_parts(c, &parts, &st, &w), STRIX_SUCCESS);
    CHECK(fake::n.mallocs == before.mallocs + 1 && fake::n.copies == before.copies + 4 &&
          fake::n.syncs == before.syncs + 1);
    const void* span = nullptr;
    uint64_t span_bytes = 0;
    STATUS(strix_weights_device_span(w, &span, &span_bytes), STRIX_SUCCESS);
    CHECK(fake::in_live_block(span, span_bytes));
    const uint8_t* base = static_cast<const uint8_t*>(span);
    uint64_t off = 0;
    for (const auto* v : {&L.trellis, &L.suh, &L.svh, &L.b}) {
        off = (off + 255) / 256 * 256;
        CHECK(std::memcmp(base + off, v->data(), v->size()) == 0);
        off += v->size();
    }
    CHECK(span_bytes == off);
    STATUS(strix_context_destroy(c), STRIX_ERROR_INVALID_ARGUMENT);   // weights still live
    fake::free_fail_at = 0;
    STATUS(strix_weights_destroy(w), STRIX_ERROR_BACKEND);            // a failed free keeps the handle
    STATUS(strix_weights_destroy(w), STRIX_SUCCESS);
    CHECK(fake::live.size() == live0);
}

struct Dense {
    HostLinear host;
    strix_weights w = nullptr;
    void *x = nullptr, *y = nullptr, *ws = nullptr;
    uint64_t rows = 0, ws_bytes = 0;
};

static strix_matmul_desc matmul(const Dense& d, uint64_t rows, uint32_t rank) {
    strix_matmul_desc m = header<strix_matmul_desc>();
    m.weights = d.w;
    m.input = tensor(d.x, rows * d.host.columns * 4, rows, d.host.columns, rank);
    m.output = tensor(d.y, rows * d.host.rows * 4, rows, d.host.rows, rank);
    m.alpha = 0.5f;
    m.beta = 0.25f;
    m.workspace = d.ws;
    m.workspace_bytes = d.ws_bytes;
    return m;
}

static void direct_calls(strix_context c, hipStream_t hs) {
    Dense d{HostLinear(1024, 2048, 4, false)};
    d.rows = 64;
    strix_stream st = stream_of(hs);
    const strix_exl3_parts_desc parts = d.host.parts();
    STATUS(strix_weights_prepare_parts(c, &parts, &st, &d.w), STRIX_SUCCESS);
    d.x = device_alloc(d.rows * d.host.columns * 4);
    d.y = device_alloc(d.rows * d.host.rows * 4);
    strix_matmul_desc m = matmul(d, d.rows, 2);
    STATUS(strix_matmul_workspace_bytes(c, &m, &d.ws_bytes), STRIX_SUCCESS);
    CHECK(d.ws_bytes > 0 && d.ws_bytes % 256 == 0);
    d.ws = device_alloc(d.ws_bytes);
    const size_t live0 = fake::live.size();

    // GEMM: one launcher call with the caller's workspace, scalars forwarded.
    m = matmul(d, d.rows, 2);
    fake::launches.clear();
    STATUS(strix_gemm(c, &m, &st), STRIX_SUCCESS);
    CHECK(fake::launches.size() == 1 && fake::launches[0].name == "gemm" && fake::launches[0].rows == d.rows);
    CHECK(fake::launches[0].workspace == d.ws && fake::launches[0].stream == hs);
    CHECK(fake::launches[0].alpha == 0.5f && fake::launches[0].beta == 0.25f);

    // GEMV of 1..8 rows and of a rank-1 vector.
    for (uint64_t r : {1u, 3u, 8u}) {
        m = matmul(d, r, 2);
        fake::launches.clear();
        STATUS(strix_gemv(c, &m, &st), STRIX_SUCCESS);
        CHECK(fake::launches.size() == 1 && fake::launches[0].name == "gemv" && fake::launches[0].rows == r);
    }
    m = matmul(d, 1, 1);
    fake::launches.clear();
    STATUS(strix_gemv(c, &m, &st), STRIX_SUCCESS);
    CHECK(fake::launches.size() == 1 && fake::launches[0].rows == 1);
    m = matmul(d, 9, 2);
    STATUS(strix_gemv(c, &m, &st), STRIX_ERROR_UNSUPPORTED_FORMAT);

    // Zero rows: success without a launch.
    m = matmul(d, 0, 2);
    fake::launches.clear();
    STATUS(strix_gemm(c, &m, &st), STRIX_SUCCESS);
    CHECK(fake::launches.empty());

    // Launch failures map to BACKEND / OUT_OF_MEMORY.
    m = matmul(d, d.rows, 2);
    fake::launch_fail_at = 0;
    STATUS(strix_gemm(c, &m, &st), STRIX_ERROR_BACKEND);
    fake::launch_fail_at = 0;
    fake::launch_error = hipErrorOutOfMemory;
    STATUS(strix_gemm(c, &m, &st), STRIX_ERROR_OUT_OF_MEMORY);
    fake::reset_failures();

    // Storage rules: host memory, short allocations, short workspaces.
    std::vector<float> host_x(d.rows * d.host.columns);
    fake::launches.clear();
    m = matmul(d, d.rows, 2);
    m.input.data = host_x.data();
    STATUS(strix_gemm(c, &m, &st), STRIX_ERROR_INVALID_ARGUMENT);
    void* short_y = device_alloc(d.rows * d.host.rows * 4 - 256);
    m = matmul(d, d.rows, 2);
    m.output.data = short_y;   // buffer_bytes claims more than the allocation holds
    STATUS(strix_gemm(c, &m, &st), STRIX_ERROR_INSUFFICIENT_BUFFER);
    m = matmul(d, d.rows, 2);
    m.workspace_bytes -= 256;
    STATUS(strix_gemm(c, &m, &st), STRIX_ERROR_INSUFFICIENT_BUFFER);
    m = matmul(d, d.rows, 2);
    m.workspace = static_cast<char*>(d.ws) + 16;   // misaligned
    STATUS(strix_gemm(c, &m, &st), STRIX_ERROR_INVALID_ARGUMENT);
    m = matmul(d, d.rows, 2);
    m.output.data = d.x;   // output aliases input
    STATUS(strix_gemm(c, &m, &st), STRIX_ERROR_INVALID_ARGUMENT);
    m = matmul(d, d.rows, 2);
    m.input.data = const_cast<void*>(static_cast<const void*>(parts.trellis.data));
    STATUS(strix_gemm(c, &m, &st), STRIX_ERROR_INVALID_ARGUMENT);
    CHECK(fake::launches.empty());
    fake::current_device = 1;
    m = matmul(d, d.rows, 2);
    STATUS(strix_gemm(c, &m, &st), STRIX_ERROR_INVALID_ARGUMENT);
    fake::current_device = 0;
    CHECK(hipFree(short_y) == hipSuccess);
    CHECK(fake::live.size() == live0);

    // Linear plans: create validates and owns its planes; submit is quiet.
    uint32_t bps = 0, splits = 0;
    STATUS(strix_amd_gemv_shape(d.w, &bps, &splits), STRIX_SUCCESS);
    CHECK(splits > 1);   // this geometry has split-K partial planes
    m = matmul(d, 4, 2);
    const fake::Counters at_create = fake::n;
    strix_linear_plan gp = nullptr;
    STATUS(strix_linear_plan_create(c, &m, &st, STRIX_OPERATION_GEMV, &gp), STRIX_SUCCESS);
    CHECK(fake::n.mallocs == at_create.mallocs + 1 && fake::n.syncs == at_create.syncs + 1);
    CHECK(fake::live.size() == live0 + 1);
    uint32_t planned = 0;
    STATUS(strix_amd_plan_launches(gp, &planned), STRIX_SUCCESS);
    CHECK(planned == 1);
    for (int rep = 0; rep < 3; ++rep) {
        fake::launches.clear();
        const fake::Counters before = fake::n;
        STATUS(strix_linear_plan_submit(gp), STRIX_SUCCESS);
        check_quiet_since(before);
        CHECK(fake::launches.size() == 1 && fake::launches[0].name == "gemv_fused");
        CHECK(fake::launches[0].rows == 4 && fake::launches[0].stream == hs && fake::launches[0].planes);
    }
    fake::launch_fail_at = 0;
    STATUS(strix_linear_plan_submit(gp), STRIX_ERROR_BACKEND);
    fake::reset_failures();

    strix_linear_plan mp = nullptr;
    m = matmul(d, d.rows, 2);
    STATUS(strix_linear_plan_create(c, &m, &st, STRIX_OPERATION_GEMM, &mp), STRIX_SUCCESS);
    fake::launches.clear();
    const fake::Counters before = fake::n;
    STATUS(strix_linear_plan_submit(mp), STRIX_SUCCESS);
    check_quiet_since(before);
    CHECK(fake::launches.size() == 1 && fake::launches[0].name == "gemm" && fake::launches[0].workspace == d.ws);

    // Plan creation failures free the planes they allocated.
    m = matmul(d, 2, 2);
    const size_t live1 = fake::live.size();
    strix_linear_plan bad = reinterpret_cast<strix_linear_plan>(0x1);
    fake::malloc_fail_at = 0;
    STATUS(strix_linear_plan_create(c, &m, &st, STRIX_OPERATION_GEMV, &bad), STRIX_ERROR_OUT_OF_MEMORY);
    CHECK(bad == nullptr && fake::live.size() == live1);
    fake::reset_failures();
    fake::launch_fail_at = 0;   // the first fill of the single-launch state
    STATUS(strix_linear_plan_create(c, &m, &st, STRIX_OPERATION_GEMV, &bad), STRIX_ERROR_BACKEND);
    CHECK(bad == nullptr && fake::live.size() == live1);
    fake::reset_failures();
    fake::sync_fail_at = 0;
    STATUS(strix_linear_plan_create(c, &m, &st, STRIX_OPERATION_GEMV, &bad), STRIX_ERROR_BACKEND);
    CHECK(bad == nullptr && fake::live.size() == live1);
    fake::reset_failures();
    STATUS(strix_linear_plan_create(c, &m, &st, 7, &bad), STRIX_ERROR_INVALID_ARGUMENT);

    // By default (the reference's rule) every plan gets a state of its own,
    // held with the weights until they are destroyed, so graphs captured from
    // a destroyed plan never share it with a later plan.
    m = matmul(d, 4, 2);
    const size_t live_before = fake::live.size();
    for (int cycle = 0; cycle < 3; ++cycle) {
        const fake::Counters c0 = fake::n;
        strix_linear_plan tp = nullptr;
        STATUS(strix_linear_plan_create(c, &m, &st, STRIX_OPERATION_GEMV, &tp), STRIX_SUCCESS);
        CHECK(fake::n.mallocs == c0.mallocs + 1);
        CHECK(fake::live.size() == live_before + size_t(cycle) + 1);
        STATUS(strix_linear_plan_destroy(tp), STRIX_SUCCESS);
    }
    // Clearing a plan's status re-initialises its whole state (two fills:
    // status and epochs, then the planes) before the synchronisation.
    {
        fake::launches.clear();
        const fake::Counters c0 = fake::n;
        uint32_t flags = 7;
        STATUS(strix_amd_plan_status(gp, 1, &flags), STRIX_SUCCESS);
        CHECK(flags == 0 && fake::n.syncs == c0.syncs + 1 && fake::n.mallocs == c0.mallocs);
        CHECK(fake::launches.size() == 2 && fake::launches[0].name == "fill" && fake::launches[1].name == "fill");
        fake::launches.clear();
        STATUS(strix_amd_plan_status(gp, 0, &flags), STRIX_SUCCESS);
        CHECK(fake::launches.empty());
    }

    // With reuse enabled, a destroyed plan's planes become idle and the next
    // plan of the same size takes them, initialised again (two fills) with no
    // allocation, so the state held stays bounded.
    STATUS(strix_amd_set_plan_state_reuse(c, 1), STRIX_SUCCESS);
    const size_t live2 = fake::live.size() - 1;   // one idle block of this size is there to take
    for (int cycle = 0; cycle < 4; ++cycle) {
        fake::launches.clear();
        const fake::Counters c0 = fake::n;
        strix_linear_plan tp = nullptr;
        STATUS(strix_linear_plan_create(c, &m, &st, STRIX_OPERATION_GEMV, &tp), STRIX_SUCCESS);
        CHECK(fake::n.mallocs == c0.mallocs);   // an idle block of the default-mode cycles
        CHECK(fake::live.size() == live2 + 1);
        CHECK(fake::launches.size() == 2 && fake::launches[0].name == "fill" && fake::launches[1].name == "fill");
        STATUS(strix_linear_plan_destroy(tp), STRIX_SUCCESS);
        CHECK(fake::live.size() == live2 + 1);
    }
    // A failed re-initialisation keeps the idle block for the next plan.
    fake::launch_fail_at = 0;
    STATUS(strix_linear_plan_create(c, &m, &st, STRIX_OPERATION_GEMV, &bad), STRIX_ERROR_BACKEND);
    fake::reset_failures();
    CHECK(bad == nullptr && fake::live.size() == live2 + 1);
    const fake::Counters c1 = fake::n;
    strix_linear_plan again = nullptr;
    STATUS(strix_linear_plan_create(c, &m, &st, STRIX_OPERATION_GEMV, &again), STRIX_SUCCESS);
    CHECK(fake::n.mallocs == c1.mallocs && fake::live.size() == live2 + 1);
    STATUS(strix_linear_plan_destroy(again), STRIX_SUCCESS);
    STATUS(strix_amd_set_plan_state_reuse(c, 0), STRIX_SUCCESS);

    // Weights outlive their plans; the planes go with the weights.
    STATUS(strix_weights_destroy(d.w), STRIX_ERROR_INVALID_ARGUMENT);
    STATUS(strix_linear_plan_destroy(gp), STRIX_SUCCESS);
    STATUS(strix_weights_destroy(d.w), STRIX_ERROR_INVALID_ARGUMENT);
    STATUS(strix_linear_plan_destroy(mp), STRIX_SUCCESS);
    STATUS(strix_weights_destroy(d.w), STRIX_SUCCESS);
    CHECK(fake::live.size() == live0 - 1);
    for (void* p : {d.x, d.y, d.ws}) CHECK(hipFree(p) == hipSuccess);
}

// Routed-expert plan over host routes: creation failures leave nothing
// behind, submission is quiet, and invalid routes are rejected up front.
// The reference's split geometry (5120 <-> 1152, top-6; reference
// src/tp_moe_split_layout.hpp:29-34): the workspace queries give its byte
// counts for 1-8 rows, hidden [rows][6][1152] F32 = rows x 27,648 bytes, then
// P [rows][6][4][5120] F32 = rows x 491,520 bytes with no padding between.
static void moe_reference_split_geometry(strix_context c, hipStream_t hs) {
    const uint32_t I = 5120, H = 1152, k = 6, experts = 6;
    strix_stream st = stream_of(hs);
    std::vector<HostLinear> host;
    for (uint32_t e = 0; e < experts; ++e) {
        host.emplace_back(H, I, 2, false);
        host.emplace_back(H, I, 2, false);
        host.emplace_back(I, H, 2, false);
    }
    std::vector<strix_weights> ws(host.size());
    for (size_t i = 0; i < host.size(); ++i) {
        const strix_exl3_parts_desc p = host[i].parts();
        STATUS(strix_weights_prepare_parts(c, &p, &st, &ws[i]), STRIX_SUCCESS);
    }
    std::vector<strix_tp_expert_desc> ex(experts);
    for (uint32_t e = 0; e < experts; ++e) {
        ex[e] = header<strix_tp_expert_desc>();
        ex[e].expert_id = e;
        ex[e].gate = ws[3 * e];
        ex[e].up = ws[3 * e + 1];
        ex[e].down = ws[3 * e + 2];
    }
    CHECK(stx::moe_split_staged(H).bps == 18 && stx::moe_split_staged(H).splits == 4);
    for (uint32_t rows = 1; rows <= 8; ++rows) {
        void* x = device_alloc(rows * I * 4);
        void* y = device_alloc(rows * I * 4);
        std::vector<uint32_t> ids(rows * k);
        std::vector<float> scores(rows * k, 1.0f / 6);
        for (uint32_t r = 0; r < rows; ++r)
            for (uint32_t q = 0; q < k; ++q) ids[r * k + q] = (r + q) % experts;
        strix_tp_moe_desc d;
        strix_tp_moe_desc_init(&d);
        d.input = tensor(x, rows * I * 4, rows, I, 2);
        d.output = tensor(y, rows * I * 4, rows, I, 2);
        d.experts = ex.data();
        d.expert_count = experts;
        d.route_ids = ids.data();
        d.route_ids_count = rows * k;
        d.route_scores = scores.data();
        d.route_scores_count = rows * k;
        uint64_t plain = 0, split = 0;
        STATUS(strix_tp_moe_workspace_bytes(c, &d, &plain), STRIX_SUCCESS);
        STATUS(strix_tp_moe_split_workspace_bytes(c, &d, &split), STRIX_SUCCESS);
        CHECK(plain == uint64_t(rows) * 27648);
        CHECK(split == uint64_t(rows) * 27648 + uint64_t(rows) * 491520);
        CHECK(hipFree(x) == hipSuccess);
        CHECK(hipFree(y) == hipSuccess);
    }
    for (strix_weights w : ws) STATUS(strix_weights_destroy(w), STRIX_SUCCESS);
}

static void moe_plan(strix_context c, hipStream_t hs) {
    const uint32_t I = 256, H = 512, rows = 2, k = 2, experts = 3;
    strix_stream st = stream_of(hs);
    std::vector<HostLinear> host;
    for (uint32_t e = 0; e < experts; ++e) {
        host.emplace_back(H, I, 2, false);
        host.emplace_back(H, I, 2, false);
        host.emplace_back(I, H, 3, false);
    }
    std::vector<strix_weights> ws(host.size());
    for (size_t i = 0; i < host.size(); ++i) {
        const strix_exl3_parts_desc p = host[i].parts();
        STATUS(strix_weights_prepare_parts(c, &p, &st, &ws[i]), STRIX_SUCCESS);
    }
    std::vector<strix_tp_expert_desc> ex(experts);
    for (uint32_t e = 0; e < experts; ++e) {
        ex[e] = header<strix_tp_expert_desc>();
        ex[e].expert_id = 10 + e;
        ex[e].gate = ws[3 * e];
        ex[e].up = ws[3 * e + 1];
        ex[e].down = ws[3 * e + 2];
    }
    void* x = device_alloc(rows * I * 4);
    void* y = device_alloc(rows * I * 4);
    uint32_t ids[rows * k] = {10, 12, 12, 11};
    float scores[rows * k] = {0.75f, 0.25f, 1.0f, 0.0f};
    strix_tp_moe_desc d;
    strix_tp_moe_desc_init(&d);
    d.input = tensor(x, rows * I * 4, rows, I, 2);
    d.output = tensor(y, rows * I * 4, rows, I, 2);
    d.experts = ex.data();
    d.expert_count = experts;
    d.route_ids = ids;
    d.route_ids_count = rows * k;
    d.route_scores = scores;
    d.route_scores_count = rows * k;
    d.alpha = 1.0f;
    uint64_t need = 0;
    STATUS(strix_tp_moe_workspace_bytes(c, &d, &need), STRIX_SUCCESS);
    CHECK(need >= uint64_t(rows) * k * H * 4);
    d.workspace = device_alloc(need);
    d.workspace_bytes = need;
    const size_t live0 = fake::live.size();

    strix_tp_moe_plan p = reinterpret_cast<strix_tp_moe_plan>(0x1);
    fake::malloc_fail_at = 0;
    STATUS(strix_tp_moe_plan_create(c, &d, &st, &p), STRIX_ERROR_OUT_OF_MEMORY);
    CHECK(p == nullptr && fake::live.size() == live0);
    fake::reset_failures();
    for (int at = 0; at < 3; ++at) {   // expert table, route ids, route scores
        fake::copy_fail_at = at;
        STATUS(strix_tp_moe_plan_create(c, &d, &st, &p), STRIX_ERROR_BACKEND);
        CHECK(p == nullptr && fake::live.size() == live0);
        fake::reset_failures();
    }
    fake::launch_fail_at = 0;   // the counter fill
    STATUS(strix_tp_moe_plan_create(c, &d, &st, &p), STRIX_ERROR_BACKEND);
    CHECK(p == nullptr && fake::live.size() == live0);
    fake::reset_failures();
    fake::sync_fail_at = 0;
    STATUS(strix_tp_moe_plan_create(c, &d, &st, &p), STRIX_ERROR_BACKEND);
    CHECK(p == nullptr && fake::live.size() == live0);
    fake::reset_failures();

    // Route rules.
    ids[1] = 99;   // unknown expert id
    STATUS(strix_tp_moe_plan_create(c, &d, &st, &p), STRIX_ERROR_INVALID_ARGUMENT);
    ids[1] = 10;   // repeated within a row
    STATUS(strix_tp_moe_plan_create(c, &d, &st, &p), STRIX_ERROR_INVALID_ARGUMENT);
    ids[1] = 12;
    scores[0] = -1.0f;
    STATUS(strix_tp_moe_plan_create(c, &d, &st, &p), STRIX_ERROR_INVALID_ARGUMENT);
    scores[0] = 0.75f;
    d.workspace_bytes = need - 4;
    STATUS(strix_tp_moe_plan_create(c, &d, &st, &p), STRIX_ERROR_INSUFFICIENT_BUFFER);
    d.workspace_bytes = need;
    CHECK(fake::live.size() == live0);

    STATUS(strix_tp_moe_plan_create(c, &d, &st, &p), STRIX_SUCCESS);
    CHECK(fake::live.size() == live0 + 1);
    STATUS(strix_weights_destroy(ws[0]), STRIX_ERROR_INVALID_ARGUMENT);   // retained by the plan
    for (int rep = 0; rep < 2; ++rep) {
        fake::launches.clear();
        const fake::Counters before = fake::n;
        STATUS(strix_tp_moe_plan_submit(p), STRIX_SUCCESS);
        check_quiet_since(before);
        CHECK(fake::launches.size() == 2 && fake::launches[0].name == "moe_gate_up" &&
              fake::launches[1].name == "moe_down");
    }
    fake::launches.clear();
    STATUS(strix_tp_moe_plan_gate_up(p), STRIX_SUCCESS);
    STATUS(strix_tp_moe_plan_down(p), STRIX_SUCCESS);
    CHECK(fake::launches.size() == 2);
    fake::launch_fail_at = 1;   // the down launch
    STATUS(strix_tp_moe_plan_submit(p), STRIX_ERROR_BACKEND);
    fake::reset_failures();
    // The staged down checkpoints need a split plan.
    STATUS(strix_tp_moe_plan_down_core(p), STRIX_ERROR_INVALID_ARGUMENT);
    STATUS(strix_tp_moe_plan_down_finish(p), STRIX_ERROR_INVALID_ARGUMENT);
    STATUS(strix_tp_moe_plan_down_reference_core(p), STRIX_ERROR_INVALID_ARGUMENT);
    STATUS(strix_tp_moe_plan_down_core(nullptr), STRIX_ERROR_INVALID_ARGUMENT);
    STATUS(strix_tp_moe_plan_destroy(p), STRIX_SUCCESS);
    CHECK(fake::live.size() == live0);

    // Split plan: P [rows][k][S][I] after hidden rounded up to 256 bytes, the
    // down planes of every launch (checked in device memory by the launchers).
    uint64_t split_need = 0;
    STATUS(strix_tp_moe_split_workspace_bytes(c, &d, &split_need), STRIX_SUCCESS);
    const uint64_t hidden_bytes = uint64_t(rows) * k * H * 4;
    const uint32_t sd = stx::moe_split_staged(H).splits;
    CHECK(split_need == ((hidden_bytes + 255) & ~uint64_t(255)) + uint64_t(rows) * k * sd * I * 4);
    STATUS(strix_tp_moe_plan_create_split(c, &d, &st, &p), STRIX_ERROR_INSUFFICIENT_BUFFER);   // hidden only
    CHECK(p == nullptr && fake::live.size() == live0);
    void* plain_ws = d.workspace;
    void* split_ws = device_alloc(split_need);
    d.workspace = split_ws;
    d.workspace_bytes = split_need - 4;
    STATUS(strix_tp_moe_plan_create_split(c, &d, &st, &p), STRIX_ERROR_INSUFFICIENT_BUFFER);
    d.workspace_bytes = split_need;
    const size_t live1 = fake::live.size();
    STATUS(strix_tp_moe_plan_create_split(c, &d, &st, &p), STRIX_SUCCESS);
    CHECK(fake::live.size() == live1 + 1);
    fake::launches.clear();
    {
        const fake::Counters before = fake::n;
        STATUS(strix_tp_moe_plan_submit(p), STRIX_SUCCESS);
        STATUS(strix_tp_moe_plan_down_core(p), STRIX_SUCCESS);
        STATUS(strix_tp_moe_plan_down_finish(p), STRIX_SUCCESS);
        STATUS(strix_tp_moe_plan_down_reference_core(p), STRIX_SUCCESS);
        check_quiet_since(before);
    }
    CHECK(fake::launches.size() == 5 && fake::launches[2].name == "moe_down_core" &&
          fake::launches[3].name == "moe_down_finish" && fake::launches[4].name == "moe_down_route_core");
    fake::launch_fail_at = 0;
    STATUS(strix_tp_moe_plan_down_finish(p), STRIX_ERROR_BACKEND);
    fake::reset_failures();
    STATUS(strix_tp_moe_plan_destroy(p), STRIX_SUCCESS);
    CHECK(fake::live.size() == live1);
    CHECK(hipFree(split_ws) == hipSuccess);
    d.workspace = plain_ws;
    d.workspace_bytes = need;

    // Device routes: bank ids are positions; the routes are device buffers.
    // The workspace query of the extension matches the host-route queries.
    std::vector<strix_tp_expert_desc> bank(ex);
    for (uint32_t e = 0; e < experts; ++e) bank[e].expert_id = e;
    auto* dev_ids = static_cast<uint32_t*>(device_alloc(rows * k * 4));
    auto* dev_scores = static_cast<float*>(device_alloc(rows * k * 4));
    strix_tp_moe_device_desc dd;
    strix_tp_moe_device_desc_init(&dd);
    dd.input = d.input;
    dd.output = d.output;
    dd.experts = bank.data();
    dd.expert_count = experts;
    dd.route_ids = dev_ids;
    dd.route_ids_bytes = rows * k * 4;
    dd.route_scores = dev_scores;
    dd.route_scores_bytes = rows * k * 4;
    uint64_t dev_plain = 0, dev_split = 0;
    STATUS(strix_amd_tp_moe_device_workspace_bytes(c, &dd, 0, &dev_plain), STRIX_SUCCESS);
    STATUS(strix_amd_tp_moe_device_workspace_bytes(c, &dd, 1, &dev_split), STRIX_SUCCESS);
    CHECK(dev_plain == need && dev_split == split_need);
    STATUS(strix_amd_tp_moe_device_workspace_bytes(c, &dd, 0, nullptr), STRIX_ERROR_INVALID_ARGUMENT);
    bank[1].expert_id = 7;   // not its position
    STATUS(strix_amd_tp_moe_device_workspace_bytes(c, &dd, 1, &dev_split), STRIX_ERROR_INVALID_ARGUMENT);
    CHECK(dev_split == 0);
    bank[1].expert_id = 1;
    dd.route_scores_bytes = rows * k * 4 - 4;   // routes of both kinds must match
    STATUS(strix_tp_moe_plan_create_device_split(c, &dd, &st, &p), STRIX_ERROR_INVALID_ARGUMENT);
    dd.route_scores_bytes = rows * k * 4;
    void* dev_ws = device_alloc(split_need);
    dd.workspace = dev_ws;
    dd.workspace_bytes = need;   // enough for a plain plan only
    STATUS(strix_tp_moe_plan_create_device_split(c, &dd, &st, &p), STRIX_ERROR_INSUFFICIENT_BUFFER);
    const size_t live2 = fake::live.size();
    STATUS(strix_tp_moe_plan_create_device(c, &dd, &st, &p), STRIX_SUCCESS);
    STATUS(strix_tp_moe_plan_down_core(p), STRIX_ERROR_INVALID_ARGUMENT);
    STATUS(strix_tp_moe_plan_destroy(p), STRIX_SUCCESS);
    dd.workspace_bytes = split_need;
    // The routes must not meet the input, the output or the workspace (hidden
    // or P), as the reference requires of all five buffers; nothing is left
    // allocated by a rejected creation.
    {
        const size_t live3 = fake::live.size();
        char* wsb = static_cast<char*>(dev_ws);
        dd.route_ids = reinterpret_cast<uint32_t*>(wsb);   // inside hidden
        STATUS(strix_tp_moe_plan_create_device_split(c, &dd, &st, &p), STRIX_ERROR_INVALID_ARGUMENT);
        STATUS(strix_tp_moe_plan_create_device(c, &dd, &st, &p), STRIX_ERROR_INVALID_ARGUMENT);
        dd.route_ids = dev_ids;
        dd.route_scores = reinterpret_cast<float*>(wsb + split_need - rows * k * 4);   // inside P
        STATUS(strix_tp_moe_plan_create_device_split(c, &dd, &st, &p), STRIX_ERROR_INVALID_ARGUMENT);
        dd.route_scores = dev_scores;
        dd.route_ids = static_cast<uint32_t*>(const_cast<void*>(dd.input.data));   // over the input
        STATUS(strix_tp_moe_plan_create_device_split(c, &dd, &st, &p), STRIX_ERROR_INVALID_ARGUMENT);
        dd.route_ids = dev_ids;
        dd.route_scores = static_cast<float*>(dd.output.data);   // over the output
        STATUS(strix_tp_moe_plan_create_device(c, &dd, &st, &p), STRIX_ERROR_INVALID_ARGUMENT);
        dd.route_scores = dev_scores;
        CHECK(fake::live.size() == live3);
    }
    STATUS(strix_tp_moe_plan_create_device_split(c, &dd, &st, &p), STRIX_SUCCESS);
    fake::launches.clear();
    STATUS(strix_tp_moe_plan_submit(p), STRIX_SUCCESS);
    STATUS(strix_tp_moe_plan_down_core(p), STRIX_SUCCESS);
    STATUS(strix_tp_moe_plan_down_reference_core(p), STRIX_SUCCESS);
    STATUS(strix_tp_moe_plan_down_finish(p), STRIX_SUCCESS);
    CHECK(fake::launches.size() == 5 && fake::launches[3].name == "moe_down_route_core" &&
          fake::launches[4].name == "moe_down_finish");
    STATUS(strix_tp_moe_plan_destroy(p), STRIX_SUCCESS);
    CHECK(fake::live.size() == live2);
    for (void* q : {static_cast<void*>(dev_ids), static_cast<void*>(dev_scores), dev_ws}) CHECK(hipFree(q) == hipSuccess);

    for (strix_weights w : ws) STATUS(strix_weights_destroy(w), STRIX_SUCCESS);
    for (void* q : {x, y, d.workspace}) CHECK(hipFree(q) == hipSuccess);
}

// Decomposition policy over a sweep of layer shapes and row counts (the
// reference checks its own policies the same way, reference
// tests/test_gemv_policy.cpp:92-97).  The shapes must cover their layer, stay
// within the kernels' limits, and follow the documented choice rules.
static void policy_rules() {
    // The benchmark layers: C1 4096^2 S = 16, 4096 -> 12288 S = 8, 5120^2 S = 10
    // (the one-round alternative of S = 20), grouped o_a 4096 -> 1024 S = 16.
    CHECK(stx::gemv_shape(4096, 4096, 4).splits == 16);
    CHECK(stx::gemv_shape(4096, 12288, 4).splits == 8);
    CHECK(stx::gemv_shape(5120, 5120, 4).splits == 10);
    CHECK(stx::gemv_shape(4096, 1024, 5).splits == 16);
    CHECK(stx::gemv_shape(3072, 4096, 4).splits == 24);   // 384 workgroups would load the busiest CU more
    const uint32_t outputs[] = {128, 256, 384, 1024, 1536, 4096, 5120, 8448, 12288};
    for (uint32_t I = 128; I <= 16384; I += 128)
        for (uint32_t N : outputs) {
            // GEMV: whole 8-block units per split, at most 128 blocks; the
            // longest split reaching 512 workgroups, else 16 or 8 blocks;
            // such a pick of more than 17 splits gives way to the most
            // workgroups (at least 384, at least half the splits, no more on
            // the busiest CU) among splits of at most 17 parts.
            const stx::GemvShape sh = stx::gemv_shape(I, N, 4);
            const uint32_t nb = I / 16, nc = N / 128, units = nb / 8;
            CHECK(sh.bps % 8 == 0 && sh.bps >= 8 && sh.bps <= 128);
            CHECK(uint64_t(sh.bps) * sh.splits == nb);
            auto one_round = [&](uint32_t picked) {   // bps of the one-round alternative, or 0
                const uint64_t w0 = uint64_t(nc) * picked;
                for (uint32_t m = 1; m <= 16; ++m) {
                    const uint32_t s = nb / (8 * m);
                    const uint64_t w1 = uint64_t(nc) * s;
                    if (units % m == 0 && s <= 17 && 2 * s >= picked && w1 >= 384 &&
                        (w1 + 255) / 256 * w0 <= (w0 + 255) / 256 * w1)
                        return 8 * m;
                }
                return 0u;
            };
            if (sh.splits > 17) CHECK(!one_round(sh.splits));   // kept only when no one-round shape exists
            bool replaced = false;   // sh is the one-round alternative of some pick of more than 17 splits
            for (uint32_t p = 18; p <= 2 * sh.splits && !replaced; ++p)
                replaced = sh.splits <= 17 && one_round(p) == sh.bps;
            if (replaced) {
                CHECK(uint64_t(nc) * sh.splits >= 384);
            } else {
                const bool reaches = uint64_t(nc) * sh.splits >= 512;
                for (uint32_t m = 1; m <= 16; ++m) {
                    if (units % m) continue;
                    const bool r = uint64_t(nc) * (nb / (8 * m)) >= 512;
                    if (reaches) CHECK(8 * m <= sh.bps || !r);   // no longer split also reaches it
                    else CHECK(!r);                              // nothing reaches it
                }
                if (!reaches) CHECK(sh.bps == 8 || sh.bps == 16);
            }
            stx::DeviceWeights w;
            w.input = I;
            w.output = N;
            w.bits = 4;
            for (uint32_t rows = 1; rows <= 8; ++rows) {
                const uint64_t ws = stx::gemv_workspace_bytes(w, rows);
                CHECK(ws % 256 == 0 && ws >= uint64_t(sh.splits > 1 ? sh.splits : 0) * rows * N * 4);
                const uint64_t fs = stx::fused_state_bytes(w, rows, 1);
                CHECK(sh.splits > 1 ? fs >= 2 * uint64_t(sh.splits - 1) * rows * N * 4 + 256 + (N / 128) * 4 : fs == 0);
                CHECK(stx::linear_workspace_bytes(w, rows) >= ws);
            }
            // GEMM: the narrow split halves whole 128-channel stages; a wide
            // split keeps at least eight 64-channel stages per part and never
            // coexists with the split-tile handoff.
            const uint32_t ns = stx::narrow_splits(w);
            CHECK(ns >= 1 && ns <= 16 && (ns & (ns - 1)) == 0 && (I / 128) % ns == 0);
            const uint64_t pass = stx::gemm_pass_rows(w);
            CHECK(pass >= 256 && pass % 256 == 0 && pass * I * 2 <= (uint64_t(1) << 30) + 256 * uint64_t(I) * 2);
            for (uint64_t m : {1ull, 100ull, 255ull, 256ull, 300ull, 512ull, 777ull, 1024ull, 2048ull, 4096ull}) {
                const uint64_t ws = stx::gemm_workspace_bytes(w, m);
                CHECK(ws % 256 == 0 && ws >= stx::afrag_bytes(w, m < pass ? m : pass));
                CHECK(stx::linear_workspace_bytes(w, m) >= ws);
                if (!stx::gemm_wide(m, w)) {
                    CHECK(stx::gemm_split_count(w, m) == ns);
                    continue;
                }
                const uint32_t s = stx::wide_splits(m, w);
                CHECK(s >= 1 && stx::gemm_split_count(w, m) == s);
                if (s > 1) CHECK((I / 64) / s >= stx::kWideSplitMinStages);
                const stx::WideSplit sp = stx::wide_split(m, w);
                CHECK(uint64_t(sp.full) * 256 + uint64_t(sp.half) * 256 == N);
                const stx::Handoff h = stx::gemm_handoff(m, w);
                if (h.x) {
                    const uint64_t tiles = ((m + 255) / 256) * (N / 256);
                    CHECK(h.x <= 128 && tiles == 256 * uint64_t(h.q) + h.x && tiles % 8 == 0 && s == 1);
                    CHECK(ws >= stx::afrag_bytes(w, m) + stx::handoff_bytes(h.x) + 4 * h.x);
                }
                if (s > 1) CHECK(ws >= stx::afrag_bytes(w, m) + uint64_t(s) * m * N * 4);
            }
        }
    // MoE: whole 8-block units per split, within the kernels' LDS maxima.
    for (uint32_t input = 128; input <= 16384; input += 128)
        for (uint32_t max_bps : {uint32_t(stx::MOE_GU_MAX_BPS), uint32_t(stx::MOE_D_MAX_BPS)}) {
            const stx::MoeSplit ms = stx::moe_split(input, max_bps);
            CHECK(ms.bps % 8 == 0 && ms.bps >= 8 && ms.bps <= max_bps && uint64_t(ms.bps) * ms.splits * 16 == input);
        }
    // Split plans' down: the reference's four equal parts up to H = 5120, and
    // every part's 128-channel groups within the down kernel's LDS.
    for (uint32_t H = 128; H <= 16384; H += 128) {
        const stx::MoeSplit ms = stx::moe_split_staged(H);
        CHECK(uint64_t(ms.bps) * ms.splits * 16 == H);
        if (H <= 5120) CHECK(ms.splits == 4);
        for (uint32_t s = 0; s < ms.splits; ++s) CHECK(stx::moe_down_groups(ms.bps, s) <= uint32_t(stx::MOE_D_MAX_BPS) / 8);
    }
    CHECK(stx::moe_split_staged(1152).bps == 18 && stx::moe_down_groups(18, 1) == 3 && stx::moe_down_groups(18, 3) == 3);
}

// Allocation-free GEMV: no allocation, free, copy or synchronisation; the
// planes go to the device's static scratch; the workspace fields must be
// empty; more than 8 rows and planes beyond the scratch are rejected.
static void noalloc_calls(strix_context c, hipStream_t hs) {
    Dense d{HostLinear(1024, 2048, 4, false)};
    strix_stream st = stream_of(hs);
    const strix_exl3_parts_desc parts = d.host.parts();
    STATUS(strix_weights_prepare_parts(c, &parts, &st, &d.w), STRIX_SUCCESS);
    d.x = device_alloc(9 * d.host.columns * 4);
    d.y = device_alloc(9 * d.host.rows * 4);
    void* scratch = nullptr;
    CHECK(stx::gemv_scratch_address(0, &scratch) == hipSuccess && scratch);
    uint32_t bps = 0, splits = 0;
    STATUS(strix_amd_gemv_shape(d.w, &bps, &splits), STRIX_SUCCESS);
    CHECK(splits > 1);
    for (uint64_t rows : {8u, 3u, 1u}) {
        strix_matmul_desc m = matmul(d, rows, 2);
        m.workspace = nullptr;
        m.workspace_bytes = 0;
        fake::launches.clear();
        const fake::Counters before = fake::n;
        STATUS(strix_amd_gemv_noalloc(c, &m, &st), STRIX_SUCCESS);
        CHECK(fake::n.mallocs == before.mallocs && fake::n.frees == before.frees);
        CHECK(fake::n.copies == before.copies && fake::n.syncs == before.syncs);
        CHECK(fake::launches.size() == 1 && fake::launches[0].name == "gemv");
        CHECK(fake::launches[0].workspace == scratch && fake::launches[0].rows == rows);
    }
    strix_matmul_desc m = matmul(d, 2, 2);   // a workspace is not accepted
    void* ws = device_alloc(1 << 20);
    m.workspace = ws;
    m.workspace_bytes = 1 << 20;
    STATUS(strix_amd_gemv_noalloc(c, &m, &st), STRIX_ERROR_INVALID_ARGUMENT);
    m.workspace = nullptr;
    STATUS(strix_amd_gemv_noalloc(c, &m, &st), STRIX_ERROR_INVALID_ARGUMENT);
    CHECK(hipFree(ws) == hipSuccess);
    m = matmul(d, 9, 2);
    m.workspace = nullptr;
    m.workspace_bytes = 0;
    STATUS(strix_amd_gemv_noalloc(c, &m, &st), STRIX_ERROR_UNSUPPORTED_FORMAT);
    m = matmul(d, 0, 2);
    m.workspace = nullptr;
    m.workspace_bytes = 0;
    fake::launches.clear();
    STATUS(strix_amd_gemv_noalloc(c, &m, &st), STRIX_SUCCESS);
    CHECK(fake::launches.empty());
    fake::launch_fail_at = 0;
    m = matmul(d, 1, 2);
    m.workspace = nullptr;
    m.workspace_bytes = 0;
    STATUS(strix_amd_gemv_noalloc(c, &m, &st), STRIX_ERROR_BACKEND);
    fake::reset_failures();
    STATUS(strix_weights_destroy(d.w), STRIX_SUCCESS);
    // 5120 -> 40960: four splits, so 8 rows need 5.2 MB of planes (> 4 MiB).
    Dense big{HostLinear(40960, 5120, 1, false)};
    const strix_exl3_parts_desc bp = big.host.parts();
    STATUS(strix_weights_prepare_parts(c, &bp, &st, &big.w), STRIX_SUCCESS);
    STATUS(strix_amd_gemv_shape(big.w, &bps, &splits), STRIX_SUCCESS);
    CHECK(uint64_t(splits) * 8 * 40960 * 4 > stx::kGemvScratchBytes);
    big.x = device_alloc(8 * big.host.columns * 4);
    big.y = device_alloc(8 * big.host.rows * 4);
    m = matmul(big, 8, 2);
    m.workspace = nullptr;
    m.workspace_bytes = 0;
    STATUS(strix_amd_gemv_noalloc(c, &m, &st), STRIX_ERROR_INSUFFICIENT_BUFFER);
    m = matmul(big, 2, 2);   // two rows fit
    m.workspace = nullptr;
    m.workspace_bytes = 0;
    STATUS(strix_amd_gemv_noalloc(c, &m, &st), STRIX_SUCCESS);
    STATUS(strix_weights_destroy(big.w), STRIX_SUCCESS);
    for (void* p : {d.x, d.y, big.x, big.y}) CHECK(hipFree(p) == hipSuccess);
}

// The streaming-read measurement kernel: every documented shape launches,
// anything else (or a slice that is not whole 16-byte loads) is refused
// before a launch.
static void stream_read_calls(strix_context c, hipStream_t hs) {
    strix_stream st = stream_of(hs);
    const uint64_t bytes = 1 << 20;
    void* src = device_alloc(bytes);
    auto* sink = static_cast<uint32_t*>(device_alloc(4096 * 4));
    for (uint32_t threads : {64u, 128u, 256u, 512u, 1024u})
        for (uint32_t depth : {1u, 2u, 4u, 8u, 16u}) {
            fake::launches.clear();
            STATUS(strix_amd_stream_read_shaped(c, src, bytes, 256, threads, depth, sink, &st), STRIX_SUCCESS);
            CHECK(fake::launches.size() == 1 && fake::launches[0].name == "stream_read");
        }
    fake::launches.clear();
    STATUS(strix_amd_stream_read_shaped(c, src, bytes, 256, 96, 4, sink, &st), STRIX_ERROR_INVALID_ARGUMENT);
    STATUS(strix_amd_stream_read_shaped(c, src, bytes, 256, 256, 3, sink, &st), STRIX_ERROR_INVALID_ARGUMENT);
    STATUS(strix_amd_stream_read_shaped(c, src, bytes, 256, 2048, 4, sink, &st), STRIX_ERROR_INVALID_ARGUMENT);
    STATUS(strix_amd_stream_read_shaped(c, src, bytes + 16, 256, 256, 4, sink, &st), STRIX_ERROR_INVALID_ARGUMENT);
    STATUS(strix_amd_stream_read_shaped(c, src, bytes, 0, 256, 4, sink, &st), STRIX_ERROR_INVALID_ARGUMENT);
    STATUS(strix_amd_stream_read_shaped(c, src, bytes, 8192, 256, 4, sink, &st), STRIX_ERROR_INSUFFICIENT_BUFFER);
    CHECK(fake::launches.empty());
    STATUS(strix_amd_stream_read(c, src, bytes, 512, sink, &st), STRIX_SUCCESS);
    CHECK(fake::launches.size() == 1);
    for (void* p : {src, static_cast<void*>(sink)}) CHECK(hipFree(p) == hipSuccess);
}

int main() {
    policy_rules();
    context_rules();
    strix_context_desc cd = header<strix_context_desc>();
    strix_context c = nullptr;
    STATUS(strix_context_create(&cd, &c), STRIX_SUCCESS);
    const hipStream_t hs = fake::make_stream(0);
    prepare_failures(c, hs);
    direct_calls(c, hs);
    moe_plan(c, hs);
    moe_reference_split_geometry(c, hs);
    noalloc_calls(c, hs);
    stream_read_calls(c, hs);
    // The default stream (NULL) is accepted everywhere a stream is.
    {
        const HostLinear L(128, 128, 2, false);
        const strix_exl3_parts_desc parts = L.parts();
        strix_stream st = stream_of(nullptr);
        strix_weights w = nullptr;
        STATUS(strix_weights_prepare_parts(c, &parts, &st, &w), STRIX_SUCCESS);
        STATUS(strix_weights_destroy(w), STRIX_SUCCESS);
    }
    STATUS(strix_context_destroy(c), STRIX_SUCCESS);
    // Only the static scratch of the allocation-free GEMV remains.
    void* scratch = nullptr;
    CHECK(stx::gemv_scratch_address(0, &scratch) == hipSuccess);
    CHECK(fake::live.size() == 1 && fake::live.count(reinterpret_cast<uintptr_t>(scratch)) == 1);
    fake::destroy_streams();
    std::printf("contract: %d checks passed\n", checks);
    return 0;
}
