// Grouped strided GEMV plans (reference include/strix_trellis.h:415-457,
// src/dense_r1_group_api.inc:27-137).
//
//   output[r][g*ogs + n] = Linear_g(input[r][g*igs + i]),  alpha 1, beta 0, rows 1..8
//
// Every group runs the generic GEMV core of its geometry in one launch (the
// grid covers every group's column groups), so each row has exactly the bits
// of that row submitted alone through
// strix_gemv (STRIX_GEMV_ROW_INVARIANT_R1).  Workspace layout, all offsets a
// function of the geometry only:
//   [group table: kMaxGroups entries][single-launch state of G groups]
// (the state's status word, launch epochs and partial planes: backend.hpp).
// The workspace is dedicated to the plan: creation uploads the table,
// initialises the state and synchronises the stream; one launch per submission.
#include "api_internal.hpp"

#include <new>

using namespace stx_api;

namespace {
constexpr uint64_t kMaxGroups = STRIX_TP_MAX_BANK_EXPERTS;
uint64_t align_up(uint64_t v) { return (v + kWorkspaceAlign - 1) & ~(kWorkspaceAlign - 1); }

struct GroupLayout {
    uint64_t table_offset = 0, state_offset = 0, state_bytes = 0, bytes = 0;
};

struct Validated {
    std::vector<strix_weights> weights;
    stx::DeviceWeights geometry{};
    uint64_t rows = 0, xrs = 0, xgs = 0, yrs = 0, ygs = 0;
    uint64_t input_bytes = 0, output_bytes = 0;
    GroupLayout layout{};
};

// Bytes up to the last F32 element touched by `count` views of `rows` rows of `width`.
bool view_bytes(uint64_t rows, uint64_t row_stride, uint64_t count, uint64_t group_stride, uint64_t width,
                uint64_t& out) {
    uint64_t a = 0, b = 0;
    if (!checked_mul(rows - 1, row_stride, a) || !checked_mul(count - 1, group_stride, b)) return false;
    if (a > UINT64_MAX - b || a + b > UINT64_MAX - width) return false;
    return checked_mul(a + b + width, 4, out);
}

strix_status validate(strix_context c, const strix_grouped_gemv_desc* d, Validated& v) {
    strix_status s = versioned(d);
    if (s != STRIX_SUCCESS) return s;
    if (!d->weights || d->group_count < 1 || d->group_count > kMaxGroups || d->rows < 1 || d->rows > 8 ||
        d->flags != STRIX_GEMV_ROW_INVARIANT_R1 || !d->input || !d->output)
        return STRIX_ERROR_INVALID_ARGUMENT;
    const uint64_t G = d->group_count;
    v.weights.assign(d->weights, d->weights + G);
    for (uint64_t g = 0; g < G; ++g) {
        const strix_weights w = v.weights[g];
        if (!w || w->owner != c) return STRIX_ERROR_INVALID_ARGUMENT;
        const stx::DeviceWeights& dw = w->dev;
        if (g == 0) {
            v.geometry = dw;
        } else if (dw.bits != v.geometry.bits || dw.input != v.geometry.input || dw.output != v.geometry.output ||
                   dw.codebook != v.geometry.codebook) {
            return STRIX_ERROR_UNSUPPORTED_FORMAT;
        }
        if (w->plans == UINT64_MAX) return STRIX_ERROR_OUT_OF_MEMORY;
    }
    const uint64_t rows = d->rows, I = v.geometry.input, N = v.geometry.output;
    v.rows = rows;
    v.xrs = rows > 1 ? d->input_row_stride : 0;
    v.xgs = G > 1 ? d->input_group_stride : 0;
    v.yrs = rows > 1 ? d->output_row_stride : 0;
    v.ygs = G > 1 ? d->output_group_stride : 0;
    if ((rows > 1 && v.xrs < I) || (G > 1 && v.ygs < N) || (rows > 1 && v.yrs < (G - 1) * v.ygs + N))
        return STRIX_ERROR_INVALID_ARGUMENT;
    if (!view_bytes(rows, v.xrs, G, v.xgs, I, v.input_bytes) || !view_bytes(rows, v.yrs, G, v.ygs, N, v.output_bytes) ||
        v.input_bytes > d->input_buffer_bytes || v.output_bytes > d->output_buffer_bytes ||
        reinterpret_cast<uintptr_t>(d->input) % 4 || reinterpret_cast<uintptr_t>(d->output) % 4 ||
        !Span(d->input, v.input_bytes).addressable() || !Span(d->output, v.output_bytes).addressable() ||
        Span(d->input, v.input_bytes).meets(Span(d->output, v.output_bytes)))
        return STRIX_ERROR_INVALID_ARGUMENT;
    for (strix_weights w : v.weights)
        if (Span(d->input, v.input_bytes).meets(Span(w->base, w->bytes)) || Span(d->output, v.output_bytes).meets(Span(w->base, w->bytes)))
            return STRIX_ERROR_INVALID_ARGUMENT;
    GroupLayout& L = v.layout;
    L.table_offset = 0;
    L.state_offset = align_up(kMaxGroups * sizeof(stx::GroupWeights));
    L.state_bytes = stx::fused_state_bytes(v.geometry, rows, uint32_t(G));
    L.bytes = L.state_offset + align_up(L.state_bytes);
    return STRIX_SUCCESS;
}
}  // namespace

struct strix_grouped_gemv_plan_impl {
    strix_context owner_ctx = nullptr;
    std::vector<strix_weights> retained;
    stx::DeviceWeights geometry{};
    stx::LinearCall call{};
    const stx::GroupWeights* table = nullptr;
    stx::FusedState fused{};   // null when one split suffices
    uint64_t state_bytes = 0;  // bytes of that state
    bool owner = false;        // owner-fold plan (no planes) instead of the split plan
    uint64_t xgs = 0, ygs = 0;
    hipStream_t stream{};
};

extern "C" {

strix_status strix_grouped_gemv_workspace_bytes(strix_context c, const strix_grouped_gemv_desc* d, uint64_t* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = 0;
    strix_status s = on_context_device(c);
    if (s != STRIX_SUCCESS) return s;
    Validated v;
    s = validate(c, d, v);
    if (s == STRIX_SUCCESS) *out = v.layout.bytes;
    return s;
}

strix_status strix_grouped_gemv_plan_create(strix_context c, const strix_grouped_gemv_desc* d,
                                            const strix_stream* stream, strix_grouped_gemv_plan* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = nullptr;
    strix_status s = on_context_device(c);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    s = borrowed_stream(c, stream, hs);
    if (s != STRIX_SUCCESS) return s;
    Validated v;
    s = validate(c, d, v);
    if (s != STRIX_SUCCESS) return s;
    if (d->workspace_bytes < v.layout.bytes) return STRIX_ERROR_INSUFFICIENT_BUFFER;
    if (!d->workspace || !Span(d->workspace, d->workspace_bytes).addressable() ||
        reinterpret_cast<uintptr_t>(d->workspace) % kWorkspaceAlign ||
        Span(d->workspace, d->workspace_bytes).meets(Span(d->input, v.input_bytes)) ||
        Span(d->workspace, d->workspace_bytes).meets(Span(d->output, v.output_bytes)))
        return STRIX_ERROR_INVALID_ARGUMENT;
    for (strix_weights w : v.weights)
        if (Span(d->workspace, d->workspace_bytes).meets(Span(w->base, w->bytes))) return STRIX_ERROR_INVALID_ARGUMENT;
    if ((s = device_resident(c, Span(d->input, v.input_bytes), 4)) != STRIX_SUCCESS) return s;
    if ((s = device_resident(c, Span(d->output, v.output_bytes), 4)) != STRIX_SUCCESS) return s;
    if ((s = device_resident(c, Span(d->workspace, d->workspace_bytes), kWorkspaceAlign)) != STRIX_SUCCESS) return s;

    auto* p = new (std::nothrow) strix_grouped_gemv_plan_impl;
    if (!p) return STRIX_ERROR_OUT_OF_MEMORY;
    std::vector<stx::GroupWeights> table;
    try {
        p->retained = v.weights;
        for (strix_weights w : v.weights) table.push_back({w->dev.trellis, w->dev.suh, w->dev.svh, w->dev.bias});
    } catch (...) {
        delete p;
        return STRIX_ERROR_OUT_OF_MEMORY;
    }
    char* base = static_cast<char*>(d->workspace);

    p->table = reinterpret_cast<const stx::GroupWeights*>(base + v.layout.table_offset);
    hipError_t e = hipMemcpyAsync(base + v.layout.table_offset, table.data(), table.size() * sizeof(table[0]),
                                  hipMemcpyHostToDevice, hs);
    if (e == hipSuccess && v.layout.state_bytes)
        e = init_fused_state(base + v.layout.state_offset, v.layout.state_bytes,
                             stx::fused_planes_offset(v.geometry, uint32_t(v.weights.size())), hs);
    const hipError_t done = hipStreamSynchronize(hs);
    if (e != hipSuccess || done != hipSuccess) {
        delete p;
        return status_of(e != hipSuccess ? e : done);
    }
    p->owner_ctx = c;
    p->geometry = v.geometry;
    p->stream = hs;
    p->xgs = v.xgs;
    p->ygs = v.ygs;
    p->call.x = d->input;
    p->call.y = d->output;
    p->call.rows = v.rows;
    p->call.x_row_stride = v.xrs;
    p->call.y_row_stride = v.yrs;
    p->call.alpha = 1.0f;
    p->call.beta = 0.0f;
    p->call.workspace = nullptr;
    if (v.layout.state_bytes) {
        p->fused = stx::fused_state_at(base + v.layout.state_offset, v.geometry, v.rows, uint32_t(v.weights.size()));
        p->state_bytes = v.layout.state_bytes;
    }
    const uint32_t G = uint32_t(v.weights.size());
    const bool want_owner = c->grouped_fold == 2 ||
                            (c->grouped_fold == 0 && stx::grouped_owner_preferred(v.geometry, G, v.rows));
    p->owner = want_owner && stx::gemv_owner_fits(v.geometry, v.rows);
    for (strix_weights w : v.weights) ++w->plans;
    *out = p;
    return STRIX_SUCCESS;
}

strix_status strix_grouped_gemv_plan_submit(strix_grouped_gemv_plan p) {
    if (!p) return STRIX_ERROR_INVALID_ARGUMENT;
    const strix_status s = on_context_device(p->owner_ctx);
    if (s != STRIX_SUCCESS) return s;
    stx::LinearCall call = p->call;
    if (p->owner)
        return status_of(stx::launch_gemv_owner(p->geometry, p->table, uint32_t(p->retained.size()), call, p->xgs,
                                               p->ygs, p->stream));
    call.gemv_poll_limit = p->owner_ctx->gemv_poll_limit;
    const stx::FusedState* st = p->fused.planes ? &p->fused : nullptr;
    if (!st && stx::gemv_shape(p->geometry.input, p->geometry.output, p->geometry.bits).splits > 1)
        return STRIX_ERROR_BACKEND;
    return status_of(stx::launch_gemv_grouped(p->geometry, p->table, uint32_t(p->retained.size()), call, p->xgs,
                                             p->ygs, st, p->stream));
}

strix_status strix_amd_grouped_plan_status(strix_grouped_gemv_plan p, uint32_t clear, uint32_t* flags) {
    if (flags) *flags = 0;
    if (!p || !flags) return STRIX_ERROR_INVALID_ARGUMENT;
    const strix_status s = on_context_device(p->owner_ctx);
    if (s != STRIX_SUCCESS) return s;
    return read_fused_status(p->fused, p->state_bytes, stx::fused_planes_offset(p->geometry, uint32_t(p->retained.size())),
                             p->stream, flags, clear);
}

strix_status strix_amd_grouped_plan_fold(strix_grouped_gemv_plan p, uint32_t* fold) {
    if (fold) *fold = 0;
    if (!p || !fold) return STRIX_ERROR_INVALID_ARGUMENT;
    *fold = p->owner ? 2u : 1u;
    return STRIX_SUCCESS;
}

strix_status strix_amd_set_grouped_fold(strix_context c, uint32_t fold) {
    const strix_status s = on_context_device(c);
    if (s != STRIX_SUCCESS) return s;
    if (fold > 2) return STRIX_ERROR_INVALID_ARGUMENT;
    c->grouped_fold = fold;
    return STRIX_SUCCESS;
}

strix_status strix_grouped_gemv_plan_destroy(strix_grouped_gemv_plan p) {
    if (!p) return STRIX_ERROR_INVALID_ARGUMENT;
    for (strix_weights w : p->retained) --w->plans;
    delete p;
    return STRIX_SUCCESS;
}

}  // extern "C"
