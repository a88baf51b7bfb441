// Tensor-parallel dense plan entry points (reference include/strix_trellis.h:314-414,
// src/tp_api.inc:198-270, src/tp_split_api.inc, src/dense_r1_api.inc; semantics
// docs/TP_RANK.md:20-50).
//
// A rank's dense projection is one complete EXL3 linear (input stage, core,
// output stage with svh, bias, alpha/beta) on the rank's weight slice, R = 1..8
// F32 rows given as row views (unit channel stride, row stride >= width; an
// engine may point straight into half of its activation).  Here every plan
// variant runs the library's single-launch decode GEMV on those views, so
// each output row has exactly the bits of strix_gemv on that row:
//   * create / create_tiled (rows_per_block is accepted, 0 = R): one launch;
//   * create_splitk (SINGLE / TWO) and create_r1 (S4 / LEGACY): the same
//     launch -- the reference's K16-partition identities are its gfx1151
//     schedules, not a different operator;
//   * pair plans (q_a || kv: two weights, one input): one launch per member;
//   * SwiGLU plans: gate and up launches, then hidden = SwiGLU(gate, up) with
//     the routed-expert block's activation; the optional diagnostic buffers
//     receive the gate and up outputs.
// Workspaces: these plans keep their split partial planes in memory owned by
// the weights (as linear plans do), so every workspace query returns 0 and a
// caller workspace is optional.  Plans retain their weights.
#include "api_internal.hpp"
#include "moe.hpp"

#include <cmath>
#include <new>

using namespace stx_api;

namespace {
struct TpMember {
    strix_weights weights = nullptr;
    stx::LinearCall call{};
    stx::FusedState fused{};
    FusedBlock block{};
};
}  // namespace

struct strix_tp_dense_plan_impl {
    virtual ~strix_tp_dense_plan_impl() = default;   // pair handles are destroyed through this type too
    strix_context owner = nullptr;
    std::vector<TpMember> members;
    hipStream_t stream{};
    // SwiGLU plans: gate/up outputs (diagnostic buffers or plan-owned scratch)
    // and the activation's destination.
    bool swiglu = false;
    float* gate = nullptr;
    float* up = nullptr;
    float* hidden = nullptr;
    uint64_t rows = 0, width = 0, hidden_stride = 0;
    void* scratch = nullptr;
};
struct strix_tp_dense_pair_plan_impl : strix_tp_dense_plan_impl {};

namespace {

// F32 rank-1 [width] or rank-2 [rows][width] row view.
strix_status view_ok(const strix_tensor_desc& t, uint64_t width, uint32_t rank, uint64_t rows, uint64_t& stride,
                     uint64_t& bytes) {
    strix_status s = versioned(&t);
    if (s != STRIX_SUCCESS) return s;
    if (raw_enum(t.dtype) != STRIX_DTYPE_F32 || t.rank != rank) return STRIX_ERROR_UNSUPPORTED_FORMAT;
    if (rank == 1) {
        if (t.shape[0] != width || t.shape[1] || t.strides[0] != 1 || t.strides[1]) return STRIX_ERROR_UNSUPPORTED_FORMAT;
        stride = width;
    } else {
        if (t.shape[0] != rows || t.shape[1] != width || t.strides[1] != 1 || t.strides[0] < width)
            return STRIX_ERROR_UNSUPPORTED_FORMAT;
        stride = t.strides[0];
    }
    uint64_t span = 0;
    if (!checked_mul(rows - 1, stride, span) || span > UINT64_MAX - width || !checked_mul(span + width, 4, bytes) ||
        !Span(t.data, bytes).addressable())
        return STRIX_ERROR_INVALID_ARGUMENT;
    if (bytes > t.buffer_bytes) return STRIX_ERROR_INSUFFICIENT_BUFFER;
    if (!t.data || reinterpret_cast<uintptr_t>(t.data) % alignof(float)) return STRIX_ERROR_INVALID_ARGUMENT;
    return STRIX_SUCCESS;
}

bool touches(const void* p, uint64_t bytes, strix_weights w) { return Span(p, bytes).meets(Span(w->base, w->bytes)); }

// Row count of an input view: rank 1 is R = 1; rank 2 takes shape[0].
strix_status rows_of(const strix_tensor_desc& in, uint64_t& rows) {
    if (in.rank != 1 && in.rank != 2) return STRIX_ERROR_UNSUPPORTED_FORMAT;
    rows = in.rank == 1 ? 1 : in.shape[0];
    return rows >= 1 && rows <= STRIX_TP_MAX_ROWS ? STRIX_SUCCESS : STRIX_ERROR_UNSUPPORTED_FORMAT;
}

// One member: weights, input view (shared), output view, scalars.
strix_status member_ok(strix_context c, strix_weights w, const strix_tensor_desc& in, const strix_tensor_desc& out,
                       float alpha, float beta, uint64_t rows, TpMember& m, uint64_t& x_bytes, uint64_t& y_bytes) {
    if (!w || w->owner != c || !std::isfinite(alpha) || !std::isfinite(beta)) return STRIX_ERROR_INVALID_ARGUMENT;
    if (w->plans == UINT64_MAX) return STRIX_ERROR_OUT_OF_MEMORY;
    uint64_t xs = 0, ys = 0;
    strix_status s = view_ok(in, w->dev.input, in.rank, rows, xs, x_bytes);
    if (s != STRIX_SUCCESS) return s;
    s = view_ok(out, w->dev.output, in.rank, rows, ys, y_bytes);
    if (s != STRIX_SUCCESS) return s;
    if (Span(in.data, x_bytes).meets(Span(out.data, y_bytes)) || touches(in.data, x_bytes, w) || touches(out.data, y_bytes, w))
        return STRIX_ERROR_INVALID_ARGUMENT;
    if ((s = device_resident(c, Span(in.data, x_bytes), 4)) != STRIX_SUCCESS) return s;
    if ((s = device_resident(c, Span(out.data, y_bytes), 4)) != STRIX_SUCCESS) return s;
    m.weights = w;
    m.call.x = static_cast<const float*>(in.data);
    m.call.y = static_cast<float*>(out.data);
    m.call.rows = rows;
    m.call.x_row_stride = xs;
    m.call.y_row_stride = ys;
    m.call.alpha = alpha;
    m.call.beta = beta;
    return STRIX_SUCCESS;
}

// Single-launch state for every member (freed with its weights), zeroed.
strix_status arm(std::vector<TpMember>& members, hipStream_t hs) {
    for (TpMember& m : members) {
        const strix_status s = make_fused_state(m.weights, m.call.rows, hs, m.fused, m.block);
        if (s != STRIX_SUCCESS) return s;
    }
    return STRIX_SUCCESS;
}

template <class Plan>
strix_status finish_create(Plan* p, strix_context c, hipStream_t hs) {
    strix_status s = arm(p->members, hs);
    if (s != STRIX_SUCCESS) {
        for (TpMember& m : p->members) release_fused_state(m.weights, m.block);
        if (p->scratch) (void)hipFree(p->scratch);
        delete p;
        return s;
    }
    p->owner = c;
    p->stream = hs;
    for (TpMember& m : p->members) ++m.weights->plans;
    return STRIX_SUCCESS;
}

hipError_t launch_member(const TpMember& m, hipStream_t hs) {
    const stx::DeviceWeights& w = m.weights->dev;
    if (!m.fused.planes) return stx::launch_gemv(w, m.call, hs);
    stx::LinearCall call = m.call;
    call.gemv_poll_limit = m.weights->owner->gemv_poll_limit;
    return stx::launch_gemv_fused(w, call, m.fused, hs);
}

strix_status dense_create(strix_context c, const strix_matmul_desc* d, const strix_stream* stream,
                          uint32_t rows_per_block, bool workspace_allowed, strix_tp_dense_plan* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = nullptr;
    strix_status s = on_context_device(c);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    if ((s = borrowed_stream(c, stream, hs)) != STRIX_SUCCESS) return s;
    if ((s = versioned(d)) != STRIX_SUCCESS) return s;
    if (!workspace_allowed && (d->workspace || d->workspace_bytes)) return STRIX_ERROR_INVALID_ARGUMENT;
    uint64_t rows = 0;
    if ((s = rows_of(d->input, rows)) != STRIX_SUCCESS) return s;
    if (rows_per_block > rows) return STRIX_ERROR_INVALID_ARGUMENT;
    TpMember m;
    uint64_t xb = 0, yb = 0;
    if ((s = member_ok(c, d->weights, d->input, d->output, d->alpha, d->beta, rows, m, xb, yb)) != STRIX_SUCCESS)
        return s;
    auto* p = new (std::nothrow) strix_tp_dense_plan_impl;
    if (!p) return STRIX_ERROR_OUT_OF_MEMORY;
    try {
        p->members.push_back(m);
    } catch (...) {
        delete p;
        return STRIX_ERROR_OUT_OF_MEMORY;
    }
    if ((s = finish_create(p, c, hs)) != STRIX_SUCCESS) return s;
    *out = p;
    return STRIX_SUCCESS;
}

// Two members sharing one input (q_a || kv).
template <class Out>
strix_status pair_create(strix_context c, const strix_tp_dense_pair_desc* d, const strix_stream* stream, Out* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = nullptr;
    strix_status s = on_context_device(c);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    if ((s = borrowed_stream(c, stream, hs)) != STRIX_SUCCESS) return s;
    if ((s = versioned(d)) != STRIX_SUCCESS) return s;
    uint64_t rows = 0;
    if ((s = rows_of(d->input, rows)) != STRIX_SUCCESS) return s;
    if (d->rows_per_block > rows || d->strategy > STRIX_TP_SPLITK_TWO) return STRIX_ERROR_INVALID_ARGUMENT;
    TpMember m[2];
    uint64_t xb[2]{}, yb[2]{};
    for (int i = 0; i < 2; ++i) {
        const strix_tp_dense_pair_member& mm = d->member[i];
        if ((s = member_ok(c, mm.weights, d->input, mm.output, mm.alpha, mm.beta, rows, m[i], xb[i], yb[i])) !=
            STRIX_SUCCESS)
            return s;
    }
    if (m[0].weights->dev.input != m[1].weights->dev.input || Span(m[0].call.y, yb[0]).meets(Span(m[1].call.y, yb[1])) ||
        touches(m[0].call.y, yb[0], m[1].weights) || touches(m[1].call.y, yb[1], m[0].weights))
        return STRIX_ERROR_INVALID_ARGUMENT;
    auto* p = new (std::nothrow) strix_tp_dense_pair_plan_impl;
    if (!p) return STRIX_ERROR_OUT_OF_MEMORY;
    try {
        p->members.assign(m, m + 2);
    } catch (...) {
        delete p;
        return STRIX_ERROR_OUT_OF_MEMORY;
    }
    if ((s = finish_create(p, c, hs)) != STRIX_SUCCESS) return s;
    *out = p;
    return STRIX_SUCCESS;
}

strix_status plan_submit(strix_tp_dense_plan_impl* p) {
    if (!p) return STRIX_ERROR_INVALID_ARGUMENT;
    const strix_status s = on_context_device(p->owner);
    if (s != STRIX_SUCCESS) return s;
    for (const TpMember& m : p->members) {
        const hipError_t e = launch_member(m, p->stream);
        if (e != hipSuccess) return status_of(e);
    }
    if (p->swiglu) {
        for (uint64_t r = 0; r < p->rows; ++r) {
            const hipError_t e = stx::launch_moe_swiglu(p->gate + r * p->width, p->up + r * p->width,
                                                        p->hidden + r * p->hidden_stride, p->width, p->stream);
            if (e != hipSuccess) return status_of(e);
        }
    }
    return STRIX_SUCCESS;
}

strix_status plan_destroy(strix_tp_dense_plan_impl* p) {
    if (!p) return STRIX_ERROR_INVALID_ARGUMENT;
    const strix_status s = on_context_device(p->owner);
    if (s != STRIX_SUCCESS) return s;
    if (p->scratch) {
        const hipError_t e = hipFree(p->scratch);
        if (e != hipSuccess) return status_of(e);
    }
    for (TpMember& m : p->members) {
        release_fused_state(m.weights, m.block);
        --m.weights->plans;
    }
    delete p;
    return STRIX_SUCCESS;
}

strix_status zero_query(strix_status s, uint64_t* out) {
    if (out) *out = 0;
    return s;
}
}  // namespace

extern "C" {

void strix_tp_dense_pair_desc_init(strix_tp_dense_pair_desc* d) {
    if (!d) return;
    *d = strix_tp_dense_pair_desc{};
    d->struct_size = sizeof(*d);
    d->abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.struct_size = sizeof(strix_tensor_desc);
    d->input.abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.dtype = STRIX_DTYPE_F32;
    for (auto& m : d->member) {
        m.output.struct_size = sizeof(strix_tensor_desc);
        m.output.abi_version = STRIX_TRELLIS_ABI_VERSION;
        m.output.dtype = STRIX_DTYPE_F32;
        m.alpha = 1.0f;
    }
}

void strix_tp_swiglu_desc_init(strix_tp_swiglu_desc* d) {
    if (!d) return;
    *d = strix_tp_swiglu_desc{};
    d->struct_size = sizeof(*d);
    d->abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.struct_size = d->hidden_output.struct_size = sizeof(strix_tensor_desc);
    d->input.abi_version = d->hidden_output.abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.dtype = d->hidden_output.dtype = STRIX_DTYPE_F32;
}

strix_status strix_tp_dense_plan_create(strix_context c, const strix_matmul_desc* d, const strix_stream* stream,
                                        strix_tp_dense_plan* out) {
    return dense_create(c, d, stream, 0, false, out);
}

strix_status strix_tp_dense_plan_create_tiled(strix_context c, const strix_matmul_desc* d, const strix_stream* stream,
                                              uint32_t rows_per_block, strix_tp_dense_plan* out) {
    return dense_create(c, d, stream, rows_per_block, false, out);
}

strix_status strix_tp_dense_workspace_bytes(strix_context c, const strix_matmul_desc* d, uint32_t rows_per_block,
                                            uint64_t* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = 0;
    strix_status s = on_context_device(c);
    if (s != STRIX_SUCCESS) return s;
    if ((s = versioned(d)) != STRIX_SUCCESS) return s;
    uint64_t rows = 0;
    if ((s = rows_of(d->input, rows)) != STRIX_SUCCESS) return s;
    return zero_query(rows_per_block > rows ? STRIX_ERROR_INVALID_ARGUMENT : STRIX_SUCCESS, out);
}

strix_status strix_tp_dense_plan_create_splitk(strix_context c, const strix_matmul_desc* d, const strix_stream* stream,
                                               uint32_t rows_per_block, uint32_t strategy, strix_tp_dense_plan* out) {
    if (strategy > STRIX_TP_SPLITK_TWO) {
        if (out) *out = nullptr;
        return STRIX_ERROR_INVALID_ARGUMENT;
    }
    return dense_create(c, d, stream, rows_per_block, true, out);
}

strix_status strix_tp_dense_r1_workspace_bytes(strix_context c, const strix_matmul_desc* d, uint32_t rows_per_block,
                                               uint32_t identity, uint64_t* out) {
    if (identity > STRIX_DENSE_R1_LEGACY) return zero_query(STRIX_ERROR_INVALID_ARGUMENT, out);
    return strix_tp_dense_workspace_bytes(c, d, rows_per_block, out);
}

strix_status strix_tp_dense_plan_create_r1(strix_context c, const strix_matmul_desc* d, const strix_stream* stream,
                                           uint32_t rows_per_block, uint32_t identity, strix_tp_dense_plan* out) {
    if (identity > STRIX_DENSE_R1_LEGACY) {
        if (out) *out = nullptr;
        return STRIX_ERROR_INVALID_ARGUMENT;
    }
    return dense_create(c, d, stream, rows_per_block, true, out);
}

strix_status strix_tp_dense_plan_submit(strix_tp_dense_plan p) { return plan_submit(p); }
strix_status strix_tp_dense_plan_destroy(strix_tp_dense_plan p) { return plan_destroy(p); }

strix_status strix_tp_dense_pair_workspace_bytes(strix_context c, const strix_tp_dense_pair_desc* d, uint64_t* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = 0;
    strix_status s = on_context_device(c);
    if (s != STRIX_SUCCESS) return s;
    return versioned(d);
}

strix_status strix_tp_dense_pair_plan_create(strix_context c, const strix_tp_dense_pair_desc* d,
                                             const strix_stream* stream, strix_tp_dense_pair_plan* out) {
    return pair_create(c, d, stream, out);
}
strix_status strix_tp_dense_pair_plan_submit(strix_tp_dense_pair_plan p) { return plan_submit(p); }
strix_status strix_tp_dense_pair_plan_destroy(strix_tp_dense_pair_plan p) { return plan_destroy(p); }

strix_status strix_tp_dense_pair_r1_workspace_bytes(strix_context c, const strix_tp_dense_pair_desc* d,
                                                    uint32_t identity, uint64_t* out) {
    if (identity > STRIX_DENSE_R1_LEGACY) return zero_query(STRIX_ERROR_INVALID_ARGUMENT, out);
    return strix_tp_dense_pair_workspace_bytes(c, d, out);
}

strix_status strix_tp_dense_pair_plan_create_r1(strix_context c, const strix_tp_dense_pair_desc* d,
                                                const strix_stream* stream, uint32_t identity,
                                                strix_tp_dense_plan* out) {
    if (identity > STRIX_DENSE_R1_LEGACY) {
        if (out) *out = nullptr;
        return STRIX_ERROR_INVALID_ARGUMENT;
    }
    strix_tp_dense_pair_plan pair = nullptr;
    const strix_status s = pair_create(c, d, stream, &pair);
    if (out) *out = pair;
    return s;
}

strix_status strix_tp_swiglu_workspace_bytes(strix_context c, const strix_tp_swiglu_desc* d, uint64_t* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = 0;
    strix_status s = on_context_device(c);
    if (s != STRIX_SUCCESS) return s;
    return versioned(d);
}

// hidden[r][n] = SwiGLU(gate(x[r])[n], up(x[r])[n]), alpha 1, beta 0 per projection.
strix_status strix_tp_swiglu_plan_create(strix_context c, const strix_tp_swiglu_desc* d, const strix_stream* stream,
                                         strix_tp_swiglu_plan* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = nullptr;
    strix_status s = on_context_device(c);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    if ((s = borrowed_stream(c, stream, hs)) != STRIX_SUCCESS) return s;
    if ((s = versioned(d)) != STRIX_SUCCESS) return s;
    uint64_t rows = 0;
    if ((s = rows_of(d->input, rows)) != STRIX_SUCCESS) return s;
    if (d->rows_per_block > rows || d->strategy > STRIX_TP_SPLITK_TWO || !d->gate || !d->up ||
        d->gate->owner != c || d->up->owner != c)
        return STRIX_ERROR_INVALID_ARGUMENT;
    const stx::DeviceWeights &g = d->gate->dev, &u = d->up->dev;
    if (g.input != u.input || g.output != u.output) return STRIX_ERROR_UNSUPPORTED_FORMAT;
    const uint64_t H = g.output;
    uint64_t hs_stride = 0, hb = 0;
    if ((s = view_ok(d->hidden_output, H, d->input.rank, rows, hs_stride, hb)) != STRIX_SUCCESS) return s;
    if ((s = device_resident(c, Span(d->hidden_output.data, hb), 4)) != STRIX_SUCCESS) return s;
    const uint64_t diag = rows * H * 4;
    const bool with_diag = d->diagnostic_gate || d->diagnostic_up;
    if (with_diag) {
        if (!d->diagnostic_gate || !d->diagnostic_up || d->diagnostic_bytes < diag ||
            Span(d->diagnostic_gate, diag).meets(Span(d->diagnostic_up, diag)))
            return STRIX_ERROR_INVALID_ARGUMENT;
        if ((s = device_resident(c, Span(d->diagnostic_gate, diag), 4)) != STRIX_SUCCESS) return s;
        if ((s = device_resident(c, Span(d->diagnostic_up, diag), 4)) != STRIX_SUCCESS) return s;
    }
    auto* p = new (std::nothrow) strix_tp_dense_pair_plan_impl;
    if (!p) return STRIX_ERROR_OUT_OF_MEMORY;
    if (with_diag) {
        p->gate = d->diagnostic_gate;
        p->up = d->diagnostic_up;
    } else {
        const hipError_t e = hipMalloc(&p->scratch, 2 * diag);
        if (e != hipSuccess) {
            delete p;
            return e == hipErrorOutOfMemory ? STRIX_ERROR_OUT_OF_MEMORY : status_of(e);
        }
        p->gate = static_cast<float*>(p->scratch);
        p->up = p->gate + rows * H;
    }
    // Gate and up write contiguous [rows][H] F32 (the diagnostic layout).
    strix_tensor_desc gview{}, uview{};
    for (strix_tensor_desc* t : {&gview, &uview}) {
        t->struct_size = sizeof(strix_tensor_desc);
        t->abi_version = STRIX_TRELLIS_ABI_VERSION;
        t->dtype = STRIX_DTYPE_F32;
        t->rank = d->input.rank;
        t->shape[0] = d->input.rank == 1 ? H : rows;
        t->shape[1] = d->input.rank == 1 ? 0 : H;
        t->strides[0] = d->input.rank == 1 ? 1 : H;
        t->strides[1] = d->input.rank == 1 ? 0 : 1;
        t->buffer_bytes = diag;
    }
    gview.data = p->gate;
    uview.data = p->up;
    TpMember m[2];
    uint64_t xb = 0, yb = 0;
    s = member_ok(c, d->gate, d->input, gview, 1.0f, 0.0f, rows, m[0], xb, yb);
    if (s == STRIX_SUCCESS) s = member_ok(c, d->up, d->input, uview, 1.0f, 0.0f, rows, m[1], xb, yb);
    if (s == STRIX_SUCCESS && (Span(d->hidden_output.data, hb).meets(Span(d->input.data, xb)) ||
                               Span(d->hidden_output.data, hb).meets(Span(p->gate, diag)) ||
                               Span(d->hidden_output.data, hb).meets(Span(p->up, diag))))
        s = STRIX_ERROR_INVALID_ARGUMENT;
    if (s == STRIX_SUCCESS) {
        try {
            p->members.assign(m, m + 2);
        } catch (...) {
            s = STRIX_ERROR_OUT_OF_MEMORY;
        }
    }
    if (s != STRIX_SUCCESS) {
        if (p->scratch) (void)hipFree(p->scratch);
        delete p;
        return s;
    }
    p->swiglu = true;
    p->hidden = static_cast<float*>(d->hidden_output.data);
    p->rows = rows;
    p->width = H;
    p->hidden_stride = hs_stride;
    if ((s = finish_create(p, c, hs)) != STRIX_SUCCESS) return s;
    *out = p;
    return STRIX_SUCCESS;
}

strix_status strix_tp_swiglu_plan_submit(strix_tp_swiglu_plan p) { return plan_submit(p); }
strix_status strix_tp_swiglu_plan_destroy(strix_tp_swiglu_plan p) { return plan_destroy(p); }

}  // extern "C"
