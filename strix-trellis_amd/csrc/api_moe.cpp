// Routed-expert block entry points (reference include/strix_trellis.h:458-523,
// src/tp_api.inc:103-198, 272-660; semantics docs/TP_RANK.md:52-140).
//
// Geometry: every expert has gate and up [I -> H] and down [H -> I], K2 or K3
// mul1 each, I and H multiples of 128 (the reference fixes I = 5120,
// H = 1152).  Routes are [rows][k] with k = route count / rows, 1 <= k <= 8
// and rows * k <= 64 (the reference fixes k = 6).  Host-route plans take the
// exact union of routed experts in any order; device-route plans take a bank
// of k..256 experts indexed by router id.  Both end up as the same device
// state: a bank table plus [rows][k] bank indices and scores that the kernels
// read on every submission.
//
// Plan-owned device memory (one allocation, freed by destroy): the bank
// table, the uploaded routes of a host-route plan, the arrival counters (zero
// between submissions), the split partial planes and the routes' FP16 gate/up
// core inputs [rows*k][2][I].  The caller's workspace
// holds hidden F32 [rows][k][H], as in the reference.  A split plan (the
// split creators) keeps its down planes in the caller's workspace instead,
// as P F32 [rows][k][S][I] from the first 256-byte boundary after hidden, the
// staged checkpoint the reference's split plans expose there, with the
// reference's four equal parts of the down input (moe_split_staged): every down
// (fused or staged core) writes P of each computed route, and the staged
// finish folds P as the caller leaves it.
#include "api_internal.hpp"
#include "moe.hpp"

#include <cmath>
#include <new>
#include <type_traits>
#include <unordered_map>

using namespace stx_api;

struct strix_tp_moe_plan_impl {
    strix_context owner = nullptr;
    std::vector<strix_weights> retained;
    hipStream_t stream{};
    stx::MoeArgs args{};
    void* device = nullptr;
    bool split = false;   // P in the caller's workspace; staged down entry points allowed
};

namespace {
uint64_t align_up(uint64_t v) { return (v + kWorkspaceAlign - 1) & ~(kWorkspaceAlign - 1); }

// F32 [rows][width] row view: unit channel stride, row stride >= width.
strix_status row_view_ok(const strix_tensor_desc& t, uint64_t width, uint64_t rows, uint64_t& stride,
                         uint64_t& bytes) {
    strix_status s = versioned(&t);
    if (s != STRIX_SUCCESS) return s;
    if (raw_enum(t.dtype) != STRIX_DTYPE_F32 || t.rank != 2 || t.shape[0] != rows || t.shape[1] != width ||
        t.strides[1] != 1 || t.strides[0] < width)
        return STRIX_ERROR_UNSUPPORTED_FORMAT;
    stride = t.strides[0];
    uint64_t span = 0;
    if (!checked_mul(rows - 1, stride, span) || span > UINT64_MAX - width || !checked_mul(span + width, 4, bytes) ||
        !Span(t.data, bytes).addressable())
        return STRIX_ERROR_INVALID_ARGUMENT;
    if (bytes > t.buffer_bytes) return STRIX_ERROR_INSUFFICIENT_BUFFER;
    if (!t.data || reinterpret_cast<uintptr_t>(t.data) % alignof(float)) return STRIX_ERROR_INVALID_ARGUMENT;
    return STRIX_SUCCESS;
}

bool touches(const void* p, uint64_t bytes, strix_weights w) { return Span(p, bytes).meets(Span(w->base, w->bytes)); }

struct MoeValidated {
    std::vector<stx::MoeExpert> bank;
    std::vector<strix_weights> retained;
    std::vector<uint32_t> ids;    // host plans: bank indices
    std::vector<float> scores;
    stx::MoeArgs args{};
    uint64_t x_bytes = 0, y_bytes = 0, hidden_bytes = 0;
    // Split plans: P at p_offset (hidden rounded up to 256 bytes), p_bytes long.
    uint64_t p_offset = 0, p_bytes = 0;
    uint64_t workspace_bytes(bool split) const { return split ? p_offset + p_bytes : hidden_bytes; }
};

// Checks shared by both descriptors: scalars, tensors, experts and geometry.
template <class D>
strix_status common_check(strix_context c, const D* d, uint64_t routes_per_row, MoeValidated& v) {
    if (!std::isfinite(d->alpha) || !std::isfinite(d->beta)) return STRIX_ERROR_INVALID_ARGUMENT;
    if (d->input.rank != 2 || d->input.shape[0] < 1 || d->input.shape[0] > STRIX_TP_MAX_ROWS)
        return STRIX_ERROR_UNSUPPORTED_FORMAT;
    const uint64_t rows = d->input.shape[0];
    if (!d->experts || d->expert_count < 1 || !Span(d->experts, d->expert_count * sizeof(strix_tp_expert_desc)).addressable())
        return STRIX_ERROR_INVALID_ARGUMENT;
    if (routes_per_row < 1 || routes_per_row > stx::MOE_MAX_TOPK || rows * routes_per_row > stx::MOE_MAX_ROUTES ||
        d->expert_count < routes_per_row)
        return STRIX_ERROR_INVALID_ARGUMENT;
    // Geometry from the first expert; every weight must match it.
    strix_status s = versioned(&d->experts[0]);
    if (s != STRIX_SUCCESS) return s;
    if (!d->experts[0].gate) return STRIX_ERROR_INVALID_ARGUMENT;
    const uint32_t I = d->experts[0].gate->dev.input, H = d->experts[0].gate->dev.output;
    const uint32_t gb = d->experts[0].gate->dev.bits, ub = d->experts[0].up ? d->experts[0].up->dev.bits : 0;
    const uint32_t db = d->experts[0].down ? d->experts[0].down->dev.bits : 0;
    s = row_view_ok(d->input, I, rows, v.args.x_stride, v.x_bytes);
    if (s != STRIX_SUCCESS) return s;
    s = row_view_ok(d->output, I, rows, v.args.y_stride, v.y_bytes);
    if (s != STRIX_SUCCESS) return s;
    if (Span(d->input.data, v.x_bytes).meets(Span(d->output.data, v.y_bytes))) return STRIX_ERROR_INVALID_ARGUMENT;
    v.bank.resize(d->expert_count);
    for (uint64_t i = 0; i < d->expert_count; ++i) {
        const strix_tp_expert_desc& e = d->experts[i];
        s = versioned(&e);
        if (s != STRIX_SUCCESS) return s;
        if (e.flags) return STRIX_ERROR_INVALID_ARGUMENT;
        const strix_weights ws[3] = {e.gate, e.up, e.down};
        const uint32_t want_in[3] = {I, I, H}, want_out[3] = {H, H, I}, want_bits[3] = {gb, ub, db};
        for (int p = 0; p < 3; ++p) {
            const strix_weights w = ws[p];
            if (!w || w->owner != c) return STRIX_ERROR_INVALID_ARGUMENT;
            const stx::DeviceWeights& dw = w->dev;
            if (dw.input != want_in[p] || dw.output != want_out[p] || dw.bits != want_bits[p] || dw.bits < 2 ||
                dw.bits > 3 || dw.codebook != 2 || dw.input % 128 || dw.output % 128)
                return STRIX_ERROR_UNSUPPORTED_FORMAT;
            if (touches(d->input.data, v.x_bytes, w) || touches(d->output.data, v.y_bytes, w))
                return STRIX_ERROR_INVALID_ARGUMENT;
            bool seen = false;
            for (strix_weights r : v.retained) seen = seen || r == w;
            if (!seen) {
                if (w->plans == UINT64_MAX) return STRIX_ERROR_OUT_OF_MEMORY;
                v.retained.push_back(w);
            }
        }
        v.bank[i] = {{e.gate->dev.trellis, e.gate->dev.suh, e.gate->dev.svh, e.gate->dev.bias},
                     {e.up->dev.trellis, e.up->dev.suh, e.up->dev.svh, e.up->dev.bias},
                     {e.down->dev.trellis, e.down->dev.suh, e.down->dev.svh, e.down->dev.bias}};
    }
    const stx::MoeSplit sgu = stx::moe_split(I, stx::MOE_GU_MAX_BPS), sd = stx::moe_split(H, stx::MOE_D_MAX_BPS);
    stx::MoeArgs& a = v.args;
    a.rows = uint32_t(rows);
    a.topk = uint32_t(routes_per_row);
    a.I = I;
    a.H = H;
    a.bank_count = uint32_t(d->expert_count);
    a.s_gu = sgu.splits;
    a.bps_gu = sgu.bps;
    a.s_d = sd.splits;
    a.bps_d = sd.bps;
    a.gate_bits = gb;
    a.up_bits = ub;
    a.down_bits = db;
    a.alpha = d->alpha;
    a.beta = d->beta;
    a.x = static_cast<const float*>(d->input.data);
    a.y = static_cast<float*>(d->output.data);
    v.hidden_bytes = rows * routes_per_row * H * sizeof(float);
    // A split plan's down runs the staged partition, whose planes are P.
    v.p_offset = align_up(v.hidden_bytes);
    v.p_bytes = rows * routes_per_row * stx::moe_split_staged(H).splits * uint64_t(I) * sizeof(float);
    return STRIX_SUCCESS;
}

// Host routes: exact union, ids distinct per row, finite non-negative scores.
strix_status host_check(strix_context c, const strix_tp_moe_desc* d, MoeValidated& v) {
    strix_status s = versioned(d);
    if (s != STRIX_SUCCESS) return s;
    if (d->input.rank != 2 || d->input.shape[0] < 1 || d->input.shape[0] > STRIX_TP_MAX_ROWS)
        return STRIX_ERROR_UNSUPPORTED_FORMAT;
    const uint64_t rows = d->input.shape[0];
    if (!d->route_ids || !d->route_scores || d->route_ids_count != d->route_scores_count ||
        d->route_ids_count % rows)
        return STRIX_ERROR_INVALID_ARGUMENT;
    const uint64_t k = d->route_ids_count / rows;
    s = common_check(c, d, k, v);
    if (s != STRIX_SUCCESS) return s;
    if (d->expert_count > rows * k || !Span(d->route_ids, d->route_ids_count * 4).addressable() ||
        !Span(d->route_scores, d->route_scores_count * 4).addressable())
        return STRIX_ERROR_INVALID_ARGUMENT;
    std::unordered_map<uint32_t, uint32_t> index;
    for (uint64_t i = 0; i < d->expert_count; ++i)
        if (!index.emplace(d->experts[i].expert_id, uint32_t(i)).second) return STRIX_ERROR_INVALID_ARGUMENT;
    std::vector<bool> used(d->expert_count, false);
    v.ids.resize(rows * k);
    v.scores.resize(rows * k);
    for (uint64_t r = 0; r < rows; ++r) {
        for (uint64_t q = 0; q < k; ++q) {
            const uint32_t id = d->route_ids[r * k + q];
            const float sc = d->route_scores[r * k + q];
            const auto it = index.find(id);
            if (it == index.end() || !std::isfinite(sc) || sc < 0.0f) return STRIX_ERROR_INVALID_ARGUMENT;
            for (uint64_t p = 0; p < q; ++p)
                if (d->route_ids[r * k + p] == id) return STRIX_ERROR_INVALID_ARGUMENT;
            v.ids[r * k + q] = it->second;
            v.scores[r * k + q] = sc;
            used[it->second] = true;
        }
    }
    for (bool u : used)
        if (!u) return STRIX_ERROR_INVALID_ARGUMENT;
    return STRIX_SUCCESS;
}

// Device routes: bank ids are positions, routes are device buffers [rows][k].
strix_status device_check(strix_context c, const strix_tp_moe_device_desc* d, MoeValidated& v) {
    strix_status s = versioned(d);
    if (s != STRIX_SUCCESS) return s;
    if (d->input.rank != 2 || d->input.shape[0] < 1 || d->input.shape[0] > STRIX_TP_MAX_ROWS)
        return STRIX_ERROR_UNSUPPORTED_FORMAT;
    const uint64_t rows = d->input.shape[0];
    if (!d->route_ids || !d->route_scores || d->route_ids_bytes != d->route_scores_bytes ||
        d->route_ids_bytes % (rows * 4))
        return STRIX_ERROR_INVALID_ARGUMENT;
    const uint64_t k = d->route_ids_bytes / (rows * 4);
    s = common_check(c, d, k, v);
    if (s != STRIX_SUCCESS) return s;
    if (d->expert_count > STRIX_TP_MAX_BANK_EXPERTS) return STRIX_ERROR_INVALID_ARGUMENT;
    for (uint64_t i = 0; i < d->expert_count; ++i)
        if (d->experts[i].expert_id != i) return STRIX_ERROR_INVALID_ARGUMENT;
    if ((s = device_resident(c, Span(d->route_ids, d->route_ids_bytes), 4)) != STRIX_SUCCESS) return s;
    if ((s = device_resident(c, Span(d->route_scores, d->route_scores_bytes), 4)) != STRIX_SUCCESS) return s;
    // Pairwise disjoint with the input and the output (the workspace is
    // checked with the others in create_plan), as the reference requires of
    // all five buffers (src/tp_api.inc:407-416): the kernels write hidden, P
    // and Y while later workgroups still read the routes.
    const Span ids(d->route_ids, d->route_ids_bytes), scores(d->route_scores, d->route_scores_bytes);
    const Span x(d->input.data, v.x_bytes), y(d->output.data, v.y_bytes);
    if (ids.meets(scores) || ids.meets(y) || scores.meets(y) || ids.meets(x) || scores.meets(x))
        return STRIX_ERROR_INVALID_ARGUMENT;
    v.args.ids = d->route_ids;
    v.args.scores = d->route_scores;
    return STRIX_SUCCESS;
}

// Caller workspace (hidden), device residency of X/Y, then the plan's own memory.
template <class D>
strix_status create_plan(strix_context c, const D* d, hipStream_t hs, MoeValidated& v, bool split,
                         strix_tp_moe_plan* out) {
    strix_status s;
    if (d->workspace_bytes < v.workspace_bytes(split)) return STRIX_ERROR_INSUFFICIENT_BUFFER;
    if (!d->workspace || !Span(d->workspace, d->workspace_bytes).addressable() ||
        reinterpret_cast<uintptr_t>(d->workspace) % kWorkspaceAlign ||
        Span(d->workspace, d->workspace_bytes).meets(Span(d->input.data, v.x_bytes)) ||
        Span(d->workspace, d->workspace_bytes).meets(Span(d->output.data, v.y_bytes)))
        return STRIX_ERROR_INVALID_ARGUMENT;
    for (strix_weights w : v.retained)
        if (touches(d->workspace, d->workspace_bytes, w)) return STRIX_ERROR_INVALID_ARGUMENT;
    if constexpr (std::is_same_v<D, strix_tp_moe_device_desc>) {
        const Span ws(d->workspace, d->workspace_bytes);
        if (ws.meets(Span(d->route_ids, d->route_ids_bytes)) || ws.meets(Span(d->route_scores, d->route_scores_bytes)))
            return STRIX_ERROR_INVALID_ARGUMENT;
    }
    if ((s = device_resident(c, Span(d->input.data, v.x_bytes), 4)) != STRIX_SUCCESS) return s;
    if ((s = device_resident(c, Span(d->output.data, v.y_bytes), 4)) != STRIX_SUCCESS) return s;
    if ((s = device_resident(c, Span(d->workspace, d->workspace_bytes), kWorkspaceAlign)) != STRIX_SUCCESS) return s;

    stx::MoeArgs& a = v.args;
    if (split) {
        const stx::MoeSplit sd = stx::moe_split_staged(a.H);
        a.s_d = sd.splits;
        a.bps_d = sd.bps;
    }
    const uint32_t routes = a.rows * a.topk;
    const uint64_t table_bytes = align_up(v.bank.size() * sizeof(stx::MoeExpert));
    const uint64_t route_bytes = v.ids.empty() ? 0 : 2 * align_up(uint64_t(routes) * 4);
    const uint64_t counter_words = stx::moe_counter_words(a.rows, routes, a.I, a.H);
    const uint64_t counter_bytes = align_up(counter_words * 4);
    const uint64_t partial_bytes = align_up(
        (split ? stx::moe_gate_up_partial_floats(routes, a.I, a.H) : stx::moe_partial_floats(routes, a.I, a.H)) * 4);
    const uint64_t input_bytes = align_up(stx::moe_core_input_bytes(routes, a.I));
    auto* p = new (std::nothrow) strix_tp_moe_plan_impl;
    if (!p) return STRIX_ERROR_OUT_OF_MEMORY;
    hipError_t e = hipMalloc(&p->device, table_bytes + route_bytes + counter_bytes + partial_bytes + input_bytes);
    if (e != hipSuccess) {
        delete p;
        return e == hipErrorOutOfMemory ? STRIX_ERROR_OUT_OF_MEMORY : status_of(e);
    }
    char* base = static_cast<char*>(p->device);
    a.bank = reinterpret_cast<const stx::MoeExpert*>(base);
    e = hipMemcpyAsync(base, v.bank.data(), v.bank.size() * sizeof(stx::MoeExpert), hipMemcpyHostToDevice, hs);
    char* cursor = base + table_bytes;
    if (!v.ids.empty()) {
        const uint64_t rb = align_up(uint64_t(routes) * 4);
        if (e == hipSuccess) e = hipMemcpyAsync(cursor, v.ids.data(), routes * 4, hipMemcpyHostToDevice, hs);
        if (e == hipSuccess) e = hipMemcpyAsync(cursor + rb, v.scores.data(), routes * 4, hipMemcpyHostToDevice, hs);
        a.ids = reinterpret_cast<const uint32_t*>(cursor);
        a.scores = reinterpret_cast<const float*>(cursor + rb);
        cursor += route_bytes;
    }
    a.c_gu = reinterpret_cast<uint32_t*>(cursor);
    a.c_d = a.c_gu + uint64_t(routes) * (a.H / 128);
    if (e == hipSuccess) e = stx::launch_fill_u32(a.c_gu, 0, counter_words, hs);
    cursor += counter_bytes;
    a.p_gu = reinterpret_cast<float*>(cursor);
    a.p_d = split ? reinterpret_cast<float*>(static_cast<char*>(d->workspace) + v.p_offset)
                  : a.p_gu + stx::moe_gate_up_partial_floats(routes, a.I, a.H);
    a.hidden = static_cast<float*>(d->workspace);
    cursor += partial_bytes;
    a.a_gu = reinterpret_cast<uint16_t*>(cursor);
    const hipError_t done = hipStreamSynchronize(hs);
    if (e != hipSuccess || done != hipSuccess) {
        (void)hipFree(p->device);
        delete p;
        return status_of(e != hipSuccess ? e : done);
    }
    p->owner = c;
    p->stream = hs;
    p->args = a;
    p->split = split;
    p->retained = v.retained;
    for (strix_weights w : v.retained) ++w->plans;
    *out = p;
    return STRIX_SUCCESS;
}

strix_status plan_ok(strix_tp_moe_plan p) {
    if (!p) return STRIX_ERROR_INVALID_ARGUMENT;
    return on_context_device(p->owner);
}

// The two creators of each route kind, with and without the split checkpoint.
strix_status create_host(strix_context c, const strix_tp_moe_desc* d, const strix_stream* stream, bool split,
                         strix_tp_moe_plan* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = nullptr;
    strix_status s = on_context_device(c);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    if ((s = borrowed_stream(c, stream, hs)) != STRIX_SUCCESS) return s;
    try {
        MoeValidated v;
        if ((s = host_check(c, d, v)) != STRIX_SUCCESS) return s;
        return create_plan(c, d, hs, v, split, out);
    } catch (...) {
        return STRIX_ERROR_OUT_OF_MEMORY;
    }
}

strix_status create_device(strix_context c, const strix_tp_moe_device_desc* d, const strix_stream* stream, bool split,
                           strix_tp_moe_plan* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = nullptr;
    strix_status s = on_context_device(c);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    if ((s = borrowed_stream(c, stream, hs)) != STRIX_SUCCESS) return s;
    try {
        MoeValidated v;
        if ((s = device_check(c, d, v)) != STRIX_SUCCESS) return s;
        return create_plan(c, d, hs, v, split, out);
    } catch (...) {
        return STRIX_ERROR_OUT_OF_MEMORY;
    }
}

strix_status host_workspace(strix_context c, const strix_tp_moe_desc* d, bool split, uint64_t* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = 0;
    strix_status s = on_context_device(c);
    if (s != STRIX_SUCCESS) return s;
    MoeValidated v;
    try {
        s = host_check(c, d, v);
    } catch (...) {
        return STRIX_ERROR_OUT_OF_MEMORY;
    }
    if (s == STRIX_SUCCESS) *out = v.workspace_bytes(split);
    return s;
}

// The staged down entry points need a split plan (P in the workspace).
strix_status split_plan_ok(strix_tp_moe_plan p) {
    const strix_status s = plan_ok(p);
    if (s != STRIX_SUCCESS) return s;
    return p->split ? STRIX_SUCCESS : STRIX_ERROR_INVALID_ARGUMENT;
}
}  // namespace

extern "C" {

void strix_tp_moe_desc_init(strix_tp_moe_desc* d) {
    if (!d) return;
    *d = strix_tp_moe_desc{};
    d->struct_size = sizeof(*d);
    d->abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.struct_size = d->output.struct_size = sizeof(strix_tensor_desc);
    d->input.abi_version = d->output.abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.dtype = d->output.dtype = STRIX_DTYPE_F32;
    d->alpha = 1.0f;
}

void strix_tp_moe_device_desc_init(strix_tp_moe_device_desc* d) {
    if (!d) return;
    *d = strix_tp_moe_device_desc{};
    d->struct_size = sizeof(*d);
    d->abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.struct_size = d->output.struct_size = sizeof(strix_tensor_desc);
    d->input.abi_version = d->output.abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.dtype = d->output.dtype = STRIX_DTYPE_F32;
    d->alpha = 1.0f;
}

strix_status strix_tp_moe_workspace_bytes(strix_context c, const strix_tp_moe_desc* d, uint64_t* out) {
    return host_workspace(c, d, false, out);
}

strix_status strix_tp_moe_plan_create(strix_context c, const strix_tp_moe_desc* d, const strix_stream* stream,
                                      strix_tp_moe_plan* out) {
    return create_host(c, d, stream, false, out);
}

strix_status strix_tp_moe_plan_create_device(strix_context c, const strix_tp_moe_device_desc* d,
                                             const strix_stream* stream, strix_tp_moe_plan* out) {
    return create_device(c, d, stream, false, out);
}

// Split plans run the same kernels; their down planes live in the caller's
// workspace (P after hidden), which the staged down entry points below use.
strix_status strix_tp_moe_split_workspace_bytes(strix_context c, const strix_tp_moe_desc* d, uint64_t* out) {
    return host_workspace(c, d, true, out);
}
strix_status strix_tp_moe_plan_create_split(strix_context c, const strix_tp_moe_desc* d, const strix_stream* stream,
                                            strix_tp_moe_plan* out) {
    return create_host(c, d, stream, true, out);
}
strix_status strix_tp_moe_plan_create_device_split(strix_context c, const strix_tp_moe_device_desc* d,
                                                   const strix_stream* stream, strix_tp_moe_plan* out) {
    return create_device(c, d, stream, true, out);
}

strix_status strix_amd_tp_moe_device_workspace_bytes(strix_context c, const strix_tp_moe_device_desc* d,
                                                     uint32_t split, uint64_t* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = 0;
    strix_status s = on_context_device(c);
    if (s != STRIX_SUCCESS) return s;
    MoeValidated v;
    try {
        s = device_check(c, d, v);
    } catch (...) {
        return STRIX_ERROR_OUT_OF_MEMORY;
    }
    if (s == STRIX_SUCCESS) *out = v.workspace_bytes(split != 0);
    return s;
}

// A8R is a different arithmetic identity (integer A8 groups); not provided.
strix_status strix_tp_moe_plan_create_a8r(strix_context, const strix_tp_moe_desc*, const strix_stream*,
                                          strix_tp_moe_plan* out) {
    if (out) *out = nullptr;
    return STRIX_ERROR_NOT_IMPLEMENTED;
}
strix_status strix_tp_moe_plan_create_device_a8r(strix_context, const strix_tp_moe_device_desc*, const strix_stream*,
                                                 strix_tp_moe_plan* out) {
    if (out) *out = nullptr;
    return STRIX_ERROR_NOT_IMPLEMENTED;
}

// Staged down of a split plan: the core alone (P of every computed route, each
// expert group streaming its weights once), the finish alone (from P as it is
// in the workspace), and the route-alone core (P again, one route per
// workgroup, without the expert grouping; same bits as the grouped core).
strix_status strix_tp_moe_plan_down_core(strix_tp_moe_plan p) {
    const strix_status s = split_plan_ok(p);
    if (s != STRIX_SUCCESS) return s;
    return status_of(stx::launch_moe_down_core(p->args, stx::kMoeDownCore, p->stream));
}
strix_status strix_tp_moe_plan_down_finish(strix_tp_moe_plan p) {
    const strix_status s = split_plan_ok(p);
    if (s != STRIX_SUCCESS) return s;
    return status_of(stx::launch_moe_down_finish(p->args, p->stream));
}
strix_status strix_tp_moe_plan_down_reference_core(strix_tp_moe_plan p) {
    const strix_status s = split_plan_ok(p);
    if (s != STRIX_SUCCESS) return s;
    return status_of(stx::launch_moe_down_core(p->args, stx::kMoeDownRouteCore, p->stream));
}

strix_status strix_tp_moe_plan_gate_up(strix_tp_moe_plan p) {
    const strix_status s = plan_ok(p);
    if (s != STRIX_SUCCESS) return s;
    return status_of(stx::launch_moe_gate_up(p->args, p->stream));
}

strix_status strix_tp_moe_plan_down(strix_tp_moe_plan p) {
    const strix_status s = plan_ok(p);
    if (s != STRIX_SUCCESS) return s;
    return status_of(stx::launch_moe_down(p->args, p->stream));
}

strix_status strix_tp_moe_plan_submit(strix_tp_moe_plan p) {
    const strix_status s = plan_ok(p);
    if (s != STRIX_SUCCESS) return s;
    hipError_t e = stx::launch_moe_gate_up(p->args, p->stream);
    if (e == hipSuccess) e = stx::launch_moe_down(p->args, p->stream);
    return status_of(e);
}

strix_status strix_amd_swiglu(strix_context c, const float* gate, const float* up, float* hidden, uint64_t count,
                              const strix_stream* stream) {
    strix_status s = on_context_device(c);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    if ((s = borrowed_stream(c, stream, hs)) != STRIX_SUCCESS) return s;
    if (!count) return STRIX_SUCCESS;
    uint64_t bytes = 0;
    if (!checked_mul(count, sizeof(float), bytes)) return STRIX_ERROR_INVALID_ARGUMENT;
    if ((s = device_resident(c, Span(gate, bytes), 4)) != STRIX_SUCCESS) return s;
    if ((s = device_resident(c, Span(up, bytes), 4)) != STRIX_SUCCESS) return s;
    if ((s = device_resident(c, Span(hidden, bytes), 4)) != STRIX_SUCCESS) return s;
    return status_of(stx::launch_moe_swiglu(gate, up, hidden, count, hs));
}

strix_status strix_tp_moe_plan_destroy(strix_tp_moe_plan p) {
    const strix_status s = plan_ok(p);
    if (s != STRIX_SUCCESS) return s;
    const hipError_t e = hipFree(p->device);
    if (e != hipSuccess) return status_of(e);
    for (strix_weights w : p->retained) --w->plans;
    delete p;
    return STRIX_SUCCESS;
}

}  // extern "C"
