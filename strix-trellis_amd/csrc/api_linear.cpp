// Linear calls: the workspace query, strix_gemv / strix_gemm, prepared linear
// plans (with the single-launch GEMV state they own) and pre-routed grouped
// MoE submissions.
//
// Contract: the reference ABI's "Buffer validation and workspace", "Prepared
// linear plans" and "Pre-routed grouped MoE" (include/strix_trellis.h and its
// docs/API.md).  A call is validated in two steps (describe_linear: the host
// descriptor; place_linear: workspace and device residence), then enqueued.
// Plans run both steps once at creation and nothing but the device check at
// submission.
#include <new>

#include "api_internal.hpp"

using namespace stx_api;

namespace stx_api {

hipError_t init_fused_state(void* base, uint64_t bytes, uint64_t planes_offset, hipStream_t hs) {
    uint32_t* words = static_cast<uint32_t*>(base);
    const hipError_t e = stx::launch_fill_u32(words, 0u, planes_offset / 4, hs);
    if (e != hipSuccess) return e;
    return stx::launch_fill_u32(words + planes_offset / 4, stx::GEMV_PLANE_EMPTY, (bytes - planes_offset) / 4, hs);
}

strix_status make_fused_state(strix_weights w, uint64_t rows, hipStream_t hs, stx::FusedState& out,
                              FusedBlock& block) {
    out = {};
    block = {};
    const uint64_t bytes = stx::fused_state_bytes(w->dev, rows, 1);
    if (!bytes) return STRIX_SUCCESS;
    void* state = nullptr;
    bool reused = false;
    for (auto it = w->idle_states.begin(); w->owner->reuse_plan_state && it != w->idle_states.end(); ++it) {
        if (it->second == bytes) {
            state = it->first;
            w->idle_states.erase(it);
            reused = true;
            break;
        }
    }
    hipError_t e = reused ? hipSuccess : hipMalloc(&state, bytes);
    if (e == hipSuccess) e = init_fused_state(state, bytes, stx::fused_planes_offset(w->dev, 1), hs);
    if (e == hipSuccess) e = hipStreamSynchronize(hs);
    if (e == hipSuccess && !reused) {
        try {
            w->counter_arrays.push_back(state);   // released with the weights
        } catch (...) {
            e = hipErrorOutOfMemory;
        }
    }
    if (e != hipSuccess) {
        FusedBlock back{state, bytes};
        if (reused)
            release_fused_state(w, back);   // still owned by the weights; initialised again on reuse
        else if (state)
            (void)hipFree(state);
        return status_of(e);
    }
    block = {state, bytes};
    out = stx::fused_state_at(state, w->dev, rows, 1);
    return STRIX_SUCCESS;
}

void release_fused_state(strix_weights w, FusedBlock& block) {
    if (!block.base) return;
    try {
        w->idle_states.emplace_back(block.base, block.bytes);
    } catch (...) {
        // not reusable then; it is still freed with the weights
    }
    block = {};
}

strix_status read_fused_status(const stx::FusedState& st, uint64_t bytes, uint64_t planes_offset, hipStream_t hs,
                               uint32_t* flags, uint32_t clear) {
    *flags = 0;
    if (!st.status) return STRIX_SUCCESS;
    uint32_t word = 0;
    hipError_t e = hipMemcpyAsync(&word, st.status, sizeof(word), hipMemcpyDeviceToHost, hs);
    if (e == hipSuccess && clear) e = init_fused_state(st.status, bytes, planes_offset, hs);
    if (e == hipSuccess) e = hipStreamSynchronize(hs);
    if (e != hipSuccess) return status_of(e);
    *flags = word;
    return STRIX_SUCCESS;
}

}  // namespace stx_api

namespace {

// One direct call: GEMV entry point (rows <= 8) or GEMM entry point (rank 2).
strix_status direct(strix_context c, const strix_matmul_desc* d, const strix_stream* stream, bool gemv) {
    hipStream_t hs{};
    LinearExtent e;
    Rules r;
    r.then([&] { return on_context_device(c); })
        .then([&] { return borrowed_stream(c, stream, hs); })
        .then([&] { return describe_linear(c, d, e); });
    if (!r.held()) return r.status();
    r.need(gemv ? e.rows <= 8 : d->input.rank == 2, STRIX_ERROR_UNSUPPORTED_FORMAT)
        .then([&] { return place_linear(c, *d, e, Span(d->workspace, d->workspace_bytes)); });
    if (!r.held() || !e.rows) return r.status();
    return status_of(stx::launch_linear(d->weights->dev, to_call(*d, e.rows, d->workspace), !gemv, hs));
}

// The groups of a pre-routed MoE submission: each an ordinary call without a
// workspace of its own; slices pairwise disjoint across groups (inputs,
// outputs and every group's weights).  `need` = the largest requirement.
strix_status check_groups(strix_context c, const strix_grouped_moe_desc* d, uint64_t& need) {
    need = 0;
    Rules r;
    r.then([&] { return versioned(d); });
    if (!r.held()) return r.status();
    uint64_t table = 0;
    r.need(checked_mul(d->group_count, sizeof(strix_matmul_desc), table) && table <= SIZE_MAX &&
               (!d->group_count || d->groups) && Span(d->groups, table).addressable(),
           STRIX_ERROR_INVALID_ARGUMENT);
    std::vector<LinearExtent> seen;
    for (uint64_t i = 0; i < d->group_count && r.held(); ++i) {
        const strix_matmul_desc& g = d->groups[i];
        LinearExtent e;
        r.need(!g.workspace && !g.workspace_bytes, STRIX_ERROR_INVALID_ARGUMENT)
            .then([&] { return describe_linear(c, &g, e); });
        if (!r.held()) break;
        if (e.workspace > need) need = e.workspace;
        const Span gw(g.weights->base, g.weights->bytes);
        for (uint64_t j = 0; j < i && r.held(); ++j) {
            const strix_matmul_desc& h = d->groups[j];
            const LinearExtent& f = seen[j];
            const Span hw(h.weights->base, h.weights->bytes);
            const bool apart = !e.x.meets(f.x) && !e.x.meets(f.y) && !e.y.meets(f.x) && !e.y.meets(f.y) &&
                               !e.x.meets(hw) && !f.x.meets(gw) && !e.y.meets(hw) && !f.y.meets(gw);
            r.need(apart, STRIX_ERROR_INVALID_ARGUMENT);
        }
        try {
            seen.push_back(e);
        } catch (...) {
            return STRIX_ERROR_OUT_OF_MEMORY;
        }
    }
    return r.status();
}

}  // namespace

extern "C" {

strix_status strix_matmul_workspace_bytes(strix_context c, const strix_matmul_desc* d, uint64_t* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = 0;
    LinearExtent e;
    Rules r;
    r.then([&] { return on_context_device(c); }).then([&] { return describe_linear(c, d, e); });
    if (r.held()) *out = e.workspace;
    return r.status();
}

strix_status strix_gemv(strix_context c, const strix_matmul_desc* d, const strix_stream* stream) {
    return direct(c, d, stream, true);
}

strix_status strix_gemm(strix_context c, const strix_matmul_desc* d, const strix_stream* stream) {
    return direct(c, d, stream, false);
}

// A GEMV plan whose layer splits its input runs as one launch on its own
// single-launch state (owned by the weights, like the reference's completion
// counters, so captured graphs outlive the plan).
strix_status strix_linear_plan_create(strix_context c, const strix_matmul_desc* d, const strix_stream* stream,
                                      uint32_t operation, strix_linear_plan* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = nullptr;
    const bool gemm = operation == STRIX_OPERATION_GEMM;
    hipStream_t hs{};
    LinearExtent e;
    Rules r;
    r.need(operation == STRIX_OPERATION_GEMV || gemm, STRIX_ERROR_INVALID_ARGUMENT)
        .then([&] { return on_context_device(c); })
        .then([&] { return borrowed_stream(c, stream, hs); })
        .then([&] { return describe_linear(c, d, e); });
    if (!r.held()) return r.status();
    r.need(gemm ? d->input.rank == 2 : e.rows <= 8, STRIX_ERROR_UNSUPPORTED_FORMAT)
        .then([&] { return place_linear(c, *d, e, Span(d->workspace, d->workspace_bytes)); })
        .need(d->weights->plans != UINT64_MAX, STRIX_ERROR_OUT_OF_MEMORY);
    if (!r.held()) return r.status();
    auto* plan = new (std::nothrow) strix_linear_plan_impl;
    if (!plan) return STRIX_ERROR_OUT_OF_MEMORY;
    strix_weights w = d->weights;
    plan->owner = c;
    plan->weights = w;
    plan->stream = hs;
    plan->gemm = gemm;
    plan->call = to_call(*d, e.rows, d->workspace);
    if (!gemm && e.rows) {
        const strix_status s = make_fused_state(w, e.rows, hs, plan->fused, plan->block);
        if (s != STRIX_SUCCESS) {
            delete plan;
            return s;
        }
    }
    plan->launches = e.rows ? stx::linear_launch_count(w->dev, e.rows, gemm, plan->fused.planes != nullptr) : 0;
    ++w->plans;
    *out = plan;
    return STRIX_SUCCESS;
}

strix_status strix_linear_plan_submit(strix_linear_plan p) {
    if (!p) return STRIX_ERROR_INVALID_ARGUMENT;
    const strix_status device = on_context_device(p->owner);
    if (device != STRIX_SUCCESS || !p->call.rows) return device;
    const stx::DeviceWeights& w = p->weights->dev;
    if (p->gemm || !p->fused.planes) return status_of(stx::launch_linear(w, p->call, p->gemm, p->stream));
    stx::LinearCall call = p->call;
    call.gemv_poll_limit = p->owner->gemv_poll_limit;
    return status_of(stx::launch_gemv_fused(w, call, p->fused, p->stream));
}

strix_status strix_linear_plan_destroy(strix_linear_plan p) {
    if (!p) return STRIX_ERROR_INVALID_ARGUMENT;
    release_fused_state(p->weights, p->block);
    --p->weights->plans;
    delete p;
    return STRIX_SUCCESS;
}

strix_status strix_grouped_moe_workspace_bytes(strix_context c, const strix_grouped_moe_desc* d, uint64_t* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = 0;
    uint64_t need = 0;
    Rules r;
    r.then([&] { return on_context_device(c); }).then([&] { return check_groups(c, d, need); });
    if (r.held()) *out = need;
    return r.status();
}

// Every group is validated (including the shared workspace against each)
// before the first is enqueued; then they run in order on the stream, reusing
// the workspace in stream order.
strix_status strix_grouped_moe(strix_context c, const strix_grouped_moe_desc* d, const strix_stream* stream) {
    hipStream_t hs{};
    uint64_t need = 0;
    Rules r;
    r.then([&] { return on_context_device(c); })
        .then([&] { return borrowed_stream(c, stream, hs); })
        .then([&] { return check_groups(c, d, need); });
    if (!r.held()) return r.status();
    const Span ws(d->workspace, d->workspace_bytes);
    r.need(ws.size >= need, STRIX_ERROR_INSUFFICIENT_BUFFER)
        .need(ws.addressable() && (!ws.size || (ws.at && ws.aligned(kWorkspaceAlign))), STRIX_ERROR_INVALID_ARGUMENT);
    for (uint64_t i = 0; i < d->group_count && r.held(); ++i) {
        LinearExtent e;
        r.then([&] { return describe_linear(c, &d->groups[i], e); })
            .then([&] { return place_linear(c, d->groups[i], e, ws); });
    }
    for (uint64_t i = 0; i < d->group_count && r.held(); ++i) {
        const strix_matmul_desc& g = d->groups[i];
        const uint64_t rows = g.input.rank == 1 ? 1 : g.input.shape[0];
        if (rows)
            r.then([&] {
                return status_of(stx::launch_linear(g.weights->dev, to_call(g, rows, d->workspace), rows > 8, hs));
            });
    }
    return r.status();
}

}  // extern "C"
