// MI355X extensions (include/strix_trellis_amd.h): stage checkpoints for the
// parity tests, the decomposition queries that fix the cores' accumulation
// orders, test hooks, the single-launch status query and the call-floor read.
// None has a counterpart in the reference ABI.  Every entry point checks the
// calling device, the stream and the device residence of its buffers as the
// ABI calls do, and only enqueues work.
#include <climits>
#include <cmath>

#include "api_internal.hpp"

using namespace stx_api;

namespace {

// Calling device and stream of a weights handle's context.
strix_status weights_call(strix_weights w, const strix_stream* stream, hipStream_t& hs) {
    if (!w) return STRIX_ERROR_INVALID_ARGUMENT;
    Rules r;
    r.then([&] { return on_context_device(w->owner); }).then([&] { return borrowed_stream(w->owner, stream, hs); });
    return r.status();
}

// rows x per_row bytes, rows bounded like a GEMM call's.
strix_status row_bytes(uint64_t rows, uint64_t per_row, uint64_t& bytes) {
    return rows <= INT_MAX && checked_mul(rows, per_row, bytes) ? STRIX_SUCCESS : STRIX_ERROR_UNSUPPORTED_FORMAT;
}

}  // namespace

extern "C" {

strix_status strix_amd_decode(strix_weights w, void* q, uint64_t q_bytes, const strix_stream* stream) {
    hipStream_t hs{};
    Rules r;
    r.then([&] { return weights_call(w, stream, hs); });
    if (!r.held()) return r.status();
    const uint64_t need = uint64_t(w->dev.input) * w->dev.output * 2;
    r.need(q_bytes >= need, STRIX_ERROR_INSUFFICIENT_BUFFER)
        .then([&] { return device_resident(w->owner, Span(q, need), 4); })
        .then([&] { return status_of(stx::launch_decode(w->dev, static_cast<_Float16*>(q), hs)); });
    return r.status();
}

strix_status strix_amd_input_stage(strix_weights w, const float* x, uint64_t rows, void* a, uint64_t a_bytes,
                                   const strix_stream* stream) {
    hipStream_t hs{};
    uint64_t need = 0;
    Rules r;
    r.then([&] { return weights_call(w, stream, hs); });
    if (!r.held()) return r.status();
    r.then([&] { return row_bytes(rows, uint64_t(w->dev.input) * 2, need); })
        .need(a_bytes >= need, STRIX_ERROR_INSUFFICIENT_BUFFER)
        .then([&] { return device_resident(w->owner, Span(x, need * 2), 4); })
        .then([&] { return device_resident(w->owner, Span(a, need), 4); })
        .then([&] { return status_of(stx::launch_input_stage(w->dev, x, rows, static_cast<_Float16*>(a), hs)); });
    return r.status();
}

strix_status strix_amd_output_stage(strix_weights w, const float* core, uint64_t rows, float* y, uint64_t y_bytes,
                                    float alpha, float beta, const strix_stream* stream) {
    hipStream_t hs{};
    uint64_t need = 0;
    Rules r;
    r.need(w && std::isfinite(alpha) && std::isfinite(beta), STRIX_ERROR_INVALID_ARGUMENT)
        .then([&] { return weights_call(w, stream, hs); });
    if (!r.held()) return r.status();
    r.then([&] { return row_bytes(rows, uint64_t(w->dev.output) * 4, need); })
        .need(y_bytes >= need, STRIX_ERROR_INSUFFICIENT_BUFFER)
        .need(!Span(core, need).meets(Span(y, need)), STRIX_ERROR_INVALID_ARGUMENT)
        .then([&] { return device_resident(w->owner, Span(core, need), 4); })
        .then([&] { return device_resident(w->owner, Span(y, need), 4); })
        .then([&] { return status_of(stx::launch_output_stage(w->dev, core, rows, y, alpha, beta, hs)); });
    return r.status();
}

strix_status strix_amd_gemv_shape(strix_weights w, uint32_t* bps, uint32_t* splits) {
    if (bps) *bps = 0;
    if (splits) *splits = 0;
    if (!w || !bps || !splits) return STRIX_ERROR_INVALID_ARGUMENT;
    const stx::GemvShape sh = stx::gemv_shape(w->dev.input, w->dev.output, w->dev.bits);
    *bps = sh.bps;
    *splits = sh.splits;
    return STRIX_SUCCESS;
}

strix_status strix_amd_gemm_splits(strix_weights w, uint64_t rows, uint32_t* splits) {
    if (splits) *splits = 0;
    if (!w || !splits) return STRIX_ERROR_INVALID_ARGUMENT;
    *splits = stx::gemm_split_count(w->dev, rows ? rows : 1);
    return STRIX_SUCCESS;
}

strix_status strix_amd_plan_launches(strix_linear_plan p, uint32_t* launches) {
    if (launches) *launches = 0;
    if (!p || !launches) return STRIX_ERROR_INVALID_ARGUMENT;
    *launches = p->launches;
    return STRIX_SUCCESS;
}

strix_status strix_amd_set_gemm_handoff(strix_context c, uint32_t always_take_over) {
    const strix_status device = on_context_device(c);
    if (device == STRIX_SUCCESS) c->gemm_handoff_poll = always_take_over ? UINT32_MAX : 4096u;
    return device;
}

strix_status strix_amd_set_gemv_poll_limit(strix_context c, uint32_t poll_limit) {
    const strix_status device = on_context_device(c);
    if (device == STRIX_SUCCESS) c->gemv_poll_limit = poll_limit;
    return device;
}

strix_status strix_amd_set_plan_state_reuse(strix_context c, uint32_t enable) {
    const strix_status device = on_context_device(c);
    if (device == STRIX_SUCCESS) c->reuse_plan_state = enable != 0;
    return device;
}

strix_status strix_amd_plan_status(strix_linear_plan p, uint32_t clear, uint32_t* flags) {
    if (flags) *flags = 0;
    if (!p || !flags) return STRIX_ERROR_INVALID_ARGUMENT;
    const strix_status device = on_context_device(p->owner);
    if (device != STRIX_SUCCESS) return device;
    return read_fused_status(p->fused, p->block.bytes, stx::fused_planes_offset(p->weights->dev, 1), p->stream, flags,
                             clear);
}

strix_status strix_amd_stream_read_shaped(strix_context c, const void* src, uint64_t bytes, uint32_t workgroups,
                                          uint32_t threads, uint32_t depth, uint32_t* sink,
                                          const strix_stream* stream) {
    hipStream_t hs{};
    Rules r;
    r.then([&] { return on_context_device(c); })
        .then([&] { return borrowed_stream(c, stream, hs); })
        .need(workgroups && bytes && bytes % (16ull * workgroups) == 0 && bytes / workgroups < (uint64_t(1) << 31) &&
                  stx::stream_read_shape_ok(threads, depth),
              STRIX_ERROR_INVALID_ARGUMENT)
        .then([&] { return device_resident(c, Span(src, bytes), 16); })
        .then([&] { return device_resident(c, Span(sink, uint64_t(workgroups) * 4), 4); })
        .then([&] { return status_of(stx::launch_stream_read(src, bytes, workgroups, threads, depth, sink, hs)); });
    return r.status();
}

strix_status strix_amd_stream_read(strix_context c, const void* src, uint64_t bytes, uint32_t workgroups,
                                   uint32_t* sink, const strix_stream* stream) {
    return strix_amd_stream_read_shaped(c, src, bytes, workgroups, 256, 4, sink, stream);
}

}  // extern "C"
