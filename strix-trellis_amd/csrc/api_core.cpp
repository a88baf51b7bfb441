// C ABI core: status mapping and strings, descriptor initialisers, contexts,
// and the checks every entry point shares (calling device, stream, device
// residence of buffers, the tensors and buffers of one linear call).
//
// The rules are the reference ABI's contract (include/strix_trellis.h and its
// docs/API.md: "Lifecycle, device and streams", "Buffer validation and
// workspace", "Errors and validation"); the device is a gfx950 with wave64,
// where the reference accepts only gfx1151 with wave32.
#include <climits>
#include <cmath>
#include <new>

#include "api_internal.hpp"

namespace stx_api {

strix_status status_of(hipError_t e) {
    switch (e) {
        case hipSuccess: return STRIX_SUCCESS;
        case hipErrorOutOfMemory: return STRIX_ERROR_OUT_OF_MEMORY;
        default: return STRIX_ERROR_BACKEND;
    }
}

strix_status on_context_device(strix_context c) {
    if (!c) return STRIX_ERROR_INVALID_ARGUMENT;
    int current = -1;
    const hipError_t e = hipGetDevice(&current);
    if (e != hipSuccess) return status_of(e);
    return current == c->device ? STRIX_SUCCESS : STRIX_ERROR_INVALID_ARGUMENT;
}

strix_status borrowed_stream(strix_context c, const strix_stream* s, hipStream_t& out) {
    const strix_status header = versioned(s);
    if (header != STRIX_SUCCESS) return header;
    out = static_cast<hipStream_t>(s->hip_stream);
    if (!out) return STRIX_SUCCESS;   // the device's default stream
    hipDevice_t owner = -1;
    unsigned flags = 0;
    const bool known = hipStreamGetDevice(out, &owner) == hipSuccess && hipStreamGetFlags(out, &flags) == hipSuccess;
    return known && owner == c->device ? STRIX_SUCCESS : STRIX_ERROR_INVALID_ARGUMENT;
}

strix_status device_resident(strix_context c, Span span, uint64_t align) {
    if (!span.size) return STRIX_SUCCESS;
    if (!span.at || !span.addressable() || !span.aligned(align)) return STRIX_ERROR_INVALID_ARGUMENT;
    hipPointerAttribute_t attr{};
    if (hipPointerGetAttributes(&attr, span.ptr()) != hipSuccess) return STRIX_ERROR_INVALID_ARGUMENT;
    if (attr.type != hipMemoryTypeDevice || attr.device != c->device || attr.isManaged)
        return STRIX_ERROR_INVALID_ARGUMENT;
    hipDeviceptr_t base{};
    size_t extent = 0;
    if (hipMemGetAddressRange(&base, &extent, span.ptr()) != hipSuccess) return STRIX_ERROR_INVALID_ARGUMENT;
    const Span allocation(base, extent);
    const bool inside = span.at >= allocation.at && span.at - allocation.at <= extent &&
                        span.size <= extent - (span.at - allocation.at);
    return inside ? STRIX_SUCCESS : STRIX_ERROR_INSUFFICIENT_BUFFER;
}

strix_status tensor_extent(const strix_tensor_desc& t, uint64_t width, uint32_t rank, uint64_t rows, Span& out) {
    // The two accepted layouts: rank 1 [width] and contiguous rank 2 [rows][width].
    const bool layout = rank == 1 ? t.shape[0] == width && t.shape[1] == 0 && t.strides[0] == 1 && t.strides[1] == 0
                                  : t.shape[0] == rows && t.shape[1] == width && t.strides[0] == width &&
                                        t.strides[1] == 1;
    uint64_t elements = 0, bytes = 0;
    const bool sized = checked_mul(rows, width, elements) && checked_mul(elements, sizeof(float), bytes);
    out = Span(t.data, bytes);
    Rules r;
    r.then([&] { return versioned(&t); })
        .need(raw_enum(t.dtype) == STRIX_DTYPE_F32 && t.rank == rank && layout, STRIX_ERROR_UNSUPPORTED_FORMAT)
        .need(sized && out.addressable(), STRIX_ERROR_INVALID_ARGUMENT)
        .need(bytes <= t.buffer_bytes, STRIX_ERROR_INSUFFICIENT_BUFFER)
        .need(!bytes || (t.data && out.aligned(alignof(float))), STRIX_ERROR_INVALID_ARGUMENT);
    return r.status();
}

strix_status describe_linear(strix_context c, const strix_matmul_desc* d, LinearExtent& e) {
    e = {};
    Rules r;
    r.then([&] { return versioned(d); });
    if (!r.held()) return r.status();
    const strix_weights w = d->weights;
    r.need(w && w->owner == c && std::isfinite(d->alpha) && std::isfinite(d->beta), STRIX_ERROR_INVALID_ARGUMENT);
    if (!r.held()) return r.status();
    const uint32_t rank = d->input.rank;
    r.need(rank == 1 || rank == 2, STRIX_ERROR_UNSUPPORTED_FORMAT);
    if (!r.held()) return r.status();
    e.rows = rank == 1 ? 1 : d->input.shape[0];
    const Span weights(w->base, w->bytes);
    r.need(e.rows <= INT_MAX, STRIX_ERROR_UNSUPPORTED_FORMAT)
        .then([&] { return tensor_extent(d->input, w->dev.input, rank, e.rows, e.x); })
        .then([&] { return tensor_extent(d->output, w->dev.output, rank, e.rows, e.y); })
        .then([&] {
            e.workspace = e.rows ? stx::linear_workspace_bytes(w->dev, e.rows) : 0;
            return e.workspace == UINT64_MAX ? STRIX_ERROR_UNSUPPORTED_FORMAT : STRIX_SUCCESS;
        })
        .need(!e.x.meets(e.y) && !e.x.meets(weights) && !e.y.meets(weights), STRIX_ERROR_INVALID_ARGUMENT);
    return r.status();
}

strix_status place_linear(strix_context c, const strix_matmul_desc& d, const LinearExtent& e, Span workspace) {
    const Span weights(d.weights->base, d.weights->bytes);
    Rules r;
    r.need(workspace.size >= e.workspace, STRIX_ERROR_INSUFFICIENT_BUFFER)
        .need(workspace.addressable() && (!workspace.size || (workspace.at && workspace.aligned(kWorkspaceAlign))),
              STRIX_ERROR_INVALID_ARGUMENT)
        .need(!workspace.meets(e.x) && !workspace.meets(e.y) && !workspace.meets(weights),
              STRIX_ERROR_INVALID_ARGUMENT);
    if (!r.held() || !e.rows) return r.status();
    r.then([&] { return device_resident(c, e.x, alignof(float)); })
        .then([&] { return device_resident(c, e.y, alignof(float)); })
        .then([&] { return device_resident(c, workspace, kWorkspaceAlign); });
    return r.status();
}

stx::LinearCall to_call(const strix_matmul_desc& d, uint64_t rows, void* workspace) {
    stx::LinearCall call;
    call.x = static_cast<const float*>(d.input.data);
    call.y = static_cast<float*>(d.output.data);
    call.rows = rows;
    call.x_row_stride = d.weights->dev.input;
    call.y_row_stride = d.weights->dev.output;
    call.alpha = d.alpha;
    call.beta = d.beta;
    call.workspace = workspace;
    call.handoff_poll_limit = d.weights->owner->gemm_handoff_poll;
    return call;
}

}  // namespace stx_api

using namespace stx_api;

namespace {

// gfx950 (HIP may append feature suffixes after a colon) running wave64.
bool mi355x(const hipDeviceProp_t& p) {
    static constexpr char kArch[] = "gfx950";
    const size_t n = sizeof(kArch) - 1;
    const char after = p.gcnArchName[n];
    return std::strncmp(p.gcnArchName, kArch, n) == 0 && (after == '\0' || after == ':') && p.warpSize == 64;
}

struct StatusText {
    strix_status status;
    const char* text;
};
// The strings are part of the ABI's observable behaviour (callers may match
// on them), so they are the reference's.
constexpr StatusText kStatusText[] = {
    {STRIX_SUCCESS, "success"},
    {STRIX_ERROR_INVALID_ARGUMENT, "invalid argument"},
    {STRIX_ERROR_ABI_MISMATCH, "ABI mismatch"},
    {STRIX_ERROR_UNSUPPORTED_FORMAT, "unsupported format"},
    {STRIX_ERROR_UNSUPPORTED_DEVICE, "unsupported device"},
    {STRIX_ERROR_INSUFFICIENT_BUFFER, "insufficient buffer"},
    {STRIX_ERROR_OUT_OF_MEMORY, "out of memory"},
    {STRIX_ERROR_BACKEND, "HIP/backend error"},
    {STRIX_ERROR_NOT_IMPLEMENTED, "not implemented"},
};

}  // namespace

extern "C" {

uint32_t strix_get_abi_version(void) { return STRIX_TRELLIS_ABI_VERSION; }

const char* strix_status_string(strix_status s) {
    for (const StatusText& t : kStatusText)
        if (t.status == s) return t.text;
    return "unknown status";
}

void strix_matmul_desc_init(strix_matmul_desc* d) {
    if (!d) return;
    strix_matmul_desc fresh{};
    fresh.struct_size = sizeof(fresh);
    fresh.abi_version = STRIX_TRELLIS_ABI_VERSION;
    fresh.alpha = 1.0f;
    for (strix_tensor_desc* t : {&fresh.input, &fresh.output}) {
        t->struct_size = sizeof(strix_tensor_desc);
        t->abi_version = STRIX_TRELLIS_ABI_VERSION;
        t->dtype = STRIX_DTYPE_F32;
    }
    *d = fresh;
}

strix_status strix_context_create(const strix_context_desc* d, strix_context* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = nullptr;
    Rules r;
    r.then([&] { return versioned(d); });
    if (!r.held()) return r.status();
    r.need(!d->flags && d->device_ordinal >= 0, STRIX_ERROR_INVALID_ARGUMENT);
    if (!r.held()) return r.status();
    hipDeviceProp_t props{};
    const hipError_t pe = hipGetDeviceProperties(&props, d->device_ordinal);
    if (pe == hipErrorInvalidDevice || pe == hipErrorNoDevice) return STRIX_ERROR_UNSUPPORTED_DEVICE;
    if (pe != hipSuccess) return status_of(pe);
    if (!mi355x(props)) return STRIX_ERROR_UNSUPPORTED_DEVICE;
    // The allocation-free GEMV's scratch on this device: looked up once per
    // device, nothing allocated.
    void* scratch = nullptr;
    const hipError_t se = stx::gemv_scratch_address(d->device_ordinal, &scratch);
    if (se != hipSuccess) return status_of(se);
    auto* c = new (std::nothrow) strix_context_impl;
    if (!c) return STRIX_ERROR_OUT_OF_MEMORY;
    c->device = d->device_ordinal;
    c->compute_units = props.multiProcessorCount;
    c->gemv_scratch = scratch;
    *out = c;
    return STRIX_SUCCESS;
}

strix_status strix_context_destroy(strix_context c) {
    if (!c || c->weights_live) return STRIX_ERROR_INVALID_ARGUMENT;
    delete c;
    return STRIX_SUCCESS;
}

}  // extern "C"
