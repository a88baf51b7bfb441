// C ABI v1 of strix_trellis for MI355X: descriptor validation, lifetimes,
// prepared weights, plans and submission.
//
// The contract (status codes, validation order, ownership, aliasing rules)
// follows the reference ABI (include/strix_trellis.h, docs/API.md) as
// implemented in reference src/api.hip:48-608; the device is a gfx950 with
// wave64 instead of the reference's gfx1151 wave32 (src/api.hip:399-401).
#include "api_internal.hpp"

#include <climits>
#include <cmath>
#include <cstring>
#include <new>

namespace stx_api {

strix_status from_hip(hipError_t e) {
    if (e == hipSuccess) return STRIX_SUCCESS;
    if (e == hipErrorOutOfMemory) return STRIX_ERROR_OUT_OF_MEMORY;
    return STRIX_ERROR_BACKEND;
}

bool mul_ok(uint64_t a, uint64_t b, uint64_t& out) {
    if (b && a > UINT64_MAX / b) return false;
    out = a * b;
    return true;
}

bool span_ok(const void* p, uint64_t bytes) {
    return bytes <= SIZE_MAX && bytes <= UINTPTR_MAX - reinterpret_cast<uintptr_t>(p);
}

bool overlaps(const void* a, uint64_t an, const void* b, uint64_t bn) {
    if (!an || !bn) return false;
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + bn && y < x + an;
}

// Calling thread's device must be the context's (reference src/api.hip:73-79).
strix_status context_ok(strix_context c) {
    if (!c) return STRIX_ERROR_INVALID_ARGUMENT;
    int device = -1;
    const hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return from_hip(e);
    return device == c->device ? STRIX_SUCCESS : STRIX_ERROR_INVALID_ARGUMENT;
}

// Mandatory stream descriptor; NULL hip_stream = default stream
// (reference src/api.hip:80-92).
strix_status stream_ok(strix_context c, const strix_stream* s, hipStream_t& out) {
    strix_status st = check_header(s);
    if (st != STRIX_SUCCESS) return st;
    out = static_cast<hipStream_t>(s->hip_stream);
    if (!out) return STRIX_SUCCESS;
    hipDevice_t device = -1;
    unsigned flags = 0;
    if (hipStreamGetDevice(out, &device) != hipSuccess || hipStreamGetFlags(out, &flags) != hipSuccess ||
        device != c->device)
        return STRIX_ERROR_INVALID_ARGUMENT;
    return STRIX_SUCCESS;
}

// Device allocation on the context device covering [p, p+bytes)
// (reference src/api.hip:93-109).
strix_status device_range_ok(strix_context c, const void* p, uint64_t bytes, uint64_t align) {
    if (!bytes) return STRIX_SUCCESS;
    if (!p || !span_ok(p, bytes) || reinterpret_cast<uintptr_t>(p) % align) return STRIX_ERROR_INVALID_ARGUMENT;
    hipPointerAttribute_t attr{};
    if (hipPointerGetAttributes(&attr, p) != hipSuccess || attr.type != hipMemoryTypeDevice ||
        attr.device != c->device || attr.isManaged)
        return STRIX_ERROR_INVALID_ARGUMENT;
    hipDeviceptr_t base{};
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, const_cast<void*>(p)) != hipSuccess)
        return STRIX_ERROR_INVALID_ARGUMENT;
    const uintptr_t start = reinterpret_cast<uintptr_t>(base), at = reinterpret_cast<uintptr_t>(p);
    if (at < start || at - start > size || bytes > size - (at - start)) return STRIX_ERROR_INSUFFICIENT_BUFFER;
    return STRIX_SUCCESS;
}

namespace {

constexpr uint64_t kAlign = STRIX_TRELLIS_WORKSPACE_ALIGNMENT;

struct Range {
    uint64_t offset, bytes;
};

// Metadata rules (reference src/api.hip:112-141, docs/API.md:80-110).
strix_status metadata_ok(const strix_exl3_metadata_v1& m, uint64_t rows, uint64_t columns) {
    if (m.struct_size != sizeof(m) || m.transport_version != STRIX_TRELLIS_TRANSPORT_VERSION)
        return STRIX_ERROR_ABI_MISMATCH;
    for (uint64_t v : m.reserved)
        if (v) return STRIX_ERROR_INVALID_ARGUMENT;
    if (m.flags) return STRIX_ERROR_INVALID_ARGUMENT;
    if (m.rows != rows || m.columns != columns || !m.rows || !m.columns || m.rows > INT_MAX ||
        m.columns > INT_MAX || m.rows % 128 || m.columns % 128)
        return STRIX_ERROR_UNSUPPORTED_FORMAT;
    if (m.bits_x2 < 2 || m.bits_x2 > 16 || m.bits_x2 % 2) return STRIX_ERROR_UNSUPPORTED_FORMAT;
    uint32_t marker = 0;
    switch (enum_raw(m.codebook)) {
        case STRIX_CODEBOOK_3INST: marker = STRIX_EXL3_MARKER_3INST; break;
        case STRIX_CODEBOOK_MCG: marker = STRIX_EXL3_MARKER_MCG; break;
        case STRIX_CODEBOOK_MUL1: marker = STRIX_EXL3_MARKER_MUL1; break;
        default: return STRIX_ERROR_UNSUPPORTED_FORMAT;
    }
    if (marker != m.marker) return STRIX_ERROR_UNSUPPORTED_FORMAT;
    uint64_t packed = 0;
    if (!mul_ok(m.rows, m.columns, packed) || !mul_ok(packed / 8, m.bits_x2 / 2, packed))
        return STRIX_ERROR_UNSUPPORTED_FORMAT;
    if (m.trellis_bytes != packed || m.suh_bytes != m.columns * 2 || m.svh_bytes != m.rows * 2 ||
        (m.bias_bytes && m.bias_bytes != m.rows * 4) || (!m.bias_bytes && m.bias_offset))
        return STRIX_ERROR_UNSUPPORTED_FORMAT;
    return STRIX_SUCCESS;
}

strix_status transport_ok(const strix_exl3_transport_desc* d, strix_exl3_metadata_v1& m) {
    strix_status s = check_header(d);
    if (s != STRIX_SUCCESS) return s;
    if (enum_raw(d->format) != STRIX_TRANSPORT_EXL3_CANONICAL ||
        d->transport_version != STRIX_TRELLIS_TRANSPORT_VERSION)
        return STRIX_ERROR_UNSUPPORTED_FORMAT;
    if (!d->metadata || d->metadata_bytes != sizeof(m)) return STRIX_ERROR_INVALID_ARGUMENT;
    std::memcpy(&m, d->metadata, sizeof(m));
    s = metadata_ok(m, d->rows, d->columns);
    if (s != STRIX_SUCCESS) return s;
    if (!d->data || !span_ok(d->data, d->data_bytes)) return STRIX_ERROR_INVALID_ARGUMENT;
    const Range regions[4] = {{m.trellis_offset, m.trellis_bytes},
                              {m.suh_offset, m.suh_bytes},
                              {m.svh_offset, m.svh_bytes},
                              {m.bias_offset, m.bias_bytes}};
    for (int i = 0; i < 4; ++i) {
        const Range r = regions[i];
        if (r.offset > d->data_bytes || r.bytes > d->data_bytes - r.offset) return STRIX_ERROR_INSUFFICIENT_BUFFER;
        const uint64_t align = (i == 1 || i == 2) ? 2 : 4;
        if (r.bytes && r.offset % align) return STRIX_ERROR_UNSUPPORTED_FORMAT;
        for (int j = 0; j < i; ++j)
            if (r.bytes && regions[j].bytes && r.offset < regions[j].offset + regions[j].bytes &&
                regions[j].offset < r.offset + r.bytes)
                return STRIX_ERROR_INVALID_ARGUMENT;
    }
    return STRIX_SUCCESS;
}

// Region descriptor -> metadata with virtual, 4-aligned offsets
// (reference src/api.hip:170-203).
strix_status parts_ok(const strix_exl3_parts_desc* d, strix_exl3_metadata_v1& m) {
    strix_status s = check_header(d);
    if (s != STRIX_SUCCESS) return s;
    if (d->transport_version != STRIX_TRELLIS_TRANSPORT_VERSION) return STRIX_ERROR_UNSUPPORTED_FORMAT;
    const strix_host_region regions[4] = {d->trellis, d->suh, d->svh, d->bias};
    uint64_t offsets[4]{}, total = 0;
    for (int i = 0; i < 4; ++i) {
        const strix_host_region& r = regions[i];
        if (!r.bytes) {
            if (r.data || i != 3) return STRIX_ERROR_INVALID_ARGUMENT;
            continue;
        }
        if (!r.data || !span_ok(r.data, r.bytes)) return STRIX_ERROR_INVALID_ARGUMENT;
        for (int j = 0; j < i; ++j)
            if (overlaps(r.data, r.bytes, regions[j].data, regions[j].bytes)) return STRIX_ERROR_INVALID_ARGUMENT;
        if (total > UINT64_MAX - 3) return STRIX_ERROR_UNSUPPORTED_FORMAT;
        total = (total + 3) & ~uint64_t(3);
        offsets[i] = total;
        if (r.bytes > UINT64_MAX - total) return STRIX_ERROR_UNSUPPORTED_FORMAT;
        total += r.bytes;
    }
    m = {};
    m.struct_size = sizeof(m);
    m.transport_version = d->transport_version;
    m.rows = d->rows;
    m.columns = d->columns;
    m.bits_x2 = d->bits_x2;
    std::memcpy(&m.codebook, &d->codebook, sizeof(m.codebook));
    m.marker = d->marker;
    m.trellis_offset = offsets[0];
    m.trellis_bytes = d->trellis.bytes;
    m.suh_offset = offsets[1];
    m.suh_bytes = d->suh.bytes;
    m.svh_offset = offsets[2];
    m.svh_bytes = d->svh.bytes;
    m.bias_offset = offsets[3];
    m.bias_bytes = d->bias.bytes;
    return metadata_ok(m, d->rows, d->columns);
}

// One private device allocation with 256-byte aligned slices; the stream is
// synchronised before returning, also after a failed copy
// (reference src/api.hip:205-250, docs/API.md:158-178).
strix_status prepare(strix_context c, const strix_exl3_metadata_v1& m, const strix_host_region* regions,
                     hipStream_t stream, strix_weights* out) {
    auto* w = new (std::nothrow) strix_weights_impl;
    if (!w) return STRIX_ERROR_OUT_OF_MEMORY;
    w->owner = c;
    w->dev.input = static_cast<uint32_t>(m.columns);
    w->dev.output = static_cast<uint32_t>(m.rows);
    w->dev.bits = m.bits_x2 / 2;
    w->dev.codebook = enum_raw(m.codebook);
    w->dev.trellis_bytes = m.trellis_bytes;
    uint64_t offsets[4]{}, total = 0;
    for (int i = 0; i < 4; ++i) {
        if (total > SIZE_MAX - (kAlign - 1)) {
            delete w;
            return STRIX_ERROR_OUT_OF_MEMORY;
        }
        total = (total + kAlign - 1) & ~(kAlign - 1);
        offsets[i] = total;
        if (regions[i].bytes > SIZE_MAX - total) {
            delete w;
            return STRIX_ERROR_OUT_OF_MEMORY;
        }
        total += regions[i].bytes;
    }
    w->bytes = total;
    hipError_t e = hipMalloc(&w->base, static_cast<size_t>(total));
    if (e != hipSuccess) {
        delete w;
        return from_hip(e);
    }
    auto* base = static_cast<unsigned char*>(w->base);
    w->dev.trellis = reinterpret_cast<const uint32_t*>(base + offsets[0]);
    w->dev.suh = reinterpret_cast<const uint16_t*>(base + offsets[1]);
    w->dev.svh = reinterpret_cast<const uint16_t*>(base + offsets[2]);
    w->dev.bias = m.bias_bytes ? reinterpret_cast<const float*>(base + offsets[3]) : nullptr;
    for (int i = 0; i < 4 && e == hipSuccess; ++i) {
        if (!regions[i].bytes) continue;
        e = hipMemcpyAsync(base + offsets[i], regions[i].data, static_cast<size_t>(regions[i].bytes),
                           hipMemcpyHostToDevice, stream);
    }
    const hipError_t done = hipStreamSynchronize(stream);
    if (e != hipSuccess || done != hipSuccess) {
        (void)hipFree(w->base);
        delete w;
        return from_hip(e != hipSuccess ? e : done);
    }
    ++c->weights_live;
    *out = w;
    return STRIX_SUCCESS;
}

}  // namespace

// Rank-1 [W] or rank-2 [rows, W] contiguous F32 tensor (reference src/api.hip:254-270).
strix_status tensor_ok(const strix_tensor_desc& t, uint64_t width, uint32_t rank, uint64_t rows, uint64_t& bytes) {
    strix_status s = check_header(&t);
    if (s != STRIX_SUCCESS) return s;
    if (enum_raw(t.dtype) != STRIX_DTYPE_F32 || t.rank != rank) return STRIX_ERROR_UNSUPPORTED_FORMAT;
    if (rank == 1) {
        if (t.shape[0] != width || t.shape[1] || t.strides[0] != 1 || t.strides[1])
            return STRIX_ERROR_UNSUPPORTED_FORMAT;
    } else if (t.shape[0] != rows || t.shape[1] != width || t.strides[0] != width || t.strides[1] != 1) {
        return STRIX_ERROR_UNSUPPORTED_FORMAT;
    }
    if (!mul_ok(rows, width, bytes) || !mul_ok(bytes, sizeof(float), bytes) || !span_ok(t.data, bytes))
        return STRIX_ERROR_INVALID_ARGUMENT;
    if (bytes > t.buffer_bytes) return STRIX_ERROR_INSUFFICIENT_BUFFER;
    if (bytes && (!t.data || reinterpret_cast<uintptr_t>(t.data) % alignof(float)))
        return STRIX_ERROR_INVALID_ARGUMENT;
    return STRIX_SUCCESS;
}

// Host-side descriptor checks, no device queries (reference src/api.hip:272-293).
strix_status call_ok(strix_context c, const strix_matmul_desc* d, Call& call) {
    strix_status s = check_header(d);
    if (s != STRIX_SUCCESS) return s;
    if (!d->weights || d->weights->owner != c || !std::isfinite(d->alpha) || !std::isfinite(d->beta))
        return STRIX_ERROR_INVALID_ARGUMENT;
    const stx::DeviceWeights& w = d->weights->dev;
    const uint32_t rank = d->input.rank;
    if (rank != 1 && rank != 2) return STRIX_ERROR_UNSUPPORTED_FORMAT;
    const uint64_t rows = rank == 1 ? 1 : d->input.shape[0];
    if (rows > INT_MAX) return STRIX_ERROR_UNSUPPORTED_FORMAT;
    call.rows = rows;
    s = tensor_ok(d->input, w.input, rank, rows, call.input_bytes);
    if (s != STRIX_SUCCESS) return s;
    s = tensor_ok(d->output, w.output, rank, rows, call.output_bytes);
    if (s != STRIX_SUCCESS) return s;
    call.workspace_bytes = rows ? stx::linear_workspace_bytes(w, rows) : 0;
    if (call.workspace_bytes == UINT64_MAX) return STRIX_ERROR_UNSUPPORTED_FORMAT;
    const strix_weights_impl* wi = d->weights;
    if (overlaps(d->input.data, call.input_bytes, d->output.data, call.output_bytes) ||
        overlaps(d->input.data, call.input_bytes, wi->base, wi->bytes) ||
        overlaps(d->output.data, call.output_bytes, wi->base, wi->bytes))
        return STRIX_ERROR_INVALID_ARGUMENT;
    return STRIX_SUCCESS;
}

// Workspace and device-allocation checks (reference src/api.hip:294-309).
strix_status storage_ok(strix_context c, const strix_matmul_desc& d, const Call& call, const void* workspace,
                        uint64_t bytes) {
    if (bytes < call.workspace_bytes) return STRIX_ERROR_INSUFFICIENT_BUFFER;
    if (!span_ok(workspace, bytes) || (bytes && (!workspace || reinterpret_cast<uintptr_t>(workspace) % kAlign)))
        return STRIX_ERROR_INVALID_ARGUMENT;
    const strix_weights_impl* wi = d.weights;
    if (overlaps(workspace, bytes, d.input.data, call.input_bytes) ||
        overlaps(workspace, bytes, d.output.data, call.output_bytes) || overlaps(workspace, bytes, wi->base, wi->bytes))
        return STRIX_ERROR_INVALID_ARGUMENT;
    if (!call.rows) return STRIX_SUCCESS;
    strix_status s = device_range_ok(c, d.input.data, call.input_bytes, alignof(float));
    if (s != STRIX_SUCCESS) return s;
    s = device_range_ok(c, d.output.data, call.output_bytes, alignof(float));
    if (s != STRIX_SUCCESS) return s;
    return device_range_ok(c, workspace, bytes, kAlign);
}

stx::LinearCall make_call(const strix_matmul_desc& d, uint64_t rows, void* workspace) {
    stx::LinearCall lc;
    lc.x = static_cast<const float*>(d.input.data);
    lc.y = static_cast<float*>(d.output.data);
    lc.rows = rows;
    lc.x_row_stride = d.weights->dev.input;
    lc.y_row_stride = d.weights->dev.output;
    lc.alpha = d.alpha;
    lc.beta = d.beta;
    lc.workspace = workspace;
    lc.handoff_poll_limit = d.weights->owner->gemm_handoff_poll;
    return lc;
}

namespace {

strix_status submit(strix_context c, const strix_matmul_desc* d, const strix_stream* stream, bool gemv) {
    strix_status s = context_ok(c);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    s = stream_ok(c, stream, hs);
    if (s != STRIX_SUCCESS) return s;
    Call call{};
    s = call_ok(c, d, call);
    if (s != STRIX_SUCCESS) return s;
    if ((gemv && call.rows > 8) || (!gemv && d->input.rank != 2)) return STRIX_ERROR_UNSUPPORTED_FORMAT;
    s = storage_ok(c, *d, call, d->workspace, d->workspace_bytes);
    if (s != STRIX_SUCCESS || !call.rows) return s;
    return from_hip(stx::launch_linear(d->weights->dev, make_call(*d, call.rows, d->workspace), !gemv, hs));
}

strix_status grouped_ok(strix_context c, const strix_grouped_moe_desc* d, uint64_t& maximum) {
    strix_status s = check_header(d);
    if (s != STRIX_SUCCESS) return s;
    if (d->group_count > SIZE_MAX / sizeof(strix_matmul_desc) || (d->group_count && !d->groups) ||
        !span_ok(d->groups, d->group_count * sizeof(strix_matmul_desc)))
        return STRIX_ERROR_INVALID_ARGUMENT;
    maximum = 0;
    for (uint64_t i = 0; i < d->group_count; ++i) {
        const strix_matmul_desc& g = d->groups[i];
        if (g.workspace || g.workspace_bytes) return STRIX_ERROR_INVALID_ARGUMENT;
        Call a{};
        s = call_ok(c, &g, a);
        if (s != STRIX_SUCCESS) return s;
        if (a.workspace_bytes > maximum) maximum = a.workspace_bytes;
        for (uint64_t j = 0; j < i; ++j) {
            const strix_matmul_desc& h = d->groups[j];
            Call b{};
            s = call_ok(c, &h, b);
            if (s != STRIX_SUCCESS) return s;
            if (overlaps(g.input.data, a.input_bytes, h.input.data, b.input_bytes) ||
                overlaps(g.input.data, a.input_bytes, h.output.data, b.output_bytes) ||
                overlaps(g.output.data, a.output_bytes, h.input.data, b.input_bytes) ||
                overlaps(g.output.data, a.output_bytes, h.output.data, b.output_bytes) ||
                overlaps(g.input.data, a.input_bytes, h.weights->base, h.weights->bytes) ||
                overlaps(h.input.data, b.input_bytes, g.weights->base, g.weights->bytes) ||
                overlaps(g.output.data, a.output_bytes, h.weights->base, h.weights->bytes) ||
                overlaps(h.output.data, b.output_bytes, g.weights->base, g.weights->bytes))
                return STRIX_ERROR_INVALID_ARGUMENT;
        }
    }
    return STRIX_SUCCESS;
}

bool is_gfx950(const hipDeviceProp_t& p) {
    return std::strncmp(p.gcnArchName, "gfx950", 6) == 0 && (p.gcnArchName[6] == 0 || p.gcnArchName[6] == ':') &&
           p.warpSize == 64;
}

}  // namespace
}  // namespace stx_api

using namespace stx_api;

extern "C" {

uint32_t strix_get_abi_version(void) { return STRIX_TRELLIS_ABI_VERSION; }

const char* strix_status_string(strix_status s) {
    switch (s) {
        case STRIX_SUCCESS: return "success";
        case STRIX_ERROR_INVALID_ARGUMENT: return "invalid argument";
        case STRIX_ERROR_ABI_MISMATCH: return "ABI mismatch";
        case STRIX_ERROR_UNSUPPORTED_FORMAT: return "unsupported format";
        case STRIX_ERROR_UNSUPPORTED_DEVICE: return "unsupported device";
        case STRIX_ERROR_INSUFFICIENT_BUFFER: return "insufficient buffer";
        case STRIX_ERROR_OUT_OF_MEMORY: return "out of memory";
        case STRIX_ERROR_BACKEND: return "HIP/backend error";
        case STRIX_ERROR_NOT_IMPLEMENTED: return "not implemented";
        default: return "unknown status";
    }
}

void strix_matmul_desc_init(strix_matmul_desc* d) {
    if (!d) return;
    *d = strix_matmul_desc{};
    d->struct_size = sizeof(*d);
    d->abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->alpha = 1.0f;
    d->input.struct_size = d->output.struct_size = sizeof(strix_tensor_desc);
    d->input.abi_version = d->output.abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.dtype = d->output.dtype = STRIX_DTYPE_F32;
}

strix_status strix_context_create(const strix_context_desc* d, strix_context* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = nullptr;
    strix_status s = check_header(d);
    if (s != STRIX_SUCCESS) return s;
    if (d->flags || d->device_ordinal < 0) return STRIX_ERROR_INVALID_ARGUMENT;
    hipDeviceProp_t props{};
    const hipError_t e = hipGetDeviceProperties(&props, d->device_ordinal);
    if (e == hipErrorInvalidDevice || e == hipErrorNoDevice) return STRIX_ERROR_UNSUPPORTED_DEVICE;
    if (e != hipSuccess) return from_hip(e);
    if (!is_gfx950(props)) return STRIX_ERROR_UNSUPPORTED_DEVICE;
    // The allocation-free GEMV's scratch address on this device (looked up
    // once per device; no allocation).
    void* scratch = nullptr;
    const hipError_t se = stx::gemv_scratch_address(d->device_ordinal, &scratch);
    if (se != hipSuccess) return from_hip(se);
    auto* c = new (std::nothrow) strix_context_impl;
    if (!c) return STRIX_ERROR_OUT_OF_MEMORY;
    c->gemv_scratch = scratch;
    c->device = d->device_ordinal;
    c->compute_units = props.multiProcessorCount;
    *out = c;
    return STRIX_SUCCESS;
}

strix_status strix_context_destroy(strix_context c) {
    if (!c || c->weights_live) return STRIX_ERROR_INVALID_ARGUMENT;
    delete c;
    return STRIX_SUCCESS;
}

strix_status strix_weights_prepare(strix_context c, const strix_exl3_transport_desc* d, const strix_stream* stream,
                                   strix_weights* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = nullptr;
    strix_status s = context_ok(c);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    s = stream_ok(c, stream, hs);
    if (s != STRIX_SUCCESS) return s;
    strix_exl3_metadata_v1 m{};
    s = transport_ok(d, m);
    if (s != STRIX_SUCCESS) return s;
    const auto* base = static_cast<const unsigned char*>(d->data);
    const strix_host_region regions[4] = {{base + m.trellis_offset, m.trellis_bytes},
                                          {base + m.suh_offset, m.suh_bytes},
                                          {base + m.svh_offset, m.svh_bytes},
                                          {m.bias_bytes ? base + m.bias_offset : nullptr, m.bias_bytes}};
    return prepare(c, m, regions, hs, out);
}

strix_status strix_weights_prepare_parts(strix_context c, const strix_exl3_parts_desc* d,
                                         const strix_stream* stream, strix_weights* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = nullptr;
    strix_status s = context_ok(c);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    s = stream_ok(c, stream, hs);
    if (s != STRIX_SUCCESS) return s;
    strix_exl3_metadata_v1 m{};
    s = parts_ok(d, m);
    if (s != STRIX_SUCCESS) return s;
    const strix_host_region regions[4] = {d->trellis, d->suh, d->svh, d->bias};
    return prepare(c, m, regions, hs, out);
}

strix_status strix_weights_destroy(strix_weights w) {
    if (!w || w->plans) return STRIX_ERROR_INVALID_ARGUMENT;
    strix_status s = context_ok(w->owner);
    if (s != STRIX_SUCCESS) return s;
    while (!w->counter_arrays.empty()) {
        const hipError_t e = hipFree(w->counter_arrays.back());
        if (e != hipSuccess) return from_hip(e);
        w->counter_arrays.pop_back();
    }
    const hipError_t e = hipFree(w->base);
    if (e != hipSuccess) return from_hip(e);
    --w->owner->weights_live;
    delete w;
    return STRIX_SUCCESS;
}

strix_status strix_weights_device_span(strix_weights w, const void** data, uint64_t* bytes) {
    if (data) *data = nullptr;
    if (bytes) *bytes = 0;
    if (!w || !data || !bytes) return STRIX_ERROR_INVALID_ARGUMENT;
    *data = w->base;
    *bytes = w->bytes;
    return STRIX_SUCCESS;
}

strix_status strix_matmul_workspace_bytes(strix_context c, const strix_matmul_desc* d, uint64_t* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = 0;
    strix_status s = context_ok(c);
    if (s != STRIX_SUCCESS) return s;
    Call call{};
    s = call_ok(c, d, call);
    if (s == STRIX_SUCCESS) *out = call.workspace_bytes;
    return s;
}

strix_status strix_gemv(strix_context c, const strix_matmul_desc* d, const strix_stream* stream) {
    return submit(c, d, stream, true);
}

strix_status strix_gemm(strix_context c, const strix_matmul_desc* d, const strix_stream* stream) {
    return submit(c, d, stream, false);
}

// Plans: validated once; a GEMV plan with split partials runs as one launch
// on dedicated partial planes owned by the weights (the reference keeps its
// completion counters there), so captured graphs stay valid after the plan is
// destroyed (reference src/api.hip:505-563, docs/API.md:230-295).
strix_status strix_linear_plan_create(strix_context c, const strix_matmul_desc* d, const strix_stream* stream,
                                      uint32_t operation, strix_linear_plan* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = nullptr;
    if (operation != STRIX_OPERATION_GEMV && operation != STRIX_OPERATION_GEMM) return STRIX_ERROR_INVALID_ARGUMENT;
    strix_status s = context_ok(c);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    s = stream_ok(c, stream, hs);
    if (s != STRIX_SUCCESS) return s;
    Call call{};
    s = call_ok(c, d, call);
    if (s != STRIX_SUCCESS) return s;
    const bool gemm = operation == STRIX_OPERATION_GEMM;
    if ((!gemm && call.rows > 8) || (gemm && d->input.rank != 2)) return STRIX_ERROR_UNSUPPORTED_FORMAT;
    s = storage_ok(c, *d, call, d->workspace, d->workspace_bytes);
    if (s != STRIX_SUCCESS) return s;
    strix_weights w = d->weights;
    if (w->plans == SIZE_MAX) return STRIX_ERROR_OUT_OF_MEMORY;
    auto* plan = new (std::nothrow) strix_linear_plan_impl;
    if (!plan) return STRIX_ERROR_OUT_OF_MEMORY;
    plan->owner = c;
    plan->weights = w;
    plan->stream = hs;
    plan->gemm = gemm;
    plan->call = make_call(*d, call.rows, d->workspace);
    plan->launches = 0;
    if (!gemm && call.rows) {
        s = make_fused_state(w, call.rows, hs, plan->fused);
        if (s != STRIX_SUCCESS) {
            delete plan;
            return s;
        }
    }
    if (call.rows) plan->launches = stx::linear_launch_count(w->dev, call.rows, gemm, plan->fused.planes != nullptr);
    ++w->plans;
    *out = plan;
    return STRIX_SUCCESS;
}

}  // extern "C"

namespace stx_api {

hipError_t init_fused_state(void* base, uint64_t bytes, uint64_t planes_offset, hipStream_t hs) {
    uint32_t* words = static_cast<uint32_t*>(base);
    hipError_t e = stx::launch_fill_u32(words, 0u, planes_offset / 4, hs);
    if (e == hipSuccess)
        e = stx::launch_fill_u32(words + planes_offset / 4, stx::GEMV_PLANE_EMPTY, (bytes - planes_offset) / 4, hs);
    return e;
}

strix_status make_fused_state(strix_weights w, uint64_t rows, hipStream_t hs, stx::FusedState& out) {
    out = {};
    const uint64_t bytes = stx::fused_state_bytes(w->dev, rows, 1);
    if (!bytes) return STRIX_SUCCESS;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e == hipSuccess) e = init_fused_state(p, bytes, stx::fused_planes_offset(w->dev, 1), hs);
    if (e == hipSuccess) e = hipStreamSynchronize(hs);
    if (e == hipSuccess) {
        try {
            w->counter_arrays.push_back(p);   // freed with the weights
        } catch (...) {
            e = hipErrorOutOfMemory;
        }
    }
    if (e != hipSuccess) {
        if (p) (void)hipFree(p);
        return from_hip(e);
    }
    out = stx::fused_state_at(p, w->dev, rows, 1);
    return STRIX_SUCCESS;
}

strix_status read_fused_status(const stx::FusedState& st, hipStream_t hs, uint32_t* flags, uint32_t clear) {
    *flags = 0;
    if (!st.status) return STRIX_SUCCESS;
    uint32_t v = 0;
    hipError_t e = hipMemcpyAsync(&v, st.status, sizeof(v), hipMemcpyDeviceToHost, hs);
    if (e == hipSuccess && clear) e = stx::launch_fill_u32(st.status, 0u, 1, hs);
    if (e == hipSuccess) e = hipStreamSynchronize(hs);
    if (e != hipSuccess) return from_hip(e);
    *flags = v;
    return STRIX_SUCCESS;
}

}  // namespace stx_api

extern "C" {

strix_status strix_linear_plan_submit(strix_linear_plan p) {
    if (!p) return STRIX_ERROR_INVALID_ARGUMENT;
    const strix_status s = context_ok(p->owner);
    if (s != STRIX_SUCCESS || !p->call.rows) return s;
    const stx::DeviceWeights& w = p->weights->dev;
    if (!p->gemm && p->fused.planes) {
        stx::LinearCall call = p->call;
        call.gemv_poll_limit = p->owner->gemv_poll_limit;
        return from_hip(stx::launch_gemv_fused(w, call, p->fused, p->stream));
    }
    return from_hip(stx::launch_linear(w, p->call, p->gemm, p->stream));
}

strix_status strix_linear_plan_destroy(strix_linear_plan p) {
    if (!p) return STRIX_ERROR_INVALID_ARGUMENT;
    --p->weights->plans;
    delete p;
    return STRIX_SUCCESS;
}

strix_status strix_grouped_moe_workspace_bytes(strix_context c, const strix_grouped_moe_desc* d, uint64_t* out) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = 0;
    strix_status s = context_ok(c);
    if (s != STRIX_SUCCESS) return s;
    uint64_t maximum = 0;
    s = grouped_ok(c, d, maximum);
    if (s == STRIX_SUCCESS) *out = maximum;
    return s;
}

// Pre-routed groups: all validated first, then enqueued in order sharing the
// workspace (reference src/api.hip:578-607).
strix_status strix_grouped_moe(strix_context c, const strix_grouped_moe_desc* d, const strix_stream* stream) {
    strix_status s = context_ok(c);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    s = stream_ok(c, stream, hs);
    if (s != STRIX_SUCCESS) return s;
    uint64_t maximum = 0;
    s = grouped_ok(c, d, maximum);
    if (s != STRIX_SUCCESS) return s;
    if (d->workspace_bytes < maximum) return STRIX_ERROR_INSUFFICIENT_BUFFER;
    if (!span_ok(d->workspace, d->workspace_bytes) ||
        (d->workspace_bytes && (!d->workspace || reinterpret_cast<uintptr_t>(d->workspace) % kAlign)))
        return STRIX_ERROR_INVALID_ARGUMENT;
    for (uint64_t i = 0; i < d->group_count; ++i) {
        Call call{};
        s = call_ok(c, &d->groups[i], call);
        if (s != STRIX_SUCCESS) return s;
        s = storage_ok(c, d->groups[i], call, d->workspace, d->workspace_bytes);
        if (s != STRIX_SUCCESS) return s;
    }
    for (uint64_t i = 0; i < d->group_count; ++i) {
        const strix_matmul_desc& g = d->groups[i];
        const uint64_t rows = g.input.rank == 1 ? 1 : g.input.shape[0];
        if (!rows) continue;
        s = from_hip(stx::launch_linear(g.weights->dev, make_call(g, rows, d->workspace), rows > 8, hs));
        if (s != STRIX_SUCCESS) return s;
    }
    return STRIX_SUCCESS;
}

// ---- MI355X diagnostic extensions (strix_trellis_amd.h) ----
strix_status strix_amd_decode(strix_weights w, void* q, uint64_t q_bytes, const strix_stream* stream) {
    if (!w) return STRIX_ERROR_INVALID_ARGUMENT;
    strix_status s = context_ok(w->owner);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    s = stream_ok(w->owner, stream, hs);
    if (s != STRIX_SUCCESS) return s;
    const uint64_t need = uint64_t(w->dev.input) * w->dev.output * 2;
    if (q_bytes < need) return STRIX_ERROR_INSUFFICIENT_BUFFER;
    s = device_range_ok(w->owner, q, need, 4);
    if (s != STRIX_SUCCESS) return s;
    return from_hip(stx::launch_decode(w->dev, static_cast<_Float16*>(q), hs));
}

strix_status strix_amd_input_stage(strix_weights w, const float* x, uint64_t rows, void* a, uint64_t a_bytes,
                                   const strix_stream* stream) {
    if (!w) return STRIX_ERROR_INVALID_ARGUMENT;
    strix_status s = context_ok(w->owner);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    s = stream_ok(w->owner, stream, hs);
    if (s != STRIX_SUCCESS) return s;
    uint64_t need = 0;
    if (rows > INT_MAX || !mul_ok(rows, uint64_t(w->dev.input) * 2, need)) return STRIX_ERROR_UNSUPPORTED_FORMAT;
    if (a_bytes < need) return STRIX_ERROR_INSUFFICIENT_BUFFER;
    if ((s = device_range_ok(w->owner, x, need * 2, 4)) != STRIX_SUCCESS) return s;
    if ((s = device_range_ok(w->owner, a, need, 4)) != STRIX_SUCCESS) return s;
    return from_hip(stx::launch_input_stage(w->dev, x, rows, static_cast<_Float16*>(a), hs));
}

strix_status strix_amd_output_stage(strix_weights w, const float* core, uint64_t rows, float* y, uint64_t y_bytes,
                                    float alpha, float beta, const strix_stream* stream) {
    if (!w || !std::isfinite(alpha) || !std::isfinite(beta)) return STRIX_ERROR_INVALID_ARGUMENT;
    strix_status s = context_ok(w->owner);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    s = stream_ok(w->owner, stream, hs);
    if (s != STRIX_SUCCESS) return s;
    uint64_t need = 0;
    if (rows > INT_MAX || !mul_ok(rows, uint64_t(w->dev.output) * 4, need)) return STRIX_ERROR_UNSUPPORTED_FORMAT;
    if (y_bytes < need) return STRIX_ERROR_INSUFFICIENT_BUFFER;
    if (overlaps(core, need, y, need)) return STRIX_ERROR_INVALID_ARGUMENT;
    if ((s = device_range_ok(w->owner, core, need, 4)) != STRIX_SUCCESS) return s;
    if ((s = device_range_ok(w->owner, y, need, 4)) != STRIX_SUCCESS) return s;
    return from_hip(stx::launch_output_stage(w->dev, core, rows, y, alpha, beta, hs));
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

strix_status strix_amd_set_gemv_poll_limit(strix_context c, uint32_t poll_limit) {
    const strix_status s = context_ok(c);
    if (s != STRIX_SUCCESS) return s;
    c->gemv_poll_limit = poll_limit;
    return STRIX_SUCCESS;
}

strix_status strix_amd_plan_status(strix_linear_plan p, uint32_t clear, uint32_t* flags) {
    if (flags) *flags = 0;
    if (!p || !flags) return STRIX_ERROR_INVALID_ARGUMENT;
    const strix_status s = context_ok(p->owner);
    if (s != STRIX_SUCCESS) return s;
    return read_fused_status(p->fused, p->stream, flags, clear);
}

strix_status strix_amd_stream_read(strix_context c, const void* src, uint64_t bytes, uint32_t workgroups,
                                   uint32_t* sink, const strix_stream* stream) {
    strix_status s = context_ok(c);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    if ((s = stream_ok(c, stream, hs)) != STRIX_SUCCESS) return s;
    if (!workgroups || !bytes || bytes % (16ull * workgroups) || bytes / workgroups >= (uint64_t(1) << 31))
        return STRIX_ERROR_INVALID_ARGUMENT;
    if ((s = device_range_ok(c, src, bytes, 16)) != STRIX_SUCCESS) return s;
    if ((s = device_range_ok(c, sink, uint64_t(workgroups) * 4, 4)) != STRIX_SUCCESS) return s;
    return from_hip(stx::launch_stream_read(src, bytes, workgroups, sink, hs));
}

strix_status strix_amd_set_gemm_handoff(strix_context c, uint32_t always_take_over) {
    const strix_status s = context_ok(c);
    if (s != STRIX_SUCCESS) return s;
    c->gemm_handoff_poll = always_take_over ? UINT32_MAX : 4096u;
    return STRIX_SUCCESS;
}

}  // extern "C"
