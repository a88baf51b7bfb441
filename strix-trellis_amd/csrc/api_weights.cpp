// Prepared weights: the EXL3 transport (one host blob + metadata, or four
// separate host regions), its validation, and the single private device
// allocation the weights live in.
//
// The contract is the reference ABI's "Modern EXL3 host transport" and
// "Preparation from separate host regions" (include/strix_trellis.h:60-109 and
// its docs/API.md): four regions with exact sizes and offset alignments, the
// codebook enum with its marker, bits 1..8, dimensions positive multiples of
// 128; preparation copies the regions into one allocation and synchronises
// the stream before returning, releasing everything on failure.
//
// Here one table describes the four regions; the metadata checks, the blob
// region checks and the device layout all read it.
#include <climits>
#include <new>

#include "api_internal.hpp"

using namespace stx_api;

namespace {

enum Region { kTrellis = 0, kSuh, kSvh, kBias, kRegions };

struct RegionRule {
    uint32_t blob_align;   // offset alignment inside a transport blob
    bool optional;
};
constexpr RegionRule kRule[kRegions] = {{4, false}, {2, false}, {2, false}, {4, true}};

// Exact byte count of each region for a layer of `rows` outputs, `columns`
// inputs and `bits` bits per weight (false when the trellis size overflows).
bool region_sizes(uint64_t rows, uint64_t columns, uint32_t bits, uint64_t (&bytes)[kRegions]) {
    uint64_t weights = 0;
    if (!checked_mul(rows, columns, weights) || !checked_mul(weights / 8, bits, bytes[kTrellis])) return false;
    bytes[kSuh] = columns * 2;
    bytes[kSvh] = rows * 2;
    bytes[kBias] = rows * 4;
    return true;
}

uint32_t marker_of(uint32_t codebook, bool& known) {
    known = true;
    switch (codebook) {
        case STRIX_CODEBOOK_3INST: return STRIX_EXL3_MARKER_3INST;
        case STRIX_CODEBOOK_MCG: return STRIX_EXL3_MARKER_MCG;
        case STRIX_CODEBOOK_MUL1: return STRIX_EXL3_MARKER_MUL1;
        default: known = false; return 0;
    }
}

// A layer's description as the transport states it, whichever entry point
// delivered it.
struct Layer {
    uint64_t rows = 0, columns = 0;
    uint32_t bits_x2 = 0, codebook = 0, marker = 0;
    uint64_t size[kRegions]{};   // the region byte counts as declared
    bool bias_offset_without_bias = false;
};

strix_status check_layer(const Layer& L) {
    const bool dims = L.rows && L.columns && L.rows <= INT_MAX && L.columns <= INT_MAX && L.rows % 128 == 0 &&
                      L.columns % 128 == 0;
    const bool rate = L.bits_x2 >= 2 && L.bits_x2 <= 16 && L.bits_x2 % 2 == 0;
    bool known = false;
    const uint32_t marker = marker_of(L.codebook, known);
    uint64_t want[kRegions]{};
    const bool sized = dims && rate && region_sizes(L.rows, L.columns, L.bits_x2 / 2, want);
    bool exact = sized;
    for (int i = 0; i < kRegions && exact; ++i)
        exact = kRule[i].optional && !L.size[i] ? true : L.size[i] == want[i];
    Rules r;
    r.need(dims && rate && known && marker == L.marker, STRIX_ERROR_UNSUPPORTED_FORMAT)
        .need(exact && !L.bias_offset_without_bias, STRIX_ERROR_UNSUPPORTED_FORMAT);
    return r.status();
}

Layer layer_of(const strix_exl3_metadata_v1& m) {
    Layer L;
    L.rows = m.rows;
    L.columns = m.columns;
    L.bits_x2 = m.bits_x2;
    L.codebook = raw_enum(m.codebook);
    L.marker = m.marker;
    L.size[kTrellis] = m.trellis_bytes;
    L.size[kSuh] = m.suh_bytes;
    L.size[kSvh] = m.svh_bytes;
    L.size[kBias] = m.bias_bytes;
    L.bias_offset_without_bias = !m.bias_bytes && m.bias_offset;
    return L;
}

// Metadata of a blob: host-native struct, its own version and size.
strix_status check_metadata(const strix_exl3_metadata_v1& m, uint64_t rows, uint64_t columns) {
    bool reserved_zero = true;
    for (uint64_t word : m.reserved) reserved_zero = reserved_zero && !word;
    Rules r;
    r.need(m.struct_size == sizeof(m) && m.transport_version == STRIX_TRELLIS_TRANSPORT_VERSION,
           STRIX_ERROR_ABI_MISMATCH)
        .need(reserved_zero && !m.flags, STRIX_ERROR_INVALID_ARGUMENT)
        .need(m.rows == rows && m.columns == columns, STRIX_ERROR_UNSUPPORTED_FORMAT)
        .then([&] { return check_layer(layer_of(m)); });
    return r.status();
}

// The four host regions a preparation copies, with the layer they describe.
struct Sources {
    Layer layer;
    strix_host_region region[kRegions]{};
};

strix_status from_blob(const strix_exl3_transport_desc* d, Sources& src) {
    Rules r;
    r.then([&] { return versioned(d); });
    if (!r.held()) return r.status();
    r.need(raw_enum(d->format) == STRIX_TRANSPORT_EXL3_CANONICAL &&
               d->transport_version == STRIX_TRELLIS_TRANSPORT_VERSION,
           STRIX_ERROR_UNSUPPORTED_FORMAT)
        .need(d->metadata && d->metadata_bytes == sizeof(strix_exl3_metadata_v1), STRIX_ERROR_INVALID_ARGUMENT);
    if (!r.held()) return r.status();
    strix_exl3_metadata_v1 m{};
    std::memcpy(&m, d->metadata, sizeof(m));   // the caller's struct may be unaligned
    const Span blob(d->data, d->data_bytes);
    r.then([&] { return check_metadata(m, d->rows, d->columns); })
        .need(d->data && blob.addressable(), STRIX_ERROR_INVALID_ARGUMENT);
    if (!r.held()) return r.status();
    const uint64_t offset[kRegions] = {m.trellis_offset, m.suh_offset, m.svh_offset, m.bias_offset};
    src.layer = layer_of(m);
    for (int i = 0; i < kRegions && r.held(); ++i) {
        const uint64_t at = offset[i], n = src.layer.size[i];
        const Span part(reinterpret_cast<const void*>(blob.at + (at <= d->data_bytes ? at : 0)), n);
        r.need(at <= d->data_bytes && n <= d->data_bytes - at, STRIX_ERROR_INSUFFICIENT_BUFFER)
            .need(!n || at % kRule[i].blob_align == 0, STRIX_ERROR_UNSUPPORTED_FORMAT);
        for (int j = 0; j < i && r.held(); ++j)
            r.need(!part.meets(Span(src.region[j].data, src.region[j].bytes)), STRIX_ERROR_INVALID_ARGUMENT);
        src.region[i] = {n ? part.ptr() : nullptr, n};
    }
    return r.status();
}

strix_status from_parts(const strix_exl3_parts_desc* d, Sources& src) {
    Rules r;
    r.then([&] { return versioned(d); });
    if (!r.held()) return r.status();
    r.need(d->transport_version == STRIX_TRELLIS_TRANSPORT_VERSION, STRIX_ERROR_UNSUPPORTED_FORMAT);
    const strix_host_region given[kRegions] = {d->trellis, d->suh, d->svh, d->bias};
    // The blob that would carry these regions, 4-byte packed, must itself be
    // describable (checked offset arithmetic).
    uint64_t packed = 0;
    for (int i = 0; i < kRegions && r.held(); ++i) {
        const strix_host_region& g = given[i];
        const Span part(g.data, g.bytes);
        if (!g.bytes) {
            r.need(!g.data && kRule[i].optional, STRIX_ERROR_INVALID_ARGUMENT);
            continue;
        }
        r.need(g.data && part.addressable(), STRIX_ERROR_INVALID_ARGUMENT);
        for (int j = 0; j < i && r.held(); ++j)
            r.need(!part.meets(Span(given[j].data, given[j].bytes)), STRIX_ERROR_INVALID_ARGUMENT);
        uint64_t at = 0;
        r.need(!__builtin_add_overflow(packed, 3u, &at), STRIX_ERROR_UNSUPPORTED_FORMAT);
        at &= ~uint64_t(3);
        r.need(!__builtin_add_overflow(at, g.bytes, &packed), STRIX_ERROR_UNSUPPORTED_FORMAT);
    }
    if (!r.held()) return r.status();
    Layer& L = src.layer;
    L.rows = d->rows;
    L.columns = d->columns;
    L.bits_x2 = d->bits_x2;
    L.codebook = raw_enum(d->codebook);
    L.marker = d->marker;
    for (int i = 0; i < kRegions; ++i) {
        L.size[i] = given[i].bytes;
        src.region[i] = given[i];
    }
    return check_layer(L);
}

// Device layout: the four regions at 256-byte aligned offsets of one allocation.
bool device_layout(const Layer& L, uint64_t (&offset)[kRegions], uint64_t& total) {
    total = 0;
    for (int i = 0; i < kRegions; ++i) {
        if (total > SIZE_MAX - (kWorkspaceAlign - 1)) return false;
        offset[i] = (total + kWorkspaceAlign - 1) & ~(kWorkspaceAlign - 1);
        if (L.size[i] > SIZE_MAX - offset[i]) return false;
        total = offset[i] + L.size[i];
    }
    return true;
}

strix_status upload(strix_context c, const Sources& src, hipStream_t stream, strix_weights* out) {
    uint64_t offset[kRegions]{}, total = 0;
    if (!device_layout(src.layer, offset, total)) return STRIX_ERROR_OUT_OF_MEMORY;
    auto* w = new (std::nothrow) strix_weights_impl;
    if (!w) return STRIX_ERROR_OUT_OF_MEMORY;
    hipError_t e = hipMalloc(&w->base, static_cast<size_t>(total));
    if (e != hipSuccess) {
        delete w;
        return status_of(e);
    }
    auto* base = static_cast<unsigned char*>(w->base);
    for (int i = 0; i < kRegions && e == hipSuccess; ++i)
        if (src.region[i].bytes)
            e = hipMemcpyAsync(base + offset[i], src.region[i].data, static_cast<size_t>(src.region[i].bytes),
                               hipMemcpyHostToDevice, stream);
    // Drain the copies before returning, also when one of them failed: the
    // caller may release the host regions as soon as this returns.
    const hipError_t drained = hipStreamSynchronize(stream);
    if (e == hipSuccess) e = drained;
    if (e != hipSuccess) {
        (void)hipFree(w->base);
        delete w;
        return status_of(e);
    }
    const Layer& L = src.layer;
    w->owner = c;
    w->bytes = total;
    w->dev.input = static_cast<uint32_t>(L.columns);
    w->dev.output = static_cast<uint32_t>(L.rows);
    w->dev.bits = L.bits_x2 / 2;
    w->dev.codebook = L.codebook;
    w->dev.trellis_bytes = L.size[kTrellis];
    w->dev.trellis = reinterpret_cast<const uint32_t*>(base + offset[kTrellis]);
    w->dev.suh = reinterpret_cast<const uint16_t*>(base + offset[kSuh]);
    w->dev.svh = reinterpret_cast<const uint16_t*>(base + offset[kSvh]);
    w->dev.bias = L.size[kBias] ? reinterpret_cast<const float*>(base + offset[kBias]) : nullptr;
    ++c->weights_live;
    *out = w;
    return STRIX_SUCCESS;
}

template <class Desc, class Read>
strix_status prepare(strix_context c, const Desc* d, const strix_stream* stream, strix_weights* out, Read read) {
    if (!out) return STRIX_ERROR_INVALID_ARGUMENT;
    *out = nullptr;
    hipStream_t hs{};
    Sources src;
    Rules r;
    r.then([&] { return on_context_device(c); })
        .then([&] { return borrowed_stream(c, stream, hs); })
        .then([&] { return read(d, src); })
        .then([&] { return upload(c, src, hs, out); });
    return r.status();
}

}  // namespace

extern "C" {

strix_status strix_weights_prepare(strix_context c, const strix_exl3_transport_desc* d, const strix_stream* stream,
                                   strix_weights* out) {
    return prepare(c, d, stream, out, from_blob);
}

strix_status strix_weights_prepare_parts(strix_context c, const strix_exl3_parts_desc* d,
                                         const strix_stream* stream, strix_weights* out) {
    return prepare(c, d, stream, out, from_parts);
}

strix_status strix_weights_destroy(strix_weights w) {
    if (!w || w->plans) return STRIX_ERROR_INVALID_ARGUMENT;
    const strix_status device = on_context_device(w->owner);
    if (device != STRIX_SUCCESS) return device;
    // Single-launch state first, then the weights themselves; a failed free
    // keeps the handle (and whatever is still allocated) alive.
    while (!w->counter_arrays.empty()) {
        const hipError_t e = hipFree(w->counter_arrays.back());
        if (e != hipSuccess) return status_of(e);
        w->counter_arrays.pop_back();
    }
    const hipError_t e = hipFree(w->base);
    if (e != hipSuccess) return status_of(e);
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

}  // extern "C"
