// Handle layouts and validation helpers shared by the C ABI translation units.
#pragma once
#include "strix_trellis.h"
#include "strix_trellis_amd.h"
#include "backend.hpp"

#include <cstring>
#include <vector>

struct strix_context_impl {
    int device = -1;
    int compute_units = 0;
    uint64_t weights_live = 0;
    uint32_t gemm_handoff_poll = 4096;   // LinearCall::handoff_poll_limit of calls made on it
    uint32_t gemv_poll_limit = stx::GEMV_DEFAULT_POLL_LIMIT;   // single-launch GEMV finishers
    void* gemv_scratch = nullptr;   // this device's static scratch (strix_amd_gemv_noalloc)
    uint32_t grouped_fold = 0;      // grouped plans created on it: 0 library's choice, 1 split, 2 owner
};

struct strix_weights_impl {
    strix_context owner = nullptr;
    stx::DeviceWeights dev{};
    void* base = nullptr;     // single private allocation: trellis | suh | svh | bias
    uint64_t bytes = 0;
    uint64_t plans = 0;       // live plans retaining these weights
    // Single-launch state (tagged planes, epochs, status) of plans created on
    // these weights.  Graphs captured from a plan may replay after the plan is
    // destroyed, so the arrays live until the weights are destroyed.
    std::vector<void*> counter_arrays;
};

struct strix_linear_plan_impl {
    strix_context owner = nullptr;
    strix_weights weights = nullptr;
    stx::LinearCall call{};
    hipStream_t stream{};
    bool gemm = false;
    stx::FusedState fused{};    // single-launch GEMV state (null when one split suffices)
    uint32_t launches = 0;
};

namespace stx_api {

template <class E>
uint32_t enum_raw(const E& value) {
    static_assert(sizeof(E) == sizeof(uint32_t), "32-bit enum ABI required");
    uint32_t raw = 0;
    std::memcpy(&raw, &value, sizeof(raw));
    return raw;
}

// Exact struct_size, ABI version 1, zero reserved words.
template <class T>
strix_status check_header(const T* d) {
    if (!d) return STRIX_ERROR_INVALID_ARGUMENT;
    if (d->struct_size != sizeof(T) || d->abi_version != STRIX_TRELLIS_ABI_VERSION) return STRIX_ERROR_ABI_MISMATCH;
    for (uint64_t v : d->reserved)
        if (v) return STRIX_ERROR_INVALID_ARGUMENT;
    return STRIX_SUCCESS;
}

struct Call {
    uint64_t rows = 0;
    uint64_t input_bytes = 0, output_bytes = 0, workspace_bytes = 0;
};

strix_status from_hip(hipError_t e);
bool mul_ok(uint64_t a, uint64_t b, uint64_t& out);
bool span_ok(const void* p, uint64_t bytes);
bool overlaps(const void* a, uint64_t an, const void* b, uint64_t bn);
strix_status context_ok(strix_context c);
strix_status stream_ok(strix_context c, const strix_stream* s, hipStream_t& out);
strix_status device_range_ok(strix_context c, const void* p, uint64_t bytes, uint64_t align);
strix_status tensor_ok(const strix_tensor_desc& t, uint64_t width, uint32_t rank, uint64_t rows, uint64_t& bytes);
strix_status call_ok(strix_context c, const strix_matmul_desc* d, Call& call);
strix_status storage_ok(strix_context c, const strix_matmul_desc& d, const Call& call, const void* workspace,
                        uint64_t bytes);
stx::LinearCall make_call(const strix_matmul_desc& d, uint64_t rows, void* workspace);
// Enqueue the initial contents of a single-launch state of `bytes` at base:
// status and epochs 0, every plane word GEMV_PLANE_EMPTY.
hipError_t init_fused_state(void* base, uint64_t bytes, uint64_t planes_offset, hipStream_t hs);
// Initialised single-launch GEMV state for `rows` rows on `w` (none when one
// split suffices), owned by the weights; the stream is synchronised.
strix_status make_fused_state(strix_weights w, uint64_t rows, hipStream_t hs, stx::FusedState& out);
// Sticky status word of a single-launch state: read (synchronising `hs`) and
// optionally cleared.
strix_status read_fused_status(const stx::FusedState& st, hipStream_t hs, uint32_t* flags, uint32_t clear);

}  // namespace stx_api
