// Handle state of the C ABI and the validation vocabulary its translation
// units (api_*.cpp) share.  Everything here is internal: the ABI is
// include/strix_trellis.h plus the MI355X extensions in strix_trellis_amd.h.
//
// Vocabulary:
//   Rules      evaluates checks in order; the first failing one decides the
//              status and the later ones are not evaluated.
//   Span       a byte range [at, at + size) with checked arithmetic: whether
//              it is addressable at all, whether two ranges meet, alignment.
//   versioned  exact struct_size, ABI version 1 and zero reserved words of a
//              descriptor header (every descriptor of the ABI carries them).
#pragma once
#include "strix_trellis.h"
#include "strix_trellis_amd.h"
#include "backend.hpp"

#include <cstring>
#include <utility>
#include <vector>

struct strix_context_impl {
    int device = -1;
    int compute_units = 0;
    uint64_t weights_live = 0;
    uint32_t gemm_handoff_poll = 4096;   // LinearCall::handoff_poll_limit of calls made on it
    uint32_t gemv_poll_limit = stx::GEMV_DEFAULT_POLL_LIMIT;   // single-launch GEMV finishers
    void* gemv_scratch = nullptr;   // this device's static scratch (strix_amd_gemv_noalloc)
    uint32_t grouped_fold = 0;      // grouped plans created on it: 0 library's choice, 1 split, 2 owner
    bool reuse_plan_state = false;  // plans created on it may take a destroyed plan's single-launch state
};

struct strix_weights_impl {
    strix_context owner = nullptr;
    stx::DeviceWeights dev{};
    void* base = nullptr;     // single private allocation: trellis | suh | svh | bias
    uint64_t bytes = 0;
    uint64_t plans = 0;       // live plans retaining these weights
    // Single-launch state (planes, epochs, status) of plans created on these
    // weights.  Graphs captured from a plan may replay after the plan is
    // destroyed, so the arrays live until the weights are destroyed, and
    // distinct plans never share one (the reference's rule for its completion
    // counters).
    std::vector<void*> counter_arrays;
    // Blocks of counter_arrays whose plans were destroyed.  Only on a context
    // that opted in (strix_amd_set_plan_state_reuse) does a later plan that
    // needs a block of the same size re-initialise and take one; the state
    // held then stays bounded by the plans alive at one time.
    std::vector<std::pair<void*, uint64_t>> idle_states;
};

// A single-launch state block held by a plan (base of a counter_arrays block).
struct FusedBlock {
    void* base = nullptr;
    uint64_t bytes = 0;
};

struct strix_linear_plan_impl {
    strix_context owner = nullptr;
    strix_weights weights = nullptr;
    stx::LinearCall call{};
    hipStream_t stream{};
    bool gemm = false;
    stx::FusedState fused{};    // single-launch GEMV state (null when one split suffices)
    FusedBlock block{};
    uint32_t launches = 0;
};

namespace stx_api {

constexpr uint64_t kWorkspaceAlign = STRIX_TRELLIS_WORKSPACE_ALIGNMENT;

class Rules {
public:
    // Fails with `otherwise` unless `ok`.
    Rules& need(bool ok, strix_status otherwise) {
        if (status_ == STRIX_SUCCESS && !ok) status_ = otherwise;
        return *this;
    }
    // Runs `check` (returning a status) only while every earlier rule held.
    template <class F>
    Rules& then(F&& check) {
        if (status_ == STRIX_SUCCESS) status_ = check();
        return *this;
    }
    bool held() const { return status_ == STRIX_SUCCESS; }
    strix_status status() const { return status_; }

private:
    strix_status status_ = STRIX_SUCCESS;
};

struct Span {
    uintptr_t at = 0;
    uint64_t size = 0;
    Span() = default;
    Span(const void* p, uint64_t bytes) : at(reinterpret_cast<uintptr_t>(p)), size(bytes) {}
    void* ptr() const { return reinterpret_cast<void*>(at); }
    // The range neither wraps the address space nor exceeds SIZE_MAX bytes.
    bool addressable() const { return size <= SIZE_MAX && size <= UINTPTR_MAX - at; }
    // Both ranges nonempty and sharing at least one byte.
    bool meets(const Span& o) const { return size && o.size && at < o.at + o.size && o.at < at + size; }
    bool aligned(uint64_t a) const { return at % a == 0; }
};

inline bool checked_mul(uint64_t a, uint64_t b, uint64_t& out) { return !__builtin_mul_overflow(a, b, &out); }

template <class E>
uint32_t raw_enum(const E& value) {
    static_assert(sizeof(E) == sizeof(uint32_t), "32-bit enum ABI required");
    uint32_t raw = 0;
    std::memcpy(&raw, &value, sizeof(raw));
    return raw;
}

template <class T>
strix_status versioned(const T* d) {
    if (!d) return STRIX_ERROR_INVALID_ARGUMENT;
    if (d->struct_size != sizeof(T) || d->abi_version != STRIX_TRELLIS_ABI_VERSION) return STRIX_ERROR_ABI_MISMATCH;
    for (uint64_t word : d->reserved)
        if (word) return STRIX_ERROR_INVALID_ARGUMENT;
    return STRIX_SUCCESS;
}

// HIP error -> ABI status: OUT_OF_MEMORY when HIP says so, else BACKEND.
strix_status status_of(hipError_t e);

// The calling thread's current device is the context's.
strix_status on_context_device(strix_context c);
// A mandatory stream descriptor; a NULL hip_stream is the device's default
// stream, any other stream must belong to the context's device.
strix_status borrowed_stream(strix_context c, const strix_stream* s, hipStream_t& out);
// [span) lies inside one HIP device allocation on the context's device
// (empty spans pass): INVALID_ARGUMENT when it is not device memory of that
// device (or misaligned), INSUFFICIENT_BUFFER when the allocation is shorter.
strix_status device_resident(strix_context c, Span span, uint64_t align);

// One linear call (strix_gemv / strix_gemm / plans): the host-side facts of a
// descriptor and the device-side checks of its buffers.
struct LinearExtent {
    uint64_t rows = 0;
    Span x, y;                 // logical bytes read and written
    uint64_t workspace = 0;    // bytes the call needs
};
// Rank 1 [width] or rank 2 [rows][width] contiguous F32 tensor.
strix_status tensor_extent(const strix_tensor_desc& t, uint64_t width, uint32_t rank, uint64_t rows, Span& out);
// Descriptor, weights, scalars, tensors, required workspace, aliasing of the
// tensors and the weights (no device memory is inspected).
strix_status describe_linear(strix_context c, const strix_matmul_desc* d, LinearExtent& e);
// The workspace (declared range) against the call, then device residence of
// every buffer.
strix_status place_linear(strix_context c, const strix_matmul_desc& d, const LinearExtent& e, Span workspace);
stx::LinearCall to_call(const strix_matmul_desc& d, uint64_t rows, void* workspace);

// Enqueue the initial contents of a single-launch state of `bytes` at base:
// status and epochs 0, every plane word GEMV_PLANE_EMPTY.
hipError_t init_fused_state(void* base, uint64_t bytes, uint64_t planes_offset, hipStream_t hs);
// Initialised single-launch GEMV state for `rows` rows on `w` (none when one
// split suffices), owned by the weights: an idle block of the same size if
// there is one, else a new one; the stream is synchronised.
strix_status make_fused_state(strix_weights w, uint64_t rows, hipStream_t hs, stx::FusedState& out,
                              FusedBlock& block);
// A destroyed plan's block becomes idle (it stays allocated with the weights).
void release_fused_state(strix_weights w, FusedBlock& block);
// Sticky status word of a single-launch state of `bytes` (planes from
// `planes_offset`): read (synchronising `hs`); with `clear` the whole state
// is re-initialised on `hs` first (status and epochs 0, every plane EMPTY),
// which also lifts a give-up's poison.
strix_status read_fused_status(const stx::FusedState& st, uint64_t bytes, uint64_t planes_offset, hipStream_t hs,
                               uint32_t* flags, uint32_t clear);

}  // namespace stx_api
