// strix_amd_gemv_noalloc: strix_gemv for 1-8 rows without a workspace and
// without any allocation.  The call is validated as strix_gemv validates it
// (descriptor, weights, tensors, device memory), except that the descriptor
// must carry no workspace: the split partial planes go to the device's
// static scratch (noalloc.hip), whose address the context looked up when it
// was created.  The kernels are strix_gemv's two-launch GEMV, so the output
// has exactly strix_gemv's bits.
#include "api_internal.hpp"

using namespace stx_api;

static_assert(STRIX_AMD_GEMV_NOALLOC_SCRATCH_BYTES == stx::kGemvScratchBytes, "scratch size in the header");

extern "C" strix_status strix_amd_gemv_noalloc(strix_context c, const strix_matmul_desc* d,
                                               const strix_stream* stream) {
    hipStream_t hs{};
    LinearExtent e;
    Rules r;
    r.then([&] { return on_context_device(c); })
        .then([&] { return borrowed_stream(c, stream, hs); })
        .then([&] { return describe_linear(c, d, e); });
    if (!r.held()) return r.status();
    r.need(!d->workspace && !d->workspace_bytes, STRIX_ERROR_INVALID_ARGUMENT)
        .need(e.rows <= 8, STRIX_ERROR_UNSUPPORTED_FORMAT);
    if (!r.held() || !e.rows) return r.status();
    const stx::DeviceWeights& w = d->weights->dev;
    r.need(stx::gemv_workspace_bytes(w, uint32_t(e.rows)) <= stx::kGemvScratchBytes, STRIX_ERROR_INSUFFICIENT_BUFFER)
        .then([&] { return device_resident(c, e.x, alignof(float)); })
        .then([&] { return device_resident(c, e.y, alignof(float)); })
        .need(c->gemv_scratch != nullptr, STRIX_ERROR_BACKEND)
        .then([&] { return status_of(stx::launch_gemv(w, to_call(*d, e.rows, c->gemv_scratch), hs)); });
    return r.status();
}
