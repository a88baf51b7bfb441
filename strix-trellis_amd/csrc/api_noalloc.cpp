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
    strix_status s = context_ok(c);
    if (s != STRIX_SUCCESS) return s;
    hipStream_t hs{};
    if ((s = stream_ok(c, stream, hs)) != STRIX_SUCCESS) return s;
    Call call{};
    if ((s = call_ok(c, d, call)) != STRIX_SUCCESS) return s;
    if (d->workspace || d->workspace_bytes) return STRIX_ERROR_INVALID_ARGUMENT;
    if (call.rows > 8) return STRIX_ERROR_UNSUPPORTED_FORMAT;
    if (!call.rows) return STRIX_SUCCESS;
    const stx::DeviceWeights& w = d->weights->dev;
    if (stx::gemv_workspace_bytes(w, uint32_t(call.rows)) > stx::kGemvScratchBytes)
        return STRIX_ERROR_INSUFFICIENT_BUFFER;
    if ((s = device_range_ok(c, d->input.data, call.input_bytes, alignof(float))) != STRIX_SUCCESS) return s;
    if ((s = device_range_ok(c, d->output.data, call.output_bytes, alignof(float))) != STRIX_SUCCESS) return s;
    if (!c->gemv_scratch) return STRIX_ERROR_BACKEND;
    return from_hip(stx::launch_gemv(w, make_call(*d, call.rows, c->gemv_scratch), hs));
}
