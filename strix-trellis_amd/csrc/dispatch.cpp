// Path selection and workspace sizing for one linear call.
//   rows 1..8 and GEMV entry points -> decode GEMV (gemv.hip)
//   GEMM entry point or rows > 8    -> prefill GEMM (gemm.hip)
// The workspace query returns one bound that covers whichever path a
// descriptor may take (reference src/backend.hip:47-60, docs/API.md:203-212).
#include "backend.hpp"

namespace stx {

uint64_t linear_workspace_bytes(const DeviceWeights& w, uint64_t rows) {
    const uint64_t gemm = gemm_workspace_bytes(w, rows);
    if (gemm == UINT64_MAX) return UINT64_MAX;
    if (rows > 8) return gemm;
    const uint64_t gemv = gemv_workspace_bytes(w, uint32_t(rows));
    return gemv > gemm ? gemv : gemm;
}

uint32_t linear_launch_count(const DeviceWeights& w, uint64_t rows, bool gemm, bool single_launch) {
    if (!rows) return 0;
    if (gemm || rows > 8) return gemm_launch_count(w, rows);
    if (single_launch) return 1;
    return gemv_shape(w.input, w.output, w.bits).splits > 1 ? 2 : 1;
}

hipError_t launch_linear(const DeviceWeights& w, const LinearCall& call, bool prefer_gemm, hipStream_t stream) {
    if (!call.rows) return hipSuccess;
    if (prefer_gemm || call.rows > 8) return launch_gemm(w, call, stream);
    return launch_gemv(w, call, stream);
}

}  // namespace stx
