// Prefill GEMM (rows > 8 or the GEMM entry point).
#include "backend.hpp"

namespace stx {

uint32_t gemm_launch_count(const DeviceWeights&, uint64_t rows) { return rows ? 2 : 0; }

hipError_t launch_gemm(const DeviceWeights&, const LinearCall&, hipStream_t) { return hipErrorNotSupported; }

}  // namespace stx
