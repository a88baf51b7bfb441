// Decode GEMV and decode kernels for K = 4 bits per weight (all codebooks, 1/2/4/8-row templates).
#include "gemv_kernel.hpp"

namespace stx {
STX_INSTANTIATE_GEMV(4)
}  // namespace stx
