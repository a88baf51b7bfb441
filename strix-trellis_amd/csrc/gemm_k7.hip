// Prefill GEMM kernels for K = 7 bits per weight (all codebooks): 128/256-row
// blocks of 128 columns, and the 256 x 256 wide kernel.
#include "gemm_wide.hpp"

namespace stx {
STX_INSTANTIATE_GEMM(7)
STX_INSTANTIATE_GEMM_WIDE(7)
}  // namespace stx
