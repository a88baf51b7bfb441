// Routed-expert kernels with K2 gate weights and K2 down weights.
#include "moe_kernel.hpp"

namespace stx {
STX_INSTANTIATE_MOE(2)
}  // namespace stx
