// Routed-expert kernels with K3 gate weights and K3 down weights.
#include "moe_kernel.hpp"

namespace stx {
STX_INSTANTIATE_MOE(3)
}  // namespace stx
