// Dilation / erosion forward for gfx950: float16 and bfloat16 instances of the kernels of
// morpho_fwd.hpp (stored in 16 bits, computed in float32).
#include "morpho_fwd.hpp"

namespace mca
{
MCA_INSTANTIATE_FWD(_Float16)
MCA_INSTANTIATE_FWD(__bf16)
}  // namespace mca
