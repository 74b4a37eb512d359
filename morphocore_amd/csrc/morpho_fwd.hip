// Dilation / erosion forward for gfx950: float32 and float64 instances of the kernels of
// morpho_fwd.hpp (float16 and bfloat16: morpho_fwd_half.hip, a separate translation unit so that the
// instances compile in parallel).
#include "morpho_fwd.hpp"

namespace mca
{
MCA_INSTANTIATE_FWD(float)
MCA_INSTANTIATE_FWD(double)
}  // namespace mca
