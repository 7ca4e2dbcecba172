// Decode kernel instantiations: f16 K/V, fused decode step.
#include "decode_kernel.cuh"

namespace rlse {
RLSE_DECODE_INSTANCES(template, f16, kModeFused)
}  // namespace rlse
