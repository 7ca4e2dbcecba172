// Decode kernel instantiations: f32 K/V, fused decode step.
#include "decode_kernel.cuh"

namespace rlse {
RLSE_DECODE_INSTANCES(template, float, kModeFused)
}  // namespace rlse
