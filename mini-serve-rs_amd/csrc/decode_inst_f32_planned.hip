// Decode kernel instantiations: f32 K/V, fused decode step with a per-step plan.
#include "decode_kernel.cuh"

namespace rlse {
RLSE_DECODE_INSTANCES(template, float, kModePlanned)
}  // namespace rlse
