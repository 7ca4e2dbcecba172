// Decode kernel instantiations: f32 K/V, fused decode step with a per-step plan,
// pages streamed with non-temporal loads.
#include "decode_kernel.cuh"

namespace rlse {
RLSE_DECODE_INSTANCES(template, float, kModePlannedStream)
}  // namespace rlse
