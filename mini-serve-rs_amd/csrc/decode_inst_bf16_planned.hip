// Decode kernel instantiations: bf16 K/V, fused decode step with a per-step plan.
#include "decode_kernel.cuh"

namespace rlse {
RLSE_DECODE_INSTANCES(template, bf16, kModePlanned)
}  // namespace rlse
