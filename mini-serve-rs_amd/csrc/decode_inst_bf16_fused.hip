// Decode kernel instantiations: bf16 K/V, fused decode step.
#include "decode_kernel.cuh"

namespace rlse {
RLSE_DECODE_INSTANCES(template, bf16, kModeFused)
}  // namespace rlse
