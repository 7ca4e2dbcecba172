// Decode kernel instantiations: f32 K/V, paged decode.
#include "decode_kernel.cuh"

namespace rlse {
RLSE_DECODE_INSTANCES(template, float, kModePlain)
}  // namespace rlse
