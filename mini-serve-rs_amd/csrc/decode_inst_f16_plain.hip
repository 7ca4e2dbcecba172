// Decode kernel instantiations: f16 K/V, paged decode.
#include "decode_kernel.cuh"

namespace rlse {
RLSE_DECODE_INSTANCES(template, f16, kModePlain)
}  // namespace rlse
