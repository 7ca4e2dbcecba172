// Decode kernel instantiations: bf16 K/V, paged decode.
#include "decode_kernel.cuh"

namespace rlse {
RLSE_DECODE_INSTANCES(template, bf16, kModePlain)
}  // namespace rlse
