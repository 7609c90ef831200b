// Decode GEMV instantiations for one weight format (split for parallel compilation).
#include "decode_kernels.h"

namespace pgmoe {
PG_DEFINE_DECODE_LAUNCHERS(PGMOE_Q6_K)
}  // namespace pgmoe
