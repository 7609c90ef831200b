// Decode kernel instantiations for one (weight format, stage), chosen at compile time by
// PG_QT (PGMOE_Q4_1 / PGMOE_Q4_K / PGMOE_Q5_K / PGMOE_Q6_K / PGMOE_Q8_0) and PG_PART (0 gate/up, 1 down,
// 2 down + combine); the Makefile builds every combination as its own object so the
// template instantiations compile in parallel.
#include "decode_kernels.h"

namespace pgmoe {
#if PG_PART == 0
PG_DEFINE_DECODE_GATEUP(PG_QT)
#elif PG_PART == 1
PG_DEFINE_DECODE_DOWN(PG_QT)
#else
PG_DEFINE_DECODE_DOWN_COMBINE(PG_QT)
#endif
}  // namespace pgmoe
