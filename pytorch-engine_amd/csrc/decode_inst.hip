// Decode kernel instantiations for one (weight format, stage), chosen at compile time by
// PG_QT (PGMOE_Q4_1 / PGMOE_Q4_K / PGMOE_Q5_K / PGMOE_Q6_K / PGMOE_Q8_0 / PGMOE_F16) and PG_PART (0 gate/up, 1 down,
// 2 down + combine); the Makefile builds every combination as its own object so the
// template instantiations compile in parallel.
#include "decode_kernels.h"

namespace pgmoe {
#if PG_PART == 0
PG_DEFINE_DECODE_GATEUP(PG_QT)
#elif PG_PART == 1
#if PG_QT == PGMOE_F16
// The per-expert down kernel holds a whole super-block a lane: 32 chunks of fp16 weights
// would not fit its registers.  fp16 down projections run on the fused down + combine
// kernels (rows of up to 32 super-blocks) instead.
template <>
int dec_down_q<PGMOE_F16>(const Mats&, const float*, const float*, int, int, const DecDisp&, int, const float*, float*,
                          hipStream_t) {
    return fail(PGMOE_E_UNSUPPORTED, "decode down: fp16 weights need the fused down + combine (at most 8192 inputs)");
}
#else
PG_DEFINE_DECODE_DOWN(PG_QT)
#endif
#else
PG_DEFINE_DECODE_DOWN_COMBINE(PG_QT)
#endif
}  // namespace pgmoe
