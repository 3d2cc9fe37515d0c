// Fused decode forms (fused.h) of the 32-value types Q8_0, Q4_0 and Q5_0: the reference-named entries over Q8_1
// slots and their _q8_0 twins over Q8_0 blocks.
#include "fused.h"

extern "C" {
QMM_DEFINE_FUSED(q8_0, QMM_TYPE_Q8_0, kActSlots, )
QMM_DEFINE_FUSED(q4_0, QMM_TYPE_Q4_0, kActSlots, )
QMM_DEFINE_FUSED(q5_0, QMM_TYPE_Q5_0, kActSlots, )
QMM_DEFINE_FUSED(q8_0, QMM_TYPE_Q8_0, kActQ8_0, _q8_0)
QMM_DEFINE_FUSED(q4_0, QMM_TYPE_Q4_0, kActQ8_0, _q8_0)
QMM_DEFINE_FUSED(q5_0, QMM_TYPE_Q5_0, kActQ8_0, _q8_0)
}
