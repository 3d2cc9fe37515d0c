// Fused decode forms (fused.h) of the super-block types Q4_K, Q6_K, Q5_K and IQ4_XS, over Q8_1 slots.
#include "fused.h"

extern "C" {
QMM_DEFINE_FUSED(q4_k, QMM_TYPE_Q4K, kActSlots, )
QMM_DEFINE_FUSED(q6_k, QMM_TYPE_Q6K, kActSlots, )
QMM_DEFINE_FUSED(q5_k, QMM_TYPE_Q5K, kActSlots, )
QMM_DEFINE_FUSED(iq4_xs, QMM_TYPE_IQ4_XS, kActSlots, )
}
