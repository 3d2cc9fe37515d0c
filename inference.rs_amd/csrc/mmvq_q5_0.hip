// Decode matvec entries of Q5_0 weights: the reference-named plain, MoE, indexed and fused-MoE entries over Q8_1 slots and their _q8_0 twins over Q8_0 blocks.  The kernels and their launch logic are in mmvq.h.
#include "mmvq.h"

extern "C" {
QMM_MMVQ_PLAIN(q5_0, QMM_TYPE_Q5_0, kActSlots, )
QMM_MMVQ_MOE(q5_0, QMM_TYPE_Q5_0, kActSlots, )
QMM_MMVQ_INDEXED(q5_0, QMM_TYPE_Q5_0, kActSlots, q8_1)
QMM_MOE_GEMV(q5_0, QMM_TYPE_Q5_0)
QMM_MMVQ_PLAIN(q5_0, QMM_TYPE_Q5_0, kActQ8_0, _q8_0)
QMM_MMVQ_MOE(q5_0, QMM_TYPE_Q5_0, kActQ8_0, _q8_0)
QMM_MMVQ_INDEXED(q5_0, QMM_TYPE_Q5_0, kActQ8_0, q8_0)
}
