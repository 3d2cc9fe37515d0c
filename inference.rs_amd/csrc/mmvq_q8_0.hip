// Decode matvec entries of Q8_0 weights: the reference-named plain, MoE, indexed and fused-MoE entries over Q8_1 slots, their _q8_0 twins over Q8_0 blocks, and the one-launch entries.  The kernels and their launch logic are in mmvq.h.
#include "mmvq.h"

extern "C" {
QMM_MMVQ_PLAIN(q8_0, QMM_TYPE_Q8_0, kActSlots, )
QMM_MMVQ_MOE(q8_0, QMM_TYPE_Q8_0, kActSlots, )
QMM_MMVQ_INDEXED(q8_0, QMM_TYPE_Q8_0, kActSlots, q8_1)
QMM_MOE_GEMV(q8_0, QMM_TYPE_Q8_0)
QMM_MMVQ_PLAIN(q8_0, QMM_TYPE_Q8_0, kActQ8_0, _q8_0)
QMM_MMVQ_MOE(q8_0, QMM_TYPE_Q8_0, kActQ8_0, _q8_0)
QMM_MMVQ_INDEXED(q8_0, QMM_TYPE_Q8_0, kActQ8_0, q8_0)
QMM_MMVQ_QUANTIZE_PLAIN(q8_0, QMM_TYPE_Q8_0)
QMM_MMVQ_FUSED_QUANTIZE(q8_0, QMM_TYPE_Q8_0)
}
