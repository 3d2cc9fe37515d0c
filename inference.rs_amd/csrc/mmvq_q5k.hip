// Decode matvec entries of Q5_K and IQ4_XS weights: the plain and MoE entries (Q5_K also the indexed and fused-MoE ones).  The kernels and their launch logic are in mmvq.h.
#include "mmvq.h"

extern "C" {
QMM_MMVQ_PLAIN(q5_k, QMM_TYPE_Q5K, kActSlots, )
QMM_MMVQ_MOE(q5_k, QMM_TYPE_Q5K, kActSlots, )
QMM_MMVQ_INDEXED(q5k, QMM_TYPE_Q5K, kActSlots, q8_1)
QMM_MOE_GEMV(q5k, QMM_TYPE_Q5K)
QMM_MMVQ_PLAIN(iq4_xs, QMM_TYPE_IQ4_XS, kActSlots, )
QMM_MMVQ_MOE(iq4_xs, QMM_TYPE_IQ4_XS, kActSlots, )
}
