// Decode matvec entries of Q4_K weights: the plain, one-launch, MoE, indexed and fused-MoE entries and the tensor-core entries.  The kernels and their launch logic are in mmvq.h.
#include "mmvq.h"

extern "C" {
QMM_MMVQ_PLAIN(q4_k, QMM_TYPE_Q4K, kActSlots, )
QMM_MMVQ_QUANTIZE_PLAIN(q4_k, QMM_TYPE_Q4K)
QMM_MMVQ_MOE(q4_k, QMM_TYPE_Q4K, kActSlots, )
QMM_MMVQ_INDEXED(q4k, QMM_TYPE_Q4K, kActSlots, q8_1)
QMM_MOE_GEMV(q4k, QMM_TYPE_Q4K)
QMM_MMVQ_TC(q4_k, QMM_TYPE_Q4K)
}
