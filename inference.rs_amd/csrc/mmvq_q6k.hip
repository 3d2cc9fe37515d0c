// Decode matvec entries of Q6_K weights: the plain, one-launch, MoE, indexed and fused-MoE entries and the tensor-core entries.  The kernels and their launch logic are in mmvq.h.
#include "mmvq.h"

extern "C" {
QMM_MMVQ_PLAIN(q6_k, QMM_TYPE_Q6K, kActSlots, )
QMM_MMVQ_QUANTIZE_PLAIN(q6_k, QMM_TYPE_Q6K)
QMM_MMVQ_FUSED_QUANTIZE(q6_k, QMM_TYPE_Q6K)
QMM_MMVQ_MOE(q6_k, QMM_TYPE_Q6K, kActSlots, )
QMM_MMVQ_INDEXED(q6k, QMM_TYPE_Q6K, kActSlots, q8_1)
QMM_MOE_GEMV(q6k, QMM_TYPE_Q6K)
QMM_MMVQ_TC(q6_k, QMM_TYPE_Q6K)
}
