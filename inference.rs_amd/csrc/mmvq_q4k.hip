// Decode matvec entries of Q4_K weights: the plain, one-launch, MoE, indexed and fused-MoE entries and the tensor-core entries.  The kernels and their launch logic are in mmvq.h.
#include "mmvq.h"

extern "C" {
QMM_MMVQ_PLAIN(q4_k, QMM_TYPE_Q4K, kActSlots, )
QMM_MMVQ_QUANTIZE_PLAIN(q4_k, QMM_TYPE_Q4K)
QMM_MMVQ_FUSED_QUANTIZE(q4_k, QMM_TYPE_Q4K)
// q and k Q4_K, v Q6_K (the mix of Q4_K_M files, whose attn_v tensors are Q6_K)
void launch_mmvq_gguf_q4_k_q6_k_f32_fused_qkv_quantize(const void *vx_q, const void *vx_k, const void *vx_v,
                                                       const float *x, void *q_dst, void *k_dst, void *v_dst,
                                                       int ncols_x, int nrows_q, int nrows_k, int nrows_v,
                                                       int stride_col_x, int b_size, void *stream) {
  fused_qkv_quantize_t<QMM_TYPE_Q4K, QMM_TYPE_Q6K, out_f32>(vx_q, vx_k, vx_v, x, q_dst, k_dst, v_dst, ncols_x, nrows_q,
                                                            nrows_k, nrows_v, stride_col_x, b_size, stream,
                                                            "mmvq_q4_k_q6_k_f32_fused_qkv_quantize");
}
QMM_MMVQ_MOE(q4_k, QMM_TYPE_Q4K, kActSlots, )
QMM_MMVQ_INDEXED(q4k, QMM_TYPE_Q4K, kActSlots, q8_1)
QMM_MOE_GEMV(q4k, QMM_TYPE_Q4K)
QMM_MMVQ_TC(q4_k, QMM_TYPE_Q4K)
}
