// Internal entry of the few-row MFMA matmul (skinny.hip), used by the decode launchers.
#pragma once

#include <hip/hip_runtime.h>

#include "qmm_blocks.h"

// From this many activation rows on, K-quant weights go through the MFMA few-row kernel, which decodes each weight
// block once for all rows (measured crossover on MI355X: Q4_K 4 rows, Q6_K 3).
#ifndef QMM_SKINNY_MIN_ROWS_Q4K
#define QMM_SKINNY_MIN_ROWS_Q4K 4
#endif
#ifndef QMM_SKINNY_MIN_ROWS_Q6K
#define QMM_SKINNY_MIN_ROWS_Q6K 3
#endif
inline int qmm_skinny_min_rows(int type) {
  return type == QMM_TYPE_Q6K ? QMM_SKINNY_MIN_ROWS_Q6K : QMM_SKINNY_MIN_ROWS_Q4K;
}

// Decode-layout activations (b rows of Q8_K blocks, stride_col_y blocks apart) against Q4_K / Q6_K weights;
// dst[j * stride_col_dst + row] of element type out_type (QMM_TYPE_F32 / F16 / BF16).  Returns false, launching
// nothing, for a case it does not serve (other weight types, b outside 1..32, K not a multiple of 256).
bool qmm_skinny_decode(int type, int out_type, const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x,
                       int stride_col_y, int stride_col_dst, int b, hipStream_t s);

// The same for the fused GLU form: dst[j * stride_col_dst + row] = act(W_gate . y_j) * (W_up . y_j).
bool qmm_skinny_glu(int type, int out_type, const void *vx_gate, const void *vx_up, const void *vy, void *dst,
                    int ncols_x, int nrows_x, int stride_col_y, int stride_col_dst, int b, int activation,
                    hipStream_t s);

// The same over the tensor-core entries' activation layout (rows of ncols_x / 256 blocks {f32 d; int8 qs[256]},
// units.h), for launch_mmvq_tc_gguf_<t>_*_plain.
bool qmm_skinny_tc(int type, int out_type, const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x,
                   int stride_col_dst, int b, hipStream_t s);

// Expert-grouped matmul (launch_mmq_gguf_<t>_moe) over prefill-layout activations when the experts receive few
// rows each: at most QMM_SKINNY_MOE_ROWS on average.  dst[ids_dst[m] * ldd + n], f32.  Returns false, launching
// nothing, for a case it does not serve.  0 (the default): never -- the grouped tile kernel's 32-row tiles with
// weights staged in LDS measured faster (MI355X, 8 x Q4_K 14336x4096 / 4096x14336 experts, 64 tokens top-2: 307
// against 319 us for the MoE step)
// Waves per workgroup of the GLU form (half on the gate rows, half on the up rows, each half splitting K).  Measured on
// MI355X, 2 x Q4_K 14336x4096: 4 waves 28.7 / 30.0 / 33.9 / 41.2 us at b = 4 / 8 / 16 / 32, against 31.0 / 32.5 /
// 36.5 / 42.9 us with 8 and 35.7 / 36.0 / 36.2 / 41.0 us with 2.
#ifndef QMM_SKINNY_GLU_NW
#define QMM_SKINNY_GLU_NW 4
#endif
#ifndef QMM_SKINNY_MOE_ROWS
#define QMM_SKINNY_MOE_ROWS 0
#endif
bool qmm_skinny_moe(int type, const void *x, const void *y, const int32_t *ids_dst, const int32_t *bounds, float *dst,
                    int64_t ncols_x, int64_t nrows_x, int64_t w_row_bytes, int64_t ncols_dst, int64_t ldd,
                    int64_t num_experts, hipStream_t s);
