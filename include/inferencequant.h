/*
 * libinferencequant.so -- the C ABI of the MI355X (gfx950) GGUF quantized-linear kernels.
 *
 * Every entry point has the argument list of the inference.rs kernel-library symbol it replaces
 * (crates/inference-quant/src/gguf/ffi.rs, bound through inference_tensor::kernel_library!,
 * crates/inference-tensor/src/kernel_library.rs:315-393).  Pointers are device pointers unless
 * noted; `stream` is a hipStream_t (null = the default stream).  The caller owns every buffer and
 * no entry point allocates device memory, as in the reference.
 *
 * Activation blocks.  The reference quantizes activations on the GPU into scratch buffers it sizes for Q8_1 (36 bytes
 * per 32 values for the decode matvec, fast_mmvq.rs:17-18, 534-542; 144 bytes per 128 values plus 128 * 144 for
 * the prefill matmul, fast_mmq.rs:20-22, 679-691), and its quantizers cannot know which weight type will read them.
 * Its CPU QMatMul -- the parity oracle -- quantizes K-quant activations to Q8_K and Q8_0-family activations to Q8_0
 * (k_quants.rs:2824-2830); both forms of one activation do not fit one Q8_1-sized buffer.  So:
 *   - the reference-named quantizers (launch_mmvq_gguf_quantize_q8_1_*, launch_mmq_quantize_q8_1_*) write Q8_K
 *     (BlockQ8K::from_float, bit-exact) in layouts that fit the reference's buffers, and every reference-named
 *     matvec / matmul reads them: the K-quant types (Q4_K, Q5_K, Q6_K, IQ4_XS) then give the CPU QMatMul's result
 *     within f32 summation order; the 32-value types (Q8_0, Q4_0, Q5_0) dot each 32 values of the same Q8_K
 *     activation, with the f32 scale of its 256, against their blocks -- a finer-than-Q8_1, coarser-than-Q8_0
 *     activation quantization;
 *   - the 32-value types also have _q8_0 entries (launch_mmvq_gguf_quantize_q8_0_* with ..._plain_q8_0, _moe_q8_0,
 *     _fused_*_q8_0, launch_indexed_moe_forward_<t>_q8_0; launch_mmq_quantize_q8_0 with launch_mmq_gguf_<t>_q8_0,
 *     _moe_q8_0) over Q8_0 blocks, which give their CPU QMatMul's result; the C++ host layer uses those.
 * Layouts (qmm_blocks.h):
 *   decode, reference names: row r = bytes [r * 36 * stride_col_y, ...), kx_padded / 256 qmm_block_q8ks of 288 bytes
 *       {f32 d; int8 qs[256]; int16 s32[8] (sums of 32); 12 zero bytes}; stride_col_y = kx_padded / 32 as the
 *       reference passes it (a multiple of 8).
 *   decode, _q8_0: row r = qmm_block_q8_0 [r * stride_col_y, ...) (34 bytes per 32 values).
 *   prefill (launch_mmq_quantize_*): per channel, for ne1 rows and nsb = ceil(ne00 / 256) (whatever ne0, the caller's
 *       k_padded: the matmuls are given K and read that many): qs[nsb][ne1][256] int8, then
 *       reference names: d[nsb][ne1] f32, s32[nsb][ne1][8] int16 sums of 32  (276 bytes per 256 values)
 *       _q8_0:           d[nsb][ne1][8] f16, one per 32 values              (272 bytes per 256 values)
 *
 * Errors.  A launcher given arguments it cannot serve launches nothing, records a message readable
 * with qmm_last_error(), and (for the int-returning ones) returns a nonzero code.  The reference's
 * launchers are void and unchecked (gguf/cuda.rs:187-193 checks only the reduce); its Rust callers
 * validate shapes first, as the C++ host (inference.rs_amd/host) does here.
 */
#ifndef INFERENCEQUANT_H
#define INFERENCEQUANT_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Build id every kernel library exports (kernel_library.rs:8, 288-297). */
extern const char inference_kernel_build_id[];

/* Last error recorded on the calling host thread, "" if none; cleared by qmm_clear_error().
 * No counterpart in the reference, whose launchers report nothing. */
const char *qmm_last_error(void);
void qmm_clear_error(void);

/* The form the plain decode matvec's persistent route takes for weight type `type`, rows of ncols_x values and nc
 * (1..8) columns per pass, from the rule the launchers apply; nothing is launched.  out[0]: 0 k_mmvq_p, 1 k_mmvq_p2,
 * 2 k_mmvq (units in passes); out[1]: units per lane the kernel holds; out[2]: 1 if it reads every unit without a
 * guard; out[3]: the row's units.  act_q8_0 selects the 32-value types' _q8_0 entries.  Returns 0, or -1 with the
 * error recorded.  No counterpart in the reference: for tests of the guard choice. */
int qmm_decode_form(int type, int ncols_x, int nc, int act_q8_0, int *out);

/* ------------------------------------------------------------------ decode activation quantizers
 * launch_mmvq_gguf_quantize_q8_1_{bf16,f16,f32} (gguf/ffi.rs:602-630; kernel mmvq_gguf/mmvq_quantize.cu:10-145; host
 * fast_mmvq.rs:534-565, gguf/cuda.rs:196-242): x = num_rows rows of kx values (row stride kx); vy = num_rows rows of
 * kx_padded / 256 Q8_1-slot blocks (36 * kx_padded / 32 bytes per row, the reference's scratch), zero beyond kx.
 * kx_padded a multiple of 256, at least kx (the reference passes pad(kx, 512)).  BlockQ8K::from_float
 * (k_quants.rs:2721-2760), bit-exact. */
void launch_mmvq_gguf_quantize_q8_1_f32(const void *x, void *vy, int kx, int kx_padded, int num_rows, void *stream);
void launch_mmvq_gguf_quantize_q8_1_f16(const void *x, void *vy, int kx, int kx_padded, int num_rows, void *stream);
void launch_mmvq_gguf_quantize_q8_1_bf16(const void *x, void *vy, int kx, int kx_padded, int num_rows, void *stream);
/* launch_mmvq_gguf_quantize_q8_0_{bf16,f16,f32}: no counterpart in the reference (whose GPU path quantizes to Q8_1
 * only); the same arguments, writing kx_padded / 32 qmm_block_q8_0 per row (kx_padded a multiple of 32), as
 * quantize_block32 (quantized/mod.rs:41-56), bit-exact: the activations of the 32-value types' _q8_0 entries. */
void launch_mmvq_gguf_quantize_q8_0_f32(const void *x, void *vy, int kx, int kx_padded, int num_rows, void *stream);
void launch_mmvq_gguf_quantize_q8_0_f16(const void *x, void *vy, int kx, int kx_padded, int num_rows, void *stream);
void launch_mmvq_gguf_quantize_q8_0_bf16(const void *x, void *vy, int kx, int kx_padded, int num_rows,
                                         void *stream);

/* ------------------------------------------------------------------ decode matvec
 * launch_mmvq_gguf_<t>_{bf16,f16,f32}_plain (gguf/ffi.rs:846-876; kernel mmvq_gguf.cuh:650-759, 1762-1834; host
 * fast_mmvq::plain, fast_mmvq.rs:534-650).  dst[j * stride_col_dst + row] = sum_k W[row, k] * Q(y_j)[k] for
 * j < b_size, row < nrows_x; vx = nrows_x rows of ncols_x / block values (GGUF bytes); vy = b_size rows from
 * launch_mmvq_gguf_quantize_q8_1_*, 36 * stride_col_y bytes apart.  The dtype suffix is dst's element type.
 * b_size 1..16, 1..32 for q4_k and q6_k (the reference's plain launcher takes 1..8, its tensor-core one up to 16).
 * Weight pointers: 16-byte aligned for q4_k / q5_k, 4-byte for iq4_xs, 2-byte for the rest.
 * launch_mmvq_gguf_{q8_0,q4_0,q5_0}_<dt>_plain_q8_0: the same over launch_mmvq_gguf_quantize_q8_0_* rows,
 * stride_col_y 34-byte blocks apart (no counterpart in the reference). */
#define QMM_DECLARE_MMVQ_PLAIN_SFX(t, sfx)                                                                        \
  void launch_mmvq_gguf_##t##_f32_plain##sfx(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x, \
                                             int stride_col_y, int stride_col_dst, int b_size, void *stream);    \
  void launch_mmvq_gguf_##t##_f16_plain##sfx(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x, \
                                             int stride_col_y, int stride_col_dst, int b_size, void *stream);    \
  void launch_mmvq_gguf_##t##_bf16_plain##sfx(const void *vx, const void *vy, void *dst, int ncols_x,            \
                                              int nrows_x, int stride_col_y, int stride_col_dst, int b_size,     \
                                              void *stream);
#define QMM_DECLARE_MMVQ_PLAIN(t) QMM_DECLARE_MMVQ_PLAIN_SFX(t, )
QMM_DECLARE_MMVQ_PLAIN(q8_0)
QMM_DECLARE_MMVQ_PLAIN(q4_k)
QMM_DECLARE_MMVQ_PLAIN(q6_k)
QMM_DECLARE_MMVQ_PLAIN_SFX(q8_0, _q8_0)
/* ------------------------------------------------------------------ tensor-core matvec entries
 * launch_mmvq_tc_quantize_{bf16,f16,f32} (gguf/ffi.rs:632-652) and launch_mmvq_tc_gguf_{q4_k,q6_k}_<dt>_plain
 * (gguf/ffi.rs:966-998), the pair fast_mmvq::plain routes 1..16 rows of a Q4_K / Q6_K weight to
 * (fast_mmvq.rs:505-513, 1897-1930).  The quantizer writes num_rows rows of kx values (kx a multiple of 256) as
 * kx / 256 blocks {f32 d; int8 qs[256]} of 260 bytes each: BlockQ8K::from_float's d and qs, bit-exact, without
 * the bsums, so b rows fit the reference's scratch of (kx / 32) * 288 bytes per 8-row half
 * (fast_mmvq.rs:92-93, 1903-1908).  The matvec reads b_size (1..32; the reference passes at most 16) such rows and writes
 * dst[j * stride_col_dst + row] as the _plain entries do; it sums the int8 values itself, so the integer dots are
 * those of the decode layout.  cfg (the reference's CUDA tile shape) is accepted and unused. */
void launch_mmvq_tc_quantize_f32(const void *x, void *vy, int kx, int num_rows, void *stream);
void launch_mmvq_tc_quantize_f16(const void *x, void *vy, int kx, int num_rows, void *stream);
void launch_mmvq_tc_quantize_bf16(const void *x, void *vy, int kx, int num_rows, void *stream);
#define QMM_DECLARE_MMVQ_TC(t)                                                                                    \
  void launch_mmvq_tc_gguf_##t##_f32_plain(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x, \
                                           int stride_col_dst, int b_size, int cfg, void *stream);              \
  void launch_mmvq_tc_gguf_##t##_f16_plain(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x, \
                                           int stride_col_dst, int b_size, int cfg, void *stream);              \
  void launch_mmvq_tc_gguf_##t##_bf16_plain(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x,\
                                            int stride_col_dst, int b_size, int cfg, void *stream);
QMM_DECLARE_MMVQ_TC(q4_k)
QMM_DECLARE_MMVQ_TC(q6_k)

/* The adjacent GGUF types on the same decode kernels (gguf/ffi.rs:1158-1169 gguf_standard_types q4_0, q5_0, q5_k;
 * 1265-1267 gguf_iq_types iq4_xs; host fast_mmvq.rs:40-81, 214-298), with the _q8_0 forms of q4_0 / q5_0.  Q5_K and
 * IQ4_XS dot Q8_K activations on the CPU (k_quants.rs:2145-2232, cpu_dot.rs:416-440), Q4_0 and Q5_0 Q8_0 blocks. */
QMM_DECLARE_MMVQ_PLAIN(q4_0)
QMM_DECLARE_MMVQ_PLAIN(q5_0)
QMM_DECLARE_MMVQ_PLAIN(q5_k)
QMM_DECLARE_MMVQ_PLAIN(iq4_xs)
QMM_DECLARE_MMVQ_PLAIN_SFX(q4_0, _q8_0)
QMM_DECLARE_MMVQ_PLAIN_SFX(q5_0, _q8_0)

/* ------------------------------------------------------------------ decode matvec with its own quantization
 * launch_mmvq_gguf_<t>_{bf16,f16,f32}_quantize_plain: no counterpart in the reference, whose decode makes two
 * launches, launch_mmvq_gguf_quantize_q8_1_<dt> then launch_mmvq_gguf_<t>_<dt>_plain (fast_mmvq.rs:534-565,
 * gguf/ffi.rs:602-640, 846-876).  This one takes the f32 activation rows x[j * stride_col_x + k] (j < b_size,
 * k < ncols_x) and gives the same dst, bit for bit, as launch_mmvq_gguf_quantize_q8_1_f32 followed by
 * launch_mmvq_gguf_<t>_<dt>_plain (q4_k, q6_k) or launch_mmvq_gguf_quantize_q8_0_f32 followed by
 * launch_mmvq_gguf_q8_0_<dt>_plain_q8_0, in one launch and without the activation scratch buffer.  b_size 1 or 2
 * with ncols_x at most 4096, or b_size 1 with ncols_x at most 16384 (x then 16-byte aligned); ncols_x a multiple
 * of 64 for Q8_0. */
#define QMM_DECLARE_MMVQ_QUANTIZE_PLAIN(t)                                                                        \
  void launch_mmvq_gguf_##t##_f32_quantize_plain(const void *vx, const float *x, void *dst, int ncols_x,          \
                                                 int nrows_x, int stride_col_x, int stride_col_dst, int b_size,  \
                                                 void *stream);                                                  \
  void launch_mmvq_gguf_##t##_f16_quantize_plain(const void *vx, const float *x, void *dst, int ncols_x,          \
                                                 int nrows_x, int stride_col_x, int stride_col_dst, int b_size,  \
                                                 void *stream);                                                  \
  void launch_mmvq_gguf_##t##_bf16_quantize_plain(const void *vx, const float *x, void *dst, int ncols_x,         \
                                                  int nrows_x, int stride_col_x, int stride_col_dst, int b_size, \
                                                  void *stream);
QMM_DECLARE_MMVQ_QUANTIZE_PLAIN(q8_0)
QMM_DECLARE_MMVQ_QUANTIZE_PLAIN(q4_k)
QMM_DECLARE_MMVQ_QUANTIZE_PLAIN(q6_k)

/* launch_mmvq_gguf_<t>_<dt>_fused_glu_quantize and _fused_qkv_quantize (t = q8_0, q4_k, q6_k; no counterpart in the
 * reference): the fused GLU / QKV decode forms over f32 activations x [b_size rows, stride_col_x apart] that the
 * launch quantizes itself, once per workgroup into LDS (the decode quantizers' blocks, bit for bit), instead of the
 * quantizer launch before them; the same output bits as that quantizer followed by _fused_glu / _fused_qkv.
 * b_size 1 or 2, ncols_x <= 4096 (Q8_0: a multiple of 64).  _fused_glu_quantize: dst[j * stride_col_dst + row] =
 * act(W_gate . x_j) * (W_up . x_j), activation as _fused_glu.  _fused_qkv_quantize: q_dst[j * nrows_q + row] and
 * likewise k, v.  launch_mmvq_gguf_q4_k_q6_k_f32_fused_qkv_quantize: the same with Q4_K q / k and Q6_K v weights. */
#define QMM_DECLARE_MMVQ_FUSED_QUANTIZE_DT(t, dt)                                                                 \
  void launch_mmvq_gguf_##t##_##dt##_fused_glu_quantize(const void *vx_gate, const void *vx_up, const float *x,     \
                                                        void *dst, int ncols_x, int nrows_x, int stride_col_x,      \
                                                        int stride_col_dst, int b_size, int activation,             \
                                                        void *stream);                                              \
  void launch_mmvq_gguf_##t##_##dt##_fused_qkv_quantize(const void *vx_q, const void *vx_k, const void *vx_v,       \
                                                        const float *x, void *q_dst, void *k_dst, void *v_dst,      \
                                                        int ncols_x, int nrows_q, int nrows_k, int nrows_v,         \
                                                        int stride_col_x, int b_size, void *stream);
#define QMM_DECLARE_MMVQ_FUSED_QUANTIZE(t)     \
  QMM_DECLARE_MMVQ_FUSED_QUANTIZE_DT(t, f32)   \
  QMM_DECLARE_MMVQ_FUSED_QUANTIZE_DT(t, f16)   \
  QMM_DECLARE_MMVQ_FUSED_QUANTIZE_DT(t, bf16)
QMM_DECLARE_MMVQ_FUSED_QUANTIZE(q8_0)
QMM_DECLARE_MMVQ_FUSED_QUANTIZE(q4_k)
QMM_DECLARE_MMVQ_FUSED_QUANTIZE(q6_k)
void launch_mmvq_gguf_q4_k_q6_k_f32_fused_qkv_quantize(const void *vx_q, const void *vx_k, const void *vx_v,
                                                       const float *x, void *q_dst, void *k_dst, void *v_dst,
                                                       int ncols_x, int nrows_q, int nrows_k, int nrows_v,
                                                       int stride_col_x, int b_size, void *stream);

/* ------------------------------------------------------------------ fused decode forms
 * launch_mmvq_gguf_<t>_{bf16,f16,f32}_fused_glu (gguf/ffi.rs:1032-1069; kernel mmvq_gguf.cuh:761-842):
 * dst[j * stride_col_dst + row] = act(W_gate[row] . Q(y_j)) * (W_up[row] . Q(y_j)) for j < b_size (1..16; 1..32 for
 * q4_k / q6_k), activation 0 SiLU, 1 GELU (tanh form), 2 ReLU, 3 GELU (erf form), 4 sigmoid; vy as for _plain.
 * launch_mmvq_gguf_<t>_{bf16,f16,f32}_fused_qkv (gguf/ffi.rs:1071-1118; kernel mmvq_gguf.cuh:844-959):
 * q_dst[j * nrows_q + row] = W_q[row] . Q(y_j), likewise k and v, one launch over one activation.
 * For every type of gguf_standard_types / gguf_iq_types served here; the _q8_0 forms of the 32-value types read
 * launch_mmvq_gguf_quantize_q8_0_* rows. */
#define QMM_DECLARE_MMVQ_FUSED_DT(t, dt, sfx)                                                                  \
  void launch_mmvq_gguf_##t##_##dt##_fused_glu##sfx(const void *vx_gate, const void *vx_up, const void *vy,    \
                                                    void *dst, int ncols_x, int nrows_x, int stride_col_y,    \
                                                    int stride_col_dst, int b_size, int activation,           \
                                                    void *stream);                                            \
  void launch_mmvq_gguf_##t##_##dt##_fused_qkv##sfx(const void *vx_q, const void *vx_k, const void *vx_v,      \
                                                    const void *vy, void *q_dst, void *k_dst, void *v_dst,     \
                                                    int ncols_x, int nrows_q, int nrows_k, int nrows_v,        \
                                                    int stride_col_y, int b_size, void *stream);
#define QMM_DECLARE_MMVQ_FUSED_SFX(t, sfx)   \
  QMM_DECLARE_MMVQ_FUSED_DT(t, bf16, sfx)    \
  QMM_DECLARE_MMVQ_FUSED_DT(t, f16, sfx)     \
  QMM_DECLARE_MMVQ_FUSED_DT(t, f32, sfx)
#define QMM_DECLARE_MMVQ_FUSED(t) QMM_DECLARE_MMVQ_FUSED_SFX(t, )
QMM_DECLARE_MMVQ_FUSED(q8_0)
QMM_DECLARE_MMVQ_FUSED(q4_k)
QMM_DECLARE_MMVQ_FUSED(q6_k)
QMM_DECLARE_MMVQ_FUSED(q4_0)
QMM_DECLARE_MMVQ_FUSED(q5_0)
QMM_DECLARE_MMVQ_FUSED(q5_k)
QMM_DECLARE_MMVQ_FUSED(iq4_xs)
QMM_DECLARE_MMVQ_FUSED_SFX(q8_0, _q8_0)
QMM_DECLARE_MMVQ_FUSED_SFX(q4_0, _q8_0)
QMM_DECLARE_MMVQ_FUSED_SFX(q5_0, _q8_0)

/* ------------------------------------------------------------------ MoE decode matvec
 * launch_mmvq_gguf_<t>_moe (gguf/ffi.rs:877-893; kernel mmvq_gguf.cuh:961-1038, 1600-1643).
 * For routed pair p < n_pairs: expert e = ids[p] (u32), activation row p / y_div of vy (as for _plain), weights
 * vx_gate + e * expert_stride bytes.
 *   vx_up == NULL: dst[p * nrows_x + row] = W_gate[e] . y
 *   vx_up != NULL: dst[p * nrows_x + row] = act(W_gate[e] . y) * (W_up[e] . y), activation 0 SiLU,
 *                  1 GELU (tanh form), 2 ReLU, 3 GELU (erf form), 4 sigmoid (glu_activation.cuh).
 * Expert ids must be valid (< the number of experts behind vx_gate); they are not checked on the device, as in
 * the reference.
 * `grouped` only orders the grid in the reference (pairs sharing an expert run together); accepted, and
 * the gfx950 grid always walks pairs innermost.
 * launch_mmvq_gguf_<t>_moe_wsum: no counterpart in the reference, whose MoE decode runs the down projection
 * (launch_mmvq_gguf_<t>_moe) and then the weighted sum over a token's routes (launch_moe_weighted_reduce_flat;
 * inference-nn/src/moe/experts/backends.rs:2418, gguf/cuda.rs:627-1000) as two launches.  This is the two in one:
 * dst[t * nrows_x + row] = sum over s < topk, in order, of weights[t * topk + s] * (W[ids[t * topk + s]][row] .
 * y[t * topk + s]) for t < n_tokens, with the same arithmetic as the two launches; a route of weight zero is not
 * read.  vy holds n_tokens * topk activation rows, ids u32.
 * The _q8_0 forms of the 32-value types read launch_mmvq_gguf_quantize_q8_0_* rows. */
#define QMM_DECLARE_MMVQ_MOE_SFX(t, sfx)                                                                         \
  void launch_mmvq_gguf_##t##_moe##sfx(const void *vx_gate, const void *vx_up, int64_t expert_stride,           \
                                       const void *vy, const void *ids, float *dst, int ncols_x, int nrows_x,   \
                                       int stride_col_y, int y_div, int n_pairs, int activation, int grouped,   \
                                       void *stream);                                                           \
  void launch_mmvq_gguf_##t##_moe_wsum##sfx(const void *vx, int64_t expert_stride, const void *vy,              \
                                            const void *ids, const float *weights, float *dst, int ncols_x,     \
                                            int nrows_x, int stride_col_y, int n_tokens, int topk, void *stream);
#define QMM_DECLARE_MMVQ_MOE(t) QMM_DECLARE_MMVQ_MOE_SFX(t, )
QMM_DECLARE_MMVQ_MOE(q8_0)
QMM_DECLARE_MMVQ_MOE(q4_k)
QMM_DECLARE_MMVQ_MOE(q6_k)
QMM_DECLARE_MMVQ_MOE(q4_0)
QMM_DECLARE_MMVQ_MOE(q5_0)
QMM_DECLARE_MMVQ_MOE(q5_k)
QMM_DECLARE_MMVQ_MOE(iq4_xs)
QMM_DECLARE_MMVQ_MOE_SFX(q8_0, _q8_0)
QMM_DECLARE_MMVQ_MOE_SFX(q4_0, _q8_0)
QMM_DECLARE_MMVQ_MOE_SFX(q5_0, _q8_0)

/* ------------------------------------------------------------------ fused MoE decode
 * The reference's MoE decode route (inference_quant::indexed_moe_fused_decode, gguf/cuda.rs:1355-1520, taken by
 * MoEExperts::forward_cuda for decode-phase batches, inference-nn/src/moe/experts/backends.rs:1440-1480,
 * 1866-1935; kernels indexed_moe.cu:1189-1330), same arguments (gguf/ffi.rs:280-440).  Inputs are
 * launch_mmvq_gguf_quantize_q8_1_* rows of k_padded values (a multiple of 256); outputs f32; the experts' weight
 * tensors [E, n, k] in GGUF bytes.
 *   launch_moe_gemv_fused_gate_up_<t>_q8_1: all_outputs[p * n + row] = act(W_gate[e] . x_b) * (W_up[e] . x_b) for
 *     route p = b * topk + s < batch * topk, e = indices[p], x_b = input row b; act_type 0 is GELU (tanh form) and
 *     every other value SiLU, as the reference's kernel reads it (indexed_moe.cu:1254-1256).
 *   launch_moe_gemv_down_aggregate_<t>_q8_1: all_outputs[b * n + row] += sum over s < topk of topk_weights[p] *
 *     (W[e] . x_p), x_p = input row p.  The reference adds each route's product with an atomic add into a buffer
 *     its caller zeroes first (gguf/cuda.rs:1475-1477); here the routes' products are summed in slot order and then
 *     added to the buffer, so the result does not depend on scheduling.  A route of weight zero is not read. */
#define QMM_DECLARE_MOE_GEMV(t)                                                                                  \
  void launch_moe_gemv_fused_gate_up_##t##_q8_1(const void *gate_weights, const void *up_weights,               \
                                                const void *all_inputs, const uint32_t *indices,                \
                                                float *all_outputs, int n, int k, int batch, int topk,          \
                                                int k_padded, int act_type, void *stream);                      \
  void launch_moe_gemv_down_aggregate_##t##_q8_1(const void *all_weights, const void *all_inputs,               \
                                                 const uint32_t *indices, const float *topk_weights,            \
                                                 float *all_outputs, int n, int k, int batch, int topk,         \
                                                 int k_padded, void *stream);
QMM_DECLARE_MOE_GEMV(q8_0)
QMM_DECLARE_MOE_GEMV(q4_0)
QMM_DECLARE_MOE_GEMV(q5_0)
QMM_DECLARE_MOE_GEMV(q4k)
QMM_DECLARE_MOE_GEMV(q5k)
QMM_DECLARE_MOE_GEMV(q6k)

/* ------------------------------------------------------------------ prefill activation quantizers
 * launch_mmq_quantize_q8_1_{D4,DS4,D2S6} (gguf/ffi.rs:657-700; kernel mmq_gguf/mmq_quantize.cu:98-195, 395-415; host
 * fast_mmq.rs:604-715), same arguments: x of type_x (0 f32, 1 f16, 30 bf16); output row i1 < ne1 of channel
 * (i2, i3) reads input row ids ? ids[i1] : i1 at x + i3*s03 + i2*s02 + row*s01 (element strides), ne00 valid values,
 * zero up to the next multiple of 256; ne0 (a multiple of 256, >= ne00; the reference passes pad(K, 512)) is checked
 * but does not shape the layout.  All three write the Q8_K tile layout above (276 bytes per 256 values: it fits the
 * reference's ne1 * ne0 / 128 * 144 + 128 * 144 bytes); the reference's
 * three scale layouts are distinctions of its own kernels.  BlockQ8K::from_float per 256 values, bit-exact. */
void launch_mmq_quantize_q8_1_D4(const void *x, const int32_t *ids, void *vy, int type_x, int64_t ne00, int64_t s01,
                                 int64_t s02, int64_t s03, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3,
                                 void *stream);
void launch_mmq_quantize_q8_1_DS4(const void *x, const int32_t *ids, void *vy, int type_x, int64_t ne00, int64_t s01,
                                  int64_t s02, int64_t s03, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3,
                                  void *stream);
void launch_mmq_quantize_q8_1_D2S6(const void *x, const int32_t *ids, void *vy, int type_x, int64_t ne00,
                                   int64_t s01, int64_t s02, int64_t s03, int64_t ne0, int64_t ne1, int64_t ne2,
                                   int64_t ne3, void *stream);
/* launch_mmq_quantize_q8k: no counterpart in the reference; the same arguments, writing `_q8k` tiles: the Q8_K tile
 * layout with the sums of each 16 values as f16 in place of the int16 sums of 32 (qs[nsb][ne1][256], d[nsb][ne1] f32,
 * h16[nsb][ne1][16] f16; 292 bytes per 256 values, more than the reference's MMQ scratch holds), which the `_q8k`
 * prefill entries of Q4_K and Q5_K read with no conversion of the sums. */
void launch_mmq_quantize_q8k(const void *x, const int32_t *ids, void *vy, int type_x, int64_t ne00, int64_t s01,
                             int64_t s02, int64_t s03, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3,
                             void *stream);
/* launch_mmq_quantize_q8_0: no counterpart in the reference; the same arguments, writing the Q8_0 tile layout
 * (quantize_block32 per 32 values, bit-exact): the activations of the 32-value types' _q8_0 prefill entries. */
void launch_mmq_quantize_q8_0(const void *x, const int32_t *ids, void *vy, int type_x, int64_t ne00, int64_t s01,
                              int64_t s02, int64_t s03, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3,
                              void *stream);

/* launch_mmq_quantize_glu_q8_1_{D4,DS4,D2S6}_f32 and launch_mmq_quantize_glu_q8_1_{D4,DS4,D2S6} (gguf/ffi.rs:700-776;
 * mmq_quantize.cu:230-330): output row i1 < ne1 = act(gate[r]) * up[r] for r = ids ? ids[i1] : i1 (row stride s01,
 * ne00 valid values, zero up to the next multiple of 256), quantized into the Q8_K tile layout.  activation: 0 SiLU, 1 GELU (tanh),
 * 2 ReLU, 3 GELU (erf), 4 sigmoid (glu_activation.cuh).  The _f32 forms take f32 gate / up; the others gate / up of
 * type_x (0 f32, 1 f16, 30 bf16), where act(gate) is rounded to that type and multiplied by up in it, as the
 * reference's mmq_glu_product does (mmq_quantize.cu:230-235).
 * launch_mmq_quantize_glu_q8_0_f32 (no counterpart in the reference): f32 gate / up into the Q8_0 tile layout.
 * launch_mmq_quantize_glu_q8k_f32 (no counterpart in the reference): f32 gate / up into the `_q8k` tile layout of
 * launch_mmq_quantize_q8k, for the `_q8k` prefill entries. */
#define QMM_DECLARE_MMQ_GLU(L)                                                                                    \
  void launch_mmq_quantize_glu_q8_1_##L##_f32(const float *gate, const float *up, const int32_t *ids, void *vy,   \
                                              int64_t ne00, int64_t s01, int64_t ne0, int64_t ne1, int activation, \
                                              void *stream);                                                      \
  void launch_mmq_quantize_glu_q8_1_##L(const void *gate, const void *up, const int32_t *ids, void *vy, int type_x, \
                                        int64_t ne00, int64_t s01, int64_t ne0, int64_t ne1, int activation,      \
                                        void *stream);
QMM_DECLARE_MMQ_GLU(D4)
QMM_DECLARE_MMQ_GLU(DS4)
QMM_DECLARE_MMQ_GLU(D2S6)
void launch_mmq_quantize_glu_q8_0_f32(const float *gate, const float *up, const int32_t *ids, void *vy, int64_t ne00,
                                      int64_t s01, int64_t ne0, int64_t ne1, int activation, void *stream);
void launch_mmq_quantize_glu_q8k_f32(const float *gate, const float *up, const int32_t *ids, void *vy, int64_t ne00,
                                     int64_t s01, int64_t ne0, int64_t ne1, int activation, void *stream);

/* ------------------------------------------------------------------ prefill matmul
 * launch_mmq_gguf_<t> (gguf/ffi.rs:902-918; host fast_mmq.rs:446-524, 604-715; kernel mmq_instance.cuh:
 * 217-256, mmq_gguf.cuh:3533-3875).  dst[col * stride_col_dst + row] for row < nrows_x (weight rows),
 * col < ncols_y (activation rows); x = weight rows of stride_row_x blocks; y = prefill-layout activations
 * with ne00 = ncols_x and ne1 = ncols_y.  type_dst 0 f32, 1 f16, 30 bf16.
 * Weight buffers: as in the reference, whose QTensor device allocations carry MATRIX_ROW_PADDING = 512 values of
 * padding (quantized/cuda.rs:25, 246-248), a kernel may read a few bytes past the last block -- here at most 4, by the
 * Q8_0 / Q4_0 / Q5_0 kernel for rows that are not whole 4-byte aligned superblocks -- so the buffer must extend at
 * least 4 bytes beyond the last row (the host QTensor pads by 512 values).
 * tmp_fixup: the caller's split-K workspace of nsm * 128 * 128 f32, as the reference sizes it (fast_mmq.rs:442-444;
 * nsm = the device's compute-unit count).  When the tile grid alone would leave compute units idle, the K range is
 * split, each split writes its partial sums to its own f32 plane there, and a second kernel adds the planes in split
 * order and stores dst: results are the same bits on every run, as with the reference's fixed-order stream-k fixup
 * (mmq_gguf.cuh:3610-3611, 3877-3930).  tmp_fixup NULL: no split.  cc, smpbo and warp_size are accepted, unused. */
#define QMM_DECLARE_MMQ(t)                                                                                     \
  void launch_mmq_gguf_##t(void *tmp_fixup, const void *x, const void *y, void *dst, int64_t ncols_x,          \
                           int64_t nrows_x, int64_t ncols_y, int64_t stride_row_x, int64_t stride_col_dst, int cc, \
                           int nsm, int64_t smpbo, int warp_size, int type_dst, void *stream);                  \
  void launch_mmq_gguf_##t##_moe(void *tmp_fixup, const void *x, const void *y, const int32_t *ids_dst,        \
                                 const int32_t *expert_bounds, void *dst, int64_t ncols_x, int64_t nrows_x,     \
                                 int64_t ncols_dst, int64_t stride_row_x, int64_t stride_col_dst,               \
                                 int64_t num_experts, int64_t ncols_max, int cc, int nsm, int64_t smpbo,        \
                                 int warp_size, void *stream);
QMM_DECLARE_MMQ(q8_0)
QMM_DECLARE_MMQ(q4_k)
QMM_DECLARE_MMQ(q6_k)
/* Q4_0 and Q5_0 (gguf/ffi.rs:906-955 gguf_mmq_type_library, gguf_standard_types): the Q8_0 kernel with their block
 * decoders */
QMM_DECLARE_MMQ(q4_0)
QMM_DECLARE_MMQ(q5_0)
/* Q5_K (gguf/ffi.rs:906-955 gguf_mmq_type_library; block k_quants.rs:200-206): the K-quant kernel with a third
 * weight plane for the fifth bit; weights 16-byte aligned */
QMM_DECLARE_MMQ(q5_k)
/* IQ4_XS (gguf/ffi.rs:906-952 gguf_mmq_type_library through gguf_iq_types, :1265-1267; mmq_instance_iq4_xs.cu): the
 * K-quant kernel with table values times (ls - 32) split into two int8 planes as Q6_K's; weights 4-byte aligned */
QMM_DECLARE_MMQ(iq4_xs)
/* launch_mmq_gguf_{q8_0,q4_0,q5_0}_q8_0 and _moe_q8_0: no counterpart in the reference; the same over the Q8_0 tile
 * layout (launch_mmq_quantize_q8_0) */
#define QMM_DECLARE_MMQ_Q8_0(t)                                                                                   \
  void launch_mmq_gguf_##t##_q8_0(void *tmp_fixup, const void *x, const void *y, void *dst, int64_t ncols_x,     \
                                  int64_t nrows_x, int64_t ncols_y, int64_t stride_row_x, int64_t stride_col_dst, \
                                  int cc, int nsm, int64_t smpbo, int warp_size, int type_dst, void *stream);    \
  void launch_mmq_gguf_##t##_moe_q8_0(void *tmp_fixup, const void *x, const void *y, const int32_t *ids_dst,     \
                                      const int32_t *expert_bounds, void *dst, int64_t ncols_x, int64_t nrows_x,  \
                                      int64_t ncols_dst, int64_t stride_row_x, int64_t stride_col_dst,            \
                                      int64_t num_experts, int64_t ncols_max, int cc, int nsm, int64_t smpbo,     \
                                      int warp_size, void *stream);
QMM_DECLARE_MMQ_Q8_0(q8_0)
QMM_DECLARE_MMQ_Q8_0(q4_0)
QMM_DECLARE_MMQ_Q8_0(q5_0)
/* launch_mmq_gguf_{q4_k,q5_k}_q8k: no counterpart in the reference; launch_mmq_gguf_<t> over `_q8k` tiles
 * (launch_mmq_quantize_q8k): the min term's activation sums come in the f16 form its MFMA takes, so the kernel skips
 * converting them (the same result, about 9% fewer vector instructions per superblock) */
void launch_mmq_gguf_q4_k_q8k(void *tmp_fixup, const void *x, const void *y, void *dst, int64_t ncols_x,
                              int64_t nrows_x, int64_t ncols_y, int64_t stride_row_x, int64_t stride_col_dst, int cc,
                              int nsm, int64_t smpbo, int warp_size, int type_dst, void *stream);
void launch_mmq_gguf_q5_k_q8k(void *tmp_fixup, const void *x, const void *y, void *dst, int64_t ncols_x,
                              int64_t nrows_x, int64_t ncols_y, int64_t stride_row_x, int64_t stride_col_dst, int cc,
                              int nsm, int64_t smpbo, int warp_size, int type_dst, void *stream);
/* launch_mmq_gguf_{q4_k,q5_k}_moe_q8k: no counterpart in the reference; launch_mmq_gguf_<t>_moe over `_q8k` tiles
 * (launch_mmq_quantize_q8k with the dispatch's row ids, or launch_mmq_quantize_glu_q8k_f32), the same results. */
void launch_mmq_gguf_q4_k_moe_q8k(void *tmp_fixup, const void *x, const void *y, const int32_t *ids_dst,
                                  const int32_t *expert_bounds, void *dst, int64_t ncols_x, int64_t nrows_x,
                                  int64_t ncols_dst, int64_t stride_row_x, int64_t stride_col_dst, int64_t num_experts,
                                  int64_t ncols_max, int cc, int nsm, int64_t smpbo, int warp_size, void *stream);
void launch_mmq_gguf_q5_k_moe_q8k(void *tmp_fixup, const void *x, const void *y, const int32_t *ids_dst,
                                  const int32_t *expert_bounds, void *dst, int64_t ncols_x, int64_t nrows_x,
                                  int64_t ncols_dst, int64_t stride_row_x, int64_t stride_col_dst, int64_t num_experts,
                                  int64_t ncols_max, int cc, int nsm, int64_t smpbo, int warp_size, void *stream);
/* launch_mmq_gguf_<t>_moe (gguf/ffi.rs:919-938; mmq_gguf.cuh:4020-4061): expert e's weights are
 * x + e * nrows_x * stride_row_x blocks; its activation columns are [expert_bounds[e], expert_bounds[e+1])
 * of y (the prefill layout with ne1 = expert_bounds[num_experts] rows, rows gathered in expert order by
 * the quantizer's ids); column c of the grouped product is written to dst[ids_dst[c] * stride_col_dst + row]
 * (f32).  ncols_max bounds the rows of any one expert. */

/* ------------------------------------------------------------------ op-level indexed MoE
 * launch_indexed_moe_forward_<t>_q8_1 (gguf/ffi.rs:60-224; kernel indexed_moe.cu:664-1000; host gguf/cuda.rs:259-498),
 * same arguments, inputs from launch_mmvq_gguf_quantize_q8_1_* with kx_padded = k_padded (a multiple of 256):
 * all_outputs[(b * topk + s) * n + row] = W[indices[b * topk + s]][row] . Q(x[b * input_dim1 + (input_dim1 == 1 ?
 * 0 : s)]) with W [E, n, k] GGUF bytes.  launch_indexed_moe_forward_{q8_0,q4_0,q5_0}_q8_0: the same over
 * launch_mmvq_gguf_quantize_q8_0_* rows (no counterpart in the reference). */
#define QMM_DECLARE_INDEXED(t, act)                                                                              \
  void launch_indexed_moe_forward_##t##_##act(const void *all_weights, const void *all_inputs,                  \
                                              const uint32_t *indices, float *all_outputs, int n, int k,        \
                                              int batch, int topk, int k_padded, int input_dim1, void *stream);
QMM_DECLARE_INDEXED(q8_0, q8_1)
QMM_DECLARE_INDEXED(q4k, q8_1)
QMM_DECLARE_INDEXED(q6k, q8_1)
QMM_DECLARE_INDEXED(q4_0, q8_1)
QMM_DECLARE_INDEXED(q5_0, q8_1)
QMM_DECLARE_INDEXED(q5k, q8_1)
QMM_DECLARE_INDEXED(q8_0, q8_0)
QMM_DECLARE_INDEXED(q4_0, q8_0)
QMM_DECLARE_INDEXED(q5_0, q8_0)

/* launch_gather_rows_u8 (gguf/ffi.rs:591-599; used by gguf/raw.rs:405 for embedding lookups on raw GGUF blocks;
 * kernel mmvq_gguf/gather_rows.cu): dst row r = src row ids[r] (u32), row_bytes bytes each, for r < n; rows is the
 * number of rows of src, and an id >= rows gives a zero row. */
void launch_gather_rows_u8(const void *src, const void *ids, void *dst, int64_t row_bytes, int64_t rows, int64_t n,
                           void *stream);

/* ------------------------------------------------------------------ MoE dispatch and reduce
 * launch_moe_dispatch (gguf/ffi.rs:227-238; moe_dispatch.cu:78-104): expert_bounds[num_experts + 1],
 * sorted_token_ids[pos] = flat route index, sorted_source_ids[pos] = route / topk, grouped by expert.
 * expert_counts / expert_cursors: caller-owned int32[num_experts] scratch. */
void launch_moe_dispatch(const int32_t *topk_ids, int32_t *expert_bounds, int32_t *sorted_token_ids,
                         int32_t *sorted_source_ids, int total_assignments, int num_experts, int topk,
                         int32_t *expert_counts, int32_t *expert_cursors, void *stream);

/* launch_moe_weighted_reduce_flat* (gguf/ffi.rs:240-276; moe_dispatch.cu:47-154):
 * out[t][h] = sum over slots s with w[t][s] != 0 of in[t][s][h] * w[t][s].  Returns 0 or a hipError_t. */
int launch_moe_weighted_reduce_flat(const void *inputs, const float *topk_weights, void *outputs, int num_tokens,
                                    int hidden, int topk, void *stream);
int launch_moe_weighted_reduce_flat_bf16(const void *inputs, const float *topk_weights, void *outputs,
                                         int num_tokens, int hidden, int topk, void *stream);
int launch_moe_weighted_reduce_flat_f16_input(const void *inputs, const float *topk_weights, void *outputs,
                                              int num_tokens, int hidden, int topk, void *stream);
int launch_moe_weighted_reduce_flat_bf16_input(const void *inputs, const float *topk_weights, void *outputs,
                                               int num_tokens, int hidden, int topk, void *stream);

/* ------------------------------------------------------------------ dequantization and the exact Q8_0 matvec
 * launch_dequantize_<t>_{f32,f16,bf16}: y[0..n) = the values of n / block_size consecutive blocks at x, as f32 or
 * rounded (nearest even) to f16 / bf16.  Replaces QCudaStorage::dequantize / dequantize_f16
 * (quantized/cuda.rs:31-135, 283-334) and its kernels dequantize_block_<t>_{f32,f16}
 * (inference-tensor-kernels/src/quantized.cu:440-608, 647-660), which the reference loads by name rather than
 * through a C launcher; the f32 values are bit-identical to the CPU to_float (k_quants.rs:905-921, 2096-2123,
 * 2649-2680).  n a multiple of the block size, y 16-byte aligned. */
#define QMM_DECLARE_DEQUANTIZE(t)                                                                                \
  void launch_dequantize_##t##_f32(const void *x, void *y, int64_t n, void *stream);                            \
  void launch_dequantize_##t##_f16(const void *x, void *y, int64_t n, void *stream);                            \
  void launch_dequantize_##t##_bf16(const void *x, void *y, int64_t n, void *stream);                           \
  /* get_rows_<t> (quantized.cu:900-975; host quantized/cuda.rs:150-240): dst row r (ne00 f32 values) = row    \
   * ids[r] of src0, whose rows are nb01 bytes apart; n_ids <= 65535 rows (the reference's grid.x) */           \
  void launch_get_rows_##t(const void *src0, const uint32_t *ids, float *dst, int64_t ne00, int64_t nb01,       \
                           int64_t n_ids, void *stream);
QMM_DECLARE_DEQUANTIZE(q8_0)
QMM_DECLARE_DEQUANTIZE(q4_k)
QMM_DECLARE_DEQUANTIZE(q6_k)
QMM_DECLARE_DEQUANTIZE(q4_0)
QMM_DECLARE_DEQUANTIZE(q5_0)
QMM_DECLARE_DEQUANTIZE(q5_k)

/* launch_dequantize_iq4_xs_{f32,f16,bf16} with the reference's own signature (gguf/ffi.rs:1125-1150, 1265-1267;
 * kernel mmvq_gguf.cuh:2128-2141, 2167-2174): the nrows * ncols values of contiguous IQ4_XS rows (ncols a multiple
 * of 256), value = (d * (ls - 32)) * kvalues_iq4nl[q] in f32, rounded to the output type. */
void launch_dequantize_iq4_xs_f32(const void *vx, void *dst, int64_t nrows, int64_t ncols, void *stream);
void launch_dequantize_iq4_xs_f16(const void *vx, void *dst, int64_t nrows, int64_t ncols, void *stream);
void launch_dequantize_iq4_xs_bf16(const void *vx, void *dst, int64_t nrows, int64_t ncols, void *stream);

/* launch_mmvq_gguf_q8_0_{bf16,f32}_exact (gguf/ffi.rs:1001-1022; host fast_mmvq.rs:415-472; kernel
 * mmvq_instance_q8_0.cu:15-146): dst[b][row] = sum_k d q_k x[b][k] with the activations x [b_size, ncols_x] left
 * unquantized (bf16 or f32), f32 sums, output in the input's dtype; b_size 1..8. */
void launch_mmvq_gguf_q8_0_f32_exact(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x,
                                     int b_size, void *stream);
void launch_mmvq_gguf_q8_0_bf16_exact(const void *vx, const void *vy, void *dst, int ncols_x, int nrows_x,
                                      int b_size, void *stream);

/* ------------------------------------------------------------------ MoE router
 * moe_router_topk_{f32,bf16,f16} (crates/inference-nn/src/cuda/ffi.rs:1137-1190; kernel
 * crates/inference-nn/kernels/cuda/sort.cu:1374-1725): logits [n_rows, n_experts] -> weights [n_rows, top_k] f32 and
 * ids [n_rows, top_k] u32.  score_mode 0 raw, 1 softmax, 2 sigmoid; selection = score + selection_bias (nullable),
 * ties to the lower expert; weight_mode 0 the score, 1 a softmax over the picked raw logits, 2 their sigmoid;
 * renormalize divides by max(sum, norm_min); weights are then scaled by output_scale * expert_scale[id] (nullable).
 * n_experts 1..1024, top_k 1..n_experts.  The stream is a hipStream_t passed as an integer, as the reference's. */
void moe_router_topk_f32(const float *logits, float *weights, uint32_t *ids, const float *selection_bias,
                         const float *expert_scale, int n_rows, int n_experts, int top_k, int score_mode,
                         int weight_mode, bool renormalize, bool clamp_logits, float clamp_min, float clamp_max,
                         float norm_min, float output_scale, int64_t stream);
void moe_router_topk_bf16(const void *logits, float *weights, uint32_t *ids, const float *selection_bias,
                          const float *expert_scale, int n_rows, int n_experts, int top_k, int score_mode,
                          int weight_mode, bool renormalize, bool clamp_logits, float clamp_min, float clamp_max,
                          float norm_min, float output_scale, int64_t stream);
void moe_router_topk_f16(const void *logits, float *weights, uint32_t *ids, const float *selection_bias,
                         const float *expert_scale, int n_rows, int n_experts, int top_k, int score_mode,
                         int weight_mode, bool renormalize, bool clamp_logits, float clamp_min, float clamp_max,
                         float norm_min, float output_scale, int64_t stream);

/* ------------------------------------------------------------------ QMatMul::forward that allocates nothing
 * qmm_qmatmul_forward_noalloc: no counterpart in the reference.  For callers that cannot allocate device memory --
 * code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc -- the host layer's
 * QMatMul::forward (qmm_qmatmul_forward in qmm_host.h, whose per-thread workspace grows with hipMalloc) with the same
 * routes and kernels: ys[rows, n] = xs[rows, k] . W^T, W = n rows of GGUF blocks of type wtype (8 q8_0, 12 q4_k,
 * 14 q6_k, 2 q4_0, 6 q5_0, 13 q5_k, 23 iq4_xs) padded as QTensor pads them; xs and ys device pointers of in_dtype
 * (0 f32, 1 f16, 30 bf16).  Quantized activations and split-K planes live in one 32 MiB device array of the library,
 * held by each device it runs on until the process ends; the quantized activations must fit in its 16 MiB
 * activation part (rows * ceil(k / 256) * 292 bytes, 272 for the 32-value block types, above 16 rows; rows * k / 256 *
 * 292 or rows * k / 32 * 34 bytes at 16 rows or fewer), else nothing is launched and the call returns -1 with
 * qmm_last_error() set.  Every call on a device shares that device's array: calls that overlap on one device race.
 * Returns 0, or -1 with the error recorded. */
int qmm_qmatmul_forward_noalloc(const void *w, uint32_t wtype, int64_t n, int64_t k, const void *xs, uint32_t in_dtype,
                                int64_t rows, void *ys, void *stream);

#ifdef __cplusplus
}
#endif
#endif
