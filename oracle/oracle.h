/*
 * TEST INFRASTRUCTURE ONLY.  A CPU restatement of inference.rs's GGUF QMatMul
 * arithmetic for Q8_0, Q4_K, Q6_K (and the Q8_K activation blocks), used as the
 * checker for the HIP library.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  Nothing in the product links it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the inference.rs repository root).
 */
#ifndef QMM_ORACLE_H
#define QMM_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* crates/inference-tensor/src/quantized/k_quants.rs:22-31 */
#define OR_QK_K 256
#define OR_QK8_0 32

/* crates/inference-tensor/src/quantized/k_quants.rs:152-157 */
typedef struct { uint16_t d; int8_t qs[32]; } or_block_q8_0;
/* k_quants.rs:188-195 */
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qs[128]; } or_block_q4k;
/* k_quants.rs:208-215 */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } or_block_q6k;
/* k_quants.rs:217-223 */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } or_block_q8k;
/* k_quants.rs:116-120: value j in qs[j] low nibble, value j + 16 in its high nibble, both offset by 8 */
typedef struct { uint16_t d; uint8_t qs[16]; } or_block_q4_0;
/* k_quants.rs:133-138: as Q4_0 with a fifth bit per value in the little-endian word qh (bit j = value j), offset 16 */
typedef struct { uint16_t d; uint8_t qh[4]; uint8_t qs[16]; } or_block_q5_0;
/* k_quants.rs:200-206: Q4_K's header and nibbles plus qh[32]; bit 2c of qh[l] is the fifth bit of value 64c + l,
 * bit 2c + 1 that of value 64c + 32 + l */
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } or_block_q5k;
/* IQ4_XS, 136 bytes per 256 values (crates/inference-quant/src/gguf/cpu_dot.rs:15-18, raw.rs:794-808): f16 d,
 * 6-bit sub-block scales (low 4 bits in scales_l nibbles, high 2 bits in scales_h), then per 32 values 16 bytes of
 * 4-bit indices into the IQ4_NL table (low nibbles the first 16 values, high nibbles the next 16) */
typedef struct { uint16_t d; uint16_t scales_h; uint8_t scales_l[4]; uint8_t qs[128]; } or_block_iq4xs;

/* GGUF type ids, crates/inference-tensor/src/quantized/mod.rs:582-603; IQ4_XS: inference-quant/src/gguf/kernel.rs:141 */
enum { OR_Q4_0 = 2, OR_Q5_0 = 6, OR_Q8_0 = 8, OR_Q4K = 12, OR_Q5K = 13, OR_Q6K = 14, OR_Q8K = 15, OR_IQ4XS = 23 };

/* the IQ4_NL / IQ4_XS value table (crates/inference-quant/src/gguf/raw.rs:13-15) */
extern const int8_t oracle_kvalues_iq4nl[16];

/* IEEE binary16 conversions, round to nearest even (the `half` crate 2.7.1's f16::from_f32 / to_f32) */
uint16_t oracle_f32_to_f16(float f);
float oracle_f16_to_f32(uint16_t h);

/* bytes per block and values per block for a GGUF type id (mod.rs:669-703); 0 for an unknown id */
size_t oracle_type_size(int type);
size_t oracle_block_size(int type);

/* quantizers (weights and activations) */
float oracle_quantize_block32(const float *x, int8_t *qs);                  /* mod.rs:43-56 */
void oracle_quantize_q8_0(const float *x, int64_t n, or_block_q8_0 *y);     /* k_quants.rs:923-949 */
void oracle_quantize_q8k(const float *x, int64_t n, or_block_q8k *y);       /* k_quants.rs:2721-2760 */
void oracle_quantize_q4k(const float *x, int64_t n, or_block_q4k *y);       /* k_quants.rs:1930-2001 */
void oracle_quantize_q6k(const float *x, int64_t n, or_block_q6k *y);       /* k_quants.rs:2590-2646 */
/* the sub-block searches alone (utils.rs:268-361, 135-264), for the tests that pin them */
float oracle_make_qkx2_quants(int nmax, const float *x, const float *weights, float rmin, float rdelta, int nstep,
                              int use_mad, uint8_t *l, float *neg_min);
float oracle_make_qx_quants(int n, int nmax, const float *x, int8_t *ls, int rmse_type);
void oracle_quantize_q4_0(const float *x, int64_t n, or_block_q4_0 *y);     /* k_quants.rs:380-418 */
void oracle_quantize_q5_0(const float *x, int64_t n, or_block_q5_0 *y);     /* k_quants.rs:681-717 */
void oracle_quantize_q5k(const float *x, int64_t n, or_block_q5k *y);       /* k_quants.rs:2256-2334 */
/* generic: quantize n values (multiple of the block size) of `type` into `out` (IQ4_XS has no quantizer: -1) */
int oracle_quantize(int type, const float *x, int64_t n, void *out);

/* dequantizers */
void oracle_dequantize(int type, const void *blocks, int64_t n, float *y);

/* vec_dot_unopt: one weight row (nblk blocks) against one activation row */
float oracle_vec_dot_q8_0_q8_0(int64_t n, const or_block_q8_0 *x, const or_block_q8_0 *y); /* k_quants.rs:982-999 */
float oracle_vec_dot_q4k_q8k(int64_t n, const or_block_q4k *x, const or_block_q8k *y);     /* k_quants.rs:1848-1928 */
float oracle_vec_dot_q6k_q8k(int64_t n, const or_block_q6k *x, const or_block_q8k *y);     /* k_quants.rs:2518-2575 */
float oracle_vec_dot_q4_0_q8_0(int64_t n, const or_block_q4_0 *x, const or_block_q8_0 *y); /* k_quants.rs:432-449 */
float oracle_vec_dot_q5_0_q8_0(int64_t n, const or_block_q5_0 *x, const or_block_q8_0 *y); /* k_quants.rs:615-637 */
float oracle_vec_dot_q5k_q8k(int64_t n, const or_block_q5k *x, const or_block_q8k *y);     /* k_quants.rs:2145-2232 */
/* crates/inference-quant/src/gguf/cpu_dot.rs:416-440 (iq4_xs_sub_scale, iq4_xs_generic) */
float oracle_vec_dot_iq4xs_q8k(int64_t n, const or_block_iq4xs *x, const or_block_q8k *y);

/* k_quants::matmul (k_quants.rs:2776-2894): dst[m][n] = vec_dot(W row n, Q8(lhs row m)).
 * `threads` <= 0 uses every available thread. Returns 0, or -1 on a bad type/shape. */
int oracle_matmul(int type, int64_t m, int64_t k, int64_t n, const float *lhs, const void *rhs, float *dst,
                  int threads);

/* The same with the activations already quantized (Q8_K rows for K-quants, Q8_0 rows for Q8_0). */
int oracle_matmul_preq(int type, int64_t m, int64_t k, int64_t n, const void *lhs_q, const void *rhs, float *dst,
                       int threads);

/* The arithmetic of this library's reference-named entries for the 32-value weight types (Q8_0, Q4_0, Q5_0): no
 * counterpart in the reference, whose GPU path gives them Q8_1 activations and whose CPU path Q8_0 ones
 * (k_quants.rs:2824-2830).  The reference sizes its activation buffers for Q8_1 (36 bytes per 32 values), which holds
 * a Q8_K quantization but not a Q8_K and a Q8_0 one, so those entries read Q8_K activations: each lhs row is quantized
 * with BlockQ8K::from_float over 256-value blocks (k padded to 256 with zeros), and
 *   dst[m][n] = sum over 32-value blocks b, in order, of (float)(sum_j w_j a_j) * d_w(b) * d_a(b / 8)
 * with the per-block integer dot of the weight's values (q - 8 for Q4_0, q - 16 for Q5_0) and the activation's int8
 * values, as vec_dot_q8_0_q8_0 / q4_0 / q5_0 scale a block (k_quants.rs:982-999, 432-449, 615-637) but with the f32
 * scale of the activation's 256-value block.  For the other types it is oracle_matmul.  Returns 0, or -1. */
int oracle_matmul_q8k_act(int type, int64_t m, int64_t k, int64_t n, const float *lhs, const void *rhs, float *dst,
                          int threads);

/* Expert-indexed matmul, the contract of QuantMethod::gather_forward
 * (crates/inference-quant/src/gguf/mod.rs:573-608, cpu.rs:23-104, quantized/mod.rs:1457-1461):
 * y[b][s][:] = W[ids[b][s]] . Q8(x[b][s % xdim1][:]),  W [E, n, k], x [batch, xdim1, k], ids [batch, topk],
 * y [batch, topk, n].  xdim1 is 1 or topk.  Returns -1 on an out-of-range expert id. */
int oracle_indexed_moe(int type, int64_t n_experts, int64_t n, int64_t k, const void *w, const float *x,
                       int64_t batch, int64_t xdim1, int64_t topk, const uint32_t *ids, float *y, int threads);

/* moe_dispatch (crates/inference-quant/kernels/cuda/moe_dispatch/moe_dispatch.cu:8-104): expert_bounds[E+1]
 * exclusive prefix of route counts; sorted_token_ids[pos] = flat route, sorted_source_ids[pos] = route / topk,
 * routes of one expert in ascending order (the stable order; the GPU may order within an expert freely). */
int oracle_moe_dispatch(const int32_t *topk_ids, int32_t total, int32_t n_experts, int32_t topk,
                        int32_t *expert_bounds, int32_t *sorted_token_ids, int32_t *sorted_source_ids);

/* moe_weighted_reduce_flat (moe_dispatch.cu:106-154): out[t][h] = sum_s w[t][s] * in[t][s][h] */
void oracle_moe_weighted_reduce(const float *in, const float *w, float *out, int32_t tokens, int32_t hidden,
                                int32_t topk);

/* x86.c: the path the reference's CPU QMatMul takes on x86-64 (repack_x86.rs, repack.rs:219-262, avx.rs), the
 * timed CPU baseline.  Levels: 0 none, 1 AVX2, 2 AVX-VNNI, 3 AVX-512 VNNI (repack_x86.rs:1318-1342). */
int oracle_x86_level(void);
int oracle_x86_amx(void);                                           /* repack_x86.rs:985-1024 */
int oracle_x86_select(int type, int64_t m, int64_t n, int64_t k);   /* repack_x86.rs:100-121 */
/* the weight with the tile forms the reference caches (repack.rs:35-70); `blocks` must outlive the handle */
void *oracle_x86_prepare(int type, const void *blocks, int64_t n, int64_t k);
void oracle_x86_release(void *handle);
/* dst [m][n] = lhs [m][k] x W^T on the reference's x86 route; returns 1 AMX, 2 tiles, 3 compact AVX2,
 * 4 scalar, -1 error */
int oracle_x86_matmul(const void *handle, int64_t m, const float *lhs, float *dst, int threads);
int oracle_x86_physical_cores(void);
int oracle_x86_describe(char *buf, int len);

#ifdef __cplusplus
}
#endif
#endif
