/*
 * GGUF block layouts and type ids for the quantized-linear path (Q8_0, Q4_K, Q6_K weights and the
 * adjacent Q4_0, Q5_0, Q5_K, IQ4_XS; Q8_0 and Q8_K activation blocks).  Plain C so the C ABI, the C++
 * host and the HIP kernels share one definition.
 *
 * Layouts follow crates/inference-tensor/src/quantized/k_quants.rs:152-223 byte for byte, since
 * weights arrive as GGUF bytes; type ids follow quantized/mod.rs:582-603 (IQ4_XS, which the
 * reference's QTensor does not hold: crates/inference-quant/src/gguf/kernel.rs:141).
 */
#ifndef QMM_BLOCKS_H
#define QMM_BLOCKS_H

#include <stddef.h>
#include <stdint.h>

#define QMM_QK_K 256
#define QMM_QK8_0 32

/* GGUF type ids (GgmlDType::to_u32, quantized/mod.rs:605-624) */
enum qmm_ggml_type {
  QMM_TYPE_F32 = 0,
  QMM_TYPE_F16 = 1,
  QMM_TYPE_Q4_0 = 2,
  QMM_TYPE_Q4_1 = 3, /* storage only (loaded and saved; no kernels) */
  QMM_TYPE_Q5_0 = 6,
  QMM_TYPE_Q5_1 = 7, /* storage only */
  QMM_TYPE_Q8_0 = 8,
  QMM_TYPE_Q8_1 = 9, /* storage only */
  QMM_TYPE_Q2K = 10, /* storage only */
  QMM_TYPE_Q3K = 11, /* storage only */
  QMM_TYPE_Q4K = 12,
  QMM_TYPE_Q5K = 13,
  QMM_TYPE_Q6K = 14,
  QMM_TYPE_Q8K = 15,
  QMM_TYPE_IQ4_XS = 23,
  QMM_TYPE_BF16 = 30,
};

/* BlockQ8_0: f16 scale, 32 int8 values; 34 bytes (k_quants.rs:152-157) */
typedef struct {
  uint16_t d;
  int8_t qs[32];
} qmm_block_q8_0;

/* BlockQ4K: f16 d, f16 dmin, 12 bytes of packed 6-bit scales/mins, 128 bytes of nibbles; 144 bytes
 * (k_quants.rs:188-195).  qs[32c + l]: low nibble = value 64c + l, high nibble = value 64c + 32 + l. */
typedef struct {
  uint16_t d;
  uint16_t dmin;
  uint8_t scales[12];
  uint8_t qs[128];
} qmm_block_q4k;

/* BlockQ6K: low 4 bits, high 2 bits, int8 scale per 16 values, f16 d; 210 bytes (k_quants.rs:208-215) */
typedef struct {
  uint8_t ql[128];
  uint8_t qh[64];
  int8_t scales[16];
  uint16_t d;
} qmm_block_q6k;

/* BlockQ8K: f32 d, 256 int8 values, int16 sums of each 16; 292 bytes (k_quants.rs:217-223) */
typedef struct {
  float d;
  int8_t qs[256];
  int16_t bsums[16];
} qmm_block_q8k;

/* The activation block of the reference-named decode entries, in the reference's Q8_1 scratch of 36 bytes per 32
 * values (crates/inference-quant/src/gguf/fast_mmvq.rs:17-18): BlockQ8K's d and qs as BlockQ8K::from_float writes
 * them, the int16 sums of each 32 qs, and 12 zero bytes; 288 bytes per 256 values.  No counterpart in the reference
 * (whose GPU quantizer writes Q8_1 blocks of 32). */
typedef struct {
  float d;
  int8_t qs[256];
  int16_t s32[8];
  uint8_t pad[12];
} qmm_block_q8ks;

/* BlockQ4_0: f16 d, 16 bytes of nibbles; value j = low nibble of qs[j] - 8, value j + 16 = its high nibble - 8;
 * 18 bytes (k_quants.rs:116-120, 313-330) */
typedef struct {
  uint16_t d;
  uint8_t qs[16];
} qmm_block_q4_0;

/* BlockQ5_0: as Q4_0 plus a fifth bit per value (bit j of the little-endian word qh is value j's), offset 16;
 * 22 bytes (k_quants.rs:133-138, 720-743) */
typedef struct {
  uint16_t d;
  uint8_t qh[4];
  uint8_t qs[16];
} qmm_block_q5_0;

/* BlockQ5K: Q4_K's header and nibbles plus qh[32]: bit 2c of qh[l] is the fifth bit of value 64c + l, bit 2c + 1
 * that of value 64c + 32 + l; 176 bytes (k_quants.rs:200-206, 2433-2467) */
typedef struct {
  uint16_t d;
  uint16_t dmin;
  uint8_t scales[12];
  uint8_t qh[32];
  uint8_t qs[128];
} qmm_block_q5k;

/* IQ4_XS: f16 d, 6-bit sub-block scales (low 4 bits: nibble ib of scales_l; high 2: bits 2ib..2ib+1 of scales_h;
 * minus 32), 16 bytes of 4-bit indices into the IQ4_NL table per 32 values (low nibbles the first 16); 136 bytes
 * (crates/inference-quant/src/gguf/cpu_dot.rs:15-18, raw.rs:794-808) */
typedef struct {
  uint16_t d;
  uint16_t scales_h;
  uint8_t scales_l[4];
  uint8_t qs[128];
} qmm_block_iq4_xs;

#ifdef __cplusplus
static_assert(sizeof(qmm_block_q4_0) == 18, "BlockQ4_0 is 18 bytes");
static_assert(sizeof(qmm_block_q5_0) == 22, "BlockQ5_0 is 22 bytes");
static_assert(sizeof(qmm_block_q5k) == 176, "BlockQ5K is 176 bytes");
static_assert(sizeof(qmm_block_iq4_xs) == 136, "IQ4_XS is 136 bytes");
static_assert(sizeof(qmm_block_q8_0) == 34, "BlockQ8_0 is 34 bytes");
static_assert(sizeof(qmm_block_q4k) == 144, "BlockQ4K is 144 bytes");
static_assert(sizeof(qmm_block_q6k) == 210, "BlockQ6K is 210 bytes");
static_assert(sizeof(qmm_block_q8k) == 292, "BlockQ8K is 292 bytes");
static_assert(sizeof(qmm_block_q8ks) == 288, "the Q8_1-slot block is 288 bytes");
#else
_Static_assert(sizeof(qmm_block_q4_0) == 18, "BlockQ4_0 is 18 bytes");
_Static_assert(sizeof(qmm_block_q5_0) == 22, "BlockQ5_0 is 22 bytes");
_Static_assert(sizeof(qmm_block_q5k) == 176, "BlockQ5K is 176 bytes");
_Static_assert(sizeof(qmm_block_iq4_xs) == 136, "IQ4_XS is 136 bytes");
_Static_assert(sizeof(qmm_block_q8_0) == 34, "BlockQ8_0 is 34 bytes");
_Static_assert(sizeof(qmm_block_q4k) == 144, "BlockQ4K is 144 bytes");
_Static_assert(sizeof(qmm_block_q6k) == 210, "BlockQ6K is 210 bytes");
_Static_assert(sizeof(qmm_block_q8k) == 292, "BlockQ8K is 292 bytes");
_Static_assert(sizeof(qmm_block_q8ks) == 288, "the Q8_1-slot block is 288 bytes");
#endif

/* bytes per block and values per block (GgmlDType::type_size / block_size, quantized/mod.rs:669-703) */
static inline size_t qmm_type_size(int t) {
  switch (t) {
    case QMM_TYPE_F32: return 4;
    case QMM_TYPE_F16: case QMM_TYPE_BF16: return 2;
    case QMM_TYPE_Q8_0: return 34;
    case QMM_TYPE_Q4K: return 144;
    case QMM_TYPE_Q6K: return 210;
    case QMM_TYPE_Q8K: return 292;
    case QMM_TYPE_Q4_0: return 18;
    case QMM_TYPE_Q5_0: return 22;
    case QMM_TYPE_Q5K: return 176;
    case QMM_TYPE_IQ4_XS: return 136;
    case QMM_TYPE_Q4_1: return 20;
    case QMM_TYPE_Q5_1: return 24;
    case QMM_TYPE_Q8_1: return 36;
    case QMM_TYPE_Q2K: return 84;
    case QMM_TYPE_Q3K: return 110;
    default: return 0;
  }
}

static inline size_t qmm_block_size(int t) {
  switch (t) {
    case QMM_TYPE_F32: case QMM_TYPE_F16: case QMM_TYPE_BF16: return 1;
    case QMM_TYPE_Q8_0: case QMM_TYPE_Q4_0: case QMM_TYPE_Q5_0: case QMM_TYPE_Q4_1: case QMM_TYPE_Q5_1:
    case QMM_TYPE_Q8_1: return 32;
    case QMM_TYPE_Q4K: case QMM_TYPE_Q6K: case QMM_TYPE_Q8K: case QMM_TYPE_Q5K: case QMM_TYPE_IQ4_XS:
    case QMM_TYPE_Q2K: case QMM_TYPE_Q3K: return 256;
    default: return 0;
  }
}

/* the activation block type a weight type is dotted with (GgmlType::VecDotType): Q8_0 for the 32-value types,
 * Q8_K for the super-block types (IQ4_XS: cpu_dot.rs:67-68) */
static inline int qmm_vec_dot_type(int t) { return qmm_block_size(t) == 32 ? QMM_TYPE_Q8_0 : QMM_TYPE_Q8K; }

/* The decode / prefill boundary of QMatMul::forward, shared by the host layer and qmm_qmatmul_forward_noalloc: up to
 * this many activation rows take the decode launchers (fast_mmvq.rs TENSOR_CORE_MAX_ROWS = 16, re-derived for gfx950:
 * Q4_K, and Q6_K rows of at most 8192 values, stay on the decode launcher up to 32 rows, where its few-row MFMA
 * kernel still beats the prefill matmul), more the prefill matmul. */
static inline int64_t qmm_max_decode_rows(int type, int64_t k) {
  return type == QMM_TYPE_Q4K || (type == QMM_TYPE_Q6K && k <= 8192) ? 32 : 16;
}

#endif
