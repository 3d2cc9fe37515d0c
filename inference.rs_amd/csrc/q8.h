// Activation block quantizers shared by the standalone quantize kernels and the matvec that quantizes its
// own activations into LDS.  Bit-exact with the reference CPU quantizers:
//   Q8_K  BlockQ8K::from_float        crates/inference-tensor/src/quantized/k_quants.rs:2721-2760
//   Q8_0  quantize_block32 + f16 d    crates/inference-tensor/src/quantized/mod.rs:41-56, k_quants.rs:923-949
// Every step is a single IEEE operation (division, multiply, roundf: half away from zero), so contraction
// cannot merge them; it is switched off here regardless.
#pragma once

#include "common.h"

namespace qmm_q8 {

// Output addressing of one 256-value Q8_K block: decode layout (array of qmm_block_q8k, bsums int16) or the
// prefill tile layout (qs[nsb][rows][256], d[nsb][rows] f32, bsums[nsb][rows][16] as f16, which holds every
// bsum exactly: |bsum| <= 16 * 128 = 2048).
struct q8k_dst {
  uint8_t *qs;
  float *d;
  uint16_t *bsums;
  bool bsums_f16;
};

__device__ __forceinline__ q8k_dst q8k_decode_dst(uint8_t *vy, int64_t block) {
  uint8_t *b = vy + block * (int64_t)sizeof(qmm_block_q8k);
  return {b + 4, (float *)b, (uint16_t *)(b + 260), false};
}

__device__ __forceinline__ q8k_dst q8k_tile_dst(uint8_t *chan, int64_t rows, int64_t nsb, int64_t sb, int64_t r) {
  const int64_t i = sb * rows + r;
  uint8_t *qs = chan + i * 256;
  float *d = (float *)(chan + nsb * rows * 256) + i;
  uint16_t *bs = (uint16_t *)(chan + nsb * rows * 260) + i * 16;
  return {qs, d, bs, true};
}

__device__ __forceinline__ uint16_t bsum_bits(int s, bool f16) {
  return f16 ? f32_to_f16_bits((float)s) : (uint16_t)(int16_t)s;
}

// One wave quantizes v[0..3] of lanes 0..63 (values 4*lane .. 4*lane+3 of the block) and writes it.
__device__ __forceinline__ void q8k_wave(const float v[4], int lane, q8k_dst dst) {
#pragma clang fp contract(off)
  float best = 0.0f;
  int bidx = 0x7fffffff;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float a = fabsf(v[i]);
    if (a > best) {  // strictly greater: the first of equal magnitudes stays
      best = a;
      bidx = lane * 4 + i;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ob = __shfl_xor(best, off, QMM_WAVE);
    const int oi = __shfl_xor(bidx, off, QMM_WAVE);
    if (ob > best || (ob == best && oi < bidx)) {
      best = ob;
      bidx = oi;
    }
  }
  if (best == 0.0f) {  // amax == 0: an all-zero block (k_quants.rs:2740-2743)
    *(uint32_t *)(dst.qs + 4 * lane) = 0u;
    if (lane == 0) *dst.d = 0.0f;
    if ((lane & 3) == 0) dst.bsums[lane >> 2] = 0;  // +0 in both encodings
    return;
  }
  const float mine = v[bidx & 3];
  const float mx = __shfl(mine, bidx >> 2, QMM_WAVE);
  const float iscale = -127.0f / mx;
  int q[4];
#pragma unroll
  for (int i = 0; i < 4; i++) q[i] = sat_i8(roundf(iscale * v[i]));
  int s = q[0] + q[1] + q[2] + q[3];
  s += __shfl_xor(s, 1, QMM_WAVE);
  s += __shfl_xor(s, 2, QMM_WAVE);
  const uint32_t packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) | ((uint32_t)(q[2] & 0xff) << 16) |
                          ((uint32_t)(q[3] & 0xff) << 24);
  *(uint32_t *)(dst.qs + 4 * lane) = packed;
  if ((lane & 3) == 0) dst.bsums[lane >> 2] = bsum_bits(s, dst.bsums_f16);
  if (lane == 0) *dst.d = 1.0f / iscale;
}

// Eight lanes quantize one 32-value Q8_0 block (4 values each); writes qs (4 bytes/lane) and the f16 scale.
__device__ __forceinline__ void q8_0_group(const float v[4], int sub, int8_t *qs, uint16_t *d_out) {
#pragma clang fp contract(off)
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = fmaxf(amax, __shfl_xor(amax, 1, QMM_WAVE));
  amax = fmaxf(amax, __shfl_xor(amax, 2, QMM_WAVE));
  amax = fmaxf(amax, __shfl_xor(amax, 4, QMM_WAVE));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  int q[4];
#pragma unroll
  for (int i = 0; i < 4; i++) q[i] = sat_i8(roundf(v[i] * id));
  // qs may be only 2-byte aligned (34-byte blocks): two 16-bit stores
  uint16_t *q16 = (uint16_t *)(qs + 4 * sub);
  q16[0] = (uint16_t)((q[0] & 0xff) | ((q[1] & 0xff) << 8));
  q16[1] = (uint16_t)((q[2] & 0xff) | ((q[3] & 0xff) << 8));
  if (sub == 0) *d_out = f32_to_f16_bits(d);
}

template <class In>
__device__ __forceinline__ void load4(const typename In::T *row, int64_t k0, int64_t kx, float v[4]) {
#pragma unroll
  for (int i = 0; i < 4; i++) v[i] = (k0 + i < kx) ? In::load(row, k0 + i) : 0.0f;
}

}  // namespace qmm_q8
